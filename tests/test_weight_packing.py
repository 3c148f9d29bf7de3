"""femtotron_amd.weight_packing: contiguous q/k/v and gate/up parameter storage.

CPU: the packed layout is detected, survives in-place updates (optimizer step,
load_state_dict) and leaves names, shapes and values unchanged; re-allocating a
parameter is detected as unpacked.  GPU: the fused layer gives bitwise identical
outputs and gradients with packed and unpacked weights (the GEMM sees the same
values in the same layout either way)."""
from __future__ import annotations

import pytest
import torch

from femtotron_amd.weight_packing import pack_layer_weights, packed
from tests.helpers import CFG1, llama_config


def _model():
    from femtotron_amd.model import build_llama_model, init_llama_weights_
    return init_llama_weights_(build_llama_model(llama_config(CFG1)), device="cpu", dtype=torch.float32)


def test_pack_keeps_names_values_and_is_detected():
    model = _model()
    before = {k: v.clone() for k, v in model.state_dict().items()}
    names = [n for n, _ in model.named_parameters()]
    params = list(model.parameters())
    assert pack_layer_weights(model) == 2 * CFG1["layers"]
    assert pack_layer_weights(model) == 0  # idempotent
    assert [n for n, _ in model.named_parameters()] == names
    assert all(a is b for a, b in zip(params, model.parameters()))
    after = model.state_dict()
    assert before.keys() == after.keys()
    for k in before:
        assert torch.equal(before[k], after[k]), k
    layer = next(iter(model.model.layers.values()))
    a, m = layer.self_attn, layer.mlp
    view = packed(a.q_proj.weight, a.k_proj.weight, a.v_proj.weight)
    assert view is not None
    assert torch.equal(view, torch.cat((a.q_proj.weight, a.k_proj.weight, a.v_proj.weight)))
    assert packed(m.gate_proj.weight, m.up_proj.weight) is not None
    assert packed(a.k_proj.weight, a.q_proj.weight) is None  # wrong order is not a packed group


def test_pack_survives_in_place_updates_and_detects_reallocation():
    model = _model()
    pack_layer_weights(model)
    opt = torch.optim.AdamW(model.parameters(), lr=1e-3)
    ids = torch.randint(0, CFG1["vocab"], (2, 16), generator=torch.Generator().manual_seed(0))
    model(ids, labels=ids)["loss"].backward()
    opt.step()
    a = next(iter(model.model.layers.values())).self_attn
    view = packed(a.q_proj.weight, a.k_proj.weight, a.v_proj.weight)
    assert view is not None
    assert torch.equal(view[: a.q_proj.weight.shape[0]], a.q_proj.weight)
    sd = {k: v.clone() + 1 for k, v in model.state_dict().items()}
    model.load_state_dict(sd)
    assert packed(a.q_proj.weight, a.k_proj.weight, a.v_proj.weight) is not None
    assert torch.equal(a.k_proj.weight, sd["model.layers.0.self_attn.k_proj.weight"])
    a.k_proj.weight.data = a.k_proj.weight.data.clone()  # re-allocation breaks the layout
    assert packed(a.q_proj.weight, a.k_proj.weight, a.v_proj.weight) is None


@pytest.mark.gpu
def test_fused_layer_bitwise_identical_with_packed_weights():
    from femtotron_amd import fused_checkpoint
    from femtotron_amd.training import ActivationCheckpointWrapper
    from oracle import torch_llama as ot
    from transformers.models.llama import modeling_llama as hf
    from tests.helpers import CFG3, layer_weights, load_into_hf_layer, randn, hf_layer_grads

    dev = "cuda:0"
    B, S = 2, 512
    cos, sin = ot.rope_cos_sin(S, 64, CFG3["theta"], torch.bfloat16, device=dev)
    x0 = randn((B, S, CFG3["hidden"]), 1).to(dev, torch.bfloat16)
    dy = randn((B, S, CFG3["hidden"]), 2).to(dev, torch.bfloat16)
    res = []
    for pack in (False, True):
        layer = hf.LlamaDecoderLayer(llama_config(CFG3, layers=1), 0)
        load_into_hf_layer(layer, layer_weights(CFG3, seed=5))
        layer = layer.to(dev, torch.bfloat16)
        if pack:
            assert pack_layer_weights(layer) == 2
        x = x0.clone().requires_grad_(True)
        out = ActivationCheckpointWrapper(layer, checkpoint_fn=fused_checkpoint)(
            x, attention_mask=None, position_embeddings=(cos, sin), past_key_values=None,
            use_cache=False)
        out.backward(dy)
        res.append((out.detach(), x.grad, hf_layer_grads(layer)))
    (o0, dx0, g0), (o1, dx1, g1) = res
    assert torch.equal(o0, o1) and torch.equal(dx0, dx1)
    for k in g0:
        assert torch.equal(g0[k], g1[k]), k
