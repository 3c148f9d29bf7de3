"""fuse_attention, host side (no GPU): the module patch, its undo, and that a
call off a HIP device runs LlamaAttention's own forward unchanged."""
from __future__ import annotations

import torch
from transformers.models.llama import modeling_llama as hf

from tests.helpers import CFG1, llama_config


def _model():
    from femtotron_amd.model import build_llama_model, init_llama_weights_
    return init_llama_weights_(build_llama_model(llama_config(CFG1, layers=2)), device="cpu",
                               dtype=torch.float32, seed=42)


def _step(model, ids):
    for p in model.parameters():
        p.grad = None
    loss = model(ids, labels=ids)["loss"]
    loss.backward()
    return loss.detach(), {n: p.grad.clone() for n, p in model.named_parameters()}


def test_patch_and_undo_keep_module_and_state_dict():
    from femtotron_amd import fuse_attention
    from femtotron_amd.fused_attention import unfuse_attention
    model = _model()
    keys = list(model.state_dict())
    attns = [m for m in model.modules() if isinstance(m, hf.LlamaAttention)]
    assert fuse_attention(model) == len(attns) == CFG1["layers"]
    assert fuse_attention(model) == 0  # already patched
    assert all(type(m) is hf.LlamaAttention and "forward" in m.__dict__ for m in attns)
    assert list(model.state_dict()) == keys
    assert unfuse_attention(model) == len(attns)
    assert all("forward" not in m.__dict__ for m in attns)
    assert unfuse_attention(model) == 0


def test_cpu_call_runs_the_modules_own_forward():
    """On the CPU every call falls back, and loss and grads equal the unpatched
    model's bit for bit."""
    from femtotron_amd import fuse_attention
    from femtotron_amd.fused_attention import (attention_dispatch_counts, last_attention_fallback_reason,
                                               reset_attention_dispatch_counts, unfuse_attention)
    model = _model()
    ids = torch.randint(0, CFG1["vocab"], (CFG1["batch"], 64), generator=torch.Generator().manual_seed(2000))
    loss0, g0 = _step(model, ids)
    fuse_attention(model)
    reset_attention_dispatch_counts()
    loss1, g1 = _step(model, ids)
    assert attention_dispatch_counts() == {"fused": 0, "fallback": CFG1["layers"]}
    assert last_attention_fallback_reason() == "hidden_states not on a HIP device"
    assert torch.equal(loss0, loss1)
    assert all(torch.equal(g0[n], g1[n]) for n in g0)
    unfuse_attention(model)


def test_only_causal_sdpa_attention_is_fusable():
    """The kernels are causal.  HF's eager attention, and an unset
    implementation (resolved to eager), attend in both directions when called
    without a mask (modeling_llama.py:202-204), so both planners refuse them;
    sdpa without a mask is causal while the module's is_causal holds."""
    from femtotron_amd.fused_checkpoint import _causal_attention_reason

    def attn(impl):
        return hf.LlamaAttention(llama_config(CFG1, layers=1, attn=impl), layer_idx=0)

    assert _causal_attention_reason(attn("sdpa")) is None
    for impl in ("eager", None):
        assert "not causal" in _causal_attention_reason(attn(impl))
    assert "flash" in _causal_attention_reason(attn("flash_attention_2"))
    a = attn("sdpa")
    a.is_causal = False
    assert _causal_attention_reason(a) == "attention module is not causal"
