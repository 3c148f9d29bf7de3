"""Golden fixtures written from the reference itself (tests/golden/make_golden.py
ran femtotron's own TP=1 model stack and ActivationCheckpointWrapper on the CPU).

CPU: the oracle (oracle/torch_llama.py) and the product's host model
(femtotron_amd.model + the API-identical AC wrapper, stock checkpoint) both
reproduce the reference's config-1 loss and every gradient to 1e-5 (fp32), and
the reference's bf16 checkpointed layer to bf16 tolerance.
GPU: the fused HIP path reproduces the same fixtures (1e-5 fp32; rtol 2e-2 /
atol 2e-3 bf16).
"""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import torch_llama as ot
from tests.helpers import CFG1, llama_config

GOLD = Path(__file__).resolve().parent / "golden"
PROJ_SEEDS = (11, 22, 33, 44)


def checksum(t: torch.Tensor) -> dict:
    """Same summary as make_golden.checksum (sum, sumsq, absmax, seeded projections)."""
    x = t.detach().double().reshape(-1).cpu()
    out = {"sum": float(x.sum()), "sumsq": float((x * x).sum()), "absmax": float(x.abs().max())}
    for s in PROJ_SEEDS:
        g = torch.Generator().manual_seed(s * 1000 + x.numel() % 997)
        out[f"proj{s}"] = float((x * torch.randn(x.numel(), generator=g, dtype=torch.float64)).sum())
    return out


def assert_checksum(t: torch.Tensor, ref: dict, rtol: float, name: str) -> None:
    """Every field within rtol of the tensor's scale: an element error of
    rtol*|x| moves a projection by about rtol*sqrt(sumsq)."""
    got = checksum(t)
    assert list(t.shape) == ref["shape"], f"{name}: shape {list(t.shape)} vs {ref['shape']}"
    scale = max(ref["sumsq"] ** 0.5, 1e-30)
    for k in ("sum", *(f"proj{s}" for s in PROJ_SEEDS)):
        assert abs(got[k] - ref[k]) <= 4 * rtol * scale, f"{name}.{k}: {got[k]!r} vs {ref[k]!r}"
    assert abs(got["sumsq"] ** 0.5 - scale) <= rtol * scale, f"{name}.norm"
    assert abs(got["absmax"] - ref["absmax"]) <= rtol * max(ref["absmax"], 1e-30), f"{name}.absmax"


def _cfg1():
    return json.loads((GOLD / "cfg1.json").read_text())


def _ids(fx):
    c = fx["config"]
    ids = torch.randint(0, c["vocab"], (c["batch"], c["seq"]),
                        generator=torch.Generator().manual_seed(c["token_seed"]))
    assert int(ids.sum()) == fx["ids_sum"]
    return ids


def _check_cfg1(fx, loss: float, named: dict, rtol: float) -> None:
    assert abs(loss - fx["loss"]) <= rtol * abs(fx["loss"]), (loss, fx["loss"])
    assert list(named) == fx["param_names"]
    for n in fx["param_names"]:
        assert_checksum(named[n].grad, fx["grads"][n], rtol, f"grad {n}")
    for n, full in fx["grads_full_small"].items():
        g = named[n].grad.double().reshape(-1).cpu()
        ref = torch.tensor(full, dtype=torch.float64)
        assert float((g - ref).abs().max()) <= rtol * float(ref.abs().max()), f"grad {n} (full)"


def test_golden_fixture_is_self_consistent():
    fx = _cfg1()
    assert fx["n_wrapped"] == fx["config"]["layers"] == 2
    assert len(fx["param_names"]) == 1 + 9 * 2 + 2
    # the wrapper hides its prefix: state_dict keys are the plain parameter names
    assert all("_checkpoint_wrapped_module" not in k for k in fx["state_dict_keys"])


def test_oracle_reproduces_reference_cfg1_fp32():
    fx = _cfg1()
    c = fx["config"]
    orc = ot.OracleLlama(vocab=c["vocab"], hidden=c["hidden"], n_layers=c["layers"], n_heads=c["heads"],
                         n_kv=c["kv_heads"], ffn=c["ffn"], theta=c["theta"], seed=c["weight_seed"],
                         std=c["init_std"])
    named = dict(orc.named_params())
    # same weights: the reference's registration order matches the oracle's draw order
    ref_order = fx["param_names"]
    assert ref_order == list(named)
    for n in named:
        assert_checksum(named[n], fx["weights"][n], 1e-12, f"weight {n}")
    ids = _ids(fx)
    logits, loss = orc.forward(ids, ids)
    loss.backward()
    assert_checksum(logits, fx["logits"], 1e-5, "logits")
    _check_cfg1(fx, loss.item(), {n: named[n] for n in ref_order}, 1e-5)


def test_product_model_cpu_reproduces_reference_cfg1_fp32():
    """femtotron_amd.model (HF layers) + API-identical wrapper with the stock
    checkpoint, on CPU: same state_dict keys, loss and gradients as the
    reference's own stack."""
    from femtotron_amd.model import build_llama_model, init_llama_weights_
    from femtotron_amd.scripts.presets import get_ac_policy
    from femtotron_amd.training import apply_activation_checkpointing
    fx = _cfg1()
    model = init_llama_weights_(build_llama_model(llama_config(CFG1)), device="cpu", dtype=torch.float32)
    named = dict(model.named_parameters())
    assert apply_activation_checkpointing(model, get_ac_policy("llama_decoder_layer"),
                                          preserve_rng_state=True) == 2
    assert list(model.state_dict().keys()) == fx["state_dict_keys"]
    ids = _ids(fx)
    out = model(ids, labels=ids)
    out["loss"].backward()
    assert_checksum(out["logits"], fx["logits"], 1e-5, "logits")
    _check_cfg1(fx, out["loss"].item(), {n: named[n] for n in fx["param_names"]}, 1e-5)


# ------------------------------------------------------------ bf16 layer
def _bits(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(a.copy()).view(torch.bfloat16)


def _layer_fixture():
    z = np.load(GOLD / "layer_bf16.npz")
    from transformers.models.llama.modeling_llama import LlamaDecoderLayer
    layer = LlamaDecoderLayer(llama_config(CFG1, layers=1), 0)
    gen = torch.Generator().manual_seed(7)
    with torch.no_grad():
        for name, p in layer.named_parameters():
            w = torch.empty(p.shape, dtype=torch.float32).normal_(0.0, 0.02, generator=gen)
            if name.endswith("layernorm.weight"):
                w += 1.0
            p.copy_(w)
    layer = layer.bfloat16()
    for name, p in layer.named_parameters():  # identical bf16 weights to the fixture's
        s = checksum(p)
        assert abs(s["sum"] - z["wsum:" + name][0]) < 1e-9 and abs(s["proj11"] - z["wsum:" + name][1]) < 1e-9
    return z, layer


def _tensor_ok(a: torch.Tensor, b: torch.Tensor, rtol: float, atol: float) -> tuple[bool, float, float]:
    a, b = a.detach().float().cpu(), b.detach().float().cpu()
    err, lim = float((a - b).abs().max()), atol + rtol * float(b.abs().max())
    return err <= lim, err, lim


def test_oracle_reproduces_reference_layer_bf16():
    z, layer = _layer_fixture()
    names = [n for n, _ in layer.named_parameters()]
    keymap = dict(zip(names, ot.LAYER_KEYS))
    w = {keymap[n]: p.detach().clone().requires_grad_(True) for n, p in layer.named_parameters()}
    x = _bits(z["x"]).clone().requires_grad_(True)
    out = ot.decoder_layer(x, _bits(z["cos"]), _bits(z["sin"]), w, 8, 4, 32, 1e-5)
    out.backward(_bits(z["dy"]))
    checks = [("out", out, _bits(z["out"])), ("dx", x.grad, _bits(z["dx"]))]
    checks += [(n, w[keymap[n]].grad, _bits(z["g:" + n])) for n in names]
    for name, a, b in checks:
        ok, err, lim = _tensor_ok(a, b, 2e-2, 2e-3)
        assert ok, f"{name}: max|a-b| {err:.3e} > {lim:.3e}"


@pytest.mark.gpu
def test_fused_gpu_reproduces_reference_layer_bf16():
    from femtotron_amd import dispatch_counts, fused_checkpoint, reset_dispatch_counts
    from femtotron_amd.training import ActivationCheckpointWrapper
    z, layer = _layer_fixture()
    layer = layer.to("cuda")
    wrapped = ActivationCheckpointWrapper(layer, checkpoint_fn=fused_checkpoint)
    x = _bits(z["x"]).cuda().requires_grad_(True)
    reset_dispatch_counts()
    out = wrapped(x, attention_mask=None, position_embeddings=(_bits(z["cos"]).cuda(), _bits(z["sin"]).cuda()),
                  past_key_values=None, use_cache=False)
    out.backward(_bits(z["dy"]).cuda())
    assert dispatch_counts()["fused"] == 1
    checks = [("out", out, _bits(z["out"])), ("dx", x.grad, _bits(z["dx"]))]
    checks += [(n, p.grad, _bits(z["g:" + n])) for n, p in layer.named_parameters()]
    for name, a, b in checks:
        ok, err, lim = _tensor_ok(a, b, 2e-2, 2e-3)
        assert ok, f"{name}: max|a-b| {err:.3e} > {lim:.3e}"


@pytest.mark.gpu
def test_fused_gpu_reproduces_reference_cfg1_fp32():
    from femtotron_amd import dispatch_counts, fused_checkpoint, reset_dispatch_counts
    from femtotron_amd.model import build_llama_model, init_llama_weights_
    from femtotron_amd.scripts.presets import get_ac_policy
    from femtotron_amd.training import apply_activation_checkpointing
    fx = _cfg1()
    model = init_llama_weights_(build_llama_model(llama_config(CFG1)), device="cuda", dtype=torch.float32)
    named = dict(model.named_parameters())
    apply_activation_checkpointing(model, get_ac_policy("llama_decoder_layer"), checkpoint_fn=fused_checkpoint)
    ids = _ids(fx).cuda()
    reset_dispatch_counts()
    out = model(ids, labels=ids)
    out["loss"].backward()
    assert dispatch_counts() == {"fused": 2, "fallback": 0}
    assert_checksum(out["logits"], fx["logits"], 1e-5, "logits")
    _check_cfg1(fx, out["loss"].item(), {n: named[n] for n in fx["param_names"]}, 1e-5)
