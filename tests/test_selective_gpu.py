"""Selective activation checkpointing (the "llama_mlp_and_norms" preset) on the fused path.

The policy wraps every LlamaMLP and LlamaRMSNorm (femtotron/scripts/presets.py:45-62,
femtotron/training/ckpt_policy.py:70-124), so ``checkpoint_fn`` receives those
modules; attention stays un-checkpointed (stock HF code outside the boundary).

Checkers: the CPU fp32 oracle (config 1, 1e-5: the checkpointing policy does
not change the arithmetic, so the model's loss and grads must equal the
oracle's), the oracle's mlp/rmsnorm functions per module, and the reference
path itself (HF modules under torch.utils.checkpoint) on the GPU in bf16 with
the north star's tensor-level metric.
"""
from __future__ import annotations

import pytest
import torch

from oracle import torch_llama as ot
from tests.helpers import (BF16_ATOL, BF16_RTOL, CFG1, CFG3, CFG4, llama_config, randn, rel_err)

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _model(c, layers, dtype, seed=42):
    from femtotron_amd.model import build_llama_model, init_llama_weights_
    return init_llama_weights_(build_llama_model(llama_config(c, layers=layers)), device=DEV,
                               dtype=dtype, seed=seed)


def _step(model, ids):
    for p in model.parameters():
        p.grad = None
    loss = model(ids, labels=ids)["loss"]
    loss.backward()
    return loss.detach(), {n.replace("._checkpoint_wrapped_module", ""): p.grad
                           for n, p in model.named_parameters()}


def test_selective_cfg1_fp32_model_vs_cpu_oracle():
    """Config 1 end to end with the selective policy: 3 fused calls per layer
    (two norms, one MLP) plus the final norm, loss and all 21 grads within 1e-5
    of the CPU fp32 oracle."""
    from femtotron_amd import dispatch_counts, fused_checkpoint, reset_dispatch_counts
    from femtotron_amd.scripts.presets import get_ac_policy
    from femtotron_amd.training import apply_activation_checkpointing

    c = CFG1
    model = _model(c, c["layers"], torch.float32)
    n_wrapped = apply_activation_checkpointing(model, get_ac_policy("llama_mlp_and_norms"),
                                               checkpoint_fn=fused_checkpoint)
    assert n_wrapped == 3 * c["layers"] + 1
    ids = torch.randint(0, c["vocab"], (c["batch"], c["seq"]), generator=torch.Generator().manual_seed(2000))
    reset_dispatch_counts()
    loss, grads = _step(model, ids.to(DEV))
    assert dispatch_counts() == {"fused": 3 * c["layers"] + 1, "fallback": 0}
    orc = ot.OracleLlama(vocab=c["vocab"], hidden=c["hidden"], n_layers=c["layers"], n_heads=c["heads"],
                         n_kv=c["kv"], ffn=c["ffn"], theta=c["theta"])
    _, oloss = orc.forward(ids, ids)
    oloss.backward()
    assert abs(loss.item() - oloss.item()) <= 1e-5 * abs(oloss.item())
    for n, t in orc.named_params():
        assert rel_err(grads[n], t.grad) < 1e-5, f"{n}: rel {rel_err(grads[n], t.grad):.3e}"


@pytest.mark.parametrize("name,c,B,S", [("tinyllama", CFG3, 2, 1024), ("llama3-slice", CFG4, 1, 1024)])
def test_selective_bf16_matches_stock_checkpoint(name, c, B, S):
    """2-layer bf16 model with the selective policy: fused vs the reference path
    (same model under torch.utils.checkpoint, debug=True) on the GPU.  Loss
    within 2e-2 relative, every gradient within the tensor-level metric."""
    from femtotron_amd import dispatch_counts, fused_checkpoint, reset_dispatch_counts
    from femtotron_amd.scripts.presets import get_ac_policy
    from femtotron_amd.training import apply_activation_checkpointing, remove_activation_checkpointing
    from torch.utils.checkpoint import checkpoint

    model = _model(c, 2, torch.bfloat16)
    policy = get_ac_policy("llama_mlp_and_norms")
    ids = torch.randint(0, c["vocab"], (B, S), generator=torch.Generator().manual_seed(2000)).to(DEV)
    apply_activation_checkpointing(model, policy, checkpoint_fn=fused_checkpoint)
    reset_dispatch_counts()
    loss_f, g_f = _step(model, ids)
    assert dispatch_counts() == {"fused": 7, "fallback": 0}
    g_f = {n: g.clone() for n, g in g_f.items()}
    remove_activation_checkpointing(model)
    apply_activation_checkpointing(model, policy, checkpoint_fn=checkpoint)
    loss_r, g_r = _step(model, ids)
    assert abs(loss_f.item() - loss_r.item()) <= BF16_RTOL * abs(loss_r.item())
    assert g_f.keys() == g_r.keys()
    for n in g_r:
        a, b = g_f[n].float(), g_r[n].float()
        err = float((a - b).abs().max())
        lim = BF16_ATOL + BF16_RTOL * float(b.abs().max())
        assert bool(torch.isfinite(a).all()) and err <= lim, f"{name} {n}: {err:.3e} > {lim:.3e}"


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-5), (torch.bfloat16, None)])
def test_fused_mlp_and_norm_modules_vs_oracle(dtype, tol):
    """One checkpointed LlamaMLP and one LlamaRMSNorm (config-1 widths, ragged
    token count) vs the oracle's mlp / rmsnorm on the CPU: fp32 within 1e-5,
    bf16 with the tensor-level metric."""
    from transformers.models.llama import modeling_llama as hf
    from femtotron_amd import dispatch_counts, fused_checkpoint, reset_dispatch_counts
    from femtotron_amd.training import ActivationCheckpointWrapper

    c = CFG1
    cfg = llama_config(c, layers=1)
    T = 77
    mlp = hf.LlamaMLP(cfg)
    norm = hf.LlamaRMSNorm(c["hidden"], eps=1e-5)
    with torch.no_grad():
        for i, p in enumerate(list(mlp.parameters()) + list(norm.parameters())):
            p.copy_(randn(p.shape, 10 + i, std=0.02, mean=1.0 if p.dim() == 1 else 0.0))
    mlp, norm = mlp.to(DEV, dtype), norm.to(DEV, dtype)
    x = randn((1, T, c["hidden"]), 3).to(DEV, dtype).requires_grad_(True)
    dy = randn((1, T, c["hidden"]), 4).to(DEV, dtype)
    reset_dispatch_counts()
    y = ActivationCheckpointWrapper(mlp, checkpoint_fn=fused_checkpoint)(
        ActivationCheckpointWrapper(norm, checkpoint_fn=fused_checkpoint)(x))
    y.backward(dy)
    assert dispatch_counts() == {"fused": 2, "fallback": 0}

    w = {k: p.detach().cpu().to(dtype).requires_grad_(True) for k, p in
         (("wg", mlp.gate_proj.weight), ("wu", mlp.up_proj.weight), ("wd", mlp.down_proj.weight),
          ("w", norm.weight))}
    xr = x.detach().cpu().requires_grad_(True)
    yr = ot.mlp(ot.rmsnorm(xr, w["w"], 1e-5), w["wg"], w["wu"], w["wd"])
    yr.backward(dy.cpu())
    pairs = [("y", y, yr), ("dx", x.grad, xr.grad), ("dwg", mlp.gate_proj.weight.grad, w["wg"].grad),
             ("dwu", mlp.up_proj.weight.grad, w["wu"].grad), ("dwd", mlp.down_proj.weight.grad, w["wd"].grad),
             ("dw", norm.weight.grad, w["w"].grad)]
    for n, a, b in pairs:
        a, b = a.detach().float().cpu(), b.detach().float()
        if tol is not None:
            assert rel_err(a, b) < tol, f"{n}: rel {rel_err(a, b):.3e}"
        else:
            err = float((a - b).abs().max())
            lim = BF16_ATOL + BF16_RTOL * float(b.abs().max())
            assert err <= lim, f"{n}: {err:.3e} > {lim:.3e}"


def test_selective_peak_memory_not_above_stock_checkpoint():
    """Peak memory of one fwd+bwd of a 2-layer TinyLlama-shaped model (B=2,
    S=2048) under the selective policy: fused <= reference path."""
    from femtotron_amd import fused_checkpoint
    from femtotron_amd.scripts.presets import get_ac_policy
    from femtotron_amd.training import apply_activation_checkpointing, remove_activation_checkpointing
    from torch.utils.checkpoint import checkpoint

    c = CFG3
    model = _model(c, 2, torch.bfloat16)
    policy = get_ac_policy("llama_mlp_and_norms")
    ids = torch.randint(0, c["vocab"], (2, 2048), generator=torch.Generator().manual_seed(2000)).to(DEV)

    def peak(fn):
        remove_activation_checkpointing(model)
        apply_activation_checkpointing(model, policy, checkpoint_fn=fn)
        for _ in range(2):  # the second pass measures, with grads already allocated
            torch.cuda.synchronize()
            torch.cuda.reset_peak_memory_stats()
            base = torch.cuda.memory_allocated()
            model(ids, labels=ids)["loss"].backward()
            torch.cuda.synchronize()
        return torch.cuda.max_memory_allocated() - base

    p_fused = peak(fused_checkpoint)
    p_ref = peak(checkpoint)
    assert p_fused <= p_ref, f"fused peak {p_fused / 2**20:.1f} MiB > reference {p_ref / 2**20:.1f} MiB"
