"""Fused checkpointed sub-modules for selective activation checkpointing.

The selective policy ``any_of(by_class_name("LlamaMLP"), by_class_name("LlamaRMSNorm"))``
(femtotron/training/ckpt_policy.py:70-124; the "llama_mlp_and_norms" preset) wraps the
MLP and the two norms of every decoder layer instead of the whole layer, so
``checkpoint_fn`` is called with those modules (femtotron/training/activation_ckpt.py:78-86,
called from HF models/llama/modeling_llama.py:311-323).  These autograd nodes are
the fused equivalents: each keeps only its input (as torch.utils.checkpoint's
``_NoopSaveInputs`` does, torch/utils/checkpoint.py:794-831) and recomputes in
backward what the backward needs.

MLP (HF models/llama/modeling_llama.py:163-177):
    g,u = z Wg^T, z Wu^T   -> one GEMM over [Wg;Wu] into a [T, 2F] buffer
    p   = silu(g)*u        (fh_swiglu_fwd, HF's two bf16 roundings; in backward fh_swiglu_bwd)
    m   = p Wd^T
RMSNorm (HF models/llama/modeling_llama.py:52-70):
    y = w * to_dtype(x * rsqrt(mean(x^2) + eps))   (fh_rmsnorm_fwd; backward
    fh_rmsnorm_bwd recomputes rstd from x, so nothing but x is kept)
"""
from __future__ import annotations

import torch

from . import ops
from .fused_layer import _cat_rows, _WgradStream, grad_target, split_rows
from .projections import linear, linear_dgrad


def mlp_forward(z2: torch.Tensor, wg: torch.Tensor, wu: torch.Tensor, wd: torch.Tensor, *,
                keep: bool):
    """z2 [T, H] -> m [T, H]; keep=True stops after the gate/up projection and
    returns gu for the backward (whose SwiGLU pass writes the product p)."""
    F_ = wg.shape[0]
    gu = linear(z2, _cat_rows(wg, wu))
    if keep:
        return gu
    p = ops.swiglu_fwd(gu[:, :F_], gu[:, F_:])
    del gu
    return linear(p, wd)


def mlp_backward(dm2: torch.Tensor, z2: torch.Tensor, wg: torch.Tensor, wu: torch.Tensor,
                 wd: torch.Tensor, gu: torch.Tensor):
    """The MLP's backward from the recomputed gu (pass it without keeping a
    reference, so that it is freed once the SwiGLU backward has read it).
    Weight gradients accumulated into existing .grad tensors come back None."""
    F_ = wg.shape[0]
    wg_stream = _WgradStream(dm2.device)
    dp = linear_dgrad(dm2, wd)
    dgu = torch.empty_like(gu)
    # also p = silu(g)*u, into dp's buffer (read before overwritten), for dWd
    ops.swiglu_bwd(dp, gu[:, :F_], gu[:, F_:], dgu[:, :F_], dgu[:, F_:], p_out=dp)
    del gu
    dwd = wg_stream.mm_tn(dm2, dp, grad_target(wd))
    del dp
    dwgu = wg_stream.mm_tn(dgu, z2, grad_target(wg, wu))
    dz = linear_dgrad(dgu, _cat_rows(wg, wu))
    wg_stream.join()
    return (dz, *split_rows(dwgu, F_, F_), dwd)


class FusedMLPFunction(torch.autograd.Function):
    """autograd node for one checkpointed LlamaMLP.  Saved: the input z only
    (plus references to the weights)."""

    @staticmethod
    def forward(ctx, z, wg, wu, wd):
        H = z.shape[-1]
        m = mlp_forward(z.reshape(-1, H), wg, wu, wd, keep=False)
        ctx.save_for_backward(z, wg, wu, wd)
        return m.view(z.shape)

    @staticmethod
    def backward(ctx, dm):
        z, wg, wu, wd = ctx.saved_tensors
        H = z.shape[-1]
        z2 = z.reshape(-1, H)
        with torch.no_grad():
            dz, dwg, dwu, dwd = mlp_backward(dm.contiguous().view(-1, H), z2, wg, wu, wd,
                                             mlp_forward(z2, wg, wu, wd, keep=True))
        return dz.view(z.shape), dwg, dwu, dwd


class FusedRMSNormFunction(torch.autograd.Function):
    """autograd node for one checkpointed LlamaRMSNorm.  Saved: the input x only
    (plus a reference to the weight); the backward kernel recomputes the row
    statistics from x."""

    @staticmethod
    def forward(ctx, x, w, eps):
        y = ops.rmsnorm_fwd(x, w, eps)
        ctx.save_for_backward(x, w)
        ctx.eps = eps
        return y

    @staticmethod
    def backward(ctx, dy):
        x, w = ctx.saved_tensors
        with torch.no_grad():
            dx, dw = ops.rmsnorm_bwd(dy.contiguous(), x, w, ctx.eps)
        return dx, dw, None
