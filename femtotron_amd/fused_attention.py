"""Fused self-attention for decoder layers whose attention is not checkpointed.

Under selective activation checkpointing (the "llama_mlp_and_norms" preset,
femtotron/scripts/presets.py:45-62, policy
``any_of(by_class_name("LlamaMLP"), by_class_name("LlamaRMSNorm"))`` from
femtotron/training/ckpt_policy.py:70-124) ``checkpoint_fn`` only receives the
MLPs and norms.  Each layer's attention runs outside it as HF's LlamaAttention
(transformers 5.15.0 models/llama/modeling_llama.py:235-281: the q/k/v
projections, apply_rotary_pos_emb, sdpa_attention_forward with is_causal, the
o projection) with its activations stored for backward.

``fuse_attention(model)`` gives every such module a forward on the femtohip
kernels.  The module, its parameters and its state-dict keys stay as they are:

    qkv    = y [Wq;Wk;Wv]^T      one GEMM over the packed weights
    q, k   = RoPE(q, k)          k: fh_rope_fwd; q: as attention loads it (or both in the GEMM)
    o, lse = attention(qkv)      fh_attn_fwd_rope, causal GQA
    a      = o Wo^T

It saves y, the rotated qkv, o and lse for backward, as the stock path saves
the projections' input and SDPA's q, k, v, output and log-sum-exp.  The
backward takes the same steps as the attention half of the fused layer: the o
and q/k/v weight gradients (in series, or on the optional side stream), and the
input-gradient chain o-projection -> fh_attn_bwd_rope (RoPE backward in the
dq/dk stores) -> q/k/v projection.

A call the kernels do not cover runs the module's own forward: off a HIP
device, another dtype, autocast, an attention mask, a KV cache, attention
dropout while training, projection biases or tensor-parallel size > 1, hooks
on the projections, or an attention implementation other than sdpa (HF's eager
attention, and an unset implementation, attend in both directions when no mask
is given, where the kernels are causal).
Under full activation checkpointing the fused decoder layer never calls the
attention module, so the two compose.
"""
from __future__ import annotations

import threading
import types

import torch

from . import _lib, ops
from .fused_checkpoint import _aligned, _causal_attention_reason, _check_params, _linear_weight
from .fused_layer import (LayerShape, _WgradStream, _cat_rows, attn_bwd, grad_target, qkv_attention,
                          split_rows)
from .projections import linear, linear_dgrad

_ACCEPTED_KWARGS = {"position_ids", "use_cache", "cache_position"}
_counts_lock = threading.Lock()
_counts = {"fused": 0, "fallback": 0}
_last_reason: list[str] = [""]


def attention_dispatch_counts() -> dict[str, int]:
    """How many calls of fused attention modules took the kernels vs. the module's own forward."""
    with _counts_lock:
        return dict(_counts)


def reset_attention_dispatch_counts() -> None:
    with _counts_lock:
        _counts["fused"] = 0
        _counts["fallback"] = 0


def last_attention_fallback_reason() -> str:
    return _last_reason[0]


class FusedAttentionFunction(torch.autograd.Function):
    """a = attention(RoPE(y Wqkv^T)) Wo^T for y [B, S, H]; saved: y, qkv, o, lse."""

    @staticmethod
    def forward(ctx, y, cos, sin, shp, wq, wk, wv, wo):
        B, S, H = y.shape
        y2 = y.reshape(B * S, H)
        qkv, o, lse = qkv_attention(y2, _cat_rows(wq, wk, wv), B, S, shp, cos, sin, keep=True)
        a = linear(o, wo)
        ctx.save_for_backward(y, cos, sin, qkv, o, lse, wq, wk, wv, wo)
        ctx.shp = shp
        return a.view(B, S, H)

    @staticmethod
    def backward(ctx, da):
        y, cos, sin, qkv, o, lse, wq, wk, wv, wo = ctx.saved_tensors
        shp = ctx.shp
        B, S, H = y.shape
        da2 = da.contiguous().view(B * S, H)
        with torch.no_grad():
            side = _WgradStream(da2.device)
            dwo = side.mm_tn(da2, o, grad_target(wo))
            do = linear_dgrad(da2, wo)
            dqkv = attn_bwd(do, qkv, o, lse, B, S, shp, cos, sin)
            del do
            dwqkv = side.mm_tn(dqkv, y.reshape(B * S, H), grad_target(wq, wk, wv))
            dy = linear_dgrad(dqkv, _cat_rows(wq, wk, wv))
            side.join()
        return (dy.view(B, S, H), None, None, None, *split_rows(dwqkv, shp.hq, shp.hkv, shp.hkv), dwo)


def _projection_hooks(attn: torch.nn.Module) -> bool:
    """Hooks that the module's own forward would run and the fused one would not:
    on the projections (or deeper), or global module hooks."""
    for m in attn.modules():
        if m is attn:
            continue
        if (m._forward_hooks or m._forward_pre_hooks or m._backward_hooks
                or getattr(m, "_backward_pre_hooks", None)):
            return True
    g = torch.nn.modules.module
    return bool(g._global_forward_hooks or g._global_forward_pre_hooks
                or g._global_backward_hooks or getattr(g, "_global_backward_pre_hooks", None))


def _plan(attn, y, position_embeddings, attention_mask, past_key_values, kwargs):
    """(shape, weights) if the call can run on the kernels, else a reason string."""
    if set(kwargs) - _ACCEPTED_KWARGS:
        return f"unsupported kwargs {sorted(set(kwargs) - _ACCEPTED_KWARGS)}"
    if not isinstance(y, torch.Tensor) or not y.is_cuda:
        return "hidden_states not on a HIP device"
    if y.dtype not in (torch.bfloat16, torch.float32):
        return f"dtype {y.dtype}"
    if y.dim() != 3:
        return "hidden_states must be [B, S, H]"
    if torch.is_autocast_enabled():
        return "autocast active"
    if attention_mask is not None:
        return "explicit attention mask"
    if past_key_values is not None:
        return "KV cache"
    reason = _causal_attention_reason(attn)
    if reason:
        return reason
    if attn.training and float(getattr(attn, "attention_dropout", 0.0) or 0.0) > 0.0:
        return "attention dropout"
    if _projection_hooks(attn):
        return "hooks on the projections"
    ws = [_linear_weight(getattr(attn, n, None)) for n in ("q_proj", "k_proj", "v_proj", "o_proj")]
    if any(w is None for w in ws):
        return "projection with bias or tensor-parallel size > 1"
    if not (isinstance(position_embeddings, (tuple, list)) and len(position_embeddings) == 2):
        return "position_embeddings (cos, sin) required"
    B, S, H = y.shape
    hd = int(attn.head_dim)
    if hd not in (32, 64, 128):
        return "head_dim must be 32, 64 or 128"
    nh, nkv = ws[0].shape[0] // hd, ws[1].shape[0] // hd
    cos, sin = position_embeddings
    for t in (cos, sin):
        if not isinstance(t, torch.Tensor) or t.device != y.device or t.dtype != y.dtype:
            return "cos/sin must match hidden_states' device and dtype"
        if t.dim() != 3 or t.shape[1] != S or t.shape[2] != hd or t.shape[0] not in (1, B):
            return "cos/sin must be [1|B, S, head_dim]"
    reason = _check_params(y, ws)
    if reason:
        return reason
    if ws[0].shape != (nh * hd, H) or ws[1].shape != (nkv * hd, H) or ws[2].shape != (nkv * hd, H):
        return "unexpected q/k/v weight shapes"
    if ws[3].shape != (H, nh * hd):
        return "unexpected o weight shape"
    if nkv == 0 or nh % nkv:
        return "n_heads not a multiple of n_kv_heads"
    if H % 8:
        return "hidden % 8 required"
    shp = LayerShape(hidden=H, n_heads=nh, n_kv_heads=nkv, head_dim=hd, ffn=0, eps1=0.0, eps2=0.0,
                     scale=float(attn.scaling))
    return shp, ws


def _fused_forward(self, hidden_states, position_embeddings=None, attention_mask=None,
                   past_key_values=None, **kwargs):
    """LlamaAttention.forward's contract: returns (attn_output [B, S, H], None)."""
    plan = _plan(self, hidden_states, position_embeddings, attention_mask, past_key_values, kwargs)
    if isinstance(plan, str):
        _last_reason[0] = plan
        with _counts_lock:
            _counts["fallback"] += 1
        return type(self).forward(self, hidden_states, position_embeddings, attention_mask,
                                  past_key_values, **kwargs)
    _lib.lib()  # raises if the HIP library is not built: no silent fallback on GPU
    shp, ws = plan
    cos, sin = position_embeddings
    with _counts_lock:
        _counts["fused"] += 1
    out = FusedAttentionFunction.apply(_aligned(hidden_states), _aligned(cos), _aligned(sin), shp, *ws)
    return out, None


def _is_llama_attention(mod: torch.nn.Module) -> bool:
    from transformers.models.llama import modeling_llama as hf
    return getattr(type(mod), "forward", None) is hf.LlamaAttention.forward


def fuse_attention(model: torch.nn.Module) -> int:
    """Give every LlamaAttention in `model` (unmodified forward, not already
    fused) the fused forward; returns how many modules were changed."""
    n = 0
    for mod in model.modules():
        if _is_llama_attention(mod) and "forward" not in mod.__dict__:
            mod.forward = types.MethodType(_fused_forward, mod)
            n += 1
    return n


def unfuse_attention(model: torch.nn.Module) -> int:
    """Undo fuse_attention; returns how many modules were restored."""
    n = 0
    for mod in model.modules():
        fwd = mod.__dict__.get("forward")
        if isinstance(fwd, types.MethodType) and fwd.__func__ is _fused_forward:
            del mod.forward
            n += 1
    return n
