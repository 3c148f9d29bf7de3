"""``fused_checkpoint``: a ``checkpoint_fn`` for ``apply_activation_checkpointing``.

Signature-compatible with ``torch.utils.checkpoint.checkpoint`` (the contract of
``CheckpointFn`` at femtotron/training/activation_ckpt.py:25-26).  A call on a HIP
device, in the configuration the reference runs (bf16 or fp32, no attention
mask, no KV cache, no hooks, no biases, SiLU MLP, TP size 1), whose module is

* a Llama decoder layer (full activation checkpointing, the
  "llama_decoder_layer" preset) runs as ``FusedDecoderLayerFunction``;
* a LlamaMLP or a LlamaRMSNorm (selective checkpointing, the
  "llama_mlp_and_norms" preset) runs as ``FusedMLPFunction`` /
  ``FusedRMSNormFunction``;

all on the femtohip kernels.  Any other call is handed to
``torch.utils.checkpoint.checkpoint`` with the same arguments, i.e. it behaves
exactly as the reference wrapper.

On a HIP device the fused path never degrades silently: if ``libfemtohip.so`` is
missing the call raises.
"""
from __future__ import annotations

import threading
from typing import Any

import torch
from torch.utils.checkpoint import checkpoint as _torch_checkpoint

from . import _lib
from .fused_layer import FusedDecoderLayerFunction, LayerShape
from .fused_parts import FusedMLPFunction, FusedRMSNormFunction

_KNOWN_KWARGS = {"attention_mask", "position_embeddings", "position_ids", "past_key_values",
                 "use_cache", "cache_position"}

_counts_lock = threading.Lock()
_counts = {"fused": 0, "fallback": 0}
_last_fallback_reason: list[str] = [""]


def dispatch_counts() -> dict[str, int]:
    """How many checkpointed calls took the fused path vs. the stock one."""
    with _counts_lock:
        return dict(_counts)


def reset_dispatch_counts() -> None:
    with _counts_lock:
        _counts["fused"] = 0
        _counts["fallback"] = 0


def last_fallback_reason() -> str:
    return _last_fallback_reason[0]


def _bump(key: str) -> None:
    with _counts_lock:
        _counts[key] += 1


def _linear_weight(mod: Any) -> torch.Tensor | None:
    """[out, in] weight of an nn.Linear or of femtotron's Column/RowParallelLinear at TP=1."""
    w = getattr(mod, "weight", None)
    if not isinstance(w, torch.Tensor) or getattr(mod, "bias", None) is not None:
        return None
    ws = getattr(mod, "world_size", 1)  # femtotron TP wrappers (tensor_parallel/linear.py:52-54)
    if ws != 1:
        return None
    if getattr(mod, "gather_output", False) or getattr(mod, "scatter_input", False):
        return None
    return w


def _has_hooks(mod: torch.nn.Module) -> bool:
    for m in mod.modules():
        if (m._forward_hooks or m._forward_pre_hooks or m._backward_hooks
                or getattr(m, "_backward_pre_hooks", None)):
            return True
    g = torch.nn.modules.module
    return bool(g._global_forward_hooks or g._global_forward_pre_hooks
                or g._global_backward_hooks or getattr(g, "_global_backward_pre_hooks", None))


def _check_input(args: tuple):
    """The single hidden_states argument, or a reason string."""
    if len(args) != 1 or not isinstance(args[0], torch.Tensor):
        return "hidden_states must be the only positional argument"
    x = args[0]
    if not x.is_cuda:
        return "hidden_states not on a HIP device"
    if x.dtype not in (torch.bfloat16, torch.float32):
        return f"dtype {x.dtype}"
    if torch.is_autocast_enabled():
        return "autocast active"
    return x


def _causal_attention_reason(attn: Any) -> str | None:
    """None if the stock attention module computes causal attention when it is
    called without a mask (the only calls that reach the kernels), else why not.

    HF picks the attention function by ``config._attn_implementation``
    (modeling_llama.py:258-260): "sdpa" is causal without a mask as long as the
    module's ``is_causal`` holds (integrations/sdpa_attention.py:126-142), but
    "eager", and an unset implementation (which ``get_interface`` resolves to
    eager), apply no mask at all without one (modeling_llama.py:202-204): every
    query attends to every key.  The kernels are causal, so those fall back."""
    cfg = getattr(attn, "config", None)
    if cfg is None:
        return "attention has no config"
    impl = getattr(cfg, "_attn_implementation", None)
    if impl != "sdpa":
        if impl in ("eager", None):
            return f"attention implementation {impl!r} without a mask is not causal"
        return f"attention implementation {impl!r}"
    if not getattr(attn, "is_causal", True):
        return "attention module is not causal"
    return None


def _check_params(x: torch.Tensor, weights) -> str | None:
    for t in weights:
        if t.device != x.device or t.dtype != x.dtype or not t.is_contiguous():
            return "weights must be contiguous, on hidden_states' device, in its dtype"
        if t.data_ptr() % 16:
            return "weights must be 16-byte aligned"
    return None


def _aligned(x: torch.Tensor) -> torch.Tensor:
    x = x.contiguous()
    return x if x.data_ptr() % 16 == 0 else x.clone()


def _plan(module: Any, args: tuple, kwargs: dict):
    """Return (autograd Function, its apply() arguments) if the call can be fused,
    else a reason string."""
    kind = _kind(module)
    if kind is None:
        return "module is not an unmodified Llama decoder layer, MLP or RMSNorm"
    x = _check_input(args)
    if isinstance(x, str):
        return x
    if _has_hooks(module):
        return "module hooks installed"
    if kind == "mlp":
        return _plan_mlp(module, x, kwargs)
    if kind == "norm":
        return _plan_norm(module, x, kwargs)
    return _plan_layer(module, x, kwargs)


def _plan_mlp(mlp: Any, x: torch.Tensor, kwargs: dict):
    if kwargs:
        return f"unsupported kwargs {sorted(kwargs)}"
    cfg = getattr(mlp, "config", None)
    if cfg is not None and getattr(cfg, "hidden_act", "silu") != "silu":
        return "MLP activation is not SiLU"
    ws = [_linear_weight(getattr(mlp, n, None)) for n in ("gate_proj", "up_proj", "down_proj")]
    if any(w is None for w in ws):
        return "projection with bias or tensor-parallel size > 1"
    wg, wu, wd = ws
    H = x.shape[-1]
    F_ = wg.shape[0]
    reason = _check_params(x, ws)
    if reason:
        return reason
    if x.dim() < 2 or wg.shape != (F_, H) or wu.shape != (F_, H) or wd.shape != (H, F_):
        return "unexpected MLP weight shapes"
    if H % 8 or F_ % 8:
        return "hidden % 8 and ffn % 8 required"
    return FusedMLPFunction, (_aligned(x), wg, wu, wd)


def _plan_norm(norm: Any, x: torch.Tensor, kwargs: dict):
    if kwargs:
        return f"unsupported kwargs {sorted(kwargs)}"
    w = getattr(norm, "weight", None)
    if not isinstance(w, torch.Tensor):
        return "RMSNorm without weight"
    reason = _check_params(x, (w,))
    if reason:
        return reason
    H = x.shape[-1]
    if w.shape != (H,):
        return "RMSNorm weight size != last dim"
    if H % 8 or H > 8192:
        return "hidden % 8 and hidden <= 8192 required"
    return FusedRMSNormFunction, (_aligned(x), w, float(norm.variance_epsilon))


def _plan_layer(module: Any, x: torch.Tensor, kwargs: dict):
    if x.dim() != 3:
        return "hidden_states must be [B, S, H]"
    if set(kwargs) - _KNOWN_KWARGS:
        return f"unsupported kwargs {sorted(set(kwargs) - _KNOWN_KWARGS)}"
    if kwargs.get("attention_mask") is not None:
        return "explicit attention mask"
    if kwargs.get("past_key_values") is not None or kwargs.get("use_cache"):
        return "KV cache"
    pe = kwargs.get("position_embeddings")
    if not (isinstance(pe, (tuple, list)) and len(pe) == 2):
        return "position_embeddings (cos, sin) required"
    cos, sin = pe
    attn = getattr(module, "self_attn", None)
    mlp = getattr(module, "mlp", None)
    ln1 = getattr(module, "input_layernorm", None)
    ln2 = getattr(module, "post_attention_layernorm", None)
    if attn is None or mlp is None or ln1 is None or ln2 is None:
        return "not a Llama decoder layer"
    reason = _causal_attention_reason(attn)
    if reason:
        return reason
    if getattr(attn.config, "hidden_act", "silu") != "silu":
        return "MLP activation is not SiLU"
    if module.training and float(getattr(attn, "attention_dropout", 0.0) or 0.0) > 0.0:
        return "attention dropout"
    ws = [_linear_weight(getattr(attn, n, None)) for n in ("q_proj", "k_proj", "v_proj", "o_proj")]
    ws += [_linear_weight(getattr(mlp, n, None)) for n in ("gate_proj", "up_proj", "down_proj")]
    if any(w is None for w in ws):
        return "projection with bias or tensor-parallel size > 1"
    w1, w2 = getattr(ln1, "weight", None), getattr(ln2, "weight", None)
    if not isinstance(w1, torch.Tensor) or not isinstance(w2, torch.Tensor):
        return "RMSNorm without weight"
    weights = (*ws, w1, w2)
    B, S, H = x.shape
    hd = int(attn.head_dim)
    nh = ws[0].shape[0] // hd
    nkv = ws[1].shape[0] // hd
    F_ = ws[4].shape[0]
    for t in (cos, sin):
        if not isinstance(t, torch.Tensor) or t.device != x.device or t.dtype != x.dtype:
            return "cos/sin must match hidden_states' device and dtype"
        if t.dim() != 3 or t.shape[1] != S or t.shape[2] != hd or t.shape[0] not in (1, B):
            return "cos/sin must be [1|B, S, head_dim]"
    reason = _check_params(x, weights)
    if reason:
        return reason
    if ws[0].shape != (nh * hd, H) or ws[1].shape != (nkv * hd, H) or ws[2].shape != (nkv * hd, H):
        return "unexpected q/k/v weight shapes"
    if ws[3].shape != (H, nh * hd) or ws[5].shape != (F_, H) or ws[6].shape != (H, F_):
        return "unexpected o/mlp weight shapes"
    if nkv == 0 or nh % nkv:
        return "n_heads not a multiple of n_kv_heads"
    if hd not in (32, 64, 128):
        return f"head_dim {hd} (the attention kernels take 32, 64 or 128)"
    if H % 8 or F_ % 8 or H > 8192:
        return "hidden % 8, ffn % 8 and hidden <= 8192 required"
    shp = LayerShape(hidden=H, n_heads=nh, n_kv_heads=nkv, head_dim=hd, ffn=F_,
                     eps1=float(ln1.variance_epsilon), eps2=float(ln2.variance_epsilon),
                     scale=float(attn.scaling))
    return FusedDecoderLayerFunction, (_aligned(x), _aligned(cos), _aligned(sin), shp, *weights)


_KINDS: dict = {}


def _kind(module: Any) -> str | None:
    """'layer' / 'mlp' / 'norm' for HF's Llama decoder layer, MLP and RMSNorm
    (or a subclass that keeps their forward), else None."""
    if not _KINDS:
        from transformers.models.llama import modeling_llama as hf
        _KINDS[hf.LlamaDecoderLayer.forward] = "layer"
        _KINDS[hf.LlamaMLP.forward] = "mlp"
        _KINDS[hf.LlamaRMSNorm.forward] = "norm"
    return _KINDS.get(getattr(type(module), "forward", None))


def fused_checkpoint(function, *args, use_reentrant: bool | None = None,
                     preserve_rng_state: bool = True, debug: bool = False, **kwargs):
    """Drop-in for ``torch.utils.checkpoint.checkpoint`` as a ``checkpoint_fn``.

    ``debug`` is accepted and has no effect on the fused path (the reference uses it
    only to format CheckpointError messages); ``preserve_rng_state`` is moot there
    because the fused layer draws no random numbers.  As in torch, reentrant mode
    together with ``debug`` raises ValueError (torch/utils/checkpoint.py:499-504)."""
    if use_reentrant and debug:
        raise ValueError("debug=True is only supported with use_reentrant=False")
    torch_only = {k: kwargs.pop(k) for k in ("context_fn", "determinism_check", "early_stop")
                  if k in kwargs}
    plan = _plan(function, args, kwargs)
    if isinstance(plan, str):
        _last_fallback_reason[0] = plan
        _bump("fallback")
        return _torch_checkpoint(function, *args, use_reentrant=use_reentrant,
                                 preserve_rng_state=preserve_rng_state, debug=debug,
                                 **torch_only, **kwargs)
    _lib.lib()  # raises if the HIP library is not built: no silent fallback on GPU
    fn, fn_args = plan
    _bump("fused")
    return fn.apply(*fn_args)
