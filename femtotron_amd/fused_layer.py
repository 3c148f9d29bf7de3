"""Fused, activation-checkpointed Llama decoder layer (forward, recompute, backward).

This is the drop-in for one ``checkpoint_fn(LlamaDecoderLayer, hidden_states, ...)``
call of femtotron/training/activation_ckpt.py:78-86.  The forward keeps only the
layer input (exactly what torch.utils.checkpoint's ``_NoopSaveInputs`` keeps,
torch/utils/checkpoint.py:794-831); backward recomputes the layer forward up to
the gate/up projection (the down projection and final residual add are not
needed, mirroring the non-reentrant checkpoint's early stop; the SwiGLU product
p is written by the SwiGLU backward, which reads g and u anyway) and then runs
the layer's backward.

Layer arithmetic (transformers 5.15.0, models/llama/modeling_llama.py:284-325):
    y1 = RMSNorm1(x)
    q,k,v = y1 Wq^T, y1 Wk^T, y1 Wv^T          -> one GEMM over [Wq;Wk;Wv]
    q,k   = RoPE(q,k)                            (k: fh_rope_fwd over the kv heads; q: as the
                                                  attention forward loads it, fh_attn_fwd_rope;
                                                  or both in the GEMM's epilogue, fh_gemm_bf16_rope)
    o     = causal GQA attention(q,k,v)
    h     = x + o Wo^T;  z = RMSNorm2(h)         (fh_add_rmsnorm_fwd)
    g,u   = z Wg^T, z Wu^T                       -> one GEMM over [Wg;Wu]
    p     = silu(g)*u                            (fh_swiglu_fwd; in backward, fh_swiglu_bwd)
    out   = h + p Wd^T                           (residual add in the GEMM epilogue)

The projections' GEMMs go through femtotron_amd.projections (fh_gemm_bf16 or
the tuned library GEMM, per shape).

Token-major layout everywhere: activations are [T, features] with T = B*S, so
q/k/v are column ranges of one [T, Hq+2Hkv] buffer and attention reads and
writes heads as column blocks (no transposes); the attention backward writes
dq, dk, dv into the same column ranges of one dqkv buffer, which the q/k/v
weight-gradient and input-gradient GEMMs consume whole.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import ops
from .projections import (linear, linear_dgrad, linear_residual, linear_rope, linear_wgrad, linear_wgrad_group,
                          linear_wgrad_into)
from .weight_packing import packed


@dataclass(frozen=True)
class LayerShape:
    hidden: int
    n_heads: int
    n_kv_heads: int
    head_dim: int
    ffn: int
    eps1: float
    eps2: float
    scale: float

    @property
    def hq(self) -> int:
        return self.n_heads * self.head_dim

    @property
    def hkv(self) -> int:
        return self.n_kv_heads * self.head_dim


def _cat_rows(*ws: torch.Tensor) -> torch.Tensor:
    """[W1; W2; ...]: a view when the weights are packed contiguously
    (femtotron_amd.weight_packing), else a concatenated copy."""
    view = packed(*ws)
    return view if view is not None else torch.cat(ws, 0)


def _qkv_split(buf: torch.Tensor, shp: "LayerShape"):
    hq, hkv = shp.hq, shp.hkv
    return buf[:, :hq], buf[:, hq:hq + hkv], buf[:, hq + hkv:hq + 2 * hkv]


def attn_fwd(qkv: torch.Tensor, batch: int, seq: int, shp: "LayerShape", *, need_lse: bool,
             rope: tuple | None = None, write_q: bool = False):
    """Causal GQA attention over the [T, Hq+2Hkv] qkv buffer (fh_attn_fwd).  With
    rope=(cos, sin) q is rotated as it is loaded (fh_attn_fwd_rope) and, with
    write_q, written back rotated into qkv for the backward."""
    q, k, v = _qkv_split(qkv, shp)
    return ops.attn_fwd(q, k, v, batch, seq, shp.n_heads, shp.n_kv_heads, shp.head_dim, shp.scale,
                        need_lse=need_lse, rope=rope, q_out=q if rope is not None and write_q else None)


def qkv_attention(y: torch.Tensor, wqkv: torch.Tensor, batch: int, seq: int, shp: "LayerShape",
                  cos: torch.Tensor, sin: torch.Tensor, *, keep: bool):
    """q/k/v projection, RoPE and causal attention: (qkv, o, lse).  qkv holds the
    rotated q and k when keep (what the backward reads).  k is rotated by a pass
    over the kv heads, q as the attention forward loads it."""
    qkv, rotated = linear_rope(y, wqkv, shp.n_heads + shp.n_kv_heads, shp.head_dim, seq, cos, sin,
                               defer_heads=shp.n_heads)
    o, lse = attn_fwd(qkv, batch, seq, shp, need_lse=keep, rope=None if rotated else (cos, sin),
                      write_q=keep)
    return qkv, o, lse


def attn_bwd(do: torch.Tensor, qkv: torch.Tensor, o: torch.Tensor, lse: torch.Tensor, batch: int,
             seq: int, shp: "LayerShape", cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """dqkv [T, Hq+2Hkv] of RoPE then attn_fwd: the attention backward with the
    RoPE backward of dq and dk fused into their stores (fh_attn_bwd_rope)."""
    q, k, v = _qkv_split(qkv, shp)
    dqkv = torch.empty_like(qkv)
    dq, dk, dv = _qkv_split(dqkv, shp)
    ops.attn_bwd(q, k, v, o, do, lse, dq, dk, dv, batch, seq, shp.n_heads, shp.n_kv_heads,
                 shp.head_dim, shp.scale, rope=(cos, sin))
    return dqkv



class _Acts:
    """Recomputed activations the backward needs."""

    __slots__ = ("y1", "rstd1", "qkv", "o", "lse", "h", "rstd2", "z", "gu")


def layer_forward(x2: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, shp: LayerShape,
                  batch: int, seq: int, w: tuple, *, keep: bool):
    """Run the layer on x2 [T, H].  keep=False returns the output [T, H];
    keep=True (recompute) stops after the gate/up projection and returns _Acts
    (the backward's SwiGLU pass writes the product p itself)."""
    wq, wk, wv, wo, wg, wu, wd, w1, w2 = w
    T, H = x2.shape
    dev = x2.device
    acts = _Acts() if keep else None
    rstd1 = torch.empty(T, dtype=torch.float32, device=dev) if keep else None
    y1 = ops.rmsnorm_fwd(x2, w1, shp.eps1, rstd=rstd1)

    qkv, o, lse = qkv_attention(y1, _cat_rows(wq, wk, wv), batch, seq, shp, cos, sin, keep=keep)
    a = linear(o, wo)
    rstd2 = torch.empty(T, dtype=torch.float32, device=dev) if keep else None
    h, z = ops.add_rmsnorm_fwd(x2, a, w2, shp.eps2, rstd=rstd2)
    del a
    gu = linear(z, _cat_rows(wg, wu))
    F_ = shp.ffn
    if keep:
        acts.y1, acts.rstd1, acts.qkv, acts.o, acts.lse = y1, rstd1, qkv, o, lse
        acts.h, acts.rstd2, acts.z, acts.gu = h, rstd2, z, gu
        return acts
    p = ops.swiglu_fwd(gu[:, :F_], gu[:, F_:])
    del gu, qkv, o, y1, z
    return linear_residual(p, wd, h)


_side_streams: dict[int, torch.cuda.Stream] = {}
_use_side_stream = False


def set_wgrad_side_stream(enabled: bool) -> None:
    """Run the weight-gradient GEMMs on a side stream next to the
    input-gradient chain (True) or in series with it (False, the default:
    measured 1.4% faster on the TinyLlama step, because the side stream's GEMM
    workgroups, one per CU with 160 KB of LDS, wait for CUs the main stream's
    kernels hold and stretch both chains)."""
    global _use_side_stream
    _use_side_stream = bool(enabled)


def wgrad_side_stream() -> bool:
    return _use_side_stream


_accumulate_in_gemm = True


def set_grad_accumulation_in_gemm(enabled: bool) -> None:
    """Accumulate weight gradients into existing bf16 .grad tensors inside the
    weight-gradient GEMM (True, the default) instead of returning them for
    autograd to add.  The reference's training loop keeps .grad between
    steps (GradAccumulator.reset zeroes it in place,
    femtotron/training/grad_accumulator.py:55-60, and micro-batches after the
    first accumulate into it, :24-36), so every backward but the very first
    adds into an existing gradient; done in the GEMM's epilogue it costs no
    separate pass over the 9 gradients (3 x their bytes per layer).  Same bits
    as autograd's addition: grad + to_bf16(dW), rounded."""
    global _accumulate_in_gemm
    _accumulate_in_gemm = bool(enabled)


def grad_accumulation_in_gemm() -> bool:
    return _accumulate_in_gemm


def grad_target(*params: torch.Tensor) -> torch.Tensor | None:
    """The existing gradients of `params` (the parameters one weight-gradient
    GEMM produces, its output rows in this order) as one [rows, cols] tensor,
    when the GEMM can accumulate into them: every .grad present, bf16,
    contiguous, of the parameter's shape, laid out row-contiguously in one
    buffer (as autograd leaves them after a first backward, which stores the
    row views of the GEMM output), and no gradient hooks on the parameters
    (their AccumulateGrad step is what the in-place accumulation skips).
    None otherwise."""
    if not _accumulate_in_gemm:
        return None
    gs = []
    for p in params:
        g = p.grad
        if (g is None or g.dtype != torch.bfloat16 or g.shape != p.shape or g.requires_grad
                or p._backward_hooks or getattr(p, "_post_accumulate_grad_hooks", None)):
            return None
        gs.append(g)
    return packed(*gs)


class _WgradStream:
    """Weight-gradient GEMMs, on a side stream (default priority) when
    set_wgrad_side_stream(True), else in order on the main stream.

    dW = dY^T X feeds nothing else in the layer's backward, so it can run next
    to the input-gradient chain (dgrad GEMMs, the attention backward, the norm
    backward) instead of in series with it.  Each GEMM waits for the main
    stream's work queued so far; its operands are marked as used by the side
    stream (so the caching allocator does not hand their memory back to the
    main stream early) and its result as used by the main stream; join() makes
    the main stream wait for every queued weight-gradient GEMM."""

    def __init__(self, device: torch.device):
        self.main = torch.cuda.current_stream(device)
        side = _side_streams.get(device.index)
        if side is None:
            side = _side_streams[device.index] = torch.cuda.Stream(device=device)
        self.side = side

    def mm_tn(self, a: torch.Tensor, b: torch.Tensor, into: torch.Tensor | None = None) -> torch.Tensor | None:
        """a^T @ b on the side stream (projections.linear_wgrad); on the main
        stream when the side stream is switched off.  With `into` (grad_target)
        the product is accumulated into it where the hand-written GEMM runs
        (returns None), else returned."""
        if not _use_side_stream:
            if into is not None and linear_wgrad_into(a, b, into):
                return None
            return linear_wgrad(a, b)
        self.side.wait_stream(self.main)
        with torch.cuda.stream(self.side):
            done = into is not None and linear_wgrad_into(a, b, into)
            out = None if done else linear_wgrad(a, b)
        a.record_stream(self.side)
        b.record_stream(self.side)
        if out is not None:
            out.record_stream(self.main)
        return out

    def mm_tn_group(self, items: list) -> list | None:
        """linear_wgrad_group (several a^T @ b in one launch) on the side stream,
        or in order on the main stream; None when the group is not taken."""
        if not _use_side_stream:
            return linear_wgrad_group(items)
        self.side.wait_stream(self.main)
        with torch.cuda.stream(self.side):
            outs = linear_wgrad_group(items)
        for a, b, _ in items:
            a.record_stream(self.side)
            b.record_stream(self.side)
        for o in outs or ():
            if o is not None:
                o.record_stream(self.main)
        return outs

    def join(self) -> None:
        if _use_side_stream:
            self.main.wait_stream(self.side)


def split_rows(dw: torch.Tensor | None, *rows: int) -> tuple:
    """Row blocks of a packed weight gradient (all None where it was
    accumulated into the existing gradients)."""
    if dw is None:
        return (None,) * len(rows)
    out, r = [], 0
    for n in rows:
        out.append(dw[r:r + n])
        r += n
    return tuple(out)


def layer_backward(dout2: torch.Tensor, x2: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                   shp: LayerShape, batch: int, seq: int, w: tuple, acts: _Acts):
    """dx and the 9 weight gradients; a weight gradient accumulated into the
    parameter's existing .grad inside its GEMM (grad_target) comes back as None."""
    wq, wk, wv, wo, wg, wu, wd, w1, w2 = w
    F_ = shp.ffn
    wg_stream = _WgradStream(dout2.device)
    # MLP: m = p Wd^T.  The SwiGLU backward also writes p (into dp's buffer,
    # each element read before it is overwritten) for the down projection's
    # weight gradient, so the recompute stops before the product.
    dp = linear_dgrad(dout2, wd)
    dgu = torch.empty_like(acts.gu)
    ops.swiglu_bwd(dp, acts.gu[:, :F_], acts.gu[:, F_:], dgu[:, :F_], dgu[:, F_:], p_out=dp)
    acts.gu = None
    dwgu = wg_stream.mm_tn(dgu, acts.z, grad_target(wg, wu))
    dz = linear_dgrad(dgu, _cat_rows(wg, wu))
    del dgu
    acts.z = None
    # post-attention norm + residual: dh = dout + RMSNorm2^T(dz)
    dh, dw2 = ops.rmsnorm_bwd(dz, acts.h, w2, shp.eps2, rstd=acts.rstd2, dres=dout2)
    del dz
    acts.h = None
    # attention output projection
    do = linear_dgrad(dh, wo)
    dqkv = attn_bwd(do, acts.qkv, acts.o, acts.lse, batch, seq, shp, cos, sin)
    del do
    acts.lse = acts.qkv = None
    # The down, o and q/k/v weight gradients (few output tiles each, the same
    # tokens) run as one grouped GEMM once dqkv exists.
    done = wg_stream.mm_tn_group([(dout2, dp, grad_target(wd)), (dh, acts.o, grad_target(wo)),
                                  (dqkv, acts.y1, grad_target(wq, wk, wv))])
    if done is None:  # not all hand-written: one by one
        dwd = wg_stream.mm_tn(dout2, dp, grad_target(wd))
        dwo = wg_stream.mm_tn(dh, acts.o, grad_target(wo))
        dwqkv = wg_stream.mm_tn(dqkv, acts.y1, grad_target(wq, wk, wv))
    else:
        dwd, dwo, dwqkv = done
    del dp
    acts.o = None
    dy1 = linear_dgrad(dqkv, _cat_rows(wq, wk, wv))
    del dqkv
    acts.y1 = None
    dx, dw1 = ops.rmsnorm_bwd(dy1, x2, w1, shp.eps1, rstd=acts.rstd1, dres=dh)
    wg_stream.join()
    dwq, dwk, dwv = split_rows(dwqkv, shp.hq, shp.hkv, shp.hkv)
    dwg, dwu = split_rows(dwgu, F_, F_)
    return dx, (dwq, dwk, dwv, dwo, dwg, dwu, dwd, dw1, dw2)


class FusedDecoderLayerFunction(torch.autograd.Function):
    """autograd node for one checkpointed decoder layer.

    Saved for backward: the layer input x (plus references to cos/sin and the
    weights, which the caller keeps alive anyway).  Nothing else survives the
    forward."""

    @staticmethod
    def forward(ctx, x, cos, sin, shp, wq, wk, wv, wo, wg, wu, wd, w1, w2):
        B, S, H = x.shape
        w = (wq, wk, wv, wo, wg, wu, wd, w1, w2)
        out = layer_forward(x.reshape(B * S, H), cos, sin, shp, B, S, w, keep=False)
        ctx.save_for_backward(x, cos, sin, *w)
        ctx.shp = shp
        return out.view(B, S, H)

    @staticmethod
    def backward(ctx, dout):
        x, cos, sin, *w = ctx.saved_tensors
        shp = ctx.shp
        B, S, H = x.shape
        x2 = x.reshape(B * S, H)
        with torch.no_grad():
            acts = layer_forward(x2, cos, sin, shp, B, S, tuple(w), keep=True)
            dx, dws = layer_backward(dout.contiguous().view(B * S, H), x2, cos, sin, shp, B, S,
                                     tuple(w), acts)
        return (dx.view(B, S, H), None, None, None, *dws)
