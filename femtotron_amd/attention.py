"""Causal GQA attention over the layer's token-major qkv buffer (femtohip flash kernels).

q, k, v are the column ranges [0, Hq), [Hq, Hq+Hkv), [Hq+Hkv, Hq+2Hkv) of the
[T, Hq+2Hkv] projection output; gradients are written into the same column
ranges of one dqkv buffer, which the QKV weight-gradient and input-gradient
GEMMs then consume whole.
"""
from __future__ import annotations

import torch

from . import ops


def _split(buf: torch.Tensor, shp):
    hq, hkv = shp.hq, shp.hkv
    return buf[:, :hq], buf[:, hq:hq + hkv], buf[:, hq + hkv:hq + 2 * hkv]


def attn_fwd(qkv: torch.Tensor, batch: int, seq: int, shp, *, need_lse: bool):
    q, k, v = _split(qkv, shp)
    return ops.attn_fwd(q, k, v, batch, seq, shp.n_heads, shp.n_kv_heads, shp.head_dim, shp.scale,
                        need_lse=need_lse)


def attn_bwd(do: torch.Tensor, qkv: torch.Tensor, o: torch.Tensor, lse: torch.Tensor, batch: int,
             seq: int, shp) -> torch.Tensor:
    q, k, v = _split(qkv, shp)
    dqkv = torch.empty_like(qkv)
    dq, dk, dv = _split(dqkv, shp)
    ops.attn_bwd(q, k, v, o, do, lse, dq, dk, dv, batch, seq, shp.n_heads, shp.n_kv_heads,
                 shp.head_dim, shp.scale)
    return dqkv
