"""Causal GQA attention over the token-major qkv buffer.

Scaffold: torch SDPA, to be replaced by the femtohip flash-attention kernels.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def _views(qkv: torch.Tensor, batch: int, seq: int, shp):
    hq, hkv, hd = shp.hq, shp.hkv, shp.head_dim
    q = qkv[:, :hq].reshape(batch, seq, shp.n_heads, hd).transpose(1, 2)
    k = qkv[:, hq:hq + hkv].reshape(batch, seq, shp.n_kv_heads, hd).transpose(1, 2)
    v = qkv[:, hq + hkv:].reshape(batch, seq, shp.n_kv_heads, hd).transpose(1, 2)
    return q, k, v


def attn_fwd(qkv: torch.Tensor, batch: int, seq: int, shp, *, need_lse: bool):
    q, k, v = _views(qkv, batch, seq, shp)
    o = F.scaled_dot_product_attention(q, k, v, is_causal=True, enable_gqa=True, scale=shp.scale)
    o = o.transpose(1, 2).reshape(batch * seq, shp.hq).contiguous()
    return o, None


def attn_bwd(do: torch.Tensor, qkv: torch.Tensor, o: torch.Tensor, lse, batch: int, seq: int, shp):
    q, k, v = (t.detach().requires_grad_(True) for t in _views(qkv, batch, seq, shp))
    with torch.enable_grad():
        out = F.scaled_dot_product_attention(q, k, v, is_causal=True, enable_gqa=True,
                                             scale=shp.scale)
        g = do.view(batch, seq, shp.n_heads, shp.head_dim).transpose(1, 2)
        dq, dk, dv = torch.autograd.grad(out, (q, k, v), g)
    T = batch * seq
    return torch.cat((dq.transpose(1, 2).reshape(T, shp.hq), dk.transpose(1, 2).reshape(T, shp.hkv),
                      dv.transpose(1, 2).reshape(T, shp.hkv)), 1).contiguous()
