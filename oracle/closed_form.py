"""ORACLE — test infrastructure only.  Closed-form fp64 NumPy statements of each
fused op of the checkpointed Llama layer, forward AND backward, written from the
mathematics (not from autograd), so they can check both the HIP kernels and the
autograd-derived gradients of oracle/torch_llama.py.

Reference arithmetic restated (transformers 5.15.0):
  rmsnorm_*   LlamaRMSNorm            models/llama/modeling_llama.py:62-67
  rope_*      apply_rotary_pos_emb    models/llama/modeling_llama.py:130-160
  swiglu_*    act_fn(gate)*up, SiLU   models/llama/modeling_llama.py:174-176
  attention_* causal SDPA with GQA    integrations/sdpa_attention.py:79-166,
                                      head map of repeat_kv modeling_llama.py:179-188

Pinning (tests/test_oracle.py): central finite differences in fp64 for every
backward; invariants (RMS of the normalised row is 1; RoPE at position 0 is
the identity and preserves each pair's norm; silu(0) = 0; attention at S = 1
returns v; causal rows ignore future keys); and agreement with torch autograd.
"""
from __future__ import annotations

import numpy as np


# ------------------------------------------------------------------ RMSNorm
def rmsnorm_fwd(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    r = 1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
    return w * (x * r)


def rmsnorm_bwd(dy: np.ndarray, x: np.ndarray, w: np.ndarray, eps: float):
    """d/dx and d/dw of sum(dy * rmsnorm_fwd(x, w)).
    With r = (mean(x^2)+eps)^-1/2, n = x r, dn = dy w:
        dx = r (dn - n mean(dn n)),   dw = sum_rows dy n."""
    H = x.shape[-1]
    r = 1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
    n = x * r
    dn = dy * w
    dx = r * (dn - n * np.sum(dn * n, axis=-1, keepdims=True) / H)
    dw = np.sum((dy * n).reshape(-1, H), axis=0)
    return dx, dw


# --------------------------------------------------------------------- RoPE
def rope_angles(positions: np.ndarray, head_dim: int, theta: float) -> np.ndarray:
    """angle[p, i] = p * theta^(-2i/d) for i < d/2."""
    inv = theta ** (-np.arange(0, head_dim, 2, dtype=np.float64) / head_dim)
    return positions[:, None].astype(np.float64) * inv[None, :]


def rope_fwd(x: np.ndarray, ang: np.ndarray) -> np.ndarray:
    """x [..., S, d] rotated pairwise: (x_i, x_{i+d/2}) by angle ang[s, i]."""
    h = x.shape[-1] // 2
    c, s = np.cos(ang), np.sin(ang)
    a, b = x[..., :h], x[..., h:]
    return np.concatenate((a * c - b * s, b * c + a * s), axis=-1)


def rope_bwd(g: np.ndarray, ang: np.ndarray) -> np.ndarray:
    """Transpose of the rotation = rotation by -angle."""
    return rope_fwd(g, -ang)


# ------------------------------------------------------------------- SwiGLU
def _sig(x):
    return 1.0 / (1.0 + np.exp(-x))


def swiglu_fwd(g: np.ndarray, u: np.ndarray) -> np.ndarray:
    return g * _sig(g) * u


def swiglu_bwd(dp: np.ndarray, g: np.ndarray, u: np.ndarray):
    """dg = dp u sig(g) (1 + g (1 - sig(g))),  du = dp silu(g)."""
    s = _sig(g)
    return dp * u * s * (1.0 + g * (1.0 - s)), dp * g * s


# ---------------------------------------------------------------- attention
def attention_fwd(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float):
    """q [B,nh,S,d], k/v [B,nkv,S,d]; q head i uses kv head i // (nh/nkv).
    Returns (o [B,nh,S,d], lse [B,nh,S]) with lse = log sum_j exp(scale q.k_j), j <= i."""
    B, nh, S, d = q.shape
    rep = nh // k.shape[1]
    kk = np.repeat(k, rep, axis=1)
    vv = np.repeat(v, rep, axis=1)
    s = np.einsum("bhid,bhjd->bhij", q, kk) * scale
    s = np.where(np.triu(np.ones((S, S), dtype=bool), 1), -np.inf, s)
    m = s.max(-1, keepdims=True)
    p = np.exp(s - m)
    l = p.sum(-1, keepdims=True)
    p /= l
    return np.einsum("bhij,bhjd->bhid", p, vv), (m + np.log(l))[..., 0]


def attention_bwd(do: np.ndarray, q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float):
    """Softmax-attention gradients: with P the probabilities, dP = dO V^T,
    dS = P (dP - rowsum(dO o)), dQ = scale dS K, dK = scale dS^T Q, dV = P^T dO;
    K/V gradients of a kv head sum over the q heads that share it."""
    B, nh, S, d = q.shape
    nkv = k.shape[1]
    rep = nh // nkv
    kk = np.repeat(k, rep, axis=1)
    vv = np.repeat(v, rep, axis=1)
    o, lse = attention_fwd(q, k, v, scale)
    s = np.einsum("bhid,bhjd->bhij", q, kk) * scale
    mask = np.triu(np.ones((S, S), dtype=bool), 1)
    p = np.where(mask, 0.0, np.exp(s - lse[..., None]))
    dp = np.einsum("bhid,bhjd->bhij", do, vv)
    delta = np.sum(do * o, axis=-1, keepdims=True)
    ds = p * (dp - delta)
    dq = scale * np.einsum("bhij,bhjd->bhid", ds, kk)
    dk_full = scale * np.einsum("bhij,bhid->bhjd", ds, q)
    dv_full = np.einsum("bhij,bhid->bhjd", p, do)
    dk = dk_full.reshape(B, nkv, rep, S, d).sum(2)
    dv = dv_full.reshape(B, nkv, rep, S, d).sum(2)
    return dq, dk, dv


def finite_diff_grad(f, x: np.ndarray, dy: np.ndarray, h: float = 1e-6) -> np.ndarray:
    """Central differences of sum(dy * f(x)) w.r.t. every entry of x (fp64; tiny x only)."""
    g = np.zeros_like(x)
    flat = x.reshape(-1)
    gf = g.reshape(-1)
    for i in range(flat.size):
        old = flat[i]
        flat[i] = old + h
        fp = np.sum(dy * f(x))
        flat[i] = old - h
        fm = np.sum(dy * f(x))
        flat[i] = old
        gf[i] = (fp - fm) / (2 * h)
    return g
