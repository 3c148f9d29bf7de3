"""Torch-tensor front end of the femtohip C ABI.

Each function validates device, dtype, shape and strides on the host, then
calls the matching ``fh_*`` entry point on the tensor's current HIP stream.
Outputs are allocated by the caller or here with ``torch.empty`` (PyTorch's
caching allocator); the library itself never allocates device memory.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib

_DT = {torch.bfloat16: _lib.FH_BF16, torch.float32: _lib.FH_F32}


def _dtype_code(t: torch.Tensor) -> int:
    try:
        return _DT[t.dtype]
    except KeyError:
        raise TypeError(f"femtohip supports bfloat16 and float32, got {t.dtype}") from None


def _require_gpu(*ts: torch.Tensor) -> None:
    dev = None
    for t in ts:
        if t is None:
            continue
        if not t.is_cuda:
            raise ValueError("femtohip ops take HIP device tensors only")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} vs {t.device}")


def _same_dtype(ref: torch.Tensor, *ts: torch.Tensor) -> None:
    for t in ts:
        if t is not None and t.dtype != ref.dtype:
            raise TypeError(f"dtype mismatch: {t.dtype} vs {ref.dtype}")


def _rowmajor(t: torch.Tensor, name: str) -> int:
    """Row stride of a 2-D view whose last dim is contiguous."""
    if t.dim() != 2 or (t.size(1) > 1 and t.stride(1) != 1):
        raise ValueError(f"{name}: expected a 2-D view with a contiguous last dim, got "
                         f"shape {tuple(t.shape)} strides {t.stride()}")
    return t.stride(0)


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _ptr(t: torch.Tensor | None):
    return None if t is None else t.data_ptr()


def _fptr(t: torch.Tensor | None):
    if t is None:
        return None
    if t.dtype != torch.float32:
        raise TypeError("fp32 tensor expected")
    return ctypes.cast(t.data_ptr(), ctypes.POINTER(ctypes.c_float))


# ------------------------------------------------------------------ RMSNorm
def rmsnorm_fwd(x: torch.Tensor, w: torch.Tensor, eps: float, *, out: torch.Tensor | None = None,
                rstd: torch.Tensor | None = None) -> torch.Tensor:
    """y = w * to_dtype(x * rsqrt(mean(x^2) + eps)) over the last dim of contiguous x."""
    _require_gpu(x, w, out, rstd)
    _same_dtype(x, w, out)
    if not x.is_contiguous() or not w.is_contiguous():
        raise ValueError("rmsnorm_fwd: x and w must be contiguous")
    cols = x.size(-1)
    rows = x.numel() // max(cols, 1)
    if w.numel() != cols:
        raise ValueError("rmsnorm_fwd: weight size != last dim")
    y = torch.empty_like(x) if out is None else out
    if rstd is not None and rstd.numel() != rows:
        raise ValueError("rmsnorm_fwd: rstd must have one entry per row")
    _lib.call("fh_rmsnorm_fwd", _dtype_code(x), _ptr(x), _ptr(w), _ptr(y), _fptr(rstd), rows,
              cols, float(eps), _stream(x))
    return y


def add_rmsnorm_fwd(x: torch.Tensor, a: torch.Tensor, w: torch.Tensor, eps: float, *,
                    rstd: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """h = to_dtype(x + a); y = rmsnorm(h). Returns (h, y)."""
    _require_gpu(x, a, w, rstd)
    _same_dtype(x, a, w)
    if not (x.is_contiguous() and a.is_contiguous() and w.is_contiguous()):
        raise ValueError("add_rmsnorm_fwd: inputs must be contiguous")
    if x.shape != a.shape:
        raise ValueError("add_rmsnorm_fwd: x and a shapes differ")
    cols = x.size(-1)
    rows = x.numel() // max(cols, 1)
    if w.numel() != cols:
        raise ValueError("add_rmsnorm_fwd: weight size != last dim")
    h = torch.empty_like(x)
    y = torch.empty_like(x)
    _lib.call("fh_add_rmsnorm_fwd", _dtype_code(x), _ptr(x), _ptr(a), _ptr(w), _ptr(h), _ptr(y),
              _fptr(rstd), rows, cols, float(eps), _stream(x))
    return h, y


def rmsnorm_bwd(dy: torch.Tensor, x: torch.Tensor, w: torch.Tensor, eps: float, *,
                rstd: torch.Tensor | None = None, dres: torch.Tensor | None = None
                ) -> tuple[torch.Tensor, torch.Tensor]:
    """Gradients of rmsnorm_fwd: returns (dx [+ dres], dw)."""
    _require_gpu(dy, x, w, rstd, dres)
    _same_dtype(x, dy, w, dres)
    for t, n in ((dy, "dy"), (x, "x"), (w, "w"), (dres, "dres")):
        if t is not None and not t.is_contiguous():
            raise ValueError(f"rmsnorm_bwd: {n} must be contiguous")
    if dy.shape != x.shape or (dres is not None and dres.shape != x.shape):
        raise ValueError("rmsnorm_bwd: shape mismatch")
    cols = x.size(-1)
    rows = x.numel() // max(cols, 1)
    if w.numel() != cols:
        raise ValueError("rmsnorm_bwd: weight size != last dim")
    dx = torch.empty_like(x)
    dw = torch.empty_like(w)
    ws_bytes = _lib.lib().fh_rmsnorm_bwd_workspace_size(rows, cols)
    ws = torch.empty(max(ws_bytes, 4) // 4, dtype=torch.float32, device=x.device)
    _lib.call("fh_rmsnorm_bwd", _dtype_code(x), _ptr(dy), _ptr(x), _ptr(w), _fptr(rstd),
              _ptr(dres), _ptr(dx), _ptr(dw), _ptr(ws), rows, cols, float(eps), _stream(x))
    return dx, dw


# --------------------------------------------------------------------- RoPE
def _rope(name: str, qk: torch.Tensor, n_heads: int, head_dim: int, seq_len: int,
          cos: torch.Tensor, sin: torch.Tensor) -> None:
    _require_gpu(qk, cos, sin)
    _same_dtype(qk, cos, sin)
    ld = _rowmajor(qk, name)
    if qk.size(1) < n_heads * head_dim:
        raise ValueError(f"{name}: buffer narrower than n_heads*head_dim")
    tokens = qk.size(0)
    cos2, sin2, per_token = _rope_tables(name, cos, sin, head_dim, seq_len, tokens)
    _lib.call(name, _dtype_code(qk), _ptr(qk), ld, tokens, seq_len, n_heads, head_dim, _ptr(cos2),
              _ptr(sin2), per_token, _stream(qk))


def _rope_tables(name: str, cos: torch.Tensor, sin: torch.Tensor, head_dim: int, seq_len: int,
                 tokens: int):
    """cos/sin as [rows, head_dim] views and the cos_per_token flag of the C ABI:
    rows == seq_len (one row per position) or rows == tokens (one per token)."""
    cos2 = cos.reshape(-1, head_dim)
    sin2 = sin.reshape(-1, head_dim)
    if not (cos2.is_contiguous() and sin2.is_contiguous()) or cos2.shape != sin2.shape:
        raise ValueError(f"{name}: cos/sin must be contiguous and of equal shape")
    if cos2.size(0) == seq_len:
        if tokens % seq_len:
            raise ValueError(f"{name}: tokens not a multiple of seq_len")
        return cos2, sin2, 0
    if cos2.size(0) == tokens:
        return cos2, sin2, 1
    raise ValueError(f"{name}: cos/sin rows ({cos2.size(0)}) match neither seq_len nor tokens")


def rope_fwd_(qk: torch.Tensor, n_heads: int, head_dim: int, seq_len: int, cos: torch.Tensor,
              sin: torch.Tensor) -> torch.Tensor:
    """Rotate heads 0..n_heads-1 of the [tokens, ld] view qk in place."""
    _rope("fh_rope_fwd", qk, n_heads, head_dim, seq_len, cos, sin)
    return qk


def rope_bwd_(dqk: torch.Tensor, n_heads: int, head_dim: int, seq_len: int, cos: torch.Tensor,
              sin: torch.Tensor) -> torch.Tensor:
    _rope("fh_rope_bwd", dqk, n_heads, head_dim, seq_len, cos, sin)
    return dqk


# ------------------------------------------------------------------- SwiGLU
def swiglu_fwd(g: torch.Tensor, u: torch.Tensor, *, out: torch.Tensor | None = None) -> torch.Tensor:
    """p = to_dtype(to_dtype(silu(g)) * u) for 2-D row-major views g, u (same row stride)."""
    _require_gpu(g, u, out)
    _same_dtype(g, u, out)
    ld_gu = _rowmajor(g, "swiglu_fwd.g")
    if _rowmajor(u, "swiglu_fwd.u") != ld_gu or g.shape != u.shape:
        raise ValueError("swiglu_fwd: g and u must share shape and row stride")
    rows, cols = g.shape
    p = torch.empty(rows, cols, dtype=g.dtype, device=g.device) if out is None else out
    _lib.call("fh_swiglu_fwd", _dtype_code(g), _ptr(g), _ptr(u), ld_gu, _ptr(p),
              _rowmajor(p, "swiglu_fwd.p"), rows, cols, _stream(g))
    return p


def swiglu_bwd(dp: torch.Tensor, g: torch.Tensor, u: torch.Tensor, dg: torch.Tensor,
               du: torch.Tensor, *, p_out: torch.Tensor | None = None) -> None:
    """dg, du of p = to_dtype(to_dtype(silu(g)) * u); with p_out, also writes p there (bit for
    bit swiglu_fwd's result).  p_out may be dp itself, which is then overwritten."""
    _require_gpu(dp, g, u, dg, du, p_out)
    _same_dtype(g, dp, u, dg, du, p_out)
    ld_gu = _rowmajor(g, "swiglu_bwd.g")
    ld_d = _rowmajor(dg, "swiglu_bwd.dg")
    if _rowmajor(u, "swiglu_bwd.u") != ld_gu or _rowmajor(du, "swiglu_bwd.du") != ld_d:
        raise ValueError("swiglu_bwd: g/u and dg/du must share row strides")
    if not (dp.shape == g.shape == u.shape == dg.shape == du.shape):
        raise ValueError("swiglu_bwd: shape mismatch")
    if p_out is not None and p_out.shape != g.shape:
        raise ValueError("swiglu_bwd: p_out shape mismatch")
    rows, cols = g.shape
    ld_p = _rowmajor(p_out, "swiglu_bwd.p_out") if p_out is not None else 0
    _lib.call("fh_swiglu_bwd", _dtype_code(g), _ptr(dp), _rowmajor(dp, "swiglu_bwd.dp"), _ptr(g),
              _ptr(u), ld_gu, _ptr(dg), _ptr(du), ld_d, _ptr(p_out), ld_p,
              rows, cols, _stream(g))


def scale(x: torch.Tensor, s: torch.Tensor, *, out: torch.Tensor | None = None) -> torch.Tensor:
    """to_dtype(x * s) (fh_scale) for a contiguous bf16/fp32 x and an fp32 scalar tensor s on the
    same device; what ``(x * s).to(x.dtype)`` gives, in one streaming pass."""
    _require_gpu(x, s, out)
    if not x.is_contiguous() or s.numel() != 1 or s.dtype != torch.float32:
        raise ValueError("scale: x must be contiguous and s a one-element fp32 tensor")
    o = torch.empty_like(x) if out is None else out
    _same_dtype(x, o)
    if o.shape != x.shape or not o.is_contiguous():
        raise ValueError("scale: out must be a contiguous tensor of x's shape")
    sc = s.contiguous()
    _lib.call("fh_scale", _dtype_code(x), _ptr(x), _ptr(o), x.numel(), _ptr(sc), _stream(x))
    return o


def add(a: torch.Tensor, b: torch.Tensor, *, out: torch.Tensor | None = None) -> torch.Tensor:
    _require_gpu(a, b, out)
    _same_dtype(a, b, out)
    if not (a.is_contiguous() and b.is_contiguous()) or a.shape != b.shape:
        raise ValueError("add: a and b must be contiguous with equal shapes")
    o = torch.empty_like(a) if out is None else out
    _lib.call("fh_add", _dtype_code(a), _ptr(a), _ptr(b), _ptr(o), a.numel(), _stream(a))
    return o


# ---------------------------------------------------------------- attention
def attn_fwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, batch: int, seq_len: int,
             n_heads: int, n_kv_heads: int, head_dim: int, scale: float, *,
             need_lse: bool = True, rope: tuple | None = None,
             q_out: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor | None]:
    """Causal GQA attention on token-major [T, *] views (head h at columns h*head_dim).
    Returns (o [T, n_heads*head_dim], lse fp32 [batch, n_heads, seq_len] or None).
    rope=(cos, sin): q is read unrotated and rotated on load (fh_attn_fwd_rope; k
    must already be rotated); q_out (may be q itself) then receives the rotated q."""
    _require_gpu(q, k, v, q_out)
    _same_dtype(q, k, v)
    T = batch * seq_len
    for t, n in ((q, "q"), (k, "k"), (v, "v")):
        if t.size(0) != T:
            raise ValueError(f"attn_fwd: {n} has {t.size(0)} rows, expected {T}")
    o = torch.empty(T, n_heads * head_dim, dtype=q.dtype, device=q.device)
    lse = (torch.empty(batch, n_heads, seq_len, dtype=torch.float32, device=q.device)
           if need_lse else None)
    head = (_dtype_code(q), _ptr(q), _rowmajor(q, "q"), _ptr(k), _rowmajor(k, "k"),
            _ptr(v), _rowmajor(v, "v"), _ptr(o), o.stride(0), _fptr(lse))
    tail = (batch, seq_len, n_heads, n_kv_heads, head_dim, float(scale))
    if rope is None:
        if q_out is not None:
            raise ValueError("attn_fwd: q_out needs rope")
        _lib.call("fh_attn_fwd", *head, *tail, _stream(q))
        return o, lse
    cos, sin = rope
    _require_gpu(cos, sin)
    _same_dtype(q, cos, sin)
    if q_out is not None:
        _same_dtype(q, q_out)
        if tuple(q_out.shape) != tuple(q.shape):
            raise ValueError("attn_fwd: q_out must have q's shape")
    cos2, sin2, per_token = _rope_tables("attn_fwd_rope", cos, sin, head_dim, seq_len, T)
    _lib.call("fh_attn_fwd_rope", *head, _ptr(q_out), 0 if q_out is None else _rowmajor(q_out, "q_out"),
              *tail, _ptr(cos2), _ptr(sin2), per_token, _stream(q))
    return o, lse


def attn_bwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, o: torch.Tensor,
             dout: torch.Tensor, lse: torch.Tensor, dq: torch.Tensor, dk: torch.Tensor,
             dv: torch.Tensor, batch: int, seq_len: int, n_heads: int, n_kv_heads: int,
             head_dim: int, scale: float, rope: tuple | None = None) -> None:
    """Writes dq, dk, dv (token-major views, may be column ranges of one buffer).
    rope=(cos, sin): dq and dk come out passed through the RoPE backward as well
    (fh_attn_bwd_rope), the gradients before the rotation of q and k."""
    _require_gpu(q, k, v, o, dout, lse, dq, dk, dv)
    _same_dtype(q, k, v, o, dout, dq, dk, dv)
    if lse.dtype != torch.float32 or not lse.is_contiguous() or lse.numel() != batch * n_heads * seq_len:
        raise ValueError("attn_bwd: lse must be contiguous fp32 [batch, n_heads, seq_len]")
    ws_bytes = _lib.lib().fh_attn_bwd_workspace_size(batch, seq_len, n_heads)
    ws = torch.empty(max(ws_bytes, 4) // 4, dtype=torch.float32, device=q.device)
    args = (_dtype_code(q), _ptr(q), _rowmajor(q, "q"), _ptr(k), _rowmajor(k, "k"),
            _ptr(v), _rowmajor(v, "v"), _ptr(o), _rowmajor(o, "o"), _ptr(dout),
            _rowmajor(dout, "dout"), _fptr(lse), _ptr(dq), _rowmajor(dq, "dq"), _ptr(dk),
            _rowmajor(dk, "dk"), _ptr(dv), _rowmajor(dv, "dv"), _ptr(ws), batch, seq_len,
            n_heads, n_kv_heads, head_dim, float(scale))
    if rope is None:
        _lib.call("fh_attn_bwd", *args, _stream(q))
        return
    cos, sin = rope
    _require_gpu(cos, sin)
    _same_dtype(q, cos, sin)
    cos2, sin2, per_token = _rope_tables("attn_bwd_rope", cos, sin, head_dim, seq_len, batch * seq_len)
    _lib.call("fh_attn_bwd_rope", *args, _ptr(cos2), _ptr(sin2), per_token, _stream(q))


# ------------------------------------------------------------- loss head
def ce_fwd_bwd_(logits: torch.Tensor, labels: torch.Tensor, inv_count: torch.Tensor,
                ignore_index: int = -100) -> torch.Tensor:
    """Cross-entropy of the rows of `logits` [rows, V] against `labels` (int64
    [rows]); overwrites `logits` with the gradient (softmax - onehot) * inv_count
    (0 for ignored rows) and returns the fp32 per-row losses.  `inv_count` is a
    device fp32 scalar, 1 / (number of non-ignored labels of the whole batch)."""
    _require_gpu(logits, labels, inv_count)
    if logits.dim() != 2 or logits.stride(1) != 1:
        raise ValueError("ce_fwd_bwd_: logits must be a row-major 2-D tensor")
    if labels.dtype != torch.int64 or not labels.is_contiguous() or labels.numel() != logits.size(0):
        raise ValueError("ce_fwd_bwd_: labels must be contiguous int64 with one entry per row")
    if inv_count.dtype != torch.float32 or inv_count.numel() != 1:
        raise ValueError("ce_fwd_bwd_: inv_count must be a one-element fp32 tensor")
    loss_rows = torch.empty(logits.size(0), dtype=torch.float32, device=logits.device)
    _lib.call("fh_ce_fwd_bwd", _dtype_code(logits), _ptr(logits), logits.stride(0), _ptr(labels),
              logits.size(0), logits.size(1), int(ignore_index), _ptr(inv_count), _fptr(loss_rows),
              _stream(logits))
    return loss_rows


# ------------------------------------------------------------- embedding
def _embedding_args(weight: torch.Tensor, ids: torch.Tensor) -> tuple[int, int]:
    if weight.dim() != 2 or not weight.is_contiguous():
        raise ValueError("embedding: weight must be a contiguous [vocab, hidden] tensor")
    if ids.dtype != torch.int64 or not ids.is_contiguous():
        raise ValueError("embedding: ids must be contiguous int64")
    vocab, hidden = weight.shape
    if hidden % 8 != 0:
        raise ValueError(f"embedding: hidden must be a multiple of 8, got {hidden}")
    return vocab, hidden


def embedding_fwd(ids: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """weight[ids] with zero rows for ids outside [0, vocab): [*ids.shape, hidden]."""
    _require_gpu(ids, weight)
    vocab, hidden = _embedding_args(weight, ids)
    out = torch.empty(*ids.shape, hidden, dtype=weight.dtype, device=weight.device)
    _lib.call("fh_embedding_fwd", _dtype_code(weight), _ptr(weight), _ptr(ids), _ptr(out),
              ids.numel(), vocab, hidden, _stream(weight))
    return out


def embedding_bwd(dy: torch.Tensor, ids: torch.Tensor, vocab: int,
                  padding_idx: int | None = None) -> torch.Tensor:
    """Weight gradient of the lookup: [vocab, hidden], row v = sum of the dy rows
    of the tokens with id v (fp32, token order), zero for unused ids; tokens with
    an id outside [0, vocab) or equal to padding_idx contribute nothing."""
    _require_gpu(dy, ids)
    hidden = dy.size(-1)
    if not dy.is_contiguous() or dy.numel() != ids.numel() * hidden:
        raise ValueError("embedding_bwd: dy must be contiguous [*ids.shape, hidden]")
    if ids.dtype != torch.int64 or not ids.is_contiguous():
        raise ValueError("embedding_bwd: ids must be contiguous int64")
    if hidden % 8 != 0:
        raise ValueError(f"embedding_bwd: hidden must be a multiple of 8, got {hidden}")
    dw = torch.empty(vocab, hidden, dtype=dy.dtype, device=dy.device)
    n = ids.numel()
    ws = torch.empty(_lib.lib().fh_embedding_bwd_workspace_size(n, vocab), dtype=torch.uint8,
                     device=dy.device)
    _lib.call("fh_embedding_bwd", _dtype_code(dy), _ptr(dy), _ptr(ids), _ptr(dw), n, vocab, hidden,
              -1 if padding_idx is None else int(padding_idx), _ptr(ws), _stream(dy))
    return dw


# ------------------------------------------------------------- GEMM
_GEMM_OPS = {"nt": _lib.FH_GEMM_NT, "nn": _lib.FH_GEMM_NN, "tn": _lib.FH_GEMM_TN}


def gemm_dims(op: str, a: torch.Tensor, b: torch.Tensor):
    """(m, n, k) of op(a) @ op(b), or None if the shapes do not chain."""
    if a.dim() != 2 or b.dim() != 2:
        return None
    if op == "nt":
        (m, k), (n, kb) = a.shape, b.shape
    elif op == "nn":
        (m, k), (kb, n) = a.shape, b.shape
    elif op == "tn":
        (k, m), (kb, n) = a.shape, b.shape
    else:
        raise ValueError(f"gemm: op must be 'nt', 'nn' or 'tn', got {op!r}")
    return (m, n, k) if k == kb else None


def gemm_supported(op: str, a: torch.Tensor, b: torch.Tensor) -> bool:
    """Whether fh_gemm_bf16 takes these operands: bf16 on one HIP device, 2-D
    with a contiguous last dim, k a multiple of 64, n (and for 'tn' also m) a
    multiple of 8, row strides multiples of 8 and 16-byte aligned data."""
    if not (a.is_cuda and b.is_cuda and a.device == b.device and a.dtype == b.dtype == torch.bfloat16):
        return False
    dims = gemm_dims(op, a, b)
    if dims is None:
        return False
    m, n, k = dims
    if min(m, n, k) <= 0 or k % 64 or n % 8 or (op == "tn" and m % 8):
        return False
    for t in (a, b):
        if t.stride(1) != 1 or t.stride(0) % 8 or t.data_ptr() % 16:
            return False
    return True


def gemm(op: str, a: torch.Tensor, b: torch.Tensor, *, residual: torch.Tensor | None = None,
         out: torch.Tensor | None = None) -> torch.Tensor:
    """op(a) @ op(b) in bf16 with fp32 accumulation (fh_gemm_bf16):
    'nt': a [m,k] @ b[n,k]^T (nn.Linear forward), 'nn': a [m,k] @ b [k,n]
    (input gradient), 'tn': a[k,m]^T @ b [k,n] (weight gradient).  With
    `residual` ([m, n]) returns residual + to_bf16(product), rounded again;
    `out` may be `residual` itself."""
    _require_gpu(a, b, residual, out)
    if not gemm_supported(op, a, b):
        raise ValueError(f"gemm({op}): unsupported operands {tuple(a.shape)} {a.stride()} x "
                         f"{tuple(b.shape)} {b.stride()} ({a.dtype}, {b.dtype})")
    m, n, k = gemm_dims(op, a, b)
    c = torch.empty(m, n, dtype=a.dtype, device=a.device) if out is None else out
    for t, name in ((c, "out"), (residual, "residual")):
        if t is None:
            continue
        if t.dtype != torch.bfloat16 or tuple(t.shape) != (m, n) or t.stride(1) != 1:
            raise ValueError(f"gemm({op}): {name} must be a bf16 [{m}, {n}] row-major view")
        if t.stride(0) % 8 or t.data_ptr() % 16:
            raise ValueError(f"gemm({op}): {name} must be 16-byte aligned with a row stride % 8 == 0")
    code = _GEMM_OPS[op]
    nbytes = _lib.lib().fh_gemm_bf16_workspace_size(code, m, n, k)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=a.device) if nbytes else None
    _lib.call("fh_gemm_bf16", code, _ptr(a), a.stride(0), _ptr(b), b.stride(0), _ptr(c), c.stride(0),
              _ptr(residual), 0 if residual is None else residual.stride(0), m, n, k, _ptr(ws),
              _stream(a))
    return c


def gemm_grouped(op: str, items: list) -> list:
    """Up to three GEMMs of layout `op` with one k in one fh_gemm_bf16_grouped
    call: each item is (a, b, residual, out) with gemm()'s meaning (residual
    and out may be None; out may be residual itself).  Returns the outputs."""
    if not 1 <= len(items) <= 3:
        raise ValueError(f"gemm_grouped({op}): between 1 and 3 problems, got {len(items)}")
    probs = (_lib.FhGemmProblem * len(items))()
    outs, ks = [], set()
    for i, (a, b, residual, out) in enumerate(items):
        _require_gpu(a, b, residual, out)
        if not gemm_supported(op, a, b):
            raise ValueError(f"gemm_grouped({op}): unsupported operands {tuple(a.shape)} {a.stride()} x "
                             f"{tuple(b.shape)} {b.stride()} ({a.dtype}, {b.dtype})")
        m, n, k = gemm_dims(op, a, b)
        ks.add(k)
        c = torch.empty(m, n, dtype=a.dtype, device=a.device) if out is None else out
        for t, name in ((c, "out"), (residual, "residual")):
            if t is None:
                continue
            if t.dtype != torch.bfloat16 or tuple(t.shape) != (m, n) or t.stride(1) != 1:
                raise ValueError(f"gemm_grouped({op}): {name} must be a bf16 [{m}, {n}] row-major view")
            if t.stride(0) % 8 or t.data_ptr() % 16:
                raise ValueError(f"gemm_grouped({op}): {name} must be 16-byte aligned with a row stride % 8 == 0")
        probs[i] = _lib.FhGemmProblem(_ptr(a), a.stride(0), _ptr(b), b.stride(0), _ptr(c), c.stride(0),
                                      _ptr(residual), 0 if residual is None else residual.stride(0), m, n)
        outs.append(c)
    if len(ks) != 1:
        raise ValueError(f"gemm_grouped({op}): the problems' k differ: {sorted(ks)}")
    k = ks.pop()
    code = _GEMM_OPS[op]
    a0 = items[0][0]
    if any(t is not None and t.device != a0.device for item in items for t in item) or \
            any(o.device != a0.device for o in outs):
        raise ValueError(f"gemm_grouped({op}): every operand and output must be on {a0.device}")
    nbytes = _lib.lib().fh_gemm_bf16_grouped_workspace_size(code, len(items), probs, k)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=a0.device) if nbytes else None
    _lib.call("fh_gemm_bf16_grouped", code, len(items), probs, k, _ptr(ws), _stream(a0))
    return outs


def gemm_rope(a: torch.Tensor, b: torch.Tensor, n_rot_heads: int, head_dim: int, seq_len: int,
              cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """a [m,k] @ b[n,k]^T (the q/k/v projection) with the rotary embedding of
    rope_fwd_ applied to heads 0..n_rot_heads-1 of the output in the GEMM's
    epilogue (fh_gemm_bf16_rope); rows of a are tokens."""
    _require_gpu(a, b, cos, sin)
    if not gemm_supported("nt", a, b):
        raise ValueError(f"gemm_rope: unsupported operands {tuple(a.shape)} {a.stride()} x "
                         f"{tuple(b.shape)} {b.stride()} ({a.dtype}, {b.dtype})")
    _same_dtype(a, cos, sin)
    m, n, k = gemm_dims("nt", a, b)
    cos2, sin2, per_token = _rope_tables("gemm_rope", cos, sin, head_dim, seq_len, m)
    c = torch.empty(m, n, dtype=a.dtype, device=a.device)
    _lib.call("fh_gemm_bf16_rope", _ptr(a), a.stride(0), _ptr(b), b.stride(0), _ptr(c), c.stride(0),
              m, n, k, n_rot_heads * head_dim, head_dim, seq_len, _ptr(cos2), _ptr(sin2), per_token,
              _stream(a))
    return c


