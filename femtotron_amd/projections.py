"""The GEMMs of the layer's seven projections, routed per shape.

Every projection of the decoder layer is femtotron's Column/RowParallelLinear
at one rank (femtotron/parallel/tensor_parallel/linear.py:66-80, 194-214),
i.e. ``F.linear(x, W)`` with W [out, in] and no bias.  Its three GEMMs are:

    forward          y  = x W^T        fh_gemm_bf16 FH_GEMM_NT   (linear)
    input gradient   dx = dy W         fh_gemm_bf16 FH_GEMM_NN   (linear_dgrad)
    weight gradient  dW = dy^T x       fh_gemm_bf16 FH_GEMM_TN   (linear_wgrad; three of
                                       them in one fh_gemm_bf16_grouped launch: linear_wgrad_group)

plus ``residual + x W^T`` with the residual add fused into the forward GEMM's
epilogue (linear_residual, the down projection; modeling_llama.py:323 rounds
the projection output to bf16, then the sum: routed by its own table entry,
``nt_res``, which compares the hand-written GEMM with that epilogue against
the library GEMM followed by fh_add), and the q/k/v projection followed by the rotary
embedding of its k heads (linear_rope: the GEMM, then fh_rope_fwd; the
attention forward rotates q as it loads it).  fh_gemm_bf16_rope, the
rotation in the GEMM's epilogue, measured slower than the plain GEMM and the
separate pass at every workload (TinyLlama q/k/v: 214 against ~157 us) and
is not dispatched.

Each call runs either the hand-written gfx950 kernel or the tuned library
GEMM (``torch.mm`` on hipBLASLt/rocBLAS), by policy:

* ``"hand"`` (default): the hand-written kernel wherever it supports the
  operands -- every projection GEMM of the layers of the shipped workloads;
* ``"auto"``: the shipped per-shape table ``tuned/gemm_dispatch_gfx950.json``
  names the shapes measured on an MI355X where the library was faster than
  the hand-written kernel; those run on the library, every other supported
  shape on the hand-written kernel.  At the shipped workloads the table
  holds the forward (NT) shapes, where the library's hand-tuned gfx950
  kernels measured 3-7% faster; a TinyLlama step runs ~2% faster with them;
* ``"library"``: always the library.

Operands the kernel does not take (fp32, k not a multiple of 64, ...) go to
the library under every policy.  ``gemm_dispatch_counts()`` tells tests and
the benchmark which path ran.
"""
from __future__ import annotations

import json
import threading
from pathlib import Path

import torch

from . import ops

TABLE_FILE = Path(__file__).resolve().parent / "tuned" / "gemm_dispatch_gfx950.json"
# The library takes a shape only when it measured at least this much faster
# than the hand-written kernel alone (the two alternate, medians compared):
# inside the TinyLlama step the input-gradient (NN) GEMMs, each within 1% of
# the library alone, ran faster hand-written (126.7k against 125.8k tokens/s
# with the library taking those near-ties).
LIBRARY_MARGIN = 1.02

_lock = threading.Lock()
_policy = ["hand"]
_table: dict[str, set] | None = None
_counts = {"hand": 0, "library": 0}


def set_gemm_policy(policy: str) -> None:
    """'hand' (the default: hand-written wherever supported), 'auto' (the measured table) or 'library'."""
    if policy not in ("auto", "hand", "library"):
        raise ValueError(f"gemm policy must be 'auto', 'hand' or 'library', got {policy!r}")
    _policy[0] = policy


def gemm_policy() -> str:
    return _policy[0]


def gemm_dispatch_counts() -> dict[str, int]:
    with _lock:
        return dict(_counts)


def reset_gemm_dispatch_counts() -> None:
    with _lock:
        _counts["hand"] = 0
        _counts["library"] = 0


def _library_shapes() -> dict[str, set]:
    global _table
    if _table is None:
        shapes: dict[str, set] = {"nt": set(), "nn": set(), "tn": set(), "nt_res": set()}
        if TABLE_FILE.is_file():
            data = json.loads(TABLE_FILE.read_text())
            for op in shapes:
                shapes[op] = {tuple(s) for s in data.get("library", {}).get(op, [])}
        _table = shapes
    return _table


def _choose_hand(op: str, a: torch.Tensor, b: torch.Tensor, table: str | None = None) -> bool:
    pol = _policy[0]
    use = pol != "library" and ops.gemm_supported(op, a, b)
    if use and pol == "auto":
        use = ops.gemm_dims(op, a, b) not in _library_shapes()[table or op]
    return use


def _count(hand: bool) -> bool:
    """Count one GEMM as hand-written or library; returns `hand`."""
    with _lock:
        _counts["hand" if hand else "library"] += 1
    return hand


def _use_hand(op: str, a: torch.Tensor, b: torch.Tensor) -> bool:
    return _count(_choose_hand(op, a, b))


def linear(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """x [T, in] @ w[out, in]^T."""
    if _use_hand("nt", x, w):
        return ops.gemm("nt", x, w)
    return torch.mm(x, w.t())


def linear_rope(x: torch.Tensor, w: torch.Tensor, n_rot_heads: int, head_dim: int, seq_len: int,
                cos: torch.Tensor, sin: torch.Tensor, *, defer_heads: int = 0) -> tuple[torch.Tensor, bool]:
    """x [T, in] @ w[out, in]^T with heads 0..n_rot_heads-1 of the output (q and
    k of the packed q/k/v projection) rotated by RoPE (rope_fwd_'s arithmetic).
    The GEMM is routed as linear's; the rotation is a separate pass that leaves
    heads 0..defer_heads-1 (q) unrotated for the caller to rotate as it reads
    them (the attention forward's q load).  Returns (y, all rotated)."""
    y = linear(x, w)  # counts this GEMM once
    if n_rot_heads > defer_heads:
        ops.rope_fwd_(y[:, defer_heads * head_dim:], n_rot_heads - defer_heads, head_dim, seq_len, cos, sin)
    return y, defer_heads == 0


def linear_residual(x: torch.Tensor, w: torch.Tensor, residual: torch.Tensor) -> torch.Tensor:
    """residual + to_dtype(x @ w^T), written into `residual`'s memory (the
    hand-written GEMM's residual epilogue; otherwise the library GEMM followed
    by fh_add into `residual`)."""
    if _count(residual.is_contiguous() and _choose_hand("nt", x, w, "nt_res")):
        return ops.gemm("nt", x, w, residual=residual, out=residual)
    m = torch.mm(x, w.t())
    if not residual.is_contiguous():
        return residual.add_(m)  # one fp32 add, one rounding, as fh_add
    return ops.add(residual, m, out=residual)


def linear_dgrad(dy: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """dy [T, out] @ w [out, in]."""
    if _use_hand("nn", dy, w):
        return ops.gemm("nn", dy, w)
    return torch.mm(dy, w)


def linear_wgrad(dy: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    """dy [T, out]^T @ x [T, in]: the [out, in] weight gradient."""
    if _use_hand("tn", dy, x):
        return ops.gemm("tn", dy, x)
    return torch.mm(dy.t(), x)


def linear_wgrad_into(dy: torch.Tensor, x: torch.Tensor, grad: torch.Tensor) -> bool:
    """grad = to_bf16(grad + to_bf16(dy^T x)) in place, where the hand-written
    GEMM takes the shape: its residual epilogue with the residual and the
    output both `grad`, the two roundings of accumulating a bf16 weight
    gradient into an existing bf16 .grad (autograd's grad + new_grad after the
    GEMM rounded new_grad).  Returns False, doing nothing, where the shape
    runs on the library (whose accumulating GEMM rounds once): the caller
    then computes the gradient and lets autograd add it."""
    if not _choose_hand("tn", dy, x):
        return False
    _count(True)
    ops.gemm("tn", dy, x, residual=grad, out=grad)
    return True


def layer_gemm_forms(tokens: int, hidden: int, q_width: int, kv_width: int, ffn: int):
    """(op, m, n, k) of every GEMM a fused decoder layer issues (packed q/k/v and
    gate/up), in fh_gemm_bf16's convention."""
    projs = [(q_width + 2 * kv_width, hidden), (hidden, q_width), (2 * ffn, hidden), (hidden, ffn)]
    forms = []
    for out_f, in_f in projs:
        forms += [("nt", tokens, out_f, in_f), ("nn", tokens, in_f, out_f), ("tn", out_f, in_f, tokens)]
    return forms


def linear_wgrad_group(items: list) -> list | None:
    """dW_i = dy_i^T x_i for up to three projections whose dy and x share one
    token count, in one hand-written launch (fh_gemm_bf16_grouped): the layer's
    q/k/v, o and down weight gradients have few output tiles each and fill the
    CUs together.  Each item is (dy, x, grad), grad the parameter's existing
    bf16 gradient to accumulate into (linear_wgrad_into's rule) or None.
    Returns the new gradients (None where accumulated), or None when the
    dispatch would not run every one of them hand-written (the caller then runs
    them one by one)."""
    if not all(_choose_hand("tn", dy, x) for dy, x, _ in items):
        return None
    for _ in items:
        _count(True)
    outs = ops.gemm_grouped("tn", [(dy, x, g, g) for dy, x, g in items])
    return [None if g is not None else o for (_, _, g), o in zip(items, outs)]


def measure_dispatch(workloads: dict, path: str | Path = TABLE_FILE, *, iters: int = 10, reps: int = 5,
                     log=print) -> Path:
    """Time the hand-written kernel against the library GEMM (with whatever
    library solutions the process has enabled) for every layer GEMM of
    `workloads` ({name: (tokens, hidden, q width, kv width, ffn, head_dim,
    seq_len)}) and write the shapes where the library was faster.  The two
    candidates run alternately, `reps`
    times `iters` launches each, and their medians are compared: the GPU's
    clock drifts by several percent between back-to-back measurements.  Needs
    a HIP device."""
    import statistics

    dev, bf = "cuda", torch.bfloat16
    g = torch.Generator(device=dev).manual_seed(0)
    lib_faster: dict[str, list] = {"nt": [], "nn": [], "tn": [], "nt_res": []}
    rows = []

    def one(fn) -> float:
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(iters):
            fn()
        e.record()
        e.synchronize()
        return s.elapsed_time(e) / iters * 1e3

    def timed_pair(hand, lib) -> tuple[float, float]:
        for _ in range(3):
            hand()
            lib()
        th, tl = [], []
        for _ in range(reps):
            th.append(one(hand))
            tl.append(one(lib))
        return statistics.median(th), statistics.median(tl)

    for name, (T, H, hq, hkv, F, hd, S) in workloads.items():
        for op, m, n, k in layer_gemm_forms(T, H, hq, hkv, F):
            a_shape = (k, m) if op == "tn" else (m, k)
            b_shape = (n, k) if op == "nt" else (k, n)
            a = torch.randn(*a_shape, device=dev, generator=g).to(bf)
            b = torch.randn(*b_shape, device=dev, generator=g).to(bf)
            lib = {"nt": lambda: torch.mm(a, b.t()), "nn": lambda: torch.mm(a, b),
                   "tn": lambda: torch.mm(a.t(), b)}[op]
            t_hand, t_lib = timed_pair(lambda: ops.gemm(op, a, b), lib)
            rows.append(dict(workload=name, op=op, m=m, n=n, k=k, hand_us=round(t_hand, 1),
                             library_us=round(t_lib, 1)))
            if t_lib * LIBRARY_MARGIN < t_hand and [m, n, k] not in lib_faster[op]:
                lib_faster[op].append([m, n, k])
            log(f"[gemm-dispatch] {name} {op} m={m} n={n} k={k}: hand {t_hand:.1f} us, "
                f"library {t_lib:.1f} us")
            del a, b
        # The down projection's residual form (linear_residual): the hand-written
        # GEMM with the residual add in its epilogue against the library GEMM
        # followed by fh_add.
        m, n, k = T, H, F
        a = torch.randn(m, k, device=dev, generator=g).to(bf)
        b = torch.randn(n, k, device=dev, generator=g).to(bf)
        r = torch.randn(m, n, device=dev, generator=g).to(bf)
        out = torch.empty_like(r)
        t_hand, t_lib = timed_pair(lambda: ops.gemm("nt", a, b, residual=r, out=out),
                                   lambda: ops.add(r, torch.mm(a, b.t()), out=out))
        rows.append(dict(workload=name, op="nt_res", m=m, n=n, k=k, hand_us=round(t_hand, 1),
                         library_us=round(t_lib, 1)))
        if t_lib * LIBRARY_MARGIN < t_hand and [m, n, k] not in lib_faster["nt_res"]:
            lib_faster["nt_res"].append([m, n, k])
        log(f"[gemm-dispatch] {name} nt_res m={m} n={n} k={k}: hand + residual epilogue {t_hand:.1f} us, "
            f"library + fh_add {t_lib:.1f} us")
        del a, b, r, out
    data = {"note": "shapes (m, n, k of fh_gemm_bf16) where the tuned library GEMM measured at least 2% "
                    "faster than the hand-written kernel on an MI355X (medians of alternating runs); "
                    "everything else runs hand-written. nt_res: the down projection with its residual "
                    "add (hand-written epilogue against library GEMM + fh_add)",
            "library": lib_faster, "measurements": rows}
    Path(path).write_text(json.dumps(data, indent=1) + "\n")
    global _table
    _table = None
    return Path(path)
