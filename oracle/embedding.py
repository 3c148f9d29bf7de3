"""ORACLE — test infrastructure only.  NumPy statement of the token embedding
of the first pipeline stage, forward and weight gradient.

Reference: femtotron/model/llama_partial_model.py:181-184 (``embed_tokens``:
nn.Embedding, padding_idx = pad_token_id) and its one-rank TP form
femtotron/parallel/tensor_parallel/embedding.py:57-79 (ids outside the vocab
range are masked to row 0, looked up, and their rows zeroed).  The weight
gradient of F.embedding is the scatter-add of the output-gradient rows into
the rows of their ids, nothing for padding_idx (torch.nn.functional.embedding).

``embedding_bwd_ordered`` fixes the summation order the fused kernel promises:
each row summed in fp32 in ascending token order, then rounded once.

Pinning (tests/test_boundary.py): torch's own F.embedding forward and backward
in fp64 on the CPU (with and without padding_idx, repeated ids, masked ids);
and the ordered fp32 sums against the exact fp64 sums (within fp32 rounding)
and against a brute-force per-row loop.
"""
from __future__ import annotations

import numpy as np


def embedding_fwd(ids: np.ndarray, w: np.ndarray) -> np.ndarray:
    """w[ids] with zero rows for ids outside [0, V)."""
    V = w.shape[0]
    ok = (ids >= 0) & (ids < V)
    out = w[np.where(ok, ids, 0)]
    out[~ok] = 0
    return out


def embedding_bwd(dy: np.ndarray, ids: np.ndarray, V: int, padding_idx: int | None = None,
                  dtype=np.float64) -> np.ndarray:
    """Exact scatter-add (in `dtype`, np.add.at order = token order)."""
    H = dy.shape[-1]
    ids = ids.reshape(-1)
    dy = dy.reshape(-1, H).astype(dtype)
    keep = (ids >= 0) & (ids < V)
    if padding_idx is not None:
        keep &= ids != padding_idx
    dw = np.zeros((V, H), dtype=dtype)
    np.add.at(dw, ids[keep], dy[keep])
    return dw


def embedding_bwd_ordered(dy: np.ndarray, ids: np.ndarray, V: int,
                          padding_idx: int | None = None) -> np.ndarray:
    """fp32 sums in ascending token order per row (the kernel's order), fp32 result."""
    H = dy.shape[-1]
    ids = ids.reshape(-1)
    dy = dy.reshape(-1, H).astype(np.float32)
    dw = np.zeros((V, H), dtype=np.float32)
    for t in range(ids.shape[0]):  # sequential: token order within every row
        v = int(ids[t])
        if 0 <= v < V and v != padding_idx:
            dw[v] = dw[v] + dy[t]
    return dw
