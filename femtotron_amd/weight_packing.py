"""Contiguous q/k/v and gate/up weights, so the fused GEMMs need no concatenation.

The layer's projections run as one GEMM over [Wq; Wk; Wv] and one over
[Wg; Wu] (femtotron_amd/fused_layer.py), the reference's separate
Column/RowParallelLinear weights (femtotron/parallel/tensor_parallel/linear.py:66-80
at TP=1) being separate tensors.  Without packing every forward, recompute and
backward concatenates them (6 copies of the layer's q/k/v and gate/up weights per
step).  ``pack_layer_weights`` moves each group into one buffer once and makes
the parameters row views of it: parameter objects, names, shapes, dtypes,
gradients and state-dict keys are unchanged, and in-place updates (optimizer
steps, ``copy_`` from fp32 masters, ``load_state_dict``) keep the layout.
Anything that re-allocates a parameter (``.to()``, flattening wrappers) simply
breaks the layout; ``packed`` then returns None and the fused path concatenates
as before, so packing never affects results.
"""
from __future__ import annotations

import torch
from torch import nn


def packed(*ws: torch.Tensor) -> torch.Tensor | None:
    """The [sum(rows), cols] tensor the row-contiguous weights `ws` form, as a
    view of their common storage, or None if they are not laid out that way."""
    first = ws[0]
    if first.dim() != 2 or not first.is_contiguous():
        return None
    cols = first.shape[1]
    store = first.untyped_storage()
    off = first.storage_offset()
    rows = 0
    for w in ws:
        if (w.dim() != 2 or w.shape[1] != cols or not w.is_contiguous() or w.dtype != first.dtype
                or w.device != first.device or w.untyped_storage().data_ptr() != store.data_ptr()
                or w.storage_offset() != off + rows * cols):
            return None
        rows += w.shape[0]
    return first.new_empty(0).set_(store, off, (rows, cols), (cols, 1))


def _pack_group(params: list[nn.Parameter]) -> bool:
    if packed(*params) is not None:
        return False
    buf = torch.cat([p.detach() for p in params], 0)
    row = 0
    with torch.no_grad():
        for p in params:
            n = p.shape[0]
            p.data = buf[row:row + n]
            row += n
    return True


def pack_layer_weights(model: nn.Module) -> int:
    """Pack q/k/v and gate/up of every Llama attention / MLP module of `model`;
    call once after building and initialising it (an optimizer holding the
    parameters may exist already: the parameter objects stay the same).
    Returns the number of groups newly packed."""
    n = 0
    for mod in model.modules():
        names = None
        if all(hasattr(mod, a) for a in ("q_proj", "k_proj", "v_proj")):
            names = ("q_proj", "k_proj", "v_proj")
        elif all(hasattr(mod, a) for a in ("gate_proj", "up_proj")):
            names = ("gate_proj", "up_proj")
        if names is None:
            continue
        ws = [getattr(getattr(mod, a), "weight", None) for a in names]
        if any(not isinstance(w, nn.Parameter) for w in ws):
            continue
        if len({(w.dtype, w.device, w.shape[1]) for w in ws}) != 1:
            continue
        n += _pack_group(ws)
    return n
