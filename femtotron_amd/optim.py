"""Fused mixed-precision AdamW (the optimizer step after the checkpointed backward).

Mirrors what the reference's ``MixedPrecisionManager.step()`` does on one device
with the NoShard strategy (femtotron/training/mixed_precision_manager.py:318-331):
fp32 master copies of the model-dtype parameters, ``master.grad =
param.grad.float()``, the ``ClipGradNorm`` transform (grad_transform.py:13-63:
coef = clamp(max_norm / (||g|| + 1e-6), max=1), applied to every gradient),
``torch.optim.AdamW`` on the masters with the reference's per-group weight
decay (femtotron/training/optimizer.py:5-45;
femtotron/scripts/train.py:264-276), and ``param.copy_(master)``.
Here the whole step is one ``fh_adamw_step`` call over a device table of all
tensors: a pass that sums the squared gradients, a one-block fold into the norm
and the clipping coefficient, then one pass that reads each element's
gradient, master and moments once and writes master, moments and the
model-dtype parameter once (30 bytes per bf16 parameter in all).  No host
synchronisation: the coefficient stays on the device and the norm is returned
as a device tensor.
"""
from __future__ import annotations

import ctypes
import math
from typing import Iterable

import torch

from . import _lib
from ._lib import FhAdamHyper

CHUNK = 2048  # elements per workgroup of fh_adamw_step


class _Tensor(ctypes.Structure):
    _fields_ = [("param", ctypes.c_void_p), ("grad", ctypes.c_void_p), ("master", ctypes.c_void_p),
                ("exp_avg", ctypes.c_void_p), ("exp_avg_sq", ctypes.c_void_p),
                ("numel", ctypes.c_int64), ("decay", ctypes.c_float), ("step_size", ctypes.c_float),
                ("bias_correction2_sqrt", ctypes.c_float), ("reserved", ctypes.c_float)]


def get_param_groups(model: torch.nn.Module, weight_decay: float = 0.01) -> list[dict]:
    """Two groups as the reference builds them (femtotron/training/optimizer.py:5-45):
    no weight decay for 1-D parameters and names containing "bias" or "embed",
    ``weight_decay`` for every other trainable parameter."""
    decay, no_decay = [], []
    for name, p in model.named_parameters():
        if not p.requires_grad:
            continue
        (no_decay if p.ndim <= 1 or "bias" in name or "embed" in name else decay).append(p)
    return [{"params": decay, "weight_decay": weight_decay}, {"params": no_decay, "weight_decay": 0.0}]


def _aligned(t: torch.Tensor) -> bool:
    return t.data_ptr() % 16 == 0


class FusedAdamW(torch.optim.Optimizer):
    """AdamW on fp32 masters of model-dtype parameters, with global grad-norm clipping.

    A ``torch.optim.Optimizer`` over the model-dtype parameters, so learning-rate
    schedulers work on it as on the reference's inner optimizer
    (femtotron/scripts/train.py:307-312 wraps it in ``LambdaLR``).  ``params``: an
    iterable of parameters or of dicts ``{"params": [...], "weight_decay": wd}``
    (the format of ``get_param_groups``).  All parameters must live on one HIP
    device in one dtype (bf16 or fp32) and be contiguous and 16-byte aligned; at a
    step every group must have the same lr, betas and eps (weight decay may differ).
    ``max_grad_norm`` <= 0 or None disables clipping.  Per-parameter state:
    ``master``, ``exp_avg``, ``exp_avg_sq`` (fp32), created at construction, and
    ``step``, the number of steps that updated the parameter; each tensor's bias
    corrections follow its own count (as torch.optim.AdamW's per-parameter
    ``step``).  A parameter without ``.grad`` takes the step with a zero
    gradient, as the reference's MixedPrecisionManager.copy_grads_to_master
    fills missing gradients with zeros before the inner optimizer's step
    (femtotron/training/mixed_precision_manager.py:224-229), so every
    parameter steps every time, as there."""

    def __init__(self, params: Iterable, lr: float = 1e-4, betas=(0.9, 0.95), eps: float = 1e-8,
                 weight_decay: float = 0.0, max_grad_norm: float | None = 1.0):
        super().__init__(params, dict(lr=float(lr), betas=tuple(float(b) for b in betas),
                                      eps=float(eps), weight_decay=float(weight_decay)))
        self.max_grad_norm = float(max_grad_norm) if max_grad_norm else 0.0
        self.step_count = 0
        dtype = device = None
        for g in self.param_groups:
            for p in g["params"]:
                if dtype is None:
                    dtype, device = p.dtype, p.device
                if p.dtype not in (torch.bfloat16, torch.float32) or not p.is_cuda:
                    raise ValueError("FusedAdamW: parameters must be bf16 or fp32 on a HIP device")
                if p.dtype != dtype or p.device != device:
                    raise ValueError("FusedAdamW: all parameters must share one dtype and device")
                if not p.is_contiguous() or not _aligned(p):
                    raise ValueError("FusedAdamW: parameters must be contiguous and 16-byte aligned")
                master = p.detach().float().clone()
                self.state[p] = {"step": 0, "master": master, "exp_avg": torch.zeros_like(master),
                                 "exp_avg_sq": torch.zeros_like(master)}
        self.dtype, self.device = dtype, device
        self.grad_norm: torch.Tensor | None = None
        self._cache = None  # (table bytes, device table, device chunk_start, total chunks)
        self._staging = [None, None]  # two pinned upload buffers, used alternately

    @property
    def entries(self) -> list[tuple[torch.Tensor, float, torch.Tensor, torch.Tensor, torch.Tensor]]:
        """(param, weight_decay, master, exp_avg, exp_avg_sq) in group order."""
        out = []
        for g in self.param_groups:
            for p in g["params"]:
                st = self.state[p]
                out.append((p, g["weight_decay"], st["master"], st["exp_avg"], st["exp_avg_sq"]))
        return out

    @property
    def masters(self) -> list[torch.Tensor]:
        return [e[2] for e in self.entries]

    def _hyper(self) -> tuple[float, float, float, float]:
        g0 = self.param_groups[0]
        lr, (b1, b2), eps = g0["lr"], g0["betas"], g0["eps"]
        for g in self.param_groups[1:]:
            if g["lr"] != lr or tuple(g["betas"]) != (b1, b2) or g["eps"] != eps:
                raise ValueError("FusedAdamW: all parameter groups must share lr, betas and eps")
        return float(lr), float(b1), float(b2), float(eps)

    def _device_table(self, live: list, grads: list, lr: float, b1: float, b2: float
                      ) -> tuple[torch.Tensor, torch.Tensor, int]:
        """The tensor table and chunk prefix sums on the device, for the step
        that is about to run (each live parameter's step count already
        incremented).  Uploaded through one of two pinned buffers used in turn,
        without blocking the host on the stream; a buffer is reused only after
        the copy that last read it has completed."""
        table = (_Tensor * len(live))()
        starts = [0]
        for i, ((p, wd, master, m, v), g) in enumerate(zip(live, grads)):
            if g.dtype != p.dtype or not g.is_contiguous() or not _aligned(g) or g.shape != p.shape \
                    or g.device != p.device:
                raise ValueError("FusedAdamW: gradients must be contiguous, aligned, of the parameter's "
                                 "dtype, shape and device")
            t = self.state[p]["step"]
            # torch.optim.AdamW (single-tensor and foreach): bias corrections in
            # double precision on the host, step_size = lr / bias_correction1
            step_size = lr / (1.0 - b1 ** t)
            bc2_sqrt = math.sqrt(1.0 - b2 ** t)
            table[i] = _Tensor(p.data_ptr(), g.data_ptr(), master.data_ptr(), m.data_ptr(), v.data_ptr(),
                               p.numel(), 1.0 - lr * wd, step_size, bc2_sqrt, 0.0)
            starts.append(starts[-1] + (p.numel() + CHUNK - 1) // CHUNK)
        key = bytes(table)
        n_tab, n_cs = len(key), 8 * len(starts)
        if self._cache is None or self._cache[0] != key:
            slot = self._staging.pop(0)
            if slot is None or slot[0].numel() < n_tab + n_cs:
                host = torch.empty(n_tab + n_cs, dtype=torch.uint8, pin_memory=True)
                slot = (host, torch.cuda.Event())
            else:
                slot[1].synchronize()  # the upload that last read this buffer is done
            host = slot[0]
            ctypes.memmove(host.data_ptr(), key, n_tab)
            ctypes.memmove(host.data_ptr() + n_tab, (ctypes.c_int64 * len(starts))(*starts), n_cs)
            dev = host[:n_tab + n_cs].to(self.device, non_blocking=True)
            slot[1].record(torch.cuda.current_stream(self.device))
            self._staging.append(slot)
            self._cache = (key, dev[:n_tab], dev[n_tab:], starts[-1])
        return self._cache[1], self._cache[2], self._cache[3]

    @torch.no_grad()
    def step(self, closure=None):
        """One optimizer step on every parameter (all in one ``fh_adamw_step``
        call; a missing gradient counts as zeros).  ``grad_norm`` then holds the pre-clipping
        global gradient norm as a device scalar."""
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        live = self.entries
        if not live:
            return loss
        grads = [e[0].grad if e[0].grad is not None else torch.zeros_like(e[0]) for e in live]
        lr, b1, b2, eps = self._hyper()
        self.step_count += 1
        for e in live:
            self.state[e[0]]["step"] += 1
        tab, chunk_start, total = self._device_table(live, grads, lr, b1, b2)
        ws = torch.empty(max(_lib.lib().fh_adamw_workspace_size(total), 4) // 4, dtype=torch.float32,
                         device=self.device)
        hyper = FhAdamHyper(1.0 - b1, b2, 1.0 - b2, eps)
        dt = 0 if self.dtype == torch.bfloat16 else 1
        stream = torch.cuda.current_stream(self.device).cuda_stream
        _lib.call("fh_adamw_step", dt, tab.data_ptr(), chunk_start.data_ptr(), len(live), total,
                  hyper, self.max_grad_norm, ws.data_ptr(), stream)
        self.grad_norm = ws[total + 1]
        return loss

    def state_dict(self) -> dict:
        """torch's optimizer format (state by parameter index, param_groups:
        per parameter ``step``, ``master``, ``exp_avg``, ``exp_avg_sq``) plus
        ``fused_step``, the number of ``step()`` calls."""
        sd = super().state_dict()
        sd["fused_step"] = self.step_count
        return sd

    def load_state_dict(self, state_dict: dict) -> None:
        """Copies masters and moments into the existing fp32 state (torch's
        default would cast them to the parameters' dtype) and restores the
        group hyper-parameters and the step count."""
        groups = state_dict["param_groups"]
        if len(groups) != len(self.param_groups) or any(
                len(a["params"]) != len(b["params"]) for a, b in zip(groups, self.param_groups)):
            raise ValueError("FusedAdamW.load_state_dict: parameter groups do not match")
        for saved, g in zip(groups, self.param_groups):
            for k, v in saved.items():
                if k != "params":
                    g[k] = v
            for idx, p in zip(saved["params"], g["params"]):
                st = state_dict["state"][idx]
                for k in ("master", "exp_avg", "exp_avg_sq"):
                    self.state[p][k].copy_(st[k])
                self.state[p]["step"] = int(st.get("step", state_dict.get("fused_step", 0)))
        self.step_count = int(state_dict.get("fused_step", 0))
        self._cache = None
