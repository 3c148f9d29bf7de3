"""fh_rmsnorm_bwd_noalloc: the allocation-free RMSNorm backward (C ABI).

Called through the C ABI with no workspace, it must give the same dx and dw,
bit for bit, as fh_rmsnorm_bwd with a caller-provided workspace: on two calls
in a row, the second with a smaller input (the library's scratch then holds
the first call's partial rows, which must not leak into the second), with
and without the residual gradient and the saved row statistics, in bf16 and
fp32.
"""
from __future__ import annotations

import ctypes

import pytest
import torch

from femtotron_amd import _lib

pytestmark = pytest.mark.gpu


def _fptr(t):
    return None if t is None else ctypes.cast(t.data_ptr(), ctypes.POINTER(ctypes.c_float))


def _ptr(t):
    return None if t is None else t.data_ptr()


def _call(noalloc: bool, dy, x, w, rstd, dres, eps=1e-5):
    L = _lib.lib()
    rows, cols = x.shape
    dt = _lib.FH_BF16 if x.dtype == torch.bfloat16 else _lib.FH_F32
    dx = torch.full_like(x, float("nan"))
    dw = torch.full_like(w, float("nan"))
    stream = torch.cuda.current_stream().cuda_stream
    if noalloc:
        st = L.fh_rmsnorm_bwd_noalloc(dt, _ptr(dy), _ptr(x), _ptr(w), _fptr(rstd), _ptr(dres), _ptr(dx),
                                      _ptr(dw), rows, cols, eps, stream)
    else:
        nbytes = L.fh_rmsnorm_bwd_workspace_size(rows, cols)
        ws = torch.empty(max(nbytes, 4), dtype=torch.uint8, device=x.device)
        st = L.fh_rmsnorm_bwd(dt, _ptr(dy), _ptr(x), _ptr(w), _fptr(rstd), _ptr(dres), _ptr(dx),
                              _ptr(dw), _ptr(ws), rows, cols, eps, stream)
    assert st == 0, L.fh_last_error()
    return dx, dw


def _inputs(rows, cols, dtype, seed, with_rstd, with_res):
    g = torch.Generator(device="cuda").manual_seed(seed)
    x = torch.randn(rows, cols, device="cuda", generator=g).to(dtype)
    dy = torch.randn(rows, cols, device="cuda", generator=g).to(dtype)
    w = (1 + 0.02 * torch.randn(cols, device="cuda", generator=g)).to(dtype)
    dres = torch.randn(rows, cols, device="cuda", generator=g).to(dtype) if with_res else None
    rstd = None
    if with_rstd:
        rstd = torch.rsqrt(x.float().pow(2).mean(-1) + 1e-5).contiguous()
    return dy, x, w, rstd, dres


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("with_rstd,with_res", [(True, True), (False, False), (False, True)])
def test_noalloc_matches_workspace_entry_on_two_calls(dtype, with_rstd, with_res):
    # first call large (512 backward blocks at 8192 columns fill the scratch),
    # second call smaller in both rows and columns
    for rows, cols, seed in ((16384, 4096, 1), (1000, 2048, 2), (37, 8192, 3)):
        args = _inputs(rows, cols, dtype, seed, with_rstd, with_res)
        want_dx, want_dw = _call(False, *args)
        got_dx, got_dw = _call(True, *args)
        torch.cuda.synchronize()
        assert torch.equal(got_dx, want_dx), (rows, cols)
        assert torch.equal(got_dw, want_dw), (rows, cols)


def test_noalloc_empty_batch_and_limits():
    L = _lib.lib()
    assert L.fh_rmsnorm_bwd_noalloc_max_workspace() >= L.fh_rmsnorm_bwd_workspace_size(1 << 24, 8192)
    w = torch.ones(512, device="cuda", dtype=torch.bfloat16)
    dw = torch.full_like(w, 7.0)
    x = torch.empty(0, 512, device="cuda", dtype=torch.bfloat16)
    st = L.fh_rmsnorm_bwd_noalloc(_lib.FH_BF16, None, None, w.data_ptr(), None, None, None, dw.data_ptr(),
                                  0, 512, 1e-5, torch.cuda.current_stream().cuda_stream)
    assert st == 0 and torch.count_nonzero(dw).item() == 0
    # columns beyond the kernels' (and the scratch's) limit are refused, not run
    st = L.fh_rmsnorm_bwd_noalloc(_lib.FH_BF16, x.data_ptr(), x.data_ptr(), w.data_ptr(), None, None,
                                  x.data_ptr(), dw.data_ptr(), 4, 8200, 1e-5, None)
    assert st == 1 and b"cols" in L.fh_last_error()
