"""ctypes binding of ``libfemtohip.so`` (the C ABI declared in include/femtohip.h).

The library is built in-tree by ``femtotron_amd.csrc.build`` (``__graft_entry__.build()``).
There is no fallback: if the library is missing or does not load, ``lib()`` raises,
so a GPU run can never silently take another code path.
"""
from __future__ import annotations

import ctypes
import threading
from ctypes import POINTER, c_char_p, c_float, c_int, c_int64, c_size_t, c_void_p
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libfemtohip.so"
ABI_VERSION = 6

FH_BF16 = 0
FH_F32 = 1

FH_OK = 0

FH_GEMM_NT = 0
FH_GEMM_NN = 1
FH_GEMM_TN = 2

_V = c_void_p
_I64 = c_int64
_F = c_float


class FhAdamHyper(ctypes.Structure):
    """FhAdamHyper of include/femtohip.h (passed by value to fh_adamw_step)."""
    _fields_ = [("one_minus_beta1", c_float), ("beta2", c_float), ("one_minus_beta2", c_float),
                ("eps", c_float)]

class FhGemmProblem(ctypes.Structure):
    """fh_gemm_problem of include/femtohip.h (an array of them is passed to
    fh_gemm_bf16_grouped)."""
    _fields_ = [("a", _V), ("lda", _I64), ("b", _V), ("ldb", _I64), ("c", _V), ("ldc", _I64),
                ("residual", _V), ("ldr", _I64), ("m", _I64), ("n", _I64)]


# name -> (restype, argtypes); mirrors include/femtohip.h exactly.
SIGNATURES: dict[str, tuple] = {
    "fh_abi_version": (c_int, []),
    "fh_last_error": (c_char_p, []),
    "fh_rmsnorm_fwd": (c_int, [c_int, _V, _V, _V, POINTER(c_float), _I64, _I64, _F, _V]),
    "fh_add_rmsnorm_fwd": (c_int, [c_int, _V, _V, _V, _V, _V, POINTER(c_float), _I64, _I64, _F, _V]),
    "fh_rmsnorm_bwd_workspace_size": (c_size_t, [_I64, _I64]),
    "fh_rmsnorm_bwd": (c_int, [c_int, _V, _V, _V, POINTER(c_float), _V, _V, _V, _V, _I64, _I64, _F, _V]),
    "fh_rmsnorm_bwd_noalloc_max_workspace": (c_size_t, []),
    "fh_rmsnorm_bwd_noalloc": (c_int, [c_int, _V, _V, _V, POINTER(c_float), _V, _V, _V, _I64, _I64, _F, _V]),
    "fh_rope_fwd": (c_int, [c_int, _V, _I64, _I64, _I64, _I64, _I64, _V, _V, c_int, _V]),
    "fh_rope_bwd": (c_int, [c_int, _V, _I64, _I64, _I64, _I64, _I64, _V, _V, c_int, _V]),
    "fh_swiglu_fwd": (c_int, [c_int, _V, _V, _I64, _V, _I64, _I64, _I64, _V]),
    "fh_swiglu_bwd": (c_int, [c_int, _V, _I64, _V, _V, _I64, _V, _V, _I64, _V, _I64, _I64, _I64, _V]),
    "fh_add": (c_int, [c_int, _V, _V, _V, _I64, _V]),
    "fh_scale": (c_int, [c_int, _V, _V, _I64, _V, _V]),
    "fh_attn_fwd": (c_int, [c_int, _V, _I64, _V, _I64, _V, _I64, _V, _I64, POINTER(c_float),
                            _I64, _I64, _I64, _I64, _I64, _F, _V]),
    "fh_attn_fwd_rope": (c_int, [c_int, _V, _I64, _V, _I64, _V, _I64, _V, _I64, POINTER(c_float), _V,
                                 _I64, _I64, _I64, _I64, _I64, _I64, _F, _V, _V, c_int, _V]),
    "fh_attn_bwd_workspace_size": (c_size_t, [_I64, _I64, _I64]),
    "fh_attn_bwd": (c_int, [c_int, _V, _I64, _V, _I64, _V, _I64, _V, _I64, _V, _I64,
                            POINTER(c_float), _V, _I64, _V, _I64, _V, _I64, _V,
                            _I64, _I64, _I64, _I64, _I64, _F, _V]),
    "fh_attn_bwd_rope": (c_int, [c_int, _V, _I64, _V, _I64, _V, _I64, _V, _I64, _V, _I64,
                                 POINTER(c_float), _V, _I64, _V, _I64, _V, _I64, _V,
                                 _I64, _I64, _I64, _I64, _I64, _F, _V, _V, c_int, _V]),
    "fh_ce_fwd_bwd": (c_int, [c_int, _V, _I64, _V, _I64, _I64, _I64, _V, POINTER(c_float), _V]),
    "fh_adamw_workspace_size": (c_size_t, [_I64]),
    "fh_gemm_bf16_workspace_size": (c_size_t, [c_int, _I64, _I64, _I64]),
    "fh_gemm_bf16": (c_int, [c_int, _V, _I64, _V, _I64, _V, _I64, _V, _I64, _I64, _I64, _I64, _V, _V]),
    "fh_gemm_bf16_rope": (c_int, [_V, _I64, _V, _I64, _V, _I64, _I64, _I64, _I64, _I64, _I64, _I64,
                                  _V, _V, c_int, _V]),
    "fh_gemm_bf16_grouped_workspace_size": (c_size_t, [c_int, c_int, POINTER(FhGemmProblem), _I64]),
    "fh_gemm_bf16_grouped": (c_int, [c_int, c_int, POINTER(FhGemmProblem), _I64, _V, _V]),
    "fh_embedding_fwd": (c_int, [c_int, _V, _V, _V, _I64, _I64, _I64, _V]),
    "fh_embedding_bwd_workspace_size": (c_size_t, [_I64, _I64]),
    "fh_embedding_bwd": (c_int, [c_int, _V, _V, _V, _I64, _I64, _I64, _I64, _V, _V]),
    "fh_adamw_step": (c_int, [c_int, _V, _V, c_int, _I64, FhAdamHyper, _F, _V, _V]),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


class FemtoHipError(RuntimeError):
    """A femtohip entry point returned a non-zero status."""


def lib() -> ctypes.CDLL:
    """Load (once) and return the library; raise if it is absent or stale."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise FemtoHipError(
                f"{LIB_PATH} is missing: build it with `python -m femtotron_amd.csrc.build` "
                "(or __graft_entry__.build()) before using the fused path")
        handle = ctypes.CDLL(str(LIB_PATH))
        # the version first: a stale library may lack entry points bound below
        handle.fh_abi_version.restype = c_int
        handle.fh_abi_version.argtypes = []
        got = handle.fh_abi_version()
        if got != ABI_VERSION:
            raise FemtoHipError(f"libfemtohip ABI {got} != expected {ABI_VERSION}: rebuild it")
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = handle
        return handle


def check(status: int, name: str) -> None:
    if status != FH_OK:
        msg = lib().fh_last_error().decode(errors="replace")
        raise FemtoHipError(f"{name} failed (status {status}): {msg}")


def call(name: str, *args) -> None:
    check(getattr(lib(), name)(*args), name)
