"""The shipped TunableOp solutions for the layer GEMMs (femtotron_amd/gemm_tuning.py).

CPU: the results file is well formed, validated for gfx950, and covers every
projection GEMM of the TinyLlama step in all three layouts (forward x@W^T,
input gradient dY@W, weight gradient dY^T@X; TunableOp's keys follow the
column-major BLAS view, so torch's x@W^T is "tn_N_T_K" and so on).
GPU: the full TinyLlama layer with the tuned solutions active still matches the
reference path (HF layer + torch checkpoint, same GEMM selection) within the
north star's tensor-level bf16 bound.
"""
from __future__ import annotations

import pytest
import torch

from femtotron_amd import gemm_tuning


def _entries():
    val, res = {}, {}
    for line in gemm_tuning.RESULTS_FILE.read_text().splitlines():
        parts = line.split(",")
        if parts[0] == "Validator":
            val[parts[1]] = parts[2]
        elif line:
            assert len(parts) == 4, line
            float(parts[3])
            res[(parts[0], parts[1].split("_ld_")[0])] = parts[2]
    return val, res


def test_shipped_results_cover_the_tinyllama_step():
    val, res = _entries()
    assert val["GCN_ARCH_NAME"].startswith("gfx950")
    assert {"PT_VERSION", "HIPBLASLT_VERSION", "ROCBLAS_VERSION"} <= set(val)
    T = gemm_tuning.WORKLOADS["tinyllama"][0]
    for name, N, K in gemm_tuning.layer_gemm_shapes("tinyllama"):
        if name in ("q", "kv", "gate"):
            continue  # shapes of the separate projections (reference path only)
        assert ("GemmTunableOp_BFloat16_TN", f"tn_{N}_{T}_{K}") in res, f"{name} forward"
        if name == "lm_head":
            continue
        assert ("GemmTunableOp_BFloat16_NN", f"nn_{K}_{T}_{N}") in res, f"{name} input gradient"
        assert ("GemmTunableOp_BFloat16_NT", f"nt_{K}_{N}_{T}") in res, f"{name} weight gradient"


@pytest.mark.gpu
def test_full_tinyllama_layer_with_tuned_gemms_matches_stock():
    from tests.helpers import BF16_ATOL, BF16_RTOL, CFG3
    from tests.test_layer_gpu import _compare, _run_layer
    tunable = torch.cuda.tunable
    assert gemm_tuning.use_tuned_gemms()
    try:
        got = _run_layer(CFG3, 8, 2048, torch.bfloat16, fused=True)
        ref = _run_layer(CFG3, 8, 2048, torch.bfloat16, fused=False)
        _compare(got, ref, BF16_RTOL, BF16_ATOL, "tinyllama-tuned-gemms")
    finally:
        tunable.enable(False)
