"""Weight-gradient GEMM fh_gemm_tn (femtotron_amd/ops.py gemm_tn): C = A^T B.

Checker: the exact product of the same bf16 inputs in fp32 (torch on the GPU,
fp32 inputs); the kernel accumulates in fp32 and rounds once, so every output
must be within half a bf16 ulp of it plus the fp32 accumulation error (bound
used: one bf16 ulp at 2^-8 relative, plus 1e-3 absolute for near-zero
sums).  Shapes cover one slice (many output tiles) and the token-split path
(few tiles: fp32 partials summed in slice order), and leading dimensions wider
than the operand (column views of a packed buffer); results must be bitwise
deterministic.  The reference path computes the same product with
torch.mm(dY.t(), X) (F.linear's weight gradient) in bf16: within one bf16 ulp
of it as well.
"""
from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _check(a, b, c):
    ref = torch.mm(a.float().t(), b.float())
    bound = ref.abs() * 2.0 ** -8 + 1e-3
    err = (c.float() - ref).abs()
    assert bool((err <= bound).all()), f"max excess {float((err - bound).max()):.3e}"
    lib = torch.mm(a.t(), b).float()
    assert bool(((c.float() - lib).abs() <= lib.abs() * 2.0 ** -7 + 1e-3).all())


@pytest.mark.parametrize("k,m,n", [(64, 256, 256), (1024, 512, 768), (4096, 2560, 2048),
                                   (16384, 2048, 2048), (8192, 11264, 2048), (2048, 256, 5632)])
def test_gemm_tn_matches_fp32_product(k, m, n):
    from femtotron_amd import ops
    g = torch.Generator(device=DEV).manual_seed(k + m + n)
    a = torch.randn(k, m, device=DEV, generator=g).bfloat16()
    b = torch.randn(k, n, device=DEV, generator=g).bfloat16()
    c = ops.gemm_tn(a, b)
    _check(a, b, c)
    assert torch.equal(c, ops.gemm_tn(a, b))  # deterministic, also on the split path


def test_gemm_tn_strided_operands_and_slices():
    """Operands as column views of wider buffers (lda, ldb > m, n), and the
    slice count the host picks for this shape is > 1 (workspace used)."""
    from femtotron_amd import _lib, ops
    g = torch.Generator(device=DEV).manual_seed(3)
    k, m, n = 8192, 512, 512
    abuf = torch.randn(k, m + 256, device=DEV, generator=g).bfloat16()
    bbuf = torch.randn(k, n + 512, device=DEV, generator=g).bfloat16()
    a, b = abuf[:, 256:], bbuf[:, :n]
    assert _lib.lib().fh_gemm_tn_workspace_size(m, n, k) > 0
    _check(a, b, ops.gemm_tn(a, b))


def test_gemm_tn_rejects_unsupported_shapes():
    from femtotron_amd import ops
    a = torch.zeros(64, 200, device=DEV, dtype=torch.bfloat16)
    b = torch.zeros(64, 256, device=DEV, dtype=torch.bfloat16)
    assert not ops.gemm_tn_supported(a, b)
    with pytest.raises(ValueError):
        ops.gemm_tn(a, b)
    assert not ops.gemm_tn_supported(b.float(), b.float())
