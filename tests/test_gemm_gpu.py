"""Projection GEMMs fh_gemm_bf16 (femtotron_amd/ops.py gemm): NT, NN and TN.

Checked against a product of the same bf16 operands accumulated in fp32 (fp64
for the small shapes): every output must lie within half a bf16 ulp of the
exact value plus the accumulation bound K * 2^-24 * (|A| |B|) -- a correctly
rounded fp32-accumulated product can be no further off; a dropped term, a
wrong operand row or an untransposed layout is off by O(|A||B|/sqrt(K)).  The
bound doubles where the reference itself is fp32.  Results must be bitwise
identical between two launches (no atomics: split-K partials are summed in
slice order, stream-form segments in k order).  Shapes: every projection GEMM
of BASELINE configs 3/4/5 in all three layouts, plus ragged, strided, split-K
and stream-form cases.
"""
from __future__ import annotations

import pytest
import torch

from femtotron_amd import _lib, ops

pytestmark = pytest.mark.gpu

DEV = "cuda"
BF = torch.bfloat16


def _ref(op, a, b, dtype):
    x, y = a.to(dtype), b.to(dtype)
    if op == "nt":
        return x @ y.t(), x.abs() @ y.abs().t()
    if op == "nn":
        return x @ y, x.abs() @ y.abs()
    return x.t() @ y, x.t().abs() @ y.abs()


def _check(op, a, b, c, *, exact=True):
    """Error of c against the product, relative to the rounding + accumulation bound."""
    m, n, k = ops.gemm_dims(op, a, b)
    ref, absref = _ref(op, a, b, torch.float64 if exact else torch.float32)
    ulp = torch.exp2(torch.floor(torch.log2(ref.abs().double().clamp_min(1e-300))) - 7)
    tol = 0.5 * ulp * 1.0001 + (1 if exact else 2) * k * 2.0 ** -24 * absref.double()
    ratio = ((c.double() - ref.double()).abs() / tol).max().item()
    assert ratio <= 1.0, f"{op} {m}x{n}x{k}: error {ratio:.3f} x the bound"
    return ratio


def _operands(op, m, n, k, g, pad=0):
    def r(*s):
        return torch.randn(*s, device=DEV, generator=g).to(BF)
    if op == "nt":
        return r(m, k + pad)[:, :k], r(n, k + pad)[:, :k]
    if op == "nn":
        return r(m, k + pad)[:, :k], r(k, n + pad)[:, :n]
    return r(k, m + pad)[:, :m], r(k, n + pad)[:, :n]


# (T, out, in) of the projection GEMMs: packed q/k/v, o, packed gate/up, down
PROJECTIONS = {
    "cfg3": (16384, [(2560, 2048), (2048, 2048), (11264, 2048), (2048, 5632)]),
    "cfg4": (8192, [(6144, 4096), (4096, 4096), (28672, 4096), (4096, 14336)]),
    "cfg5": (32768, [(12288, 4096), (4096, 4096), (22016, 4096), (4096, 11008)]),
}
CASES = [(cfg, T, o, i, op) for cfg, (T, shapes) in PROJECTIONS.items() for (o, i) in shapes
         for op in ("nt", "nn", "tn")]


@pytest.mark.parametrize("cfg,T,out_f,in_f,op", CASES,
                         ids=[f"{c}-{o}x{i}-{op}" for c, _, o, i, op in CASES])
def test_projection_gemm_matches_fp32_product(cfg, T, out_f, in_f, op):
    g = torch.Generator(device=DEV).manual_seed(out_f * 7 + in_f)
    x = torch.randn(T, in_f, device=DEV, generator=g).to(BF)
    w = torch.randn(out_f, in_f, device=DEV, generator=g).to(BF)
    dy = torch.randn(T, out_f, device=DEV, generator=g).to(BF)
    a, b = {"nt": (x, w), "nn": (dy, w), "tn": (dy, x)}[op]
    c = ops.gemm(op, a, b)
    _check(op, a, b, c, exact=False)
    assert torch.equal(c, ops.gemm(op, a, b)), "not bitwise deterministic"


SMALL = [(256, 256, 64, 0), (512, 768, 256, 8), (264, 520, 192, 0), (1000, 264, 128, 8),
         (256, 2048, 16384, 0), (8, 8, 64, 0), (2048, 2048, 4096, 0), (24, 1032, 640, 16)]


@pytest.mark.parametrize("op", ["nt", "nn", "tn"])
@pytest.mark.parametrize("m,n,k,pad", SMALL)
def test_gemm_ragged_strided_split(op, m, n, k, pad):
    if op == "tn" and m % 8:
        pytest.skip("FH_GEMM_TN needs m % 8 == 0")
    g = torch.Generator(device=DEV).manual_seed(m + 3 * n + 7 * k)
    a, b = _operands(op, m, n, k, g, pad)
    c = ops.gemm(op, a, b)
    _check(op, a, b, c, exact=True)
    assert torch.equal(c, ops.gemm(op, a, b))


_OPCODE = {"nt": _lib.FH_GEMM_NT, "nn": _lib.FH_GEMM_NN, "tn": _lib.FH_GEMM_TN}


@pytest.mark.parametrize("op", ["nt", "nn", "tn"])
@pytest.mark.parametrize("m,n,k,pad", [(10232, 2040, 16384, 0), (4104, 4088, 8192, 8), (6400, 3000, 8192, 0),
                                       (12280, 2040, 16384, 8), (12288, 2048, 11264, 0)])
def test_stream_form_matches_and_is_deterministic(op, m, n, k, pad):
    # Shapes whose tiles leave the last round of CUs partly idle: the stream
    # form spreads the k-steps evenly over the CUs and adds the split tiles'
    # fp32 segments in k order.  Its workspace is the segment slots (two
    # 256 x 256 fp32 tiles per CU).  A tail of whole chunks of CUs / 8 tiles
    # (64, 128 and 96 tail tiles here) runs in XCD slabs, the others (16 and
    # 44) linearly.  The plan depends on (m, n, k) only, so every layout takes
    # it: TN (weight gradients), NN (input gradients such as the gate/up one
    # at 12288 tokens) and NT.
    cus = torch.cuda.get_device_properties(0).multi_processor_count // 8 * 8
    assert _lib.lib().fh_gemm_bf16_workspace_size(_OPCODE[op], m, n, k) == 2 * cus * 256 * 256 * 4
    g = torch.Generator(device=DEV).manual_seed(m + n + k)
    a, b = _operands(op, m, n, k, g, pad)
    c = ops.gemm(op, a, b)
    _check(op, a, b, c, exact=True)
    assert torch.equal(c, ops.gemm(op, a, b))


@pytest.mark.parametrize("op", ["nt", "nn", "tn"])
@pytest.mark.parametrize("m,n,k", [(4104, 4088, 8192), (10240, 2048, 4096)])
def test_stream_form_residual_epilogue_rounds_like_the_unfused_add(op, m, n, k):
    """The stream form's residual epilogue (whole tiles in the GEMM, split tiles
    in the fixup; linear tail and XCD slabs) gives to_bf16(R + to_bf16(A.B))
    bit for bit, also in place."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count // 8 * 8
    assert _lib.lib().fh_gemm_bf16_workspace_size(_OPCODE[op], m, n, k) == 2 * cus * 256 * 256 * 4
    g = torch.Generator(device=DEV).manual_seed(17)
    a, b = _operands(op, m, n, k, g)
    r = torch.randn(m, n, device=DEV, generator=g).to(BF)
    fused = ops.gemm(op, a, b, residual=r)
    unfused = (r.float() + ops.gemm(op, a, b).float()).to(BF)
    assert torch.equal(fused, unfused)
    inplace = r.clone()
    ops.gemm(op, a, b, residual=inplace, out=inplace)
    assert torch.equal(inplace, fused)


@pytest.mark.parametrize("m,n,k,pad", [(16384, 2048, 5632, 0), (6144, 3072, 512, 0), (6144, 3072, 512, 64)])
def test_persistent_form_residual_epilogue_rounds_like_the_unfused_add(m, n, k, pad):
    """The persistent form's residual epilogue (the down projection at config
    3: 512 tiles, two whole rounds; 288 tiles: a partial second round; with
    pad, R and C views of wider rows, ldr != ldc != n) gives
    to_bf16(R + to_bf16(A.B^T)) bit for bit, also in place (R = C)."""
    g = torch.Generator(device=DEV).manual_seed(m + k)
    a, b = _operands("nt", m, n, k, g)
    r = torch.randn(m, n + pad, device=DEV, generator=g).to(BF)[:, :n]
    product = ops.gemm("nt", a, b)
    _check("nt", a, b, product, exact=True)
    out = torch.full((m, n + 2 * pad), 7.0, device=DEV, dtype=BF)
    fused = ops.gemm("nt", a, b, residual=r, out=out[:, :n])
    assert torch.equal(fused, (r.float() + product.float()).to(BF))
    assert pad == 0 or bool((out[:, n:] == 7.0).all()), "columns past n written"
    inplace = r.clone()
    ops.gemm("nt", a, b, residual=inplace, out=inplace)
    assert torch.equal(inplace, fused)


def test_split_k_path_is_used_and_matches():
    # 512 x 512 outputs are 4 tiles: the k range is split into slices
    m = n = 512
    k = 16384
    assert _lib.lib().fh_gemm_bf16_workspace_size(_lib.FH_GEMM_TN, m, n, k) > 0
    g = torch.Generator(device=DEV).manual_seed(5)
    a, b = _operands("tn", m, n, k, g)
    c = ops.gemm("tn", a, b)
    _check("tn", a, b, c, exact=True)
    assert torch.equal(c, ops.gemm("tn", a, b))


@pytest.mark.parametrize("op", ["nt", "nn", "tn"])
@pytest.mark.parametrize("m,n,k", [(512, 768, 256), (264, 520, 192), (512, 512, 16384)])
def test_residual_epilogue_rounds_like_the_unfused_add(op, m, n, k):
    """C = to_bf16(R + to_bf16(A.B)) -- the projection output rounded, then the
    residual add of modeling_llama.py:323 rounded again -- bit for bit."""
    g = torch.Generator(device=DEV).manual_seed(m + n)
    a, b = _operands(op, m, n, k, g)
    r = torch.randn(m, n, device=DEV, generator=g).to(BF)
    fused = ops.gemm(op, a, b, residual=r)
    unfused = (r.float() + ops.gemm(op, a, b).float()).to(BF)
    assert torch.equal(fused, unfused)
    inplace = r.clone()
    ops.gemm(op, a, b, residual=inplace, out=inplace)
    assert torch.equal(inplace, fused)


@pytest.mark.parametrize("op,shapes,k,one_launch", [
    # the layer's q/k/v, o and down weight gradients at config 3: 80 + 64 + 176
    # tiles, one stream launch (a whole round, then 64 tail tiles in XCD slabs)
    ("tn", [(2560, 2048), (2048, 2048), (2048, 5632)], 16384, True),
    ("tn", [(2560, 2048), (2048, 2048), (2048, 5632)], 256, True),       # 4 k-steps
    ("tn", [(6144, 4096), (4096, 4096), (4096, 14336)], 1024, True),     # config 4's: six whole rounds, no tail
    ("tn", [(520, 264), (1032, 776)], 8192, False),                      # ragged, too few tiles: one call each
    ("tn", [(2600, 2056), (2048, 2048), (2048, 5640)], 4096, True),      # ragged edge tiles in one launch
    ("nn", [(4096, 2048), (4096, 2560)], 2048, True),                    # the other layouts: 128 + 160 tiles
    ("nt", [(4096, 2048), (4104, 2568)], 2048, True),
])
def test_grouped_matches_each_product_and_accumulates(op, shapes, k, one_launch):
    """fh_gemm_bf16_grouped: every problem within the product's bound, bitwise
    repeatable, and with residual == C the accumulating epilogue
    to_bf16(R + to_bf16(A^T B)) bit for bit (whole tiles in the GEMM, split ones
    in the fixup); a group whose tiles do not fill a round runs as separate
    fh_gemm_bf16 calls."""
    g = torch.Generator(device=DEV).manual_seed(k + len(shapes))
    ops_ = [_operands(op, m, n, k, g) for m, n in shapes]
    probs = (_lib.FhGemmProblem * len(shapes))()
    for i, ((a, b), (m, n)) in enumerate(zip(ops_, shapes)):
        probs[i] = _lib.FhGemmProblem(a.data_ptr(), a.stride(0), b.data_ptr(), b.stride(0), None, n, None, 0, m, n)
    code = {"nt": _lib.FH_GEMM_NT, "nn": _lib.FH_GEMM_NN, "tn": _lib.FH_GEMM_TN}[op]
    ws = _lib.lib().fh_gemm_bf16_grouped_workspace_size(code, len(shapes), probs, k)
    cus = torch.cuda.get_device_properties(0).multi_processor_count // 8 * 8
    if one_launch:
        assert ws == 2 * cus * 256 * 256 * 4
    outs = ops.gemm_grouped(op, [(a, b, None, None) for a, b in ops_])
    for (a, b), c in zip(ops_, outs):
        _check(op, a, b, c, exact=True)
    again = ops.gemm_grouped(op, [(a, b, None, None) for a, b in ops_])
    assert all(torch.equal(x, y) for x, y in zip(outs, again))
    if not one_launch:  # separate calls: each is its own fh_gemm_bf16
        assert all(torch.equal(c, ops.gemm(op, a, b)) for (a, b), c in zip(ops_, outs))
    rs = [torch.randn(m, n, device=DEV, generator=g).to(BF) for m, n in shapes]
    acc = [r.clone() for r in rs]
    got = ops.gemm_grouped(op, [(a, b, x, x) for (a, b), x in zip(ops_, acc)])
    for r, x, y, c in zip(rs, acc, got, outs):
        assert y.data_ptr() == x.data_ptr()
        assert torch.equal(x, (r.float() + c.float()).to(BF))


def test_grouped_rejects_bad_arguments():
    x = torch.randn(256, 256, device=DEV).to(BF)
    with pytest.raises(ValueError):
        ops.gemm_grouped("tn", [])
    with pytest.raises(ValueError):
        ops.gemm_grouped("tn", [(x, x, None, None)] * 4)
    with pytest.raises(ValueError):  # the problems' k differ
        ops.gemm_grouped("tn", [(x, x, None, None), (x[:128], x[:128], None, None)])
    probs = (_lib.FhGemmProblem * 1)()
    probs[0] = _lib.FhGemmProblem(x.data_ptr(), 256, x.data_ptr(), 256, x.data_ptr(), 256, None, 0, 256, 256)
    st = _lib.lib().fh_gemm_bf16_grouped(_lib.FH_GEMM_TN, 4, probs, 256, None, None)
    assert st == 1 and b"between 1 and 3" in _lib.lib().fh_last_error()
    st = _lib.lib().fh_gemm_bf16_grouped(_lib.FH_GEMM_TN, 1, probs, 96, None, None)
    assert st == 1 and b"multiple of 64" in _lib.lib().fh_last_error()


def test_gemm_rejects_unsupported_operands():
    a = torch.randn(128, 96, device=DEV).to(BF)  # k = 96 is not a multiple of 64
    b = torch.randn(256, 96, device=DEV).to(BF)
    assert not ops.gemm_supported("nt", a, b)
    with pytest.raises(ValueError):
        ops.gemm("nt", a, b)
    assert not ops.gemm_supported("nt", a.float(), b.float())
    x = torch.randn(256, 128, device=DEV).to(BF)
    assert not ops.gemm_supported("tn", x[:, :100], x)  # m % 8 for TN
    # the C ABI itself refuses bad arguments with a message, never aborts
    st = _lib.lib().fh_gemm_bf16(7, x.data_ptr(), 128, x.data_ptr(), 128, x.data_ptr(), 128, None, 0,
                                 128, 128, 128, None, None)
    assert st == 1 and b"op" in _lib.lib().fh_last_error()
    st = _lib.lib().fh_gemm_bf16(_lib.FH_GEMM_NT, x.data_ptr(), 128, x.data_ptr(), 128, x.data_ptr(),
                                 128, None, 0, 128, 128, 96, None, None)
    assert st == 1 and b"multiple of 64" in _lib.lib().fh_last_error()
    # the output tile is written in 16-byte rows: C and the residual need ldc % 8 and 16-byte alignment
    st = _lib.lib().fh_gemm_bf16(_lib.FH_GEMM_NT, x.data_ptr(), 128, x.data_ptr(), 128, x.data_ptr(),
                                 132, None, 0, 128, 128, 128, None, None)
    assert st == 1 and b"multiples of 8" in _lib.lib().fh_last_error()
    st = _lib.lib().fh_gemm_bf16(_lib.FH_GEMM_NT, x.data_ptr(), 128, x.data_ptr(), 128, x.data_ptr() + 8,
                                 128, None, 0, 64, 128, 128, None, None)
    assert st == 1 and b"16-byte aligned" in _lib.lib().fh_last_error()
    wide = torch.empty(128, 132, device=DEV, dtype=BF)
    with pytest.raises(ValueError):
        ops.gemm("nt", x, x, out=wide[:, :128])


@pytest.mark.parametrize("m,seq,nh,nkv,hd,k,per_token", [
    (16384, 2048, 32, 4, 64, 2048, False),  # the TinyLlama q/k/v projection
    (600, 200, 8, 2, 64, 256, False),       # ragged m (not a multiple of the 256-row tile), 3 sequences
    (333, 111, 4, 4, 32, 128, True),        # per-token tables, MHA, head_dim 32
    (512, 256, 4, 1, 128, 192, False),      # head_dim 128, MQA
])
def test_gemm_rope_equals_gemm_then_rope_fwd(m, seq, nh, nkv, hd, k, per_token):
    """fh_gemm_bf16_rope == fh_gemm_bf16 (NT) followed by fh_rope_fwd over the q and
    k heads, bit for bit; the v heads are the plain product.  Random tables
    (cos[i] != cos[i + hd/2]) so that a partner or sign mix-up shows."""
    g = torch.Generator(device=DEV).manual_seed(m + hd)
    n = (nh + 2 * nkv) * hd
    a, b = _operands("nt", m, n, k, g)
    rows = m if per_token else seq
    cos = torch.randn(rows, hd, device=DEV, generator=g).to(BF)
    sin = torch.randn(rows, hd, device=DEV, generator=g).to(BF)
    assert _lib.lib().fh_gemm_bf16_workspace_size(_lib.FH_GEMM_NT, m, n, k) == 0  # one K slice
    ref = ops.gemm("nt", a, b)
    plain_v = ref[:, (nh + nkv) * hd:].clone()
    ops.rope_fwd_(ref, nh + nkv, hd, seq, cos, sin)
    assert torch.equal(ref[:, (nh + nkv) * hd:], plain_v)
    got = ops.gemm_rope(a, b, nh + nkv, hd, seq, cos, sin)
    assert torch.equal(got, ref)


def test_gemm_rope_rejects_bad_arguments():
    from femtotron_amd._lib import FemtoHipError
    x = torch.randn(256, 128, device=DEV).to(BF)
    cos = torch.randn(256, 48, device=DEV).to(BF)
    with pytest.raises(FemtoHipError, match="head_dim"):
        ops.gemm_rope(x, x, 2, 48, 256, cos, cos)
    c64 = torch.randn(256, 64, device=DEV).to(BF)
    lib = _lib.lib()
    # rot_cols beyond n, and m not a multiple of seq_len with per-position tables
    st = lib.fh_gemm_bf16_rope(x.data_ptr(), 128, x.data_ptr(), 128, x.data_ptr(), 128, 256, 128, 128,
                               192, 64, 256, c64.data_ptr(), c64.data_ptr(), 0, None)
    assert st == 1 and b"rot_cols" in lib.fh_last_error()
    st = lib.fh_gemm_bf16_rope(x.data_ptr(), 128, x.data_ptr(), 128, x.data_ptr(), 128, 256, 128, 128,
                               128, 64, 100, c64.data_ptr(), c64.data_ptr(), 0, None)
    assert st == 1 and b"multiple of seq_len" in lib.fh_last_error()
