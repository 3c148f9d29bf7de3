"""Parity of the femtohip flash-attention kernels (GPU) with the closed-form /
oracle attention: forward output and lse, and dq/dk/dv, for GQA groupings,
head dims 32/64/128, ragged sequence lengths (not multiples of the 64/128
tiles) and batch > 1.  bf16 runs on MFMA and is checked against the fp64 closed
form on the same bf16-valued inputs; fp32 at 1e-5.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import closed_form as cf
from tests.helpers import randn

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _ops():
    from femtotron_amd import ops
    return ops


def _inputs(B, S, nh, nkv, hd, dtype, seed):
    """Token-major q|k|v buffer [T, (nh+2nkv)*hd] (the layer's layout) and dO."""
    T = B * S
    buf = randn((T, (nh + 2 * nkv) * hd), seed).to(dtype)
    do = randn((T, nh * hd), seed + 1).to(dtype)
    return buf, do


def _heads(x, B, S, n, hd):
    """[T, n*hd] token-major -> [B, n, S, hd] float64 numpy."""
    return x.double().reshape(B, S, n, hd).permute(0, 2, 1, 3).numpy()


def _tok(a, B, S, n, hd):
    return torch.from_numpy(np.ascontiguousarray(a.transpose(0, 2, 1, 3).reshape(B * S, n * hd)))


def _run(B, S, nh, nkv, hd, dtype, seed=0):
    ops = _ops()
    buf, do = _inputs(B, S, nh, nkv, hd, dtype, seed)
    g = buf.to(DEV)
    hq, hkv = nh * hd, nkv * hd
    q, k, v = g[:, :hq], g[:, hq:hq + hkv], g[:, hq + hkv:]
    scale = hd ** -0.5
    o, lse = ops.attn_fwd(q, k, v, B, S, nh, nkv, hd, scale)
    dg = torch.empty_like(g)
    dq, dk, dv = dg[:, :hq], dg[:, hq:hq + hkv], dg[:, hq + hkv:]
    ops.attn_bwd(q, k, v, o, do.to(DEV), lse, dq, dk, dv, B, S, nh, nkv, hd, scale)
    # closed form on the same (rounded) values
    qn = _heads(buf[:, :hq], B, S, nh, hd)
    kn = _heads(buf[:, hq:hq + hkv], B, S, nkv, hd)
    vn = _heads(buf[:, hq + hkv:], B, S, nkv, hd)
    don = _heads(do, B, S, nh, hd)
    ro, rl = cf.attention_fwd(qn, kn, vn, scale)
    rdq, rdk, rdv = cf.attention_bwd(don, qn, kn, vn, scale)
    ref = dict(o=_tok(ro, B, S, nh, hd), lse=torch.from_numpy(rl), dq=_tok(rdq, B, S, nh, hd),
               dk=_tok(rdk, B, S, nkv, hd), dv=_tok(rdv, B, S, nkv, hd))
    got = dict(o=o, lse=lse, dq=dq, dk=dk, dv=dv)
    return {k_: got[k_].float().cpu() for k_ in got}, {k_: ref[k_].float() for k_ in ref}


def _tensor_err(a, b):
    return float((a - b).abs().max() / b.abs().max().clamp_min(1e-30))


@pytest.mark.parametrize("B,S,nh,nkv,hd", [
    (2, 128, 8, 4, 32),     # cfg 1 heads
    (1, 256, 32, 4, 64),    # TinyLlama heads, short
    (2, 200, 4, 1, 64),     # ragged S, MQA
    (1, 300, 8, 8, 128),    # MHA, hd 128, ragged
    (1, 130, 32, 8, 128),   # Llama-3 grouping
    (3, 65, 2, 2, 64),      # S just past one key block
    (1, 300, 4, 2, 64),     # odd count of 128-key blocks: the middle block is paired with itself
    (1, 1, 4, 2, 64),       # single token: output is v
    (2, 77, 4, 2, 32),      # hd 32, ragged
    (1, 33, 4, 4, 128),     # hd 128, one partial 32-query tile past a full one
])
def test_attention_bf16_matches_closed_form(B, S, nh, nkv, hd):
    got, ref = _run(B, S, nh, nkv, hd, torch.bfloat16)
    assert torch.isfinite(got["o"]).all() and torch.isfinite(got["dq"]).all()
    # bf16 output rounding + bf16 P operand: a few 1e-3 relative at the tensor level
    assert _tensor_err(got["o"], ref["o"]) < 1e-2, _tensor_err(got["o"], ref["o"])
    assert (got["lse"] - ref["lse"]).abs().max() < 2e-3
    for name in ("dq", "dk", "dv"):
        # max|a-b| <= rtol*max|b| + atol; atol covers gradients that vanish
        # mathematically (S = 1 makes dq exactly 0)
        err = float((got[name] - ref[name]).abs().max())
        assert err <= 2e-2 * float(ref[name].abs().max()) + 1e-3, f"{name}: {err:.3e}"


@pytest.mark.parametrize("B,S,nh,nkv,hd", [(2, 128, 8, 4, 32), (1, 77, 4, 2, 64), (1, 40, 2, 1, 128)])
def test_attention_fp32_matches_closed_form_1e5(B, S, nh, nkv, hd):
    got, ref = _run(B, S, nh, nkv, hd, torch.float32)
    for name in ("o", "dq", "dk", "dv"):
        e = _tensor_err(got[name], ref[name])
        assert e < 1e-5, f"{name}: {e:.3e}"
    assert (got["lse"] - ref["lse"]).abs().max() < 1e-5


@pytest.mark.parametrize("hd", [32, 64, 128])
def test_attention_ragged_tiles_stay_inside_their_sequence(hd):
    """Tiles that run past S load clamped rows of their own sequence, never the
    next one: with every q/k/v/dO value of sequence 1 set to NaN, sequence 0's
    output, lse and gradients are bit-identical to a run with finite values
    there (a read of sequence 1 would carry a NaN through P V or dS Q)."""
    ops = _ops()
    B, S, nh, nkv = 2, 77, 4, 2
    hq, hkv = nh * hd, nkv * hd
    buf, do = _inputs(B, S, nh, nkv, hd, torch.bfloat16, 9)
    outs = []
    for poison in (False, True):
        g, d = buf.clone().to(DEV), do.clone().to(DEV)
        if poison:
            g[S:] = float("nan")
            d[S:] = float("nan")
        q, k, v = g[:, :hq], g[:, hq:hq + hkv], g[:, hq + hkv:]
        o, lse = ops.attn_fwd(q, k, v, B, S, nh, nkv, hd, hd ** -0.5)
        dg = torch.empty_like(g)
        ops.attn_bwd(q, k, v, o, d, lse, dg[:, :hq], dg[:, hq:hq + hkv], dg[:, hq + hkv:], B, S, nh, nkv, hd,
                     hd ** -0.5)
        outs.append((o[:S].cpu(), lse.view(B, nh, S)[0].cpu(), dg[:S].cpu()))
    for a, b in zip(*outs):
        assert torch.isfinite(a).all() and torch.equal(a, b)


def test_attention_single_token_is_v():
    got, ref = _run(1, 1, 4, 2, 64, torch.bfloat16)
    buf, _ = _inputs(1, 1, 4, 2, 64, torch.bfloat16, 0)
    v = buf[:, (4 + 2) * 64:].float()
    expect = torch.cat([v[:, :64], v[:, :64], v[:, 64:], v[:, 64:]], 1)  # q heads 0,1 -> kv 0; 2,3 -> kv 1
    assert torch.equal(got["o"], expect)


def test_attention_deterministic_and_causal_full_size():
    """TinyLlama attention shape (B=8, S=2048, 32/4 heads, hd 64): run-to-run
    bitwise determinism, and causality (perturbing the last token's k/v changes
    only the last query's output)."""
    ops = _ops()
    B, S, nh, nkv, hd = 8, 2048, 32, 4, 64
    buf, do = _inputs(B, S, nh, nkv, hd, torch.bfloat16, 5)
    g = buf.to(DEV)
    hq, hkv = nh * hd, nkv * hd
    args = (B, S, nh, nkv, hd, hd ** -0.5)
    o1, l1 = ops.attn_fwd(g[:, :hq], g[:, hq:hq + hkv], g[:, hq + hkv:], *args)
    o2, l2 = ops.attn_fwd(g[:, :hq], g[:, hq:hq + hkv], g[:, hq + hkv:], *args)
    assert torch.equal(o1, o2) and torch.equal(l1, l2)
    grads = []
    for _ in range(2):
        dg = torch.empty_like(g)
        ops.attn_bwd(g[:, :hq], g[:, hq:hq + hkv], g[:, hq + hkv:], o1, do.to(DEV), l1,
                     dg[:, :hq], dg[:, hq:hq + hkv], dg[:, hq + hkv:], *args)
        grads.append(dg)
    assert torch.equal(grads[0], grads[1])
    g2 = g.clone()
    last = torch.arange(B, device=DEV) * S + S - 1
    g2[last, hq:] += 1.0
    o3, _ = ops.attn_fwd(g2[:, :hq], g2[:, hq:hq + hkv], g2[:, hq + hkv:], *args)
    keep = torch.ones(B * S, dtype=torch.bool, device=DEV)
    keep[last] = False
    assert torch.equal(o3[keep], o1[keep])
    assert not torch.equal(o3[last], o1[last])
    # sanity against the fp32 math on one (batch, head) slice
    qb = buf[:S, :hd].double()
    kb = buf[:S, hq:hq + hd].double()
    vb = buf[:S, hq + hkv:hq + hkv + hd].double()
    s = (qb @ kb.T) * hd ** -0.5
    s = s.masked_fill(torch.ones(S, S, dtype=torch.bool).triu(1), float("-inf"))
    ref = torch.softmax(s, -1) @ vb
    assert _tensor_err(o1[:S, :hd].float().cpu(), ref.float()) < 1e-2


def test_attention_rejects_bad_head_dim():
    from femtotron_amd._lib import FemtoHipError
    x = torch.zeros(16, 3 * 48, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(FemtoHipError, match="head_dim"):
        _ops().attn_fwd(x[:, :48], x[:, 48:96], x[:, 96:], 1, 16, 1, 1, 48, 0.1)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
@pytest.mark.parametrize("B,S,nh,nkv,hd,per_token", [
    (2, 200, 8, 2, 64, False),    # GQA, ragged S, the TinyLlama head_dim
    (1, 77, 4, 4, 32, True),      # MHA, per-token tables
    (2, 131, 4, 1, 128, False),   # MQA, head_dim 128 (split-role dK/dV kernel)
    (3, 64, 32, 4, 64, True),     # TinyLlama heads, per-token tables over 3 sequences
])
def test_attention_bwd_rope_equals_bwd_then_rope_bwd(dtype, B, S, nh, nkv, hd, per_token):
    """fh_attn_bwd_rope == fh_attn_bwd followed by fh_rope_bwd over the dq and dk
    heads, bit for bit (dv untouched).  The tables are random rather than real
    cos/sin, so cos[i] != cos[i + hd/2] and sin[i] != sin[i + hd/2]: a rotation
    that took the pair's own sin in place of its partner's, or rotated by the
    wrong row, would differ."""
    ops = _ops()
    buf, do = _inputs(B, S, nh, nkv, hd, dtype, 21)
    rows = B * S if per_token else S
    cos = randn((rows, hd), 22).to(dtype).to(DEV)
    sin = randn((rows, hd), 23).to(dtype).to(DEV)
    g, d = buf.to(DEV), do.to(DEV)
    hq, hkv = nh * hd, nkv * hd
    q, k, v = g[:, :hq], g[:, hq:hq + hkv], g[:, hq + hkv:]
    args = (B, S, nh, nkv, hd, hd ** -0.5)
    o, lse = ops.attn_fwd(q, k, v, *args)
    ref = torch.empty_like(g)
    ops.attn_bwd(q, k, v, o, d, lse, ref[:, :hq], ref[:, hq:hq + hkv], ref[:, hq + hkv:], *args)
    plain_dv = ref[:, hq + hkv:].clone()
    ops.rope_bwd_(ref, nh + nkv, hd, S, cos, sin)
    assert torch.equal(ref[:, hq + hkv:], plain_dv)
    got = torch.full_like(g, float("nan"))
    ops.attn_bwd(q, k, v, o, d, lse, got[:, :hq], got[:, hq:hq + hkv], got[:, hq + hkv:], *args,
                 rope=(cos, sin))
    torch.cuda.synchronize()
    assert torch.isfinite(got).all()
    assert torch.equal(got, ref)


def test_attention_bwd_rope_rejects_bad_tables():
    ops = _ops()
    B, S, nh, nkv, hd = 1, 16, 2, 1, 32
    g = torch.zeros(B * S, (nh + 2 * nkv) * hd, dtype=torch.bfloat16, device=DEV)
    hq, hkv = nh * hd, nkv * hd
    o, lse = ops.attn_fwd(g[:, :hq], g[:, hq:hq + hkv], g[:, hq + hkv:], B, S, nh, nkv, hd, 0.1)
    dg = torch.empty_like(g)
    cos = torch.zeros(S + 1, hd, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(ValueError, match="neither seq_len nor tokens"):
        ops.attn_bwd(g[:, :hq], g[:, hq:hq + hkv], g[:, hq + hkv:], o, g[:, :hq], lse, dg[:, :hq],
                     dg[:, hq:hq + hkv], dg[:, hq + hkv:], B, S, nh, nkv, hd, 0.1, rope=(cos, cos))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
@pytest.mark.parametrize("B,S,nh,nkv,hd,per_token", [
    (2, 200, 8, 2, 64, False),
    (1, 77, 4, 4, 32, True),
    (2, 131, 4, 1, 128, False),
])
def test_attention_fwd_rope_equals_rope_then_fwd(dtype, B, S, nh, nkv, hd, per_token):
    """fh_attn_fwd_rope (q rotated on load, k already rotated) == fh_rope_fwd over
    q's heads followed by fh_attn_fwd, bit for bit: output, lse and the rotated q
    it writes out (also in place over q itself)."""
    ops = _ops()
    buf, _ = _inputs(B, S, nh, nkv, hd, dtype, 31)
    rows = B * S if per_token else S
    cos = randn((rows, hd), 32).to(dtype).to(DEV)
    sin = randn((rows, hd), 33).to(dtype).to(DEV)
    hq, hkv = nh * hd, nkv * hd
    args = (B, S, nh, nkv, hd, hd ** -0.5)
    ref = buf.to(DEV)
    ops.rope_fwd_(ref, nh + nkv, hd, S, cos, sin)  # q and k rotated
    o_ref, l_ref = ops.attn_fwd(ref[:, :hq], ref[:, hq:hq + hkv], ref[:, hq + hkv:], *args)
    g = buf.to(DEV)
    ops.rope_fwd_(g[:, hq:], nkv, hd, S, cos, sin)  # k only
    q_rot = torch.full_like(g[:, :hq], float("nan"))
    o, lse = ops.attn_fwd(g[:, :hq], g[:, hq:hq + hkv], g[:, hq + hkv:], *args, rope=(cos, sin), q_out=q_rot)
    torch.cuda.synchronize()
    assert torch.equal(o, o_ref) and torch.equal(lse, l_ref)
    assert torch.equal(q_rot, ref[:, :hq])
    o2, _ = ops.attn_fwd(g[:, :hq], g[:, hq:hq + hkv], g[:, hq + hkv:], *args, rope=(cos, sin), q_out=g[:, :hq])
    assert torch.equal(o2, o_ref) and torch.equal(g, ref)
