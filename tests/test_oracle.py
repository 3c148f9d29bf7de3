"""Pins the oracle (CPU, no GPU needed).

* oracle/torch_llama.py vs the Hugging Face modules the reference instantiates
  (LlamaDecoderLayer, LlamaRMSNorm, apply_rotary_pos_emb, LlamaRotaryEmbedding):
  fp32 to ~1e-6, bf16 to bf16 noise.
* oracle/closed_form.py (fp64, written from the math) vs central finite
  differences and vs invariants; then the oracle's autograd gradients vs the
  closed forms.  A dropped term, a sign error or a transposed head mapping in
  either statement fails one of these.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch
from transformers.models.llama import modeling_llama as hf

from oracle import closed_form as cf
from oracle import torch_llama as ot
from tests.helpers import (CFG1, F32_TOL, assert_close, hf_layer_grads, layer_weights,
                           llama_config, load_into_hf_layer, randn)


# --------------------------------------------------------------- vs HF (fp32)
@pytest.mark.parametrize("kv", [4, 8])
def test_decoder_layer_matches_hf_fp32(kv):
    c = dict(CFG1, kv=kv)
    cfg = llama_config(c, layers=1)
    layer = hf.LlamaDecoderLayer(cfg, layer_idx=0).float()
    w = layer_weights(c, seed=42, norm_mean=1.0)
    load_into_hf_layer(layer, w)
    B, S, H, hd = 2, 64, c["hidden"], c["hidden"] // c["heads"]
    x = randn((B, S, H), 7)
    cos, sin = ot.rope_cos_sin(S, hd, c["theta"], torch.float32)
    rot = hf.LlamaRotaryEmbedding(cfg)
    hc, hs = rot(x, torch.arange(S)[None])
    assert torch.equal(hc, cos) and torch.equal(hs, sin)

    x1 = x.clone().requires_grad_(True)
    ref = layer(x1, attention_mask=None, position_embeddings=(cos, sin),
                position_ids=torch.arange(S)[None], past_key_values=None, use_cache=False)
    dy = randn((B, S, H), 8)
    ref.backward(dy)

    wt = {k: v.clone().requires_grad_(True) for k, v in w.items()}
    x2 = x.clone().requires_grad_(True)
    out = ot.decoder_layer(x2, cos, sin, wt, c["heads"], kv, hd, 1e-5)
    out.backward(dy)
    assert_close(out, ref, F32_TOL, F32_TOL, "out")
    assert_close(x2.grad, x1.grad, F32_TOL, F32_TOL, "dx")
    g = hf_layer_grads(layer)
    for k in ot.LAYER_KEYS:
        assert_close(wt[k].grad, g[k], 1e-4, 1e-5, f"d{k}")


def test_decoder_layer_matches_hf_bf16():
    c = CFG1
    cfg = llama_config(c, layers=1)
    layer = hf.LlamaDecoderLayer(cfg, layer_idx=0)
    w = layer_weights(c, seed=3, norm_mean=1.0)
    load_into_hf_layer(layer, w)
    layer = layer.bfloat16()
    B, S, H, hd = 2, 32, c["hidden"], c["hidden"] // c["heads"]
    x = randn((B, S, H), 11).bfloat16()
    cos, sin = ot.rope_cos_sin(S, hd, c["theta"], torch.bfloat16)
    ref = layer(x, attention_mask=None, position_embeddings=(cos, sin),
                position_ids=torch.arange(S)[None], past_key_values=None, use_cache=False)
    wb = {k: v.bfloat16() for k, v in w.items()}
    out = ot.decoder_layer(x, cos, sin, wb, c["heads"], c["kv"], hd, 1e-5)
    assert_close(out, ref, 2e-2, 2e-2, "bf16 out")


def test_rmsnorm_and_rope_are_hf_bit_exact():
    x = randn((4, 3, 256), 1).bfloat16()
    w = (1 + randn((256,), 2, 0.02)).bfloat16()
    m = hf.LlamaRMSNorm(256, eps=1e-5)
    with torch.no_grad():
        m.weight.copy_(w.float())
    m = m.bfloat16()
    assert torch.equal(m(x), ot.rmsnorm(x, w, 1e-5))
    q = randn((2, 8, 16, 64), 3).bfloat16()
    k = randn((2, 4, 16, 64), 4).bfloat16()
    cos, sin = ot.rope_cos_sin(16, 64, 500000.0, torch.bfloat16)
    a = hf.apply_rotary_pos_emb(q, k, cos, sin)
    b = ot.rope(q, k, cos, sin)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


# ------------------------------------------------ closed forms vs finite diff
def _rng(seed):
    return np.random.default_rng(seed)


def test_rmsnorm_closed_form_finite_difference():
    r = _rng(0)
    x = r.standard_normal((3, 16))
    w = 1 + 0.1 * r.standard_normal(16)
    dy = r.standard_normal((3, 16))
    dx, dw = cf.rmsnorm_bwd(dy, x, w, 1e-5)
    assert np.allclose(dx, cf.finite_diff_grad(lambda t: cf.rmsnorm_fwd(t, w, 1e-5), x, dy), atol=1e-7)
    assert np.allclose(dw, cf.finite_diff_grad(lambda t: cf.rmsnorm_fwd(x, t, 1e-5), w.copy(), dy), atol=1e-7)
    # invariant: the normalised row has unit RMS (eps -> 0)
    n = cf.rmsnorm_fwd(x, np.ones(16), 0.0)
    assert np.allclose(np.sqrt(np.mean(n * n, -1)), 1.0)
    # invariant: with w = 1 the input gradient is orthogonal to x
    dx1, _ = cf.rmsnorm_bwd(dy, x, np.ones(16), 0.0)
    assert np.allclose(np.sum(dx1 * x, -1), 0.0, atol=1e-12)


def test_rope_closed_form_properties():
    r = _rng(1)
    x = r.standard_normal((2, 5, 32))
    ang = cf.rope_angles(np.arange(5), 32, 10000.0)
    y = cf.rope_fwd(x, ang)
    assert np.allclose(y[:, 0], x[:, 0])  # position 0 is the identity
    h = 16
    assert np.allclose(x[..., :h] ** 2 + x[..., h:] ** 2, y[..., :h] ** 2 + y[..., h:] ** 2)
    dy = r.standard_normal(x.shape)
    assert np.allclose(cf.rope_bwd(dy, ang), cf.finite_diff_grad(lambda t: cf.rope_fwd(t, ang), x, dy), atol=1e-7)
    assert np.allclose(cf.rope_bwd(cf.rope_fwd(x, ang), ang), x)  # orthogonal


def test_swiglu_closed_form_finite_difference():
    r = _rng(2)
    g, u, dp = (r.standard_normal((4, 8)) for _ in range(3))
    dg, du = cf.swiglu_bwd(dp, g, u)
    assert np.allclose(dg, cf.finite_diff_grad(lambda t: cf.swiglu_fwd(t, u), g, dp), atol=1e-7)
    assert np.allclose(du, cf.finite_diff_grad(lambda t: cf.swiglu_fwd(g, t), u, dp), atol=1e-7)
    assert cf.swiglu_fwd(np.zeros(3), np.ones(3)).tolist() == [0.0, 0.0, 0.0]


@pytest.mark.parametrize("nh,nkv", [(4, 2), (4, 4), (4, 1)])
def test_attention_closed_form_finite_difference(nh, nkv):
    r = _rng(3)
    B, S, d = 1, 5, 4
    q = r.standard_normal((B, nh, S, d))
    k = r.standard_normal((B, nkv, S, d))
    v = r.standard_normal((B, nkv, S, d))
    do = r.standard_normal((B, nh, S, d))
    sc = d ** -0.5
    dq, dk, dv = cf.attention_bwd(do, q, k, v, sc)
    f = lambda qq, kk, vv: cf.attention_fwd(qq, kk, vv, sc)[0]
    assert np.allclose(dq, cf.finite_diff_grad(lambda t: f(t, k, v), q, do), atol=1e-6)
    assert np.allclose(dk, cf.finite_diff_grad(lambda t: f(q, t, v), k, do), atol=1e-6)
    assert np.allclose(dv, cf.finite_diff_grad(lambda t: f(q, k, t), v, do), atol=1e-6)


def test_attention_closed_form_invariants():
    r = _rng(4)
    q = r.standard_normal((1, 2, 1, 8))
    k = r.standard_normal((1, 1, 1, 8))
    v = r.standard_normal((1, 1, 1, 8))
    o, lse = cf.attention_fwd(q, k, v, 0.3)
    assert np.allclose(o, np.repeat(v, 2, axis=1))  # S = 1: output is v
    assert np.allclose(lse[..., 0], 0.3 * np.einsum("bhd,bhd->bh", q[:, :, 0], np.repeat(k, 2, 1)[:, :, 0]))
    # causality: changing a future key/value leaves earlier rows unchanged
    q = r.standard_normal((1, 2, 6, 8)); k = r.standard_normal((1, 2, 6, 8)); v = r.standard_normal((1, 2, 6, 8))
    o1, _ = cf.attention_fwd(q, k, v, 0.5)
    k2, v2 = k.copy(), v.copy()
    k2[:, :, 5] += 3.0; v2[:, :, 5] -= 2.0
    o2, _ = cf.attention_fwd(q, k2, v2, 0.5)
    assert np.allclose(o1[:, :, :5], o2[:, :, :5]) and not np.allclose(o1[:, :, 5], o2[:, :, 5])


# ---------------------------------- oracle autograd vs closed forms (fp64)
def test_oracle_autograd_matches_closed_forms():
    r = _rng(5)
    B, nh, nkv, S, d = 2, 4, 2, 7, 8
    q = torch.tensor(r.standard_normal((B, nh, S, d)), requires_grad=True)
    k = torch.tensor(r.standard_normal((B, nkv, S, d)), requires_grad=True)
    v = torch.tensor(r.standard_normal((B, nkv, S, d)), requires_grad=True)
    do = r.standard_normal((B, nh, S, d))
    o = ot.attention(q, k, v, d ** -0.5)  # [B,S,nh*d]
    o_cf, _ = cf.attention_fwd(q.detach().numpy(), k.detach().numpy(), v.detach().numpy(), d ** -0.5)
    assert np.allclose(o.detach().numpy(), o_cf.transpose(0, 2, 1, 3).reshape(B, S, nh * d))
    o.backward(torch.tensor(do.transpose(0, 2, 1, 3).reshape(B, S, nh * d)))
    dq, dk, dv = cf.attention_bwd(do, q.detach().numpy(), k.detach().numpy(), v.detach().numpy(), d ** -0.5)
    assert np.allclose(q.grad.numpy(), dq) and np.allclose(k.grad.numpy(), dk) and np.allclose(v.grad.numpy(), dv)

    x = torch.tensor(r.standard_normal((3, 32)), requires_grad=True)
    w = torch.tensor(1 + 0.1 * r.standard_normal(32), requires_grad=True)
    dy = r.standard_normal((3, 32))
    ot.rmsnorm(x, w, 1e-5).backward(torch.tensor(dy))
    dx, dw = cf.rmsnorm_bwd(dy, x.detach().numpy(), w.detach().numpy(), 1e-5)
    assert np.allclose(x.grad.numpy(), dx) and np.allclose(w.grad.numpy(), dw)

    qq = torch.tensor(r.standard_normal((1, 1, 6, 16)), requires_grad=True)
    cos, sin = ot.rope_cos_sin(6, 16, 10000.0, torch.float64)
    qe, _ = ot.rope(qq, qq, cos, sin)
    ang = cf.rope_angles(np.arange(6), 16, 10000.0)
    assert np.allclose(qe.detach().numpy(), cf.rope_fwd(qq.detach().numpy(), ang))
    g = r.standard_normal(qe.shape)
    qe.backward(torch.tensor(g))
    assert np.allclose(qq.grad.numpy(), cf.rope_bwd(g, ang))


def test_oracle_model_matches_product_model_cpu():
    """OracleLlama and femtotron_amd.model.LlamaForTraining (HF layers, stock
    torch checkpoint through the API-identical wrapper) agree on CPU in fp32 for
    cfg 1 shapes: same seeded weights, loss and every gradient."""
    from femtotron_amd.model import build_llama_model, init_llama_weights_
    from femtotron_amd.scripts.presets import get_ac_policy
    from femtotron_amd.training import apply_activation_checkpointing

    c = CFG1
    cfg = llama_config(c)
    model = init_llama_weights_(build_llama_model(cfg), device="cpu", dtype=torch.float32)
    names = dict(model.named_parameters())  # wrapping keeps the same tensor objects
    n = apply_activation_checkpointing(model, get_ac_policy("llama_decoder_layer"),
                                       preserve_rng_state=True)
    assert n == c["layers"]
    orc = ot.OracleLlama(vocab=c["vocab"], hidden=c["hidden"], n_layers=c["layers"],
                         n_heads=c["heads"], n_kv=c["kv"], ffn=c["ffn"], theta=c["theta"])
    assert set(model.state_dict()) >= set(names)  # wrapper prefix hidden from state_dict
    for name, t in orc.named_params():
        assert torch.equal(names[name].detach(), t.detach()), name
    ids = torch.randint(0, c["vocab"], (c["batch"], c["seq"]), generator=torch.Generator().manual_seed(2000))
    loss = model(ids, labels=ids)["loss"]
    loss.backward()
    _, oloss = orc.forward(ids, ids)
    oloss.backward()
    assert abs(loss.item() - oloss.item()) <= 1e-6 * abs(oloss.item())
    for name, t in orc.named_params():
        assert_close(names[name].grad, t.grad, 1e-4, 1e-7, name)
