"""Parity of the fused checkpointed decoder layer (GPU) with the reference path.

Checkers:
  * oracle/torch_llama.py on the CPU (bf16 op-by-op like the reference; fp32
    for the 1e-5 config) on identical seeded weights/inputs;
  * the reference path itself on the GPU: Hugging Face LlamaDecoderLayer under
    torch.utils.checkpoint through the API-identical wrapper (debug=True), at
    the full TinyLlama layer shape where the CPU oracle would be too slow.
Tolerances are the north star's: rtol 2e-2 / atol 2e-3 in bf16, 1e-5 in fp32.
"""
from __future__ import annotations

import pytest
import torch
from transformers.models.llama import modeling_llama as hf

from oracle import torch_llama as ot
from tests.helpers import (BF16_ATOL, BF16_RTOL, CFG1, CFG3, CFG4, CFG5, assert_close, hf_layer_grads,
                           layer_weights, llama_config, load_into_hf_layer, randn, rel_err)

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _wrapped(layer, fused: bool):
    from femtotron_amd import fused_checkpoint
    from femtotron_amd.training import ActivationCheckpointWrapper
    from torch.utils.checkpoint import checkpoint
    return ActivationCheckpointWrapper(layer, checkpoint_fn=fused_checkpoint if fused else checkpoint,
                                       preserve_rng_state=True)


def _run_layer(c, B, S, dtype, *, fused: bool, norm_mean=1.0, seed=42, device=DEV):
    cfg = llama_config(c, layers=1)
    layer = hf.LlamaDecoderLayer(cfg, layer_idx=0)
    load_into_hf_layer(layer, layer_weights(c, seed=seed, norm_mean=norm_mean))
    layer = layer.to(device=device, dtype=dtype)
    hd = c["hidden"] // c["heads"]
    cos, sin = ot.rope_cos_sin(S, hd, c["theta"], dtype, device=device)
    x = randn((B, S, c["hidden"]), seed + 1).to(device=device, dtype=dtype).requires_grad_(True)
    dy = randn((B, S, c["hidden"]), seed + 2).to(device=device, dtype=dtype)
    w = _wrapped(layer, fused)
    out = w(x, attention_mask=None, position_embeddings=(cos, sin),
            position_ids=torch.arange(S, device=device)[None], past_key_values=None, use_cache=False)
    out.backward(dy)
    return out.detach(), x.grad, hf_layer_grads(layer)


def _oracle_layer(c, B, S, dtype, *, norm_mean=1.0, seed=42):
    w = {k: v.to(dtype).requires_grad_(True) for k, v in
         layer_weights(c, seed=seed, norm_mean=norm_mean).items()}
    hd = c["hidden"] // c["heads"]
    cos, sin = ot.rope_cos_sin(S, hd, c["theta"], dtype)
    x = randn((B, S, c["hidden"]), seed + 1).to(dtype).requires_grad_(True)
    dy = randn((B, S, c["hidden"]), seed + 2).to(dtype)
    out = ot.decoder_layer(x, cos, sin, w, c["heads"], c["kv"], hd, 1e-5)
    out.backward(dy)
    return out.detach(), x.grad, {k: v.grad for k, v in w.items()}


def _compare(got, ref, rtol, atol, tag):
    """Per tensor max|a-b| <= atol + rtol*max|b|, the form of the reference's
    compare_grads (femtotron/test/unit/test_pipeline_stage.py:82-128, whose rtol
    1.5e-3 is for paths running identical arithmetic), with the north star's
    rtol 2e-2 / atol 2e-3 for two independent bf16 implementations.  An element-wise bound cannot be
    the bar in bf16: the reference's own bf16 path differs from the exact math of
    the same layer by several times its magnitude on entries near zero (outputs
    and input grads are sums such as x + attn(x) that cancel, weight grads are
    sums over all tokens).  test_fused_layer_at_least_as_accurate_as_reference_bf16
    and the fp32 tests carry the tighter checks."""
    out, dx, gw = got
    rout, rdx, rgw = ref
    pairs = [("out", out, rout), ("dx", dx, rdx)] + [(f"d{k}", gw[k], rgw[k]) for k in ot.LAYER_KEYS]
    for name, a, b in pairs:
        a, b = a.float().cpu(), b.float().cpu()
        assert a.shape == b.shape and bool(torch.isfinite(a).all()), f"{tag} {name}: shape/finite"
        err = float((a - b).abs().max())
        lim = atol + rtol * float(b.abs().max())
        assert err <= lim, f"{tag} {name}: max|a-b|={err:.3e} > {lim:.3e}"


@pytest.mark.parametrize("name,c,B,S", [
    ("cfg1", CFG1, 2, 128),
    ("cfg1-mha", dict(CFG1, kv=8), 1, 64),
    ("tinyllama-256tok", CFG3, 1, 256),
    ("llama3-128tok", CFG4, 1, 128),
])
def test_fused_layer_matches_oracle_bf16(name, c, B, S):
    from femtotron_amd import dispatch_counts, reset_dispatch_counts
    reset_dispatch_counts()
    got = _run_layer(c, B, S, torch.bfloat16, fused=True)
    assert dispatch_counts()["fused"] == 1, "the fused HIP path was not taken"
    ref = _oracle_layer(c, B, S, torch.bfloat16)
    _compare(got, ref, BF16_RTOL, BF16_ATOL, name)


@pytest.mark.parametrize("name,c,B,S", [("cfg1", CFG1, 2, 128), ("tinyllama-256tok", CFG3, 1, 256)])
def test_fused_layer_at_least_as_accurate_as_reference_bf16(name, c, B, S):
    """Against the exact math (fp32 oracle on the same bf16-valued inputs), the
    fused bf16 path is no less accurate than the reference's own bf16 path."""
    got = _run_layer(c, B, S, torch.bfloat16, fused=True)
    ref = _oracle_layer(c, B, S, torch.bfloat16)
    w32 = {k: v.bfloat16().float().requires_grad_(True)
           for k, v in layer_weights(c, seed=42, norm_mean=1.0).items()}
    hd = c["hidden"] // c["heads"]
    cos, sin = (t.float() for t in ot.rope_cos_sin(S, hd, c["theta"], torch.bfloat16))
    x = randn((B, S, c["hidden"]), 43).bfloat16().float().requires_grad_(True)
    dy = randn((B, S, c["hidden"]), 44).bfloat16().float()
    out = ot.decoder_layer(x, cos, sin, w32, c["heads"], c["kv"], hd, 1e-5)
    out.backward(dy)
    exact = (out.detach(), x.grad, {k: v.grad for k, v in w32.items()})
    pairs = [("out", got[0], ref[0], exact[0]), ("dx", got[1], ref[1], exact[1])]
    pairs += [(f"d{k}", got[2][k], ref[2][k], exact[2][k]) for k in ot.LAYER_KEYS]
    for tag, g, r, e in pairs:
        eg, er = rel_err(g, e), rel_err(r, e)
        assert eg <= 1.25 * er + 1e-3, f"{name} {tag}: fused err {eg:.2e} vs reference bf16 err {er:.2e}"


@pytest.mark.parametrize("policy", ["hand", "library"])
@pytest.mark.parametrize("name,c,B,S", [("tinyllama-2048tok", CFG3, 1, 2048), ("llama3-512tok", CFG4, 1, 512)])
def test_fused_layer_under_each_gemm_policy_matches_stock_checkpoint(policy, name, c, B, S):
    """Every projection GEMM on the hand-written kernel (NT forward and
    recompute, the down projection's residual epilogue, NN, TN and the grouped
    weight gradients), or every one on the library: the layer still matches
    the HF layer under torch.utils.checkpoint, and the routing counters show
    that the policy held."""
    from femtotron_amd import projections
    projections.reset_gemm_dispatch_counts()
    before = projections.gemm_policy()
    projections.set_gemm_policy(policy)
    try:
        got = _run_layer(c, B, S, torch.bfloat16, fused=True)
        counts = projections.gemm_dispatch_counts()
    finally:
        projections.set_gemm_policy(before)
    torch.cuda.synchronize()
    ref = _run_layer(c, B, S, torch.bfloat16, fused=False)
    _compare(got, ref, BF16_RTOL, BF16_ATOL, f"{name}-{policy}")
    # forward 4 (q/k/v, o, gate/up, down) + recompute 3 + backward 4 NN and 4 TN
    assert counts == ({"hand": 15, "library": 0} if policy == "hand" else {"hand": 0, "library": 15}), counts


def test_weight_gradients_on_side_stream_match_serial_bitwise():
    """The weight-gradient GEMMs give the same bits whether they run in series
    with the input-gradient chain (the default) or on a side stream: every
    kernel is deterministic and the side stream only changes the order."""
    from femtotron_amd.fused_layer import set_wgrad_side_stream, wgrad_side_stream
    assert not wgrad_side_stream()
    serial = _run_layer(CFG3, 1, 256, torch.bfloat16, fused=True)
    set_wgrad_side_stream(True)
    try:
        side = _run_layer(CFG3, 1, 256, torch.bfloat16, fused=True)
    finally:
        set_wgrad_side_stream(False)
    assert torch.equal(serial[0], side[0]) and torch.equal(serial[1], side[1])
    for k in serial[2]:
        assert torch.equal(serial[2][k], side[2][k]), k


def test_fused_layer_reference_init_bf16():
    """All parameters N(0, 0.02) (norm weights too), the reference's own init."""
    got = _run_layer(CFG1, 2, 128, torch.bfloat16, fused=True, norm_mean=0.0)
    ref = _oracle_layer(CFG1, 2, 128, torch.bfloat16, norm_mean=0.0)
    _compare(got, ref, BF16_RTOL, BF16_ATOL, "ref-init")


def test_fused_layer_fp32_matches_oracle_1e5():
    got = _run_layer(CFG1, 2, 128, torch.float32, fused=True)
    ref = _oracle_layer(CFG1, 2, 128, torch.float32)
    out, dx, gw = got
    assert_close(out, ref[0], 1e-5, 1e-5, "out")
    assert_close(dx, ref[1], 1e-5, 1e-5, "dx")
    for k in ot.LAYER_KEYS:
        assert rel_err(gw[k], ref[2][k]) < 1e-5, f"d{k} rel {rel_err(gw[k], ref[2][k]):.3e}"


@pytest.mark.parametrize("name,c", [("tinyllama", CFG3), ("llama3-8b", CFG4), ("llama2-7b-long", CFG5)])
def test_fused_layer_matches_stock_checkpoint_full_shape(name, c):
    """One layer at each GPU config's full shape: TinyLlama (B=8, S=2048, GQA 32/4,
    hd 64), Llama-3-8B (S=8192, GQA 32/8, hd 128, F=14336), Llama-2-7B long
    context (S=32768, MHA 32/32, hd 128): fused vs HF layer + torch checkpoint
    on the GPU, tensor-level metric."""
    got = _run_layer(c, c["batch"], c["seq"], torch.bfloat16, fused=True)
    torch.cuda.synchronize()
    ref = _run_layer(c, c["batch"], c["seq"], torch.bfloat16, fused=False)
    _compare(got, ref, BF16_RTOL, BF16_ATOL, f"{name}-full")


def test_cfg1_model_step_gpu_fp32_vs_cpu_oracle():
    """BASELINE config 1 end to end (embed, 2 fused layers, norm, lm_head, CE):
    loss and every gradient vs the CPU fp32 oracle within 1e-5."""
    from femtotron_amd import dispatch_counts, fused_checkpoint, reset_dispatch_counts
    from femtotron_amd.model import build_llama_model, init_llama_weights_
    from femtotron_amd.scripts.presets import get_ac_policy
    from femtotron_amd.training import apply_activation_checkpointing

    c = CFG1
    model = init_llama_weights_(build_llama_model(llama_config(c)), device=DEV, dtype=torch.float32)
    names = dict(model.named_parameters())
    assert apply_activation_checkpointing(model, get_ac_policy("llama_decoder_layer"),
                                          checkpoint_fn=fused_checkpoint) == 2
    ids = torch.randint(0, c["vocab"], (c["batch"], c["seq"]), generator=torch.Generator().manual_seed(2000))
    reset_dispatch_counts()
    loss = model(ids.to(DEV), labels=ids.to(DEV))["loss"]
    loss.backward()
    assert dispatch_counts() == {"fused": 2, "fallback": 0}
    orc = ot.OracleLlama(vocab=c["vocab"], hidden=c["hidden"], n_layers=c["layers"], n_heads=c["heads"],
                         n_kv=c["kv"], ffn=c["ffn"], theta=c["theta"])
    _, oloss = orc.forward(ids, ids)
    oloss.backward()
    assert abs(loss.item() - oloss.item()) <= 1e-5 * abs(oloss.item())
    for n, t in orc.named_params():
        assert rel_err(names[n].grad, t.grad) < 1e-5, f"{n}: rel {rel_err(names[n].grad, t.grad):.3e}"


def test_fallback_is_the_stock_path_and_counts():
    """Calls the fused path cannot take (explicit mask) go to torch checkpoint."""
    from femtotron_amd import dispatch_counts, fused_checkpoint, last_fallback_reason, reset_dispatch_counts
    c = CFG1
    layer = hf.LlamaDecoderLayer(llama_config(c, layers=1), 0).to(DEV, torch.bfloat16)
    S = 16
    cos, sin = ot.rope_cos_sin(S, 32, 1e4, torch.bfloat16, device=DEV)
    x = torch.randn(1, S, 256, device=DEV, dtype=torch.bfloat16)
    mask = torch.zeros(1, 1, S, S, device=DEV, dtype=torch.bfloat16)
    reset_dispatch_counts()
    fused_checkpoint(layer, x, use_reentrant=False, debug=True, attention_mask=mask,
                     position_embeddings=(cos, sin))
    assert dispatch_counts() == {"fused": 0, "fallback": 1}
    assert "mask" in last_fallback_reason()
    with pytest.raises(ValueError):
        fused_checkpoint(layer, x, use_reentrant=True, debug=True, position_embeddings=(cos, sin))


def test_peak_memory_not_above_stock_checkpoint():
    """Peak activation memory of fwd+bwd over a 4-layer TinyLlama-shaped stack
    (B=2, S=2048): fused path <= reference path (HF + torch checkpoint)."""
    c = CFG3
    cfg = llama_config(c, layers=4)
    layers = [hf.LlamaDecoderLayer(cfg, i) for i in range(4)]
    for i, l in enumerate(layers):
        load_into_hf_layer(l, layer_weights(c, seed=100 + i))
    layers = [l.to(DEV, torch.bfloat16) for l in layers]
    B, S = 2, 2048
    cos, sin = ot.rope_cos_sin(S, 64, c["theta"], torch.bfloat16, device=DEV)
    x0 = randn((B, S, c["hidden"]), 1).to(DEV, torch.bfloat16)

    def peak(fused):
        ws = [_wrapped(l, fused) for l in layers]
        for l in layers:
            for p in l.parameters():
                p.grad = None
        # warm-up pass so grads exist (the reference's measuring method)
        for _ in range(2):
            torch.cuda.synchronize()
            torch.cuda.reset_peak_memory_stats()
            base = torch.cuda.memory_allocated()
            h = x0.clone().requires_grad_(True)
            for w in ws:
                h = w(h, attention_mask=None, position_embeddings=(cos, sin), past_key_values=None,
                      use_cache=False)
            h.float().sum().backward()
            torch.cuda.synchronize()
        return torch.cuda.max_memory_allocated() - base

    p_fused = peak(True)
    p_ref = peak(False)
    assert p_fused <= p_ref, f"fused peak {p_fused / 2**20:.1f} MiB > reference {p_ref / 2**20:.1f} MiB"


def test_fused_checkpointing_saves_memory_and_matches_no_checkpointing():
    """The reference's own invariants for activation checkpointing
    (femtotron tests/test_zero_ac.py:265-280) on a 4-layer TinyLlama-shaped
    stack (B=2, S=2048): the fused checkpointed stack's peak memory is below
    the same layers run without checkpointing, and its output sum differs from
    theirs by less than 1e-2 relative (the layers' gradients agree within the
    tensor-level bf16 metric)."""
    c = CFG3
    cfg = llama_config(c, layers=4)
    layers = [hf.LlamaDecoderLayer(cfg, i) for i in range(4)]
    for i, l in enumerate(layers):
        load_into_hf_layer(l, layer_weights(c, seed=200 + i))
    layers = [l.to(DEV, torch.bfloat16) for l in layers]
    B, S = 2, 2048
    cos, sin = ot.rope_cos_sin(S, 64, c["theta"], torch.bfloat16, device=DEV)
    x0 = randn((B, S, c["hidden"]), 2).to(DEV, torch.bfloat16)

    def run(fused):
        mods = [_wrapped(l, True) for l in layers] if fused else layers
        for _ in range(2):  # the second pass measures, with grads already allocated
            for l in layers:
                for p in l.parameters():
                    p.grad = None
            torch.cuda.synchronize()
            torch.cuda.reset_peak_memory_stats()
            base = torch.cuda.memory_allocated()
            h = x0.clone().requires_grad_(True)
            for m in mods:
                out = m(h, attention_mask=None, position_embeddings=(cos, sin), past_key_values=None,
                        use_cache=False)
                h = out[0] if isinstance(out, tuple) else out
            total = h.float().sum()
            total.backward()
            torch.cuda.synchronize()
        peak = torch.cuda.max_memory_allocated() - base
        grads = [p.grad.detach().float().clone() for l in layers for p in l.parameters()]
        return peak, float(total.detach()), grads

    p_ac, s_ac, g_ac = run(True)
    p_no, s_no, g_no = run(False)
    assert p_ac < p_no, f"checkpointed peak {p_ac / 2**20:.1f} MiB >= plain {p_no / 2**20:.1f} MiB"
    assert abs(s_ac - s_no) <= 1e-2 * abs(s_no)
    for a, b in zip(g_ac, g_no):
        err = float((a - b).abs().max())
        assert err <= BF16_ATOL + BF16_RTOL * float(b.abs().max()), err
