"""Parity evidence at the full shapes and at the boundary's contracts (GPU).

* Element-wise accuracy of the fused bf16 layer against the exact math at the
  full layer shapes of configs 3 and 4 (and config 5's MHA widths at S = 8192):
  the exact reference is the Hugging Face layer itself run in fp32 on the same
  bf16-valued weights and inputs.  For every output and gradient tensor the
  fraction of elements outside the north star's element-wise bound
  |a - e| <= 2e-3 + 2e-2 |e| is computed for the fused path and for the
  reference's own bf16 path (HF layer under torch.utils.checkpoint); the fused
  path may not be meaningfully worse: fraction <= 1.25 x the reference's +
  1e-4, and max-error relative to the tensor's peak <= 1.25 x the reference's +
  1e-3.
* The gradient contract to the optimizer (femtotron/training/grad_accumulator.py:24-59
  with grad_acc_dtype=None; femtotron/sharding/no_shard.py:30-45): two
  micro-batches' backward passes accumulate into the existing bf16
  param.grad, with and without the packed q/k/v and gate/up weights, and
  match two stock (HF + torch checkpoint) backward passes; sibling gradients
  that are row views of one buffer stay independent.
* Dispatch with femtotron's tensor-parallel linears
  (femtotron/parallel/tensor_parallel/linear.py:42-64, 170-191; plan
  femtotron/model/parallel_plan.py:98-107): fused at world size 1, the stock
  checkpoint at world size 2 or with gather_output / scatter_input.
"""
from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F
from transformers.models.llama import modeling_llama as hf

from oracle import torch_llama as ot
from tests.helpers import (BF16_ATOL, BF16_RTOL, CFG3, CFG4, CFG5, layer_weights, llama_config,
                           load_into_hf_layer, randn)
from tests.test_layer_gpu import _run_layer, _wrapped

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _exact_layer(c, B, S, seed=42):
    """HF layer in fp32 on the GPU, on bf16-valued weights, inputs and cos/sin."""
    cfg = llama_config(c, layers=1)
    layer = hf.LlamaDecoderLayer(cfg, layer_idx=0)
    w = {k: v.bfloat16().float() for k, v in layer_weights(c, seed=seed, norm_mean=1.0).items()}
    load_into_hf_layer(layer, w)
    layer = layer.to(DEV, torch.float32)
    hd = c["hidden"] // c["heads"]
    cos, sin = (t.float() for t in ot.rope_cos_sin(S, hd, c["theta"], torch.bfloat16, device=DEV))
    x = randn((B, S, c["hidden"]), seed + 1).bfloat16().float().to(DEV).requires_grad_(True)
    dy = randn((B, S, c["hidden"]), seed + 2).bfloat16().float().to(DEV)
    out = layer(x, attention_mask=None, position_embeddings=(cos, sin),
                position_ids=torch.arange(S, device=DEV)[None], past_key_values=None, use_cache=False)
    out = out[0] if isinstance(out, tuple) else out
    out.backward(dy)
    a, m = layer.self_attn, layer.mlp
    grads = {"wq": a.q_proj.weight.grad, "wk": a.k_proj.weight.grad, "wv": a.v_proj.weight.grad,
             "wo": a.o_proj.weight.grad, "wg": m.gate_proj.weight.grad, "wu": m.up_proj.weight.grad,
             "wd": m.down_proj.weight.grad, "w1": layer.input_layernorm.weight.grad,
             "w2": layer.post_attention_layernorm.weight.grad}
    return out.detach(), x.grad, grads


def _outside(a, e):
    """Fraction of elements outside the element-wise bound, and max error / max |e|."""
    a, e = a.float(), e.float()
    err = (a - e).abs()
    frac = float((err > BF16_ATOL + BF16_RTOL * e.abs()).float().mean())
    return frac, float(err.max() / e.abs().max().clamp_min(1e-30))


@pytest.mark.parametrize("name,c,B,S", [("cfg3", CFG3, 8, 2048), ("cfg4", CFG4, 1, 8192),
                                         ("cfg5-widths", CFG5, 1, 8192)])
def test_full_shape_elementwise_accuracy_vs_exact(name, c, B, S):
    fused = _run_layer(c, B, S, torch.bfloat16, fused=True)
    torch.cuda.synchronize()
    stock = _run_layer(c, B, S, torch.bfloat16, fused=False)
    torch.cuda.synchronize()
    exact = _exact_layer(c, B, S)
    pairs = [("out", fused[0], stock[0], exact[0]), ("dx", fused[1], stock[1], exact[1])]
    pairs += [(f"d{k}", fused[2][k], stock[2][k], exact[2][k]) for k in ot.LAYER_KEYS]
    report = []
    for tag, f_, s_, e_ in pairs:
        ff, fr = _outside(f_, e_)
        sf, sr = _outside(s_, e_)
        report.append(f"{tag}: fused {ff:.2e} / {fr:.2e}, reference {sf:.2e} / {sr:.2e}")
        assert ff <= 1.25 * sf + 1e-4, f"{name} {tag}: fraction outside {ff:.3e} vs reference {sf:.3e}"
        assert fr <= 1.25 * sr + 1e-3, f"{name} {tag}: max rel err {fr:.3e} vs reference {sr:.3e}"
    print(f"\n[{name}] fraction outside rtol 2e-2/atol 2e-3 / max err rel to peak:\n  " + "\n  ".join(report))


def _run_layer_selective(c, B, S, *, fused: bool, seed=42):
    """One bf16 decoder layer under the selective policy ("llama_mlp_and_norms":
    both norms and the MLP checkpointed, attention outside the checkpoints;
    femtotron/scripts/presets.py:45-62, ckpt_policy.py:70-87).  fused: the
    checkpointed modules through fused_checkpoint and the attention through
    fuse_attention; else the reference path (torch.utils.checkpoint, stock
    HF attention)."""
    from femtotron_amd import dispatch_counts, fuse_attention, fused_checkpoint, reset_dispatch_counts
    from femtotron_amd.fused_attention import attention_dispatch_counts, reset_attention_dispatch_counts
    from femtotron_amd.scripts.presets import get_ac_policy
    from femtotron_amd.training import apply_activation_checkpointing
    from torch.utils.checkpoint import checkpoint

    layer = hf.LlamaDecoderLayer(llama_config(c, layers=1), layer_idx=0)
    load_into_hf_layer(layer, layer_weights(c, seed=seed, norm_mean=1.0))
    layer = layer.to(DEV, torch.bfloat16)
    holder = torch.nn.Module()
    holder.layer = layer
    assert apply_activation_checkpointing(holder, get_ac_policy("llama_mlp_and_norms"),
                                          checkpoint_fn=fused_checkpoint if fused else checkpoint) == 3
    if fused:
        assert fuse_attention(holder) == 1
    hd = c["hidden"] // c["heads"]
    cos, sin = ot.rope_cos_sin(S, hd, c["theta"], torch.bfloat16, device=DEV)
    x = randn((B, S, c["hidden"]), seed + 1).to(DEV, torch.bfloat16).requires_grad_(True)
    dy = randn((B, S, c["hidden"]), seed + 2).to(DEV, torch.bfloat16)
    reset_dispatch_counts()
    reset_attention_dispatch_counts()
    out = layer(x, attention_mask=None, position_embeddings=(cos, sin),
                position_ids=torch.arange(S, device=DEV)[None], past_key_values=None, use_cache=False)
    out = out[0] if isinstance(out, tuple) else out
    out.backward(dy)
    if fused:
        assert dispatch_counts() == {"fused": 3, "fallback": 0}
        assert attention_dispatch_counts() == {"fused": 1, "fallback": 0}
    a, m = layer.self_attn, layer.mlp.inner_module
    grads = {"wq": a.q_proj.weight.grad, "wk": a.k_proj.weight.grad, "wv": a.v_proj.weight.grad,
             "wo": a.o_proj.weight.grad, "wg": m.gate_proj.weight.grad, "wu": m.up_proj.weight.grad,
             "wd": m.down_proj.weight.grad, "w1": layer.input_layernorm.inner_module.weight.grad,
             "w2": layer.post_attention_layernorm.inner_module.weight.grad}
    return out.detach(), x.grad, grads


def test_full_length_selective_cfg4_elementwise_accuracy_vs_exact():
    """BASELINE config 4 at its own length (1 x 8192) under selective
    checkpointing with the fused attention: element-wise accuracy against the
    exact fp32 layer, by the same measure as the full-AC test above."""
    c, B, S = CFG4, 1, 8192
    fused = _run_layer_selective(c, B, S, fused=True)
    torch.cuda.synchronize()
    stock = _run_layer_selective(c, B, S, fused=False)
    torch.cuda.synchronize()
    exact = _exact_layer(c, B, S)
    pairs = [("out", fused[0], stock[0], exact[0]), ("dx", fused[1], stock[1], exact[1])]
    pairs += [(f"d{k}", fused[2][k], stock[2][k], exact[2][k]) for k in ot.LAYER_KEYS]
    report = []
    for tag, f_, s_, e_ in pairs:
        ff, fr = _outside(f_, e_)
        sf, sr = _outside(s_, e_)
        report.append(f"{tag}: fused {ff:.2e} / {fr:.2e}, reference {sf:.2e} / {sr:.2e}")
        assert ff <= 1.25 * sf + 1e-4, f"selective {tag}: fraction outside {ff:.3e} vs reference {sf:.3e}"
        assert fr <= 1.25 * sr + 1e-3, f"selective {tag}: max rel err {fr:.3e} vs reference {sr:.3e}"
    print("\n[cfg4 selective] fraction outside rtol 2e-2/atol 2e-3 / max err rel to peak:\n  "
          + "\n  ".join(report))


def _stack(c, n, seed, packed):
    from femtotron_amd import pack_layer_weights
    cfg = llama_config(c, layers=n)
    layers = torch.nn.ModuleList([hf.LlamaDecoderLayer(cfg, i) for i in range(n)])
    for i, l in enumerate(layers):
        load_into_hf_layer(l, layer_weights(c, seed=seed + i, norm_mean=1.0))
    layers = layers.to(DEV, torch.bfloat16)
    if packed:
        holder = torch.nn.Module()
        holder.layers = layers
        assert pack_layer_weights(holder) == 2 * n
    return layers


def _two_micro_batches(layers, c, S, fused):
    hd = c["hidden"] // c["heads"]
    cos, sin = ot.rope_cos_sin(S, hd, c["theta"], torch.bfloat16, device=DEV)
    ws = [_wrapped(l, fused) for l in layers]
    for p in layers.parameters():
        p.grad = None
    for mb in range(2):
        h = randn((2, S, c["hidden"]), 300 + mb).to(DEV, torch.bfloat16).requires_grad_(True)
        for w in ws:
            h = w(h, attention_mask=None, position_embeddings=(cos, sin), past_key_values=None,
                  use_cache=False)
        h.backward(randn((2, S, c["hidden"]), 400 + mb).to(DEV, torch.bfloat16))
    return [p.grad for p in layers.parameters()]


@pytest.mark.parametrize("packed", [False, True], ids=["unpacked", "packed"])
def test_grad_accumulates_over_two_micro_batches(packed):
    from femtotron_amd import dispatch_counts, reset_dispatch_counts
    c = CFG3
    fused_layers = _stack(c, 2, 500, packed)
    stock_layers = _stack(c, 2, 500, False)
    reset_dispatch_counts()
    g_fused = _two_micro_batches(fused_layers, c, 256, fused=True)
    assert dispatch_counts() == {"fused": 4, "fallback": 0}
    g_stock = _two_micro_batches(stock_layers, c, 256, fused=False)
    for i, (a, b) in enumerate(zip(g_fused, g_stock)):
        assert a.dtype == torch.bfloat16 and a.shape == b.shape
        err = float((a.float() - b.float()).abs().max())
        assert err <= BF16_ATOL + BF16_RTOL * float(b.float().abs().max()), f"param {i}: {err:.3e}"
    # sibling gradients (row views of one dq/dk/dv or dgate/dup buffer) are independent
    attn = fused_layers[0].self_attn
    gk, gv = attn.k_proj.weight.grad.clone(), attn.v_proj.weight.grad.clone()
    attn.q_proj.weight.grad.zero_()
    assert torch.equal(attn.k_proj.weight.grad, gk) and torch.equal(attn.v_proj.weight.grad, gv)
    mlp = fused_layers[0].mlp
    gu = mlp.up_proj.weight.grad.clone()
    mlp.gate_proj.weight.grad.zero_()
    assert torch.equal(mlp.up_proj.weight.grad, gu)


def test_accumulated_grad_is_the_sum_of_the_micro_batches():
    """Exactness of the accumulation itself: the fused path's accumulated bf16
    .grad equals the bf16 sum of its own two single-micro-batch gradients."""
    c = CFG3
    hd = c["hidden"] // c["heads"]
    S = 256
    cos, sin = ot.rope_cos_sin(S, hd, c["theta"], torch.bfloat16, device=DEV)
    layers = _stack(c, 1, 700, packed=True)
    w = _wrapped(layers[0], True)
    xs = [randn((2, S, c["hidden"]), 800 + i).to(DEV, torch.bfloat16) for i in range(2)]
    dys = [randn((2, S, c["hidden"]), 900 + i).to(DEV, torch.bfloat16) for i in range(2)]
    per = []
    for i in range(2):
        for p in layers.parameters():
            p.grad = None
        w(xs[i].requires_grad_(True), attention_mask=None, position_embeddings=(cos, sin)).backward(dys[i])
        per.append([p.grad.clone() for p in layers.parameters()])
    for p in layers.parameters():
        p.grad = None
    for i in range(2):
        w(xs[i].detach().requires_grad_(True), attention_mask=None,
          position_embeddings=(cos, sin)).backward(dys[i])
    for p, a, b in zip(layers.parameters(), per[0], per[1]):
        assert torch.equal(p.grad, a + b)


class _ColumnLike(torch.nn.Module):
    """Attributes of femtotron's ColumnParallelLinear (tensor_parallel/linear.py:42-64)."""

    def __init__(self, lin: torch.nn.Linear, world_size=1, gather_output=False):
        super().__init__()
        self.weight = lin.weight
        self.bias = None
        self.world_size, self.rank, self.gather_output = world_size, 0, gather_output

    def forward(self, x):
        return F.linear(x, self.weight)


class _RowLike(torch.nn.Module):
    """Attributes of femtotron's RowParallelLinear (tensor_parallel/linear.py:170-191)."""

    def __init__(self, lin: torch.nn.Linear, world_size=1, scatter_input=False):
        super().__init__()
        self.weight = lin.weight
        self.bias = None
        self.world_size, self.rank, self.scatter_input = world_size, 0, scatter_input

    def forward(self, x):
        return F.linear(x, self.weight)


def _tp_layer(world_size=1, gather=False, scatter=False):
    c = dict(CFG3)
    layer = hf.LlamaDecoderLayer(llama_config(c, layers=1), 0)
    load_into_hf_layer(layer, layer_weights(c, seed=42, norm_mean=1.0))
    layer = layer.to(DEV, torch.bfloat16)
    a, m = layer.self_attn, layer.mlp
    for name in ("q_proj", "k_proj", "v_proj"):
        setattr(a, name, _ColumnLike(getattr(a, name), world_size, gather))
    a.o_proj = _RowLike(a.o_proj, world_size, scatter)
    for name in ("gate_proj", "up_proj"):
        setattr(m, name, _ColumnLike(getattr(m, name), world_size, gather))
    m.down_proj = _RowLike(m.down_proj, world_size, scatter)
    return layer


def test_dispatch_with_tensor_parallel_linears():
    from femtotron_amd import dispatch_counts, fused_checkpoint, last_fallback_reason, reset_dispatch_counts
    S = 128
    cos, sin = ot.rope_cos_sin(S, 64, CFG3["theta"], torch.bfloat16, device=DEV)
    x = randn((1, S, 2048), 5).to(DEV, torch.bfloat16)
    plain = hf.LlamaDecoderLayer(llama_config(CFG3, layers=1), 0)
    load_into_hf_layer(plain, layer_weights(CFG3, seed=42, norm_mean=1.0))
    plain = plain.to(DEV, torch.bfloat16)
    reset_dispatch_counts()
    want = fused_checkpoint(plain, x, use_reentrant=False, debug=True, position_embeddings=(cos, sin))
    got = fused_checkpoint(_tp_layer(1), x, use_reentrant=False, debug=True, position_embeddings=(cos, sin))
    assert dispatch_counts() == {"fused": 2, "fallback": 0}
    assert torch.equal(got, want)
    for kw in (dict(world_size=2), dict(gather=True), dict(scatter=True)):
        reset_dispatch_counts()
        fused_checkpoint(_tp_layer(**kw), x, use_reentrant=False, debug=True, position_embeddings=(cos, sin))
        assert dispatch_counts() == {"fused": 0, "fallback": 1}, kw
        assert "tensor-parallel" in last_fallback_reason(), (kw, last_fallback_reason())


@pytest.mark.parametrize("hd", [16, 48, 96])
def test_unsupported_head_dim_falls_back_to_stock_checkpoint(hd):
    from femtotron_amd import dispatch_counts, fused_checkpoint, last_fallback_reason, reset_dispatch_counts
    from torch.utils.checkpoint import checkpoint
    heads = 4
    c = dict(hidden=hd * heads, heads=heads, kv=2, ffn=256, vocab=128, layers=1, theta=1e4, batch=1, seq=32)
    layer = hf.LlamaDecoderLayer(llama_config(c, layers=1), 0)
    load_into_hf_layer(layer, layer_weights(c, seed=3, norm_mean=1.0))
    layer = layer.to(DEV, torch.bfloat16)
    S = 32
    cos, sin = ot.rope_cos_sin(S, hd, 1e4, torch.bfloat16, device=DEV)
    x = randn((1, S, c["hidden"]), 6).to(DEV, torch.bfloat16)
    reset_dispatch_counts()
    got = fused_checkpoint(layer, x, use_reentrant=False, debug=True, position_embeddings=(cos, sin))
    assert dispatch_counts() == {"fused": 0, "fallback": 1}
    assert "head_dim" in last_fallback_reason()
    want = checkpoint(layer, x, use_reentrant=False, position_embeddings=(cos, sin))
    want = want[0] if isinstance(want, tuple) else want
    assert torch.equal(got, want)


@pytest.mark.parametrize("packed", [False, True], ids=["unpacked", "packed"])
def test_gradient_accumulation_in_the_gemm_equals_autograds(packed):
    """With .grad already present (the reference's GradAccumulator keeps it
    between steps and accumulates micro-batches into it,
    femtotron/training/grad_accumulator.py:24-60), the weight-gradient GEMMs
    add into it in their epilogue.  The result must be autograd's own
    accumulation of the same gradients bit for bit: to_bf16(grad + to_bf16(dW)).
    A .grad that is not laid out as the GEMM's output (here: a fresh
    non-contiguous tensor) takes autograd's path."""
    from femtotron_amd import dispatch_counts, reset_dispatch_counts
    from femtotron_amd.fused_layer import grad_accumulation_in_gemm, set_grad_accumulation_in_gemm
    from femtotron_amd.projections import gemm_dispatch_counts, reset_gemm_dispatch_counts
    c = CFG3
    assert grad_accumulation_in_gemm()
    results = []
    try:
        for in_gemm in (False, True):
            set_grad_accumulation_in_gemm(in_gemm)
            layers = _stack(c, 2, 600, packed)
            reset_dispatch_counts()
            reset_gemm_dispatch_counts()
            results.append(_two_micro_batches(layers, c, 256, fused=True))
            assert dispatch_counts() == {"fused": 4, "fallback": 0}
    finally:
        set_grad_accumulation_in_gemm(True)
    for i, (a, b) in enumerate(zip(*results)):
        assert torch.equal(a, b), f"param {i}"
    # a gradient the GEMM cannot write (transposed storage) is left to autograd
    layers = _stack(c, 1, 700, packed)
    wo = layers[0].self_attn.o_proj.weight
    wo.grad = torch.zeros(wo.shape[1], wo.shape[0], device=DEV, dtype=torch.bfloat16).t()
    assert not wo.grad.is_contiguous()
    hd = c["hidden"] // c["heads"]
    cos, sin = ot.rope_cos_sin(128, hd, c["theta"], torch.bfloat16, device=DEV)
    x = randn((1, 128, c["hidden"]), 5).to(DEV, torch.bfloat16).requires_grad_(True)
    _wrapped(layers[0], True)(x, attention_mask=None, position_embeddings=(cos, sin)).backward(
        randn((1, 128, c["hidden"]), 6).to(DEV, torch.bfloat16))
    ref = _stack(c, 1, 700, packed)
    _wrapped(ref[0], True)(x.detach().requires_grad_(True), attention_mask=None,
                           position_embeddings=(cos, sin)).backward(
        randn((1, 128, c["hidden"]), 6).to(DEV, torch.bfloat16))
    assert torch.equal(wo.grad, ref[0].self_attn.o_proj.weight.grad)
