"""Layers whose attention is not causal without a mask never reach the kernels.

HF's eager attention (and an unset ``_attn_implementation``, which HF resolves
to eager) applies no mask when it is called without one
(transformers 5.15.0 models/llama/modeling_llama.py:202-204): every query
attends to every key.  The fused kernels are causal, so ``fused_checkpoint``
and ``fuse_attention`` must hand such calls to the stock path, whose result is
then the reference's own, bit for bit.
"""
from __future__ import annotations

import pytest
import torch
from transformers.models.llama import modeling_llama as hf

from oracle import torch_llama as ot
from tests.helpers import CFG1, layer_weights, llama_config, load_into_hf_layer, randn

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _layer(attn: str | None, dtype):
    c = CFG1
    cfg = llama_config(c, layers=1, attn=attn)
    layer = hf.LlamaDecoderLayer(cfg, layer_idx=0)
    load_into_hf_layer(layer, layer_weights(c, seed=42, norm_mean=1.0))
    return layer.to(device=DEV, dtype=dtype)


def _inputs(dtype, B=2, S=64):
    c = CFG1
    hd = c["hidden"] // c["heads"]
    cos, sin = ot.rope_cos_sin(S, hd, c["theta"], dtype, device=DEV)
    x = randn((B, S, c["hidden"]), 43).to(device=DEV, dtype=dtype)
    dy = randn((B, S, c["hidden"]), 44).to(device=DEV, dtype=dtype)
    return x, dy, cos, sin


@pytest.mark.parametrize("attn", ["eager", None])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_fused_checkpoint_falls_back_for_eager_without_mask(attn, dtype):
    from femtotron_amd import dispatch_counts, fused_checkpoint, reset_dispatch_counts
    from femtotron_amd.fused_checkpoint import last_fallback_reason
    from torch.utils.checkpoint import checkpoint

    x0, dy, cos, sin = _inputs(dtype)
    S = x0.shape[1]
    kw = dict(attention_mask=None, position_embeddings=(cos, sin),
              position_ids=torch.arange(S, device=DEV)[None], past_key_values=None, use_cache=False)
    results = []
    for fn in (fused_checkpoint, checkpoint):
        layer = _layer(attn, dtype)
        x = x0.clone().requires_grad_(True)
        reset_dispatch_counts()
        out = fn(layer, x, use_reentrant=False, preserve_rng_state=True, debug=False, **kw)
        out.backward(dy)
        if fn is fused_checkpoint:
            assert dispatch_counts() == {"fused": 0, "fallback": 1}
            assert "not causal" in last_fallback_reason()
        results.append((out.detach(), x.grad, [p.grad for p in layer.parameters()]))
    (o1, dx1, g1), (o2, dx2, g2) = results
    assert torch.equal(o1, o2) and torch.equal(dx1, dx2)
    assert all(torch.equal(a, b) for a, b in zip(g1, g2))
    # The fused layer (causal) would differ: the fallback is what keeps parity.
    assert not torch.equal(o1, _layer("sdpa", dtype)(x0, **kw))


@pytest.mark.parametrize("attn", ["eager", None])
def test_fuse_attention_falls_back_for_eager_without_mask(attn):
    from femtotron_amd import fuse_attention
    from femtotron_amd.fused_attention import (attention_dispatch_counts, last_attention_fallback_reason,
                                               reset_attention_dispatch_counts)

    dtype = torch.bfloat16
    x0, dy, cos, sin = _inputs(dtype)
    outs = []
    for fused in (True, False):
        layer = _layer(attn, dtype)
        attn_mod = layer.self_attn
        if fused:
            assert fuse_attention(layer) == 1
        x = x0.clone().requires_grad_(True)
        reset_attention_dispatch_counts()
        a, _ = attn_mod(x, position_embeddings=(cos, sin), attention_mask=None)
        a.backward(dy)
        if fused:
            assert attention_dispatch_counts() == {"fused": 0, "fallback": 1}
            assert "not causal" in last_attention_fallback_reason()
        outs.append((a.detach(), x.grad, [p.grad for p in attn_mod.parameters()]))
    (a1, dx1, g1), (a2, dx2, g2) = outs
    assert torch.equal(a1, a2) and torch.equal(dx1, dx2)
    assert all(torch.equal(p, q) for p, q in zip(g1, g2))
