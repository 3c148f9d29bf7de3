"""Embedding forward/backward and final RMSNorm kernels on the GPU
(femtotron_amd/boundary_ops.py, fh_embedding_fwd / fh_embedding_bwd).

Checkers: oracle/embedding.py (pinned against torch's F.embedding in
tests/test_boundary.py) — the forward bit-exact, the weight gradient bit-exact
against the fp32 sums in ascending token order (the kernel's documented order;
rounded once to bf16 for bf16), which also proves the radix sort stable and the
result run-independent; torch's own F.embedding backward on the GPU (the
reference's op) within one bf16 ulp at the TinyLlama shape; the CPU fp32 oracle
model end to end (config 1, 1e-5); the stock modules at a TinyLlama-shaped
2-layer bf16 model (the north star's tensor-level bf16 metric).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import embedding as oe
from tests.helpers import BF16_ATOL, BF16_RTOL, CFG1, CFG3, llama_config, rel_err

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _ids(T, V, seed, bad=0, hot=None):
    g = np.random.default_rng(seed)
    ids = g.integers(0, V, size=T).astype(np.int64)
    if hot is not None:  # a long run of one id spread over the whole batch
        ids[g.random(T) < 0.3] = hot
    if bad:
        pos = g.choice(T, size=bad, replace=False)
        ids[pos[: bad // 2]] = -1 - g.integers(0, 5, size=bad // 2)
        ids[pos[bad // 2:]] = V + g.integers(0, 5, size=bad - bad // 2)
    return ids


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("T,V,H", [(1, 10, 8), (1000, 300, 520), (4097, 32000, 2048)])
def test_embedding_fwd_exact(dtype, T, V, H):
    from femtotron_amd import ops
    w = torch.randn(V, H, generator=torch.Generator().manual_seed(T)).to(dtype)
    ids = _ids(T, V, T, bad=min(T // 2, 10))
    out = ops.embedding_fwd(torch.from_numpy(ids).to(DEV), w.to(DEV)).cpu()
    want = torch.from_numpy(oe.embedding_fwd(ids, w.float().numpy())).to(dtype)
    assert torch.equal(out, want)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("T,V,H,pad,bad,hot", [
    (0, 100, 64, None, 0, None),        # no tokens: all-zero gradient
    (1, 100, 64, None, 0, None),
    (1000, 50, 64, None, 0, None),      # ~20 tokens per id
    (5000, 7, 16, 3, 0, None),          # 7 ids, very long rows, padding_idx
    (4097, 32000, 136, None, 40, 17),   # ragged last tile, masked ids, one hot id
    (3000, 128256, 64, 0, 0, None),     # 17-bit keys: three radix passes
    (70000, 1000, 8, None, 0, 5),       # 69 tiles, a 21k-token row
])
def test_embedding_bwd_ordered_exact(dtype, T, V, H, pad, bad, hot):
    from femtotron_amd import ops
    ids = _ids(T, V, T + V, bad=bad, hot=hot)
    dy = torch.randn(T, H, generator=torch.Generator().manual_seed(V)).to(dtype)
    got = ops.embedding_bwd(dy.to(DEV), torch.from_numpy(ids).to(DEV), V, pad).cpu()
    want32 = torch.from_numpy(oe.embedding_bwd_ordered(dy.float().numpy(), ids, V, pad))
    assert torch.equal(got, want32.to(dtype))


def test_embedding_bwd_tinyllama_vs_torch_and_deterministic():
    """TinyLlama step shape (16384 tokens, V = 32000, H = 2048, bf16): within one
    bf16 ulp of torch's F.embedding backward on the GPU and of the fp64 sums;
    two runs bitwise equal."""
    from femtotron_amd import ops
    T, V, H = 16384, 32000, 2048
    ids = torch.from_numpy(_ids(T, V, 11)).to(DEV)
    dy = torch.randn(T, H, device=DEV, generator=torch.Generator(device=DEV).manual_seed(1)).bfloat16()
    a = ops.embedding_bwd(dy, ids, V)
    b = ops.embedding_bwd(dy, ids, V)
    assert torch.equal(a, b)
    w = torch.zeros(V, H, device=DEV, dtype=torch.bfloat16, requires_grad=True)
    F.embedding(ids, w).backward(dy)
    exact = torch.zeros(V, H, device=DEV, dtype=torch.float64).index_add_(0, ids, dy.double())
    for ref in (w.grad.float(), exact):
        ulp = (ref.abs() * 2.0 ** -7).clamp(min=2.0 ** -126)
        assert bool(((a.float() - ref).abs() <= ulp).all())


def test_final_norm_matches_llama_rmsnorm():
    """FusedRMSNorm vs the Hugging Face LlamaRMSNorm it replaces, bf16 [2, 512, 2048]:
    output and both gradients within the tensor-level bf16 metric."""
    from transformers.models.llama.modeling_llama import LlamaRMSNorm

    from femtotron_amd.boundary_ops import FusedRMSNorm
    ref = LlamaRMSNorm(2048, eps=1e-5).to(DEV, torch.bfloat16)
    with torch.no_grad():
        ref.weight.copy_(1 + 0.02 * torch.randn(2048, device=DEV))
    fused = FusedRMSNorm.from_module(ref)
    g = torch.Generator(device=DEV).manual_seed(5)
    x = torch.randn(2, 512, 2048, device=DEV, generator=g).bfloat16()
    dy = torch.randn(2, 512, 2048, device=DEV, generator=g).bfloat16()
    res = []
    for m in (fused, ref):
        xi = x.clone().requires_grad_(True)
        m.weight.grad = None
        y = m(xi)
        y.backward(dy)
        res.append((y.detach().float(), xi.grad.float(), m.weight.grad.float()))
    for a, b in zip(*res):
        assert float((a - b).abs().max()) <= BF16_ATOL + BF16_RTOL * float(b.abs().max())


def _model(c, layers, dtype, seed=42):
    from femtotron_amd.model import build_llama_model, init_llama_weights_
    return init_llama_weights_(build_llama_model(llama_config(c, layers=layers)), device=DEV,
                               dtype=dtype, seed=seed)


def test_boundary_cfg1_fp32_vs_cpu_oracle():
    """Config 1 end to end on the fused path (embedding, layers, final norm, loss
    head): loss and all 21 gradients within 1e-5 of the CPU fp32 oracle."""
    from femtotron_amd import dispatch_counts, fuse_boundary_ops, fused_checkpoint, reset_dispatch_counts
    from femtotron_amd.boundary_ops import FusedEmbedding, FusedRMSNorm
    from femtotron_amd.scripts.presets import get_ac_policy
    from femtotron_amd.training import apply_activation_checkpointing
    from oracle import torch_llama as ot
    c = CFG1
    model = _model(c, c["layers"], torch.float32)
    assert fuse_boundary_ops(model) == 2
    assert isinstance(model.model.embed_tokens, FusedEmbedding) and isinstance(model.model.norm, FusedRMSNorm)
    apply_activation_checkpointing(model, get_ac_policy("llama_decoder_layer"), checkpoint_fn=fused_checkpoint)
    ids = torch.randint(0, c["vocab"], (c["batch"], c["seq"]), generator=torch.Generator().manual_seed(2000))
    reset_dispatch_counts()
    out = model(ids.to(DEV), labels=ids.to(DEV), materialize_logits=False)
    out["loss"].backward()
    assert dispatch_counts()["fallback"] == 0
    grads = {n.replace("._checkpoint_wrapped_module", ""): p.grad for n, p in model.named_parameters()}
    orc = ot.OracleLlama(vocab=c["vocab"], hidden=c["hidden"], n_layers=c["layers"], n_heads=c["heads"],
                         n_kv=c["kv"], ffn=c["ffn"], theta=c["theta"])
    _, oloss = orc.forward(ids, ids)
    oloss.backward()
    assert abs(out["loss"].item() - oloss.item()) <= 1e-5 * abs(oloss.item())
    for n, t in orc.named_params():
        assert rel_err(grads[n], t.grad) < 1e-5, f"{n}: rel {rel_err(grads[n], t.grad):.3e}"


def test_boundary_bf16_matches_stock_modules():
    """2-layer TinyLlama-shaped bf16 model, B=2, S=1024: fused embedding and final
    norm vs the stock nn.Embedding / LlamaRMSNorm on the same weights (fused
    layers and loss head on both sides): loss within 1e-3 relative, every
    gradient within the tensor-level bf16 metric."""
    from femtotron_amd import fuse_boundary_ops, fused_checkpoint
    from femtotron_amd.scripts.presets import get_ac_policy
    from femtotron_amd.training import apply_activation_checkpointing
    ids = torch.randint(0, CFG3["vocab"], (2, 1024), generator=torch.Generator().manual_seed(7)).to(DEV)
    res = []
    for fused in (True, False):
        model = _model(CFG3, 2, torch.bfloat16)
        if fused:
            fuse_boundary_ops(model)
        apply_activation_checkpointing(model, get_ac_policy("llama_decoder_layer"), checkpoint_fn=fused_checkpoint)
        loss = model(ids, labels=ids, materialize_logits=False)["loss"]
        loss.backward()
        res.append((loss.detach().float(), {n: p.grad.float() for n, p in model.named_parameters()}))
        del model
    (lf, gf), (lr, gr) = res
    assert abs(lf.item() - lr.item()) <= 1e-3 * abs(lr.item())
    for n in gr:
        err = float((gf[n] - gr[n]).abs().max())
        lim = BF16_ATOL + BF16_RTOL * float(gr[n].abs().max())
        assert err <= lim, f"{n}: {err:.3e} > {lim:.3e}"
