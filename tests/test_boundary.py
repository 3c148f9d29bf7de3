"""Embedding and final-norm boundary ops, host side (no GPU): the oracle pinned
against torch's own F.embedding, and the module swap of fuse_boundary_ops."""
from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

from oracle import embedding as oe
from tests.helpers import CFG1, llama_config


def _ids(T, V, seed, bad=0):
    g = np.random.default_rng(seed)
    ids = g.integers(0, V, size=T)
    if bad:
        pos = g.choice(T, size=bad, replace=False)
        ids[pos[: bad // 2]] = -g.integers(1, 5, size=bad // 2)
        ids[pos[bad // 2:]] = V + g.integers(0, 5, size=bad - bad // 2)
    return ids.astype(np.int64)


def test_oracle_matches_torch_embedding_fp64():
    """Forward and weight gradient vs torch's F.embedding in fp64, with repeated
    ids and padding_idx; masked ids (outside [0, V)) follow the one-rank
    VocabParallelEmbedding: zero rows, no gradient."""
    V, H, T = 50, 16, 300
    g = torch.Generator().manual_seed(0)
    w = torch.randn(V, H, dtype=torch.float64, generator=g)
    dy = torch.randn(T, H, dtype=torch.float64, generator=g)
    ids = _ids(T, V, 1)
    for pad in (None, 7):
        wr = w.clone().requires_grad_(True)
        out = F.embedding(torch.from_numpy(ids), wr, padding_idx=pad)
        out.backward(dy)
        assert np.array_equal(oe.embedding_fwd(ids, w.numpy()), out.detach().numpy())
        assert np.allclose(oe.embedding_bwd(dy.numpy(), ids, V, pad), wr.grad.numpy(), rtol=1e-13, atol=1e-13)
    # masked ids: the reference's mask -> row 0 -> zero output; gradient skips them
    bad = _ids(T, V, 2, bad=20)
    mask = torch.from_numpy((bad < 0) | (bad >= V))
    wr = w.clone().requires_grad_(True)
    out = F.embedding(torch.from_numpy(bad).masked_fill(mask, 0), wr).masked_fill(mask[:, None], 0)
    out.backward(dy)
    assert np.array_equal(oe.embedding_fwd(bad, w.numpy()), out.detach().numpy())
    assert np.allclose(oe.embedding_bwd(dy.numpy(), bad, V), wr.grad.numpy(), rtol=1e-13, atol=1e-13)


def test_ordered_fp32_sums():
    """The ordered fp32 statement vs a brute-force per-row loop in token order
    (bit-exact) and vs the exact fp64 sums (within fp32 rounding)."""
    V, H, T = 40, 8, 500
    ids = _ids(T, V, 3)
    ids[:60] = 5  # one long row
    dy = np.random.default_rng(4).standard_normal((T, H)).astype(np.float32)
    got = oe.embedding_bwd_ordered(dy, ids, V, padding_idx=9)
    want = np.zeros((V, H), np.float32)
    for v in range(V):
        if v == 9:
            continue
        acc = np.zeros(H, np.float32)
        for t in np.nonzero(ids == v)[0]:
            acc = acc + dy[t]
        want[v] = acc
    assert np.array_equal(got, want)
    exact = oe.embedding_bwd(dy, ids, V, 9)
    assert np.allclose(got, exact, rtol=1e-5, atol=1e-5)
    assert np.all(got[9] == 0)


def test_fuse_boundary_ops_swaps_modules_keeping_parameters():
    from transformers.models.llama.modeling_llama import LlamaRMSNorm

    from femtotron_amd import fuse_boundary_ops
    from femtotron_amd.boundary_ops import FusedEmbedding, FusedRMSNorm
    from femtotron_amd.model import build_llama_model, init_llama_weights_
    model = init_llama_weights_(build_llama_model(llama_config(CFG1)), device="cpu", dtype=torch.float32)
    emb, norm = model.model.embed_tokens, model.model.norm
    assert isinstance(norm, LlamaRMSNorm)
    keys = list(model.state_dict().keys())
    ids = torch.randint(0, CFG1["vocab"], (2, 16), generator=torch.Generator().manual_seed(0))
    x = torch.randn(2, 16, CFG1["hidden"], generator=torch.Generator().manual_seed(1))
    e_ref, n_ref = emb(ids), norm(x)
    out_ref = model(ids, labels=ids)["loss"]
    assert fuse_boundary_ops(model) == 2
    assert isinstance(model.model.embed_tokens, FusedEmbedding) and isinstance(model.model.norm, FusedRMSNorm)
    assert model.model.embed_tokens.weight is emb.weight and model.model.norm.weight is norm.weight
    assert list(model.state_dict().keys()) == keys
    assert fuse_boundary_ops(model) == 0  # idempotent
    # off the GPU the swapped modules compute what the replaced ones did
    assert torch.equal(model.model.embed_tokens(ids), e_ref)
    assert torch.equal(model.model.norm(x), n_ref)
    assert torch.equal(model(ids, labels=ids)["loss"], out_ref)
    bad = ids.clone()
    bad[0, 0], bad[1, 3] = -1, CFG1["vocab"]
    out = model.model.embed_tokens(bad)
    assert torch.all(out[0, 0] == 0) and torch.all(out[1, 3] == 0)
    from femtotron_amd.boundary_ops import unfuse_boundary_ops
    assert unfuse_boundary_ops(model) == 2
    assert type(model.model.embed_tokens) is torch.nn.Embedding and type(model.model.norm) is LlamaRMSNorm
    assert model.model.embed_tokens.weight is emb.weight and model.model.norm.weight is norm.weight
    assert torch.equal(model(ids, labels=ids)["loss"], out_ref)
