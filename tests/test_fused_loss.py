"""Fused lm_head + chunked cross-entropy (femtotron_amd/fused_loss.py, fh_ce_fwd_bwd).

Checkers: the reference's loss head itself (femtotron/model/llama.py:91-111:
shifted logits, .float(), F.cross_entropy with ignore_index -100) in fp64 on
the CPU for the label shift and the kernel's per-row losses and gradients; the
CPU fp32 oracle model (config 1, 1e-5) end to end; the stock loss head of the
same model on the GPU (bf16, the north star's tensor-level metric).
"""
from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from femtotron_amd.fused_loss import IGNORE_INDEX, shift_labels
from tests.helpers import BF16_ATOL, BF16_RTOL, CFG1, CFG3, llama_config, rel_err

DEV = "cuda:0"


def _labels(B, S, V, seed, ignore_frac=0.1):
    g = torch.Generator().manual_seed(seed)
    lab = torch.randint(0, V, (B, S), generator=g)
    lab[torch.rand(B, S, generator=g) < ignore_frac] = IGNORE_INDEX
    return lab


def test_label_shift_pairs_like_the_reference():
    """CE over all rows with shifted labels == the reference's CE over shifted
    logits (same pairs, same valid count), loss and gradient, fp64."""
    B, S, V = 3, 17, 50
    logits = torch.randn(B, S, V, dtype=torch.float64, generator=torch.Generator().manual_seed(1))
    labels = _labels(B, S, V, 2)
    a = logits.clone().requires_grad_(True)
    ref = F.cross_entropy(a[..., :-1, :].reshape(-1, V), labels[..., 1:].reshape(-1), ignore_index=-100)
    ref.backward()
    b = logits.clone().requires_grad_(True)
    got = F.cross_entropy(b.reshape(-1, V), shift_labels(labels), ignore_index=-100)
    got.backward()
    assert torch.allclose(got, ref, rtol=1e-14, atol=0)
    assert torch.allclose(b.grad, a.grad, rtol=1e-12, atol=1e-16)


def test_materialize_flag_keeps_reference_behaviour_off_device():
    from femtotron_amd.model import build_llama_model, init_llama_weights_
    model = init_llama_weights_(build_llama_model(llama_config(CFG1)), device="cpu", dtype=torch.float32)
    ids = torch.randint(0, CFG1["vocab"], (2, 16), generator=torch.Generator().manual_seed(0))
    a = model(ids, labels=ids)
    b = model(ids, labels=ids, materialize_logits=False)
    assert b["logits"] is not None and torch.equal(a["loss"], b["loss"])


def _ce_truth(x64, labels, inv):
    """Per-row loss and gradient of the reference's CE in fp64."""
    valid = labels != IGNORE_INDEX
    lse = torch.logsumexp(x64, dim=1)
    safe = labels.clamp(min=0)
    loss = torch.where(valid, lse - x64.gather(1, safe[:, None])[:, 0], torch.zeros_like(lse))
    p = torch.softmax(x64, dim=1)
    p[torch.arange(len(labels)), safe] -= 1.0
    grad = torch.where(valid[:, None], p * inv, torch.zeros_like(p))
    return loss, grad


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("rows,V", [(37, 1024), (64, 32000), (9, 70016)])
def test_ce_kernel_matches_fp64(dtype, rows, V):
    """Row losses and the in-place gradient vs the fp64 reference: fp32 within
    1e-5 (relative, per tensor); bf16 gradient = the fp64 value rounded to bf16
    up to one bf16 ulp.  V = 70016 takes the streaming path (> 65536)."""
    from femtotron_amd import ops
    g = torch.Generator().manual_seed(rows + V)
    x = (torch.randn(rows, V, generator=g) * 3).to(dtype)
    labels = _labels(1, rows, V, rows)[0]
    n_valid = int((labels != IGNORE_INDEX).sum())
    inv = 1.0 / n_valid
    loss_t, grad_t = _ce_truth(x.double(), labels, inv)
    xd = x.to(DEV)
    loss_rows = ops.ce_fwd_bwd_(xd, labels.to(DEV), torch.tensor([inv], dtype=torch.float32, device=DEV))
    assert rel_err(loss_rows.double().cpu(), loss_t) < 1e-5
    got = xd.cpu()
    if dtype == torch.float32:
        assert rel_err(got.double(), grad_t) < 1e-5
    else:
        want = grad_t.to(torch.bfloat16)
        ulp = (want.float().abs() * 2.0 ** -7).clamp(min=2.0 ** -126)
        assert bool(((got.float() - want.float()).abs() <= ulp).all())
        assert torch.equal(got[labels == IGNORE_INDEX], torch.zeros_like(got[labels == IGNORE_INDEX]))


@pytest.mark.gpu
def test_ce_kernel_out_of_range_label_gives_nan_row():
    """A label outside [0, V) (torch raises) yields a NaN loss and gradient row;
    the kernel never addresses memory with it."""
    from femtotron_amd import ops
    x = torch.randn(4, 1024, device=DEV)
    labels = torch.tensor([3, 1024, -100, -5], device=DEV)
    loss = ops.ce_fwd_bwd_(x, labels, torch.tensor([0.5], device=DEV))
    assert torch.isfinite(loss[0]) and torch.isnan(loss[1]) and loss[2] == 0 and torch.isnan(loss[3])
    assert torch.isnan(x[1]).all() and (x[2] == 0).all() and torch.isfinite(x[0]).all()


def _model(c, layers, dtype, seed=42):
    from femtotron_amd.model import build_llama_model, init_llama_weights_
    return init_llama_weights_(build_llama_model(llama_config(c, layers=layers)), device=DEV,
                               dtype=dtype, seed=seed)


@pytest.mark.gpu
def test_fused_loss_cfg1_fp32_vs_cpu_oracle():
    """Config 1 end to end with fused layers and the fused loss head: loss and
    all 21 gradients within 1e-5 of the CPU fp32 oracle."""
    from femtotron_amd import fused_checkpoint
    from femtotron_amd.scripts.presets import get_ac_policy
    from femtotron_amd.training import apply_activation_checkpointing
    from oracle import torch_llama as ot
    c = CFG1
    model = _model(c, c["layers"], torch.float32)
    apply_activation_checkpointing(model, get_ac_policy("llama_decoder_layer"), checkpoint_fn=fused_checkpoint)
    ids = torch.randint(0, c["vocab"], (c["batch"], c["seq"]), generator=torch.Generator().manual_seed(2000))
    out = model(ids.to(DEV), labels=ids.to(DEV), materialize_logits=False)
    assert out["logits"] is None
    out["loss"].backward()
    grads = {n.replace("._checkpoint_wrapped_module", ""): p.grad for n, p in model.named_parameters()}
    orc = ot.OracleLlama(vocab=c["vocab"], hidden=c["hidden"], n_layers=c["layers"], n_heads=c["heads"],
                         n_kv=c["kv"], ffn=c["ffn"], theta=c["theta"])
    _, oloss = orc.forward(ids, ids)
    oloss.backward()
    assert abs(out["loss"].item() - oloss.item()) <= 1e-5 * abs(oloss.item())
    for n, t in orc.named_params():
        assert rel_err(grads[n], t.grad) < 1e-5, f"{n}: rel {rel_err(grads[n], t.grad):.3e}"


@pytest.mark.gpu
def test_fused_loss_bf16_matches_stock_loss_head():
    """2-layer TinyLlama-shaped bf16 model, B=2, S=1024 (two chunks of logits):
    fused loss head vs the stock one, same model and weights; loss within 1e-3
    relative, every gradient within the tensor-level bf16 metric."""
    from femtotron_amd import fused_checkpoint
    from femtotron_amd.scripts.presets import get_ac_policy
    from femtotron_amd.training import apply_activation_checkpointing
    import femtotron_amd.fused_loss as fl
    model = _model(CFG3, 2, torch.bfloat16)
    apply_activation_checkpointing(model, get_ac_policy("llama_decoder_layer"), checkpoint_fn=fused_checkpoint)
    ids = torch.randint(0, CFG3["vocab"], (2, 1024), generator=torch.Generator().manual_seed(7)).to(DEV)
    res = []
    old = fl.CHUNK_BYTES
    fl.CHUNK_BYTES = 64 << 20  # 1024 rows per chunk at V = 32000: exercise chunking
    try:
        for fused in (True, False):
            for p in model.parameters():
                p.grad = None
            loss = model(ids, labels=ids, materialize_logits=not fused)["loss"]
            loss.backward()
            res.append((loss.detach().float(), {n: p.grad.float() for n, p in model.named_parameters()}))
    finally:
        fl.CHUNK_BYTES = old
    (lf, gf), (lr, gr) = res
    assert abs(lf.item() - lr.item()) <= 1e-3 * abs(lr.item())
    for n in gr:
        err = float((gf[n] - gr[n]).abs().max())
        lim = BF16_ATOL + BF16_RTOL * float(gr[n].abs().max())
        assert err <= lim, f"{n}: {err:.3e} > {lim:.3e}"


@pytest.mark.gpu
def test_fused_loss_lowers_peak_activation_memory():
    """Peak memory of one fwd+bwd of a 2-layer TinyLlama-shaped model (B=4, S=2048):
    the fused loss head needs less than half of the stock one's (no [T, V] fp32 logits)."""
    from femtotron_amd import fused_checkpoint
    from femtotron_amd.scripts.presets import get_ac_policy
    from femtotron_amd.training import apply_activation_checkpointing
    model = _model(CFG3, 2, torch.bfloat16)
    apply_activation_checkpointing(model, get_ac_policy("llama_decoder_layer"), checkpoint_fn=fused_checkpoint)
    ids = torch.randint(0, CFG3["vocab"], (4, 2048), generator=torch.Generator().manual_seed(3)).to(DEV)

    def peak(fused):
        for _ in range(2):
            torch.cuda.synchronize()
            torch.cuda.reset_peak_memory_stats()
            base = torch.cuda.memory_allocated()
            model(ids, labels=ids, materialize_logits=not fused)["loss"].backward()
            torch.cuda.synchronize()
        return torch.cuda.max_memory_allocated() - base

    p_stock = peak(False)
    p_fused = peak(True)
    assert p_fused < 0.5 * p_stock, f"fused {p_fused / 2**20:.0f} MiB vs stock {p_stock / 2**20:.0f} MiB"
