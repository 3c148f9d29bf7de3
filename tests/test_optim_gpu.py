"""Fused mixed-precision AdamW (femtotron_amd/optim.py, fh_adamw_step) vs the reference's step.

The checker is the reference's own sequence on the GPU in fp32
(femtotron/training/mixed_precision_manager.py:318-331): master.grad =
param.grad.float(); ClipGradNorm (grad_transform.py:13-63, coef =
clamp(max_norm / (norm + 1e-6), max=1) applied to every gradient);
torch.optim.AdamW (foreach) on the masters with per-group weight decay;
param.copy_(master).  Three steps with fresh gradients and a changing learning
rate; tensor sizes include non-multiples of 8 and both weight-decay groups.  Bar: masters, moments within
1e-6 relative (fp32 arithmetic in a different operation order), the model-dtype
parameters equal up to one bf16 ulp on a vanishing fraction of elements.
"""
from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
SHAPES = [(256, 688), (1000,), (7,), (2048,), (33, 24)]


def _setup(dtype, seed):
    g = torch.Generator().manual_seed(seed)
    ps = [torch.randn(*s, generator=g).mul_(0.02).to(DEV, dtype) for s in SHAPES]
    groups = [{"params": [p for p in ps if p.dim() > 1], "weight_decay": 0.01},
              {"params": [p for p in ps if p.dim() <= 1], "weight_decay": 0.0}]
    return ps, groups


def _reference_step(ps, masters, opt, max_norm):
    for p, m in zip(ps, masters):
        m.grad = p.grad.float()
    grads = [m.grad for m in masters]
    total = torch.zeros((), device=DEV)
    for gr in grads:
        total += gr.float().pow(2).sum()
    norm = total.sqrt()
    coef = (max_norm / (norm + 1e-6)).clamp(max=1.0)
    for gr in grads:
        gr.mul_(coef)
    opt.step()
    with torch.no_grad():
        for p, m in zip(ps, masters):
            p.copy_(m)
    return norm


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("grad_scale,max_norm", [(1.0, 1.0), (0.001, 1.0), (1.0, 0.0)])
def test_fused_adamw_matches_reference_step(dtype, grad_scale, max_norm):
    """grad_scale 1: the global norm (~18) is clipped to 1; 0.001: no clipping
    (coef = 1); max_norm 0: clipping disabled."""
    from femtotron_amd.optim import FusedAdamW
    ps_f, groups_f = _setup(dtype, 1)
    ps_r, groups_r = _setup(dtype, 1)
    kw = dict(lr=3e-3, betas=(0.9, 0.95), eps=1e-8)
    fused = FusedAdamW(groups_f, max_grad_norm=max_norm, **kw)
    masters_r = [p.detach().float().clone().requires_grad_(True) for p in ps_r]
    mgroups = [{"params": [m for m, p in zip(masters_r, ps_r) if any(p is q for q in g["params"])],
                "weight_decay": g["weight_decay"]} for g in groups_r]
    ref = torch.optim.AdamW(mgroups, foreach=True, **kw)
    gen = torch.Generator().manual_seed(5)
    for step in range(3):
        lr = 3e-3 * (1.0 - 0.25 * step)  # a schedule: the device table is rebuilt each step
        for g in ref.param_groups:
            g["lr"] = lr
        grads = [torch.randn(*s, generator=gen).mul_(grad_scale) for s in SHAPES]
        for p, gr in zip(ps_f, grads):
            p.grad = gr.to(DEV, dtype)
        for p, gr in zip(ps_r, grads):
            p.grad = gr.to(DEV, dtype)
        for g in fused.param_groups:
            g["lr"] = lr
        fused.step()
        if max_norm > 0:
            norm_r = _reference_step(ps_r, masters_r, ref, max_norm)
        else:
            for p, m in zip(ps_r, masters_r):
                m.grad = p.grad.float()
            ref.step()
            with torch.no_grad():
                for p, m in zip(ps_r, masters_r):
                    p.copy_(m)
            norm_r = torch.sqrt(sum((m.grad.float() ** 2).sum() for m in masters_r))
        assert abs(fused.grad_norm.item() - norm_r.item()) <= 1e-5 * norm_r.item()
        by_param = {id(e[0]): e for e in fused.entries}
        assert len(by_param) == len(SHAPES)
        for pf, pr, mr in zip(ps_f, ps_r, masters_r):
            p, _, m, e1, e2 = by_param[id(pf)]
            st = ref.state[mr]
            for a, b, n in ((m, mr, "master"), (e1, st["exp_avg"], "exp_avg"), (e2, st["exp_avg_sq"], "exp_avg_sq")):
                b = b.detach()
                err = float((a - b).abs().max())
                assert err <= 1e-6 * float(b.abs().max()) + 1e-12, f"step {step} {n}: {err:.3e}"
            if dtype == torch.float32:
                assert float((p - pr).abs().max()) <= 1e-6 * float(pr.abs().max())
            else:
                diff = (p.float() - pr.float()).abs()
                ulp = pr.float().abs() * 2.0 ** -7
                assert bool((diff <= ulp).all())
                assert float((diff > 0).float().mean()) < 1e-2


def test_fused_adamw_on_a_model_step():
    """A config-1 bf16 model trained with the fused path end to end (fused
    layers, fused loss head, fused optimizer) under the reference's LambdaLR
    warm-up schedule: the loss decreases, the parameters track their fp32
    masters, and a state_dict round trip resumes bit-identically."""
    from femtotron_amd import fused_checkpoint, pack_layer_weights
    from femtotron_amd.model import build_llama_model, init_llama_weights_
    from femtotron_amd.optim import FusedAdamW, get_param_groups
    from femtotron_amd.scripts.presets import get_ac_policy
    from femtotron_amd.training import apply_activation_checkpointing
    from tests.helpers import CFG1, llama_config
    model = init_llama_weights_(build_llama_model(llama_config(CFG1)), device=DEV, dtype=torch.bfloat16)
    pack_layer_weights(model)
    apply_activation_checkpointing(model, get_ac_policy("llama_decoder_layer"), checkpoint_fn=fused_checkpoint)
    opt = FusedAdamW(get_param_groups(model, 0.01), lr=1e-2, max_grad_norm=1.0)
    sched = torch.optim.lr_scheduler.LambdaLR(opt, lambda s: min(1.0, (s + 1) / 3))
    ids = torch.randint(0, CFG1["vocab"], (2, 128), generator=torch.Generator().manual_seed(0)).to(DEV)

    def train_step():
        loss = model(ids, labels=ids, materialize_logits=False)["loss"]
        loss.backward()
        opt.step()
        opt.zero_grad()
        sched.step()
        return loss.item()

    losses = [train_step() for _ in range(4)]
    assert losses[3] < losses[0]
    assert opt.step_count == 4 and torch.isfinite(opt.grad_norm)
    assert opt.param_groups[0]["lr"] == pytest.approx(1e-2)
    for p, _, m, _, _ in opt.entries:
        assert torch.equal(p, m.to(torch.bfloat16))
    # resume: the state of step 4, then step 5 twice from it
    saved = {k: v for k, v in opt.state_dict().items()}
    saved["state"] = {i: {k: t.clone() if torch.is_tensor(t) else t for k, t in st.items()}
                      for i, st in saved["state"].items()}
    params0 = [p.detach().clone() for p in model.parameters()]
    train_step()
    after = [p.detach().clone() for p in model.parameters()]
    with torch.no_grad():
        for p, p0 in zip(model.parameters(), params0):
            p.copy_(p0)
    opt.load_state_dict(saved)
    assert opt.step_count == 4
    train_step()
    for p, a in zip(model.parameters(), after):
        assert torch.equal(p, a)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_parameter_without_grad_steps_like_the_reference(dtype):
    """Three steps where one parameter has no gradient on step 2: the
    reference's MixedPrecisionManager fills it with zeros before
    torch.optim.AdamW's step (mixed_precision_manager.py:224-229), so the
    parameter still decays and its moments and step count advance; the fused
    step must match that sequence, bias corrections included."""
    from femtotron_amd.optim import FusedAdamW
    ps_f, groups_f = _setup(dtype, 3)
    ps_r, groups_r = _setup(dtype, 3)
    kw = dict(lr=3e-3, betas=(0.9, 0.95), eps=1e-8)
    fused = FusedAdamW(groups_f, max_grad_norm=1.0, **kw)
    masters_r = [p.detach().float().clone().requires_grad_(True) for p in ps_r]
    mgroups = [{"params": [m for m, p in zip(masters_r, ps_r) if any(p is q for q in g["params"])],
                "weight_decay": g["weight_decay"]} for g in groups_r]
    ref = torch.optim.AdamW(mgroups, foreach=True, **kw)
    gen = torch.Generator().manual_seed(9)
    skip = 0  # the [256, 688] weight (weight-decay group) has no gradient on step 2
    for step in range(3):
        grads = [torch.randn(*s, generator=gen) for s in SHAPES]
        for i, (pf, pr, gr) in enumerate(zip(ps_f, ps_r, grads)):
            if step == 1 and i == skip:
                pf.grad = None
                pr.grad = torch.zeros_like(pr)  # the reference's zeros_like fill
            else:
                pf.grad = gr.to(DEV, dtype)
                pr.grad = gr.to(DEV, dtype)
        fused.step()
        _reference_step(ps_r, masters_r, ref, 1.0)
        by_param = {id(e[0]): e for e in fused.entries}
        for pf, pr, mr in zip(ps_f, ps_r, masters_r):
            p, _, m, e1, e2 = by_param[id(pf)]
            st = ref.state[mr]
            assert fused.state[pf]["step"] == int(st["step"]) == step + 1
            for a, b, n in ((m, mr, "master"), (e1, st["exp_avg"], "exp_avg"), (e2, st["exp_avg_sq"], "exp_avg_sq")):
                b = b.detach()
                err = float((a - b).abs().max())
                assert err <= 1e-6 * float(b.abs().max()) + 1e-12, f"step {step} {n}: {err:.3e}"


def test_per_tensor_step_counts_after_restore():
    """Tensors whose restored step counts differ get their own bias
    corrections: state with steps (5, 1) then one step equals torch AdamW
    restored to the same per-parameter state."""
    from femtotron_amd.optim import FusedAdamW
    g = torch.Generator().manual_seed(4)
    shapes = [(64, 40), (96,)]
    ps = [torch.randn(*s, generator=g).mul_(0.02).to(DEV, torch.float32) for s in shapes]
    masters = [p.detach().clone().requires_grad_(True) for p in ps]
    kw = dict(lr=1e-2, betas=(0.9, 0.95), eps=1e-8)
    fused = FusedAdamW([{"params": ps, "weight_decay": 0.1}], max_grad_norm=0.0, **kw)
    ref = torch.optim.AdamW([{"params": masters, "weight_decay": 0.1}], foreach=False, **kw)
    m1 = [torch.randn(*s, generator=g).mul_(0.01) for s in shapes]
    m2 = [torch.randn(*s, generator=g).abs().mul_(1e-4) for s in shapes]
    sd = fused.state_dict()
    for i, steps in enumerate((5, 1)):
        sd["state"][i] = {"step": steps, "master": ps[i].detach().float().clone(),
                          "exp_avg": m1[i].to(DEV), "exp_avg_sq": m2[i].to(DEV)}
        ref.state[masters[i]] = {"step": torch.tensor(float(steps)), "exp_avg": m1[i].to(DEV).clone(),
                                 "exp_avg_sq": m2[i].to(DEV).clone()}
    fused.load_state_dict(sd)
    grads = [torch.randn(*s, generator=g).to(DEV) for s in shapes]
    for p, m, gr in zip(ps, masters, grads):
        p.grad = gr.clone()
        m.grad = gr.clone()
    fused.step()
    ref.step()
    for p, m in zip(ps, masters):
        assert float((p - m.detach()).abs().max()) <= 1e-6 * float(m.detach().abs().max())
