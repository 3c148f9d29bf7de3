"""Shared test helpers: configs, seeded inputs, tolerance checks."""
from __future__ import annotations

import torch
from transformers import LlamaConfig

# BASELINE configs (hidden, heads, kv heads, ffn, vocab, layers, theta, batch, seq)
CFG1 = dict(hidden=256, heads=8, kv=4, ffn=688, vocab=1024, layers=2, theta=10000.0, batch=2, seq=128)
CFG3 = dict(hidden=2048, heads=32, kv=4, ffn=5632, vocab=32000, layers=22, theta=10000.0, batch=8, seq=2048)
CFG4 = dict(hidden=4096, heads=32, kv=8, ffn=14336, vocab=128256, layers=8, theta=500000.0, batch=1, seq=8192)
CFG5 = dict(hidden=4096, heads=32, kv=32, ffn=11008, vocab=32000, layers=4, theta=10000.0, batch=1, seq=32768)

# bf16 tolerance of the north star, and the fp32 one.
BF16_RTOL, BF16_ATOL = 2e-2, 2e-3
F32_TOL = 1e-5


def llama_config(c: dict, layers: int | None = None, attn: str = "sdpa") -> LlamaConfig:
    cfg = LlamaConfig(hidden_size=c["hidden"], intermediate_size=c["ffn"],
                      num_attention_heads=c["heads"], num_key_value_heads=c["kv"],
                      num_hidden_layers=layers if layers is not None else c["layers"],
                      vocab_size=c["vocab"], rms_norm_eps=1e-5, hidden_act="silu",
                      max_position_embeddings=max(2048, c["seq"]), tie_word_embeddings=False,
                      rope_theta=c["theta"], attention_dropout=0.0)
    cfg._attn_implementation = attn
    return cfg


def gen(seed: int) -> torch.Generator:
    return torch.Generator(device="cpu").manual_seed(seed)


def randn(shape, seed: int, std: float = 1.0, mean: float = 0.0) -> torch.Tensor:
    return torch.randn(shape, generator=gen(seed), dtype=torch.float32) * std + mean


def layer_weights(c: dict, seed: int = 42, std: float = 0.02, norm_mean: float = 0.0) -> dict:
    """The 9 weights of one layer, N(0, std) from CPU Generator(seed) in the
    reference's registration order; norm weights optionally shifted by norm_mean."""
    from oracle.torch_llama import LAYER_KEYS, layer_weight_shapes
    g = gen(seed)
    hd = c["hidden"] // c["heads"]
    shapes = layer_weight_shapes(c["hidden"], c["heads"], c["kv"], hd, c["ffn"])
    out = {}
    for k in LAYER_KEYS:
        t = torch.empty(shapes[k], dtype=torch.float32).normal_(0.0, std, generator=g)
        if k in ("w1", "w2"):
            t = t + norm_mean
        out[k] = t
    return out


def load_into_hf_layer(layer, w: dict) -> None:
    with torch.no_grad():
        a, m = layer.self_attn, layer.mlp
        a.q_proj.weight.copy_(w["wq"]); a.k_proj.weight.copy_(w["wk"])
        a.v_proj.weight.copy_(w["wv"]); a.o_proj.weight.copy_(w["wo"])
        m.gate_proj.weight.copy_(w["wg"]); m.up_proj.weight.copy_(w["wu"])
        m.down_proj.weight.copy_(w["wd"])
        layer.input_layernorm.weight.copy_(w["w1"])
        layer.post_attention_layernorm.weight.copy_(w["w2"])


def hf_layer_grads(layer) -> dict:
    a, m = layer.self_attn, layer.mlp
    return {"wq": a.q_proj.weight.grad, "wk": a.k_proj.weight.grad, "wv": a.v_proj.weight.grad,
            "wo": a.o_proj.weight.grad, "wg": m.gate_proj.weight.grad, "wu": m.up_proj.weight.grad,
            "wd": m.down_proj.weight.grad, "w1": layer.input_layernorm.weight.grad,
            "w2": layer.post_attention_layernorm.weight.grad}


def assert_close(a: torch.Tensor, b: torch.Tensor, rtol: float, atol: float, name: str = "") -> None:
    a = a.detach().float().cpu()
    b = b.detach().float().cpu()
    assert a.shape == b.shape, f"{name}: shape {tuple(a.shape)} vs {tuple(b.shape)}"
    assert torch.isfinite(a).all(), f"{name}: non-finite values"
    err = (a - b).abs()
    bound = atol + rtol * b.abs()
    bad = err > bound
    if bad.any():
        i = int(torch.argmax((err - bound).flatten()))
        raise AssertionError(
            f"{name}: {int(bad.sum())}/{a.numel()} elements outside rtol={rtol} atol={atol}; "
            f"worst |a-b|={err.flatten()[i]:.3e} at b={b.flatten()[i]:.3e}; "
            f"max|a-b|={err.max():.3e}, max|b|={b.abs().max():.3e}")


def assert_tensor_close(a: torch.Tensor, b: torch.Tensor, rtol: float, atol: float, name: str = "") -> None:
    """Per tensor max|a-b| <= atol + rtol * max|b|: the form of the reference's
    compare_grads (femtotron/test/unit/test_pipeline_stage.py:82-128, rtol
    1.5e-3 there, for paths with identical arithmetic); callers pass the north
    star's rtol 2e-2 / atol 2e-3 for independent bf16 implementations."""
    a = a.detach().float().cpu()
    b = b.detach().float().cpu()
    assert a.shape == b.shape, f"{name}: shape {tuple(a.shape)} vs {tuple(b.shape)}"
    assert torch.isfinite(a).all(), f"{name}: non-finite values"
    err = float((a - b).abs().max())
    lim = atol + rtol * float(b.abs().max())
    assert err <= lim, f"{name}: max|a-b|={err:.3e} > {lim:.3e}"


def rel_err(a: torch.Tensor, b: torch.Tensor) -> float:
    a = a.detach().float().cpu()
    b = b.detach().float().cpu()
    return float((a - b).abs().max() / b.abs().max().clamp_min(1e-30))
