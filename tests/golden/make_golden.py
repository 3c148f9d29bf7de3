"""Writes the golden fixtures of the reference's checkpointed model (run in the
survey/build container only; the GPU box never runs this).

What only the reference itself can pin: its own end-to-end model stack at
TP = 1 — femtotron's LlamaForTraining / LlamaPartialModel with the layer linears
swapped for ColumnParallelLinear / RowParallelLinear and the embedding for
VocabParallelEmbedding by parallelize_model (femtotron/model/llama.py:161-194),
the shifted fp32 cross-entropy (llama.py:91-111), and every layer wrapped by
femtotron's ActivationCheckpointWrapper (activation_ckpt.py:34-132, which calls
torch.utils.checkpoint with debug=True).  This script imports that stack from
/root/reference on the CPU (gloo, world size 1, as the reference's
ParallelContext needs an initialised process group) and records its outputs and
gradients for:

  cfg1.json   BASELINE config 1: 2 layers, hidden 256, 8/4 heads, ffn 688,
              vocab 1024, fp32, batch 2 x seq 128, token ids from CPU
              Generator(2000), all weights N(0, 0.02) drawn in the reference's
              parameter registration order from CPU Generator(42).
  layer_bf16.npz  one checkpointed LlamaDecoderLayer of config 1 in bf16 on
              (2, 32) tokens: input, output, input gradient and weight
              gradients as exact bf16 bit patterns (weights drawn from CPU
              Generator(7) in registration order, norm weights 1 + N(0, 0.02),
              the others N(0, 0.02); their checksums are stored to verify a
              regeneration).

Large tensors are stored as checksums that pin every element: sum, sum of
squares, max |x|, and four seeded random projections (float64).  The
fixtures hold data only (inputs and outputs); no reference source is copied.

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import json
import os
import sys
from collections import OrderedDict
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
REF = Path("/root/reference")
PROJ_SEEDS = (11, 22, 33, 44)


def checksum(t: torch.Tensor) -> dict:
    """Element-pinning summary of a tensor (float64 arithmetic)."""
    x = t.detach().double().reshape(-1).cpu()
    out = {"shape": list(t.shape), "sum": float(x.sum()), "sumsq": float((x * x).sum()),
           "absmax": float(x.abs().max()) if x.numel() else 0.0}
    for s in PROJ_SEEDS:
        g = torch.Generator().manual_seed(s * 1000 + x.numel() % 997)
        r = torch.randn(x.numel(), generator=g, dtype=torch.float64)
        out[f"proj{s}"] = float((x * r).sum())
    return out


def main() -> None:
    sys.path.insert(0, str(REF))
    import torch.distributed as dist
    os.environ.setdefault("MASTER_ADDR", "127.0.0.1")
    os.environ.setdefault("MASTER_PORT", "29533")
    dist.init_process_group("gloo", rank=0, world_size=1)
    from transformers import LlamaConfig
    from transformers.models.llama.modeling_llama import LlamaDecoderLayer

    from femtotron.model.llama import build_llama_model
    from femtotron.parallel_context import ParallelContext
    from femtotron.scripts.presets import get_ac_policy
    from femtotron.training.activation_ckpt import (ActivationCheckpointWrapper,
                                                    apply_activation_checkpointing)

    torch.manual_seed(0)
    cfg = LlamaConfig(hidden_size=256, intermediate_size=688, num_attention_heads=8,
                      num_key_value_heads=4, num_hidden_layers=2, vocab_size=1024,
                      rms_norm_eps=1e-5, hidden_act="silu", max_position_embeddings=512,
                      tie_word_embeddings=False, rope_theta=10000.0, attention_dropout=0.0)
    ctx = ParallelContext(OrderedDict([("tp", 1)]))

    # ---------------------------------------------------------------- cfg 1
    model = build_llama_model(cfg, ctx).to_empty(device="cpu")
    gen = torch.Generator().manual_seed(42)
    names = []
    with torch.no_grad():
        for name, p in model.named_parameters():
            p.copy_(torch.empty(p.shape, dtype=torch.float32).normal_(0.0, 0.02, generator=gen))
            names.append(name)
        for m in model.modules():  # to_empty leaves inv_freq uninitialised
            if type(m).__name__ == "LlamaRotaryEmbedding":
                inv, _ = m.compute_default_rope_parameters(m.config)
                m.inv_freq = inv.clone()
                m.original_inv_freq = inv.clone()
    n_wrapped = apply_activation_checkpointing(model, get_ac_policy("llama_decoder_layer"),
                                               use_reentrant=False, preserve_rng_state=True)
    ids = torch.randint(0, 1024, (2, 128), generator=torch.Generator().manual_seed(2000))
    out = model(ids, labels=ids)
    out["loss"].backward()
    # parameter names without the wrapper's child name (as state_dict shows them)
    params = {n.replace("_checkpoint_wrapped_module.", ""): p for n, p in model.named_parameters()}
    assert list(params) == names
    sd_names = list(model.state_dict().keys())
    fixture = {
        "config": {"hidden": 256, "heads": 8, "kv_heads": 4, "ffn": 688, "vocab": 1024, "layers": 2,
                   "eps": 1e-5, "theta": 10000.0, "batch": 2, "seq": 128, "dtype": "float32",
                   "weight_seed": 42, "token_seed": 2000, "init_std": 0.02},
        "n_wrapped": n_wrapped,
        "param_names": names,
        "state_dict_keys": sd_names,
        "ids_sum": int(ids.sum()),
        "loss": float(out["loss"].item()),
        "logits": checksum(out["logits"]),
        "weights": {n: checksum(p) for n, p in params.items()},
        "grads": {n: checksum(p.grad) for n, p in params.items()},
        "grads_full_small": {n: p.grad.double().reshape(-1).tolist()
                             for n, p in params.items() if p.numel() <= 4096},
    }
    (HERE / "cfg1.json").write_text(json.dumps(fixture, indent=1))
    print(f"cfg1: loss {fixture['loss']:.8f}, {len(names)} params, {n_wrapped} wrapped")

    # -------------------------------------------------- one bf16 layer
    layer = LlamaDecoderLayer(cfg, layer_idx=0)
    gen = torch.Generator().manual_seed(7)
    with torch.no_grad():
        for name, p in layer.named_parameters():
            w = torch.empty(p.shape, dtype=torch.float32).normal_(0.0, 0.02, generator=gen)
            if name.endswith("layernorm.weight"):
                w += 1.0
            p.copy_(w)
    layer = layer.bfloat16()
    wrapped = ActivationCheckpointWrapper(layer, use_reentrant=False, preserve_rng_state=True)
    S = 32
    x = torch.randn(2, S, 256, generator=torch.Generator().manual_seed(8)).bfloat16()
    dy = torch.randn(2, S, 256, generator=torch.Generator().manual_seed(9)).bfloat16()
    inv = 1.0 / (10000.0 ** (torch.arange(0, 32, 2, dtype=torch.float32) / 32))
    freqs = torch.arange(S, dtype=torch.float32)[:, None] * inv[None]
    emb = torch.cat((freqs, freqs), -1)
    cos, sin = emb.cos()[None].bfloat16(), emb.sin()[None].bfloat16()
    xg = x.clone().requires_grad_(True)
    y = wrapped(xg, attention_mask=None, position_embeddings=(cos, sin),
                position_ids=torch.arange(S)[None], past_key_values=None, use_cache=False)
    y.backward(dy)
    def bits(t):  # bf16 values stored exactly, as their 16-bit patterns
        return t.detach().contiguous().view(torch.int16).numpy()

    arrays = {"x": bits(x), "dy": bits(dy), "cos": bits(cos), "sin": bits(sin),
              "out": bits(y), "dx": bits(xg.grad)}
    for name, p in layer.named_parameters():
        arrays["wsum:" + name] = np.array([checksum(p)["sum"], checksum(p)["proj11"]])
        arrays["g:" + name] = bits(p.grad)
    np.savez_compressed(HERE / "layer_bf16.npz", **arrays)
    print(f"layer_bf16: out absmax {float(y.detach().abs().max()):.4f}")
    dist.destroy_process_group()


if __name__ == "__main__":
    main()
