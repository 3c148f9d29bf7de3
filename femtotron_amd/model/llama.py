"""LlamaForTraining + build_llama_model + seeded initialisation.

``LlamaForTraining`` mirrors femtotron/model/llama.py:20-123: backbone
``self.model = LlamaPartialModel``, ``self.lm_head`` (bias-free Linear, tied to
the embedding when ``tie_word_embeddings``), ``use_cache = False``, and
``forward(input_ids, labels=None, materialize_logits=True) -> {"logits", "loss"}``
with the shifted next-token cross-entropy computed on fp32 logits, ignore_index
-100 (:72-111); ``materialize_logits=False`` selects the fused loss head.

``build_llama_model`` mirrors llama.py:161-194 (construction on the meta
device).  At TP = 1 the reference's ``parallelize_model`` only swaps the
linears for wrappers that add identity single-rank all-reduces; this build keeps
plain nn.Linear (the fused path accepts either).

``init_llama_weights_`` reproduces the reference's random initialisation
(femtotron/scripts/train.py:213-219: ``to_empty``, N(0, std) for every
parameter in registration order, then a dtype cast that also casts buffers),
drawing from a CPU ``torch.Generator`` so the weights are identical on any
device, and re-deriving the rotary ``inv_freq`` buffer that ``to_empty`` leaves
uninitialised (the reference's tests do the same,
femtotron/test/unit/test_pipeline_stage.py:200-221).
"""
from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import nn
from transformers import LlamaConfig

from .. import fused_loss
from .llama_partial_model import LlamaPartialModel


class LlamaForTraining(nn.Module):
    def __init__(self, model_config: LlamaConfig, parallel_ctx=None):
        super().__init__()
        self.config = model_config
        self.parallel_ctx = parallel_ctx
        self.model = LlamaPartialModel(model_config, parallel_ctx)
        self.lm_head = nn.Linear(model_config.hidden_size, model_config.vocab_size, bias=False)
        if model_config.tie_word_embeddings:
            self.tie_weights()
        self.model.config.use_cache = False

    def tie_weights(self):
        self.lm_head.weight = self.model.embed_tokens.weight

    def forward(self, input_ids: torch.Tensor, labels: torch.Tensor | None = None,
                materialize_logits: bool = True) -> dict:
        """materialize_logits=False (the flag of femtotron/model/base.py:15) asks
        for the loss only: with labels, on a HIP device, it is computed by the
        fused lm_head + chunked cross-entropy (femtotron_amd/fused_loss.py) and
        "logits" is None; otherwise the logits are materialised as the
        reference does."""
        hidden = self.model(input_ids)
        if (labels is not None and not materialize_logits and isinstance(self.lm_head, nn.Linear)
                and self.lm_head.bias is None and fused_loss.supported(hidden, self.lm_head.weight)):
            return {"logits": None,
                    "loss": fused_loss.fused_causal_lm_loss(hidden, self.lm_head.weight, labels)}
        logits = self.lm_head(hidden)
        out: dict = {"logits": logits}
        if labels is not None:
            shift_logits = logits[..., :-1, :].contiguous()
            shift_labels = labels[..., 1:].contiguous()
            out["loss"] = self._compute_loss(shift_logits, shift_labels)
        return out

    def _compute_loss(self, logits: torch.Tensor, labels: torch.Tensor) -> torch.Tensor:
        return F.cross_entropy(logits.float().view(-1, logits.size(-1)), labels.view(-1),
                               ignore_index=-100)

    @property
    def is_first(self) -> bool:
        return True

    @property
    def is_last(self) -> bool:
        return True

    @property
    def hidden_size(self) -> int:
        return self.config.hidden_size


def _check_single_gpu(parallel_ctx) -> None:
    if parallel_ctx is None:
        return
    get_size = getattr(parallel_ctx, "get_size", None)
    for dim in ("tp", "pp"):
        size = get_size(dim) if callable(get_size) else getattr(parallel_ctx, f"{dim}_size", 1)
        if size not in (None, 1):
            raise NotImplementedError(f"{dim} size {size}: this build runs TP = PP = 1 only")


def build_llama_model(model_config: LlamaConfig, parallel_ctx=None, *, use_pp_aware: bool = False,
                      layer_range: range | None = None) -> nn.Module:
    """Construct LlamaForTraining on the meta device (materialise with init_llama_weights_)."""
    if use_pp_aware or layer_range is not None:
        raise NotImplementedError("pipeline-parallel model variants are out of scope (PP = 1)")
    _check_single_gpu(parallel_ctx)
    with torch.device("meta"):
        model = LlamaForTraining(model_config, parallel_ctx)
    return model


def reset_rotary_inv_freq_(model: nn.Module) -> None:
    """Recompute every LlamaRotaryEmbedding's inv_freq buffer from its config."""
    for m in model.modules():
        if type(m).__name__ == "LlamaRotaryEmbedding":
            inv, scaling = m.compute_default_rope_parameters(m.config)
            m.inv_freq = inv.to(device=m.inv_freq.device, dtype=torch.float32)
            m.original_inv_freq = m.inv_freq.clone()
            m.attention_scaling = scaling


def init_llama_weights_(model: nn.Module, *, device: torch.device | str, dtype: torch.dtype,
                        std: float = 0.02, seed: int = 42, generator_device: str = "cpu") -> nn.Module:
    """Materialise ``model`` on ``device`` with every parameter ~ N(0, std) drawn
    in registration order, then cast to ``dtype``.

    generator_device="cpu" (default) draws from CPU Generator(seed): identical
    weights on every machine.  generator_device="cuda" draws on the device from a
    seeded device generator (fast for billion-parameter models; the values then
    depend on the device's random-number kernels)."""
    model = model.to_empty(device=device)
    gen = torch.Generator(device=generator_device).manual_seed(seed)
    with torch.no_grad():
        for p in model.parameters():
            if not p.requires_grad:
                continue
            if generator_device == "cpu":
                p.copy_(torch.empty(p.shape, dtype=torch.float32).normal_(0.0, std, generator=gen))
            else:
                p.normal_(0.0, std, generator=gen)
    reset_rotary_inv_freq_(model)
    return model.to(dtype)
