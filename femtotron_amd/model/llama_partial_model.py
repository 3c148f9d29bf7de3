"""LlamaPartialModel: the layer-stack owner that calls the checkpointed layers.

Same constructor, parameter names and forward as
femtotron/model/llama_partial_model.py:72-220 (embed_tokens on the first stage,
``layers`` as a ModuleDict keyed by the global layer index, one
``LlamaRotaryEmbedding``, final ``norm`` on the last stage).  The decoder layers
are the Hugging Face ``LlamaDecoderLayer`` objects themselves, so the
``llama_decoder_layer`` checkpoint policy and any checkpoint_fn see exactly the
module the reference hands them.

``parallel_ctx`` is optional here: this build is single-GPU (TP = PP = 1).
"""
from __future__ import annotations

import torch
import torch.nn as nn
from transformers import LlamaConfig
from transformers.models.llama.modeling_llama import (LlamaDecoderLayer, LlamaRMSNorm,
                                                      LlamaRotaryEmbedding)


class LlamaPartialModel(nn.Module):
    def __init__(self, model_config: LlamaConfig, parallel_ctx=None,
                 layer_range: range | None = None, is_first: bool | None = None,
                 is_last: bool | None = None):
        super().__init__()
        n_layers = model_config.num_hidden_layers
        if layer_range is None:
            layer_range = range(n_layers)
        if not isinstance(layer_range, range):
            raise ValueError(f"layer_range must be a range, got {type(layer_range).__name__}")
        if layer_range.start < 0 or layer_range.stop > n_layers:
            raise ValueError(f"layer_range {layer_range} out of bounds for {n_layers} layers")
        if layer_range.step != 1:
            raise ValueError(f"layer_range must be contiguous (step=1), got step={layer_range.step}")
        if is_first is None:
            is_first = layer_range.start == 0
        if is_last is None:
            is_last = layer_range.stop == n_layers
        # Not a PreTrainedModel, so pick the attention implementation the way
        # the reference does (llama_partial_model.py:118-123): sdpa by default.
        if getattr(model_config, "_attn_implementation", None) is None:
            model_config._attn_implementation = (
                getattr(model_config, "attn_implementation", None) or "sdpa")

        self.config = model_config
        self.parallel_ctx = parallel_ctx
        self.layer_range = layer_range
        self.is_first = is_first
        self.is_last = is_last
        if is_first:
            self.embed_tokens = nn.Embedding(model_config.vocab_size, model_config.hidden_size,
                                             padding_idx=model_config.pad_token_id)
        self.layers = nn.ModuleDict(
            {str(i): LlamaDecoderLayer(model_config, layer_idx=i) for i in layer_range})
        self.rotary_emb = LlamaRotaryEmbedding(config=model_config)
        if is_last:
            self.norm = LlamaRMSNorm(model_config.hidden_size, eps=model_config.rms_norm_eps)

    def forward(self, x: torch.Tensor, attention_mask: torch.Tensor | None = None,
                position_ids: torch.Tensor | None = None) -> torch.Tensor:
        hidden = self.embed_tokens(x) if self.is_first else x
        _, seqlen, _ = hidden.shape
        if position_ids is None:
            position_ids = torch.arange(seqlen, device=hidden.device, dtype=torch.long).unsqueeze(0)
        from transformers.masking_utils import create_causal_mask
        causal_mask = create_causal_mask(config=self.config, inputs_embeds=hidden,
                                         attention_mask=attention_mask, past_key_values=None,
                                         position_ids=position_ids)
        position_embeddings = self.rotary_emb(hidden, position_ids=position_ids)
        for layer in self.layers.values():
            hidden = layer(hidden, attention_mask=causal_mask,
                           position_embeddings=position_embeddings, position_ids=position_ids,
                           past_key_values=None, use_cache=False)
        if self.is_last:
            hidden = self.norm(hidden)
        return hidden
