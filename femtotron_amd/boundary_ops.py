"""Fused ops on either side of the decoder-layer stack: the token embedding and
the final RMSNorm.

Reference (femtotron/model/llama_partial_model.py:181-184, 217-218): the first
stage embeds the token ids with ``embed_tokens`` (an ``nn.Embedding``, which
femtotron's TP plan swaps for ``VocabParallelEmbedding``,
femtotron/parallel/tensor_parallel/embedding.py:57-79), the last stage applies
the final ``LlamaRMSNorm``.  ``fuse_boundary_ops(model)`` swaps the two modules
for ``FusedEmbedding`` / ``FusedRMSNorm`` holding the *same* ``Parameter``
objects (state-dict keys and weight tying unchanged):

* ``FusedEmbedding`` — forward ``fh_embedding_fwd`` (row gather; ids outside
  [0, vocab) give zero rows, as VocabParallelEmbedding at one rank does),
  backward ``fh_embedding_bwd`` (deterministic scatter-add: stable radix sort
  of the ids, fp32 sums in token order, no floating-point atomics; skips
  nn.Embedding's ``padding_idx``).
* ``FusedRMSNorm`` — the same ``fh_rmsnorm_fwd`` / ``fh_rmsnorm_bwd`` kernels
  the checkpointed layers use, saving only the input.

Off a HIP device (or in a dtype the kernels do not take) both modules compute
what the modules they replace compute.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import nn

from . import ops
from .fused_parts import FusedRMSNormFunction

_DTYPES = (torch.bfloat16, torch.float32)


class FusedEmbeddingFunction(torch.autograd.Function):
    """out = weight[ids] (zero rows for ids outside [0, vocab)); saved: ids."""

    @staticmethod
    def forward(ctx, ids, weight, padding_idx):
        ctx.save_for_backward(ids)
        ctx.vocab = weight.shape[0]
        ctx.padding_idx = padding_idx
        return ops.embedding_fwd(ids, weight)

    @staticmethod
    def backward(ctx, dy):
        (ids,) = ctx.saved_tensors
        dw = None
        if ctx.needs_input_grad[1]:
            dw = ops.embedding_bwd(dy.contiguous(), ids, ctx.vocab, ctx.padding_idx)
        return None, dw, None


class FusedEmbedding(nn.Module):
    """Token embedding on the fused kernels; ``weight`` is the replaced module's Parameter."""

    def __init__(self, weight: nn.Parameter, padding_idx: int | None = None):
        super().__init__()
        self.weight = weight
        self.num_embeddings, self.embedding_dim = weight.shape
        self.padding_idx = padding_idx

    @classmethod
    def from_module(cls, emb: nn.Module) -> "FusedEmbedding":
        return cls(emb.weight, getattr(emb, "padding_idx", None))

    def _fused(self, ids: torch.Tensor) -> bool:
        w = self.weight
        return (w.is_cuda and ids.device == w.device and w.dtype in _DTYPES and w.is_contiguous()
                and self.embedding_dim % 8 == 0 and w.data_ptr() % 16 == 0
                and ids.dtype == torch.int64)

    def forward(self, ids: torch.Tensor) -> torch.Tensor:
        if self._fused(ids):
            return FusedEmbeddingFunction.apply(ids.contiguous(), self.weight, self.padding_idx)
        # the replaced module's computation (VocabParallelEmbedding at one rank)
        mask = (ids < 0) | (ids >= self.num_embeddings)
        out = F.embedding(ids.masked_fill(mask, 0), self.weight, self.padding_idx)
        return out.masked_fill(mask.unsqueeze(-1), 0)

    def extra_repr(self) -> str:
        return f"{self.num_embeddings}, {self.embedding_dim}, padding_idx={self.padding_idx}"


class FusedRMSNorm(nn.Module):
    """LlamaRMSNorm on the fused kernels; ``weight`` is the replaced module's Parameter."""

    def __init__(self, weight: nn.Parameter, eps: float):
        super().__init__()
        self.weight = weight
        self.variance_epsilon = float(eps)

    @classmethod
    def from_module(cls, norm: nn.Module) -> "FusedRMSNorm":
        return cls(norm.weight, norm.variance_epsilon)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        w = self.weight
        if (x.is_cuda and w.is_cuda and x.dtype in _DTYPES and w.dtype == x.dtype
                and w.is_contiguous() and not torch.is_autocast_enabled()):
            return FusedRMSNormFunction.apply(x.contiguous(), w, self.variance_epsilon)
        # Hugging Face LlamaRMSNorm (transformers models/llama/modeling_llama.py)
        dt = x.dtype
        h = x.to(torch.float32)
        h = h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + self.variance_epsilon)
        return w * h.to(dt)

    def extra_repr(self) -> str:
        return f"{tuple(self.weight.shape)}, eps={self.variance_epsilon}"


def fuse_boundary_ops(model: nn.Module) -> int:
    """Swap every layer-stack owner's ``embed_tokens`` (nn.Embedding) and final
    ``norm`` (LlamaRMSNorm) for the fused modules, keeping their Parameters.
    Embeddings with max_norm, sparse gradients or scale_grad_by_freq are left
    alone, and so is a norm already wrapped for activation checkpointing (the
    checkpoint path fuses it).  Returns the number of modules swapped."""
    from transformers.models.llama.modeling_llama import LlamaRMSNorm
    n = 0
    for owner in list(model.modules()):
        emb = getattr(owner, "embed_tokens", None)
        if type(emb) is nn.Embedding and emb.max_norm is None and not emb.sparse \
                and not emb.scale_grad_by_freq:
            owner.embed_tokens = FusedEmbedding.from_module(emb)
            n += 1
        norm = getattr(owner, "norm", None)
        if type(norm) is LlamaRMSNorm:
            owner.norm = FusedRMSNorm.from_module(norm)
            n += 1
    return n


def unfuse_boundary_ops(model: nn.Module) -> int:
    """Undo ``fuse_boundary_ops``: put nn.Embedding / LlamaRMSNorm modules back,
    holding the same Parameters.  Returns the number of modules swapped."""
    from transformers.models.llama.modeling_llama import LlamaRMSNorm
    n = 0
    for owner in list(model.modules()):
        emb = getattr(owner, "embed_tokens", None)
        if isinstance(emb, FusedEmbedding):
            new = nn.Embedding(emb.num_embeddings, emb.embedding_dim, padding_idx=emb.padding_idx,
                               device="meta")
            new.weight = emb.weight
            owner.embed_tokens = new
            n += 1
        norm = getattr(owner, "norm", None)
        if isinstance(norm, FusedRMSNorm):
            new = LlamaRMSNorm(norm.weight.shape[0], eps=norm.variance_epsilon)
            new.weight = norm.weight
            owner.norm = new
            n += 1
    return n
