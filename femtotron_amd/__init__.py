"""femtotron_amd — MI355X-native activation-checkpointed Llama decoder layer.

Drop-in for Femtotron's checkpointed decoder-layer path: build the model with
``femtotron_amd.model`` (Hugging Face LlamaDecoderLayer modules, Femtotron's
LlamaPartialModel/LlamaForTraining API) and wrap it with
``femtotron_amd.training.apply_activation_checkpointing(model, policy,
checkpoint_fn=femtotron_amd.fused_checkpoint)``.  Decoder-layer calls on a HIP
device then run on the hand-written gfx950 kernels of ``libfemtohip.so``.
"""
from .fused_checkpoint import (dispatch_counts, fused_checkpoint, last_fallback_reason,
                               reset_dispatch_counts)
from .boundary_ops import fuse_boundary_ops
from .fused_attention import fuse_attention
from .weight_packing import pack_layer_weights

__all__ = ["fused_checkpoint", "dispatch_counts", "reset_dispatch_counts", "last_fallback_reason",
           "pack_layer_weights", "fuse_boundary_ops", "fuse_attention"]
