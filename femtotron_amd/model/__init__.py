"""Llama model modules (mirror of femtotron.model's LlamaPartialModel/LlamaForTraining)."""
from .llama import (LlamaForTraining, build_llama_model, init_llama_weights_,
                    reset_rotary_inv_freq_)
from .llama_partial_model import LlamaPartialModel

__all__ = ["LlamaForTraining", "LlamaPartialModel", "build_llama_model", "init_llama_weights_",
           "reset_rotary_inv_freq_"]
