"""String presets for activation-checkpoint (and ZeRO-3 wrap) policies.

Mirrors femtotron/scripts/presets.py:19-62: YAML configs name a policy by
string; ``get_ac_policy``/``get_wrap_policy`` resolve it and raise ValueError
listing the known names for anything else.

Added here (no counterpart in the reference): ``"llama_mlp_and_norms"``, the
selective policy that checkpoints only the RMSNorms and the MLP and keeps
attention activations (used to compare full vs. selective activation bytes).
"""
from __future__ import annotations

from typing import Callable

import torch.nn as nn

from ..training.ckpt_policy import any_of, by_class, by_class_name


def _llama_decoder_layer_cls():
    from transformers.models.llama.modeling_llama import LlamaDecoderLayer
    return LlamaDecoderLayer


def _wrap_llama_decoder_layer() -> Callable[[nn.Module], bool]:
    cls = _llama_decoder_layer_cls()

    def policy(m: nn.Module) -> bool:
        return isinstance(m, cls)

    policy.__name__ = "wrap_llama_decoder_layer"
    return policy


WRAP_POLICY_PRESETS: dict[str, Callable[[], Callable[[nn.Module], bool]]] = {
    "llama_decoder_layer": _wrap_llama_decoder_layer,
}

AC_POLICY_PRESETS: dict[str, Callable[[], Callable[[nn.Module], bool]]] = {
    "llama_decoder_layer": lambda: by_class(_llama_decoder_layer_cls()),
    "llama_mlp_and_norms": lambda: any_of(by_class_name("LlamaMLP"), by_class_name("LlamaRMSNorm")),
}


def _resolve(kind: str, table: dict, name: str):
    if name not in table:
        raise ValueError(f"Unknown {kind} preset {name!r}. Available: {list(table)}")
    return table[name]()


def get_wrap_policy(name: str) -> Callable[[nn.Module], bool]:
    return _resolve("wrap_policy", WRAP_POLICY_PRESETS, name)


def get_ac_policy(name: str) -> Callable[[nn.Module], bool]:
    return _resolve("ac_policy", AC_POLICY_PRESETS, name)
