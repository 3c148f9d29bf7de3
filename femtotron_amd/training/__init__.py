"""Activation-checkpointing API (mirror of femtotron.training's AC modules)."""
from .activation_ckpt import (ActivationCheckpointWrapper, CheckpointFn, CheckpointPolicy,
                              apply_activation_checkpointing, is_activation_checkpointed,
                              remove_activation_checkpointing)
from .ckpt_config import policy_from_config
from .ckpt_policy import ALWAYS, NEVER, all_of, always, any_of, by_class, by_class_name, never, not_of

__all__ = [
    "ActivationCheckpointWrapper", "CheckpointFn", "CheckpointPolicy",
    "apply_activation_checkpointing", "is_activation_checkpointed",
    "remove_activation_checkpointing", "policy_from_config", "ALWAYS", "NEVER", "all_of",
    "always", "any_of", "by_class", "by_class_name", "never", "not_of",
]
