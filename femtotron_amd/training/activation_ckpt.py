"""Activation-checkpoint wrapper and in-place apply/remove utilities.

Public API and behaviour follow femtotron/training/activation_ckpt.py:
  * ``ActivationCheckpointWrapper(module, *, checkpoint_fn, use_reentrant,
    preserve_rng_state)`` registers the wrapped module under the child name
    ``_checkpoint_wrapped_module`` (:30,63) and forwards every call as
    ``checkpoint_fn(inner, *args, use_reentrant=..., preserve_rng_state=...,
    debug=True, **kwargs)`` (:78-86);
  * state-dict keys never show the wrapper: its prefix is stripped on save and
    re-inserted on load (:201-236);
  * ``apply_activation_checkpointing`` (:92-132) first collects every
    (parent, name, child) the policy selects, then swaps them, and returns the
    count; a selected module that already contains a wrapper raises ValueError
    (:183-194); children that are wrappers themselves are skipped;
  * ``remove_activation_checkpointing`` (:135-153) restores the inner modules and
    returns how many it unwrapped; ``is_activation_checkpointed`` (:156-158).

The MI355X hot path plugs in through ``checkpoint_fn``: pass
``femtotron_amd.fused_checkpoint`` to route Llama decoder layers to the fused
HIP implementation.  The default stays ``torch.utils.checkpoint.checkpoint``.
"""
from __future__ import annotations

from typing import Any, Callable, Final

from torch import nn
from torch.utils.checkpoint import checkpoint as _torch_checkpoint

CheckpointPolicy = Callable[[nn.Module], bool]
CheckpointFn = Callable[..., Any]

_WRAPPED_MODULE_KEY: Final[str] = "_checkpoint_wrapped_module"
_WRAPPED_MODULE_PREFIX: Final[str] = _WRAPPED_MODULE_KEY + "."


class ActivationCheckpointWrapper(nn.Module):
    """Runs the wrapped module through ``checkpoint_fn`` on every forward.

    Parameters and buffers stay owned by the inner module, so
    ``model.parameters()`` yields the same tensor objects before and after
    wrapping, and ``state_dict()`` keys are unchanged."""

    def __init__(self, module: nn.Module, *, checkpoint_fn: CheckpointFn = _torch_checkpoint,
                 use_reentrant: bool = False, preserve_rng_state: bool = False) -> None:
        super().__init__()
        self.add_module(_WRAPPED_MODULE_KEY, module)
        self.checkpoint_fn = checkpoint_fn
        self.use_reentrant = use_reentrant
        self.preserve_rng_state = preserve_rng_state
        self._register_state_dict_hook(_strip_prefix_on_save)
        # The public registration passes the module first, which is the hook's
        # signature.  (The reference registers the same module-first hook through
        # the private _register_load_state_dict_pre_hook without with_module=True,
        # so torch calls it one argument short and load_state_dict on a wrapped
        # model raises TypeError; the save-side prefix stripping is unaffected.)
        self.register_load_state_dict_pre_hook(_add_prefix_on_load)

    @property
    def inner_module(self) -> nn.Module:
        return self._modules[_WRAPPED_MODULE_KEY]

    def forward(self, *args: Any, **kwargs: Any) -> Any:
        return self.checkpoint_fn(self.inner_module, *args, use_reentrant=self.use_reentrant,
                                  preserve_rng_state=self.preserve_rng_state, debug=True,
                                  **kwargs)

    def extra_repr(self) -> str:
        return f"use_reentrant={self.use_reentrant}, preserve_rng_state={self.preserve_rng_state}"


def apply_activation_checkpointing(model: nn.Module, policy: CheckpointPolicy, *,
                                   checkpoint_fn: CheckpointFn = _torch_checkpoint,
                                   use_reentrant: bool = False,
                                   preserve_rng_state: bool = False) -> int:
    """Wrap, in place, every module of ``model`` that ``policy`` selects.

    Returns the number of modules wrapped.  Raises ValueError if a selected
    module already contains an ActivationCheckpointWrapper (nested checkpointing
    would recompute the inner region twice)."""
    chosen = _select(model, policy)
    for parent, name, child in chosen:
        setattr(parent, name, ActivationCheckpointWrapper(
            child, checkpoint_fn=checkpoint_fn, use_reentrant=use_reentrant,
            preserve_rng_state=preserve_rng_state))
    return len(chosen)


def remove_activation_checkpointing(model: nn.Module) -> int:
    """Undo every wrapper in ``model``; returns how many were removed (0 if none)."""
    found = [(parent, name, child) for parent in model.modules()
             for name, child in parent.named_children()
             if isinstance(child, ActivationCheckpointWrapper)]
    for parent, name, wrapper in found:
        setattr(parent, name, wrapper.inner_module)
    return len(found)


def is_activation_checkpointed(module: nn.Module) -> bool:
    return isinstance(module, ActivationCheckpointWrapper)


def _select(model: nn.Module, policy: CheckpointPolicy) -> list[tuple[nn.Module, str, nn.Module]]:
    # Collect first, mutate afterwards: replacing children while iterating
    # model.modules() would change the traversal.
    chosen: list[tuple[nn.Module, str, nn.Module]] = []
    for parent in model.modules():
        for name, child in parent.named_children():
            if isinstance(child, ActivationCheckpointWrapper) or not policy(child):
                continue
            nested = next((m for m in child.modules()
                           if m is not child and isinstance(m, ActivationCheckpointWrapper)), None)
            if nested is not None:
                raise ValueError(
                    f"Cannot wrap {type(child).__name__!r} for activation checkpointing: it "
                    f"contains a nested ActivationCheckpointWrapper around "
                    f"{type(nested.inner_module).__name__!r}. Nested checkpointing causes "
                    f"redundant recompute and is not supported.")
            chosen.append((parent, name, child))
    return chosen


def _strip_prefix_on_save(module: nn.Module, state_dict: dict[str, Any], prefix: str,
                          local_metadata: dict[str, Any]) -> None:
    inner = prefix + _WRAPPED_MODULE_PREFIX
    for key in [k for k in state_dict if k.startswith(inner)]:
        state_dict[prefix + key[len(inner):]] = state_dict.pop(key)


def _add_prefix_on_load(module: nn.Module, state_dict: dict[str, Any], prefix: str,
                        local_metadata: dict[str, Any], strict: bool, missing_keys: list[str],
                        unexpected_keys: list[str], error_msgs: list[str]) -> None:
    inner = prefix + _WRAPPED_MODULE_PREFIX
    for key in [k for k in state_dict if k.startswith(prefix) and not k.startswith(inner)]:
        state_dict[inner + key[len(prefix):]] = state_dict.pop(key)
