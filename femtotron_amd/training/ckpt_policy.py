"""Module-selection policies for activation checkpointing.

Same factories, combinators, names and errors as
femtotron/training/ckpt_policy.py: ``by_class`` (:25-41), ``by_class_name``
(:44-63), ``any_of`` (:70-87), ``all_of`` (:90-111), ``not_of`` (:114-124),
``never``/``always`` and the ``NEVER``/``ALWAYS`` constants (:131-142).  Each
policy is a ``Callable[[nn.Module], bool]`` carrying a readable ``__name__``.
"""
from __future__ import annotations

from typing import Final

from torch import nn

from .activation_ckpt import CheckpointPolicy


def _named(fn: CheckpointPolicy, name: str) -> CheckpointPolicy:
    fn.__name__ = name
    return fn


def _name(policy: CheckpointPolicy) -> str:
    return getattr(policy, "__name__", "<unnamed>")


def by_class(*classes: type[nn.Module]) -> CheckpointPolicy:
    """Select instances of any of ``classes``."""
    if not classes:
        raise ValueError("by_class() requires at least one class")
    frozen = tuple(classes)
    return _named(lambda m: isinstance(m, frozen),
                  f"by_class({', '.join(c.__name__ for c in frozen)})")


def by_class_name(*names: str) -> CheckpointPolicy:
    """Select modules whose ``type(m).__name__`` is one of ``names``."""
    if not names:
        raise ValueError("by_class_name() requires at least one name")
    wanted = frozenset(names)
    return _named(lambda m: type(m).__name__ in wanted,
                  f"by_class_name({', '.join(repr(n) for n in names)})")


def any_of(*policies: CheckpointPolicy) -> CheckpointPolicy:
    """Logical OR; a single policy is returned unchanged."""
    if not policies:
        raise ValueError("any_of() requires at least one policy")
    if len(policies) == 1:
        return policies[0]
    ps = tuple(policies)
    return _named(lambda m: any(p(m) for p in ps), f"any_of({', '.join(_name(p) for p in ps)})")


def all_of(*policies: CheckpointPolicy) -> CheckpointPolicy:
    """Logical AND; a single policy is returned unchanged."""
    if not policies:
        raise ValueError("all_of() requires at least one policy")
    if len(policies) == 1:
        return policies[0]
    ps = tuple(policies)
    return _named(lambda m: all(p(m) for p in ps), f"all_of({', '.join(_name(p) for p in ps)})")


def not_of(policy: CheckpointPolicy) -> CheckpointPolicy:
    """Logical NOT."""
    return _named(lambda m: not policy(m), f"not_of({_name(policy)})")


def never(module: nn.Module) -> bool:
    """Selects nothing (checkpointing disabled)."""
    return False


def always(module: nn.Module) -> bool:
    """Selects everything (will hit the nested-wrap error on real models)."""
    return True


NEVER: Final[CheckpointPolicy] = never
ALWAYS: Final[CheckpointPolicy] = always
