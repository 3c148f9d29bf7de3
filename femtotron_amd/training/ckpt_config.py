"""Build a checkpoint policy from a YAML/JSON-style dict.

Schema and errors as femtotron/training/ckpt_config.py:23-65:
    None                                   -> NEVER
    {"type": "never"} / {"type": "always"}
    {"type": "by_class_name", "names": [str, ...]}
    {"type": "any_of" | "all_of", "policies": [<config>, ...]}
    {"type": "not_of", "policy": <config>}
Class objects are not serialisable, so ``by_class`` has no config form.
"""
from __future__ import annotations

from typing import Any

from .activation_ckpt import CheckpointPolicy
from .ckpt_policy import ALWAYS, NEVER, all_of, any_of, by_class_name, not_of


def policy_from_config(config: dict[str, Any] | None) -> CheckpointPolicy:
    if config is None:
        return NEVER
    kind = config.get("type")
    if kind == "never":
        return NEVER
    if kind == "always":
        return ALWAYS
    if kind == "by_class_name":
        names = config["names"]
        if not isinstance(names, list) or not all(isinstance(n, str) for n in names):
            raise ValueError(f"by_class_name expects 'names' to be a list of strings, got {names!r}")
        return by_class_name(*names)
    if kind in ("any_of", "all_of"):
        subs = [policy_from_config(c) for c in config["policies"]]
        return any_of(*subs) if kind == "any_of" else all_of(*subs)
    if kind == "not_of":
        return not_of(policy_from_config(config["policy"]))
    raise ValueError(f"Unknown policy type {kind!r}. "
                     f"Valid types: never, always, by_class_name, any_of, all_of, not_of.")
