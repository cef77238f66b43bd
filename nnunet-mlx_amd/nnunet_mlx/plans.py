"""Minimal plans contract: configuration inheritance and the fields inference reads.

Reference: PlansContract / PlanConfiguration (src/nnunet_mlx/plans.py:154-372).  Only
what the inference path consumes is parsed here: the inheritance-resolved
configuration, its ``patch_size`` and ``architecture``.
"""

from __future__ import annotations

import json
from collections.abc import Mapping
from pathlib import Path

from nnunet_mlx.errors import ContractError


def read_json_object(path: str | Path) -> dict[str, object]:
    file = Path(path)
    if not file.is_file():
        raise ContractError(f"required file does not exist: {file}")
    try:
        payload = json.loads(file.read_text(encoding="utf-8"))
    except (UnicodeDecodeError, json.JSONDecodeError) as error:
        raise ContractError(f"{file.name} is invalid JSON") from error
    if not isinstance(payload, dict):
        raise ContractError(f"{file.name} must contain a JSON object")
    return payload


def resolve_configuration(plans: Mapping[str, object], configuration: str) -> dict[str, object]:
    """Follow ``inherits_from`` (child keys win) and return the resolved mapping."""
    configurations = plans.get("configurations")
    if not isinstance(configurations, Mapping) or configuration not in configurations:
        raise ContractError(f"nnU-Net plans lack configuration {configuration!r}")
    chain: list[str] = []
    name: str | None = configuration
    while name is not None:
        if name in chain:
            raise ContractError("plans configuration inheritance is cyclic")
        if name not in configurations:
            raise ContractError(f"nnU-Net plans lack configuration {name!r}")
        chain.append(name)
        raw = configurations[name]
        if not isinstance(raw, Mapping):
            raise ContractError(f"configuration {name!r} must be a mapping")
        parent = raw.get("inherits_from")
        name = parent if isinstance(parent, str) else None
    resolved: dict[str, object] = {}
    for item in reversed(chain):
        resolved.update({k: v for k, v in configurations[item].items() if k != "inherits_from"})
    return resolved


def topology_payload(plans: Mapping[str, object], configuration: str) -> dict[str, object]:
    """Plans whose ``configurations`` hold only the resolved configuration."""
    return {**plans, "configurations": {configuration: resolve_configuration(plans, configuration)}}


def patch_size(plans: Mapping[str, object], configuration: str) -> tuple[int, ...]:
    raw = resolve_configuration(plans, configuration).get("patch_size")
    if not isinstance(raw, list) or not all(isinstance(v, int) and not isinstance(v, bool) and v > 0 for v in raw):
        raise ContractError("plans patch_size must be a list of positive integers")
    return tuple(raw)
