"""Minimal plans contract: configuration inheritance and the fields inference reads.

Reference: PlansContract / PlanConfiguration (src/nnunet_mlx/plans.py:154-372).  Only
what the inference path consumes is parsed here: the inheritance-resolved
configuration, its ``patch_size`` and ``architecture``, and the resampling contract
that restoration reads.
"""

from __future__ import annotations

import json
from collections.abc import Mapping
from dataclasses import dataclass
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


# ---- resampling contract ------------------------------------------------------------
# Reference: ResamplingContract (src/nnunet_mlx/plans.py:31-160).  The fields the
# restoration policy reads; the parser accepts the two upstream resampling functions and
# keeps nnU-Net 2.8.1's defaults for omitted spline options (order 3, order_z 0,
# force_separate_z False, anisotropy threshold 3; the Torch resampler: order 1, order_z 0,
# force_separate_z None, mode "linear", aniso_axis_mode "nearest-exact", seg_tiebreak
# "nearest").


RESAMPLING_FUNCTIONS = ("resample_data_or_seg_to_shape", "resample_torch_fornnunet")
INTERPOLATION_MODES = ("linear", "nearest", "nearest-exact")
SEG_TIEBREAKS = ("nearest", "lowest", "highest")
TORCH_RESAMPLING_KWARGS = frozenset({
    "is_seg", "force_separate_z", "seg_tiebreak", "mode", "aniso_axis_mode",
    "separate_z_anisotropy_threshold", "num_threads", "device", "memefficient_seg_resampling"})
SPLINE_RESAMPLING_KWARGS = frozenset({
    "is_seg", "order", "order_z", "force_separate_z", "seg_tiebreak",
    "separate_z_anisotropy_threshold"})


@dataclass(frozen=True)
class ResamplingContract:
    """One upstream ``resampling_fn_*`` plan entry (the fields restoration reads)."""

    function_name: str
    order: int
    order_z: int
    force_separate_z: bool | None
    separate_z_anisotropy_threshold: float = 3.0
    mode: str = "linear"                    # Torch resampler: in-plane (or only) pass
    aniso_axis_mode: str = "nearest-exact"  # Torch resampler: the separate axis's pass
    seg_tiebreak: str | None = None

    @classmethod
    def from_configuration(cls, configuration: Mapping[str, object], *, field: str,
                           expected_is_seg: bool) -> "ResamplingContract":
        """Parse ``configuration[field]`` and ``<field>_kwargs``
        (src/nnunet_mlx/plans.py:60-160); raises ContractError on unsupported entries."""
        name = configuration.get(field)
        if name not in RESAMPLING_FUNCTIONS:
            raise ContractError(f"unsupported nnU-Net resampling function {name!r}")
        kwargs = configuration.get(f"{field}_kwargs", {})
        if not isinstance(kwargs, Mapping):
            raise ContractError(f"{field}_kwargs must be a mapping")
        torch_resampling = name == "resample_torch_fornnunet"
        is_seg = kwargs.get("is_seg", False)
        if not isinstance(is_seg, bool) or is_seg is not expected_is_seg:
            raise ContractError(f"{field}.is_seg does not match its runtime role")
        force = kwargs.get("force_separate_z", None if torch_resampling else False)
        if force is not None and not isinstance(force, bool):
            raise ContractError(f"{field}.force_separate_z must be boolean or null")
        threshold = kwargs.get("separate_z_anisotropy_threshold", 3.0)
        if isinstance(threshold, bool) or not isinstance(threshold, (int, float)) or threshold <= 0:
            raise ContractError(f"{field}.separate_z_anisotropy_threshold must be positive")
        tiebreak = kwargs.get("seg_tiebreak")
        if "seg_tiebreak" in kwargs and tiebreak not in SEG_TIEBREAKS:
            raise ContractError(f"{field}.seg_tiebreak must be 'nearest', 'lowest', or 'highest'")
        unknown = set(kwargs) - (TORCH_RESAMPLING_KWARGS if torch_resampling
                                 else SPLINE_RESAMPLING_KWARGS)
        if unknown:
            kind = "resample_torch_fornnunet" if torch_resampling else "spline"
            raise ContractError(f"{field}: unsupported {kind} kwargs: {', '.join(sorted(unknown))}")
        if torch_resampling:
            threads = kwargs.get("num_threads", 4)
            if isinstance(threads, bool) or not isinstance(threads, int) or threads <= 0:
                raise ContractError(f"{field}.num_threads must be a positive integer")
            if not isinstance(kwargs.get("memefficient_seg_resampling", True), bool):
                raise ContractError(f"{field}.memefficient_seg_resampling must be boolean")
            if kwargs.get("device", "cpu") != "cpu":
                raise ContractError(f"{field}.device supports only 'cpu' host resampling")
            modes = {}
            for key, default in (("mode", "linear"), ("aniso_axis_mode", "nearest-exact")):
                modes[key] = kwargs.get(key, default)
                if modes[key] not in INTERPOLATION_MODES:
                    raise ContractError(
                        f"{field}.{key} must be 'linear', 'nearest', or 'nearest-exact'")
            return cls(name, 1, 0, force, float(threshold), mode=modes["mode"],
                       aniso_axis_mode=modes["aniso_axis_mode"],
                       seg_tiebreak=tiebreak or "nearest")
        order, order_z = kwargs.get("order", 3), kwargs.get("order_z", 0)
        for label, value in (("order", order), ("order_z", order_z)):
            if isinstance(value, bool) or not isinstance(value, int) or not 0 <= value <= 5:
                raise ContractError(f"{field}.{label} must be an integer in [0, 5]")
        return cls(name, order, order_z, force, float(threshold), seg_tiebreak=tiebreak)
