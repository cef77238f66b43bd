"""Resampling policy shared by restoration (the host-side rules, no interpolation).

Reference: src/nnunet_mlx/data/resampling.py:587-622 (``separate_z_axis``,
``validate_spacing``).
"""

from __future__ import annotations

import math
from collections.abc import Sequence

from nnunet_mlx.errors import ContractError

ANISOTROPY_THRESHOLD = 3.0


def validate_spacing(value: Sequence[float], *, name: str) -> tuple[float, float, float]:
    """Require three finite, positive numeric spacings, rejecting booleans
    (src/nnunet_mlx/data/resampling.py:617-622)."""
    result = []
    for item in value:
        if isinstance(item, bool) or not isinstance(item, (int, float)) or not math.isfinite(item):
            raise ContractError(f"{name} must contain finite numbers")
        result.append(float(item))
    if len(result) != 3 or any(item <= 0 for item in result):
        raise ContractError(f"{name} must contain three positive values")
    return tuple(result)  # type: ignore[return-value]


def separate_z_axis(current_spacing: tuple[float, float, float],
                    new_spacing: tuple[float, float, float], *, force: bool | None,
                    threshold: float = ANISOTROPY_THRESHOLD) -> tuple[bool, int | None]:
    """Choose a unique coarsest axis for separate resampling, if the policy permits it
    (src/nnunet_mlx/data/resampling.py:587-614).

    With ``force=None`` a max/min spacing ratio above ``threshold`` enables separation,
    using the current spacing when it is anisotropic and otherwise the target spacing; a
    forced true uses the current spacing; false disables separation.  A tie for the
    coarsest axis disables it.
    """
    if force is None:
        current_anisotropic = max(current_spacing) / min(current_spacing) > threshold
        separate = current_anisotropic or max(new_spacing) / min(new_spacing) > threshold
        basis = current_spacing if current_anisotropic else new_spacing
    else:
        separate = force
        basis = current_spacing
    if not separate:
        return False, None
    maximum = max(basis)
    axes = tuple(index for index, spacing in enumerate(basis) if maximum / spacing == 1)
    if len(axes) != 1:
        return False, None
    return True, axes[0]
