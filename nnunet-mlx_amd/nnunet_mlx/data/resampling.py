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


# ---- Torch-grid resampling on the GPU ------------------------------------------------
# Reference: torch_resize / resample_torch (src/nnunet_mlx/kernels/metal_torch_resample.py:
# 146-215), the device form of upstream nnU-Net's resample_torch_fornnunet.  Images and
# probabilities only (is_seg false): float32 coordinates, float64 corner sums rounded
# once to float32 (``nnx_torch_resize``).

TORCH_MODES = {"linear": 0, "nearest": 1, "nearest-exact": 2}


def _torch_mode(mode: str) -> int:
    if mode not in TORCH_MODES:
        raise ContractError("Torch-grid mode must be 'linear', 'nearest', or 'nearest-exact'")
    return TORCH_MODES[mode]


def _check_torch_grid_input(values, shape, *, name: str) -> tuple[int, int, int]:
    import torch

    target = tuple(int(s) for s in shape)
    if (not isinstance(values, torch.Tensor) or values.dim() != 4 or len(target) != 3
            or values.dtype not in (torch.float32, torch.float16) or values.device.type != "cuda"):
        raise ContractError(f"{name} requires a (C, X, Y, Z) float32/float16 GPU tensor and "
                            "a three-axis target shape")
    if min(*values.shape, *target) < 1:
        raise ContractError(f"{name} requires positive dimensions")
    return target  # type: ignore[return-value]


def torch_resize_device(values, shape, mode: str, *, channels_last: bool = False):
    """One Torch-grid pass of (C, X, Y, Z) ``values`` (float32 or float16, any strides, on
    the GPU) to spatial ``shape``; returns float32 (C, *shape), stored channels-last (a
    permuted view of (*shape, C) memory) when ``channels_last``.  Equal shapes return the
    values as float32, as the reference returns its input
    (src/nnunet_mlx/kernels/metal_torch_resample.py:146-192)."""
    import torch

    from nnunet_mlx import _native

    target = _check_torch_grid_input(values, shape, name="Torch-grid resampling")
    code = _torch_mode(mode)
    if tuple(values.shape[1:]) == target:
        return values.float()
    channels = int(values.shape[0])
    if channels_last:
        out = torch.empty((*target, channels), dtype=torch.float32,
                          device=values.device).permute(3, 0, 1, 2)
    else:
        out = torch.empty((channels, *target), dtype=torch.float32, device=values.device)
    lib = _native.load()
    _native.check(lib.nnx_torch_resize(
        values.data_ptr(), 1 if values.dtype == torch.float16 else 0, channels,
        _native.ints(values.shape[1:]), _native.i64s(values.stride()), out.data_ptr(),
        _native.ints(target), _native.i64s(out.stride()), code,
        _native.stream_handle(values.device)), "nnx_torch_resize")
    return out


def _plane_shape(source, target, axis: int) -> tuple[int, int, int]:
    """The in-plane pass's shape: the target's, with ``axis`` kept at its source size."""
    return tuple(int(source[a]) if a == axis else int(target[a]) for a in range(3))  # type: ignore[return-value]


def resample_torch_device(values, shape, *, axis: int | None, mode: str = "linear",
                          aniso_axis_mode: str = "nearest-exact", channels_last: bool = False):
    """The plans' Torch resampler on (C, X, Y, Z) GPU values: one pass with ``mode``, or,
    with a separate ``axis``, the planes across it with ``mode`` and then the axis with
    ``aniso_axis_mode`` (src/nnunet_mlx/kernels/metal_torch_resample.py:195-215)."""
    target = _check_torch_grid_input(values, shape, name="Torch-grid resampling")
    if axis is None:
        return torch_resize_device(values, target, mode, channels_last=channels_last)
    if axis not in (0, 1, 2):
        raise ContractError("Torch-grid separate axis must be 0, 1 or 2")
    planes = torch_resize_device(values, _plane_shape(values.shape[1:], target, axis), mode,
                                 channels_last=channels_last)
    return torch_resize_device(planes, target, aniso_axis_mode, channels_last=channels_last)


def resample_torch_argmax_device(logits, shape, *, axis: int | None, mode: str = "linear",
                                 aniso_axis_mode: str = "nearest-exact", out=None):
    """Channels-last (X, Y, Z, C) float32/float16 GPU logits through the plans' Torch
    resampler to ``shape``, then the first-maximum class per voxel: (*shape) uint16 labels
    on the device.  The last pass and the argmax run fused (``nnx_torch_resize_argmax``);
    a separate-axis plan resamples the planes first into a float32 channels-last
    intermediate (src/nnunet_mlx/kernels/metal_torch_resample.py:195-215 followed by the
    export's argmax, src/nnunet_mlx/prediction/export.py:137-202)."""
    import torch

    from nnunet_mlx import _native

    if not isinstance(logits, torch.Tensor) or logits.dim() != 4:
        raise ContractError("Torch-grid restoration requires (X, Y, Z, C) logits")
    values = logits.permute(3, 0, 1, 2)
    target = _check_torch_grid_input(values, shape, name="Torch-grid restoration")
    classes = int(values.shape[0])
    if classes > 65536:
        raise ContractError("Torch-grid restoration supports at most 65536 classes")
    last_mode = mode
    if axis is not None:
        if axis not in (0, 1, 2):
            raise ContractError("Torch-grid separate axis must be 0, 1 or 2")
        values = torch_resize_device(values, _plane_shape(values.shape[1:], target, axis), mode,
                                     channels_last=True)
        last_mode = aniso_axis_mode
    code = _torch_mode(last_mode)
    if out is None:
        out = torch.empty(target, dtype=torch.uint16, device=logits.device)
    elif tuple(out.shape) != target or out.dtype != torch.uint16 or not out.is_contiguous():
        raise ContractError("restoration output must be a contiguous uint16 target-shape tensor")
    lib = _native.load()
    _native.check(lib.nnx_torch_resize_argmax(
        values.data_ptr(), 1 if values.dtype == torch.float16 else 0, classes,
        _native.ints(values.shape[1:]), _native.i64s(values.stride()), _native.ints(target),
        code, out.data_ptr(), _native.stream_handle(logits.device)), "nnx_torch_resize_argmax")
    return out
