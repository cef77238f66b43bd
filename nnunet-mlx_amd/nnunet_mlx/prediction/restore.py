"""Restoration of class logits to the original grid on the GPU.

Reference: the fused Metal restoration and its dispatch policy
(src/nnunet_mlx/kernels/metal_restore.py:296-427) as called by
``restore_device_segmentation`` (src/nnunet_mlx/prediction/export.py:321-356).  The HIP
kernel (``nnx_restore_labels``) resamples channels-last device logits with half-pixel
trilinear interpolation clamped to the source edges, in float64, and writes the
first-maximum argmax as uint16 labels; only the labels leave the device.

Supported, as in the reference: equal source and target shapes (argmax only, whatever
the policy), or the spline resampler ``resample_data_or_seg_to_shape`` with ``order`` 1
and no separate-axis resampling.  Other cases return ``None`` so the caller restores on
the host.  float16 logits (the runner's fp16 accumulation) are rounded to float16 after
the interpolation, as the reference's host path stores them.

``restore_class_labels_device`` adds the cases the reference leaves to its host
restoration (src/nnunet_mlx/prediction/restore.py:28-158): spline plans with separate-axis
resampling (``order_z`` 0) or ``order`` 3 run ``nnx_restore_labels_spline`` — each class
resampled as ``resample_probabilities_or_data`` does (float64, clipped, one rounding to
the logits' precision) and folded into the first-maximum argmax on the device; Torch-grid
plans (``resample_torch_fornnunet``) run ``nnx_torch_resize`` for the in-plane pass of a
separate-axis plan and ``nnx_torch_resize_argmax`` for the last pass and the argmax
(float32 values, as the reference's Torch resampler returns them for float16 logits too).
"""

from __future__ import annotations

from collections.abc import Sequence

import numpy as np
import torch

from nnunet_mlx import _native
from nnunet_mlx.data.resampling import (resample_torch_argmax_device, separate_z_axis,
                                        validate_spacing)
from nnunet_mlx.errors import ContractError
from nnunet_mlx.plans import ResamplingContract

_INT32_MAX = np.iinfo(np.int32).max


def _target_shape(new_shape: Sequence[int]) -> tuple[int, int, int]:
    """Require a three-dimensional positive target shape
    (src/nnunet_mlx/kernels/metal_restore.py:492-497)."""
    result = tuple(int(value) for value in new_shape)
    if len(result) != 3 or any(value < 1 for value in result):
        raise ContractError("restoration target shape must contain three positive values")
    return result  # type: ignore[return-value]


def _validate_index_range(source_shape: Sequence[int], target: tuple[int, int, int]) -> None:
    """Reject dimensions outside the int32 range the reference admits
    (src/nnunet_mlx/kernels/metal_restore.py:500-509)."""
    if any(int(value) > _INT32_MAX for value in (*source_shape, *target)):
        raise ContractError("restoration dimensions exceed the int32 range")
    if target[1] * target[2] > _INT32_MAX or target[0] * target[1] * target[2] > _INT32_MAX:
        raise ContractError("restoration target volume exceeds the int32 range")


def device_class_restore_supported(source_shape: Sequence[int], new_shape: Sequence[int],
                                   current_spacing: Sequence[float],
                                   new_spacing: Sequence[float], contract: ResamplingContract,
                                   *, classes: int) -> bool:
    """Geometry and interpolation support, decided before any logits are allocated
    (src/nnunet_mlx/kernels/metal_restore.py:330-355)."""
    target = _target_shape(new_shape)
    if len(source_shape) != 3 or classes < 1 or classes > np.iinfo(np.uint16).max + 1:
        return False
    _validate_index_range((classes, *source_shape), target)
    if tuple(int(v) for v in source_shape) == target:
        return True
    if contract.function_name != "resample_data_or_seg_to_shape" or contract.order != 1:
        return False
    separate, _ = separate_z_axis(
        validate_spacing(current_spacing, name="current spacing"),
        validate_spacing(new_spacing, name="new spacing"),
        force=contract.force_separate_z,
        threshold=contract.separate_z_anisotropy_threshold,
    )
    return not separate


def resample_class_logits_argmax_device(logits: torch.Tensor, new_shape: Sequence[int], *,
                                        out: torch.Tensor | None = None) -> torch.Tensor:
    """Interpolate channels-last (D, H, W, C) float32/float16 device logits to
    ``new_shape`` and return the (D', H', W') uint16 first-maximum labels on the device.

    No spacing or separate-axis policy is applied (the direct entry, like
    ``resample_class_logits_argmax_metal``, src/nnunet_mlx/kernels/metal_restore.py:270-297).
    """
    target = _target_shape(new_shape)
    if logits.ndim != 4 or logits.dtype not in (torch.float32, torch.float16):
        raise ContractError("restoration requires non-empty float32 or float16 (D,H,W,C) logits")
    if logits.device.type != "cuda":
        raise ContractError("device restoration requires logits on the GPU")
    classes = int(logits.shape[-1])
    if classes < 1 or classes > np.iinfo(np.uint16).max + 1 or logits.numel() == 0:
        raise ContractError("restoration requires 1..65536 classes and a non-empty grid")
    _validate_index_range(logits.shape, target)
    logits = logits.contiguous()
    if out is None:
        out = torch.empty(target, dtype=torch.uint16, device=logits.device)
    elif tuple(out.shape) != target or out.dtype != torch.uint16 or not out.is_contiguous():
        raise ContractError("restoration output must be a contiguous uint16 target-shape tensor")
    lib = _native.load()
    _native.check(lib.nnx_restore_labels(
        logits.data_ptr(), 1 if logits.dtype == torch.float16 else 0, classes,
        _native.ints(logits.shape[:3]), _native.ints(target), out.data_ptr(),
        _native.stream_handle(logits.device)), "nnx_restore_labels")
    return out


def resample_device_logits_argmax(logits: torch.Tensor, new_shape: Sequence[int],
                                  current_spacing: Sequence[float], new_spacing: Sequence[float],
                                  contract: ResamplingContract, *, return_device: bool = False):
    """Restore labels from GPU-resident channels-last logits
    (src/nnunet_mlx/kernels/metal_restore.py:358-398).

    Returns host uint16 labels (or the device tensor with ``return_device``), or ``None``
    when the policy is not supported on the device, so the caller restores on the host.
    The caller has already rejected non-finite logits (the sliding window does).
    """
    if logits.ndim != 4 or logits.dtype not in (torch.float32, torch.float16):
        return None
    classes = int(logits.shape[-1])
    source = tuple(int(v) for v in logits.shape[:3])
    if not device_class_restore_supported(source, new_shape, current_spacing, new_spacing,
                                          contract, classes=classes):
        return None
    labels = resample_class_logits_argmax_device(logits, new_shape)
    if return_device:
        return labels
    return np.ascontiguousarray(labels.cpu().numpy().view(np.uint16))


def device_spline_restore_supported(source_shape: Sequence[int], new_shape: Sequence[int],
                                    contract: ResamplingContract, *, classes: int) -> bool:
    """Whether ``nnx_restore_labels_spline`` covers the plans' probability resampling:
    the spline resampler with order 1 or 3 and, when an axis is resampled separately,
    nearest indices along it (``order_z`` 0)."""
    target = _target_shape(new_shape)
    if len(source_shape) != 3 or classes < 1 or classes > np.iinfo(np.uint16).max + 1:
        return False
    _validate_index_range((classes, *source_shape), target)
    return (contract.function_name == "resample_data_or_seg_to_shape"
            and contract.order in (1, 3) and contract.order_z == 0)


def resample_class_logits_argmax_spline_device(logits: torch.Tensor, new_shape: Sequence[int], *,
                                               order: int, separate_axis: int | None,
                                               out: torch.Tensor | None = None) -> torch.Tensor:
    """Channels-last (D, H, W, C) float32/float16 device logits -> (D', H', W') uint16
    first-maximum labels along the spline resampler (``separate_axis`` None: whole volume)."""
    target = _target_shape(new_shape)
    if logits.ndim != 4 or logits.dtype not in (torch.float32, torch.float16):
        raise ContractError("restoration requires non-empty float32 or float16 (D,H,W,C) logits")
    if logits.device.type != "cuda":
        raise ContractError("device restoration requires logits on the GPU")
    classes = int(logits.shape[-1])
    if classes < 1 or classes > np.iinfo(np.uint16).max + 1 or logits.numel() == 0:
        raise ContractError("restoration requires 1..65536 classes and a non-empty grid")
    if order not in (1, 3):
        raise ContractError("device spline restoration supports orders 1 and 3")
    _validate_index_range(logits.shape, target)
    axis = -1 if separate_axis is None else int(separate_axis)
    logits = logits.contiguous()
    if out is None:
        out = torch.empty(target, dtype=torch.uint16, device=logits.device)
    elif tuple(out.shape) != target or out.dtype != torch.uint16 or not out.is_contiguous():
        raise ContractError("restoration output must be a contiguous uint16 target-shape tensor")
    lib = _native.load()
    src = _native.ints(logits.shape[:3])
    dst = _native.ints(target)
    size = lib.nnx_restore_labels_spline_workspace(src, dst, axis)
    if size == 0:
        raise ContractError("invalid restoration shapes")
    work = torch.empty(size, dtype=torch.uint8, device=logits.device)
    _native.check(lib.nnx_restore_labels_spline(
        logits.data_ptr(), 1 if logits.dtype == torch.float16 else 0, classes, src, dst, order,
        axis, work.data_ptr(), size, out.data_ptr(), _native.stream_handle(logits.device)),
        "nnx_restore_labels_spline")
    return out


def restore_class_labels_device(logits: torch.Tensor, new_shape: Sequence[int],
                                current_spacing: Sequence[float], new_spacing: Sequence[float],
                                contract: ResamplingContract) -> torch.Tensor | None:
    """Device uint16 labels on the target grid: the trilinear entry where the reference's
    fused path applies, the spline entry for separate-axis or order-3 spline plans, the
    Torch-grid entries for Torch plans (the reference's host restoration); ``None`` for
    spline plans with ``order_z`` above 0 or orders other than 1 and 3."""
    if logits.ndim != 4 or logits.dtype not in (torch.float32, torch.float16):
        raise ContractError("restoration requires float32 or float16 (D,H,W,C) logits")
    labels = resample_device_logits_argmax(logits, new_shape, current_spacing, new_spacing,
                                           contract, return_device=True)
    if labels is not None:
        return labels
    classes = int(logits.shape[-1])
    source = tuple(int(v) for v in logits.shape[:3])
    if contract.function_name == "resample_torch_fornnunet":
        target = _target_shape(new_shape)
        _validate_index_range((classes, *source), target)
        _, axis = separate_z_axis(
            validate_spacing(current_spacing, name="current spacing"),
            validate_spacing(new_spacing, name="new spacing"),
            force=contract.force_separate_z,
            threshold=contract.separate_z_anisotropy_threshold,
        )
        return resample_torch_argmax_device(logits, target, axis=axis, mode=contract.mode,
                                            aniso_axis_mode=contract.aniso_axis_mode)
    if not device_spline_restore_supported(source, new_shape, contract, classes=classes):
        return None
    separate, axis = separate_z_axis(
        validate_spacing(current_spacing, name="current spacing"),
        validate_spacing(new_spacing, name="new spacing"),
        force=contract.force_separate_z,
        threshold=contract.separate_z_anisotropy_threshold,
    )
    return resample_class_logits_argmax_spline_device(
        logits, new_shape, order=contract.order, separate_axis=axis if separate else None)
