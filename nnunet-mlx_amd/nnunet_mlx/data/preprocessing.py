"""Raw-case preprocessing on the GPU: transpose, crop to nonzero, CT normalisation and the
spline resampling of nnU-Net plans.

Reference: ``preprocess_raw_case`` (src/nnunet_mlx/data/preprocessing.py:63-163) with
``crop_to_nonzero`` (:166-214), ``_normalize_channel`` (:263-301), ``compute_new_shape``
and ``resample_probabilities_or_data`` (src/nnunet_mlx/data/resampling.py:46-172) and the
plans fields it reads (``PlansContract``, src/nnunet_mlx/plans.py:154-372).

The same step order as the reference: the raw (C, X, Y, Z) case is cast to float32,
transposed into the plans' axis order, cropped to the bounds of its nonzero voxels,
normalised per channel, and resampled to the configuration's spacing.  Every array step
runs in HIP kernels (``nnx_nonzero_bbox``, ``nnx_nonzero_mask_filled``,
``nnx_zscore_stats``, ``nnx_crop_normalize_masked``, ``nnx_resample_spline``); the host
computes shapes and reads back the six crop bounds and the z-score statistics.  The device
path covers CTNormalization, NoNormalization and ZScoreNormalization (with or without the
filled nonzero mask; mean and std accumulated in float64 and rounded to float32, within a
few float32 steps of numpy's float32 statistics) and spline plans
(``resample_data_or_seg_to_shape``; orders 1 and 3, order_z 0); RescaleTo01 and RGBTo01 run
as the z-score form with host-computed (min, max - min) and (0, 255) after a device min/max
(``nnx_channel_minmax``).  Torch-grid plans (``resample_torch_fornnunet``) resample with
``nnx_torch_resize`` (one pass, or the planes and then the separate axis;
src/nnunet_mlx/kernels/metal_torch_resample.py:195-215).  Cascade inputs raise
``ContractError`` rather than run elsewhere.
"""

from __future__ import annotations

import ctypes
from collections.abc import Mapping, Sequence
from dataclasses import dataclass

import numpy as np

from nnunet_mlx import _native
from nnunet_mlx.data.resampling import resample_torch_device, separate_z_axis, validate_spacing
from nnunet_mlx.errors import ContractError
from nnunet_mlx.plans import ResamplingContract, resolve_configuration

DEVICE_SCHEMES = {"NoNormalization": _native.NNX_NORM_NONE, "CTNormalization": _native.NNX_NORM_CT,
                  "ZScoreNormalization": _native.NNX_NORM_ZSCORE,
                  # (x - min) / max(max - min, 1e-8) and x / 255: the z-score form with
                  # host-computed (mean, std)
                  "RescaleTo01Normalization": _native.NNX_NORM_ZSCORE,
                  "RGBTo01Normalization": _native.NNX_NORM_ZSCORE}


@dataclass(frozen=True)
class PreprocessPlan:
    """The plans fields preprocessing reads (src/nnunet_mlx/plans.py:154-372).

    ``transpose_forward`` maps the raw spatial axes into the plans' axis order; ``spacing``
    is the configuration's target spacing in that order (``None`` keeps the image's
    spacing on that axis); ``normalization_schemes`` and ``use_mask_for_norm`` have one
    entry per channel; ``intensity_properties[str(c)]`` holds the CT statistics
    (``mean``, ``std``, ``percentile_00_5``, ``percentile_99_5``)."""

    transpose_forward: tuple[int, int, int]
    spacing: tuple[float | None, ...]
    normalization_schemes: tuple[str, ...]
    use_mask_for_norm: tuple[bool, ...]
    intensity_properties: Mapping[str, Mapping[str, object]]
    data_resampling: ResamplingContract

    @classmethod
    def from_plans(cls, plans: Mapping[str, object], configuration: str) -> "PreprocessPlan":
        resolved = resolve_configuration(plans, configuration)
        forward = plans.get("transpose_forward")
        if (not isinstance(forward, (list, tuple)) or sorted(forward) != [0, 1, 2]
                or any(isinstance(a, bool) for a in forward)):
            raise ContractError("transpose_forward must be a permutation of [0, 1, 2]")
        backward = plans.get("transpose_backward")
        if backward is not None and list(backward) != [list(forward).index(a) for a in range(3)]:
            raise ContractError("transpose_backward is not the inverse of transpose_forward")
        spacing = resolved.get("spacing")
        if not isinstance(spacing, (list, tuple)) or len(spacing) not in (2, 3):
            raise ContractError("plan spacing must hold 2 or 3 values")
        for value in spacing:
            if value is not None and (isinstance(value, bool) or not isinstance(value, (int, float))
                                      or not np.isfinite(value) or value <= 0):
                raise ContractError("plan spacing values must be positive numbers or null")
        schemes = resolved.get("normalization_schemes")
        masks = resolved.get("use_mask_for_norm")
        if not isinstance(schemes, (list, tuple)) or not all(isinstance(s, str) for s in schemes):
            raise ContractError("normalization_schemes must be a list of names")
        if (not isinstance(masks, (list, tuple)) or len(masks) != len(schemes)
                or not all(isinstance(m, bool) for m in masks)):
            raise ContractError("use_mask_for_norm must hold one boolean per channel")
        intensity = plans.get("foreground_intensity_properties_per_channel", {})
        if not isinstance(intensity, Mapping):
            raise ContractError("foreground_intensity_properties_per_channel must be a mapping")
        return cls(
            transpose_forward=tuple(int(a) for a in forward),
            spacing=tuple(None if v is None else float(v) for v in spacing),
            normalization_schemes=tuple(schemes),
            use_mask_for_norm=tuple(masks),
            intensity_properties=intensity,
            data_resampling=ResamplingContract.from_configuration(
                resolved, field="resampling_fn_data", expected_is_seg=False),
        )


@dataclass(frozen=True)
class PreprocessedRawCase:
    """``data`` (C, X', Y', Z') float32 on the GPU in the plans' axis order and spacing;
    ``properties`` extends the input properties with ``shape_before_cropping``,
    ``bbox_used_for_cropping`` and ``shape_after_cropping_and_before_resampling``
    (plans' axis order), which restoration needs to invert the crop."""

    data: object
    previous_stage: None
    properties: dict[str, object]


def compute_new_shape(old_shape: Sequence[int], old_spacing: Sequence[float],
                      new_spacing: Sequence[float]) -> tuple[int, ...]:
    """round(old_spacing / new_spacing * size) per axis, Python rounding
    (src/nnunet_mlx/data/resampling.py:46-69)."""
    if not (len(old_shape) == len(old_spacing) == len(new_spacing) and len(old_shape) in (2, 3)):
        raise ContractError("shape and spacing ranks must match in 2-D or 3-D")
    if any(s < 1 for s in old_shape) or any(v <= 0 for v in (*old_spacing, *new_spacing)):
        raise ContractError("resampling shape and spacing values must be positive")
    return tuple(round(old / new * size) for old, new, size in zip(old_spacing, new_spacing, old_shape))


def _ct_statistics(plan: PreprocessPlan, channel: int) -> tuple[float, float, float, float]:
    stats = plan.intensity_properties.get(str(channel), {})
    values = []
    for key in ("mean", "std", "percentile_00_5", "percentile_99_5"):
        value = stats.get(key) if isinstance(stats, Mapping) else None
        if isinstance(value, bool) or not isinstance(value, (int, float)) or not np.isfinite(value):
            raise ContractError(f"CT {key} must be a finite number")
        values.append(float(value))
    mean, std, lower, upper = values
    if std <= 0:
        raise ContractError("CT std must be positive")
    if lower > upper:
        raise ContractError("CT intensity percentiles are reversed")
    return mean, std, lower, upper


def _check_finite(lib, tensor, message: str) -> None:
    import torch

    count = torch.zeros(1, dtype=torch.int32, device=tensor.device)
    _native.check(lib.nnx_count_nonfinite(tensor.data_ptr(), tensor.numel(), count.data_ptr(),
                                          _native.stream_handle()))
    if int(count.item()) != 0:
        raise ContractError(message)


def preprocess_raw_case(data, properties: Mapping[str, object], plan: PreprocessPlan, *,
                        segmentation_previous_stage=None) -> PreprocessedRawCase:
    """Transpose, crop to nonzero, normalise and resample one raw case on the GPU.

    ``data``: (C, X, Y, Z) real numeric values (numpy array or CUDA tensor) in the raw
    image's axis order; ``properties["spacing"]``: three positive voxel sizes in the same
    order.  Returns the preprocessed case with ``data`` a CUDA float32 tensor."""
    import torch

    if segmentation_previous_stage is not None:
        raise ContractError("cascade previous-stage inputs are not supported on the device path")
    lib = _native.load()
    device = torch.device("cuda", torch.cuda.current_device())
    if isinstance(data, torch.Tensor):
        if data.dim() != 4 or data.shape[0] < 1 or data.is_complex() or data.dtype == torch.bool:
            raise ContractError("raw nnU-Net cases must have CXYZ layout with real values")
        values = data.to(device=device, dtype=torch.float32).contiguous()
    else:
        array = np.asarray(data)
        if array.ndim != 4 or array.shape[0] < 1:
            raise ContractError("raw nnU-Net cases must have CXYZ layout")
        if array.dtype.kind not in "iuf":
            raise ContractError("raw nnU-Net cases must contain finite real numeric values")
        values = torch.from_numpy(np.ascontiguousarray(array)).to(device=device,
                                                                 dtype=torch.float32)
    channels = int(values.shape[0])
    _check_finite(lib, values, "raw nnU-Net cases must remain finite after float32 conversion")
    if len(plan.normalization_schemes) != channels:
        raise ContractError("normalization schemes do not match the input channels")
    for scheme in plan.normalization_schemes:
        if scheme not in DEVICE_SCHEMES:
            raise ContractError(f"normalization scheme {scheme!r} is not supported on the device path")
    spacing = validate_spacing(properties.get("spacing", ()), name="image spacing")
    forward = plan.transpose_forward
    raw_shape = tuple(int(s) for s in values.shape[1:])
    transposed_shape = tuple(raw_shape[a] for a in forward)
    result = dict(properties)
    result["shape_before_cropping"] = transposed_shape

    st = _native.stream_handle()
    bbox = torch.empty(6, dtype=torch.int32, device=device)
    _native.check(lib.nnx_nonzero_bbox(values.data_ptr(), channels, _native.i64s(raw_shape),
                                       bbox.data_ptr(), st))
    raw_bounds = bbox.cpu().numpy().reshape(3, 2)
    if int(raw_bounds[0, 1]) < 0:
        raise ContractError("raw nnU-Net case has no nonzero voxels")
    # bounds in the plans' axis order: out axis k is raw axis forward[k]
    bounds = [(int(raw_bounds[a, 0]), int(raw_bounds[a, 1]) + 1) for a in forward]
    result["bbox_used_for_cropping"] = [list(pair) for pair in bounds]
    cropped_shape = tuple(stop - start for start, stop in bounds)
    result["shape_after_cropping_and_before_resampling"] = cropped_shape

    schemes = [DEVICE_SCHEMES[s] for s in plan.normalization_schemes]
    norm = np.zeros((channels, 4), dtype=np.float32)
    raw_start = [int(raw_bounds[a, 0]) for a in range(3)]
    raw_extent = [int(raw_bounds[a, 1]) + 1 - int(raw_bounds[a, 0]) for a in range(3)]
    mask = None
    if any(s == "ZScoreNormalization" and m
           for s, m in zip(plan.normalization_schemes, plan.use_mask_for_norm)):
        # the filled nonzero mask of crop_to_nonzero, over the crop box in raw order
        mask = torch.empty(raw_extent, dtype=torch.uint8, device=device)
        flag = torch.empty(64, dtype=torch.int32, device=device)
        _native.check(min(0, lib.nnx_nonzero_mask_filled(
            values.data_ptr(), channels, _native.i64s(raw_shape), _native.i64s(raw_start),
            _native.i64s(raw_extent), mask.data_ptr(), flag.data_ptr(), st)),
            "nnx_nonzero_mask_filled")
    stats = torch.empty((channels, 2), dtype=torch.float32, device=device)
    stat_work = None
    for c, scheme in enumerate(plan.normalization_schemes):
        if scheme == "CTNormalization":
            mean, std, lower, upper = _ct_statistics(plan, c)
            norm[c] = (mean, max(std, 1e-8), lower, upper)
        elif scheme == "ZScoreNormalization":
            if stat_work is None:
                stat_work = torch.empty(lib.nnx_zscore_stats_workspace(), dtype=torch.uint8,
                                        device=device)
            use_mask = plan.use_mask_for_norm[c]
            _native.check(lib.nnx_zscore_stats(
                values.data_ptr(), channels, _native.i64s(raw_shape), c,
                _native.i64s(raw_start), _native.i64s(raw_extent),
                mask.data_ptr() if use_mask else None, stats[c].data_ptr(),
                stat_work.data_ptr(), st))
            if use_mask:
                schemes[c] = _native.NNX_NORM_ZSCORE_MASKED
        elif scheme in ("RescaleTo01Normalization", "RGBTo01Normalization"):
            if stat_work is None:
                stat_work = torch.empty(lib.nnx_zscore_stats_workspace(), dtype=torch.uint8,
                                        device=device)
            _native.check(lib.nnx_channel_minmax(
                values.data_ptr(), channels, _native.i64s(raw_shape), c,
                _native.i64s(raw_start), _native.i64s(raw_extent), stats[c].data_ptr(),
                stat_work.data_ptr(), st))
    if stat_work is not None:
        host_stats = stats.cpu().numpy()
        for c, scheme in enumerate(plan.normalization_schemes):
            if scheme == "RescaleTo01Normalization":
                low, high = (np.float32(v) for v in host_stats[c])
                # the float32 operations of _normalize_channel: x - min, then / max(x - min)
                norm[c, :2] = (low, max(float(np.float32(high - low)), 1e-8))
            elif scheme == "RGBTo01Normalization":
                low, high = (float(v) for v in host_stats[c])
                if low < 0 or high > 255:
                    raise ContractError("RGB normalization requires values in [0, 255]")
                norm[c, :2] = (0.0, 255.0)
        for c, scheme in enumerate(plan.normalization_schemes):
            if scheme == "ZScoreNormalization":
                mean, std = (float(v) for v in host_stats[c])
                if not (np.isfinite(mean) and np.isfinite(std)):
                    raise ContractError("z-score normalization mask is empty")
                norm[c, :2] = (mean, std)
    cropped = torch.empty((channels, *cropped_shape), dtype=torch.float32, device=device)
    _native.check(lib.nnx_crop_normalize_masked(
        values.data_ptr(), channels, _native.i64s(raw_shape), _native.ints(forward),
        _native.i64s([start for start, _ in bounds]), _native.i64s(cropped_shape),
        _native.ints(schemes), norm.ctypes.data_as(ctypes.POINTER(ctypes.c_float)),
        mask.data_ptr() if mask is not None else None, _native.i64s(raw_start),
        _native.i64s(raw_extent), cropped.data_ptr(), st))
    _check_finite(lib, cropped, "normalization produced non-finite values")

    original_spacing = tuple(spacing[a] for a in forward)
    configured = plan.spacing if len(plan.spacing) == 3 else (original_spacing[0], *plan.spacing)
    target_spacing = tuple(o if c is None else c for c, o in zip(configured, original_spacing))
    new_shape = compute_new_shape(cropped_shape, original_spacing, target_spacing)
    if any(s < 1 for s in new_shape):
        raise ContractError("resampling target shape must be positive")
    if tuple(new_shape) == cropped_shape:
        return PreprocessedRawCase(cropped, None, result)
    contract = plan.data_resampling
    if contract.function_name == "resample_torch_fornnunet":
        _, axis = separate_z_axis(validate_spacing(original_spacing, name="current spacing"),
                                  validate_spacing(target_spacing, name="new spacing"),
                                  force=contract.force_separate_z,
                                  threshold=contract.separate_z_anisotropy_threshold)
        out = resample_torch_device(cropped, new_shape, axis=axis, mode=contract.mode,
                                    aniso_axis_mode=contract.aniso_axis_mode)
        _check_finite(lib, out, "resampling produced non-finite values")
        return PreprocessedRawCase(out, None, result)
    if contract.function_name != "resample_data_or_seg_to_shape":
        raise ContractError(f"data resampling {contract.function_name!r} is not supported on the device path")
    separate, axis = separate_z_axis(validate_spacing(original_spacing, name="current spacing"),
                                     validate_spacing(target_spacing, name="new spacing"),
                                     force=contract.force_separate_z,
                                     threshold=contract.separate_z_anisotropy_threshold)
    sep_axis = axis if separate else -1
    order_z = contract.order_z if separate else 0
    work_bytes = lib.nnx_resample_spline_workspace(_native.i64s(cropped_shape),
                                                   _native.i64s(new_shape), sep_axis)
    if work_bytes == 0:
        raise ContractError("invalid resampling shapes")
    work = torch.empty(work_bytes, dtype=torch.uint8, device=device)
    out = torch.empty((channels, *new_shape), dtype=torch.float32, device=device)
    _native.check(lib.nnx_resample_spline(
        cropped.data_ptr(), channels, _native.i64s(cropped_shape), _native.i64s(new_shape),
        contract.order, sep_axis, order_z, work.data_ptr(), work_bytes, out.data_ptr(), st))
    del work
    _check_finite(lib, out, "resampling produced non-finite values")
    return PreprocessedRawCase(out, None, result)
