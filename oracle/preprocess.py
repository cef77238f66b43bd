"""Oracle: raw-case preprocessing (crop to nonzero, CT normalisation, spline resampling).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Restates, in numpy:
  * ``nonzero_bbox``: the crop bounds of ``crop_to_nonzero`` without a mask
    (src/nnunet_mlx/data/preprocessing.py:166-214): per spatial axis the first and one past
    the last index where any channel is nonzero; no nonzero voxel is an error.
  * ``ct_normalize``: the CTNormalization branch of ``_normalize_channel``
    (src/nnunet_mlx/data/preprocessing.py:274-285): float32 clip to the stored 0.5 / 99.5
    percentiles, minus the mean, divided by max(std, 1e-8), each a float32 operation.
  * ``resize_spline``: the data resize the reference delegates to scikit-image,
    ``resize(channel, shape, order, mode="edge", anti_aliasing=False)``
    (src/nnunet_mlx/data/resampling.py:476-501, 625-634).  scikit-image (absent here) maps
    it to ``scipy.ndimage.zoom(channel, shape / in_shape, order, mode="nearest",
    grid_mode=True)`` followed by a clip of the output to the input's [min, max]; that
    zoom, for order > 1, pads the input by 12 voxels with edge replication, builds B-spline
    coefficients along each axis in turn (gain, then the causal and anticausal recursions
    with the pole sqrt(3) - 2 and the boundary initialisation SciPy uses for edge
    extension), and evaluates each output voxel at the half-pixel coordinate
    (o + 0.5) * in / out - 0.5 (+ 12) from the 4 (order 3) or 2 (order 1) neighbouring
    coefficients per axis with the cardinal B-spline weights, in float64.  Output in the
    input's float type (float32 stays float32), then the clip.
  * ``resample_data``: ``resample_probabilities_or_data`` for spline plans
    (src/nnunet_mlx/data/resampling.py:87-172, 268-306, 379-442): unchanged shape casts;
    separate-z resizes each plane of the other two axes with the spline (float64, clipped
    per plane) and then the coarse axis with half-pixel nearest indices (order 0),
    rounding to float32 once.

  * ``filled_nonzero_mask`` / ``zscore_normalize``: the filled nonzero mask of
    ``crop_to_nonzero`` (SciPy's ``binary_fill_holes``, the reference's own call) and the
    ZScoreNormalization branch in numpy float32.

Pinned by tests/test_oracle_preprocess.py against ``scipy.ndimage.spline_filter1d``
(prefilter coefficients), ``scipy.ndimage.zoom`` (whole resize, float64 and float32, orders
1 and 3, 2-D and 3-D, up- and down-sampling), closed forms (constant and linear volumes
are reproduced), numpy for crop bounds and normalisation, a breadth-first flood fill from
the border for the filled mask, and the float64 closed form of the z-score (constant
channel -> zeros).
"""

from __future__ import annotations

import math

import numpy as np

SPLINE_PAD = 12
POLE3 = math.sqrt(3.0) - 2.0


def nonzero_bbox(data: np.ndarray) -> tuple[tuple[int, int], ...]:
    """Half-open (start, stop) per spatial axis of voxels where any channel is nonzero."""
    mask = np.any(np.asarray(data) != 0, axis=0)
    bounds = []
    for axis in range(mask.ndim):
        hits = np.flatnonzero(np.any(mask, axis=tuple(a for a in range(mask.ndim) if a != axis)))
        if not hits.size:
            raise ValueError("no nonzero voxel")
        bounds.append((int(hits[0]), int(hits[-1]) + 1))
    return tuple(bounds)


def filled_nonzero_mask(data: np.ndarray) -> np.ndarray:
    """The mask of ``crop_to_nonzero`` (src/nnunet_mlx/data/preprocessing.py:193-195): any
    channel nonzero, enclosed background filled by SciPy's ``binary_fill_holes`` (the
    reference's own dependency; default 6-connected structure)."""
    from scipy import ndimage

    return ndimage.binary_fill_holes(np.any(np.asarray(data) != 0, axis=0))


def zscore_normalize(values: np.ndarray, mask: np.ndarray | None = None) -> np.ndarray:
    """ZScoreNormalization of ``_normalize_channel`` (src/nnunet_mlx/data/preprocessing.py:
    298-307): numpy float32 mean and std of the selected voxels, then (x - mean) /
    max(std, 1e-8) in float32 on the selection; other voxels unchanged."""
    result = np.asarray(values, dtype=np.float32).copy()
    selection = np.ones(result.shape, dtype=bool) if mask is None else np.asarray(mask, bool)
    selected = result[selection]
    mean = float(selected.mean())
    std = float(selected.std())
    result[selection] = (result[selection] - mean) / max(std, 1e-8)
    return result


def rescale01_normalize(values: np.ndarray) -> np.ndarray:
    """RescaleTo01Normalization (src/nnunet_mlx/data/preprocessing.py:310-313), numpy float32."""
    result = np.asarray(values, dtype=np.float32).copy()
    result -= float(result.min())
    result /= max(float(result.max()), 1e-8)
    return result


def rgb01_normalize(values: np.ndarray) -> np.ndarray:
    """RGBTo01Normalization (src/nnunet_mlx/data/preprocessing.py:314-318), numpy float32."""
    result = np.asarray(values, dtype=np.float32).copy()
    if float(result.min()) < 0 or float(result.max()) > 255:
        raise ValueError("RGB normalization requires values in [0, 255]")
    result /= 255
    return result


def ct_normalize(values: np.ndarray, mean: float, std: float, lower: float,
                 upper: float) -> np.ndarray:
    """float32 clip, subtract, divide in the reference's order."""
    result = np.asarray(values, dtype=np.float32).copy()
    np.clip(result, np.float32(lower), np.float32(upper), out=result)
    result -= np.float32(mean)
    result /= np.float32(max(std, 1e-8))
    return result


def _prefilter_axis(c: np.ndarray, axis: int) -> np.ndarray:
    """Cubic B-spline coefficients along ``axis`` (float64, in place on a copy)."""
    c = np.moveaxis(np.array(c, dtype=np.float64, copy=True), axis, 0)
    n = c.shape[0]
    z = POLE3
    if n == 1:
        return np.moveaxis(c, 0, axis)
    c *= (1.0 - z) * (1.0 - 1.0 / z)
    # causal initialisation for edge extension (the reflected sequence)
    z_n = z ** n
    c0 = c[0].copy()
    acc = c[0] + z_n * c[n - 1]
    z_i = z
    for i in range(1, n):
        acc = acc + z_i * (c[i] + z_n * c[n - 1 - i])
        z_i *= z
    c[0] = acc * (z / (1.0 - z_n * z_n)) + c0
    for i in range(1, n):
        c[i] = c[i] + z * c[i - 1]
    c[n - 1] = c[n - 1] * (z / (z - 1.0))
    for i in range(n - 2, -1, -1):
        c[i] = z * (c[i + 1] - c[i])
    return np.moveaxis(c, 0, axis)


def spline_coefficients(values: np.ndarray) -> np.ndarray:
    """Edge-padded (by 12) float64 cubic B-spline coefficients, axes filtered in order."""
    c = np.pad(np.asarray(values, dtype=np.float64), SPLINE_PAD, mode="edge")
    for axis in range(c.ndim):
        c = _prefilter_axis(c, axis)
    return c


def _axis_taps(n_in: int, n_out: int, order: int):
    """(start index into the padded coefficients, weights) per output index of one axis."""
    o = np.arange(n_out, dtype=np.float64)
    cc = (o + 0.5) * (n_in / n_out) - 0.5 + SPLINE_PAD
    f = np.floor(cc)
    t = cc - f
    if order == 3:
        start = f.astype(np.int64) - 1
        w = np.stack([(1.0 - t) ** 3 / 6.0,
                      2.0 / 3.0 - t * t + t ** 3 / 2.0,
                      2.0 / 3.0 - (1.0 - t) ** 2 + (1.0 - t) ** 3 / 2.0,
                      t ** 3 / 6.0], axis=-1)
    elif order == 1:
        start = f.astype(np.int64)
        w = np.stack([1.0 - t, t], axis=-1)
    else:
        raise ValueError("orders 1 and 3 are restated")
    return start, w


def zoom_spline(values: np.ndarray, new_shape, order: int) -> np.ndarray:
    """float64 spline zoom (grid mode, edge extension), before the output cast and clip."""
    values = np.asarray(values)
    if order == 3:
        c = spline_coefficients(values)
    else:
        c = np.pad(np.asarray(values, dtype=np.float64), SPLINE_PAD, mode="edge")
    # separable evaluation, one axis at a time
    for axis, (n_in, n_out) in enumerate(zip(values.shape, new_shape)):
        start, w = _axis_taps(n_in, n_out, order)
        moved = np.moveaxis(c, axis, 0)
        out = np.zeros((n_out, *moved.shape[1:]), dtype=np.float64)
        for k in range(w.shape[1]):
            out += moved[start + k] * w[:, k].reshape((-1,) + (1,) * (moved.ndim - 1))
        c = np.moveaxis(out, 0, axis)
    # drop the padding of the axes not yet interpolated: every axis was interpolated
    return c


def resize_spline(values: np.ndarray, new_shape, order: int = 3, dtype=None) -> np.ndarray:
    """scikit-image resize semantics: zoom, cast to ``dtype`` (default: the input's float
    type), clip to the input's [min, max]."""
    values = np.asarray(values)
    dtype = dtype or (np.float32 if values.dtype == np.float32 else np.float64)
    src = values if values.dtype == dtype else values.astype(dtype)
    out = zoom_spline(src, new_shape, order).astype(dtype)
    np.clip(out, src.min(), src.max(), out=out)
    return out


def nearest_axis_indices(old: int, new: int) -> np.ndarray:
    """Half-pixel nearest indices (src/nnunet_mlx/data/resampling.py:401-407)."""
    coordinates = float(old) / new * (np.arange(new, dtype=np.float64) + 0.5) - 0.5
    return np.clip(np.floor(coordinates + 0.5).astype(np.int64), 0, old - 1)


def resample_data(data: np.ndarray, new_shape, *, order: int = 3, order_z: int = 0,
                  separate_axis: int | None = None, dtype=np.float32) -> np.ndarray:
    """(C, X, Y, Z) float32 -> (C, *new_shape) float32 along the spline plan.

    ``dtype=np.float16`` is the reference's float16-logit case
    (src/nnunet_mlx/data/resampling.py:133, 484-501): the float64 result is rounded once
    to float16 and returned as float32."""
    data = np.asarray(data)
    new_shape = tuple(int(s) for s in new_shape)
    if data.shape[1:] == new_shape:
        return data.astype(dtype).astype(np.float32)
    out = np.empty((data.shape[0], *new_shape), dtype=np.float32)
    for ch in range(data.shape[0]):
        if separate_axis is None:
            if dtype == np.float32:
                out[ch] = resize_spline(data[ch].astype(np.float32), new_shape, order)
            else:
                out[ch] = resize_spline(data[ch].astype(np.float64), new_shape, order,
                                        dtype=np.float64).astype(dtype)
            continue
        axis = separate_axis
        plane_shape = tuple(s for i, s in enumerate(new_shape) if i != axis)
        inter_shape = list(new_shape)
        inter_shape[axis] = data.shape[1 + axis]
        inter = np.empty(inter_shape, dtype=np.float64)
        for k in range(data.shape[1 + axis]):
            plane = np.take(data[ch], k, axis=axis)
            sel = [slice(None)] * 3
            sel[axis] = k
            inter[tuple(sel)] = resize_spline(plane.astype(np.float64), plane_shape, order,
                                              dtype=np.float64)
        if order_z != 0:
            raise ValueError("order_z 0 is restated")
        idx = nearest_axis_indices(inter_shape[axis], new_shape[axis])
        out[ch] = np.take(inter, idx, axis=axis).astype(dtype)
    return out
