"""Oracle: class-logit restoration to the original grid (half-pixel trilinear + argmax).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Restates, in numpy float64:
  * the per-axis interpolation metadata of the reference's fused restoration
    (src/nnunet_mlx/kernels/metal_restore.py:464-489): coordinate
    c = (i + 0.5) * (S / T) - 0.5 clipped to [0, S - 1], lower = floor(c),
    upper = min(lower + 1, S - 1), upper weight c - lower, lower weight 1 - that;
  * the per-voxel value (src/nnunet_mlx/kernels/metal_restore.py:121-133): for each
    class, the eight corners in the order 000, 001, 010, 011, 100, 101, 110, 111
    (z, y, x bits), each term ((v * w_z) * w_y) * w_x, summed left to right — in float64,
    which the reference emulates with double-single arithmetic because SciPy's
    interpolation is float64 (src/nnunet_mlx/kernels/metal_restore.py:37-38);
  * the value handed to the argmax: the float64 sum rounded to float32, or to float16
    (nearest even) for float16 logits (src/nnunet_mlx/kernels/metal_restore.py:51-64);
  * the argmax: strict ``>`` over classes in order from -inf, so ties keep the earliest
    class (src/nnunet_mlx/kernels/metal_restore.py:119-137;
    src/nnunet_mlx/prediction/restore.py:195-215).

``restore_labels_spline`` is the reference's host restoration for spline plans
(src/nnunet_mlx/prediction/restore.py:28-158): each class resampled by
``preprocess.resample_data`` (separate axis or whole volume, float16 logits rounded once to
float16), then numpy's first-maximum argmax.  Its order-1 whole-volume route is pinned
against ``restore_labels`` (the same interpolation reached independently) and its
separate-axis route per plane against ``scipy.ndimage.zoom``.

Pinned by tests/test_oracle_restore.py against: scipy.ndimage.zoom(order=1,
mode="nearest", grid_mode=True) in float64 (the host resampler's order-1 half-pixel
interpolation with edge extension; values to 1e-12, labels exactly), a per-voxel
pure-Python brute force on tiny grids (bit-identical), the identity case (equal shapes
reduce to numpy's first-maximum argmax), and numpy's float64 -> float16 rounding.
"""

from __future__ import annotations

import numpy as np


def axis_metadata(source: int, target: int):
    """(lower, upper, lower_weight, upper_weight) for one axis, float64 weights."""
    coordinates = (np.arange(target, dtype=np.float64) + 0.5) * (source / target) - 0.5
    coordinates = np.clip(coordinates, 0, source - 1)
    lower = np.floor(coordinates).astype(np.int64)
    upper = np.minimum(lower + 1, source - 1)
    upper_weight = coordinates - lower
    lower_weight = 1.0 - upper_weight
    return lower, upper, lower_weight, upper_weight


def interpolate_channel(values: np.ndarray, target: tuple[int, int, int]) -> np.ndarray:
    """float64 trilinear value of one (Z, Y, X) channel on the target grid."""
    v = np.asarray(values, dtype=np.float64)
    (lz, uz, wz0, wz1), (ly, uy, wy0, wy1), (lx, ux, wx0, wx1) = (
        axis_metadata(s, t) for s, t in zip(v.shape, target)
    )
    zi = (lz[:, None, None], uz[:, None, None])
    yi = (ly[None, :, None], uy[None, :, None])
    xi = (lx[None, None, :], ux[None, None, :])
    wz = (wz0[:, None, None], wz1[:, None, None])
    wy = (wy0[None, :, None], wy1[None, :, None])
    wx = (wx0[None, None, :], wx1[None, None, :])
    total = np.zeros(target, dtype=np.float64)
    for bz in (0, 1):
        for by in (0, 1):
            for bx in (0, 1):
                term = ((v[zi[bz], yi[by], xi[bx]] * wz[bz]) * wy[by]) * wx[bx]
                total = total + term
    return total


def restore_labels(logits: np.ndarray, target: tuple[int, int, int]) -> np.ndarray:
    """Channels-last (Z, Y, X, K) float32 or float16 logits -> (Z', Y', X') uint16."""
    logits = np.asarray(logits)
    half = logits.dtype == np.float16
    best = np.full(target, -np.inf, dtype=np.float32)
    labels = np.zeros(target, dtype=np.uint16)
    for k in range(logits.shape[-1]):
        value = interpolate_channel(logits[..., k], target)
        value = value.astype(np.float16).astype(np.float32) if half else value.astype(np.float32)
        better = value > best
        best = np.where(better, value, best)
        labels[better] = k
    return labels


def brute_force_labels(logits: np.ndarray, target: tuple[int, int, int]) -> np.ndarray:
    """Per-voxel loops over the same arithmetic (tiny grids only)."""
    logits = np.asarray(logits)
    half = logits.dtype == np.float16
    meta = [axis_metadata(s, t) for s, t in zip(logits.shape[:3], target)]
    out = np.zeros(target, dtype=np.uint16)
    for z in range(target[0]):
        for y in range(target[1]):
            for x in range(target[2]):
                corners_z = ((meta[0][0][z], meta[0][2][z]), (meta[0][1][z], meta[0][3][z]))
                corners_y = ((meta[1][0][y], meta[1][2][y]), (meta[1][1][y], meta[1][3][y]))
                corners_x = ((meta[2][0][x], meta[2][2][x]), (meta[2][1][x], meta[2][3][x]))
                best, label = -np.inf, 0
                for k in range(logits.shape[-1]):
                    total = 0.0
                    for iz, wz in corners_z:
                        for iy, wy in corners_y:
                            for ix, wx in corners_x:
                                v = float(logits[iz, iy, ix, k])
                                total = total + ((v * float(wz)) * float(wy)) * float(wx)
                    value = float(np.float16(total)) if half else float(np.float32(total))
                    if value > best:
                        best, label = value, k
                out[z, y, x] = label
    return out


def restore_labels_spline(logits: np.ndarray, target: tuple[int, int, int], *, order: int,
                          separate_axis: int | None) -> tuple[np.ndarray, np.ndarray]:
    """The reference's host restoration for spline plans
    (src/nnunet_mlx/prediction/restore.py:28-158 over
    src/nnunet_mlx/data/resampling.py:87-172): each class of channels-last (D, H, W, C)
    logits resampled by the spline plan (``preprocess.resample_data``; float16 logits
    rounded to float16), then the first-maximum argmax.  Returns (labels uint16, the
    resampled (C, D', H', W') float32 values)."""
    from oracle.preprocess import resample_data

    values = np.moveaxis(np.asarray(logits), -1, 0)
    dtype = np.float16 if values.dtype == np.float16 else np.float32
    resampled = resample_data(values.astype(np.float32), target, order=order,
                              separate_axis=separate_axis, dtype=dtype)
    return np.argmax(resampled, axis=0).astype(np.uint16), resampled
