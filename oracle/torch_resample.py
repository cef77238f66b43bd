"""Oracle: nnU-Net's Torch-grid resampler (``resample_torch_fornnunet``).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Restates, in numpy (float32 coordinates, float64 products and sums), the reference's
Torch-grid kernel (src/nnunet_mlx/kernels/metal_torch_resample.py:56-133), which reproduces
upstream nnU-Net's ``resample_torch_fornnunet`` (torch ``interpolate`` with
``align_corners=False``):

  * per axis (source size S, target size T, float32 scale = float32(S / T)):
    ``scaled = scale * float32(i + 0.5)`` in float32 (``i`` alone for mode "nearest"); the
    nearest index is ``min(int(scaled), S - 1)`` (lines 63-66);
  * linear: ``coordinate = max(scaled - 0.5, 0)`` in float32, ``lower = min(int(coordinate),
    S - 1)``, ``upper = min(lower + 1, S - 1)``, ``fraction = coordinate - floor(coordinate)``,
    weights ``(1 - fraction, fraction)`` (lines 67-74);
  * data: the eight corners in the order 000 ... 111 (axis 0 the high bit), each term
    ``((v * w0) * w1) * w2`` and the terms summed in corner order — float64 here, which the
    reference emulates with double-single arithmetic — then rounded to float32 (lines
    79-102);
  * labels: per corner ``((1000 * w0) * w1) * w2``; per label of the stencil (first
    occurrence order) the sum of its corners' terms, rounded to float32 and then to float16;
    the highest score wins, ties by the rule "lowest", "highest" or "nearest" (the label at
    the nearest-exact position, else the lower label) (lines 103-127);
  * separate-axis resampling: the planes across ``axis`` resized with ``mode``, then the
    whole volume with ``aniso_axis_mode`` (src/nnunet_mlx/kernels/metal_torch_resample.py:
    199-215); between the passes data is float32 and labels are decided.

Pinned by tests/test_oracle_torch_resample.py against torch.nn.functional.interpolate
(the upstream resampler's own routine; float32 values to 1e-5, nearest indices exactly) and
the reference's recorded upstream outputs (tests/fixtures/darwin-arm64/torch_resampling.npz
of the reference: every label case bit-exactly, the class-model restoration cases'
labels exactly and probabilities to 1e-5).
"""

from __future__ import annotations

import numpy as np

MODES = ("linear", "nearest", "nearest-exact")
TIEBREAKS = ("lowest", "highest", "nearest")


def axis_grid(source: int, target: int, mode: str):
    """(nearest, lower, upper, lower_weight, upper_weight) per target index of one axis;
    weights float64 (exact values of the float32 fraction and of 1 - fraction)."""
    scale = np.float32(source / target)
    pos = np.arange(target, dtype=np.float32)
    shifted = pos if mode == "nearest" else pos + np.float32(0.5)
    scaled = (scale * shifted).astype(np.float32)
    nearest = np.minimum(scaled.astype(np.int64), source - 1)
    coordinate = np.maximum(scaled - np.float32(0.5), np.float32(0.0)).astype(np.float32)
    lower = np.minimum(coordinate.astype(np.int64), source - 1)
    upper = np.minimum(lower + 1, source - 1)
    fraction = (coordinate - np.floor(coordinate)).astype(np.float32).astype(np.float64)
    return nearest, lower, upper, 1.0 - fraction, fraction


def _grids(src_shape, dst_shape, mode):
    return [axis_grid(s, t, mode) for s, t in zip(src_shape, dst_shape)]


def resize_data(values: np.ndarray, shape, mode: str) -> np.ndarray:
    """One pass over (C, A0, A1, A2) float data to spatial ``shape``: float32 result."""
    v = np.asarray(values)
    if v.shape[1:] == tuple(shape):
        return v.astype(np.float32)
    g = _grids(v.shape[1:], shape, mode)
    if mode != "linear":
        n0, n1, n2 = (grid[0] for grid in g)
        return v[:, n0[:, None, None], n1[None, :, None], n2[None, None, :]].astype(np.float32)
    v64 = v.astype(np.float32).astype(np.float64)
    total = np.zeros((v.shape[0], *shape), dtype=np.float64)
    for corner in range(8):
        sides = [(corner >> (2 - axis)) & 1 for axis in range(3)]
        idx = [g[a][1 + sides[a]] for a in range(3)]
        w = [g[a][3 + sides[a]] for a in range(3)]
        term = v64[:, idx[0][:, None, None], idx[1][None, :, None], idx[2][None, None, :]]
        term = term * w[0][:, None, None]
        term = term * w[1][None, :, None]
        term = term * w[2][None, None, :]
        total = total + term
    return total.astype(np.float32)


def resize_labels(values: np.ndarray, shape, mode: str, tiebreak: str) -> np.ndarray:
    """One pass over (C, A0, A1, A2) integer labels: scale-1000 float16-quantised scores
    per stencil label (pure Python per voxel: small inputs only)."""
    v = np.asarray(values)
    if v.shape[1:] == tuple(shape):
        return v.copy()
    g = _grids(v.shape[1:], shape, mode)
    out = np.empty((v.shape[0], *shape), dtype=v.dtype)
    for c in range(v.shape[0]):
        for i in range(shape[0]):
            for j in range(shape[1]):
                for k in range(shape[2]):
                    pos = (i, j, k)
                    nearest = v[c, g[0][0][i], g[1][0][j], g[2][0][k]]
                    if mode != "linear":
                        out[c, i, j, k] = nearest
                        continue
                    samples, terms = [], []
                    for corner in range(8):
                        sides = [(corner >> (2 - axis)) & 1 for axis in range(3)]
                        ix = [int(g[a][1 + sides[a]][pos[a]]) for a in range(3)]
                        t = 1000.0
                        for a in range(3):
                            t = t * float(g[a][3 + sides[a]][pos[a]])
                        samples.append(int(v[c, ix[0], ix[1], ix[2]]))
                        terms.append(t)
                    best, winner = -1.0, 0
                    for n, label in enumerate(samples):
                        if label in samples[:n]:
                            continue
                        score = 0.0
                        for m, other in enumerate(samples):
                            if other == label:
                                score = score + terms[m]
                        rounded = float(np.float16(np.float32(score)))
                        if tiebreak == "lowest":
                            preferred = label < winner
                        elif tiebreak == "highest":
                            preferred = label > winner
                        else:
                            preferred = label == nearest or (winner != nearest and label < winner)
                        if rounded > best or (rounded == best and preferred):
                            best, winner = rounded, label
                    out[c, i, j, k] = winner
    return out


def resample(values: np.ndarray, shape, *, axis: int | None, mode: str = "linear",
             aniso_axis_mode: str = "nearest-exact", is_seg: bool = False,
             tiebreak: str = "nearest") -> np.ndarray:
    """(C, A0, A1, A2) to spatial ``shape``: one pass, or the planes across ``axis`` first
    (their size along ``axis`` kept) and then ``axis`` with ``aniso_axis_mode``."""
    def one(v, s, m):
        return resize_labels(v, s, m, tiebreak) if is_seg else resize_data(v, s, m)

    shape = tuple(int(s) for s in shape)
    if axis is None:
        return one(values, shape, mode)
    v = np.asarray(values)
    inplane = tuple(v.shape[1 + a] if a == axis else shape[a] for a in range(3))
    return one(one(v, inplane, mode), shape, aniso_axis_mode)
