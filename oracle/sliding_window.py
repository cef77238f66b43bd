"""Oracle sliding window: numpy restatement of the reference's Gaussian sliding window.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Follows src/nnunet_mlx/prediction/sliding_window.py:
  * compute_steps / _axis_steps (:32-67): count = ceil((I-P)/(P*f)) + 1, stride =
    (I-P)/(count-1) in float64, offsets round(stride*k) with Python's half-to-even round.
  * _pad_minimum (:542-562): before = (P-I)//2, after = the rest; crop slices.
  * gaussian_importance (:70-93): float32 exp(-0.5 * sum(((i - P//2)/(P/8))^2)), / max,
    zeros -> float32 tiny.
  * nnunet_fp16_gaussian (:96-113): scipy.ndimage.gaussian_filter of a centred impulse
    (sigma = P/8, mode constant), scaled to max 10, float16, zeros -> smallest nonzero.
  * mirrored_prediction (:489-527): views none, then itertools.combinations(axes, r) for
    r = 1..len(axes); outputs flipped back and summed left to right in float32, / count.
  * _accumulate_logits (:359-460): tiles in itertools.product order; float32 mode
    acc += pred*g, norm += g; nnunet-fp16 mode acc = f16(f32(acc) + pred*f32(g)),
    norm = f16(norm + g).
  * finalizers (:200-356) and fold averaging (src/nnunet_mlx/prediction/inference.py:93-149):
    q = f32(acc)/f32(norm) cast to the accumulation dtype; folds summed in that dtype;
    average = dtype(f32(total)/f32(n)); labels = argmax, earliest channel on ties.
  * host fold average (src/nnunet_mlx/prediction/inference.py:25-90) for the fp16 rounding
    fixtures.

Pinned by tests/test_oracle_sliding_window.py: closed forms and brute force for steps
and padding, the published step tables, float64 closed-form Gaussians (within one
float32 ulp), scipy's documented kernel for the fp16 Gaussian, a pointwise fake network
(the mirrored average of a pointwise model equals the model), and the reference's
recorded fp16 fold-rounding fixtures (tests/fixtures/darwin-arm64/upstream_runner.npz).
"""

from __future__ import annotations

from collections.abc import Callable, Sequence
from itertools import combinations, product

import numpy as np

Model = Callable[[np.ndarray], np.ndarray]


def axis_steps(image: int, patch: int, step_fraction: float) -> tuple[int, ...]:
    count = int(np.ceil((image - patch) / (patch * step_fraction))) + 1
    maximum = image - patch
    actual = maximum / (count - 1) if count > 1 else 0.0
    return tuple(round(actual * index) for index in range(count))


def compute_steps(image_size: Sequence[int], patch_size: Sequence[int], step_fraction: float = 0.5):
    return tuple(axis_steps(int(i), int(p), step_fraction) for i, p in zip(image_size, patch_size))


def pad_minimum(shape: Sequence[int], patch: Sequence[int]):
    """Return (pad_before, pad_after, crop slices) for spatial ``shape``."""
    before, after, crop = [], [], []
    for size, minimum in zip(shape, patch):
        total = max(0, minimum - size)
        b = total // 2
        before.append(b)
        after.append(total - b)
        crop.append(slice(b, b + size))
    return tuple(before), tuple(after), tuple(crop)


def gaussian_importance(patch_size: tuple[int, ...]) -> np.ndarray:
    exponent = np.zeros(patch_size, dtype=np.float32)
    for axis, size in enumerate(patch_size):
        center = size // 2
        sigma = size / 8
        coordinates = np.arange(size, dtype=np.float32)
        shape = tuple(size if index == axis else 1 for index in range(len(patch_size)))
        exponent += (((coordinates - center) / sigma) ** 2).reshape(shape)
    values = np.exp(-0.5 * exponent).astype(np.float32, copy=False)
    values /= np.float32(values.max())
    values[values == 0] = np.finfo(np.float32).tiny
    return values


def nnunet_fp16_gaussian(patch_size: tuple[int, ...]) -> np.ndarray:
    from scipy.ndimage import gaussian_filter

    impulse = np.zeros(patch_size)
    impulse[tuple(size // 2 for size in patch_size)] = 1
    weights = gaussian_filter(impulse, [size / 8 for size in patch_size], mode="constant")
    rounded = (weights / (weights.max() / 10)).astype(np.float16)
    rounded[rounded == 0] = rounded[rounded != 0].min()
    return rounded


def mirror_views(axes: Sequence[int]) -> list[tuple[int, ...]]:
    views: list[tuple[int, ...]] = [()]
    for count in range(1, len(axes) + 1):
        views.extend(combinations(tuple(axes), count))
    return views


def mirrored_prediction(model: Model, tile: np.ndarray, axes: Sequence[int]) -> np.ndarray:
    """``tile`` is channels-last (1, *patch, C); returns (1, *patch, K) float32."""
    views = mirror_views(axes)
    prediction = np.asarray(model(tile), dtype=np.float32)
    if len(views) == 1:
        return prediction
    for selected in views[1:]:
        flip_axes = tuple(a + 1 for a in selected)
        mirrored = np.ascontiguousarray(np.flip(tile, axis=flip_axes))
        current = np.flip(np.asarray(model(mirrored), dtype=np.float32), axis=flip_axes)
        prediction = prediction + current
    return prediction / np.float32(len(views))


def accumulate(
    model: Model,
    data: np.ndarray,
    patch: tuple[int, ...],
    *,
    num_classes: int,
    axes: Sequence[int] = (),
    step_fraction: float = 0.5,
    accumulation: str = "float32",
):
    """Return (acc, norm, crop) over the padded channels-last volume."""
    before, after, crop = pad_minimum(data.shape[1:], patch)
    padded = np.pad(data, [(0, 0)] + list(zip(before, after)))
    spatial = padded.shape[1:]
    steps = compute_steps(spatial, patch, step_fraction)
    fp16 = accumulation == "nnunet-fp16"
    dtype = np.float16 if fp16 else np.float32
    acc = np.zeros((*spatial, num_classes), dtype=dtype)
    norm = np.zeros((*spatial, 1), dtype=dtype)
    g = (nnunet_fp16_gaussian(patch) if fp16 else gaussian_importance(patch))[..., None]
    g32 = g.astype(np.float32)
    volume = np.moveaxis(padded, 0, -1)
    for offsets in product(*steps):
        sl = tuple(slice(o, o + p) for o, p in zip(offsets, patch))
        pred = mirrored_prediction(model, np.ascontiguousarray(volume[sl][None]), axes)[0]
        if fp16:
            acc[sl] = (acc[sl].astype(np.float32) + pred * g32).astype(np.float16)
            norm[sl] = norm[sl] + g
        else:
            acc[sl] += pred * g
            norm[sl] += g
    return acc, norm, crop


def normalized(acc: np.ndarray, norm: np.ndarray, crop, accumulation: str) -> np.ndarray:
    dtype = np.float16 if accumulation == "nnunet-fp16" else np.float32
    q = (acc.astype(np.float32) / norm.astype(np.float32)).astype(dtype)
    return q[crop]


def fold_average_device(values: Sequence[np.ndarray], accumulation: str) -> np.ndarray:
    """average_fold_device_logits arithmetic on channels-last fold logits."""
    total = values[0].copy()
    for v in values[1:]:
        total = (total + v).astype(total.dtype)
    if len(values) > 1:
        total = (total.astype(np.float32) / np.float32(len(values))).astype(total.dtype)
    return total


def fold_average_host(values: Sequence[np.ndarray], accumulation: str) -> np.ndarray:
    """average_fold_logits (host) arithmetic: fp16 folds, in-place sum, /= float32(n)."""
    fp16 = accumulation == "nnunet-fp16"
    total = None
    for current in values:
        v = np.asarray(current, dtype=np.float16) if fp16 else np.array(current, dtype=np.float32)
        if total is None:
            total = v.copy()
        else:
            total += v
    total /= np.float32(len(values))
    return np.asarray(total, dtype=np.float16 if fp16 else np.float32)


def labels(values: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Channels-last scores -> (uint16 argmax with earliest ties, invalid mask)."""
    v = values.astype(np.float32)
    invalid = ~np.isfinite(v).all(axis=-1)
    safe = np.where(np.isfinite(v), v, -np.inf)
    out = np.argmax(safe, axis=-1).astype(np.uint16)
    out[invalid] = 65535
    return out, invalid


def predict(
    models: Sequence[Model],
    data: np.ndarray,
    patch: tuple[int, ...],
    *,
    num_classes: int,
    axes: Sequence[int] = (),
    step_fraction: float = 0.5,
    accumulation: str = "float32",
) -> tuple[np.ndarray, np.ndarray]:
    """Fold-averaged channels-last logits (accumulation dtype) and uint16 labels."""
    per_fold = []
    for model in models:
        acc, norm, crop = accumulate(
            model, data, patch, num_classes=num_classes, axes=axes,
            step_fraction=step_fraction, accumulation=accumulation,
        )
        per_fold.append(normalized(acc, norm, crop, accumulation))
    logits = fold_average_device(per_fold, accumulation)
    lab, _ = labels(logits)
    return logits, lab
