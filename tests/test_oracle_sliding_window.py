"""Pinning of the sliding-window oracle (and the product's host arithmetic) on the CPU.

Each check compares against something other than the formula under test: published step
tables, exact rationals with half-to-even rounding, float64 closed forms, scipy's
documented Gaussian kernel, a pointwise fake network (known answer), and the reference's
recorded fp16 fold-rounding and head fixtures (tests/golden/upstream_runner_subset.npz,
extracted from the reference's tests/fixtures/darwin-arm64/upstream_runner.npz).
"""

from __future__ import annotations

import math
from fractions import Fraction
from itertools import combinations
from pathlib import Path

import numpy as np
import pytest

from nnunet_mlx.prediction import sliding_window as sw
from oracle import sliding_window as osw

GOLDEN = Path(__file__).resolve().parent / "golden" / "upstream_runner_subset.npz"

# Published step tables for the four benchmark shapes (padded size, patch) -> offsets.
STEP_TABLES = {
    "liver": ((128, 768, 768), (128, 128, 128),
              ((0,), tuple(range(0, 641, 64)), tuple(range(0, 641, 64)))),
    "brats": ((155, 240, 240), (128, 128, 128), ((0, 27), (0, 56, 112), (0, 56, 112))),
    "autopet": ((284, 400, 400), (112, 160, 128),
                ((0, 43, 86, 129, 172), (0, 80, 160, 240), (0, 54, 109, 163, 218, 272))),
    "pancreas": ((128, 768, 768), (128, 160, 160),
                 ((0,), tuple(range(0, 609, 76)), tuple(range(0, 609, 76)))),
}


@pytest.mark.parametrize("name", list(STEP_TABLES))
def test_steps_match_published_tables(name):
    image, patch, expected = STEP_TABLES[name]
    assert osw.compute_steps(image, patch, 0.5) == expected
    assert sw.compute_steps(image, patch, step_fraction=0.5) == expected


def test_tile_counts_of_the_benchmarks():
    counts = {n: int(np.prod([len(a) for a in t[2]])) for n, t in STEP_TABLES.items()}
    assert counts == {"liver": 121, "brats": 18, "autopet": 120, "pancreas": 81}


def _exact_steps(image: int, patch: int, fraction: Fraction) -> tuple[int, ...]:
    """Exact-rational restatement: smallest count with stride <= patch*fraction, offsets
    rounded half to even."""
    span = image - patch
    if span == 0:
        return (0,)
    count = 2
    while Fraction(span, count - 1) > patch * fraction:
        count += 1
    return tuple(round(Fraction(span * k, count - 1)) for k in range(count))


def test_steps_brute_force_against_exact_rationals():
    rng = np.random.default_rng(0)
    for _ in range(3000):
        patch = int(rng.integers(1, 200))
        image = patch + int(rng.integers(0, 600))
        fraction = Fraction(int(rng.integers(1, 9)), 8)
        expected = _exact_steps(image, patch, fraction)
        got = osw.axis_steps(image, patch, float(fraction))
        # float64 stride*k can land one ulp off an exact .5; allow only those cases
        if got != expected:
            diffs = [(g, e, Fraction((image - patch) * k, len(expected) - 1))
                     for k, (g, e) in enumerate(zip(got, expected)) if g != e]
            assert len(got) == len(expected)
            assert all(f.denominator == 2 for _, _, f in diffs), (image, patch, fraction, diffs)
        assert got[0] == 0 and got[-1] == image - patch
        assert sw._axis_steps(image, patch, step_fraction=float(fraction)) == got


def test_steps_round_half_to_even():
    # span 5 over 2 gaps gives 2.5 -> 2 (Python's round), not 3
    assert osw.axis_steps(10, 5, 0.5) == (0, 2, 5)
    assert sw._axis_steps(10, 5, step_fraction=0.5) == (0, 2, 5)


def test_steps_reject_bad_requests():
    from nnunet_mlx.errors import ContractError

    with pytest.raises(ContractError):
        sw.compute_steps((10, 10, 10), (12, 8, 8))
    with pytest.raises(ContractError):
        sw.compute_steps((10, 10, 10), (8, 8, 8), step_fraction=0.0)
    with pytest.raises(ContractError):
        sw.compute_steps((10, 10, 10, 10), (8, 8, 8, 8))


def test_minimum_padding():
    before, after, crop = osw.pad_minimum((101, 768, 768), (128, 128, 128))
    assert before == (13, 0, 0) and after == (14, 0, 0)
    assert crop[0] == slice(13, 114)
    rng = np.random.default_rng(1)
    for _ in range(200):
        size = tuple(int(v) for v in rng.integers(1, 50, 3))
        patch = tuple(int(v) for v in rng.integers(1, 50, 3))
        b, a, c = osw.pad_minimum(size, patch)
        pb, padded, pc = sw.pad_minimum(size, patch)
        for i in range(3):
            assert b[i] + size[i] + a[i] == max(size[i], patch[i])
            assert b[i] == max(0, patch[i] - size[i]) // 2
            assert c[i] == slice(b[i], b[i] + size[i]) == pc[i]
        assert pb == b and padded == tuple(max(s, p) for s, p in zip(size, patch))


@pytest.mark.parametrize("patch", [(128, 128, 128), (112, 160, 128), (128, 160, 160), (7, 9, 4)])
def test_gaussian_against_float64_closed_form(patch):
    g = osw.gaussian_importance(patch)
    np.testing.assert_array_equal(g, sw.gaussian_importance(patch))
    grids = np.meshgrid(*[np.arange(s, dtype=np.float64) for s in patch], indexing="ij")
    exponent = sum(((grid - s // 2) / (s / 8)) ** 2 for grid, s in zip(grids, patch))
    closed = np.exp(-0.5 * exponent)
    closed = np.maximum(closed / closed.max(), np.finfo(np.float32).tiny)
    # the float32 exponent carries ~1 ulp, amplified by exp in the far tail
    np.testing.assert_allclose(g, closed, rtol=2e-5, atol=0)
    assert g[tuple(s // 2 for s in patch)] == np.float32(1.0)
    assert g.dtype == np.float32 and g.min() > 0


def test_gaussian_is_symmetric_about_the_centre():
    g = osw.gaussian_importance((16, 12, 10))
    for axis, size in enumerate((16, 12, 10)):
        c = size // 2
        for d in range(1, min(c, size - 1 - c) + 1):
            lo = np.take(g, c - d, axis=axis)
            hi = np.take(g, c + d, axis=axis)
            np.testing.assert_array_equal(lo, hi)


def _scipy_kernel(sigma: float, truncate: float = 4.0) -> np.ndarray:
    """scipy.ndimage's documented 1-D Gaussian: radius int(truncate*sigma + 0.5),
    weights exp(-0.5 x^2 / sigma^2) normalised to sum 1."""
    radius = int(truncate * sigma + 0.5)
    x = np.arange(-radius, radius + 1, dtype=np.float64)
    w = np.exp(-0.5 / sigma**2 * x**2)
    return w / w.sum()


@pytest.mark.parametrize("patch", [(128, 128, 128), (112, 160, 128), (16, 12, 10)])
def test_fp16_gaussian_against_documented_kernel(patch):
    weights = np.ones(patch)
    for axis, size in enumerate(patch):
        kernel = _scipy_kernel(size / 8)
        radius = (len(kernel) - 1) // 2
        line = np.zeros(size)
        for i in range(size):
            d = i - size // 2
            if -radius <= d <= radius:
                line[i] = kernel[d + radius]
        weights = weights * line.reshape(tuple(size if a == axis else 1 for a in range(3)))
    expected = (weights / (weights.max() / 10)).astype(np.float16)
    expected[expected == 0] = expected[expected != 0].min()
    got = osw.nnunet_fp16_gaussian(patch)
    np.testing.assert_array_equal(got, expected)
    np.testing.assert_array_equal(got, sw.nnunet_fp16_gaussian(patch))
    assert got.max() == np.float16(10)


def test_mirror_order():
    assert osw.mirror_views((0, 1, 2)) == [(), (0,), (1,), (2,), (0, 1), (0, 2), (1, 2), (0, 1, 2)]
    assert sw.mirror_flip_masks((0, 1, 2)) == (0, 1, 2, 4, 3, 5, 6, 7)
    assert sw.mirror_flip_masks((1, 2)) == (0, 2, 4, 6)
    assert sw.mirror_flip_masks(()) == (0,)
    for axes in [(0,), (2, 0), (0, 1, 2)]:
        views = [()] + [c for r in range(1, len(axes) + 1) for c in combinations(axes, r)]
        assert sw.mirror_flip_masks(axes) == tuple(sum(1 << a for a in v) for v in views)


class Pointwise:
    def __init__(self, scale=1.0):
        self.scale = np.float32(scale)

    def __call__(self, values):
        return np.concatenate((values * self.scale, -values * self.scale), axis=-1)


@pytest.mark.parametrize("accumulation", ["float32", "nnunet-fp16"])
@pytest.mark.parametrize("axes", [(), (0, 1, 2), (1,)])
def test_pointwise_model_is_reproduced(accumulation, axes):
    """Gaussian normalisation cancels and a pointwise model commutes with flips, so the
    prediction equals the model (a dropped tile, wrong flip or misplaced add breaks it)."""
    data = np.random.default_rng(2).standard_normal((1, 11, 20, 9)).astype(np.float32)
    logits, labels = osw.predict([Pointwise()], data, (8, 8, 8), num_classes=2, axes=axes,
                                 accumulation=accumulation)
    if accumulation == "float32":
        tol, checked = 1e-6, np.ones(data.shape[1:], dtype=bool)
    else:
        # nnU-Net's float16 map floors far corners at the smallest float16; voxels covered
        # only by such weights keep half-precision noise, so check well-weighted voxels.
        _, norm, crop = osw.accumulate(Pointwise(), data, (8, 8, 8), num_classes=2, axes=axes,
                                       accumulation=accumulation)
        tol, checked = 4e-3, norm[crop][..., 0].astype(np.float32) >= 0.1
        assert checked.mean() > 0.25
    np.testing.assert_allclose(logits[..., 0][checked], data[0][checked], rtol=tol, atol=tol)
    np.testing.assert_allclose(logits[..., 1][checked], -data[0][checked], rtol=tol, atol=tol)
    decided = checked & (np.abs(data[0]) > 1e-2)
    np.testing.assert_array_equal(labels[decided], (data[0] < 0)[decided].astype(np.uint16))


def test_position_dependent_model_detects_flip_errors():
    """A model whose output depends on position within the tile is not flip-invariant:
    the mirrored average must equal the explicit average of flipped-back outputs."""
    tile = np.random.default_rng(3).standard_normal((1, 4, 5, 6, 1)).astype(np.float32)
    ramp = np.arange(4 * 5 * 6, dtype=np.float32).reshape(1, 4, 5, 6, 1)

    def model(values):
        return values * ramp

    got = osw.mirrored_prediction(model, tile, (0, 1, 2))
    terms = []
    for axes in osw.mirror_views((0, 1, 2)):
        a = tuple(x + 1 for x in axes)
        terms.append(np.flip(np.flip(tile, a) * ramp, a))
    expected = terms[0]
    for t in terms[1:]:
        expected = expected + t
    np.testing.assert_array_equal(got, expected / np.float32(8))
    assert not np.allclose(got, model(tile))


def test_fp16_fold_rounding_matches_recorded_upstream():
    arrays = np.load(GOLDEN, allow_pickle=False)
    for count in (1, 2, 3, 7):
        folds = [arrays[f"rounding_input_{i}"] for i in range(count)]
        expected = arrays[f"rounding_output_{count}"]
        host = osw.fold_average_host(folds, "nnunet-fp16")
        np.testing.assert_array_equal(host, expected)
        device = osw.fold_average_device([f.astype(np.float16) for f in folds], "nnunet-fp16")
        np.testing.assert_array_equal(device.astype(np.float32), expected)


@pytest.mark.parametrize("head", ["class", "region"])
def test_heads_match_recorded_upstream(head):
    from nnunet_mlx.prediction.inference import logits_to_probabilities, probabilities_to_segmentation

    arrays = np.load(GOLDEN, allow_pickle=False)
    probs = logits_to_probabilities(arrays[f"head_logits_{head}"], has_regions=head == "region")
    np.testing.assert_array_max_ulp(probs, arrays[f"head_probabilities_{head}"], maxulp=2)
    seg = probabilities_to_segmentation(probs, regions_class_order=(1, 2) if head == "region" else None)
    np.testing.assert_array_equal(seg, arrays[f"head_segmentation_{head}"])


def test_labels_tie_and_invalid_rules():
    values = np.array([[[[1.0, 1.0, 0.0], [0.0, 2.0, 2.0], [np.nan, 0.0, 1.0], [np.inf, 0.0, 0.0]]]],
                      dtype=np.float32)
    labels, invalid = osw.labels(values)
    np.testing.assert_array_equal(labels[0, 0], [0, 1, 65535, 65535])
    np.testing.assert_array_equal(invalid[0, 0], [False, False, True, True])
    assert math.isfinite(float(labels.max()))
