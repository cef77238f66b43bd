"""The preprocessing oracle pinned against SciPy, numpy and closed forms (CPU only)."""

from __future__ import annotations

import numpy as np
import pytest
import scipy.ndimage as ndi

from oracle import preprocess as op


@pytest.mark.parametrize("axis", [0, 1, 2])
def test_prefilter_matches_scipy(axis):
    rng = np.random.default_rng(axis)
    padded = np.pad(rng.standard_normal((7, 9, 11)), op.SPLINE_PAD, mode="edge")
    ref = ndi.spline_filter1d(padded, order=3, axis=axis, mode="nearest", output=np.float64)
    np.testing.assert_allclose(op._prefilter_axis(padded, axis), ref, rtol=0, atol=1e-13)


ZOOM_CASES = [
    ((7, 9, 11), (12, 5, 20), 3),
    ((20, 16, 9), (13, 31, 9), 3),
    ((5, 6, 7), (5, 6, 15), 3),
    ((30, 40), (55, 17), 3),
    ((7, 9, 11), (12, 5, 20), 1),
]


@pytest.mark.parametrize("shape_in,shape_out,order", ZOOM_CASES)
def test_zoom_matches_scipy(shape_in, shape_out, order):
    """scipy.ndimage.zoom(order, mode="nearest", grid_mode=True) is what scikit-image's
    resize(mode="edge", anti_aliasing=False) evaluates."""
    rng = np.random.default_rng(len(shape_in) * 10 + order)
    x = rng.standard_normal(shape_in)
    zoom = np.array(shape_out) / np.array(shape_in)
    ref = ndi.zoom(x, zoom, order=order, mode="nearest", grid_mode=True)
    assert ref.shape == tuple(shape_out)
    np.testing.assert_allclose(op.zoom_spline(x, shape_out, order), ref, rtol=0, atol=1e-13)
    # float32 input: float64 arithmetic, one rounding to float32
    x32 = x.astype(np.float32)
    ref32 = ndi.zoom(x32, zoom, order=order, mode="nearest", grid_mode=True)
    got32 = op.zoom_spline(x32, shape_out, order).astype(np.float32)
    if order == 3:
        np.testing.assert_array_equal(got32, ref32)
    else:
        assert np.abs(got32.astype(np.float64) - ref32).max() <= 2 ** -22 * np.abs(ref32).max()


def test_spline_reproduces_constants_and_cubics_in_the_interior():
    const = np.full((9, 8, 10), 3.25)
    np.testing.assert_allclose(op.zoom_spline(const, (13, 5, 17), 3), 3.25, rtol=0, atol=1e-13)
    # a cubic polynomial is reproduced exactly away from the edge extension
    # (the edge's influence decays as |sqrt(3) - 2|^distance: 25 voxels leave < 1e-14)
    i = np.arange(80, dtype=np.float64)
    f = lambda u: 1e-4 * u ** 3 - 0.02 * u ** 2 + u - 4.0  # noqa: E731
    line = f(i)[:, None, None] * np.ones((1, 3, 3))
    out = op.zoom_spline(line, (113, 3, 3), 3)[:, 1, 1]
    coords = (np.arange(113) + 0.5) * (80 / 113) - 0.5
    interior = (coords > 25) & (coords < 54)
    assert interior.sum() > 30
    np.testing.assert_allclose(out[interior], f(coords[interior]), rtol=0, atol=1e-9)


def test_resize_clips_to_the_input_range():
    """A step edge overshoots under the cubic spline; scikit-image clips to [min, max]."""
    x = np.zeros((6, 6, 12), dtype=np.float32)
    x[..., 6:] = 1.0
    raw = op.zoom_spline(x, (6, 6, 29), 3)
    assert raw.min() < 0 and raw.max() > 1
    out = op.resize_spline(x, (6, 6, 29), 3)
    assert out.dtype == np.float32 and out.min() == 0.0 and out.max() == 1.0


def test_separate_axis_resample_matches_composition():
    rng = np.random.default_rng(3)
    data = rng.standard_normal((2, 5, 12, 14)).astype(np.float32)
    got = op.resample_data(data, (9, 17, 10), separate_axis=0)
    for ch in range(2):
        planes = np.stack([np.clip(ndi.zoom(data[ch, k].astype(np.float64), (17 / 12, 10 / 14),
                                            order=3, mode="nearest", grid_mode=True),
                                   data[ch, k].min(), data[ch, k].max()) for k in range(5)])
        idx = np.clip(np.floor(5 / 9 * (np.arange(9) + 0.5) - 0.5 + 0.5).astype(int), 0, 4)
        np.testing.assert_array_equal(got[ch], planes[idx].astype(np.float32))


def test_nearest_axis_indices_known_values():
    np.testing.assert_array_equal(op.nearest_axis_indices(5, 9), [0, 0, 1, 1, 2, 3, 3, 4, 4])
    np.testing.assert_array_equal(op.nearest_axis_indices(4, 2), [1, 3])


def test_nonzero_bbox_and_ct_normalize():
    data = np.zeros((2, 7, 8, 9), dtype=np.float32)
    data[0, 2, 3, 4] = 1.0
    data[1, 5, 1, 6] = -2.0
    assert op.nonzero_bbox(data) == ((2, 6), (1, 4), (4, 7))
    with pytest.raises(ValueError):
        op.nonzero_bbox(np.zeros((1, 2, 2, 2)))
    v = np.array([-2000.0, -57.3, 0.0, 41.7, 3000.0], dtype=np.float32)
    got = op.ct_normalize(v, mean=41.5, std=60.25, lower=-1000.0, upper=1500.0)
    clipped = np.minimum(np.maximum(v, np.float32(-1000.0)), np.float32(1500.0))
    want = (clipped - np.float32(41.5)) / np.float32(60.25)
    np.testing.assert_array_equal(got, want.astype(np.float32))
    assert got.dtype == np.float32


def _brute_force_fill(mask):
    """Enclosed background by breadth-first search from the border (6-neighbours)."""
    from collections import deque

    reached = np.zeros(mask.shape, dtype=bool)
    queue = deque()
    for idx in np.ndindex(mask.shape):
        if not mask[idx] and any(i in (0, n - 1) for i, n in zip(idx, mask.shape)):
            reached[idx] = True
            queue.append(idx)
    while queue:
        idx = queue.popleft()
        for axis in range(3):
            for step in (-1, 1):
                nb = list(idx)
                nb[axis] += step
                nb = tuple(nb)
                if all(0 <= i < n for i, n in zip(nb, mask.shape)) and not mask[nb] and not reached[nb]:
                    reached[nb] = True
                    queue.append(nb)
    return ~reached


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_filled_mask_is_six_connected_hole_filling(seed):
    from oracle.preprocess import filled_nonzero_mask

    rng = np.random.default_rng(seed)
    data = (rng.random((2, 7, 8, 9)) < 0.35).astype(np.float32) * rng.standard_normal((2, 7, 8, 9))
    data[0, 2:5, 2:6, 2:7] = 1.0
    data[0, 3, 3:5, 3:6] = 0.0          # sealed cavity
    got = filled_nonzero_mask(data)
    np.testing.assert_array_equal(got, _brute_force_fill(np.any(data != 0, axis=0)))
    assert got[3, 3, 3]


def test_zscore_normalize_closed_form():
    from oracle.preprocess import zscore_normalize

    rng = np.random.default_rng(5)
    x = (rng.standard_normal((6, 7, 8)) * 30 + 100).astype(np.float32)
    mask = rng.random(x.shape) < 0.6
    got = zscore_normalize(x, mask)
    sel = x[mask].astype(np.float64)
    want = (x.astype(np.float64) - sel.mean()) / sel.std()
    np.testing.assert_allclose(got[mask], want[mask], rtol=0, atol=2e-5)
    np.testing.assert_array_equal(got[~mask], x[~mask])
    const = zscore_normalize(np.full((3, 3, 3), 7.0, dtype=np.float32))
    np.testing.assert_array_equal(const, np.zeros((3, 3, 3), dtype=np.float32))


def test_rescale_and_rgb_closed_forms():
    from oracle.preprocess import rescale01_normalize, rgb01_normalize

    x = np.array([[[3.0, 7.0], [5.0, 11.0]]], dtype=np.float32)
    np.testing.assert_allclose(rescale01_normalize(x), (x - 3.0) / 8.0, rtol=0, atol=1e-7)
    assert rescale01_normalize(x).min() == 0.0 and rescale01_normalize(x).max() == 1.0
    np.testing.assert_array_equal(rescale01_normalize(np.full((2, 2, 2), 4.0, np.float32)),
                                  np.zeros((2, 2, 2), np.float32))
    np.testing.assert_array_equal(rgb01_normalize(np.array([0.0, 255.0, 51.0], np.float32)),
                                  np.array([0.0, 1.0, 0.2], np.float32))
    with pytest.raises(ValueError):
        rgb01_normalize(np.array([-1.0, 3.0], np.float32))
