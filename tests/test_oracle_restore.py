"""Pinning of the restoration oracle on the CPU (half-pixel trilinear + argmax)."""

from __future__ import annotations

import numpy as np
import pytest
from scipy import ndimage

from oracle.restore import axis_metadata, brute_force_labels, interpolate_channel, restore_labels

SHAPES = [((5, 7, 6), (9, 4, 6)), ((3, 4, 5), (3, 4, 5)), ((1, 6, 3), (4, 2, 7)),
          ((8, 8, 8), (3, 11, 5)), ((2, 3, 2), (2, 3, 9))]


@pytest.mark.parametrize("source,target", SHAPES)
def test_interpolation_matches_scipy_zoom(source, target):
    """The host resampler's order-1 half-pixel zoom with edge extension."""
    v = np.random.default_rng(1).standard_normal(source)
    got = interpolate_channel(v, target)
    zoom = [t / s for s, t in zip(source, target)]
    ref = ndimage.zoom(v, zoom, order=1, mode="nearest", grid_mode=True)
    assert ref.shape == tuple(target)
    np.testing.assert_allclose(got, ref, rtol=0, atol=1e-12)


@pytest.mark.parametrize("source,target", SHAPES)
@pytest.mark.parametrize("dtype", [np.float32, np.float16])
def test_labels_match_brute_force_and_zoom(source, target, dtype):
    logits = np.random.default_rng(2).standard_normal((*source, 4)).astype(dtype)
    got = restore_labels(logits, target)
    np.testing.assert_array_equal(got, brute_force_labels(logits, target))
    zoom = [t / s for s, t in zip(source, target)]
    scores = np.stack([ndimage.zoom(logits[..., k].astype(np.float64), zoom, order=1,
                                    mode="nearest", grid_mode=True) for k in range(4)], -1)
    scores = scores.astype(np.float16 if dtype == np.float16 else np.float32)
    np.testing.assert_array_equal(got, np.argmax(scores, axis=-1))


def test_identity_is_first_maximum_argmax():
    logits = np.random.default_rng(3).integers(-2, 3, (4, 5, 6, 3)).astype(np.float32)  # many ties
    np.testing.assert_array_equal(restore_labels(logits, (4, 5, 6)), np.argmax(logits, -1))


def test_axis_metadata_closed_form():
    lower, upper, wl, wu = axis_metadata(4, 8)  # upsampling by 2: c = i/2 - 0.25
    np.testing.assert_array_equal(lower, [0, 0, 0, 1, 1, 2, 2, 3])
    np.testing.assert_array_equal(upper, [1, 1, 1, 2, 2, 3, 3, 3])
    np.testing.assert_allclose(wu, [0, 0.25, 0.75, 0.25, 0.75, 0.25, 0.75, 0])
    np.testing.assert_allclose(wl + wu, 1.0)
    lower, upper, wl, wu = axis_metadata(9, 3)  # downsampling by 3: centres 1, 4, 7
    np.testing.assert_array_equal(lower, [1, 4, 7])
    np.testing.assert_array_equal(wu, [0, 0, 0])


@pytest.mark.parametrize("source,target", SHAPES)
@pytest.mark.parametrize("dtype", [np.float32, np.float16])
def test_spline_route_order1_equals_trilinear_route(source, target, dtype):
    """Order-1 whole-volume spline restoration and the trilinear restoration are the same
    half-pixel interpolation reached by two independent oracle routes."""
    from oracle.restore import restore_labels_spline

    logits = np.random.default_rng(3).standard_normal((*source, 3)).astype(dtype)
    labels, values = restore_labels_spline(logits, target, order=1, separate_axis=None)
    assert labels.shape == tuple(target)
    agree = (labels == restore_labels(logits, target)).mean()
    assert agree >= 0.999
    if dtype == np.float16:
        np.testing.assert_array_equal(values, values.astype(np.float16).astype(np.float32))


def test_spline_route_separate_axis_is_planewise_then_nearest():
    """Separate-axis restoration: every target plane is the in-plane resize of the nearest
    source plane (scipy.ndimage.zoom order 1 on that plane), argmax over classes."""
    from oracle.restore import restore_labels_spline

    rng = np.random.default_rng(4)
    logits = rng.standard_normal((5, 9, 7, 3)).astype(np.float32)
    target = (12, 6, 11)
    labels, values = restore_labels_spline(logits, target, order=1, separate_axis=0)
    for o in range(target[0]):
        k = min(max(int(np.floor(5 / 12 * (o + 0.5) - 0.5 + 0.5)), 0), 4)
        for c in range(3):
            plane = logits[k, :, :, c].astype(np.float64)
            ref = ndimage.zoom(plane, (6 / 9, 11 / 7), order=1, mode="nearest", grid_mode=True)
            np.testing.assert_allclose(values[c, o], ref, rtol=1e-6, atol=1e-6)
    np.testing.assert_array_equal(labels, np.argmax(values, axis=0))
