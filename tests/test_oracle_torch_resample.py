"""Pins of oracle/torch_resample.py (CPU).

* torch.nn.functional.interpolate — the routine upstream's resample_torch_fornnunet calls —
  on random volumes: nearest and nearest-exact indices exactly, linear values within
  float32 rounding (torch computes in float32, the oracle in float64);
* the reference's recorded upstream outputs (tests/golden/torch_resampling.npz): every
  label-resampling case bit-exactly (3-D, separate axis 0/1/2 with each axis mode, forced
  and disabled separation, tie rules, float16 near-ties, identity and constant inputs), and
  the class-model restoration cases (logits at the plans' spacing back to the cropped image
  grid, uncropped and transposed back): labels exactly, probabilities to the reference's own
  1e-5.
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from nnunet_mlx.data.resampling import separate_z_axis
from oracle import torch_resample as otr

GOLDEN = Path(__file__).resolve().parent / "golden" / "torch_resampling.npz"


@pytest.fixture(scope="module")
def recorded():
    with np.load(GOLDEN, allow_pickle=False) as saved:
        data = {name: saved[name] for name in saved.files}
    return data, json.loads(str(data.pop("metadata").item()))


@pytest.mark.parametrize("mode", otr.MODES)
@pytest.mark.parametrize("src,dst", [((5, 7, 9), (9, 4, 13)), ((3, 8, 6), (3, 17, 6)),
                                     ((11, 2, 5), (4, 7, 5)), ((1, 6, 7), (1, 9, 3))])
def test_single_pass_matches_torch_interpolate(mode, src, dst):
    rng = np.random.default_rng(sum(src) * 31 + sum(dst))
    x = (rng.standard_normal((2, *src)) * rng.uniform(0.1, 100)).astype(np.float32)
    got = otr.resize_data(x, dst, mode)
    tmode = {"linear": "trilinear", "nearest": "nearest", "nearest-exact": "nearest-exact"}[mode]
    kwargs = {"align_corners": False} if mode == "linear" else {}
    want = F.interpolate(torch.from_numpy(x)[None], size=dst, mode=tmode, **kwargs)[0].numpy()
    assert got.dtype == np.float32 and got.shape == (2, *dst)
    if mode == "linear":
        np.testing.assert_allclose(got, want, rtol=2e-6, atol=1e-6 * np.abs(x).max())
    else:
        np.testing.assert_array_equal(got, want)


def test_linear_pass_is_a_convex_combination():
    """Known answers: a constant volume stays constant; a linear ramp along one axis is
    reproduced inside the edge-clamped region."""
    c = np.full((1, 4, 5, 6), 3.25, dtype=np.float32)
    np.testing.assert_array_equal(otr.resize_data(c, (7, 3, 11), "linear"), 3.25)
    ramp = np.broadcast_to(np.arange(8, dtype=np.float32)[None, None, None, :], (1, 2, 2, 8))
    got = otr.resize_data(ramp, (2, 2, 16), "linear")[0, 0, 0]
    # target i samples source (i + 0.5) / 2 - 0.5, clamped to [0, 7]
    want = np.clip((np.arange(16) + 0.5) / 2 - 0.5, 0, 7)
    np.testing.assert_allclose(got, want, rtol=0, atol=1e-6)


def _contract_axis(case):
    kwargs = case["kwargs"]
    spacing = tuple(float(v) for v in case["spacing"])
    new_spacing = tuple(float(v) for v in case["new_spacing"])
    _, axis = separate_z_axis(spacing, new_spacing, force=kwargs.get("force_separate_z"),
                              threshold=float(kwargs.get("separate_z_anisotropy_threshold", 3.0)))
    return axis


def test_label_cases_match_the_recorded_upstream_outputs(recorded):
    data, meta = recorded
    assert len(meta["cases"]) == 72
    for case in meta["cases"]:
        kwargs = case["kwargs"]
        values = data[f"{case['name']}-input"]
        expected = data[f"{case['name']}-expected"]
        got = otr.resample(values, case["shape"], axis=_contract_axis(case),
                           mode=kwargs.get("mode", "linear"),
                           aniso_axis_mode=kwargs.get("aniso_axis_mode", "nearest-exact"),
                           is_seg=True, tiebreak=kwargs["seg_tiebreak"])
        np.testing.assert_array_equal(got, expected, err_msg=case["name"])
        assert got.dtype == values.dtype


def _restore(logits, case):
    """The class-model restoration chain (reference src/nnunet_mlx/prediction/export.py:
    137-202, 376-444): logits at the plans' spacing resampled to the cropped image grid,
    then per voxel argmax (labels) or float32 softmax (probabilities), uncropped into the
    pre-cropping shape (background outside the box) and transposed back."""
    plans = case["plans"]
    config = plans["configurations"]["selected"]
    geometry = case["geometry"]
    crop = tuple(geometry["shape_after_cropping_and_before_resampling"])
    spacing = case["properties"]["spacing"]
    forward = plans["transpose_forward"]
    spacing_t = tuple(float(spacing[a]) for a in forward)
    configured = config["spacing"]
    if len(configured) != 3:
        configured = [spacing_t[0], *configured]
    current = tuple(o if c is None else float(c) for c, o in zip(configured, spacing_t))
    kwargs = config["resampling_fn_probabilities_kwargs"]
    _, axis = separate_z_axis(current, spacing_t, force=kwargs.get("force_separate_z"),
                              threshold=float(kwargs.get("separate_z_anisotropy_threshold", 3.0)))
    resampled = otr.resample(logits, crop, axis=axis, mode=kwargs.get("mode", "linear"),
                             aniso_axis_mode=kwargs.get("aniso_axis_mode", "nearest-exact"))
    z = resampled - resampled.max(axis=0, keepdims=True)
    e = np.exp(z, dtype=np.float32)
    probs = (e / e.sum(axis=0, keepdims=True)).astype(np.float32)
    box = tuple(slice(lo, hi) for lo, hi in geometry["bbox_used_for_cropping"])
    before = tuple(geometry["shape_before_cropping"])
    labels = np.zeros(before, dtype=np.uint8)
    labels[box] = resampled.argmax(axis=0)
    seg = np.zeros(before, dtype=np.uint8)
    seg[box] = probs.argmax(axis=0)
    full = np.zeros((probs.shape[0], *before), dtype=np.float32)
    full[0] = 1.0
    full[(slice(None), *box)] = probs
    back = plans["transpose_backward"]
    return (labels.transpose(back), seg.transpose(back),
            full.transpose([0, *(b + 1 for b in back)]))


def test_restoration_cases_match_the_recorded_upstream_outputs(recorded):
    data, meta = recorded
    assert [case["name"] for case in meta["pipeline"]] == [f"pipeline-{k}" for k in range(0, 12, 2)]
    for case in meta["pipeline"]:
        key = case["name"]
        labels, seg, probs = _restore(data[f"{key}-logits"], case)
        np.testing.assert_array_equal(labels, data[f"{key}-label-only"], err_msg=key)
        np.testing.assert_array_equal(seg, data[f"{key}-segmentation"], err_msg=key)
        np.testing.assert_allclose(probs, data[f"{key}-probabilities"], rtol=1e-5, atol=5e-6,
                                   err_msg=key)
