"""Torch-grid resampling on the GPU (``nnx_torch_resize``, ``nnx_torch_resize_argmax``) against
oracle/torch_resample.py, bit-exactly: the kernel and the oracle compute the same float32
coordinates and the same float64 corner sums in the same order, so every float32 value and
every label agrees.  Also the two plans-driven callers: Torch-plan data preprocessing and
the class-label restoration of the reference's recorded upstream cases
(tests/golden/torch_resampling.npz, labels exactly)."""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from nnunet_mlx.data.resampling import (resample_torch_argmax_device, resample_torch_device,
                                        separate_z_axis, torch_resize_device)
from nnunet_mlx.errors import ContractError
from nnunet_mlx.plans import ResamplingContract
from oracle import torch_resample as otr

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden" / "torch_resampling.npz"

SHAPES = [((5, 7, 9), (9, 4, 13)), ((3, 8, 6), (3, 17, 6)), ((11, 2, 5), (4, 7, 5)),
          ((1, 6, 7), (1, 9, 3)), ((6, 1, 4), (2, 5, 1)), ((16, 20, 24), (40, 50, 10))]
# seeded grids beside them (size-1 axes included)
SHAPES += [tuple(tuple(int(v) for v in g) for g in pair) for pair in
           np.random.default_rng(2033).integers(1, 33, (4, 2, 3))]


def _values(rng, channels, shape, dtype):
    x = (rng.standard_normal((channels, *shape)) * rng.uniform(0.1, 100)).astype(np.float32)
    return x.astype(np.float16) if dtype == torch.float16 else x


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
@pytest.mark.parametrize("mode", otr.MODES)
@pytest.mark.parametrize("src,dst", SHAPES)
def test_single_pass_is_bit_exact(device, src, dst, mode, dtype):
    rng = np.random.default_rng(sum(src) * 7 + sum(dst))
    x = _values(rng, 3, src, dtype)
    want = otr.resize_data(x.astype(np.float32), dst, mode)
    print(f"torch-grid pass {src}->{dst} mode={mode} dtype={dtype}", flush=True)
    first = torch.from_numpy(x).to(device)
    got = torch_resize_device(first, dst, mode).cpu().numpy()
    assert got.dtype == np.float32 and got.shape == want.shape
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
    # channels-last input and output (the logits' layout): strided reads and writes
    last = torch.from_numpy(np.ascontiguousarray(np.moveaxis(x, 0, -1))).to(device)
    got = torch_resize_device(last.permute(3, 0, 1, 2), dst, mode, channels_last=True)
    assert got.permute(1, 2, 3, 0).is_contiguous() or tuple(dst) == tuple(src)
    np.testing.assert_array_equal(got.cpu().numpy().view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("axis", [0, 1, 2])
@pytest.mark.parametrize("modes", [("linear", "nearest-exact"), ("linear", "linear"),
                                   ("nearest", "nearest"), ("nearest-exact", "linear")])
def test_separate_axis_resampling_is_bit_exact(device, axis, modes):
    rng = np.random.default_rng(axis * 11 + len(modes[0]) + 3 * len(modes[1]))
    x = _values(rng, 2, (9, 12, 10), torch.float32)
    shape = (5, 17, 23)
    want = otr.resample(x, shape, axis=axis, mode=modes[0], aniso_axis_mode=modes[1])
    print(f"torch-grid separate axis {axis} modes {modes}", flush=True)
    got = resample_torch_device(torch.from_numpy(x).to(device), shape, axis=axis, mode=modes[0],
                                aniso_axis_mode=modes[1]).cpu().numpy()
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


def _first_argmax(values):
    return values.argmax(axis=0).astype(np.uint16)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
@pytest.mark.parametrize("axis,modes", [(None, ("linear", "nearest-exact")),
                                        (None, ("nearest", "nearest-exact")),
                                        (0, ("linear", "nearest-exact")),
                                        (2, ("linear", "linear")),
                                        (1, ("nearest-exact", "nearest"))])
def test_fused_argmax_matches_resampled_argmax(device, axis, modes, dtype):
    """Labels of the fused last pass equal the argmax of the oracle's resampled float32
    values, ties included (logits quantised to a coarse grid make many exact ties)."""
    rng = np.random.default_rng(5 + (axis or 0))
    classes, src, dst = 4, (10, 12, 9), (23, 7, 15)
    x = np.round(rng.standard_normal((classes, *src)) * 2).astype(np.float32)
    x = x.astype(np.float16) if dtype == torch.float16 else x
    want = _first_argmax(otr.resample(x.astype(np.float32), dst, axis=axis, mode=modes[0],
                                      aniso_axis_mode=modes[1]))
    print(f"torch-grid argmax axis={axis} modes={modes} dtype={dtype}", flush=True)
    logits = torch.from_numpy(np.ascontiguousarray(np.moveaxis(x, 0, -1))).to(device)
    got = resample_torch_argmax_device(logits, dst, axis=axis, mode=modes[0],
                                       aniso_axis_mode=modes[1])
    np.testing.assert_array_equal(got.cpu().numpy().view(np.uint16), want)


def test_larger_volume_round_trip_and_identity(device):
    """At a CT-like size: an identity-shaped pass returns the values unchanged, an
    upsample-then-downsample by an integer factor with nearest-exact is the identity, and a
    linear upsample of a constant volume stays constant (size-independent properties)."""
    rng = np.random.default_rng(1)
    x = torch.from_numpy(rng.standard_normal((2, 96, 160, 160)).astype(np.float32)).to(device)
    assert torch.equal(torch_resize_device(x, (96, 160, 160), "linear"), x)
    up = torch_resize_device(x, (192, 320, 320), "nearest-exact")
    assert torch.equal(torch_resize_device(up, (96, 160, 160), "nearest-exact"), x)
    const = torch.full((1, 64, 80, 96), -2.75, device=device)
    assert bool((torch_resize_device(const, (150, 33, 200), "linear") == -2.75).all())


def test_rejects_bad_arguments(device):
    x = torch.zeros((1, 4, 4, 4), device=device)
    with pytest.raises(ContractError):
        torch_resize_device(x, (2, 2, 2), "cubic")
    with pytest.raises(ContractError):
        torch_resize_device(x.cpu(), (2, 2, 2), "linear")
    with pytest.raises(ContractError):
        torch_resize_device(x, (2, 0, 2), "linear")
    with pytest.raises(ContractError):
        torch_resize_device(x.double(), (2, 2, 2), "linear")
    with pytest.raises(ContractError):
        resample_torch_device(x, (2, 2, 2), axis=3)
    with pytest.raises(ContractError):
        resample_torch_argmax_device(torch.zeros((4, 4, 4), device=device), (2, 2, 2), axis=None)


@pytest.fixture(scope="module")
def recorded():
    with np.load(GOLDEN, allow_pickle=False) as saved:
        data = {name: saved[name] for name in saved.files}
    return data, json.loads(str(data.pop("metadata").item()))


def test_restoration_cases_match_the_recorded_upstream_labels(device, recorded):
    """The class-model restoration of the recorded upstream cases (logits at the plans'
    spacing back to the cropped grid, separate-axis and single-pass plans, 2-D and 3-D
    spacing entries) through ``restore_class_labels_device``: uncropped and transposed back,
    the labels equal the recorded ones exactly."""
    from nnunet_mlx.prediction.restore import restore_class_labels_device

    data, meta = recorded
    for case in meta["pipeline"]:
        key = case["name"]
        plans = case["plans"]
        config = plans["configurations"]["selected"]
        contract = ResamplingContract.from_configuration(
            config, field="resampling_fn_probabilities", expected_is_seg=False)
        geometry = case["geometry"]
        crop = tuple(geometry["shape_after_cropping_and_before_resampling"])
        forward = plans["transpose_forward"]
        spacing_t = tuple(float(case["properties"]["spacing"][a]) for a in forward)
        configured = config["spacing"]
        if len(configured) != 3:
            configured = [spacing_t[0], *configured]
        current = tuple(o if c is None else float(c) for c, o in zip(configured, spacing_t))
        logits = data[f"{key}-logits"]
        print(f"torch-plan restoration {key}: logits {logits.shape} -> {crop}", flush=True)
        dev_logits = torch.from_numpy(np.ascontiguousarray(np.moveaxis(logits, 0, -1))).to(device)
        got = restore_class_labels_device(dev_logits, crop, current, spacing_t, contract)
        labels = got.cpu().numpy().view(np.uint16)
        before = tuple(geometry["shape_before_cropping"])
        full = np.zeros(before, dtype=np.uint8)
        full[tuple(slice(lo, hi) for lo, hi in geometry["bbox_used_for_cropping"])] = labels
        np.testing.assert_array_equal(full.transpose(plans["transpose_backward"]),
                                      data[f"{key}-label-only"], err_msg=key)
        _, axis = separate_z_axis(current, spacing_t, force=contract.force_separate_z,
                                  threshold=contract.separate_z_anisotropy_threshold)
        half = resample_torch_argmax_device(dev_logits.half(), crop, axis=axis)
        want = _first_argmax(otr.resample(logits.astype(np.float16).astype(np.float32), crop,
                                          axis=axis))
        np.testing.assert_array_equal(half.cpu().numpy().view(np.uint16), want, err_msg=key)


def _torch_plan(spacing, transpose, mode, aniso):
    from nnunet_mlx.data.preprocessing import PreprocessPlan

    plans = {
        "transpose_forward": list(transpose),
        "transpose_backward": [list(transpose).index(a) for a in range(3)],
        "foreground_intensity_properties_per_channel": {
            "0": {"mean": 99.4, "std": 137.2, "percentile_00_5": -958.0, "percentile_99_5": 327.0}},
        "configurations": {"3d_fullres": {
            "spacing": list(spacing), "normalization_schemes": ["CTNormalization"],
            "use_mask_for_norm": [False], "patch_size": [64, 64, 64],
            "resampling_fn_data": "resample_torch_fornnunet",
            "resampling_fn_data_kwargs": {"is_seg": False, "force_separate_z": None,
                                          "memefficient_seg_resampling": False,
                                          "mode": mode, "aniso_axis_mode": aniso}}},
    }
    return PreprocessPlan.from_plans(plans, "3d_fullres")


@pytest.mark.parametrize("spacing,target,transpose,modes", [
    ((2.5, 0.8, 0.8), (1.0, 0.78, 0.78), (0, 1, 2), ("linear", "nearest-exact")),  # axis 0
    ((0.7, 0.7, 1.6), (1.0, 1.0, 1.0), (2, 0, 1), ("linear", "nearest-exact")),    # one pass
    ((0.8, 3.0, 0.8), (0.5, 1.0, 0.5), (0, 1, 2), ("nearest-exact", "linear")),    # axis 1
])
def test_torch_plan_preprocessing_matches_oracle(device, spacing, target, transpose, modes):
    """A Torch-plan raw case: transpose, crop, CT normalisation (the oracle's, bit-exact on
    the device already) and the Torch resampler with the plan's modes, bit-exactly."""
    from nnunet_mlx.data.preprocessing import preprocess_raw_case
    from oracle import preprocess as op

    print(f"torch-plan preprocess spacing {spacing} target {target} modes {modes}", flush=True)
    rng = np.random.default_rng(17)
    raw = np.zeros((1, 24, 40, 36), dtype=np.int16)
    raw[0, 3:21, 5:37, 2:30] = (rng.standard_normal((18, 32, 28)) * 400 - 200).astype(np.int16)
    plan = _torch_plan(target, transpose, *modes)
    out = preprocess_raw_case(raw, {"spacing": list(spacing)}, plan)
    t = raw.astype(np.float32).transpose((0, *(a + 1 for a in transpose)))
    bbox = op.nonzero_bbox(t)
    crop = t[(slice(None), *(slice(a, b) for a, b in bbox))]
    st = plan.intensity_properties["0"]
    norm = op.ct_normalize(crop[0], st["mean"], st["std"], st["percentile_00_5"],
                           st["percentile_99_5"])[None]
    original = tuple(spacing[a] for a in transpose)
    new_shape = tuple(round(o / n * s) for o, n, s in zip(original, target, crop.shape[1:]))
    _, axis = separate_z_axis(original, tuple(target), force=None)
    want = otr.resample(norm.astype(np.float32), new_shape, axis=axis, mode=modes[0],
                        aniso_axis_mode=modes[1])
    assert out.properties["bbox_used_for_cropping"] == [list(b) for b in bbox]
    got = out.data.cpu().numpy()
    assert got.shape == want.shape
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
