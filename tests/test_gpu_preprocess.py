"""Device preprocessing against the oracle (crop bounds, crop/transpose/normalise bit-exact;
spline resampling to one float32 rounding of the float64 oracle)."""

from __future__ import annotations

import ctypes
import itertools

import numpy as np
import pytest
import torch

from nnunet_mlx import _native
from nnunet_mlx.data.preprocessing import PreprocessPlan, preprocess_raw_case
from nnunet_mlx.errors import ContractError
from oracle import preprocess as op

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lib():
    return _native.load()


def stream():
    return _native.stream_handle()


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def sparse_volume(rng, shape, boxes):
    data = np.zeros(shape, dtype=np.float32)
    for c, (lo, hi) in boxes:
        sl = tuple(slice(a, b) for a, b in zip(lo, hi))
        data[(c, *sl)] = rng.standard_normal(tuple(b - a for a, b in zip(lo, hi))).astype(np.float32)
    return data


@pytest.mark.parametrize("shape,boxes", [
    ((1, 9, 10, 11), [(0, ((2, 3, 4), (5, 9, 6)))]),
    ((2, 17, 5, 33), [(0, ((0, 1, 30), (3, 2, 33))), (1, ((10, 0, 2), (17, 4, 3)))]),
    ((3, 64, 48, 40), [(2, ((1, 1, 1), (63, 47, 39)))]),
])
def test_nonzero_bbox(lib, shape, boxes):
    print(f"bbox case {shape}", flush=True)
    data = sparse_volume(np.random.default_rng(len(shape) + shape[1]), shape, boxes)
    bbox = torch.empty(6, dtype=torch.int32, device="cuda")
    _native.check(lib.nnx_nonzero_bbox(dev(data).data_ptr(), shape[0], _native.i64s(shape[1:]),
                                       bbox.data_ptr(), stream()))
    got = bbox.cpu().numpy().reshape(3, 2)
    want = op.nonzero_bbox(data)
    assert [(int(a), int(b) + 1) for a, b in got] == list(want)


def test_nonzero_bbox_empty(lib):
    data = np.zeros((1, 4, 5, 6), dtype=np.float32)
    bbox = torch.empty(6, dtype=torch.int32, device="cuda")
    _native.check(lib.nnx_nonzero_bbox(dev(data).data_ptr(), 1, _native.i64s((4, 5, 6)),
                                       bbox.data_ptr(), stream()))
    got = bbox.cpu().numpy().reshape(3, 2)
    assert (got[:, 1] == -1).all()


@pytest.mark.parametrize("transpose", list(itertools.permutations(range(3))))
def test_crop_normalize_exact(lib, transpose):
    print(f"crop/normalise transpose {transpose}", flush=True)
    rng = np.random.default_rng(sum(i * 3 ** k for k, i in enumerate(transpose)))
    raw = (rng.standard_normal((2, 11, 13, 7)) * 900).astype(np.float32)
    norm = np.array([[41.5, 60.25, -1000.0, 1500.0], [0, 0, 0, 0]], dtype=np.float32)
    schemes = [_native.NNX_NORM_CT, _native.NNX_NORM_NONE]
    tshape = tuple(raw.shape[1 + a] for a in transpose)
    start = (1, 2, 0)
    out_size = tuple(s - st - 1 for s, st in zip(tshape, start))
    out = torch.full((2, *out_size), float("nan"), device="cuda")
    _native.check(lib.nnx_crop_normalize(
        dev(raw).data_ptr(), 2, _native.i64s(raw.shape[1:]), _native.ints(transpose),
        _native.i64s(start), _native.i64s(out_size), _native.ints(schemes),
        norm.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), out.data_ptr(),
        stream()))
    t = raw.transpose((0, *(a + 1 for a in transpose)))
    crop = t[(slice(None), *(slice(s, s + n) for s, n in zip(start, out_size)))]
    want0 = op.ct_normalize(crop[0], 41.5, 60.25, -1000.0, 1500.0)
    got = out.cpu().numpy()
    np.testing.assert_array_equal(got[0], want0)
    np.testing.assert_array_equal(got[1], crop[1])


def spline_device(lib, data, new_shape, order=3, separate_axis=-1):
    size = data.shape[1:]
    work = lib.nnx_resample_spline_workspace(_native.i64s(size), _native.i64s(new_shape), separate_axis)
    assert work > 0
    buf = torch.empty(work, dtype=torch.uint8, device="cuda")
    out = torch.full((data.shape[0], *new_shape), float("nan"), device="cuda")
    _native.check(lib.nnx_resample_spline(dev(data).data_ptr(), data.shape[0], _native.i64s(size),
                                          _native.i64s(new_shape), order, separate_axis, 0,
                                          buf.data_ptr(), work, out.data_ptr(), stream()))
    return out.cpu().numpy()


def assert_one_rounding(got, want):
    """float32 results of the same float64 value: equal, or one float32 step apart where
    the two float64 evaluations straddle a rounding boundary."""
    assert got.shape == want.shape and np.isfinite(got).all()
    ulp = np.spacing(np.abs(want).astype(np.float32))
    diff = np.abs(got.astype(np.float64) - want.astype(np.float64))
    assert (diff <= ulp).all(), float((diff / np.maximum(ulp, 1e-45)).max())
    assert (got == want).mean() >= 0.999


SPLINE_CASES = [
    ((1, 20, 24, 18), (33, 17, 18), 3),
    ((2, 31, 12, 40), (19, 25, 57), 3),
    ((1, 9, 64, 64), (9, 101, 77), 3),
    ((1, 20, 24, 18), (33, 17, 29), 1),
]


def _random_spline_cases(seed, n):
    """Seeded grids: up- and downsampling per axis, 1-2 channels, orders 1 and 3."""
    rng = np.random.default_rng(seed)
    return [((int(rng.integers(1, 3)), *(int(v) for v in rng.integers(2, 31, 3))),
             tuple(int(v) for v in rng.integers(2, 41, 3)), int(rng.choice([1, 3])))
            for _ in range(n)]


@pytest.mark.parametrize("shape,new_shape,order", SPLINE_CASES + _random_spline_cases(2032, 6))
def test_resample_spline_whole_volume(lib, shape, new_shape, order):
    print(f"spline case {shape} -> {new_shape} order {order}", flush=True)
    rng = np.random.default_rng(shape[1] + new_shape[2])
    data = (rng.standard_normal(shape) * 3).astype(np.float32)
    got = spline_device(lib, data, new_shape, order)
    want = op.resample_data(data, new_shape, order=order)
    assert_one_rounding(got, want)
    # the clip keeps every channel inside its input range
    for c in range(shape[0]):
        assert got[c].min() >= data[c].min() and got[c].max() <= data[c].max()


@pytest.mark.parametrize("axis", [0, 1, 2])
def test_resample_spline_separate_axis(lib, axis):
    print(f"separate-axis spline case axis {axis}", flush=True)
    rng = np.random.default_rng(40 + axis)
    shape = (2, 11, 23, 19)
    new_shape = [30, 16, 27]
    new_shape[axis] = {0: 26, 1: 41, 2: 8}[axis]
    data = (rng.standard_normal(shape) * 5).astype(np.float32)
    got = spline_device(lib, data, tuple(new_shape), 3, axis)
    want = op.resample_data(data, tuple(new_shape), separate_axis=axis)
    assert_one_rounding(got, want)


def ct_plan(spacing, transpose=(0, 1, 2), resampling=None):
    plans = {
        "transpose_forward": list(transpose),
        "transpose_backward": [list(transpose).index(a) for a in range(3)],
        "foreground_intensity_properties_per_channel": {
            "0": {"mean": 99.4, "std": 137.2, "percentile_00_5": -958.0, "percentile_99_5": 327.0}},
        "configurations": {"3d_fullres": {
            "spacing": list(spacing), "normalization_schemes": ["CTNormalization"],
            "use_mask_for_norm": [False], "patch_size": [64, 64, 64],
            "resampling_fn_data": resampling or "resample_data_or_seg_to_shape",
            "resampling_fn_data_kwargs": {"is_seg": False, "order": 3, "order_z": 0,
                                          "force_separate_z": None}}},
    }
    return PreprocessPlan.from_plans(plans, "3d_fullres")


def oracle_case(raw, spacing, plan):
    forward = plan.transpose_forward
    t = raw.astype(np.float32).transpose((0, *(a + 1 for a in forward)))
    bbox = op.nonzero_bbox(t)
    crop = t[(slice(None), *(slice(a, b) for a, b in bbox))]
    st = plan.intensity_properties["0"]
    norm = op.ct_normalize(crop[0], st["mean"], st["std"], st["percentile_00_5"],
                           st["percentile_99_5"])[None]
    original = tuple(spacing[a] for a in forward)
    target = tuple(o if c is None else c for c, o in zip(plan.spacing, original))
    new_shape = tuple(round(o / n * s) for o, n, s in zip(original, target, crop.shape[1:]))
    ratio = max(original) / min(original)
    separate = None
    if ratio > 3 or max(target) / min(target) > 3:
        basis = original if ratio > 3 else target
        axes = [i for i, s in enumerate(basis) if max(basis) / s == 1]
        separate = axes[0] if len(axes) == 1 else None
    return bbox, op.resample_data(norm, new_shape, separate_axis=separate)


@pytest.mark.parametrize("spacing,target,transpose", [
    ((2.5, 0.8, 0.8), (1.0, 0.78, 0.78), (0, 1, 2)),      # anisotropic: separate axis 0
    ((0.7, 0.7, 1.6), (1.0, 1.0, 1.0), (2, 0, 1)),        # isotropic-enough, transposed
])
def test_preprocess_raw_case_matches_oracle(spacing, target, transpose):
    print(f"preprocess case spacing {spacing} target {target} transpose {transpose}", flush=True)
    rng = np.random.default_rng(7)
    raw = np.zeros((1, 24, 40, 36), dtype=np.int16)
    raw[0, 3:21, 5:37, 2:30] = (rng.standard_normal((18, 32, 28)) * 400 - 200).astype(np.int16)
    plan = ct_plan(target, transpose)
    out = preprocess_raw_case(raw, {"spacing": list(spacing)}, plan)
    bbox, want = oracle_case(raw, spacing, plan)
    assert out.properties["bbox_used_for_cropping"] == [list(b) for b in bbox]
    assert out.properties["shape_before_cropping"] == tuple(raw.shape[1 + a] for a in transpose)
    assert_one_rounding(out.data.cpu().numpy(), want)


def test_preprocess_rejects_unsupported():
    plan = ct_plan((1.0, 1.0, 1.0))
    with pytest.raises(ContractError):
        preprocess_raw_case(np.zeros((1, 4, 4, 4), dtype=np.float32), {"spacing": [1, 1, 1]}, plan)
    zplan = PreprocessPlan(plan.transpose_forward, plan.spacing, ("MyOwnNormalization",),
                           (False,), plan.intensity_properties, plan.data_resampling)
    with pytest.raises(ContractError):
        preprocess_raw_case(np.ones((1, 4, 4, 4), dtype=np.float32), {"spacing": [1, 1, 1]}, zplan)
    with pytest.raises(ContractError):   # cascade inputs stay off the device path
        preprocess_raw_case(np.ones((1, 8, 8, 8), dtype=np.float32), {"spacing": [1, 1, 1]}, plan,
                            segmentation_previous_stage=np.zeros((1, 8, 8, 8), dtype=np.int16))


def hollow_volume(rng, shape):
    """Random blobs plus a closed shell with a sealed cavity, a shell with a tunnel to the
    outside (not a hole), and a winding corridor that needs several sweep rounds."""
    data = np.zeros(shape, dtype=np.float32)
    z, y, x = np.indices(shape[1:])
    cz, cy, cx = (s // 2 for s in shape[1:])
    r = np.sqrt((z - cz) ** 2 + (y - cy) ** 2 + (x - cx) ** 2)
    shell = (r >= 4) & (r < 6)
    data[0][shell] = rng.standard_normal(int(shell.sum())) + 3
    open_shell = (np.abs(z - 3) <= 2) & (np.abs(y - 4) <= 3) & (np.abs(x - 4) <= 3)
    inner = (np.abs(z - 3) <= 1) & (np.abs(y - 4) <= 2) & (np.abs(x - 4) <= 2)
    data[-1][open_shell & ~inner] = 1.5
    data[-1][(np.abs(z - 3) <= 0) & (y == 4) & (x >= 4) & (x <= 7)] = 0   # tunnel out
    # serpentine wall: background corridor that turns several times, sealed at one end
    wall = np.zeros(shape[1:], dtype=bool)
    wall[:, -9:-1, -9:-1] = True
    for k, row in enumerate(range(-8, -2, 2)):
        wall[:, row, (-8 if k % 2 else -7):(-2 if k % 2 else -1)] = False
    data[0][wall] = 2.0
    return data


@pytest.mark.parametrize("shape", [(1, 18, 20, 22), (2, 24, 17, 30)])
def test_filled_nonzero_mask_matches_scipy(lib, shape):
    print(f"filled mask {shape}", flush=True)
    data = hollow_volume(np.random.default_rng(shape[1]), shape)
    bbox = op.nonzero_bbox(data)
    start = [a for a, _ in bbox]
    extent = [b - a for a, b in bbox]
    mask = torch.empty(extent, dtype=torch.uint8, device="cuda")
    flag = torch.empty(64, dtype=torch.int32, device="cuda")
    rounds = lib.nnx_nonzero_mask_filled(dev(data).data_ptr(), shape[0], _native.i64s(shape[1:]),
                                         _native.i64s(start), _native.i64s(extent),
                                         mask.data_ptr(), flag.data_ptr(), stream())
    assert rounds >= 1
    want = op.filled_nonzero_mask(data)[tuple(slice(a, b) for a, b in bbox)]
    np.testing.assert_array_equal(mask.cpu().numpy().astype(bool), want)


@pytest.mark.parametrize("use_mask", [False, True])
def test_zscore_stats_are_float64_statistics_rounded(lib, use_mask):
    rng = np.random.default_rng(9)
    shape = (2, 30, 40, 50)
    data = hollow_volume(rng, shape)
    data[1] += (rng.standard_normal(shape[1:]) * 50 + 100).astype(np.float32) * (data[1] != 0)
    bbox = op.nonzero_bbox(data)
    start, extent = [a for a, _ in bbox], [b - a for a, b in bbox]
    crop = data[(slice(None), *(slice(a, b) for a, b in bbox))]
    mask_np = op.filled_nonzero_mask(data)[tuple(slice(a, b) for a, b in bbox)]
    mask = torch.from_numpy(mask_np.astype(np.uint8)).cuda() if use_mask else None
    work = torch.empty(lib.nnx_zscore_stats_workspace(), dtype=torch.uint8, device="cuda")
    for c in range(2):
        stats = torch.empty(2, dtype=torch.float32, device="cuda")
        _native.check(lib.nnx_zscore_stats(dev(data).data_ptr(), 2, _native.i64s(shape[1:]), c,
                                           _native.i64s(start), _native.i64s(extent),
                                           mask.data_ptr() if use_mask else None,
                                           stats.data_ptr(), work.data_ptr(), stream()))
        sel = crop[c][mask_np] if use_mask else crop[c].ravel()
        mean32 = np.float32(sel.astype(np.float64).mean())
        std32 = np.float32(np.sqrt(((sel.astype(np.float64) - np.float64(mean32)) ** 2).mean()))
        got = stats.cpu().numpy()
        assert abs(got[0] - mean32) <= np.spacing(abs(mean32))
        assert abs(got[1] - std32) <= np.spacing(std32)
        # numpy's own float32 statistics (the reference's) lie within a few float32 steps
        assert abs(got[0] - sel.mean()) <= 8 * np.spacing(max(abs(mean32), std32))
        assert abs(got[1] - sel.std()) <= 8 * np.spacing(std32)


@pytest.mark.parametrize("use_mask", [False, True])
def test_preprocess_zscore_case_matches_oracle(use_mask):
    print(f"z-score case use_mask={use_mask}", flush=True)
    rng = np.random.default_rng(21)
    raw = hollow_volume(rng, (2, 20, 28, 26))
    raw[1] = raw[1] * 40 + (raw[1] != 0) * 300
    plans = {
        "transpose_forward": [2, 0, 1], "transpose_backward": [1, 2, 0],
        "configurations": {"3d_fullres": {
            "spacing": [1.0, 1.0, 1.0],
            "normalization_schemes": ["ZScoreNormalization", "ZScoreNormalization"],
            "use_mask_for_norm": [use_mask, use_mask], "patch_size": [16, 16, 16],
            "resampling_fn_data": "resample_data_or_seg_to_shape",
            "resampling_fn_data_kwargs": {"is_seg": False, "order": 3, "order_z": 0,
                                          "force_separate_z": None}}},
    }
    plan = PreprocessPlan.from_plans(plans, "3d_fullres")
    spacing = (1.3, 0.9, 1.1)
    out = preprocess_raw_case(raw, {"spacing": list(spacing)}, plan)
    forward = (2, 0, 1)
    t = raw.transpose((0, *(a + 1 for a in forward)))
    bbox = op.nonzero_bbox(t)
    sl = tuple(slice(a, b) for a, b in bbox)
    crop = t[(slice(None), *sl)]
    mask = op.filled_nonzero_mask(t)[sl] if use_mask else None
    norm = np.stack([op.zscore_normalize(crop[c], mask) for c in range(2)])
    original = tuple(spacing[a] for a in forward)
    new_shape = tuple(round(o / 1.0 * s) for o, s in zip(original, crop.shape[1:]))
    want = op.resample_data(norm, new_shape)
    got = out.data.cpu().numpy()
    assert got.shape == want.shape
    np.testing.assert_allclose(got, want, rtol=2e-5, atol=2e-5)


def test_preprocess_rescale_and_rgb_match_oracle():
    print("rescale01 / rgb01 case", flush=True)
    rng = np.random.default_rng(31)
    raw = np.zeros((2, 14, 18, 16), dtype=np.float32)
    raw[0, 2:12, 3:15, 1:14] = rng.standard_normal((10, 12, 13)).astype(np.float32) * 70 + 20
    raw[1, 2:12, 3:15, 1:14] = rng.integers(0, 256, (10, 12, 13)).astype(np.float32)
    plans = {
        "transpose_forward": [0, 1, 2], "transpose_backward": [0, 1, 2],
        "configurations": {"3d_fullres": {
            "spacing": [1.0, 1.0, 1.0],
            "normalization_schemes": ["RescaleTo01Normalization", "RGBTo01Normalization"],
            "use_mask_for_norm": [False, False], "patch_size": [16, 16, 16],
            "resampling_fn_data": "resample_data_or_seg_to_shape",
            "resampling_fn_data_kwargs": {"is_seg": False, "order": 3, "order_z": 0,
                                          "force_separate_z": None}}},
    }
    plan = PreprocessPlan.from_plans(plans, "3d_fullres")
    out = preprocess_raw_case(raw, {"spacing": [1.0, 1.0, 1.0]}, plan)
    bbox = op.nonzero_bbox(raw)
    crop = raw[(slice(None), *(slice(a, b) for a, b in bbox))]
    want = np.stack([op.rescale01_normalize(crop[0]), op.rgb01_normalize(crop[1])])
    np.testing.assert_array_equal(out.data.cpu().numpy(), want)
    bad = raw.copy()
    bad[1, 5, 5, 5] = 300.0
    with pytest.raises(ContractError, match="RGB"):
        preprocess_raw_case(bad, {"spacing": [1.0, 1.0, 1.0]}, plan)
