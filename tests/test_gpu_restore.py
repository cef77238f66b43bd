"""Device restoration of class logits (half-pixel trilinear in float64 + argmax) against
the oracle: labels bit-identical."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from nnunet_mlx.prediction.restore import (
    resample_class_logits_argmax_device,
    resample_device_logits_argmax,
)
from nnunet_mlx.plans import ResamplingContract
from oracle.restore import restore_labels

pytestmark = pytest.mark.gpu

CASES = [
    ((5, 7, 6), (9, 4, 6), 3),      # up / down / identity per axis
    ((3, 4, 5), (3, 4, 5), 4),      # identity: first-maximum argmax
    ((1, 6, 3), (4, 2, 7), 2),      # a size-1 source axis
    ((8, 8, 8), (3, 11, 5), 5),
    ((16, 40, 36), (21, 31, 50), 3),
    ((24, 64, 48), (24, 96, 72), 14),
]


def _random_cases(seed, n):
    """Seeded source and target grids (size-1 axes included) and class counts."""
    rng = np.random.default_rng(seed)
    return [(tuple(int(v) for v in rng.integers(1, 21, 3)), tuple(int(v) for v in rng.integers(1, 31, 3)),
             int(rng.integers(1, 9))) for _ in range(n)]


@pytest.mark.parametrize("source,target,classes", CASES + _random_cases(2030, 8), ids=str)
@pytest.mark.parametrize("dtype", [np.float32, np.float16], ids=["f32", "f16"])
def test_restore_labels_match_oracle(device, source, target, classes, dtype):
    print(f"restore {source} -> {target} K={classes} {np.dtype(dtype).name}", flush=True)
    rng = np.random.default_rng(sum(source) + classes)
    logits = (rng.standard_normal((*source, classes)) * 4).astype(dtype)
    got = resample_class_logits_argmax_device(torch.from_numpy(logits).to(device), target)
    got = got.cpu().numpy().view(np.uint16)
    ref = restore_labels(logits, target)
    assert got.shape == tuple(target)
    np.testing.assert_array_equal(got, ref)


def test_restore_ties_keep_the_earliest_class(device):
    """Integer logits tie often; identity and 2x downsampling (weights 0.5/0.5)."""
    logits = np.random.default_rng(3).integers(-2, 3, (6, 8, 10, 4)).astype(np.float32)
    for target in ((6, 8, 10), (3, 4, 5)):
        got = resample_class_logits_argmax_device(torch.from_numpy(logits).to(device), target)
        np.testing.assert_array_equal(got.cpu().numpy().view(np.uint16), restore_labels(logits, target))


def test_restore_float16_rounds_half_to_even(device):
    """Downsampling by 2 along x averages two fp16 values (weights 0.5, 0.5): class 1
    lands exactly halfway between two fp16 neighbours and must round to the even one."""
    one, ulp = 1.0, 2.0**-10
    logits = np.zeros((1, 1, 2, 2), dtype=np.float16)
    logits[0, 0, :, 0] = one + ulp                 # class 0: exactly 1 + ulp
    logits[0, 0, :, 1] = [one + ulp, one + 2 * ulp]  # class 1: 1 + 1.5 ulp -> 1 + 2 ulp (even)
    got = resample_class_logits_argmax_device(torch.from_numpy(logits).to(device), (1, 1, 1))
    assert int(got.cpu().numpy().view(np.uint16)[0, 0, 0]) == 1
    logits[0, 0, :, 1] = [one, one + ulp]          # class 1: 1 + 0.5 ulp -> 1 (even) < class 0
    got = resample_class_logits_argmax_device(torch.from_numpy(logits).to(device), (1, 1, 1))
    assert int(got.cpu().numpy().view(np.uint16)[0, 0, 0]) == 0
    np.testing.assert_array_equal(restore_labels(logits, (1, 1, 1)), [[[0]]])


def test_restore_policy_dispatch(device):
    order1 = ResamplingContract("resample_data_or_seg_to_shape", 1, 0, False)
    order3 = ResamplingContract("resample_data_or_seg_to_shape", 3, 0, False)
    logits = torch.randn((6, 8, 10, 3), device=device)
    labels = resample_device_logits_argmax(logits, (7, 9, 12), (1.0, 1.0, 1.0), (0.9, 0.9, 0.8), order1)
    np.testing.assert_array_equal(labels, restore_labels(logits.cpu().numpy(), (7, 9, 12)))
    # cubic splines are host-only; equal shapes need only the argmax whatever the policy
    assert resample_device_logits_argmax(logits, (7, 9, 12), (1, 1, 1), (1, 1, 1), order3) is None
    same = resample_device_logits_argmax(logits, (6, 8, 10), (1, 1, 1), (1, 1, 1), order3)
    np.testing.assert_array_equal(same, logits.cpu().numpy().argmax(-1))
    # anisotropic spacing selects separate-axis resampling (when not forced off): host-only
    auto = ResamplingContract("resample_data_or_seg_to_shape", 1, 0, None)
    assert resample_device_logits_argmax(logits, (7, 9, 12), (4.0, 1.0, 1.0), (4.0, 1.0, 1.0),
                                         auto) is None
    assert resample_device_logits_argmax(logits, (7, 9, 12), (4.0, 1.0, 1.0), (4.0, 1.0, 1.0),
                                         order1) is not None


SPLINE_CASES = [
    ((5, 9, 7), (12, 6, 11), 3, 1, 0),        # separate axis 0, upsampled along it
    ((11, 6, 9), (7, 13, 9), 4, 1, 1),        # separate axis 1, downsampled along it
    ((8, 10, 5), (16, 12, 3), 2, 1, 2),
    ((6, 7, 8), (9, 5, 12), 3, 3, None),      # order 3, whole volume
    ((6, 20, 18), (15, 31, 27), 3, 3, 0),     # order 3 in-plane, separate axis 0
    ((24, 40, 40), (60, 52, 52), 3, 1, 0),    # liver-like anisotropic restoration
]


def near_tie(values, got, ref, dtype):
    """Voxels where the device and oracle winners differ by at most one rounding step of
    the logits' precision (both evaluate the same float64 sum; one rounding may differ)."""
    flat = values.reshape(values.shape[0], -1)
    g, r = got.reshape(-1).astype(np.int64), ref.reshape(-1).astype(np.int64)
    idx = np.nonzero(g != r)[0]
    a, b = flat[g[idx], idx], flat[r[idx], idx]
    step = np.spacing(np.abs(b).astype(dtype)).astype(np.float32)
    return bool((np.abs(a - b) <= step).all())


@pytest.mark.parametrize("source,target,classes,order,axis", SPLINE_CASES, ids=str)
@pytest.mark.parametrize("dtype", [np.float32, np.float16], ids=["f32", "f16"])
def test_spline_restore_labels_match_oracle(device, source, target, classes, order, axis, dtype):
    from nnunet_mlx.prediction.restore import resample_class_logits_argmax_spline_device
    from oracle.restore import restore_labels_spline

    print(f"spline restore {source} -> {target} K={classes} order {order} axis {axis} "
          f"{np.dtype(dtype).name}", flush=True)
    rng = np.random.default_rng(sum(source) + 7 * classes + order)
    logits = (rng.standard_normal((*source, classes)) * 3).astype(dtype)
    got = resample_class_logits_argmax_spline_device(torch.from_numpy(logits).to(device), target,
                                                     order=order, separate_axis=axis)
    got = got.cpu().numpy().view(np.uint16)
    ref, values = restore_labels_spline(logits, target, order=order, separate_axis=axis)
    assert got.shape == tuple(target)
    assert (got == ref).mean() >= 0.9999
    assert near_tie(values, got, ref, dtype)


def test_restore_class_labels_device_policy(device):
    """Separate-axis plans restore on the device through the spline entry; the trilinear
    entry keeps the cases the reference's fused path takes; Torch plans run the Torch-grid
    entries; spline plans with order_z above 0 return None."""
    from nnunet_mlx.prediction.restore import restore_class_labels_device
    from oracle import torch_resample as otr
    from oracle.restore import restore_labels_spline

    rng = np.random.default_rng(11)
    logits = rng.standard_normal((10, 16, 16, 3)).astype(np.float32)
    dev = torch.from_numpy(logits).to(device)
    spline = ResamplingContract("resample_data_or_seg_to_shape", 1, 0, None)
    # 2.5 mm slices -> 1 mm: anisotropic, separate axis 0
    got = restore_class_labels_device(dev, (25, 20, 20), (2.5, 0.8, 0.8), (1.0, 0.64, 0.64), spline)
    ref, _ = restore_labels_spline(logits, (25, 20, 20), order=1, separate_axis=0)
    assert (got.cpu().numpy().view(np.uint16) == ref).mean() >= 0.9999
    got = restore_class_labels_device(dev, (12, 20, 20), (1.0, 1.0, 1.0), (0.8, 0.8, 0.8), spline)
    np.testing.assert_array_equal(got.cpu().numpy().view(np.uint16), restore_labels(logits, (12, 20, 20)))
    torch_plan = ResamplingContract("resample_torch_fornnunet", 1, 0, None)
    got = restore_class_labels_device(dev, (12, 20, 20), (1.0, 1.0, 1.0), (0.8, 0.8, 0.8),
                                      torch_plan)
    want = otr.resample(np.moveaxis(logits, -1, 0), (12, 20, 20), axis=None).argmax(axis=0)
    np.testing.assert_array_equal(got.cpu().numpy().view(np.uint16), want)
    order_z1 = ResamplingContract("resample_data_or_seg_to_shape", 1, 1, None)
    assert restore_class_labels_device(dev, (25, 20, 20), (2.5, 0.8, 0.8), (1.0, 0.64, 0.64),
                                       order_z1) is None
