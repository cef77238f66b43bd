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


@pytest.mark.parametrize("source,target,classes", CASES, ids=str)
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
