"""GPU sliding window vs the numpy oracle.

With a pointwise fake network (the reference's PointwiseModel, tests/test_sliding_window.py:20-28
of the reference) every float operation of the pipeline is reproducible on the CPU, so
logits and labels must match the oracle bit for bit — padding, tile order, mirror
order, Gaussian weights, float32/float16 accumulation, fold averaging and argmax.  With
the real network the logits follow the fp32 parity bar.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from nnunet_mlx.errors import ContractError
from nnunet_mlx.model.network import build_network
from nnunet_mlx.model.topology import PlainConvUNetSpec
from nnunet_mlx.prediction import sliding_window as sw
from nnunet_mlx.storage.synthetic import random_weights
from oracle import sliding_window as osw
from oracle.network import OracleNetwork
from tests.helpers import rel_l2, report

pytestmark = pytest.mark.gpu


class TorchPointwise:
    def __init__(self, scale: float) -> None:
        self.scale = scale

    def __call__(self, values: torch.Tensor) -> torch.Tensor:
        return torch.cat((values * self.scale, -values * self.scale), dim=-1)


class NumpyPointwise:
    def __init__(self, scale: float) -> None:
        self.scale = np.float32(scale)

    def __call__(self, values: np.ndarray) -> np.ndarray:
        return np.concatenate((values * self.scale, -values * self.scale), axis=-1)


POINTWISE_CASES = [
    # shape (C, Z, Y, X), patch, axes, accumulation, fold scales
    ((1, 12, 20, 18), (8, 8, 8), (0, 1, 2), "float32", (1.0,)),
    ((2, 5, 9, 17), (8, 8, 8), (1, 2), "float32", (1.0, 0.7)),
    ((1, 12, 20, 18), (8, 8, 8), (0, 1, 2), "nnunet-fp16", (1.0,)),
    ((1, 9, 7, 22), (6, 8, 8), (0,), "nnunet-fp16", (1.0, 0.7, 1.3)),
    ((1, 16, 16, 16), (16, 16, 16), (), "float32", (0.5,)),
]


def _random_pointwise_cases(seed, n):
    """Seeded volumes (some smaller than the patch on an axis), patches, mirror-axis subsets,
    accumulations and fold counts."""
    rng = np.random.default_rng(seed)
    cases = []
    for _ in range(n):
        shape = (int(rng.integers(1, 4)), *(int(v) for v in rng.integers(1, 31, 3)))
        patch = tuple(int(v) for v in rng.integers(1, 17, 3))
        axes = tuple(a for a in range(3) if rng.random() < 0.5)
        accumulation = str(rng.choice(["float32", "nnunet-fp16"]))
        scales = tuple(float(v) for v in np.round(rng.uniform(0.3, 1.5, int(rng.integers(1, 4))), 2))
        cases.append((shape, patch, axes, accumulation, scales))
    return cases


@pytest.mark.parametrize("case", POINTWISE_CASES + _random_pointwise_cases(2031, 10), ids=str)
def test_pointwise_pipeline_bitwise(device, case):
    shape, patch, axes, accumulation, scales = case
    print(f"pointwise case {case}", flush=True)
    rng = np.random.default_rng(21)
    data = rng.standard_normal(shape).astype(np.float32)
    models = [TorchPointwise(s) for s in scales]
    classes = 2 * shape[0]
    logits = sw.average_fold_device_logits(
        models, data, patch_size=patch, num_outputs=classes, mirroring_axes=axes,
        accumulation=accumulation).cpu().numpy()
    labels = sw.average_fold_labels(
        models, data, patch_size=patch, num_outputs=classes, mirroring_axes=axes,
        accumulation=accumulation)
    ref_logits, ref_labels = osw.predict(
        [NumpyPointwise(s) for s in scales], data, patch, num_classes=classes, axes=axes,
        accumulation=accumulation)
    np.testing.assert_array_equal(logits, ref_logits)
    np.testing.assert_array_equal(labels, ref_labels)


def test_pointwise_mirrored_average_equals_model(device):
    """A pointwise model commutes with flips: the 8-view average equals the model itself
    up to the rounding of the float32 sum (known answer independent of the oracle)."""
    data = np.random.default_rng(3).standard_normal((1, 10, 12, 14)).astype(np.float32)
    logits = sw.predict_logits(TorchPointwise(1.0), data, patch_size=(8, 8, 8), num_classes=2,
                               mirroring_axes=(0, 1, 2))
    np.testing.assert_allclose(logits[0], data[0], rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(logits[1], -data[0], rtol=1e-6, atol=1e-6)


def test_rejects_nonfinite_input_and_bad_requests(device):
    data = np.zeros((1, 8, 8, 8), dtype=np.float32)
    data[0, 1, 2, 3] = np.nan
    with pytest.raises(ContractError):
        sw.predict_logits(TorchPointwise(1.0), data, patch_size=(8, 8, 8), num_classes=2)
    good = np.zeros((1, 8, 8, 8), dtype=np.float32)
    with pytest.raises(ContractError):
        sw.predict_logits(TorchPointwise(1.0), good, patch_size=(8, 8, 8), num_classes=2,
                          mirroring_axes=(0, 0))
    with pytest.raises(ContractError):
        sw.predict_logits(TorchPointwise(1.0), good, patch_size=(8, 8, 8), num_classes=2,
                          accumulation="bfloat16")
    with pytest.raises(ContractError):
        sw.predict_logits(TorchPointwise(1.0), good.astype(np.float64), patch_size=(8, 8, 8),
                          num_classes=2)


def test_nonfinite_logits_raise(device):
    class Exploding:
        def __call__(self, values):
            out = torch.cat((values, -values), dim=-1)
            out[0, 0, 0, 0, 0] = float("inf")
            return out

    data = np.ones((1, 8, 8, 8), dtype=np.float32)
    with pytest.raises(ContractError, match="non-finite"):
        sw.predict_labels(Exploding(), data, patch_size=(8, 8, 8), num_classes=2)


def _small_net(seed: int, cin=1, classes=3):
    spec = PlainConvUNetSpec(cin, classes, (8, 16, 32), ((3, 3, 3),) * 3,
                             ((1, 1, 1), (2, 2, 2), (2, 2, 2)), (2, 2, 2), (2, 2))
    weights = random_weights(spec, seed=seed, random_affine=True)
    net = build_network(spec)
    net.load_weights(weights)
    return spec, net, OracleNetwork(spec, weights)


@pytest.mark.parametrize("accumulation", ["float32", "nnunet-fp16"])
def test_network_pipeline_matches_oracle(device, accumulation):
    spec, net, oracle_net = _small_net(4)
    _, net2, oracle_net2 = _small_net(5)
    net2.share_workspace(net)
    data = np.random.default_rng(2).standard_normal((1, 14, 30, 26)).astype(np.float32)
    patch = (16, 16, 16)
    logits = sw.average_fold_device_logits(
        (net, net2), data, patch_size=patch, num_outputs=3, mirroring_axes=(0, 1, 2),
        accumulation=accumulation).cpu().numpy().astype(np.float32)
    ref, ref_labels = osw.predict([oracle_net, oracle_net2], data, patch, num_classes=3,
                                  axes=(0, 1, 2), accumulation=accumulation)
    ref = ref.astype(np.float32)
    msg = report(accumulation, logits, ref)
    print(msg, flush=True)
    if accumulation == "float32":
        assert np.abs(logits - ref).max() <= 1e-3, msg
        assert rel_l2(logits, ref) <= 1e-5, msg
    else:
        assert rel_l2(logits, ref) <= 1e-3, msg
    labels = sw.average_fold_labels((net, net2), data, patch_size=patch, num_outputs=3,
                                    mirroring_axes=(0, 1, 2), accumulation=accumulation)
    assert (labels == ref_labels).mean() >= 0.9999


def test_native_loop_equals_python_loop(device):
    """The C++ tile loop (nnx_sw_predict) and the Python-driven loop over the same kernels
    give identical bits."""
    _, net, _ = _small_net(6)
    data = np.random.default_rng(4).standard_normal((1, 20, 18, 24)).astype(np.float32)
    kwargs = dict(patch_size=(16, 16, 16), num_outputs=3, mirroring_axes=(0, 2))
    native = sw.average_fold_device_logits((net,), data, **kwargs).cpu().numpy()
    wrapped = sw.average_fold_device_logits((lambda t: net(t),), data, **kwargs).cpu().numpy()
    np.testing.assert_array_equal(native, wrapped)
