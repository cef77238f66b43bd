"""Fold ensembles, probability/label heads and ``ArrayPredictor`` on the HIP path.

Reference: src/nnunet_mlx/prediction/inference.py:25-339.  Fold logits are produced and
averaged on the GPU (``average_fold_device_logits``); the host variant returns the
same values channel-first.  The softmax/sigmoid heads and region decoding are host
numpy functions with the reference's arithmetic (they run once per case on the final
logits).
"""

from __future__ import annotations

from collections.abc import Sequence

import numpy as np

from nnunet_mlx.errors import ContractError
from nnunet_mlx.prediction import sliding_window


def average_fold_device_logits(models, data_channels_first, *, patch_size: Sequence[int],
                               num_outputs: int, mirroring_axes: Sequence[int] = (),
                               step_fraction: float = 0.5, accumulation: str = "float32",
                               tiles_per_batch: int | None = None):
    """Fold-averaged channels-last ``(*spatial, C)`` logits on the GPU (inference.py:93-149)."""
    if not models:
        raise ContractError("fold inference requires at least one model")
    if len(patch_size) != 3:
        raise ContractError("device fold averaging requires a three-dimensional patch")
    return sliding_window.average_fold_device_logits(
        tuple(models), data_channels_first, patch_size=patch_size, num_outputs=num_outputs,
        mirroring_axes=mirroring_axes, step_fraction=step_fraction, accumulation=accumulation,
        tiles_per_batch=tiles_per_batch,
    )


def average_fold_logits(models, data_channels_first, *, patch_size: Sequence[int], num_outputs: int,
                        mirroring_axes: Sequence[int] = (), step_fraction: float = 0.5,
                        accumulation: str = "float32", tiles_per_batch: int | None = None):
    """Host channel-first fold-averaged logits: float16 for nnunet-fp16, else float32.

    The fold sum and division run on the GPU with the device ensemble's arithmetic
    (sum in the accumulation dtype, divide in float32, round back).
    """
    logits = average_fold_device_logits(
        models, data_channels_first, patch_size=patch_size, num_outputs=num_outputs,
        mirroring_axes=mirroring_axes, step_fraction=step_fraction, accumulation=accumulation,
        tiles_per_batch=tiles_per_batch,
    )
    host = np.ascontiguousarray(np.moveaxis(logits.cpu().numpy(), -1, 0))
    if not np.isfinite(host).all():
        raise ContractError("fold averaging produced non-finite logits")
    return host


def device_logits_to_host(logits) -> np.ndarray:
    """Channels-last device logits -> channel-first host logits, dtype kept."""
    return np.ascontiguousarray(np.moveaxis(logits.cpu().numpy(), -1, 0))


def logits_to_probabilities(logits: np.ndarray, *, has_regions: bool) -> np.ndarray:
    """Softmax over axis 0 (class models) or independent sigmoids (region models)
    of finite channel-first logits, float32 (inference.py:210-233)."""
    values = np.asarray(logits, dtype=np.float32)
    if values.ndim not in (3, 4) or not np.isfinite(values).all():
        raise ContractError(f"expected finite channel-first 2-D/3-D logits, got {values.shape}")
    if has_regions:
        probabilities = np.empty_like(values)
        positive = values >= 0
        probabilities[positive] = 1 / (1 + np.exp(-values[positive]))
        exponent = np.exp(values[~positive])
        probabilities[~positive] = exponent / (1 + exponent)
    else:
        probabilities = np.empty_like(values, order="K")
        np.subtract(values, np.max(values, axis=0, keepdims=True), out=probabilities)
        np.exp(probabilities, out=probabilities)
        np.divide(probabilities, np.sum(probabilities, axis=0, keepdims=True), out=probabilities)
    return np.ascontiguousarray(probabilities, dtype=np.float32)


def probabilities_to_segmentation(probabilities: np.ndarray, *,
                                  regions_class_order: Sequence[int] | None) -> np.ndarray:
    """Axis-0 argmax (class models) or ordered region overwrite at > 0.5, uint16
    (inference.py:246-269)."""
    values = np.asarray(probabilities, dtype=np.float32)
    if values.ndim not in (3, 4) or not np.isfinite(values).all():
        raise ContractError(f"expected finite channel-first 2-D/3-D probabilities, got {values.shape}")
    if regions_class_order is None:
        return np.asarray(np.argmax(values, axis=0), dtype=np.uint16)
    order = tuple(int(v) for v in regions_class_order)
    if len(order) != values.shape[0] or any(v < 1 for v in order):
        raise ContractError("regions_class_order does not match output channels")
    segmentation = np.zeros(values.shape[1:], dtype=np.uint16)
    for channel, label in enumerate(order):
        segmentation[values[channel] > 0.5] = label
    return segmentation


class ArrayPredictor:
    """Predict from preprocessed ``(C, *spatial)`` arrays with a fold ensemble
    (inference.py:280-339); method names follow upstream's ``nnUNetPredictor``."""

    def __init__(self, models, *, patch_size: Sequence[int], num_outputs: int,
                 mirroring_axes: Sequence[int] = (), regions_class_order: Sequence[int] | None = None,
                 step_fraction: float = 0.5, accumulation: str = "float32") -> None:
        if regions_class_order is None and num_outputs < 2:
            raise ContractError("class inference requires at least two output channels")
        if not models:
            raise ContractError("predictor requires at least one fold model")
        self.models = tuple(models)
        self.patch_size = tuple(int(v) for v in patch_size)
        self.num_outputs = num_outputs
        self.mirroring_axes = tuple(int(a) for a in mirroring_axes)
        self.regions_class_order = regions_class_order
        self.step_fraction = step_fraction
        self.accumulation = accumulation

    def _kwargs(self) -> dict[str, object]:
        return dict(patch_size=self.patch_size, num_outputs=self.num_outputs,
                    mirroring_axes=self.mirroring_axes, step_fraction=self.step_fraction,
                    accumulation=self.accumulation)

    def predict_logits_from_preprocessed_data(self, data_channels_first) -> np.ndarray:
        return average_fold_logits(self.models, data_channels_first, **self._kwargs())

    def predict_device_logits_from_preprocessed_data(self, data_channels_first):
        return average_fold_device_logits(self.models, data_channels_first, **self._kwargs())

    def predict_labels_from_preprocessed_data(self, data_channels_first) -> np.ndarray:
        """uint16 argmax labels of the fold average; only labels leave the GPU."""
        if self.regions_class_order is not None:
            raise ContractError("label-only inference requires a class-based model")
        return sliding_window.average_fold_labels(self.models, data_channels_first, **self._kwargs())
