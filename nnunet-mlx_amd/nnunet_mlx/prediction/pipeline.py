"""Raw case -> label image with every compute step on the GPU.

Reference: ``ModelFolderPredictor`` (src/nnunet_mlx/prediction/pipeline.py:171-449,
696-742) with its preprocessing hand-off (src/nnunet_mlx/prediction/io.py:78-128) and the
label restoration of ``restore_device_segmentation`` / ``restore_prediction``
(src/nnunet_mlx/prediction/export.py:265-373, src/nnunet_mlx/prediction/restore.py:28-158).

One case flows: read the channel images (host) -> ``preprocess_raw_case`` (transpose, crop
to nonzero, normalisation, spline or Torch-grid resampling; HIP) -> fold-averaged sliding-window
logits (HIP, left on the device) -> class-logit restoration to the cropped original grid
with the first-maximum argmax (HIP) -> uint16 labels to the host -> uncrop and inverse
transpose -> label image with the input's geometry.  Only the raw volume goes to the
device and only the labels come back.  Class-label models only (region models and
probability export are not on this path).
"""

from __future__ import annotations

import re
from collections.abc import Mapping, Sequence
from dataclasses import dataclass, field
from pathlib import Path
from time import perf_counter

import numpy as np

from nnunet_mlx.errors import ContractError
from nnunet_mlx.plans import ResamplingContract, resolve_configuration

ACCUMULATIONS = ("float32", "nnunet-fp16")


@dataclass(frozen=True)
class CasePrediction:
    """Result of one case: the written label image (or None), the raw-grid labels, the
    preprocessed shape and per-stage wall times in seconds."""

    files: tuple[Path, ...]
    segmentation: np.ndarray
    preprocessed_shape: tuple[int, ...]
    metrics: dict[str, float] = field(default_factory=dict)
    decoding: str = "argmax-logits"


def _spacings(properties: Mapping[str, object], plan_spacing: Sequence[float | None],
              transpose_forward: Sequence[int]) -> tuple[tuple[float, ...], tuple[float, ...]]:
    """(spacing of the predicted logits, spacing of the cropped image), both in the plans'
    axis order (src/nnunet_mlx/prediction/export.py:418-446)."""
    spacing = properties.get("spacing")
    if not isinstance(spacing, (list, tuple)) or len(spacing) != 3:
        raise ContractError("prediction properties spacing must contain three values")
    transposed = tuple(float(spacing[a]) for a in transpose_forward)
    configured = (tuple(plan_spacing) if len(plan_spacing) == 3
                  else (transposed[0], *plan_spacing))
    current = tuple(o if c is None else float(c) for c, o in zip(configured, transposed))
    return current, transposed


def uncrop_segmentation(cropped: np.ndarray, shape_before: Sequence[int],
                        bbox: Sequence[Sequence[int]],
                        transpose_backward: Sequence[int]) -> np.ndarray:
    """Place cropped labels into zeros of ``shape_before`` at ``bbox`` and return them in
    the raw image's axis order (src/nnunet_mlx/prediction/export.py:359-370)."""
    shape_before = tuple(int(s) for s in shape_before)
    window = tuple(slice(int(a), int(b)) for a, b in bbox)
    if len(window) != 3 or tuple(s.stop - s.start for s in window) != cropped.shape:
        raise ContractError("cropped segmentation does not fit its bounding box")
    if any(s.start < 0 or s.stop > n for s, n in zip(window, shape_before)):
        raise ContractError("bounding box lies outside the uncropped shape")
    segmentation = np.zeros(shape_before, dtype=np.uint16)
    segmentation[window] = cropped
    return np.ascontiguousarray(segmentation.transpose(tuple(transpose_backward)))


class ModelFolderPredictor:
    """Predicts raw cases with a loaded model bundle (``nnunet_mlx.model.folder``).

    ``accumulation``: ``"float32"`` (the default of direct Python use) or
    ``"nnunet-fp16"`` (what the runners and the CLI use, as nnU-Net v2.8.1 does).
    """

    def __init__(self, bundle, *, step_fraction: float = 0.5, accumulation: str = "float32",
                 tiles_per_batch: int | None = None) -> None:
        from nnunet_mlx.data.preprocessing import PreprocessPlan

        if accumulation not in ACCUMULATIONS:
            raise ContractError(f"unsupported accumulation {accumulation!r}")
        if isinstance(step_fraction, bool) or not 0 < float(step_fraction) <= 1:
            raise ContractError("step_fraction must be in (0, 1]")
        if bundle.dataset_json.get("regions_class_order") is not None:
            raise ContractError("region-based models are not supported on the device case path")
        if len(bundle.patch_size) != 3:
            raise ContractError("the device case path runs 3-D configurations")
        self.bundle = bundle
        self.step_fraction = float(step_fraction)
        self.accumulation = accumulation
        self.tiles_per_batch = tiles_per_batch
        self.plan = PreprocessPlan.from_plans(bundle.plans, bundle.configuration)
        resolved = resolve_configuration(bundle.plans, bundle.configuration)
        self.probability_resampling = ResamplingContract.from_configuration(
            resolved, field="resampling_fn_probabilities", expected_is_seg=False)
        backward = bundle.plans.get("transpose_backward")
        forward = self.plan.transpose_forward
        self.transpose_backward = (tuple(int(a) for a in backward) if backward is not None
                                   else tuple(list(forward).index(a) for a in range(3)))

    @property
    def models(self):
        return self.bundle.models

    def predict_raw(self, data, properties: Mapping[str, object]) -> tuple[np.ndarray, dict]:
        """(C, Z, Y, X) raw channels + ``properties["spacing"]`` -> ((Z, Y, X) uint16
        labels on the raw grid, details with the preprocessed shape and stage times)."""
        import torch

        from nnunet_mlx.data.preprocessing import preprocess_raw_case
        from nnunet_mlx.prediction.restore import restore_class_labels_device
        from nnunet_mlx.prediction.sliding_window import average_fold_device_logits

        bundle = self.bundle
        channels = int(data.shape[0]) if getattr(data, "ndim", 0) == 4 else None
        if channels != bundle.image_channels:
            raise ContractError(f"the model expects (C, Z, Y, X) input with "
                                f"{bundle.image_channels} channels, got {channels}")
        times: dict[str, float] = {}
        start = perf_counter()
        case = preprocess_raw_case(data, properties, self.plan)
        torch.cuda.synchronize()
        times["preprocess_s"] = perf_counter() - start
        start = perf_counter()
        logits = average_fold_device_logits(
            bundle.models, case.data, patch_size=bundle.patch_size,
            num_outputs=bundle.num_outputs, mirroring_axes=bundle.mirroring_axes,
            step_fraction=self.step_fraction, accumulation=self.accumulation,
            tiles_per_batch=self.tiles_per_batch)
        torch.cuda.synchronize()
        times["predict_s"] = perf_counter() - start
        start = perf_counter()
        props = case.properties
        crop_shape = tuple(int(s) for s in props["shape_after_cropping_and_before_resampling"])
        current, original = _spacings(props, self.plan.spacing, self.plan.transpose_forward)
        labels = restore_class_labels_device(logits, crop_shape, current, original,
                                             self.probability_resampling)
        if labels is None:
            raise ContractError("the plans' probability resampling "
                                f"({self.probability_resampling.function_name}, order_z "
                                f"{self.probability_resampling.order_z}) has no device path")
        cropped = labels.cpu().numpy().view(np.uint16)
        del logits
        segmentation = uncrop_segmentation(cropped, props["shape_before_cropping"],
                                           props["bbox_used_for_cropping"],
                                           self.transpose_backward)
        times["restore_s"] = perf_counter() - start
        details = {"preprocessed_shape": tuple(int(s) for s in case.data.shape),
                   "metrics": times}
        return segmentation, details

    def predict_case(self, image_files: Sequence[str | Path], output_file: str | Path | None,
                     *, overwrite: bool = False) -> CasePrediction:
        """Read the case's channel images, predict, and write the label image (NIfTI, on the
        first image's grid) unless ``output_file`` is None."""
        from nnunet_mlx.storage.nifti import read_images, write_segmentation

        start = perf_counter()
        if output_file is not None and Path(output_file).exists() and not overwrite:
            raise ContractError(f"segmentation output already exists: {output_file}")
        data, properties = read_images(image_files)
        read_s = perf_counter() - start
        segmentation, details = self.predict_raw(data, properties)
        files: tuple[Path, ...] = ()
        start = perf_counter()
        if output_file is not None:
            write_segmentation(segmentation, output_file, properties, overwrite=overwrite)
            files = (Path(output_file),)
        metrics = {"read_s": read_s, **details["metrics"], "write_s": perf_counter() - start}
        return CasePrediction(files, segmentation, details["preprocessed_shape"], metrics)

    def predict_folder(self, input_folder: str | Path, output_folder: str | Path, *,
                       overwrite: bool = False, continue_prediction: bool = False
                       ) -> list[CasePrediction]:
        """Predict every case of an nnU-Net input folder (``<case>_<XXXX><ending>`` per
        channel) into ``<output>/<case><ending>`` (src/nnunet_mlx/prediction/pipeline.py:389-449).

        Host I/O overlaps the GPU: one reader thread loads (and decompresses) the next case
        while the current one runs, and one writer thread compresses and writes the
        previous label image; every GPU call stays on the calling thread."""
        from concurrent.futures import ThreadPoolExecutor

        from nnunet_mlx.storage.nifti import read_images, write_segmentation

        cases = case_files(input_folder, self.bundle.file_ending, self.bundle.image_channels)
        out = Path(output_folder)
        out.mkdir(parents=True, exist_ok=True)
        todo = []
        for case, files in cases.items():
            target = out / f"{case}{self.bundle.file_ending}"
            if continue_prediction and target.is_file():
                continue
            if target.exists() and not overwrite:
                raise ContractError(f"segmentation output already exists: {target}")
            todo.append((files, target))
        results: list[CasePrediction] = []
        with ThreadPoolExecutor(1) as reader, ThreadPoolExecutor(1) as writer:
            pending_read = reader.submit(read_images, todo[0][0]) if todo else None
            pending_write = None
            for index, (files, target) in enumerate(todo):
                start = perf_counter()
                data, properties = pending_read.result()
                read_wait = perf_counter() - start
                if index + 1 < len(todo):
                    pending_read = reader.submit(read_images, todo[index + 1][0])
                segmentation, details = self.predict_raw(data, properties)
                del data
                if pending_write is not None:
                    pending_write.result()
                pending_write = writer.submit(write_segmentation, segmentation, target,
                                              properties, overwrite=True)
                metrics = {"read_wait_s": read_wait, **details["metrics"]}
                results.append(CasePrediction((target,), segmentation,
                                              details["preprocessed_shape"], metrics))
            if pending_write is not None:
                pending_write.result()
        return results


def case_files(input_folder: str | Path, file_ending: str, channels: int) -> dict[str, list[Path]]:
    """Group ``<case>_<4-digit channel><file_ending>`` files by case, channels in order; every
    case must have exactly channels 0..channels-1."""
    folder = Path(input_folder)
    if not folder.is_dir():
        raise ContractError(f"input folder does not exist: {folder}")
    pattern = re.compile(r"(.+)_(\d{4})" + re.escape(file_ending) + r"$")
    grouped: dict[str, dict[int, Path]] = {}
    for path in sorted(folder.iterdir()):
        match = pattern.fullmatch(path.name)
        if match and path.is_file():
            grouped.setdefault(match.group(1), {})[int(match.group(2))] = path
    if not grouped:
        raise ContractError(f"no <case>_XXXX{file_ending} images in {folder}")
    cases = {}
    for case, by_channel in sorted(grouped.items()):
        if sorted(by_channel) != list(range(channels)):
            raise ContractError(f"case {case} needs channels 0..{channels - 1}, "
                                f"found {sorted(by_channel)}")
        cases[case] = [by_channel[c] for c in range(channels)]
    return cases
