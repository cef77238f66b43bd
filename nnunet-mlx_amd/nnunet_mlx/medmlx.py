"""Public one-case API: ``run``, ``load_model`` and ``segment_case``.

Reference: src/nnunet_mlx/medmlx.py:121-605 (``predictor``, ``check_request``, ``run``,
``segment_case``, ``NnUNetModel``, ``load_model``).  Same keyword arguments and the same
result dictionary (``outputs`` / ``artifacts`` / ``details``); the case itself runs through
``ModelFolderPredictor`` with every compute step on the GPU.  Windows and folds accumulate
in float16 as nnU-Net v2.8.1 does (``ACCUMULATION``).

Not carried over: weight downloads (``weights_path`` must be a local converted model
folder), probability export (``save_probabilities=True`` raises ``ContractError``), the
``torch-order-fp32`` precision and non-default source profiles.
"""

from __future__ import annotations

import os
import shutil
import tempfile
from collections.abc import Mapping, Sequence
from dataclasses import replace
from pathlib import Path
from time import perf_counter

from nnunet_mlx.errors import ContractError
from nnunet_mlx.storage.nifti import NIFTI_ENDINGS

ACCUMULATION = "nnunet-fp16"
SEGMENTATION_STEM = "mask"
DEFAULT_SOURCE_PROFILE = "nnunet-v2.8.1-default"
_WEIGHTS_HINT = "pass a local converted model folder as weights_path"

PathLike = str | os.PathLike


def dataset_labels(dataset_json: Mapping[str, object]) -> list[dict[str, object]]:
    """``[{"value": v, "name": n}, ...]`` sorted by value, without ``ignore``
    (src/nnunet_mlx/medmlx.py:55-61)."""
    labels = dataset_json.get("labels")
    if not isinstance(labels, Mapping):
        raise ContractError("dataset.json labels must be a mapping")
    items = [{"value": int(v), "name": str(k)} for k, v in labels.items() if k != "ignore"]
    return sorted(items, key=lambda item: item["value"])


def output_kind(labels: Sequence[Mapping[str, object]]) -> str:
    """``binary_mask`` for a 0/1 label table, else ``label_map`` (src/nnunet_mlx/medmlx.py:64-69)."""
    return "binary_mask" if sorted(int(i["value"]) for i in labels) == [0, 1] else "label_map"


def predictor(bundle, *, step_fraction: float):
    """The predictor the runners and the CLI use: float16 window and fold accumulation."""
    from nnunet_mlx.prediction.pipeline import ModelFolderPredictor

    return ModelFolderPredictor(bundle, accumulation=ACCUMULATION, step_fraction=step_fraction)


def _boolean(value: object, name: str) -> bool:
    if not isinstance(value, bool):
        raise ContractError(f"{name} must be a boolean")
    return value


def check_request(image_paths: Sequence[PathLike], *, output_dir: PathLike,
                  overwrite: object = False, folds: Sequence[int | str] | None = None,
                  source_profile: str | None = None, precision: str = "native",
                  step_fraction: object = 0.5, use_mirroring: object = True,
                  save_probabilities: object = False
                  ) -> tuple[list[Path], tuple[int | str, ...] | None]:
    """Validate the arguments that need no model folder (src/nnunet_mlx/medmlx.py:137-200)."""
    from nnunet_mlx.model.folder import validate_folds

    if (not isinstance(image_paths, (list, tuple)) or not image_paths
            or not all(isinstance(p, (str, os.PathLike)) for p in image_paths)):
        raise ContractError("image_paths must be a non-empty list of NIfTI images, one per "
                            "modality in channel order")
    images = [Path(p).expanduser() for p in image_paths]
    for image in images:
        if not image.is_file():
            raise ContractError(f"Missing input image: {image}")
        if not image.name.endswith(NIFTI_ENDINGS):
            raise ContractError(f"nnU-Net input must be a NIfTI image (.nii or .nii.gz): {image}")
    for name, flag in (("overwrite", overwrite), ("use_mirroring", use_mirroring),
                       ("save_probabilities", save_probabilities)):
        _boolean(flag, name)
    if save_probabilities:
        raise ContractError("probability export is not available on the device case path")
    selected = None if folds is None else validate_folds(list(folds))
    if isinstance(step_fraction, bool) or not isinstance(step_fraction, (int, float)):
        raise ContractError("step_fraction must be a number")
    if not 0 < float(step_fraction) <= 1:
        raise ContractError(f"step_fraction must be in (0, 1], got {step_fraction}")
    if precision != "native":
        raise ContractError(f"unsupported precision {precision!r}")
    if source_profile not in (None, DEFAULT_SOURCE_PROFILE):
        raise ContractError(f"unsupported source profile {source_profile!r}")
    output = Path(output_dir).expanduser()
    if output.exists() and not output.is_dir():
        raise ContractError(f"output_dir must be a directory: {output}")
    return images, selected


def _mask_target(folder: Path, output: Path) -> tuple[Path, list[dict[str, object]]]:
    from nnunet_mlx.plans import read_json_object

    if not folder.is_dir():
        raise ContractError(f"nnU-Net model folder does not exist: {folder}; {_WEIGHTS_HINT}")
    if not (folder / "dataset.json").is_file():
        raise ContractError(f"model folder lacks dataset.json: {folder}; {_WEIGHTS_HINT}")
    dataset_json = read_json_object(folder / "dataset.json")
    ending = dataset_json.get("file_ending")
    if ending not in NIFTI_ENDINGS:
        raise ContractError(f"runs write NIfTI; dataset.json file_ending is {ending!r}")
    return output / f"{SEGMENTATION_STEM}{ending}", dataset_labels(dataset_json)


def segment_case(*, prepared=None, grid_of: str = "image_paths", weights_path: PathLike,
                 image_paths: Sequence[PathLike], output_dir: PathLike, overwrite: bool = False,
                 configuration: str | None = None, folds: Sequence[int | str] | None = None,
                 checkpoint_name: str = "checkpoint_final", source_profile: str | None = None,
                 precision: str = "native", step_fraction: float = 0.5,
                 use_mirroring: bool = True, save_probabilities: bool = False) -> dict:
    """Segment one case and write ``mask.nii.gz`` on the input grid
    (src/nnunet_mlx/medmlx.py:280-444).  ``prepared`` is a (bundle, predictor) pair of a
    loaded ``NnUNetModel``."""
    images, selected = check_request(
        image_paths, output_dir=output_dir, overwrite=overwrite, folds=folds,
        source_profile=source_profile, precision=precision, step_fraction=step_fraction,
        use_mirroring=use_mirroring, save_probabilities=save_probabilities)
    folder = Path(weights_path).expanduser()
    output = Path(output_dir).expanduser()
    target, labels = _mask_target(folder, output)
    resolved_inputs = {p.resolve() for p in images}
    if target.resolve() in resolved_inputs:
        raise ContractError(f"output {target} would overwrite an input image")
    if target.exists() and not overwrite:
        raise ContractError(f"output already exists: {target} (pass overwrite=True)")
    configuration = configuration or "3d_fullres"
    started = perf_counter()
    if prepared is None:
        from nnunet_mlx.model.folder import load_model_bundle

        bundle = load_model_bundle(folder, configuration=configuration, folds=selected,
                                   checkpoint_name=checkpoint_name)
        if not use_mirroring:
            bundle = replace(bundle, mirroring_axes=())
        case_predictor = predictor(bundle, step_fraction=float(step_fraction))
        model_load_s = perf_counter() - started
    else:
        bundle, case_predictor = prepared
        model_load_s = 0.0
    output.mkdir(parents=True, exist_ok=True)
    staging = Path(tempfile.mkdtemp(prefix=".nnunet-mlx-", dir=output))
    try:
        staged = staging / target.name
        result = case_predictor.predict_case(images, staged, overwrite=True)
        staged.replace(target)
    finally:
        shutil.rmtree(staging, ignore_errors=True)
    metrics = dict(result.metrics)
    metrics.update(model_load_s=model_load_s, total_wall_s=perf_counter() - started)
    try:
        import torch

        metrics["peak_memory_bytes"] = int(torch.cuda.max_memory_allocated())
    except Exception:  # noqa: BLE001 - reporting only
        pass
    return {
        "outputs": {"mask": target.resolve().as_posix()},
        "artifacts": {"mask": {"kind": output_kind(labels), "coordinate_space": "image_physical",
                               "grid_of": grid_of, "labels": labels}},
        "details": {
            "labels": labels, "configuration": configuration,
            "source_profile": source_profile or DEFAULT_SOURCE_PROFILE,
            "precision": precision, "folds": list(bundle.folds),
            "checkpoints": [c.to_payload() for c in bundle.checkpoints],
            "mirroring_axes": list(bundle.mirroring_axes), "step_fraction": step_fraction,
            "accumulation": ACCUMULATION, "decoding": result.decoding,
            "save_probabilities": False, "backend": "hip-gfx950",
            "preprocessed_shape": list(result.preprocessed_shape), "metrics": metrics,
        },
    }


def run(*, weights_path: PathLike, image_paths: Sequence[PathLike], output_dir: PathLike,
        overwrite: bool = False, configuration: str | None = None,
        folds: Sequence[int | str] | None = None, checkpoint_name: str = "checkpoint_final",
        source_profile: str | None = None, precision: str = "native",
        step_fraction: float = 0.5, use_mirroring: bool = True,
        save_probabilities: bool = False) -> dict:
    """Segment one case and restore the label map to the input image's grid
    (src/nnunet_mlx/medmlx.py:203-277).  ``outputs["mask"]`` is the written label image."""
    return segment_case(
        weights_path=weights_path, image_paths=image_paths, output_dir=output_dir,
        overwrite=overwrite, configuration=configuration, folds=folds,
        checkpoint_name=checkpoint_name, source_profile=source_profile, precision=precision,
        step_fraction=step_fraction, use_mirroring=use_mirroring,
        save_probabilities=save_probabilities)


def source_signature(folder: Path, checkpoint_name: str) -> tuple[tuple, ...]:
    """Stat records of the files a loaded model was built from: ``plans.json``,
    ``dataset.json`` and each ``fold_*/<checkpoint_name>/{state.json,weights.safetensors}``
    (src/nnunet_mlx/medmlx.py:454-469).  Each record is (relative path, device, inode,
    size, modification time ns, status-change time ns), so a rewrite, a replacement or a
    ``touch`` of any of them changes the signature without the weights being read again."""
    files = [folder / "plans.json", folder / "dataset.json"]
    for fold in sorted(folder.glob(f"fold_*/{checkpoint_name}")):
        files += [fold / "state.json", fold / "weights.safetensors"]
    records = []
    for path in files:
        try:
            st = path.stat()
        except OSError as error:
            raise ContractError(f"model file missing or unreadable: {path}") from error
        records.append((path.relative_to(folder).as_posix(), st.st_dev, st.st_ino, st.st_size,
                        st.st_mtime_ns, st.st_ctime_ns))
    return tuple(records)


class NnUNetModel:
    """One loaded model folder reused for serial cases until closed
    (src/nnunet_mlx/medmlx.py:486-587).

    The model folder must stay as it was while the model is loaded: its source signature
    (``source_signature``) is taken before loading, checked again after loading and before
    every case, and a difference raises ``ContractError`` (load the model again to pick up
    the edit)."""

    def __init__(self, *, weights_path: PathLike, configuration: str = "3d_fullres",
                 folds: Sequence[int | str] | None = None,
                 checkpoint_name: str = "checkpoint_final", source_profile: str | None = None,
                 precision: str = "native", step_fraction: float = 0.5,
                 use_mirroring: bool = True) -> None:
        from nnunet_mlx.model.folder import load_model_bundle, validate_folds

        if Path(checkpoint_name).name != checkpoint_name or checkpoint_name in {".", ".."}:
            raise ContractError("checkpoint_name must name a checkpoint directory")
        _boolean(use_mirroring, "use_mirroring")
        if isinstance(step_fraction, bool) or not 0 < float(step_fraction) <= 1:
            raise ContractError("step_fraction must be in (0, 1]")
        if precision != "native":
            raise ContractError(f"unsupported precision {precision!r}")
        if source_profile not in (None, DEFAULT_SOURCE_PROFILE):
            raise ContractError(f"unsupported source profile {source_profile!r}")
        self._folder = Path(weights_path).expanduser().absolute()
        self._options = {"configuration": configuration,
                         "folds": None if folds is None else validate_folds(list(folds)),
                         "checkpoint_name": checkpoint_name, "source_profile": source_profile,
                         "precision": precision, "step_fraction": step_fraction,
                         "use_mirroring": use_mirroring}
        self._signature = source_signature(self._folder, checkpoint_name)
        bundle = load_model_bundle(self._folder, configuration=configuration,
                                   folds=self._options["folds"], checkpoint_name=checkpoint_name)
        if source_signature(self._folder, checkpoint_name) != self._signature:
            for model in bundle.models:
                model.close()
            raise ContractError("the model folder was modified during loading; load the model again")
        if not use_mirroring:
            bundle = replace(bundle, mirroring_axes=())
        self._state = (bundle, predictor(bundle, step_fraction=float(step_fraction)))

    def run(self, *, image_paths: Sequence[PathLike], output_dir: PathLike,
            overwrite: bool = False, save_probabilities: bool = False) -> dict:
        return self.segment_case(image_paths=image_paths, output_dir=output_dir,
                                 overwrite=overwrite, save_probabilities=save_probabilities)

    def segment_case(self, *, image_paths: Sequence[PathLike], output_dir: PathLike,
                     overwrite: bool, save_probabilities: bool = False,
                     grid_of: str = "image_paths") -> dict:
        if self._state is None:
            raise RuntimeError("nnU-Net model is closed")
        if source_signature(self._folder, self._options["checkpoint_name"]) != self._signature:
            raise ContractError("the model folder changed after this model was loaded; "
                                "load the model again")
        return segment_case(prepared=self._state, grid_of=grid_of, weights_path=self._folder,
                            image_paths=image_paths, output_dir=output_dir, overwrite=overwrite,
                            save_probabilities=save_probabilities, **self._options)

    def close(self) -> None:
        """Release the model; later calls raise ``RuntimeError``."""
        if self._state is not None:
            for model in self._state[0].models:
                model.close()
        self._state = None

    def __enter__(self) -> "NnUNetModel":
        return self

    def __exit__(self, *args: object) -> None:
        self.close()


def load_model(*, weights_path: PathLike, configuration: str = "3d_fullres",
               folds: Sequence[int | str] | None = None, checkpoint_name: str = "checkpoint_final",
               source_profile: str | None = None, precision: str = "native",
               step_fraction: float = 0.5, use_mirroring: bool = True) -> NnUNetModel:
    """Load a converted model folder once to segment several cases
    (src/nnunet_mlx/medmlx.py:590-605)."""
    return NnUNetModel(weights_path=weights_path, configuration=configuration, folds=folds,
                       checkpoint_name=checkpoint_name, source_profile=source_profile,
                       precision=precision, step_fraction=step_fraction,
                       use_mirroring=use_mirroring)
