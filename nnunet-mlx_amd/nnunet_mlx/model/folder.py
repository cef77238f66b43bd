"""Loading of converted nnU-Net model folders onto the GPU.

Reference: load_model_bundle (src/nnunet_mlx/model/folder.py:87-227).  The folder
layout is read unchanged: ``plans.json``, ``dataset.json`` and
``fold_<k>/<checkpoint_name>/{state.json, weights.safetensors}``.  Unlike the
reference, which swaps one resident network between folds on every fold switch
(src/nnunet_mlx/model/residency.py:51-109), every selected fold keeps its own repacked
weights resident in HBM (about 125 MB per fold for the 6-stage nets) and the folds share
one activation workspace.
"""

from __future__ import annotations

import re
from collections.abc import Mapping, Sequence
from dataclasses import dataclass
from pathlib import Path

from nnunet_mlx.errors import ContractError
from nnunet_mlx.model.factory import spec_from_plans
from nnunet_mlx.model.network import NativeNetwork, build_network
from nnunet_mlx.plans import patch_size as plans_patch_size
from nnunet_mlx.plans import read_json_object, topology_payload
from nnunet_mlx.storage.checkpoint import (
    checkpoint_weights_signature,
    load_inference_checkpoint,
)


@dataclass(frozen=True)
class CheckpointProvenance:
    fold: int | str
    checkpoint: str
    weights_signature: list[int]

    def to_payload(self) -> dict[str, object]:
        return {"fold": self.fold, "checkpoint": self.checkpoint,
                "weights_signature": self.weights_signature}


@dataclass(frozen=True)
class ModelBundle:
    folder: Path
    plans: dict[str, object]
    configuration: str
    dataset_json: dict[str, object]
    models: tuple[NativeNetwork, ...]
    folds: tuple[int | str, ...]
    checkpoints: tuple[CheckpointProvenance, ...]
    mirroring_axes: tuple[int, ...]
    patch_size: tuple[int, ...]
    num_outputs: int
    image_channels: int
    input_channels: int
    file_ending: str
    arithmetic: str = "native"


def input_channel_count(dataset_json: Mapping[str, object]) -> int:
    channels = dataset_json.get("channel_names") or dataset_json.get("modality")
    if not isinstance(channels, Mapping) or not channels:
        raise ContractError("dataset channel_names must not be empty")
    keys = sorted(int(k) for k in channels)
    if keys != list(range(len(keys))):
        raise ContractError("dataset channel_names keys must be canonical integers 0..N-1")
    return len(keys)


def output_channel_count(dataset_json: Mapping[str, object]) -> int:
    labels = dataset_json.get("labels")
    if not isinstance(labels, Mapping) or not labels:
        raise ContractError("dataset labels must not be empty")
    if dataset_json.get("regions_class_order") is not None:
        return len(dataset_json["regions_class_order"])  # type: ignore[arg-type]
    values = set()
    for name, value in labels.items():
        if name == "ignore":
            continue
        values.add(int(value))
    return len(values)


def validate_folds(values: Sequence[int | str]) -> tuple[int | str, ...]:
    folds = tuple(values)
    if not folds or len(folds) != len(set(folds)):
        raise ContractError("model folds must be non-empty and unique")
    for fold in folds:
        ok = (isinstance(fold, int) and not isinstance(fold, bool) and fold >= 0) or fold == "all"
        if not ok:
            raise ContractError("model folds must be non-negative integers or 'all'")
    return folds


def auto_detect_folds(model_folder: str | Path, *, checkpoint_name: str) -> tuple[int, ...]:
    folds = []
    for child in Path(model_folder).iterdir():
        match = re.fullmatch(r"fold_(\d+)", child.name)
        if match and (child / checkpoint_name).is_dir():
            folds.append(int(match.group(1)))
    if not folds:
        raise ContractError(f"no fold checkpoints named {checkpoint_name!r} in {model_folder}")
    return tuple(sorted(folds))


def load_model_bundle(
    model_folder: str | Path, *, configuration: str, folds: Sequence[int | str] | None = None,
    checkpoint_name: str = "checkpoint_final", arithmetic: str = "native",
) -> ModelBundle:
    """Load and verify a converted model folder; every fold is resident on the GPU."""
    if arithmetic != "native":
        raise ContractError(f"unsupported inference arithmetic {arithmetic!r}")
    folder = Path(model_folder)
    if not folder.is_dir():
        raise ContractError(f"model folder does not exist: {folder}")
    plans = read_json_object(folder / "plans.json")
    dataset_json = read_json_object(folder / "dataset.json")
    channels = input_channel_count(dataset_json)
    outputs = output_channel_count(dataset_json)
    selected = auto_detect_folds(folder, checkpoint_name=checkpoint_name) if folds is None else validate_folds(folds)
    spec = spec_from_plans(topology_payload(plans, configuration), configuration=configuration,
                           input_channels=channels, output_channels=outputs)
    models: list[NativeNetwork] = []
    provenance: list[CheckpointProvenance] = []
    axes_seen: list[tuple[int, ...]] = []
    for fold in selected:
        checkpoint = folder / f"fold_{fold}" / checkpoint_name
        if checkpoint.is_file() or checkpoint.suffix == ".pth":
            raise ContractError("checkpoint must be a native nnunet-mlx safetensors directory")
        model = build_network(spec)
        state = load_inference_checkpoint(checkpoint, model=model)
        if state.identity.configuration != configuration:
            raise ContractError("checkpoint configuration does not match the requested one")
        if state.identity.fold != fold:
            raise ContractError("checkpoint fold does not match its folder")
        if models:
            model.share_workspace(models[0])
        models.append(model)
        axes_seen.append(state.inference_allowed_mirroring_axes)
        provenance.append(CheckpointProvenance(fold=fold, checkpoint=checkpoint_name,
                                               weights_signature=checkpoint_weights_signature(checkpoint)))
    if any(axes != axes_seen[0] for axes in axes_seen[1:]):
        raise ContractError("model folds disagree on inference mirroring axes")
    file_ending = dataset_json.get("file_ending")
    if not isinstance(file_ending, str) or not file_ending.startswith("."):
        raise ContractError("dataset file_ending must start with a dot")
    return ModelBundle(
        folder=folder, plans=plans, configuration=configuration, dataset_json=dataset_json,
        models=tuple(models), folds=selected, checkpoints=tuple(provenance),
        mirroring_axes=axes_seen[0], patch_size=plans_patch_size(plans, configuration),
        num_outputs=outputs, image_channels=channels, input_channels=channels,
        file_ending=file_ending,
    )
