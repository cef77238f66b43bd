"""Upstream nnU-Net v2 trained models -> converted model folders (host, torch CPU).

Reference: src/nnunet_mlx/storage/upstream.py:94-405 (``load_upstream_checkpoint``,
``detect_upstream_folds``, ``convert_trained_model``, ``resolve_results_folder``,
``cached_conversion``) and src/nnunet_mlx/storage/weights.py:48-192
(``map_key_and_layout``, ``convert_state_dict``).

An upstream trained model folder holds ``plans.json``, ``dataset.json`` and
``fold_<f>/checkpoint_final.pth`` (a torch pickle with ``network_weights``,
``trainer_name``, ``init_args.configuration``, ``inference_allowed_mirroring_axes`` and
``current_epoch``).  Conversion renames every network parameter to the reference's MLX
names, moves convolution weights to channels-last kernel layout, checks the result against
the network the plans describe, and writes the converted folder this package loads
(``plans.json``, ``dataset.json``, ``conversion.json``, ``fold_<f>/checkpoint_final/``
with ``state.json`` + ``weights.safetensors``).  Checkpoints are read with
``torch.load(weights_only=True)``; only numpy scalar and dtype reconstructors are admitted
beside tensors and containers.
"""

from __future__ import annotations

import json
import os
import re
import shutil
import tempfile
from collections.abc import Mapping, Sequence
from dataclasses import dataclass
from pathlib import Path

import numpy as np

from nnunet_mlx.errors import ContractError
from nnunet_mlx.plans import read_json_object, topology_payload
from nnunet_mlx.storage.checkpoint import (
    CheckpointIdentity,
    InferenceCheckpointState,
    save_inference_checkpoint,
)

UPSTREAM_CHECKPOINT = "checkpoint_final.pth"
CONVERTED_CHECKPOINT = "checkpoint_final"
CONVERSION_FILENAME = "conversion.json"
CONVERSION_SCHEMA = "nnunet-mlx.conversion.v1"
CONVERSION_CONTRACT_VERSION = 1

# Trainers of nnU-Net v2.8.1 that build their network from plans.json (any other trainer
# may have changed the architecture, which the plans would then not describe); the names
# are upstream trainer classes (same table as src/nnunet_mlx/prediction/source.py:29-56).
PLANS_BUILT_TRAINERS = frozenset(
    ["nnUNetTrainer", "nnUNet_Trainer_BS8"]
    + [f"nnUNetTrainer{name}" for name in (
        "Adam", "Adam1en3", "Adam3en4", "Adan", "Adan1en1", "Adan1en3", "Adan3en4",
        "AdanCosAnneal", "Benchmark_5epochs", "Benchmark_5epochs_noDataLoading", "CELoss",
        "CELoss_5epochs", "CosAnneal", "DA5", "DA5Segord0", "DA5_10epochs", "DA5ord0",
        "DiceCELoss_noSmooth", "DiceLoss", "DiceTopK10Loss", "NoDA", "NoDeepSupervision",
        "NoMirroring", "Topk10Loss", "Topk10LossLS01", "VanillaAdam", "VanillaAdam1en3",
        "VanillaAdam3en4")]
    + [f"nnUNetTrainer_{name}" for name in (
        "1epoch", "5epochs", "10epochs", "20epochs", "50epochs", "100epochs", "250epochs",
        "500epochs", "750epochs", "2000epochs", "4000epochs", "8000epochs",
        "250epochs_NoMirroring", "2000epochs_NoMirroring", "4000epochs_NoMirroring",
        "8000epochs_NoMirroring", "DASegOrd0", "DASegOrd0_NoMirroring", "noDummy2DDA",
        "onlyMirror01", "onlyMirror01_1500ep", "onlyMirror01_DA5", "onlyMirror01_DASegOrd0",
        "probabilisticOversampling", "probabilisticOversampling_010",
        "probabilisticOversampling_033", "warmup")]
)


# ---- state-dict mapping ----------------------------------------------------------------

def _conv_layout(array: np.ndarray) -> np.ndarray:
    """torch (C_out, C_in, *kernel) -> (C_out, *kernel, C_in)."""
    if array.ndim not in (4, 5):
        raise ContractError(f"expected a 2-D or 3-D convolution weight, got {array.shape}")
    return np.moveaxis(array, 1, -1)


def _transposed_conv_layout(array: np.ndarray) -> np.ndarray:
    """torch ConvTranspose (C_in, C_out, *kernel) -> (C_out, *kernel, C_in)."""
    if array.ndim not in (4, 5):
        raise ContractError(f"expected a 2-D or 3-D transposed weight, got {array.shape}")
    return np.moveaxis(array, 0, -1)


# (pattern over the upstream key, converted name, layout of a convolution weight):
# module/parameter groups are carried over by name; "conv" weights change layout.
_RULES = (
    (re.compile(r"encoder\.stages\.(\d+)\.\d+\.convs\.(\d+)\.(\w+)\.(\w+)"),
     lambda m: f"enc{m[1]}.block{m[2]}.{m[3]}.{m[4]}", "conv"),
    (re.compile(r"encoder\.stem\.convs\.0\.(\w+)\.(\w+)"),
     lambda m: f"stem.{m[1]}.{m[2]}", "conv"),
    (re.compile(r"encoder\.stages\.(\d+)\.blocks\.(\d+)\.(conv1|conv2|conv3)\.(\w+)\.(\w+)"),
     lambda m: f"res{m[1]}.block{m[2]}.{m[3]}.{m[4]}.{m[5]}", "conv"),
    (re.compile(r"encoder\.stages\.(\d+)\.blocks\.(\d+)\.skip\.\d+\.(\w+)\.(\w+)"),
     lambda m: f"res{m[1]}.block{m[2]}.proj.{m[3]}.{m[4]}", "conv"),
    (re.compile(r"decoder\.stages\.(\d+)\.convs\.(\d+)\.(\w+)\.(\w+)"),
     lambda m: f"dec{m[1]}.block{m[2]}.{m[3]}.{m[4]}", "conv"),
    (re.compile(r"decoder\.transpconvs\.(\d+)\.(\w+)"),
     lambda m: f"up{m[1]}.{m[2]}", "transposed"),
    (re.compile(r"decoder\.seg_layers\.(\d+)\.(\w+)"),
     lambda m: f"seg{m[1]}.{m[2]}", "seg"),
)


def map_key_and_layout(key: str, array: np.ndarray) -> tuple[str, np.ndarray] | None:
    """Converted name and layout of one upstream parameter, or None when the key is an
    ``all_modules`` alias or matches no PlainConvUNet / ResidualEncoderUNet parameter."""
    if "all_modules" in key.split("."):
        return None
    for pattern, name, kind in _RULES:
        m = pattern.fullmatch(key)
        if not m:
            continue
        converted = name(m)
        if converted.endswith(".weight"):
            if kind == "transposed":
                return converted, _transposed_conv_layout(array)
            if kind == "seg" or converted.endswith(".conv.weight"):
                return converted, _conv_layout(array)
        return converted, array
    return None


@dataclass(frozen=True)
class ConvertedState:
    """Converted float32 weights by name, and the upstream keys dropped on purpose."""

    weights: dict[str, np.ndarray]
    dropped_keys: tuple[str, ...]


def _host_array(value: object, *, name: str) -> np.ndarray:
    detach = getattr(value, "detach", None)
    if not callable(detach):
        raise ContractError(f"nnU-Net parameter {name!r} is not a tensor")
    tensor = detach().cpu()
    if tensor.is_complex():
        raise ContractError(f"nnU-Net parameter {name!r} is complex")
    return tensor.float().numpy()


def convert_state_dict(state: Mapping[str, object], *,
                       allow_lesiontracer_auxiliary_head: bool = False) -> ConvertedState:
    """Convert an upstream ``state_dict``.  ``decoder.encoder.*`` (the encoder registered a
    second time inside the decoder) and ``all_modules`` aliases are dropped; with
    ``allow_lesiontracer_auxiliary_head`` the ``decoder.organ_seg_layers.*`` heads (11
    outputs, never executed at inference) are dropped too.  Non-tensors, non-finite
    values, unknown keys, name collisions and an empty result raise ContractError."""
    weights: dict[str, np.ndarray] = {}
    dropped: list[str] = []
    for key, tensor in state.items():
        array = _host_array(tensor, name=key)
        if not np.isfinite(array).all():
            raise ContractError(f"nnU-Net parameter {key!r} contains non-finite values")
        if allow_lesiontracer_auxiliary_head and key.startswith("decoder.organ_seg_layers."):
            m = re.fullmatch(r"decoder\.organ_seg_layers\.(\d+)\.(weight|bias)", key)
            if not m:
                raise ContractError(f"unsupported LesionTracer auxiliary key {key!r}")
            companion = state.get(f"decoder.seg_layers.{m[1]}.{m[2]}")
            shape = _host_array(companion, name=key).shape if companion is not None else ()
            if not shape or array.shape != (11, *shape[1:]):
                raise ContractError(f"invalid LesionTracer auxiliary head shape for {key!r}")
            dropped.append(key)
            continue
        mapped = map_key_and_layout(key, array)
        if mapped is None:
            if key.startswith("decoder.encoder.") or "all_modules" in key.split("."):
                dropped.append(key)
                continue
            raise ContractError(f"unsupported nnU-Net checkpoint key {key!r}")
        name, converted = mapped
        if name in weights:
            raise ContractError(f"duplicate converted key {name!r}")
        weights[name] = np.ascontiguousarray(converted, dtype=np.float32)
    if not weights:
        raise ContractError("checkpoint did not contain convertible weights")
    return ConvertedState(weights, tuple(sorted(dropped)))


# ---- upstream checkpoints ---------------------------------------------------------------

@dataclass(frozen=True)
class UpstreamCheckpoint:
    network_weights: Mapping[str, object]
    trainer_name: str
    configuration: str
    mirroring_axes: tuple[int, ...]
    current_epoch: int | None


def load_upstream_checkpoint(path: str | Path) -> UpstreamCheckpoint:
    """Read ``checkpoint_final.pth`` with torch's restricted unpickler."""
    import torch

    source = Path(path)
    if not source.is_file():
        raise ContractError(f"upstream checkpoint does not exist: {source}")
    from numpy._core.multiarray import scalar

    allowed = [scalar, np.dtype, *(type(np.dtype(t)) for t in (
        np.bool_, np.int8, np.int16, np.int32, np.int64, np.uint8, np.uint16, np.uint32,
        np.uint64, np.float16, np.float32, np.float64, np.complex64, np.complex128))]
    with torch.serialization.safe_globals(allowed):
        try:
            raw = torch.load(source, map_location="cpu", weights_only=True)
        except Exception as error:  # restricted unpickling, damaged archive, I/O
            raise ContractError(f"cannot read upstream checkpoint {source}: {error}") from error
    if not isinstance(raw, Mapping):
        raise ContractError(f"{source.name} must hold a mapping")
    weights = raw.get("network_weights")
    trainer = raw.get("trainer_name")
    init_args = raw.get("init_args")
    if not isinstance(weights, Mapping) or not isinstance(trainer, str) or not isinstance(init_args, Mapping):
        raise ContractError(f"{source.name} lacks network_weights, trainer_name or init_args")
    configuration = init_args.get("configuration")
    if not isinstance(configuration, str) or not configuration:
        raise ContractError(f"{source.name} lacks init_args.configuration")
    axes = raw.get("inference_allowed_mirroring_axes")
    if axes is None:
        mirroring: tuple[int, ...] = ()
    elif isinstance(axes, (list, tuple)) and all(isinstance(a, int) and not isinstance(a, bool) for a in axes):
        mirroring = tuple(int(a) for a in axes)
    else:
        raise ContractError("inference_allowed_mirroring_axes must be integer axes or null")
    epoch = raw.get("current_epoch")
    if epoch is not None and (isinstance(epoch, bool) or not isinstance(epoch, int)):
        raise ContractError("current_epoch must be an integer")
    return UpstreamCheckpoint(weights, trainer, configuration, mirroring,
                              None if epoch is None else int(epoch))


def detect_upstream_folds(model_folder: str | Path, *,
                          checkpoint_name: str = UPSTREAM_CHECKPOINT) -> tuple[int | str, ...]:
    """Numeric folds in order, then ``"all"``, whose folder holds ``checkpoint_name``."""
    numeric: list[int] = []
    has_all = False
    for candidate in Path(model_folder).glob("fold_*"):
        if not (candidate / checkpoint_name).is_file():
            continue
        suffix = candidate.name[len("fold_"):]
        if suffix.isdigit() and str(int(suffix)) == suffix:
            numeric.append(int(suffix))
        elif suffix == "all":
            has_all = True
    folds: tuple[int | str, ...] = (*sorted(numeric), *(("all",) if has_all else ()))
    if not folds:
        raise ContractError(f"no fold_* folder in {model_folder} contains {checkpoint_name}")
    return folds


@dataclass(frozen=True)
class ConversionResult:
    destination: Path
    configuration: str
    trainer_name: str
    folds: tuple[int | str, ...]


def convert_trained_model(source: str | Path, destination: str | Path, *,
                          folds: Sequence[int | str] | None = None,
                          checkpoint_name: str = UPSTREAM_CHECKPOINT) -> ConversionResult:
    """Convert an upstream trained model folder into a new converted model folder.

    All folds must come from one plans-built trainer and one configuration, and each
    fold's converted weights must match the network of the plans exactly (names and
    shapes).  The folder is assembled next to ``destination`` and moved into place only
    when complete; ``destination`` must not exist."""
    from nnunet_mlx.model.factory import spec_from_plans
    from nnunet_mlx.model.folder import input_channel_count, output_channel_count, validate_folds
    from nnunet_mlx.model.network import build_network

    folder = Path(source)
    target = Path(destination)
    if not folder.is_dir():
        raise ContractError(f"trained model folder does not exist: {folder}")
    if Path(checkpoint_name).name != checkpoint_name:
        raise ContractError("checkpoint name must be a file name")
    if target.exists():
        raise ContractError(f"conversion destination already exists: {target}")
    plans = read_json_object(folder / "plans.json")
    dataset = read_json_object(folder / "dataset.json")
    selected = (detect_upstream_folds(folder, checkpoint_name=checkpoint_name)
                if folds is None else validate_folds(folds))
    paths = [folder / f"fold_{fold}" / checkpoint_name for fold in selected]
    first = load_upstream_checkpoint(paths[0])
    if first.trainer_name not in PLANS_BUILT_TRAINERS:
        raise ContractError(f"trainer {first.trainer_name!r} is not supported: only nnU-Net "
                            "v2.8.1 trainers that build the network from plans.json convert")
    configuration = first.configuration
    resolved = topology_payload(plans, configuration)["configurations"][configuration]
    if "architecture" not in resolved:
        raise ContractError("plans without an architecture block (nnU-Net < 2.4) are not supported")
    spec = spec_from_plans(topology_payload(plans, configuration), configuration=configuration,
                           input_channels=input_channel_count(dataset),
                           output_channels=output_channel_count(dataset))
    expected = build_network(spec).parameter_shapes()
    architecture = resolved["architecture"]
    staging = Path(tempfile.mkdtemp(prefix=f".{target.name}.", dir=str(target.parent)))
    try:
        shutil.copyfile(folder / "plans.json", staging / "plans.json")
        shutil.copyfile(folder / "dataset.json", staging / "dataset.json")
        entries = []
        for fold, path in zip(selected, paths):
            checkpoint = first if path == paths[0] else load_upstream_checkpoint(path)
            if (checkpoint.trainer_name, checkpoint.configuration) != (first.trainer_name, configuration):
                raise ContractError(f"fold {fold} was trained with a different trainer or "
                                    "configuration than the other folds")
            converted = convert_state_dict(checkpoint.network_weights)
            got = {k: v.shape for k, v in converted.weights.items()}
            if got != expected:
                missing = sorted(set(expected) - set(got))[:5]
                extra = sorted(set(got) - set(expected))[:5]
                wrong = sorted(k for k in set(got) & set(expected) if got[k] != expected[k])[:5]
                raise ContractError(f"fold {fold} weights do not match the network planned in "
                                    f"plans.json (missing {missing}, unexpected {extra}, "
                                    f"shape mismatch {wrong})")
            save_inference_checkpoint(
                staging / f"fold_{fold}" / CONVERTED_CHECKPOINT, weights=converted.weights,
                state=InferenceCheckpointState(
                    identity=CheckpointIdentity(checkpoint.trainer_name, configuration, fold),
                    current_epoch=checkpoint.current_epoch, spatial_dims=3,
                    inference_allowed_mirroring_axes=checkpoint.mirroring_axes,
                    dropped_source_keys=converted.dropped_keys))
            stat = path.stat()
            entries.append({"fold": fold, "checkpoint": CONVERTED_CHECKPOINT,
                            "source_checkpoint": checkpoint_name,
                            "source_size_bytes": stat.st_size,
                            "source_mtime_ns": stat.st_mtime_ns})
        manifest = {
            "schema_version": CONVERSION_SCHEMA,
            "conversion_contract_version": CONVERSION_CONTRACT_VERSION,
            "source_plans": plans, "source_dataset": dataset,
            "engine_version": "nnunet-mlx-amd", "configuration": configuration,
            "architecture": architecture.get("network_class_name") if isinstance(architecture, Mapping) else None,
            "spatial_dims": 3, "folds": entries,
        }
        (staging / CONVERSION_FILENAME).write_text(
            json.dumps(manifest, indent=2, sort_keys=True) + "\n", encoding="utf-8")
        staging.rename(target)
    except BaseException:
        shutil.rmtree(staging, ignore_errors=True)
        raise
    return ConversionResult(target, configuration, first.trainer_name, tuple(selected))


RESULTS_VARIABLE = "nnUNet_results"
CACHE_VARIABLE = "NNUNET_MLX_CACHE"
SOURCE_MARKER = ".source"


def resolve_results_folder(dataset: str, *, configuration: str, trainer: str = "nnUNetTrainer",
                           plans: str = "nnUNetPlans", results: str | Path | None = None) -> Path:
    """``<results>/<dataset>/<trainer>__<plans>__<configuration>``, nnU-Net's results layout.

    ``dataset`` is a full name (``Dataset003_Liver``) or a numeric ID, which must match
    exactly one ``DatasetNNN_*`` folder.  ``results`` defaults to ``$nnUNet_results``.
    Reference: src/nnunet_mlx/storage/upstream.py:298-323."""
    base = results if results is not None else os.environ.get(RESULTS_VARIABLE)
    if not base:
        raise ContractError(f"set {RESULTS_VARIABLE}, or pass a trained model folder with -m")
    root = Path(base).expanduser()
    if dataset.isdigit():
        prefix = f"Dataset{int(dataset):03d}_"
        names = sorted(p.name for p in root.glob(prefix + "*")
                       if p.is_dir() and len(p.name) > len(prefix))
        if len(names) != 1:
            raise ContractError(f"expected one {prefix}* folder in {root}, found {len(names)}")
        dataset = names[0]
    folder = root / dataset / f"{trainer}__{plans}__{configuration}"
    if not folder.is_dir():
        raise ContractError(f"trained model folder does not exist: {folder}")
    return folder


def conversion_is_current(target: Path, source: Path, folds: Sequence[int | str],
                          checkpoint_name: str) -> bool:
    """Whether ``target`` is a complete conversion of ``source`` as it is now: same source
    folder, same conversion contract, identical plans/dataset JSON, the same fold set, each
    source checkpoint with its recorded size and modification time, every payload file
    present.  Reference: src/nnunet_mlx/storage/upstream.py:366-405."""
    marker = target / SOURCE_MARKER
    try:
        if not marker.is_file() or marker.read_text(encoding="utf-8").strip() != str(source):
            return False
        manifest = read_json_object(target / CONVERSION_FILENAME)
        plans = read_json_object(source / "plans.json")
        dataset = read_json_object(source / "dataset.json")
        if (manifest.get("schema_version") != CONVERSION_SCHEMA
                or manifest.get("conversion_contract_version") != CONVERSION_CONTRACT_VERSION
                or manifest.get("source_plans") != plans or manifest.get("source_dataset") != dataset
                or read_json_object(target / "plans.json") != plans
                or read_json_object(target / "dataset.json") != dataset):
            return False
        entries = manifest.get("folds")
        if not isinstance(entries, list) or not all(isinstance(e, Mapping) for e in entries):
            return False
        recorded = {e.get("fold"): e for e in entries}
        if len(recorded) != len(entries) or set(recorded) != set(folds):
            return False
        for fold in folds:
            entry = recorded[fold]
            stat = (source / f"fold_{fold}" / checkpoint_name).stat()
            if (entry.get("source_checkpoint"), entry.get("source_size_bytes"),
                    entry.get("source_mtime_ns")) != (checkpoint_name, stat.st_size, stat.st_mtime_ns):
                return False
            payload = target / f"fold_{fold}" / CONVERTED_CHECKPOINT
            if not ((payload / "weights.safetensors").is_file() and (payload / "state.json").is_file()):
                return False
    except (ContractError, OSError, ValueError):
        return False
    return True


def cached_conversion(trained_folder: str | Path, *, folds: Sequence[int | str] | None = None,
                      checkpoint_name: str = UPSTREAM_CHECKPOINT,
                      cache: str | Path | None = None) -> Path:
    """A converted copy of ``trained_folder``, converting only when no current one exists.

    Entries live at ``<cache>/converted/<dataset folder>/<model folder>`` with ``cache``
    defaulting to ``$NNUNET_MLX_CACHE`` or ``~/.cache/nnunet-mlx``; every available fold is
    converted so later fold selections reuse the entry.  A stale entry (see
    ``conversion_is_current``) is deleted and rebuilt.  Symlinked cache parents or entries
    are refused, so the deletion never leaves the cache.
    Reference: src/nnunet_mlx/storage/upstream.py:326-363."""
    from nnunet_mlx.model.folder import validate_folds

    source = Path(os.path.normpath(str(Path(trained_folder).absolute())))
    if not source.name or not source.parent.name:
        raise ContractError("trained folder needs dataset and model directory names")
    available = detect_upstream_folds(source, checkpoint_name=checkpoint_name)
    if folds is not None:
        absent = [f for f in validate_folds(folds) if f not in available]
        if absent:
            raise ContractError(f"folds {absent} have no {checkpoint_name} in {source}")
    root = Path(cache if cache is not None else
                os.environ.get(CACHE_VARIABLE, "~/.cache/nnunet-mlx")).expanduser()
    parent = root / "converted" / source.parent.name
    parent.mkdir(parents=True, exist_ok=True)
    if parent.resolve() != root.resolve() / "converted" / source.parent.name:
        raise ContractError(f"conversion cache has a symlinked parent: {parent}")
    target = parent / source.name
    if target.is_symlink():
        raise ContractError(f"conversion cache entry must not be a symlink: {target}")
    if conversion_is_current(target, source, available, checkpoint_name):
        return target
    if target.exists():
        shutil.rmtree(target)
    convert_trained_model(source, target, folds=available, checkpoint_name=checkpoint_name)
    (target / SOURCE_MARKER).write_text(f"{source}\n", encoding="utf-8")
    return target
