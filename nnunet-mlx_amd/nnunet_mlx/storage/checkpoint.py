"""Converted nnU-Net inference checkpoints: ``state.json`` + ``weights.safetensors``.

Reads the reference's converted-checkpoint layout unchanged
(src/nnunet_mlx/storage/checkpoint.py:27-165): schema
``nnunet-mlx.inference-checkpoint.v2`` (or the training schema
``nnunet-mlx.checkpoint.v2``), an exact file set, source nnU-Net v2.8.1, and float32
weights keyed by the reference's parameter names in MLX layout.  Weights are read with
``safetensors.numpy`` (no pickle).
"""

from __future__ import annotations

import json
from collections.abc import Mapping
from dataclasses import asdict, dataclass
from pathlib import Path

import numpy as np

from nnunet_mlx.errors import ContractError

SCHEMA_VERSION = "nnunet-mlx.checkpoint.v2"
INFERENCE_SCHEMA_VERSION = "nnunet-mlx.inference-checkpoint.v2"
SOURCE_NNUNET_VERSION = "v2.8.1"
_PAYLOAD_FILES = ("weights.safetensors", "optimizer.safetensors", "rng.safetensors")
_INFERENCE_PAYLOAD_FILES = ("weights.safetensors",)


@dataclass(frozen=True)
class CheckpointIdentity:
    trainer_name: str
    configuration: str
    fold: int | str

    def __post_init__(self) -> None:
        if not self.trainer_name or not self.configuration:
            raise ContractError("checkpoint trainer and configuration must be non-empty")
        ok_int = isinstance(self.fold, int) and not isinstance(self.fold, bool) and self.fold >= 0
        if not (ok_int or self.fold == "all"):
            raise ContractError("checkpoint fold must be a non-negative integer or 'all'")


@dataclass(frozen=True)
class InferenceCheckpointState:
    identity: CheckpointIdentity
    current_epoch: int | None
    spatial_dims: int
    inference_allowed_mirroring_axes: tuple[int, ...]
    dropped_source_keys: tuple[str, ...]

    def __post_init__(self) -> None:
        if self.current_epoch is not None and self.current_epoch < 0:
            raise ContractError("checkpoint epoch must be non-negative")
        _validate_axes(self.spatial_dims, self.inference_allowed_mirroring_axes)
        if len(set(self.dropped_source_keys)) != len(self.dropped_source_keys):
            raise ContractError("dropped source checkpoint keys must be unique")

    def to_payload(self) -> dict[str, object]:
        return {
            "schema_version": INFERENCE_SCHEMA_VERSION,
            "source_nnunet_version": SOURCE_NNUNET_VERSION,
            "identity": asdict(self.identity),
            "current_epoch": self.current_epoch,
            "spatial_dims": self.spatial_dims,
            "inference_allowed_mirroring_axes": list(self.inference_allowed_mirroring_axes),
            "dropped_source_keys": list(self.dropped_source_keys),
        }


def _validate_axes(spatial_dims: int, axes: tuple[int, ...]) -> None:
    if spatial_dims not in (2, 3):
        raise ContractError("checkpoint spatial dimensions must be 2 or 3")
    if len(set(axes)) != len(axes) or any(a not in range(spatial_dims) for a in axes):
        raise ContractError(f"invalid checkpoint mirroring axes {axes}")


def _integer(value: object, *, name: str) -> int:
    if isinstance(value, bool) or not isinstance(value, int):
        raise ContractError(f"{name} must be an integer")
    return value


def _identity(value: object) -> CheckpointIdentity:
    if not isinstance(value, Mapping):
        raise ContractError("checkpoint identity must be a mapping")
    fold = value.get("fold")
    return CheckpointIdentity(
        trainer_name=str(value.get("trainer_name") or ""),
        configuration=str(value.get("configuration") or ""),
        fold="all" if fold == "all" else _integer(fold, name="fold"),
    )


def _int_tuple(value: object, *, name: str) -> tuple[int, ...]:
    if not isinstance(value, list):
        raise ContractError(f"{name} must be an integer array")
    return tuple(_integer(v, name=name) for v in value)


def read_state(directory: str | Path) -> InferenceCheckpointState:
    """Parse and validate ``state.json`` and the checkpoint's exact file set."""
    source = Path(directory)
    if not source.is_dir():
        raise ContractError(f"checkpoint directory does not exist: {source}")
    state_file = source / "state.json"
    if not state_file.is_file():
        raise ContractError("checkpoint state.json does not exist")
    try:
        payload = json.loads(state_file.read_text(encoding="utf-8"))
    except (UnicodeDecodeError, json.JSONDecodeError) as error:
        raise ContractError("checkpoint state is invalid JSON") from error
    if not isinstance(payload, Mapping):
        raise ContractError("checkpoint state must be a mapping")
    schema = payload.get("schema_version")
    if payload.get("source_nnunet_version") != SOURCE_NNUNET_VERSION:
        raise ContractError("checkpoint source nnU-Net version does not match")
    if schema == SCHEMA_VERSION:
        _verify_file_set(source, _PAYLOAD_FILES)
        dropped: tuple[str, ...] = ("best_ema", "optimizer_config", "schedule_config")
        epoch = _integer(payload.get("current_epoch"), name="current epoch")
    elif schema == INFERENCE_SCHEMA_VERSION:
        _verify_file_set(source, _INFERENCE_PAYLOAD_FILES)
        raw = payload.get("dropped_source_keys")
        if not isinstance(raw, list) or not all(isinstance(v, str) for v in raw):
            raise ContractError("dropped source keys must be a string array")
        dropped = tuple(raw)
        epoch_raw = payload.get("current_epoch")
        epoch = None if epoch_raw is None else _integer(epoch_raw, name="current epoch")
    else:
        raise ContractError(f"unsupported inference checkpoint schema {schema!r}")
    return InferenceCheckpointState(
        identity=_identity(payload.get("identity")),
        current_epoch=epoch,
        spatial_dims=_integer(payload.get("spatial_dims"), name="spatial dimensions"),
        inference_allowed_mirroring_axes=_int_tuple(
            payload.get("inference_allowed_mirroring_axes"), name="mirroring axes"),
        dropped_source_keys=dropped,
    )


def _verify_file_set(directory: Path, payload_files: tuple[str, ...]) -> None:
    expected = {*payload_files, "state.json"}
    actual = {p.name for p in directory.iterdir()}
    if actual != expected:
        raise ContractError(
            f"checkpoint file set mismatch: expected {sorted(expected)}, found {sorted(actual)}"
        )


def read_weights(directory: str | Path) -> dict[str, np.ndarray]:
    """float32 host weights from ``weights.safetensors``; non-finite tensors are rejected."""
    from safetensors.numpy import load_file

    weights = load_file(str(Path(directory) / "weights.safetensors"))
    out: dict[str, np.ndarray] = {}
    for name, value in weights.items():
        array = np.asarray(value, dtype=np.float32)
        if not np.isfinite(array).all():
            raise ContractError(f"model tensor {name!r} is non-finite")
        out[name] = array
    return out


def load_inference_checkpoint(directory: str | Path, *, model) -> InferenceCheckpointState:
    """Validate the checkpoint, then load its weights strictly into ``model``."""
    state = read_state(directory)
    model.load_weights(read_weights(directory), strict=True)
    return state


def save_inference_checkpoint(directory: str | Path, *, weights: Mapping[str, np.ndarray],
                              state: InferenceCheckpointState) -> None:
    """Write a new converted inference checkpoint directory."""
    from safetensors.numpy import save_file

    target = Path(directory)
    target.mkdir(parents=True, exist_ok=False)
    save_file({k: np.ascontiguousarray(v, dtype=np.float32) for k, v in weights.items()},
              str(target / "weights.safetensors"))
    (target / "state.json").write_text(
        json.dumps(state.to_payload(), indent=2, sort_keys=True) + "\n", encoding="utf-8")


def checkpoint_weights_signature(directory: str | Path) -> list[int]:
    """``[size_bytes, mtime_ns]`` of the weights file (a change detector, not a digest)."""
    weights = Path(directory) / "weights.safetensors"
    try:
        meta = weights.stat()
    except OSError as error:
        raise ContractError(f"checkpoint weights are unavailable: {weights}") from error
    return [meta.st_size, meta.st_mtime_ns]
