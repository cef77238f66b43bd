"""Released nnU-Net models, one module each, with fixed configurations.

Reference: src/nnunet_mlx/named_models/__init__.py:21-37 and the per-model modules.  Each
module declares ``MODEL`` and ``run`` (and ``load_model`` where the reference has one);
``outputs["mask"]`` is the label map on the input grid.  Weights are never downloaded
here: ``weights_path`` must name a local converted model folder.
"""

from __future__ import annotations

import os
from collections.abc import Mapping, Sequence
from pathlib import Path

from nnunet_mlx import medmlx
from nnunet_mlx.errors import ContractError

PathLike = str | os.PathLike
READINESS = "nnunet_mlx.medmlx:check_request"


def model_folder(model_id: str, weights_path: PathLike | None) -> Path:
    """The local model folder of ``model_id``; downloads are not available."""
    if weights_path is None:
        raise ContractError(f"{model_id}: weight download is not available; pass weights_path "
                            "(a local converted model folder)")
    folder = Path(weights_path).expanduser()
    if not folder.is_dir():
        raise ContractError(f"{model_id}: model folder does not exist: {folder}")
    return folder


def input_channels(image_paths: Mapping[str, PathLike], names: Sequence[str]) -> dict[str, PathLike]:
    """Images keyed exactly by the model's channel names, in network channel order."""
    if not isinstance(image_paths, Mapping) or set(image_paths) != set(names):
        raise ContractError(f"image_paths must map exactly {list(names)} to NIfTI files")
    return {name: image_paths[name] for name in names}


def segment_folder(folder: Path, images: Sequence[Path], output_dir: PathLike,
                   configuration: str, folds: list[int] | None, *, overwrite: bool,
                   grid_of: str, use_mirroring: bool = True, step_fraction: float = 0.5) -> dict:
    """Segment one case of a released model through the generic path."""
    return medmlx.segment_case(
        grid_of=grid_of, weights_path=folder, image_paths=images, output_dir=output_dir,
        configuration=configuration, folds=folds, use_mirroring=use_mirroring,
        step_fraction=step_fraction, overwrite=overwrite)
