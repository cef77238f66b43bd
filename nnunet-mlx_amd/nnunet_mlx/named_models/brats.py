"""Named model ``nnunet-brats2021``: nnU-Net brain-tumour segmentation of four MRI
sequences.

Reference: src/nnunet_mlx/named_models/brats.py:15-62.
"""

from __future__ import annotations

from collections.abc import Mapping

from nnunet_mlx import medmlx
from nnunet_mlx.errors import ContractError
from nnunet_mlx.named_models import (READINESS, PathLike, input_channels, model_folder,
                                     segment_folder)

MODEL = {
    "id": "nnunet-brats2021", "label": "nnU-Net BraTS 2021", "task": "segmentation",
    "readiness": READINESS, "run": "nnunet_mlx.named_models.brats:run",
    # Measured MI355X device peak (library workspace + torch allocations) for a 4x155x240x240
    # case, five folds, 8 mirror views, 32 views a forward (bench.py --workload brats-sw);
    # larger inputs need more.
    "peak_memory_gb": 62.4,
    "summary": "Dataset002_BRATS19 with its original BAMF labels.",
    "labels": {"1": "edema", "2": "nonenhancing", "3": "empty", "4": "enhancing"},
}

CHANNELS = ("t1", "t1ce", "t2", "flair")


def run(*, image_paths: Mapping[str, PathLike], output_dir: PathLike,
        weights_path: PathLike | None = None, overwrite: bool = False, fold: int | None = None,
        use_mirroring: bool = True) -> dict:
    """Label a brain tumour from the mapping ``{"t1": ..., "t1ce": ..., "t2": ..., "flair":
    ...}`` of co-registered NIfTI volumes.  The five trained folds are averaged; an integer
    ``fold`` between 0 and 4 uses that fold alone."""
    if fold is not None and (isinstance(fold, bool) or fold not in range(5)):
        raise ContractError("BraTS fold must be between 0 and 4")
    channels = input_channels(image_paths, CHANNELS)
    images, _ = medmlx.check_request(list(channels.values()), output_dir=output_dir,
                                     overwrite=overwrite,
                                     folds=None if fold is None else [fold],
                                     use_mirroring=use_mirroring)
    folder = model_folder("nnunet-brats2021", weights_path)
    folds = list(range(5)) if fold is None else [fold]
    return segment_folder(folder, images, output_dir, "3d_fullres", folds, overwrite=overwrite,
                          grid_of="image_paths", use_mirroring=use_mirroring)
