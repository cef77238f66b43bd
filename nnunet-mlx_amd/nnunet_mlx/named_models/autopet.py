"""Named model ``nnunet-autopet``: nnU-Net lesion segmentation of whole-body PET/CT
(AutoPET II).

Reference: src/nnunet_mlx/named_models/autopet.py:14-57.
"""

from __future__ import annotations

from collections.abc import Mapping

from nnunet_mlx import medmlx
from nnunet_mlx.named_models import (READINESS, PathLike, input_channels, model_folder,
                                     segment_folder)

MODEL = {
    "id": "nnunet-autopet", "label": "nnU-Net AutoPET II", "task": "segmentation",
    "readiness": READINESS, "run": "nnunet_mlx.named_models.autopet:run",
    # Measured MI355X device peak (library workspace + torch allocations) for a 2x284x400x400
    # case, five folds, 8 mirror views, 32 views a forward (bench.py --workload autopet-sw);
    # larger inputs need more.
    "peak_memory_gb": 51.4,
    "summary": "Tumor lesion segmentation of co-registered CT and SUV PET volumes.",
    "labels": {"1": "tumor"},
}

CHANNELS = ("ct", "pet")


def run(*, image_paths: Mapping[str, PathLike], output_dir: PathLike,
        weights_path: PathLike | None = None, overwrite: bool = False,
        use_mirroring: bool = True, step_fraction: float = 0.5) -> dict:
    """Label tumour lesions from the mapping ``{"ct": ..., "pet": ...}`` (co-registered CT
    and SUV PET, NIfTI), averaging all folds of the ``3d_fullres_resenc_bs80``
    configuration."""
    channels = input_channels(image_paths, CHANNELS)
    images, _ = medmlx.check_request(list(channels.values()), output_dir=output_dir,
                                     overwrite=overwrite, use_mirroring=use_mirroring,
                                     step_fraction=step_fraction)
    folder = model_folder("nnunet-autopet", weights_path)
    return segment_folder(folder, images, output_dir, "3d_fullres_resenc_bs80", None,
                          overwrite=overwrite, grid_of="image_paths",
                          use_mirroring=use_mirroring, step_fraction=step_fraction)
