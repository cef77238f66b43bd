"""Named model ``nnunet-pancreas``: segmentation of the pancreas and its tumours in CT.

Reference: src/nnunet_mlx/named_models/pancreas.py:12-49.
"""

from __future__ import annotations

from nnunet_mlx import medmlx
from nnunet_mlx.named_models import READINESS, PathLike, model_folder, segment_folder

MODEL = {
    "id": "nnunet-pancreas", "label": "Pancreas segmentation", "task": "segmentation",
    "readiness": READINESS, "run": "nnunet_mlx.named_models.pancreas:run",
    # Measured MI355X device peak (library workspace + torch allocations) for a 101x768x768
    # CT, ResEnc-L in bf16-mixed, 32 patches a forward (bench.py --workload pancreas-sw);
    # larger inputs need more.
    "peak_memory_gb": 75.3,
    "summary": "PancCTMultiTalentV2 pancreas and cancer segmentation.",
    "labels": {"1": "pancreas", "2": "cancer"},
}


def run(*, image_path: PathLike, output_dir: PathLike, weights_path: PathLike | None = None,
        overwrite: bool = False, fold: int = 0, use_mirroring: bool = True) -> dict:
    """Label one CT volume (NIfTI): 1 = pancreas, 2 = tumour.  Runs the ``3d_fullres_bs4``
    configuration from converted checkpoint slot ``fold`` (slot 0 holds the network
    trained on all data)."""
    images, _ = medmlx.check_request([image_path], output_dir=output_dir, overwrite=overwrite,
                                     folds=[fold], use_mirroring=use_mirroring)
    folder = model_folder("nnunet-pancreas", weights_path)
    return segment_folder(folder, images, output_dir, "3d_fullres_bs4", [fold],
                          overwrite=overwrite, grid_of="image_path", use_mirroring=use_mirroring)
