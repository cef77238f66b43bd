"""Named model ``nnunet-liver``: nnU-Net segmentation of the liver and its tumours in CT.

Reference: src/nnunet_mlx/named_models/liver.py:12-99.
"""

from __future__ import annotations

from nnunet_mlx import medmlx
from nnunet_mlx.named_models import READINESS, PathLike, model_folder, segment_folder

MODEL = {
    "id": "nnunet-liver", "label": "nnU-Net liver CT", "task": "segmentation",
    "readiness": READINESS, "run": "nnunet_mlx.named_models.liver:run",
    "cohort": "nnunet_mlx.named_models.liver:load_model",
    # Measured MI355X device peak (library workspace + torch allocations) for a 512x512x120
    # liver CT preprocessed to 300x534x534, 8 mirror views, 32 views a forward (bench.py
    # --workload liver-raw-case); larger inputs need more.
    "peak_memory_gb": 63.3,
    "summary": "Liver and liver cancer segmentation of one CT volume.",
    "labels": {"1": "liver", "2": "cancer"},
}


def run(*, image_path: PathLike, output_dir: PathLike, weights_path: PathLike | None = None,
        overwrite: bool = False, use_mirroring: bool = True, step_fraction: float = 0.5) -> dict:
    """Label one Hounsfield-unit CT volume (NIfTI): 1 = liver, 2 = tumour, 0 elsewhere.
    The label map keeps the input's voxel grid and is written as ``mask.nii.gz`` in
    ``output_dir``.  Defaults reproduce the published setup: every test-time flip of the
    three axes (8 forwards per tile) and tiles half a patch apart."""
    images, _ = medmlx.check_request([image_path], output_dir=output_dir, overwrite=overwrite,
                                     use_mirroring=use_mirroring, step_fraction=step_fraction)
    folder = model_folder("nnunet-liver", weights_path)
    return segment_folder(folder, images, output_dir, "3d_fullres", None, overwrite=overwrite,
                          grid_of="image_path", use_mirroring=use_mirroring,
                          step_fraction=step_fraction)


class LiverModel:
    """A resident liver model: weights go to the GPU once, then :meth:`run` labels one CT
    per call with the options given to :func:`load_model`."""

    def __init__(self, model: medmlx.NnUNetModel) -> None:
        self._model = model

    def run(self, *, image_path: PathLike, output_dir: PathLike, overwrite: bool = False) -> dict:
        return self._model.segment_case(image_paths=[image_path], output_dir=output_dir,
                                        overwrite=overwrite, grid_of="image_path")

    def close(self) -> None:
        self._model.close()

    def __enter__(self) -> "LiverModel":
        return self

    def __exit__(self, *args: object) -> None:
        self.close()


def load_model(*, weights_path: PathLike | None = None, use_mirroring: bool = True,
               step_fraction: float = 0.5) -> LiverModel:
    """Put the liver model on the GPU for repeated :meth:`LiverModel.run` calls."""
    folder = model_folder("nnunet-liver", weights_path)
    return LiverModel(medmlx.load_model(weights_path=folder, configuration="3d_fullres",
                                        use_mirroring=use_mirroring,
                                        step_fraction=step_fraction))
