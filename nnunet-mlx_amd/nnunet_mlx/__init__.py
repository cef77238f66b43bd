"""nnU-Net v2 inference on AMD Instinct MI355X (gfx950) with hand-written HIP kernels.

Drop-in for the network forward and the Gaussian sliding-window predictor of
MedMLX/nnunet-mlx: same module layout (``nnunet_mlx.model``, ``nnunet_mlx.prediction``,
``nnunet_mlx.storage``), class and function names, parameter names and converted
checkpoint folders.  Compute runs in libnnunet_hip.so (``nnunet_mlx._native``); there is
no CPU fallback.  Importing the package does not load torch or the HIP library.
"""

from __future__ import annotations

from nnunet_mlx.errors import ContractError
from nnunet_mlx.model.topology import PlainConvUNetSpec, ResidualEncoderUNetSpec

__version__ = "0.1.0"

__all__ = [
    "ContractError",
    "PlainConvUNetSpec",
    "ResidualEncoderUNetSpec",
    "load_model",
    "load_model_bundle",
    "run",
]


def __getattr__(name: str):
    if name == "load_model_bundle":
        from nnunet_mlx.model.folder import load_model_bundle

        return load_model_bundle
    if name in ("run", "load_model"):
        from nnunet_mlx import medmlx

        return getattr(medmlx, name)
    raise AttributeError(name)
