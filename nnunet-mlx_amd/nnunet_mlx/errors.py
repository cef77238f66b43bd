"""Error types of the nnU-Net HIP inference path.

``ContractError`` keeps the reference's semantics (src/nnunet_mlx/errors.py:4): a
``ValueError`` raised for contract violations and non-finite results.
"""

from __future__ import annotations


class ContractError(ValueError):
    """An input, model or result violates the inference contract."""


class NativeError(RuntimeError):
    """The HIP library reported a runtime failure (device error, allocation failure)."""
