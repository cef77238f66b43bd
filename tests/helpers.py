"""Small shared helpers for the GPU parity tests."""

from __future__ import annotations

import numpy as np
import torch

from nnunet_mlx import _native


def dev(array: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(array)).cuda()


def host(tensor: torch.Tensor) -> np.ndarray:
    torch.cuda.synchronize()
    return tensor.cpu().numpy()


def stream() -> int:
    return _native.stream_handle()


def rel_l2(actual: np.ndarray, expected: np.ndarray) -> float:
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    return float(np.linalg.norm(a - e) / max(np.linalg.norm(e), 1e-300))


def report(name: str, actual: np.ndarray, expected: np.ndarray) -> str:
    diff = np.abs(np.asarray(actual, np.float64) - np.asarray(expected, np.float64))
    return f"{name}: max_abs={diff.max():.3e} rel_l2={rel_l2(actual, expected):.3e}"
