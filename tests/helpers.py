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


def install_package(target) -> "Path":
    """pip-install this repository (offline, no dependencies) into ``target``; returns the
    directory holding the console scripts."""
    import subprocess
    import sys
    from pathlib import Path

    root = Path(__file__).resolve().parents[1]
    subprocess.run([sys.executable, "-m", "pip", "install", "--quiet", "--no-deps", "--no-index",
                    "--no-build-isolation", "--target", str(target), str(root)],
                   check=True, capture_output=True, text=True)
    return Path(target) / "bin"
