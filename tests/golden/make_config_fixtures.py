"""Write the oracle fixtures of the real-shape workloads (CPU, a few minutes).

  config_forwards.npz      probes (tests/golden/config_cases.py:probe) of the CPU oracle's
                           float32 logits for batch items 0 and 31 of every workload in
                           config_cases.WORKLOADS, and of its bf16 emulation for the
                           pancreas ResEnc-L; keys "<workload>__<item>__<arithmetic>__<probe>"
  liver_volume_digest.json SHA-256 of the oracle sliding window's logits (float32, C order,
                           (101, 768, 768, 3)) and labels (uint16) over the full liver-shape
                           volume with a pointwise model, 8 mirror views, patch 128^3, step
                           0.5, in float32 and nnunet-fp16 accumulation

Run from the repository root: python tests/golden/make_config_fixtures.py
"""

from __future__ import annotations

import hashlib
import json
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
for path in (ROOT / "nnunet-mlx_amd", ROOT):
    if str(path) not in sys.path:
        sys.path.insert(0, str(path))

from nnunet_mlx.model.topology import ResidualEncoderUNetSpec  # noqa: E402
from nnunet_mlx.storage.synthetic import random_weights  # noqa: E402
from oracle import sliding_window as osw  # noqa: E402
from oracle.network import OracleNetwork  # noqa: E402
from tests.golden import config_cases as cc  # noqa: E402

HERE = Path(__file__).resolve().parent
LIVER_VOLUME_SHAPE = (1, 101, 768, 768)
LIVER_VOLUME_SEED = 101


class PointwiseModel:
    """Three pointwise classes of a one-channel input: (1.5 v, -1.5 v, v * v)."""

    def __call__(self, values: np.ndarray) -> np.ndarray:
        s = np.float32(1.5)
        return np.concatenate((values * s, -values * s, values * values), axis=-1)


def liver_volume() -> np.ndarray:
    return np.random.default_rng(LIVER_VOLUME_SEED).standard_normal(LIVER_VOLUME_SHAPE,
                                                                    dtype=np.float32)


def digest(array: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(array).tobytes()).hexdigest()


def forwards() -> None:
    out = {}
    for name, w in cc.WORKLOADS.items():
        spec = w["spec"]
        weights = random_weights(spec, seed=w["seed"])
        residual = isinstance(spec, ResidualEncoderUNetSpec)
        x = np.stack([cc.item_input(name, i) for i in cc.ITEMS])
        kinds = [("fp32", False)] + ([("bf16emu", True)] if name == "pancreas" else [])
        for label, bf16 in kinds:
            t = time.time()
            y = OracleNetwork(spec, weights, residual=residual, bf16=bf16)(x)
            print(f"{name} {label}: {time.time() - t:.1f} s", flush=True)
            for item, logits in zip(cc.ITEMS, y):
                for key, value in cc.probe(logits).items():
                    out[f"{name}__{item}__{label}__{key}"] = value
    np.savez_compressed(HERE / "config_forwards.npz", **out)


def liver_digests() -> None:
    data = liver_volume()
    result = {"shape": list(LIVER_VOLUME_SHAPE), "seed": LIVER_VOLUME_SEED,
              "patch": [128, 128, 128], "axes": [0, 1, 2], "num_classes": 3}
    for accumulation in ("float32", "nnunet-fp16"):
        t = time.time()
        logits, labels = osw.predict([PointwiseModel()], data, (128, 128, 128), num_classes=3,
                                     axes=(0, 1, 2), accumulation=accumulation)
        print(f"liver volume {accumulation}: {time.time() - t:.1f} s", flush=True)
        result[accumulation] = {"logits_sha256": digest(logits), "labels_sha256": digest(labels),
                                "logits_dtype": str(logits.dtype),
                                "label_counts": np.bincount(labels.reshape(-1)).tolist()}
    (HERE / "liver_volume_digest.json").write_text(json.dumps(result, indent=1) + "\n")


if __name__ == "__main__":
    which = sys.argv[1:] or ["forwards", "liver"]
    if "forwards" in which:
        forwards()
    if "liver" in which:
        liver_digests()
