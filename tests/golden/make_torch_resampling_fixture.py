"""Copy the reference's recorded upstream Torch-grid resampling outputs into this tree.

  torch_resampling.npz  from the reference's tests/fixtures/darwin-arm64/torch_resampling.npz
                        (recorded from upstream nnU-Net 17cb295's resample_torch_fornnunet
                        and export code with torch 2.13): every label-resampling case
                        ("<case>-input" / "<case>-expected", int16 labels), the class-model
                        restoration cases (even "pipeline-<k>-*": logits, probabilities,
                        segmentation, label-only) and "metadata" (JSON: the cases' target
                        shapes, spacings and resampler options; the restoration cases' plans,
                        properties and cropping geometry).

Data only: arrays and their JSON description, loaded without pickle.  Run from the
repository root in a container that has the reference checked out:
    python tests/golden/make_torch_resampling_fixture.py
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np

SOURCE = Path("/root/reference/tests/fixtures/darwin-arm64/torch_resampling.npz")
TARGET = Path(__file__).resolve().parent / "torch_resampling.npz"


def main() -> None:
    with np.load(SOURCE, allow_pickle=False) as saved:
        metadata = json.loads(str(saved["metadata"].item()))
        keep = {}
        for case in metadata["cases"]:
            name = case["name"]
            if case["kwargs"].get("is_seg") is True:
                keep[f"{name}-input"] = saved[f"{name}-input"]
                keep[f"{name}-expected"] = saved[f"{name}-expected"]
        pipeline = [case for case in metadata["pipeline"] if not case["regions"]]
        for case in pipeline:
            for part in ("logits", "probabilities", "segmentation", "label-only"):
                keep[f"{case['name']}-{part}"] = saved[f"{case['name']}-{part}"]
    description = {
        "cases": [case for case in metadata["cases"] if case["kwargs"].get("is_seg") is True],
        "pipeline": pipeline,
        "source": "upstream nnU-Net " + metadata["reference_commit"] + ", torch " + metadata["torch"],
    }
    np.savez_compressed(TARGET, metadata=np.array(json.dumps(description)), **keep)
    print(f"wrote {TARGET} ({len(keep)} arrays)")


if __name__ == "__main__":
    main()
