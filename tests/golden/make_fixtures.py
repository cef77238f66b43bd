"""Extract the data fixtures the parity tests use from the reference's tracked files.

Reads /root/reference/tests/fixtures/darwin-arm64/upstream_runner.npz (numpy, no pickle)
and keeps only the arrays the tests consume:
  * rounding_input_0..6 and rounding_output_{1,2,3,7}: fp16 fold-average rounding probes
    recorded from upstream nnU-Net (used by the reference at
    tests/host/test_upstream_runner_recording.py:226-246);
  * head_{logits,probabilities,segmentation}_{class,region}: softmax/sigmoid head and
    argmax/region decoding (tests/host/test_upstream_runner_recording.py:150-169).
Writes tests/golden/upstream_runner_subset.npz.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np

SOURCE = Path("/root/reference/tests/fixtures/darwin-arm64/upstream_runner.npz")
TARGET = Path(__file__).resolve().parent / "upstream_runner_subset.npz"


def main() -> None:
    data = np.load(SOURCE, allow_pickle=False)
    keep = [k for k in data.files if k.startswith(("rounding_", "head_"))]
    np.savez_compressed(TARGET, **{k: data[k] for k in keep})
    print(f"wrote {TARGET} with {sorted(keep)}")


if __name__ == "__main__":
    main()
