"""CPU checks of bench.py's contract pieces that need no GPU: the kernel-name to kernel-class
map its roofline and traffic summaries use, and the one-GPU refusal."""

from __future__ import annotations

import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def test_kernel_names_map_to_the_profiled_classes():
    sys.path.insert(0, str(ROOT))
    import bench

    cases = {
        "wino_x3_kernel": "conv3d_wino",
        "wino_x3p_kernel": "conv3d_wino",
        "igemm_x3_kernel<2, 2, 2, 2, 7, true, 0>": "conv3d_x3_m64n64",
        "igemm_x3_kernel<2, 4, 2, 2, 7, true, 0>": "conv3d_x3_m64n128",
        "igemm_x3s_kernel<4, 2, 4, 1, 7, true, 1>": "conv3d_x3s_bf16_m256n32",
        "igemm_kernel<4, 4, 4, 1, false>": "conv3d_igemm_m256n64",
        "accumulate_kernel<false>": None,
    }
    for name, cls in cases.items():
        assert bench.kernel_class_of(name) == cls, name
    short = bench._short_kernel("void nnx::(anonymous namespace)::wino_x3p_kernel("
                                "nnx::(anonymous namespace)::WinoArgs)")
    assert short == "wino_x3p_kernel"


def test_more_than_one_gpu_is_refused():
    proc = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"],
                          capture_output=True, text=True, timeout=300)
    assert proc.returncode == 2
    assert "one GPU" in proc.stderr
