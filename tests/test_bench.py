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


def test_kernel_table_prices_each_class_on_its_own_unit():
    """Split-fp16 classes report their issued fraction of the dense fp16 MFMA peak (three
    products per float32 product; the Winograd class 64 transform positions per 8 x 27
    taps), the HBM-bound head its fraction of HBM, and the roofline object follows the
    class with the largest share of the time."""
    sys.path.insert(0, str(ROOT))
    import bench

    classes = {
        "conv3d_wino": {"ms": 100.0, "flops": 4.0e13, "bytes": 0.0, "launches": 16},
        "conv3d_x3_m64n64": {"ms": 10.0, "flops": 1.5e12, "bytes": 0.0, "launches": 3},
        "tconv3d_x3": {"ms": 5.0, "flops": 7.0e11, "bytes": 1.0e10, "launches": 5},
        "tconv3d_x3_bf16": {"ms": 5.0, "flops": 7.0e11, "bytes": 1.0e10, "launches": 5},
        "conv1x1_head": {"ms": 2.0, "flops": 1.0e10, "bytes": 9.0e9, "launches": 1},
        "instnorm_merge": {"ms": 1.0, "flops": 0.0, "bytes": 1.0e9, "launches": 22},
    }
    k, roof = bench.kernel_table(classes, 1, traffic=False)
    p16 = bench.PEAK_FP16_MFMA_TFLOPS
    assert k["conv3d_wino"]["tflops"] == 400.0
    assert abs(k["conv3d_wino"]["frac_fp16_mfma_issued"] - 400.0 * 3 * 64 / 216 / p16) < 1e-4
    assert abs(k["conv3d_x3_m64n64"]["frac_fp16_mfma_issued"] - 150.0 * 3 * 28 / 27 / p16) < 1e-4
    assert abs(k["tconv3d_x3"]["frac_fp16_mfma_issued"] - 140.0 * 3 / p16) < 1e-4
    assert abs(k["tconv3d_x3_bf16"]["frac_bf16_mfma_issued"] - 140.0 / p16) < 1e-4
    assert k["tconv3d_x3"]["gbs"] == 2000.0 and "frac_fp32_mfma" not in k["tconv3d_x3"]
    assert k["conv1x1_head"]["gbs"] == 4500.0
    assert abs(k["conv1x1_head"]["frac_hbm"] - 4500.0 / bench.PEAK_HBM_GBS) < 1e-4
    assert k["instnorm_merge"]["gbs"] == 1000.0
    assert roof["kernel"] == "conv3d_wino" and roof["peak"] == p16 and roof["bound"] == "mfma"
    assert roof["frac"] == round(400.0 / p16, 4)


def test_more_than_one_gpu_is_refused():
    proc = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"],
                          capture_output=True, text=True, timeout=300)
    assert proc.returncode == 2
    assert "one GPU" in proc.stderr
