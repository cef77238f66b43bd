#!/usr/bin/env python3
"""Liver-shape sliding-window benchmark of the nnU-Net HIP path on one MI355X.

Workload: a synthetic z-scored CT volume (1, 101, 768, 768) float32 through a random-init
6-stage PlainConvUNet (features 32..320, 1 -> 3 classes, seed 1), patch 128^3, step 0.5
(121 tiles), Gaussian weighting sigma = patch/8, 8 mirror views per tile (968 forwards),
one fold, float32 accumulation, argmax labels.  One step = one whole case, volume already
resident in HBM, labels left in HBM.  Prints one JSON line.

The `roofline` object covers the dominant kernel (largest share of the timed region),
timed live with HIP events on its launch stream; `cpu_baseline` times the CPU oracle
(torch-CPU float32 network + numpy accumulation) on a bounded sample of the same work.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (str(ROOT / "nnunet-mlx_amd"), str(ROOT)):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "sliding-window voxels/s, liver 768²×101 8×TTA; conv3d MFMA % of peak"
PEAK_FP32_MFMA_TFLOPS = 157.3
PEAK_FP16_MFMA_TFLOPS = 2500.0   # dense
# arithmetic the path computes in, per network precision
DTYPES = {
    "fp32": "f32",
    "fp32-split": "f32 (fp16-split products, f32 accumulate)",
    "bf16": "bf16 products, f32 accumulate",
    "bf16-mixed": "bf16 products below full resolution, fp16-split at full resolution, f32 accumulate",
}
SPLIT_PRODUCTS = 3               # hi*hi + hi*lo + lo*hi per float32 product
PEAK_HBM_GBS = 8000.0
VOLUME_SHAPE = (1, 101, 768, 768)
PATCH = (128, 128, 128)


class DevicePeak:
    """Device memory a workload holds at its peak, in GB: the bytes in use on the GPU
    (hipMemGetInfo: the library's own allocations, which it keeps for reuse, and torch's
    cached blocks) above what was in use when the object was made, plus whatever part of
    torch's cached-allocator peak was released again before the reading."""

    def __init__(self) -> None:
        import torch

        torch.cuda.synchronize()
        free, total = torch.cuda.mem_get_info()
        self.base = total - free
        torch.cuda.reset_peak_memory_stats()

    def gb(self) -> float:
        import torch

        torch.cuda.synchronize()
        free, total = torch.cuda.mem_get_info()
        released = torch.cuda.max_memory_reserved() - torch.cuda.memory_reserved()
        return round((total - free - self.base + released) / 1e9, 2)


def conv_mfma_frac(classes: dict, precision: str) -> float | None:
    """Rate of the 3x3x3 convolution kernels (algorithmic float32-product FLOPs over their
    launch time) as a fraction of the MFMA peak of the arithmetic they issue: 157.3 TFLOP/s
    for float32 products, a third of the dense fp16 peak for fp16-split (three products per
    term), the dense bf16 peak for bf16."""
    conv = [c for n, c in classes.items()
            if n.startswith(("conv3d_igemm", "conv3d_x3", "conv3d_wino"))]
    flops = sum(c["flops"] for c in conv)
    ms = sum(c["ms"] for c in conv)
    peak = {"fp32": PEAK_FP32_MFMA_TFLOPS, "fp32-split": PEAK_FP16_MFMA_TFLOPS / SPLIT_PRODUCTS,
            "bf16": PEAK_FP16_MFMA_TFLOPS, "bf16-mixed": PEAK_FP16_MFMA_TFLOPS}[precision]
    return round(flops / (ms * 1e-3) / 1e12 / peak, 4) if ms else None


def liver_spec():
    from nnunet_mlx.model.topology import PlainConvUNetSpec

    return PlainConvUNetSpec(
        input_channels=1, num_classes=3, features=(32, 64, 128, 256, 320, 320),
        kernel_sizes=((3, 3, 3),) * 6, strides=((1, 1, 1),) + ((2, 2, 2),) * 5,
        encoder_convs=(2,) * 6, decoder_convs=(2,) * 5,
    )


def synthetic_ct(shape=VOLUME_SHAPE, seed: int = 101):
    """z-scored CT-like volume: 70% N(0, 0.3) soft tissue, 30% N(-2.5, 0.2) air, plus 12
    ellipsoid blobs filled with N(mu_k, 0.1), mu_k ~ U(0.5, 2)."""
    import numpy as np

    rng = np.random.default_rng(seed)
    _, Z, Y, X = shape
    air = rng.random((Z, Y, X), dtype=np.float32) < 0.3
    vol = rng.standard_normal((Z, Y, X), dtype=np.float32)
    vol *= np.where(air, np.float32(0.2), np.float32(0.3))
    vol += np.where(air, np.float32(-2.5), np.float32(0.0))
    zz, yy, xx = np.ogrid[:Z, :Y, :X]
    for _ in range(12):
        cz, cy, cx = rng.uniform(0, Z), rng.uniform(0, Y), rng.uniform(0, X)
        az, ay, ax = rng.uniform(5, 30), rng.uniform(20, 120), rng.uniform(20, 120)
        mu = rng.uniform(0.5, 2.0)
        z0, z1 = max(0, int(cz - az)), min(Z, int(cz + az) + 1)
        y0, y1 = max(0, int(cy - ay)), min(Y, int(cy + ay) + 1)
        x0, x1 = max(0, int(cx - ax)), min(X, int(cx + ax) + 1)
        inside = (((zz[z0:z1] - cz) / az) ** 2 + ((yy[:, y0:y1] - cy) / ay) ** 2
                  + ((xx[:, :, x0:x1] - cx) / ax) ** 2) <= 1.0
        block = vol[z0:z1, y0:y1, x0:x1]
        noise = (mu + 0.1 * rng.standard_normal(block.shape)).astype(np.float32)
        block[inside] = noise[inside]
    return vol[None]


# raw-case preprocessing workload: a liver-like CT as the scanner writes it (int16 HU,
# 512 x 512 slices 0.8 mm apart in-plane, 120 slices 2.5 mm apart), preprocessed to a
# 3d_fullres plan of 1.0 x 0.7676 x 0.7676 mm with CT normalisation and cubic spline data
# resampling (the anisotropic spacing selects the separate-axis path)
PREP_RAW_SHAPE = (1, 120, 512, 512)
PREP_SPACING = (2.5, 0.8, 0.8)
PREP_PLANS = {
    "transpose_forward": [0, 1, 2], "transpose_backward": [0, 1, 2],
    "foreground_intensity_properties_per_channel": {
        "0": {"mean": 99.4, "std": 137.2, "percentile_00_5": -958.0, "percentile_99_5": 327.0}},
    "configurations": {"3d_fullres": {
        "spacing": [1.0, 0.7676, 0.7676], "normalization_schemes": ["CTNormalization"],
        "use_mask_for_norm": [False], "patch_size": [128, 128, 128],
        "resampling_fn_data": "resample_data_or_seg_to_shape",
        "resampling_fn_data_kwargs": {"is_seg": False, "order": 3, "order_z": 0,
                                      "force_separate_z": None}}},
}


# the same plan with upstream's Torch-grid resampler (resample_torch_fornnunet: linear in
# plane, nearest-exact along the separate axis)
TORCH_RESAMPLING = {"resampling_fn_data": "resample_torch_fornnunet",
                    "resampling_fn_data_kwargs": {"is_seg": False, "force_separate_z": None,
                                                  "memefficient_seg_resampling": False}}


def prep_plans(resampler: str) -> dict:
    plans = json.loads(json.dumps(PREP_PLANS))
    if resampler == "torch":
        plans["configurations"]["3d_fullres"].update(TORCH_RESAMPLING)
    return plans


def synthetic_raw_ct(shape=PREP_RAW_SHAPE, seed: int = 5):
    """int16 CT: air (-1000 HU) outside an elliptic body section, N(40, 60) HU inside."""
    import numpy as np

    rng = np.random.default_rng(seed)
    _, Z, Y, X = shape
    raw = np.full(shape, -1000, dtype=np.int16)
    yy, xx = np.ogrid[:Y, :X]
    body = ((yy - Y / 2) / (0.39 * Y)) ** 2 + ((xx - X / 2) / (0.45 * X)) ** 2 <= 1
    inside = np.broadcast_to(body, (Z, Y, X))
    raw[0][inside] = (rng.standard_normal(int(body.sum()) * Z) * 60 + 40).astype(np.int16)
    return raw


def preprocess_workload(args) -> int:
    """Raw liver CT -> plans spacing on the GPU (transpose, nonzero crop, CT normalisation,
    separate-axis cubic spline resampling); value = output voxels per second."""
    import numpy as np
    import torch

    from nnunet_mlx import _native
    from nnunet_mlx.data.preprocessing import PreprocessPlan, preprocess_raw_case

    torch.cuda.set_device(0)
    raw = synthetic_raw_ct()
    torch_grid = args.resampler == "torch"
    plan = PreprocessPlan.from_plans(prep_plans(args.resampler), "3d_fullres")
    props = {"spacing": list(PREP_SPACING)}
    d_raw = torch.from_numpy(raw).cuda()
    for _ in range(max(args.warmup, 1)):
        out = preprocess_raw_case(d_raw, props, plan)
    torch.cuda.synchronize()
    with _native.KernelProfile() as prof:
        t0 = time.perf_counter()
        for _ in range(args.steps):
            out = preprocess_raw_case(d_raw, props, plan)
        torch.cuda.synchronize()
        step_s = (time.perf_counter() - t0) / args.steps
    out_vox = int(np.prod(out.data.shape[1:]))
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    host_out = preprocess_raw_case(raw, props, plan)
    torch.cuda.synchronize()
    pcie_s = time.perf_counter() - t0
    kernels = {}
    for name, c in sorted(prof.classes.items(), key=lambda kv: -kv[1]["ms"]):
        entry = {"launches": c["launches"], "ms": round(c["ms"] / args.steps, 4)}
        if c["bytes"]:
            entry["gbs"] = round(c["bytes"] / (c["ms"] * 1e-3) / 1e9, 1)
            entry["frac_hbm"] = round(entry["gbs"] / PEAK_HBM_GBS, 4)
        kernels[name] = entry
    dominant = max(prof.classes, key=lambda n: prof.classes[n]["ms"])
    d = prof.classes[dominant]
    achieved = d["bytes"] / (d["ms"] * 1e-3) / 1e9
    roofline = {"kernel": dominant, "bound": "hbm", "achieved": round(achieved, 1),
                "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBS, 4),
                "traffic": None}
    cpu = None
    if not args.no_cpu_baseline:
        from oracle import preprocess as op

        # bounded sample: the oracle's crop and normalisation of the whole case, and its
        # separate-axis resampling of 12 of the 120 slices (the in-plane work is per slice),
        # scaled to the whole case
        t0 = time.perf_counter()
        v = raw.astype(np.float32)
        bbox = op.nonzero_bbox(v)
        crop = v[(slice(None), *(slice(a, b) for a, b in bbox))]
        norm = op.ct_normalize(crop[0], 99.4, 137.2, -958.0, 327.0)[None]
        base_s = time.perf_counter() - t0
        sample = 12
        new_shape = tuple(int(s) for s in out.data.shape[1:])
        sample_shape = (round(new_shape[0] * sample / crop.shape[1]), *new_shape[1:])
        t0 = time.perf_counter()
        if torch_grid:
            from oracle import torch_resample as otr

            otr.resample(norm[:, :sample], sample_shape, axis=0)
        else:
            op.resample_data(norm[:, :sample], sample_shape, separate_axis=0)
        sample_s = time.perf_counter() - t0
        case_s = base_s + sample_s * crop.shape[1] / sample
        kind = "Torch-grid (linear, nearest-exact axis)" if torch_grid else "cubic"
        cpu = {"value": round(out_vox / case_s, 1), "unit": "voxels/s", "cores": 1, "kind": "port",
               "sample": f"oracle (numpy) crop + CT normalisation of the whole case ({base_s:.2f} s) "
                         f"and its separate-axis {kind} resampling of {sample} of "
                         f"{crop.shape[1]} slices ({sample_s:.2f} s), scaled to the case: "
                         f"{case_s:.1f} s per case"}
    resampling = ("Torch-grid resampler, linear in plane, nearest-exact separate axis"
                  if torch_grid else "cubic spline, separate axis")
    line = {
        "metric": "raw-case preprocessing output voxels/s, liver CT 512x512x120 int16 -> "
                  f"300x534x534 (CT normalisation, {resampling})",
        "value": round(out_vox / step_s, 1), "unit": "voxels/s", "n_gpus": 1, "steps": args.steps,
        "warmup": max(args.warmup, 1), "ms_per_step": round(step_s * 1e3, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32 data, f64 " + ("corner sums" if torch_grid else "spline arithmetic"),
        "data": "synthetic",
        "config": {"workload": "raw CT (1, 120, 512, 512) int16 resident in HBM at spacing "
                               "(2.5, 0.8, 0.8) mm -> plans spacing (1.0, 0.7676, 0.7676) mm",
                   "resampler": args.resampler, "output_shape": list(out.data.shape)},
        "pcie_inclusive_voxels_per_s": round(out_vox / pcie_s, 1),
        "roofline": roofline, "cpu_baseline": cpu, "kernels": kernels,
    }
    del host_out
    print(json.dumps(line), flush=True)
    return 0


def restore_workload(args) -> int:
    """Class-logit restoration of the liver raw case on the GPU: float16 channels-last
    logits of the preprocessed grid (300 x 534 x 534 x 3, what the sliding window leaves on
    the device) back to the cropped original grid (120 x 512 x 512) at spacing
    (1.0, 0.7676, 0.7676) -> (2.5, 0.8, 0.8) mm (separate axis 0), with the first-maximum
    argmax; the plans' probability resampler is the order-1 spline or the Torch-grid
    resampler (``--resampler``).  value = output voxels per second."""
    import numpy as np
    import torch

    from nnunet_mlx import _native
    from nnunet_mlx.plans import ResamplingContract
    from nnunet_mlx.prediction.restore import restore_class_labels_device

    torch.cuda.set_device(0)
    torch_grid = args.resampler == "torch"
    name = "resample_torch_fornnunet" if torch_grid else "resample_data_or_seg_to_shape"
    kwargs = {"is_seg": False, "force_separate_z": None}
    if not torch_grid:
        kwargs.update(order=1, order_z=0)
    contract = ResamplingContract.from_configuration(
        {"f": name, "f_kwargs": kwargs}, field="f", expected_is_seg=False)
    source, target = (300, 534, 534), (120, 512, 512)
    current, original = (1.0, 0.7676, 0.7676), PREP_SPACING
    rng = np.random.default_rng(3)
    # smooth-ish logits: three classes whose maxima form regions, as a network leaves them
    coarse = torch.from_numpy(rng.standard_normal((3, 38, 67, 67)).astype(np.float32))
    logits = torch.nn.functional.interpolate(coarse[None].cuda(), size=source, mode="trilinear",
                                             align_corners=False)[0]
    logits = (logits * 4).permute(1, 2, 3, 0).contiguous().half()
    del coarse
    for _ in range(max(args.warmup, 1)):
        labels = restore_class_labels_device(logits, target, current, original, contract)
    torch.cuda.synchronize()
    with _native.KernelProfile() as prof:
        t0 = time.perf_counter()
        for _ in range(args.steps):
            labels = restore_class_labels_device(logits, target, current, original, contract)
        torch.cuda.synchronize()
        step_s = (time.perf_counter() - t0) / args.steps
    out_vox = int(np.prod(target))
    kernels = {}
    for kname, c in sorted(prof.classes.items(), key=lambda kv: -kv[1]["ms"]):
        entry = {"launches": c["launches"], "ms": round(c["ms"] / args.steps, 4)}
        if c["bytes"]:
            entry["gbs"] = round(c["bytes"] / (c["ms"] * 1e-3) / 1e9, 1)
            entry["frac_hbm"] = round(entry["gbs"] / PEAK_HBM_GBS, 4)
        kernels[kname] = entry
    dominant = max(prof.classes, key=lambda n: prof.classes[n]["ms"])
    d = prof.classes[dominant]
    achieved = d["bytes"] / (d["ms"] * 1e-3) / 1e9
    roofline = {"kernel": dominant, "bound": "hbm", "achieved": round(achieved, 1),
                "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBS, 4),
                "traffic": None}
    cpu = None
    if not args.no_cpu_baseline:
        # bounded sample: the oracle's restoration of the first 30 of 300 source slices
        # (-> 12 target slices; the separate-axis pass is nearest along axis 0, so slabs
        # are independent), scaled to the case
        host = logits[:30].float().cpu().numpy()
        t0 = time.perf_counter()
        if torch_grid:
            from oracle import torch_resample as otr

            otr.resample(np.moveaxis(host, -1, 0), (12, *target[1:]), axis=0).argmax(axis=0)
        else:
            from oracle.restore import restore_labels_spline

            restore_labels_spline(host.astype(np.float16), (12, *target[1:]), order=1,
                                  separate_axis=0)
        sample_s = time.perf_counter() - t0
        case_s = sample_s * target[0] / 12
        cpu = {"value": round(out_vox / case_s, 1), "unit": "voxels/s", "cores": 1, "kind": "port",
               "sample": f"oracle (numpy) restoration of 30 of 300 source slices -> 12 of 120 "
                         f"target slices ({sample_s:.2f} s), scaled to the case: "
                         f"{case_s:.1f} s per case"}
    resampling = ("Torch-grid resampler, linear in plane, nearest-exact separate axis"
                  if torch_grid else "order-1 spline, separate axis")
    line = {
        "metric": "class-logit restoration output voxels/s, liver case 300x534x534x3 float16 "
                  f"logits -> 120x512x512 labels ({resampling}, first-maximum argmax)",
        "value": round(out_vox / step_s, 1), "unit": "voxels/s", "n_gpus": 1, "steps": args.steps,
        "warmup": max(args.warmup, 1), "ms_per_step": round(step_s * 1e3, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f16 logits, f64 interpolation", "data": "synthetic",
        "config": {"workload": "float16 logits (300, 534, 534, 3) resident in HBM, spacing "
                               "(1.0, 0.7676, 0.7676) -> (2.5, 0.8, 0.8) mm",
                   "resampler": args.resampler,
                   "label_counts": torch.bincount(labels.view(torch.int16).long().flatten(),
                                                  minlength=3).tolist()},
        "roofline": roofline, "cpu_baseline": cpu, "kernels": kernels,
    }
    print(json.dumps(line), flush=True)
    return 0


def _short_kernel(name: str) -> str:
    import re

    name = name.replace("void ", "").replace("nnx::(anonymous namespace)::", "")
    return re.split(r"\((?!anon)", name)[0].strip()


def kernel_class_of(short: str) -> str | None:
    """Map a rocprof kernel name to the profiling class bench.py reports
    (igemm_kernel<MB, NB, WM, WN, ...> -> conv3d_igemm_m{16*MB*WM}n{16*NB*WN}, the
    split-fp16 kernels igemm_x3s_kernel / igemm_x3_kernel -> conv3d_x3s_* / conv3d_x3_*, and
    both Winograd kernels, one box a workgroup and persistent, -> conv3d_wino)."""
    import re

    if short.startswith(("wino_x3_kernel", "wino_x3p_kernel")):
        return "conv3d_wino"
    m = re.match(r"igemm(_x3s|_x3)?_kernel<(\d+), (\d+), (\d+), (\d+)([^>]*)>", short)
    if not m:
        return None
    prefix = {None: "conv3d_igemm", "_x3s": "conv3d_x3s", "_x3": "conv3d_x3"}[m.group(1)]
    if m.group(1) and m.group(6).split(",")[-1].strip() == "1":  # bf16 arithmetic
        prefix += "_bf16"
    mb, nb, wm, wn = (int(g) for g in m.groups()[1:5])
    return f"{prefix}_m{16 * mb * wm}n{16 * nb * wn}"


TRAFFIC_FILE = ROOT / "profiles" / "hbm_traffic_liver_case.md"
SOURCES_LINE = "Kernel sources sha256: "


def kernel_sources_digest() -> str:
    """SHA-256 (16 hex digits) of the HIP sources and the C-ABI header: a counter summary
    describes the kernels built from exactly these sources."""
    import hashlib

    h = hashlib.sha256()
    files = sorted((ROOT / "nnunet-mlx_amd" / "csrc").glob("*.hip"))
    files += sorted((ROOT / "nnunet-mlx_amd" / "csrc").glob("*.h")) + [ROOT / "include" / "nnx.h"]
    for f in files:
        h.update(f.name.encode())
        h.update(f.read_bytes())
    return h.hexdigest()[:16]


def summarize_profiles(directory: str) -> None:
    """Write the profiles/ summaries from rocprofv3 CSV output under `directory`
    (prof_trace/liver_kernel_stats.csv, prof_fetch/fetch_counter_collection.csv,
    prof_write/write_counter_collection.csv)."""
    import csv
    from collections import defaultdict

    base = Path(directory)
    out = ROOT / "profiles"
    out.mkdir(exist_ok=True)
    rows = list(csv.DictReader(open(base / "prof_trace" / "liver_kernel_stats.csv")))
    lines = [
        "# Kernel time, liver-shape sliding window (121 tiles x 8 views), warmup + 1 timed case",
        "",
        "Command (repo root on the MI355X box):",
        "",
        "    rocprofv3 --kernel-trace --stats -f csv -d gpurun_out/prof_trace -o liver -- \\",
        "        python -u bench.py --warmup 1 --steps 1 --no-cpu-baseline --no-pcie --no-alt",
        "",
        "Calls count the warmup and the timed case (2 cases). Average = per launch.",
        "",
        "| kernel | calls | total ms | average us | % |",
        "|---|---:|---:|---:|---:|",
    ]
    for r in rows[:16]:
        lines.append(f"| `{_short_kernel(r['Name'])}` | {r['Calls']} | {float(r['TotalDurationNs'])/1e6:.1f} | "
                     f"{float(r['AverageNs'])/1e3:.1f} | {float(r['Percentage']):.2f} |")
    (out / "kernel_stats_liver.md").write_text("\n".join(lines) + "\n")

    per = defaultdict(dict)
    for name, ctr in (("prof_fetch/fetch_counter_collection.csv", "FETCH_SIZE"),
                      ("prof_write/write_counter_collection.csv", "WRITE_SIZE")):
        for r in csv.DictReader(open(base / name)):
            if r["Counter_Name"] == ctr:
                per[(int(r["Dispatch_Id"]), _short_kernel(r["Kernel_Name"]))][ctr] = float(r["Counter_Value"])
    calib = {k[1]: v for k, v in per.items() if "neg_kernel" in k[1]}
    (neg,) = calib.values()
    gib_kib = 1024.0 * 1024.0
    fetch_factor = gib_kib / neg["FETCH_SIZE"]
    write_factor = gib_kib / neg["WRITE_SIZE"]
    agg = defaultdict(lambda: [0, 0.0, 0.0])
    for (_, short), v in per.items():
        a = agg[short]
        a[0] += 1
        a[1] += v.get("FETCH_SIZE", 0.0) * fetch_factor * 1024
        a[2] += v.get("WRITE_SIZE", 0.0) * write_factor * 1024
    lines = [
        "# HBM traffic per launch, liver-shape case (121 tiles x 8 views, 32 views a forward batch)",
        "",
        "Commands (repo root on the MI355X box), one counter per run:",
        "",
        "    rocprofv3 --pmc FETCH_SIZE -f csv -d gpurun_out/prof_fetch -o fetch -- \\",
        "        python -u bench.py --warmup 0 --steps 1 --no-cpu-baseline --no-pcie --no-alt --copy-calibration",
        "    rocprofv3 --pmc WRITE_SIZE -f csv -d gpurun_out/prof_write -o write -- \\",
        "        python -u bench.py --warmup 0 --steps 1 --no-cpu-baseline --no-pcie --no-alt --copy-calibration",
        "",
        f"Calibration: torch.neg over 1 GiB (reads 1 GiB, writes 1 GiB) reads FETCH_SIZE = "
        f"{neg['FETCH_SIZE']:.0f} KiB and WRITE_SIZE = {neg['WRITE_SIZE']:.0f} KiB, so FETCH_SIZE is "
        f"scaled by {fetch_factor:.4f} and WRITE_SIZE by {write_factor:.4f}.",
        "",
        f"{SOURCES_LINE}{kernel_sources_digest()} (bench.py reports this traffic only while the "
        "sources are unchanged).",
        "",
        "| kernel | launches | fetch bytes/launch | write bytes/launch | traffic bytes/launch |",
        "|---|---:|---:|---:|---:|",
    ]
    for short, (n, f, w) in sorted(agg.items(), key=lambda kv: -(kv[1][1] + kv[1][2])):
        if n == 0 or (f + w) / n < 1e6:
            continue
        cls = kernel_class_of(short) or short
        lines.append(f"| `{cls}` | {n} | {f/n:.4g} | {w/n:.4g} | {(f+w)/n:.4g} |")
    TRAFFIC_FILE.write_text("\n".join(lines) + "\n")
    print(f"wrote {out / 'kernel_stats_liver.md'} and {TRAFFIC_FILE}")
    if (base / "sq" / "p1" / "p_counter_collection.csv").is_file():
        summarize_sq_counters(base / "sq", out / "sq_counters_liver.md")


SQ_PASSES = (
    "SQ_WAVES SQ_BUSY_CYCLES SQ_WAVE_CYCLES SQ_INSTS_VALU SQ_INSTS_MFMA SQ_INSTS_LDS "
    "SQ_VALU_MFMA_BUSY_CYCLES SQ_ACTIVE_INST_VALU GRBM_GUI_ACTIVE",
    "SQ_WAIT_INST_LDS SQ_WAIT_INST_ANY SQ_WAIT_ANY SQ_ACTIVE_INST_LDS SQ_LDS_BANK_CONFLICT "
    "SQ_ACTIVE_INST_ANY SQ_INSTS_VMEM SQ_ACTIVE_INST_VMEM",
)


def summarize_sq_counters(base: Path, target: Path) -> None:
    """Per-dispatch averages of two rocprofv3 --pmc passes of SQ counters (p1/, p2/ under
    `base`) for the kernels with the most GRBM_GUI_ACTIVE cycles."""
    import csv
    from collections import defaultdict

    per = defaultdict(lambda: defaultdict(float))  # (kernel) -> counter -> summed value
    dispatches = defaultdict(set)
    for sub in ("p1", "p2"):
        for r in csv.DictReader(open(base / sub / "p_counter_collection.csv")):
            k = _short_kernel(r["Kernel_Name"])
            per[k][r["Counter_Name"]] += float(r["Counter_Value"])
            dispatches[(k, sub)].add(int(r["Dispatch_Id"]))
    rows = []
    for k, c in per.items():
        n1, n2 = len(dispatches[(k, "p1")]), len(dispatches[(k, "p2")])
        if not n1 or not n2 or not c.get("SQ_WAVES"):
            continue
        avg = {name: v / (n1 if name in SQ_PASSES[0].split() else n2) for name, v in c.items()}
        rows.append((k, n1, avg))
    rows.sort(key=lambda r: -r[2].get("GRBM_GUI_ACTIVE", 0.0) * r[1])
    lines = [
        "# SQ counters, liver-shape sliding window (121 tiles x 8 views, one case)",
        "",
        "Commands (repo root on the MI355X box), one pass per line, each on its own run:",
        "",
        f"    rocprofv3 --pmc {SQ_PASSES[0]} -f csv -d gpurun_out/sq/p1 -o p -- \\",
        "        python3 -u bench.py --warmup 0 --steps 1 --no-cpu-baseline --no-pcie --no-alt",
        f"    rocprofv3 --pmc {SQ_PASSES[1]} -f csv -d gpurun_out/sq/p2 -o p -- \\",
        "        python3 -u bench.py --warmup 0 --steps 1 --no-cpu-baseline --no-pcie --no-alt",
        "",
        "Per-dispatch averages over the case's launches of each kernel. Per-wave counts divide by",
        "SQ_WAVES; the wait and VALU-active shares divide by SQ_WAVE_CYCLES (both summed over",
        "waves). GRBM_GUI_ACTIVE reads 8 x the kernel's duration in cycles (summed over the 8",
        "XCDs), so per-SIMD and per-CU shares divide by GRBM_GUI_ACTIVE / 8 x 1024 SIMDs or x 256",
        "CUs.",
        "",
        f"{SOURCES_LINE}{kernel_sources_digest()}.",
        "",
        "| kernel | dispatches | waves | VALU / wave | MFMA / wave | LDS / wave | VMEM / wave | "
        "MFMA busy / SIMD cycles | LDS bank-conflict cycles / CU cycles | wait-any / wave cycles "
        "| VALU active / wave cycles |",
        "|---|---:|---:|---:|---:|---:|---:|---:|---:|---:|---:|",
    ]
    for k, n, a in rows[:8]:
        waves = a["SQ_WAVES"]
        cyc = a["GRBM_GUI_ACTIVE"] / 8.0
        lines.append(
            f"| `{k}` | {n} | {waves:.3g} | {a['SQ_INSTS_VALU'] / waves:.0f} | "
            f"{a['SQ_INSTS_MFMA'] / waves:.1f} | {a['SQ_INSTS_LDS'] / waves:.0f} | "
            f"{a['SQ_INSTS_VMEM'] / waves:.1f} | "
            f"{a['SQ_VALU_MFMA_BUSY_CYCLES'] / (cyc * 1024):.3f} | "
            f"{a['SQ_LDS_BANK_CONFLICT'] / (cyc * 256):.3f} | "
            f"{a['SQ_WAIT_ANY'] / a['SQ_WAVE_CYCLES']:.3f} | "
            f"{a['SQ_ACTIVE_INST_VALU'] / a['SQ_WAVE_CYCLES']:.3f} |")
    target.write_text("\n".join(lines) + "\n")
    print(f"wrote {target}")


CONFIG_WORKLOADS = ("brats-sw", "autopet-sw", "pancreas-sw")


def summarize_configs(directory: str) -> None:
    """Write profiles/bench_configurations.md from the bench lines cfg/<W>.json and the
    kernel traces cfg/prof_<W>/<W>_kernel_stats.csv under `directory` (W = each multi-fold or
    bf16 workload), plus a device-peak table that also takes cfg/liver-sw.json and
    cfg/liver-raw-case.json when present."""
    import csv

    base = Path(directory) / "cfg"
    lines = [
        "# Configuration benchmarks: BraTS, AutoPET and pancreas shapes (one MI355X)",
        "",
        "Commands (repo root on the MI355X box), per workload W in brats-sw, autopet-sw, pancreas-sw:",
        "",
        "    python -u bench.py --workload W --steps 1 --warmup 1 > gpurun_out/cfg/W.json",
        "    rocprofv3 --kernel-trace --stats -f csv -d gpurun_out/cfg/prof_W -o W -- \\",
        "        python3 -u bench.py --workload W --steps 1 --warmup 1 --no-cpu-baseline",
        "    python bench.py --summarize-configs gpurun_out",
        "",
        "Kernel-trace calls count the warm-up and the timed case (2 cases); average = per launch.",
        "",
        f"{SOURCES_LINE}{kernel_sources_digest()}.",
    ]
    peaks = []
    for w in CONFIG_WORKLOADS:
        rec = json.loads((base / f"{w}.json").read_text().strip().splitlines()[-1])
        roof, cpu = rec["roofline"], rec["cpu_baseline"]
        lines += [
            "", f"## {w}", "",
            f"Workload: {rec['config']['workload']}", "",
            f"* value: **{rec['value']:.4g} voxels/s** ({rec['ms_per_step'] / 1e3:.3f} s per case), "
            f"dtype {rec['dtype']}",
            f"* roofline (dominant kernel `{roof['kernel']}`): achieved {roof['achieved']} "
            f"{roof['unit']} of {roof['peak']} (frac {roof['frac']}, issued {roof.get('issued_frac')})",
        ]
        if cpu:
            lines.append(f"* cpu_baseline: {cpu['value']:.4g} {cpu['unit']} on {cpu['cores']} cores "
                         f"({cpu['kind']}): {cpu['sample']}")
        lines += [f"* label counts: {rec['config']['label_counts']}", "",
                  "| kernel | calls | total ms | average us | % |", "|---|---:|---:|---:|---:|"]
        for r in list(csv.DictReader(open(base / f"prof_{w}" / f"{w}_kernel_stats.csv")))[:10]:
            lines.append(f"| `{_short_kernel(r['Name'])}` | {r['Calls']} | "
                         f"{float(r['TotalDurationNs']) / 1e6:.1f} | {float(r['AverageNs']) / 1e3:.1f} | "
                         f"{float(r['Percentage']):.2f} |")
        peaks.append((w, rec))
    described = {
        "liver-sw": "liver-sw (1x101x768x768, 1 fold, float32 accumulation)",
        "liver-raw-case": "liver-raw-case (512x512x120 int16 CT -> 300x534x534, float16 "
                          "accumulation, restoration)",
        "brats-sw": "brats-sw (4x155x240x240, 5 folds)",
        "autopet-sw": "autopet-sw (2x284x400x400, 5 folds)",
        "pancreas-sw": "pancreas-sw (1x101x768x768, ResEnc-L bf16-mixed)",
    }
    for w in ("liver-raw-case", "liver-sw"):
        if (base / f"{w}.json").is_file():
            peaks.insert(0, (w, json.loads((base / f"{w}.json").read_text().strip().splitlines()[-1])))
    lines += [
        "", "", "## Device memory peaks", "",
        "`device_peak_gb` of each workload's bench line: the bytes in use on the GPU (hipMemGetInfo:",
        "the library's kept workspace and torch's cached blocks) above what was in use before the",
        "workload allocated anything, plus whatever part of torch's cached-allocator peak was released",
        "before the reading. Liver lines from",
        "`python -u bench.py --steps 2 --warmup 1 --no-cpu-baseline --no-pcie --no-alt > gpurun_out/cfg/liver-sw.json`",
        "and `python -u bench.py --workload liver-raw-case --steps 2 --warmup 1 > "
        "gpurun_out/cfg/liver-raw-case.json`. All at the default 32 views (4 mirrored tiles) a forward.",
        "",
        "| workload | s per case | device peak GB |",
        "|---|---:|---:|",
    ]
    for w, rec in peaks:
        lines.append(f"| {described[w]} | {rec['ms_per_step'] / 1e3:.3f} | {rec['device_peak_gb']} |")
    lines += ["", "These are the `peak_memory_gb` values of the named models (liver from the raw-case "
              "line, which runs what `named_models.liver.run` runs)."]
    target = ROOT / "profiles" / "bench_configurations.md"
    target.write_text("\n".join(lines) + "\n")
    print(f"wrote {target}")


def measured_traffic(kernel_class: str) -> float | None:
    """HBM bytes per launch of `kernel_class` from the committed counter summary, or None
    when the summary is missing or was measured on other kernel sources than these."""
    if not TRAFFIC_FILE.is_file():
        return None
    text = TRAFFIC_FILE.read_text()
    if f"{SOURCES_LINE}{kernel_sources_digest()}" not in text:
        print("[bench] the HBM traffic summary describes other kernel sources: traffic omitted",
              file=sys.stderr, flush=True)
        return None
    for line in text.splitlines():
        cells = [c.strip().strip("`") for c in line.strip("|").split("|")]
        if len(cells) == 5 and cells[0] == kernel_class:
            return float(cells[4])
    return None


def kernel_table(classes: dict, steps: int, traffic: bool = True) -> tuple[dict, dict]:
    """Per-kernel-class rates of a KernelProfile (launches and ms per step) and the roofline
    object of the dominant class (largest share of the timed region): algorithmic FLOPs or
    bytes over its launch time, against the published peak of the unit that bounds it.
    `traffic`: take the HBM bytes per launch from the liver-case counter summary (only the
    liver workload's launches are the ones it measured)."""
    kernels = {}
    for name, c in sorted(classes.items(), key=lambda kv: -kv[1]["ms"]):
        entry = {"launches": c["launches"] // steps, "ms": round(c["ms"] / steps, 3)}
        if c["flops"]:
            entry["tflops"] = round(c["flops"] / (c["ms"] * 1e-3) / 1e12, 2)
            if name.startswith("conv3d_x3") and "_bf16" in name:
                # issued bf16 MFMA work: 1 product per term, 4-tap groups (27 -> 28 taps)
                entry["frac_bf16_mfma_issued"] = round(
                    entry["tflops"] * 28 / 27 / PEAK_FP16_MFMA_TFLOPS, 4)
            elif name.startswith("conv3d_x3"):
                # issued fp16 MFMA work: 3 products per term, 4-tap groups (27 -> 28 taps)
                entry["frac_fp16_mfma_issued"] = round(
                    entry["tflops"] * SPLIT_PRODUCTS * 28 / 27 / PEAK_FP16_MFMA_TFLOPS, 4)
            elif name == "conv3d_wino":
                # issued fp16 MFMA work: 3 products per term, 64 transform positions per 8
                # outputs in place of 8 x 27 taps
                entry["frac_fp16_mfma_issued"] = round(
                    entry["tflops"] * SPLIT_PRODUCTS * 64 / 216 / PEAK_FP16_MFMA_TFLOPS, 4)
            elif name.startswith("tconv3d_x3"):
                # issued MFMA work of the pointwise GEMM: 3 fp16 products per term (1 bf16
                # product in the bf16 variant; bf16 and fp16 share the dense peak); the
                # kernel is bound by its output stream, so its HBM rate goes beside it
                if name.endswith("_bf16"):
                    entry["frac_bf16_mfma_issued"] = round(
                        entry["tflops"] / PEAK_FP16_MFMA_TFLOPS, 4)
                else:
                    entry["frac_fp16_mfma_issued"] = round(
                        entry["tflops"] * SPLIT_PRODUCTS / PEAK_FP16_MFMA_TFLOPS, 4)
                if c["bytes"]:
                    entry["gbs"] = round(c["bytes"] / (c["ms"] * 1e-3) / 1e9, 1)
                    entry["frac_hbm"] = round(entry["gbs"] / PEAK_HBM_GBS, 4)
            elif name.startswith("conv1x1_head"):
                # VALU dot products over a voxel's channels: bound by the HBM stream of the
                # input rows and outputs, so priced against HBM
                entry["gbs"] = round(c["bytes"] / (c["ms"] * 1e-3) / 1e9, 1)
                entry["frac_hbm"] = round(entry["gbs"] / PEAK_HBM_GBS, 4)
            else:
                entry["frac_fp32_mfma"] = round(entry["tflops"] / PEAK_FP32_MFMA_TFLOPS, 4)
        elif c["bytes"]:
            entry["gbs"] = round(c["bytes"] / (c["ms"] * 1e-3) / 1e9, 1)
            entry["frac_hbm"] = round(entry["gbs"] / PEAK_HBM_GBS, 4)
        kernels[name] = entry
    dominant = max(classes, key=lambda n: classes[n]["ms"])
    d = classes[dominant]
    if d["flops"]:
        achieved = d["flops"] / (d["ms"] * 1e-3) / 1e12
        # the split kernels run on fp16 MFMA: their algorithmic (float32-product) rate is
        # priced against the dense fp16 peak, the issued rate is reported beside it
        fp16 = dominant.startswith(("conv3d_x3", "conv3d_wino", "tconv3d_x3"))
        peak = PEAK_FP16_MFMA_TFLOPS if fp16 else PEAK_FP32_MFMA_TFLOPS
        roofline = {"kernel": dominant, "bound": "mfma", "achieved": round(achieved, 2),
                    "peak": peak, "unit": "TFLOP/s", "frac": round(achieved / peak, 4),
                    "traffic": measured_traffic(dominant) if traffic else None}
        if fp16:
            roofline["issued_frac"] = kernels[dominant].get(
                "frac_bf16_mfma_issued", kernels[dominant].get("frac_fp16_mfma_issued"))
    else:
        achieved = d["bytes"] / (d["ms"] * 1e-3) / 1e9
        roofline = {"kernel": dominant, "bound": "hbm", "achieved": round(achieved, 1),
                    "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBS, 4),
                    "traffic": None}
    return kernels, roofline


def cpu_baseline(spec, weights, *, patch=None, forwards=968, accumulations=121,
                 axes=(0, 1, 2), voxels=None, residual=False, case="case") -> dict:
    """The CPU oracle on a bounded sample of a case: one patch forward (median of 3 after one
    warm-up) and one tile's mirrored average + Gaussian accumulation with the oracle's own
    flips (flip, forward output, flip back, sum, divide, accumulate; median of 3),
    extrapolated to the case's forwards (tiles x folds x views) and accumulations (tiles x
    folds).  Defaults: the liver case (968 forwards, 121 tiles)."""
    import statistics

    import numpy as np
    import torch

    from oracle import sliding_window as osw
    from oracle.network import OracleNetwork

    patch = tuple(patch or PATCH)
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    net = OracleNetwork(spec, weights, residual=residual)
    x = np.random.default_rng(3).standard_normal((1, *patch, spec.input_channels)).astype(np.float32)
    pred = net(x)                                          # warm-up
    forward_times = []
    for _ in range(3):
        t0 = time.perf_counter()
        pred = net(x)
        forward_times.append(time.perf_counter() - t0)
    forward_s = statistics.median(forward_times)
    g = osw.gaussian_importance(patch)[..., None]
    acc = np.zeros((*patch, spec.num_classes), dtype=np.float32)
    norm = np.zeros((*patch, 1), dtype=np.float32)
    cached = pred  # the network's output stands in for each view's forward
    accumulate_times = []
    for _ in range(3):
        t0 = time.perf_counter()
        p = osw.mirrored_prediction(lambda tile: cached, x, tuple(axes))[0]
        acc += p * g
        norm += g
        accumulate_times.append(time.perf_counter() - t0)
    accumulate_s = statistics.median(accumulate_times)
    case_s = forwards * forward_s + accumulations * accumulate_s
    voxels = voxels or int(np.prod(VOLUME_SHAPE[1:]))
    cpu_model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu_model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {
        "value": voxels / case_s,
        "unit": "voxels/s",
        "cores": cores,
        "kind": "port",
        "sample": (f"CPU oracle (torch-CPU fp32 network, numpy sliding window) on {cores} "
                   f"threads of {cpu_model or 'the host CPU'}: one {'x'.join(map(str, patch))} "
                   f"forward {forward_s:.2f} s (median of 3 after a warm-up) and one tile's "
                   f"{2 ** len(axes)}-view mirrored average + Gaussian accumulation "
                   f"{accumulate_s:.3f} s (median of 3), extrapolated to {forwards} forwards + "
                   f"{accumulations} tile accumulations = {case_s:.0f} s per {case}"),
    }


def ensemble_volume(name: str, seed: int = 7):
    """Synthetic volumes of the multi-channel configurations: BraTS (4 x 155 x 240 x 240,
    N(0, 1) inside a random ellipsoid brain mask, 0 outside) and AutoPET (2 x 284 x 400 x 400:
    z-scored CT with ellipsoid regions; PET log-normal(0, 1) clipped to [0, 30] with 0.1 % of
    voxels at SUV 5-20)."""
    import numpy as np

    rng = np.random.default_rng(seed)
    if name == "brats-sw":
        c, shape = 4, (155, 240, 240)
        zz, yy, xx = np.ogrid[:shape[0], :shape[1], :shape[2]]
        vol = np.zeros((c, *shape), dtype=np.float32)
        for ch in range(c):
            cz, cy, cx = (s / 2 + rng.uniform(-8, 8) for s in shape)
            az, ay, ax = rng.uniform(55, 70), rng.uniform(80, 100), rng.uniform(65, 85)
            brain = ((zz - cz) / az) ** 2 + ((yy - cy) / ay) ** 2 + ((xx - cx) / ax) ** 2 <= 1
            vol[ch][brain] = rng.standard_normal(int(brain.sum()), dtype=np.float32)
        return vol
    shape = (284, 400, 400)
    ct = rng.standard_normal(shape, dtype=np.float32)
    zz, yy, xx = np.ogrid[:shape[0], :shape[1], :shape[2]]
    for _ in range(12):
        cz, cy, cx = (rng.uniform(0, s) for s in shape)
        az, ay, ax = rng.uniform(10, 60), rng.uniform(20, 100), rng.uniform(20, 100)
        inside = ((zz - cz) / az) ** 2 + ((yy - cy) / ay) ** 2 + ((xx - cx) / ax) ** 2 <= 1
        ct[inside] += np.float32(rng.uniform(-1.0, 1.5))
    pet = np.clip(rng.lognormal(0.0, 1.0, shape).astype(np.float32), 0, 30)
    hot = rng.random(shape) < 1e-3
    pet[hot] = rng.uniform(5, 20, int(hot.sum())).astype(np.float32)
    return np.stack([ct, pet])


def ensemble_workload(args) -> int:
    """The multi-fold and bf16 configurations as whole cases resident in HBM: BraTS (5 folds,
    4 -> 5 classes, 8x mirroring), AutoPET (5 folds, 2 -> 2 classes, patch 112 x 160 x 128,
    8x mirroring) and pancreas (ResEnc-L, bf16, patch 128 x 160 x 160, no mirroring); labels of
    the fold-averaged logits.  value = volume voxels per second."""
    import numpy as np
    import torch

    from nnunet_mlx import _native
    from nnunet_mlx.model.network import build_network
    from nnunet_mlx.model.topology import PlainConvUNetSpec, ResidualEncoderUNetSpec
    from nnunet_mlx.prediction import sliding_window as sw
    from nnunet_mlx.storage.synthetic import random_weights

    torch.cuda.set_device(0)
    k3 = ((3, 3, 3),)
    if args.workload == "brats-sw":
        spec = PlainConvUNetSpec(4, 5, (32, 64, 128, 256, 320, 320), k3 * 6,
                                 ((1, 1, 1),) + ((2, 2, 2),) * 5, (2,) * 6, (2,) * 5)
        patch, seeds, axes, precision = (128, 128, 128), range(5), (0, 1, 2), args.precision
        volume = ensemble_volume("brats-sw")
    elif args.workload == "autopet-sw":
        spec = PlainConvUNetSpec(2, 2, (32, 64, 128, 256, 320, 320), k3 * 6,
                                 ((1, 1, 1),) + ((2, 2, 2),) * 4 + ((1, 2, 2),), (2,) * 6, (2,) * 5)
        patch, seeds, axes, precision = (112, 160, 128), range(5), (0, 1, 2), args.precision
        volume = ensemble_volume("autopet-sw")
    else:
        spec = ResidualEncoderUNetSpec(1, 3, (32, 64, 128, 256, 320, 320, 320), k3 * 7,
                                       ((1, 1, 1),) + ((2, 2, 2),) * 5 + ((2, 1, 1),),
                                       (1, 3, 4, 6, 6, 6, 6), (1,) * 6)
        patch, seeds, axes, precision = (128, 160, 160), (4,), (), "bf16-mixed"
        volume = synthetic_ct()
    peak = DevicePeak()
    nets = []
    for seed in seeds:
        net = build_network(spec, precision=precision)
        net.load_weights(random_weights(spec, seed=seed))
        if nets:
            net.share_workspace(nets[0])
        nets.append(net)
    d_volume = torch.from_numpy(volume).cuda()
    kwargs = dict(patch_size=patch, num_outputs=spec.num_classes, mirroring_axes=axes,
                  step_fraction=0.5, accumulation="float32", tiles_per_batch=args.tiles_per_batch)
    for i in range(max(args.warmup, 1)):
        print(f"[bench] {args.workload} warmup {i + 1}", file=sys.stderr, flush=True)
        sw.average_fold_labels(nets, d_volume, return_device=True, **kwargs)
    torch.cuda.synchronize()
    with _native.KernelProfile() as prof:
        t0 = time.perf_counter()
        for i in range(args.steps):
            print(f"[bench] {args.workload} step {i + 1}/{args.steps}", file=sys.stderr, flush=True)
            labels = sw.average_fold_labels(nets, d_volume, return_device=True, **kwargs)
        torch.cuda.synchronize()
        step_s = (time.perf_counter() - t0) / args.steps
    device_peak_gb = peak.gb()
    kernels, roofline = kernel_table(prof.classes, steps=args.steps, traffic=False)
    steps = [len(s) for s in sw.compute_steps([max(a, b) for a, b in zip(volume.shape[1:], patch)],
                                              patch, step_fraction=0.5)]
    tiles = int(np.prod(steps))
    voxels = int(np.prod(volume.shape[1:]))
    baseline = None
    if not args.no_cpu_baseline:
        print(f"[bench] {args.workload} CPU baseline sample", file=sys.stderr, flush=True)
        baseline = cpu_baseline(spec, random_weights(spec, seed=seeds[0]), patch=patch,
                                forwards=tiles * len(nets) * 2 ** len(axes),
                                accumulations=tiles * len(nets), axes=axes, voxels=voxels,
                                residual=isinstance(spec, ResidualEncoderUNetSpec),
                                case=f"{args.workload} case")
    line = {
        "metric": f"sliding-window voxels/s, {args.workload} configuration",
        "value": round(voxels / step_s, 1), "unit": "voxels/s", "n_gpus": 1, "steps": args.steps,
        "warmup": max(args.warmup, 1), "ms_per_step": round(step_s * 1e3, 1),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": DTYPES[precision],
        "data": "synthetic",
        "config": {"workload": f"{args.workload}: volume {list(volume.shape)} fp32 resident in HBM, "
                               f"{len(nets)} fold(s), patch {list(patch)}, step 0.5, "
                               f"mirror axes {list(axes)}, {tiles} tiles, "
                               f"{tiles * len(nets) * 2 ** len(axes)} forwards",
                   "label_counts": torch.bincount(labels.reshape(-1).to(torch.int64),
                                                  minlength=spec.num_classes).tolist()},
        "conv3d_mfma_frac": conv_mfma_frac(prof.classes, precision),
        "device_peak_gb": device_peak_gb,
        "kernels": kernels, "roofline": roofline, "cpu_baseline": baseline,
    }
    for net in nets:
        net.close()
    print(json.dumps(line), flush=True)
    return 0


def raw_case_workload(args) -> int:
    """Raw liver CT resident in HBM -> uint16 labels on the raw grid on the host: GPU
    preprocessing, the 8x-mirrored sliding window with float16 accumulation (what the
    runners compute), separate-axis logit restoration and argmax on the device, uncrop on
    the host.  value = raw-case voxels per second."""
    import tempfile

    import numpy as np
    import torch

    from nnunet_mlx.model.folder import load_model_bundle
    from nnunet_mlx.prediction.pipeline import ModelFolderPredictor
    from nnunet_mlx.storage.synthetic import write_random_model_folder

    torch.cuda.set_device(0)
    raw = synthetic_raw_ct()
    peak = DevicePeak()
    with tempfile.TemporaryDirectory(prefix="nnx-bench-") as tmp:
        folder = write_random_model_folder(Path(tmp) / "liver", liver_spec(), patch_size=PATCH,
                                           seeds=(1,), labels=("liver", "tumor"))
        plans = json.loads((folder / "plans.json").read_text())
        cfg = plans["configurations"]["3d_fullres"]
        prep = prep_plans(args.resampler)
        cfg.update(prep["configurations"]["3d_fullres"])
        if args.resampler == "torch":
            cfg["resampling_fn_probabilities"] = "resample_torch_fornnunet"
            cfg["resampling_fn_probabilities_kwargs"] = dict(
                TORCH_RESAMPLING["resampling_fn_data_kwargs"])
        plans["foreground_intensity_properties_per_channel"] = \
            prep["foreground_intensity_properties_per_channel"]
        (folder / "plans.json").write_text(json.dumps(plans))
        bundle = load_model_bundle(folder, configuration="3d_fullres")
    predictor = ModelFolderPredictor(bundle, accumulation="nnunet-fp16", step_fraction=0.5,
                                     tiles_per_batch=args.tiles_per_batch)
    props = {"spacing": list(PREP_SPACING)}
    d_raw = torch.from_numpy(raw).cuda()
    for i in range(max(args.warmup, 1)):
        print(f"[bench] raw-case warmup {i + 1}", file=sys.stderr, flush=True)
        labels, details = predictor.predict_raw(d_raw, props)
    torch.cuda.synchronize()
    stages: dict[str, float] = {}
    t0 = time.perf_counter()
    for i in range(args.steps):
        print(f"[bench] raw-case step {i + 1}/{args.steps}", file=sys.stderr, flush=True)
        labels, details = predictor.predict_raw(d_raw, props)
        for k, v in details["metrics"].items():
            stages[k] = stages.get(k, 0.0) + v / args.steps
    torch.cuda.synchronize()
    step_s = (time.perf_counter() - t0) / args.steps
    device_peak_gb = peak.gb()
    voxels = int(np.prod(raw.shape[1:]))
    line = {
        "metric": "raw-case voxels/s, liver CT 512x512x120 int16 -> labels on the raw grid "
                  "(GPU preprocessing, 8x TTA sliding window, fp16 accumulation, "
                  "separate-axis restoration"
                  + (", Torch-grid resampler)" if args.resampler == "torch" else ")"),
        "value": round(voxels / step_s, 1), "unit": "voxels/s", "n_gpus": 1,
        "steps": args.steps, "warmup": max(args.warmup, 1), "ms_per_step": round(step_s * 1e3, 1),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32 (fp16-split products), fp16 accumulation", "data": "synthetic",
        "config": {"workload": "raw CT (1, 120, 512, 512) int16 resident in HBM at spacing "
                               "(2.5, 0.8, 0.8) mm, liver 3d_fullres network (random weights), "
                               "patch 128^3, step 0.5, mirror axes (0, 1, 2)",
                   "resampler": args.resampler,
                   "preprocessed_shape": list(details["preprocessed_shape"]),
                   "label_counts": np.bincount(labels.ravel(), minlength=3).tolist()},
        "stages_s": {k: round(v, 4) for k, v in stages.items()},
        "device_peak_gb": device_peak_gb,
        "roofline": None, "cpu_baseline": None,
    }
    for model in bundle.models:
        model.close()
    print(json.dumps(line), flush=True)
    return 0


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__)
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=1)
    parser.add_argument("--warmup", type=int, default=1)
    parser.add_argument("--tiles-per-batch", type=int, default=None,
                        help="tiles per forward batch (default: the library's, 4 tiles = 32 views)")
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--no-pcie", action="store_true")
    parser.add_argument("--copy-calibration", action="store_true",
                        help="first run a plain 1 GiB read + 1 GiB write elementwise kernel "
                             "(torch.neg) whose HBM counters calibrate FETCH_SIZE/WRITE_SIZE")
    parser.add_argument("--summarize-profiles", metavar="DIR",
                        help="write the profiles/ summaries from rocprofv3 CSV output in DIR and exit")
    parser.add_argument("--summarize-configs", metavar="DIR",
                        help="write profiles/bench_configurations.md from the configuration bench "
                             "lines and kernel traces under DIR/cfg and exit")
    parser.add_argument("--precision", choices=tuple(DTYPES), default="fp32-split",
                        help="convolution arithmetic: fp16-split products (3 per term) on fp16 "
                             "MFMA (default), or float32 products on fp32 MFMA; both float32 I/O "
                             "and accumulation, both within the float32 logits tolerance")
    parser.add_argument("--no-alt", action="store_true",
                        help="skip the one-step measurement of the other precision")
    parser.add_argument("--shape", type=int, nargs=3, default=VOLUME_SHAPE[1:],
                        help="volume size (Z Y X); the default is the liver case")
    parser.add_argument("--resampler", choices=("spline", "torch"), default="spline",
                        help="preprocess-ct / restore-ct / liver-raw-case: the plans' resampler "
                             "(order-3 / order-1 spline, or upstream's Torch-grid resampler)")
    parser.add_argument("--workload", choices=("liver-sw", "preprocess-ct", "liver-raw-case",
                                               "restore-ct", "brats-sw", "autopet-sw",
                                               "pancreas-sw"),
                        default="liver-sw",
                        help="liver-sw: the sliding-window case (default); preprocess-ct: raw "
                             "CT preprocessing on the GPU; liver-raw-case: raw CT to labels on "
                             "the raw grid (preprocessing, sliding window, restoration); "
                             "restore-ct: class-logit restoration of the liver case; "
                             "brats-sw / autopet-sw / pancreas-sw: the multi-fold and bf16 "
                             "configurations")
    args = parser.parse_args()
    if args.summarize_profiles:
        summarize_profiles(args.summarize_profiles)
        return 0
    if args.summarize_configs:
        summarize_configs(args.summarize_configs)
        return 0
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(tiles would shard across GPUs with one halo exchange; see the design notes). "
              "Run with --gpus 1.", file=sys.stderr)
        return 2
    if args.workload == "preprocess-ct":
        return preprocess_workload(args)
    if args.workload == "liver-raw-case":
        return raw_case_workload(args)
    if args.workload == "restore-ct":
        return restore_workload(args)
    if args.workload in ("brats-sw", "autopet-sw", "pancreas-sw"):
        return ensemble_workload(args)

    import numpy as np
    import torch

    from nnunet_mlx import _native
    from nnunet_mlx.model.network import build_network
    from nnunet_mlx.prediction import sliding_window as sw
    from nnunet_mlx.storage.synthetic import random_weights

    torch.cuda.set_device(0)
    device = torch.device("cuda", 0)
    if args.copy_calibration:
        src = torch.ones(1 << 28, dtype=torch.float32, device=device)
        dst = torch.empty_like(src)
        torch.neg(src, out=dst)
        torch.cuda.synchronize()
        del src, dst
    shape = (1, *args.shape)
    spec = liver_spec()
    weights = random_weights(spec, seed=1)
    peak = DevicePeak()
    net = build_network(spec, precision=args.precision)
    net.load_weights(weights)
    print(f"[bench] synthesising volume {shape}", file=sys.stderr, flush=True)
    host_volume = synthetic_ct(shape)
    volume = torch.from_numpy(host_volume).to(device)
    kwargs = dict(patch_size=PATCH, num_outputs=3, mirroring_axes=(0, 1, 2), step_fraction=0.5,
                  accumulation="float32", tiles_per_batch=args.tiles_per_batch)
    ntiles = int(np.prod([len(s) for s in sw.compute_steps(
        [max(a, b) for a, b in zip(shape[1:], PATCH)], PATCH, step_fraction=0.5)]))
    for i in range(args.warmup):
        print(f"[bench] warmup step {i + 1}/{args.warmup}", file=sys.stderr, flush=True)
        sw.average_fold_labels((net,), volume, return_device=True, **kwargs)
    torch.cuda.synchronize()
    with _native.KernelProfile() as prof:
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(args.steps):
            labels = sw.average_fold_labels((net,), volume, return_device=True, **kwargs)
            print(f"[bench] timed step {i + 1}/{args.steps} queued", file=sys.stderr, flush=True)
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - t0
    step_s = elapsed / args.steps
    voxels = int(np.prod(shape[1:]))
    counts = np.bincount(labels.cpu().numpy().view(np.uint16).ravel(), minlength=3)
    print(f"[bench] {step_s:.3f} s per case; label counts {counts.tolist()}", file=sys.stderr, flush=True)

    device_peak_gb = peak.gb()
    classes = prof.classes
    kernels, roofline = kernel_table(classes, steps=args.steps)
    # 3x3x3 convolution rate against the float32-class MFMA peak of the arithmetic used
    conv_frac = conv_mfma_frac(classes, args.precision)

    alt = None
    if not args.no_alt:
        other = "fp32" if args.precision != "fp32" else "fp32-split"
        print(f"[bench] one step with precision {other}", file=sys.stderr, flush=True)
        alt_net = build_network(spec, precision=other)
        alt_net.load_weights(weights)
        alt_net.share_workspace(net)
        sw.average_fold_labels((alt_net,), volume, return_device=True, **kwargs)
        torch.cuda.synchronize()
        with _native.KernelProfile() as alt_prof:
            t0 = time.perf_counter()
            alt_labels = sw.average_fold_labels((alt_net,), volume, return_device=True, **kwargs)
            torch.cuda.synchronize()
            alt_s = time.perf_counter() - t0
        agree = float((alt_labels == labels).float().mean())
        alt_conv = conv_mfma_frac(alt_prof.classes, other)
        alt = {"precision": other, "value": round(voxels / alt_s, 1),
               "ms_per_step": round(alt_s * 1e3, 2), "label_agreement": round(agree, 7),
               "conv3d_mfma_frac": alt_conv,
               "conv3d_mfma_peak_tflops": PEAK_FP32_MFMA_TFLOPS if other == "fp32"
               else round(PEAK_FP16_MFMA_TFLOPS / SPLIT_PRODUCTS, 1)}
        alt_net.close()
        del alt_labels

    pcie = None
    if not args.no_pcie:
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        host_labels = sw.average_fold_labels((net,), host_volume, **kwargs)
        pcie_s = time.perf_counter() - t0
        pcie = voxels / pcie_s
        del host_labels

    baseline = None
    if not args.no_cpu_baseline:
        print("[bench] timing the CPU baseline", file=sys.stderr, flush=True)
        baseline = cpu_baseline(spec, weights)

    nforwards = ntiles * 8
    result = {
        "metric": METRIC,
        "value": round(voxels / step_s, 1),
        "unit": "voxels/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_s * 1e3, 2),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": DTYPES[args.precision],
        "precision": args.precision,
        "data": "synthetic",
        "config": {
            "workload": (f"liver-shape sliding window: CT volume 1x{shape[1]}x{shape[2]}x{shape[3]} "
                         f"fp32 resident in HBM, random-init 6-stage PlainConvUNet [32..320] 1->3 "
                         f"classes, patch 128^3, step 0.5 ({ntiles} tiles), 8x mirror TTA "
                         f"({nforwards} forwards), 1 fold, fp32 Gaussian accumulation, argmax labels"),
            "tiles": ntiles,
            "forwards": nforwards,
            "views_per_forward_batch": 8 * min(args.tiles_per_batch or 4, ntiles),
        },
        "ms_per_forward": round(step_s * 1e3 / nforwards, 3),
        "ms_per_tile": round(step_s * 1e3 / ntiles, 2),
        "conv3d_mfma_frac": conv_frac,
        "pcie_inclusive_voxels_per_s": round(pcie, 1) if pcie else None,
        "device_peak_gb": device_peak_gb,
        "other_precision": alt,
        "roofline": roofline,
        "cpu_baseline": baseline,
        "kernels": kernels,
    }
    print(json.dumps(result))
    return 0


if __name__ == "__main__":
    sys.exit(main())
