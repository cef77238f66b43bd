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
PEAK_HBM_GBS = 8000.0
VOLUME_SHAPE = (1, 101, 768, 768)
PATCH = (128, 128, 128)


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


def cpu_baseline(spec, weights) -> dict:
    """Oracle forward of one 128^3 view on the host cores + one tile's accumulation,
    extrapolated to the case (968 forwards, 121 accumulations)."""
    import numpy as np
    import torch

    from oracle import sliding_window as osw
    from oracle.network import OracleNetwork

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    net = OracleNetwork(spec, weights)
    x = np.random.default_rng(0).standard_normal((1, *PATCH, 1)).astype(np.float32)
    t0 = time.perf_counter()
    pred = net(x)
    forward_s = time.perf_counter() - t0
    g = osw.gaussian_importance(PATCH)[..., None]
    acc = np.zeros((*PATCH, 3), dtype=np.float32)
    norm = np.zeros((*PATCH, 1), dtype=np.float32)
    views = [pred[0]] * 8
    t0 = time.perf_counter()
    s = views[0].copy()
    for v in views[1:]:
        s = s + v
    s = s / np.float32(8)
    acc += s * g
    norm += g
    accumulate_s = time.perf_counter() - t0
    case_s = 968 * forward_s + 121 * accumulate_s
    voxels = int(np.prod(VOLUME_SHAPE[1:]))
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
        "sample": (f"one 128^3 forward ({forward_s:.2f} s) + one tile accumulation "
                   f"({accumulate_s:.3f} s) of the CPU oracle (torch-CPU fp32 network, numpy "
                   f"accumulation), extrapolated to 968 forwards + 121 accumulations "
                   f"= {case_s:.0f} s per case; {cores} threads on {cpu_model or 'host CPU'}"),
    }


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__)
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=1)
    parser.add_argument("--warmup", type=int, default=1)
    parser.add_argument("--tiles-per-batch", type=int, default=1)
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--no-pcie", action="store_true")
    parser.add_argument("--shape", type=int, nargs=3, default=VOLUME_SHAPE[1:],
                        help="volume size (Z Y X); the default is the liver case")
    args = parser.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(tiles would shard across GPUs with one halo exchange; see the design notes). "
              "Run with --gpus 1.", file=sys.stderr)
        return 2

    import numpy as np
    import torch

    from nnunet_mlx import _native
    from nnunet_mlx.model.network import build_network
    from nnunet_mlx.prediction import sliding_window as sw
    from nnunet_mlx.storage.synthetic import random_weights

    torch.cuda.set_device(0)
    device = torch.device("cuda", 0)
    shape = (1, *args.shape)
    spec = liver_spec()
    weights = random_weights(spec, seed=1)
    net = build_network(spec)
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

    classes = prof.classes
    kernels = {}
    for name, c in sorted(classes.items(), key=lambda kv: -kv[1]["ms"]):
        entry = {"launches": c["launches"], "ms": round(c["ms"], 3)}
        if c["flops"]:
            entry["tflops"] = round(c["flops"] / (c["ms"] * 1e-3) / 1e12, 2)
            entry["frac_fp32_mfma"] = round(entry["tflops"] / PEAK_FP32_MFMA_TFLOPS, 4)
        elif c["bytes"]:
            entry["gbs"] = round(c["bytes"] / (c["ms"] * 1e-3) / 1e9, 1)
            entry["frac_hbm"] = round(entry["gbs"] / PEAK_HBM_GBS, 4)
        kernels[name] = entry
    dominant = max(classes, key=lambda n: classes[n]["ms"])
    d = classes[dominant]
    if d["flops"]:
        achieved = d["flops"] / (d["ms"] * 1e-3) / 1e12
        roofline = {"kernel": dominant, "bound": "mfma", "achieved": round(achieved, 2),
                    "peak": PEAK_FP32_MFMA_TFLOPS, "unit": "TFLOP/s",
                    "frac": round(achieved / PEAK_FP32_MFMA_TFLOPS, 4), "traffic": None}
    else:
        achieved = d["bytes"] / (d["ms"] * 1e-3) / 1e9
        roofline = {"kernel": dominant, "bound": "hbm", "achieved": round(achieved, 1),
                    "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBS, 4),
                    "traffic": None}
    conv = [c for n, c in classes.items() if n.startswith("conv3d_igemm")]
    conv_flops = sum(c["flops"] for c in conv)
    conv_ms = sum(c["ms"] for c in conv)
    conv_frac = conv_flops / (conv_ms * 1e-3) / 1e12 / PEAK_FP32_MFMA_TFLOPS if conv_ms else None

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
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": (f"liver-shape sliding window: CT volume 1x{shape[1]}x{shape[2]}x{shape[3]} "
                         f"fp32 resident in HBM, random-init 6-stage PlainConvUNet [32..320] 1->3 "
                         f"classes, patch 128^3, step 0.5 ({ntiles} tiles), 8x mirror TTA "
                         f"({nforwards} forwards), 1 fold, fp32 Gaussian accumulation, argmax labels"),
            "tiles": ntiles,
            "forwards": nforwards,
            "views_per_forward_batch": 8 * args.tiles_per_batch,
        },
        "ms_per_forward": round(step_s * 1e3 / nforwards, 3),
        "ms_per_tile": round(step_s * 1e3 / ntiles, 2),
        "conv3d_mfma_frac": round(conv_frac, 4) if conv_frac else None,
        "pcie_inclusive_voxels_per_s": round(pcie, 1) if pcie else None,
        "roofline": roofline,
        "cpu_baseline": baseline,
        "kernels": kernels,
    }
    print(json.dumps(result))
    return 0


if __name__ == "__main__":
    sys.exit(main())
