"""Network workloads at their real shapes: specs, seeded inputs and output probes.

Shared by ``make_config_fixtures.py`` (which runs the CPU oracle on two batch items per
workload and stores probes of its logits in ``config_forwards.npz``) and by the GPU test
``tests/test_gpu_configs.py`` (which forwards a batch of 32 items on the device, items 0
and 31 being the two stored ones, and compares the same probes).

Workloads (patch, channels, classes, network, seed):
  liver     128x128x128, 1 -> 3, 6-stage PlainConvUNet [32..320], seed 1, CT-like input
  brats     128x128x128, 4 -> 5, same network, seed 0, MRI-like input (noise in an ellipsoid)
  autopet   112x160x128, 2 -> 2, strides [1,2,2,2,2,(1,2,2)], seed 0, CT + PET-like input
  pancreas  128x160x160, 1 -> 3, 7-stage ResEnc-L (blocks 1,3,4,6,6,6,6), seed 4, CT-like
"""

from __future__ import annotations

import numpy as np

from nnunet_mlx.model.topology import PlainConvUNetSpec, ResidualEncoderUNetSpec

K3 = ((3, 3, 3),)
BATCH = 32
ITEMS = (0, BATCH - 1)  # batch positions with stored oracle probes


def liver_spec(cin: int = 1, classes: int = 3, strides=None) -> PlainConvUNetSpec:
    return PlainConvUNetSpec(
        input_channels=cin, num_classes=classes, features=(32, 64, 128, 256, 320, 320),
        kernel_sizes=K3 * 6, strides=strides or ((1, 1, 1),) + ((2, 2, 2),) * 5,
        encoder_convs=(2,) * 6, decoder_convs=(2,) * 5)


def pancreas_spec() -> ResidualEncoderUNetSpec:
    return ResidualEncoderUNetSpec(
        input_channels=1, num_classes=3, features=(32, 64, 128, 256, 320, 320, 320),
        kernel_sizes=K3 * 7, strides=((1, 1, 1),) + ((2, 2, 2),) * 5 + ((2, 1, 1),),
        encoder_blocks=(1, 3, 4, 6, 6, 6, 6), decoder_convs=(1,) * 6)


WORKLOADS = {
    "liver": dict(spec=liver_spec(), patch=(128, 128, 128), seed=1, kind="ct"),
    "brats": dict(spec=liver_spec(cin=4, classes=5), patch=(128, 128, 128), seed=0, kind="mri"),
    "autopet": dict(spec=liver_spec(cin=2, classes=2,
                                    strides=((1, 1, 1),) + ((2, 2, 2),) * 4 + ((1, 2, 2),)),
                    patch=(112, 160, 128), seed=0, kind="petct"),
    "pancreas": dict(spec=pancreas_spec(), patch=(128, 160, 160), seed=4, kind="ct"),
}


def item_input(name: str, item: int) -> np.ndarray:
    """Channels-last (Z, Y, X, C) float32 input of batch position ``item`` (seeded)."""
    w = WORKLOADS[name]
    z, y, x = w["patch"]
    rng = np.random.default_rng([1000 + item, len(name)])
    if w["kind"] == "ct":
        # z-scored CT: 70 % soft tissue N(0, 0.3), 30 % air N(-2.5, 0.2)
        air = rng.random((z, y, x), dtype=np.float32) < 0.3
        v = rng.standard_normal((z, y, x), dtype=np.float32)
        v *= np.where(air, np.float32(0.2), np.float32(0.3))
        v += np.where(air, np.float32(-2.5), np.float32(0.0))
        return v[..., None]
    if w["kind"] == "mri":
        # four z-scored channels inside an ellipsoid brain mask, 0 outside
        zz, yy, xx = np.ogrid[:z, :y, :x]
        mask = (((zz - z / 2) / (0.45 * z)) ** 2 + ((yy - y / 2) / (0.4 * y)) ** 2
                + ((xx - x / 2) / (0.35 * x)) ** 2) <= 1.0
        v = rng.standard_normal((z, y, x, 4), dtype=np.float32)
        return (v * mask[..., None]).astype(np.float32)
    # CT N(0, 1) beside PET: log-normal(0, 1) clipped to [0, 30], 0.1 % of voxels SUV 5..20
    ct = rng.standard_normal((z, y, x), dtype=np.float32)
    pet = np.clip(rng.lognormal(0.0, 1.0, (z, y, x)), 0.0, 30.0).astype(np.float32)
    hot = rng.random((z, y, x)) < 1e-3
    pet[hot] = rng.uniform(5.0, 20.0, int(hot.sum())).astype(np.float32)
    return np.stack([ct, pet], axis=-1)


def probe(logits: np.ndarray) -> dict[str, np.ndarray]:
    """Probes of one item's channels-last logits (Z, Y, X, K): every 8th voxel per axis from
    offset 3; every 7th voxel per axis from offsets (1, 2, 5) ("residues": 7 is prime to
    every power of two, so the sample holds each (z mod 2^a, y mod 2^b, x mod 2^c) position
    of the convolution kernels' output boxes and tiles, which the 8-stride sample, always at
    box position (3, 3, 3) of a 4x8x8 box, does not); the 16^3 corner block (zero-padding
    region of every convolution); and the float64 per-class sums and sums of squares over
    the whole output."""
    v = np.asarray(logits, dtype=np.float32)
    return {
        "strided": np.ascontiguousarray(v[3::8, 3::8, 3::8]),
        "residues": np.ascontiguousarray(v[1::7, 2::7, 5::7]),
        "corner": np.ascontiguousarray(v[:16, :16, :16]),
        "sums": v.astype(np.float64).sum(axis=(0, 1, 2)),
        "squares": (v.astype(np.float64) ** 2).sum(axis=(0, 1, 2)),
    }
