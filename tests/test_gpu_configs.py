"""The benchmark workloads at their real shapes on the GPU.

* Network forwards at the production batch of 32 views per launch: the liver, BraTS and
  AutoPET PlainConvUNets and the pancreas ResEnc-L (whose 32-item batch holds 3.4e9
  elements in each full-resolution activation).  Items 0 and 31 are seeded inputs whose
  CPU-oracle logits were probed once (tests/golden/make_config_fixtures.py); the other
  items are device noise.  Bar: the float32 one (max-abs <= 1e-3, relative L2 <= 1e-5,
  argmax agreement >= 99.99 %) on every probed voxel for fp32-split (and fp32 products for
  the liver); for bf16 the distance to float32 recorded below.  One liver item is also
  compared with the oracle run live.
* The liver-shape sliding window over the whole 1x101x768x768 volume (121 tiles, 8 views,
  batches of 32 views, a 128x768x768x3 accumulator) with a pointwise model: logits and
  labels bit-identical to the oracle's (SHA-256 of the oracle's arrays, committed), in
  float32 and nnunet-fp16 accumulation, and equal to the pointwise model itself up to the
  float32 rounding of the weighted mean (a known answer that needs no oracle).
"""

from __future__ import annotations

import hashlib
import json
from pathlib import Path

import numpy as np
import pytest
import torch

from nnunet_mlx.model.network import build_network
from nnunet_mlx.prediction import sliding_window as sw
from nnunet_mlx.storage.synthetic import random_weights
from tests.golden import config_cases as cc
from tests.helpers import rel_l2, report

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"


@pytest.fixture(scope="module")
def fixtures():
    return np.load(GOLDEN / "config_forwards.npz", allow_pickle=False)


def _batch(name: str, device) -> torch.Tensor:
    """32-item channels-last batch: the two seeded items at positions 0 and 31, N(0, 1)
    device noise elsewhere."""
    w = cc.WORKLOADS[name]
    cin = w["spec"].input_channels
    gen = torch.Generator(device=device).manual_seed(7)
    x = torch.randn((cc.BATCH, *w["patch"], cin), generator=gen, device=device)
    for item in cc.ITEMS:
        x[item] = torch.from_numpy(cc.item_input(name, item)).to(device)
    return x


def _label_flips(mine: np.ndarray, ref: np.ndarray) -> tuple[int, int, int]:
    """(voxels, argmax disagreements, disagreements where the oracle's two best classes are
    more than 2e-3 apart, i.e. beyond what two logits within the 1e-3 bar can swap)."""
    a, b = mine.reshape(-1, mine.shape[-1]), ref.reshape(-1, ref.shape[-1])
    flips = a.argmax(-1) != b.argmax(-1)
    top2 = np.sort(b, axis=-1)[:, -2:]
    margin = top2[:, 1] - top2[:, 0]
    return len(a), int(flips.sum()), int((flips & (margin > 2e-3)).sum())


def _check_probes(name, precision, got, fixtures, label="fp32", bar="fp32"):
    """Compare the probes of the device logits of items 0 and 31 with the oracle's.  The
    argmax agreement bar (>= 99.99 % of a volume's voxels) is read on the probed sample as:
    no disagreement beyond a near-tie, and at most one in 10^4 voxels (or one voxel)."""
    lines = []
    voxels = flips = hard = 0
    for item, logits in zip(cc.ITEMS, got):
        mine = cc.probe(logits)
        for key in ("strided", "residues", "corner"):
            ref = fixtures[f"{name}__{item}__{label}__{key}"]
            msg = report(f"{name} item {item} {precision} {key} vs {label}", mine[key], ref)
            lines.append(msg)
            print(msg, flush=True)
            assert mine[key].shape == ref.shape and np.isfinite(mine[key]).all(), msg
            if bar == "fp32":
                assert np.abs(mine[key] - ref).max() <= 1e-3, msg
                assert rel_l2(mine[key], ref) <= 1e-5, msg
                n, f, h = _label_flips(mine[key], ref)
                voxels, flips, hard = voxels + n, flips + f, hard + h
        sums = fixtures[f"{name}__{item}__{label}__sums"]
        squares = fixtures[f"{name}__{item}__{label}__squares"]
        if bar == "fp32":
            # whole-output moments, every voxel: relative L2 <= 1e-5 over the N voxels of a
            # class bounds its sum by Cauchy-Schwarz, |sum(d)| <= sqrt(N) |d| <= 1e-5
            # sqrt(N * sum(v^2)), and its sum of squares to about 2e-5 relative
            voxels_per_class = logits.size // logits.shape[-1]
            np.testing.assert_allclose(mine["squares"], squares, rtol=4e-5)
            bound = 1e-5 * np.sqrt(voxels_per_class * squares)
            assert (np.abs(mine["sums"] - sums) <= bound).all(), (mine["sums"], sums, bound)
    if bar == "fp32":
        print(f"{name} {precision}: {flips} argmax disagreements in {voxels} probed voxels "
              f"({hard} beyond a near-tie)", flush=True)
        assert hard == 0 and flips <= max(1, voxels // 10000), (flips, hard, voxels)
    return lines


def _sampled(probes, prefix: str = "") -> np.ndarray:
    """The two voxel samples of one item ("strided" and "residues") as one (N, K) array."""
    return np.concatenate([np.asarray(probes[prefix + key]).reshape(-1, probes[prefix + key].shape[-1])
                           for key in ("strided", "residues")])


def _forward(name, precision, device):
    w = cc.WORKLOADS[name]
    spec = w["spec"]
    net = build_network(spec, precision=precision)
    net.load_weights(random_weights(spec, seed=w["seed"]))
    x = _batch(name, device)
    print(f"config {name} {precision}: forward of batch {tuple(x.shape)}", flush=True)
    out = net(x)
    torch.cuda.synchronize()
    assert tuple(out.shape) == (cc.BATCH, *w["patch"], spec.num_classes)
    got = out[list(cc.ITEMS)].cpu().numpy()
    finite = bool(torch.isfinite(out).all())
    net.close()
    del x, out
    torch.cuda.empty_cache()
    assert finite, f"{name} {precision}: non-finite logits in the batch"
    return got


@pytest.mark.parametrize("name,precision", [
    ("liver", "fp32-split"), ("liver", "fp32"), ("brats", "fp32-split"),
    ("autopet", "fp32-split"), ("pancreas", "fp32-split")])
def test_workload_forward_matches_oracle_fixtures(device, fixtures, name, precision):
    got = _forward(name, precision, device)
    _check_probes(name, precision, got, fixtures)


def test_pancreas_bf16_forward(device, fixtures):
    """bf16 ResEnc-L at the pancreas shape, batch 32.  The bf16 rounding itself, emulated
    on the CPU, puts the logits at relative L2 ~1.1e-2 of the float32 ones on this network;
    the device result must stay within 1.25x of that distance on both items (the north
    star's 1e-2 is not met by this arithmetic on random-init networks)."""
    got = _forward("pancreas", "bf16", device)
    for item, logits in zip(cc.ITEMS, got):
        mine = _sampled(cc.probe(logits))
        ref = _sampled(fixtures, f"pancreas__{item}__fp32__")
        emu = _sampled(fixtures, f"pancreas__{item}__bf16emu__")
        inherent = rel_l2(emu, ref)
        dist = rel_l2(mine, ref)
        agree = (mine.argmax(-1) == ref.argmax(-1)).mean()
        print(f"pancreas bf16 item {item}: vs float32 {dist:.3e} (emulation {inherent:.3e}), "
              f"vs emulation {rel_l2(mine, emu):.3e}, argmax agreement {agree:.5f}", flush=True)
        assert np.isfinite(mine).all()
        assert dist <= 1.25 * inherent
        assert agree >= 0.98


def test_pancreas_bf16_mixed_forward(device, fixtures):
    """The pancreas ResEnc-L in "bf16-mixed" (bf16 below full resolution, fp16-split at full
    resolution: two thirds of the convolution FLOPs in bf16) meets the north star's bf16 bar,
    relative L2 <= 1e-2 of the float32 logits, on both probed items."""
    got = _forward("pancreas", "bf16-mixed", device)
    for item, logits in zip(cc.ITEMS, got):
        mine = _sampled(cc.probe(logits))
        ref = _sampled(fixtures, f"pancreas__{item}__fp32__")
        dist = rel_l2(mine, ref)
        agree = (mine.argmax(-1) == ref.argmax(-1)).mean()
        print(f"pancreas bf16-mixed item {item}: vs float32 {dist:.3e}, argmax agreement "
              f"{agree:.5f}", flush=True)
        assert np.isfinite(mine).all()
        assert dist <= 1e-2
        assert agree >= 0.99


def test_liver_item_matches_live_oracle(device):
    """One 128^3 liver item against the oracle run here (no fixture in between)."""
    from oracle.network import OracleNetwork

    w = cc.WORKLOADS["liver"]
    spec = w["spec"]
    weights = random_weights(spec, seed=w["seed"])
    x = cc.item_input("liver", 5)[None]
    print("config liver live oracle: one 128^3 item", flush=True)
    ref = OracleNetwork(spec, weights)(x)
    net = build_network(spec)
    net.load_weights(weights)
    got = net(torch.from_numpy(x).to(device)).cpu().numpy()
    net.close()
    msg = report("liver live", got, ref)
    print(msg, flush=True)
    assert np.abs(got - ref).max() <= 1e-3 and rel_l2(got, ref) <= 1e-5, msg


class TorchPointwise:
    """The oracle fixture's pointwise model, (1.5 v, -1.5 v, v * v), on the device."""

    def __call__(self, values: torch.Tensor) -> torch.Tensor:
        s = 1.5
        return torch.cat((values * s, -values * s, values * values), dim=-1)


def _sha(tensor: torch.Tensor) -> str:
    return hashlib.sha256(np.ascontiguousarray(tensor.cpu().numpy()).tobytes()).hexdigest()


@pytest.mark.parametrize("accumulation", ["float32", "nnunet-fp16"])
def test_liver_volume_sliding_window_bitwise(device, accumulation):
    meta = json.loads((GOLDEN / "liver_volume_digest.json").read_text())
    data = np.random.default_rng(meta["seed"]).standard_normal(tuple(meta["shape"]),
                                                              dtype=np.float32)
    volume = torch.from_numpy(data).to(device)
    patch = tuple(meta["patch"])
    print(f"liver volume {tuple(data.shape)} pointwise, {accumulation}", flush=True)
    assert sw.default_tiles_per_batch([TorchPointwise()], patch, 8) * 8 == 32
    logits = sw.average_fold_device_logits(
        [TorchPointwise()], volume, patch_size=patch, num_outputs=3, mirroring_axes=(0, 1, 2),
        accumulation=accumulation)
    labels = sw.average_fold_labels(
        [TorchPointwise()], volume, patch_size=patch, num_outputs=3, mirroring_axes=(0, 1, 2),
        accumulation=accumulation, return_device=True)
    want = meta[accumulation]
    assert str(logits.dtype).replace("torch.", "") == want["logits_dtype"]
    counts = torch.bincount(labels.reshape(-1).to(torch.int64)).tolist()
    print(f"label counts {counts} (oracle {want['label_counts']})", flush=True)
    assert counts == want["label_counts"]
    assert _sha(logits) == want["logits_sha256"]
    assert _sha(labels.view(torch.int16)) == want["labels_sha256"]
    # known answer: a pointwise model commutes with the flips, so the Gaussian-weighted
    # mean of its tiles is the model itself up to the rounding of the weighted sums.  In
    # float16 accumulation the Gaussian's far corners are the smallest subnormal half
    # (the runner's zero replacement), so voxels reached only by tile corners (the volume's
    # corners) carry products quantised to a few subnormal steps: there the bound holds
    # for all but a tiny fraction of the voxels.
    v = volume[0]
    expect = torch.stack((v * 1.5, -v * 1.5, v * v), dim=-1)
    dev_rel = (logits.float() - expect).abs() / (expect.abs() + 1.0)
    if accumulation == "float32":
        err = dev_rel.max().item()
        print(f"weighted mean vs model: max relative deviation {err:.3e}", flush=True)
        assert err <= 1e-5
    else:
        frac = (dev_rel > 1e-2).float().mean().item()
        print(f"weighted mean vs model: {frac:.2e} of values deviate by more than 1e-2",
              flush=True)
        assert frac <= 1e-3
