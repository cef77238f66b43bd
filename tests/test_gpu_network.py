"""Full-network forward on the HIP path vs the torch-CPU float32 oracle.

Tolerances are the fp32 parity bar: max-abs <= 1e-3 and relative-L2 <= 1e-5 on the
logits, and identical argmax labels on >= 99.99% of voxels.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from nnunet_mlx.model.network import build_network
from nnunet_mlx.model.topology import PlainConvUNetSpec, ResidualEncoderUNetSpec
from nnunet_mlx.storage.synthetic import random_weights
from oracle.network import OracleNetwork
from tests.helpers import rel_l2, report

pytestmark = pytest.mark.gpu

K3 = ((3, 3, 3),)


def liver_spec(cin=1, classes=3, strides=None) -> PlainConvUNetSpec:
    return PlainConvUNetSpec(
        input_channels=cin, num_classes=classes, features=(32, 64, 128, 256, 320, 320),
        kernel_sizes=K3 * 6,
        strides=strides or ((1, 1, 1),) + ((2, 2, 2),) * 5,
        encoder_convs=(2,) * 6, decoder_convs=(2,) * 5,
    )


def resenc_spec() -> ResidualEncoderUNetSpec:
    return ResidualEncoderUNetSpec(
        input_channels=1, num_classes=3, features=(32, 64, 128, 256, 320, 320, 320),
        kernel_sizes=K3 * 7,
        strides=((1, 1, 1),) + ((2, 2, 2),) * 5 + ((2, 1, 1),),
        encoder_blocks=(1, 3, 4, 6, 6, 6, 6), decoder_convs=(1,) * 6,
    )


CASES = {
    "liver-32": (liver_spec(), (32, 32, 32), 2, False),
    "liver-32-affine": (liver_spec(), (32, 32, 32), 1, True),
    "brats-4ch": (liver_spec(cin=4, classes=5), (32, 32, 32), 1, True),
    "autopet-aniso": (liver_spec(cin=2, classes=2, strides=((1, 1, 1),) + ((2, 2, 2),) * 4 + ((1, 2, 2),)),
                      (16, 32, 32), 1, True),
    "tiny-plain": (PlainConvUNetSpec(1, 3, (4, 8), K3 * 2, ((1, 1, 1), (2, 2, 2)), (2, 2), (2,)),
                   (8, 8, 8), 2, True),
    "tiny-residual": (ResidualEncoderUNetSpec(1, 3, (4, 8, 16), K3 * 3, ((1, 1, 1), (2, 2, 2), (2, 2, 2)),
                                              (1, 3, 4), (1, 1)), (8, 8, 8), 2, True),
    "tiny-bottleneck": (ResidualEncoderUNetSpec(1, 3, (4, 8, 16), K3 * 3, ((1, 1, 1), (2, 2, 2), (2, 2, 2)),
                                                (1, 2, 2), (1, 1), bottleneck_channels=(2, 4, 8)),
                        (8, 8, 8), 1, True),
    "resenc-L": (resenc_spec(), (128, 64, 64), 1, True),
    "liver-128": (liver_spec(), (128, 128, 128), 1, True),
    # patch not divisible by the total stride: the decoder centre-crops each upsample
    "plain-nondivisible": (PlainConvUNetSpec(1, 3, (8, 16, 32), K3 * 3,
                                             ((1, 1, 1), (2, 2, 2), (2, 2, 2)), (2, 2, 2), (2, 2)),
                           (13, 18, 21), 2, True),
    # 12 head channels (not a power-of-two number of float4 groups) and batch items that
    # end inside a 256-voxel block of the head
    "plain-12ch-ragged": (PlainConvUNetSpec(1, 3, (12, 24), K3 * 2, ((1, 1, 1), (2, 2, 2)),
                                            (2, 2), (2,)), (7, 9, 11), 2, True),
}


@pytest.mark.parametrize("name", list(CASES))
def test_forward_matches_oracle(device, name):
    """All three convolution arithmetics against the float32 oracle: "fp32" products and
    "fp32-split" fp16-split products at the float32 bar.  "bf16" against the oracle's bf16
    emulation (operands rounded at the same points): identical up to float32 accumulation
    on the two-stage network; on deeper networks a bf16 rounding flipped by a last-bit
    accumulation difference cascades, so there the bar is that the bf16 network lies no
    further from the float32 logits than bf16 rounding itself puts the emulation (x1.25)."""
    spec, patch, batch, affine = CASES[name]
    weights = random_weights(spec, seed=1, random_affine=affine)
    rng = np.random.default_rng(0)
    x = rng.standard_normal((batch, *patch, spec.input_channels)).astype(np.float32)
    residual = isinstance(spec, ResidualEncoderUNetSpec)
    ref = OracleNetwork(spec, weights, residual=residual)(x)
    ref16 = OracleNetwork(spec, weights, residual=residual, bf16=True)(x)
    for precision in ("fp32", "fp32-split", "bf16"):
        print(f"network case {name} patch={patch} batch={batch} precision={precision}", flush=True)
        net = build_network(spec, precision=precision)
        net.load_weights(weights)
        got = net(torch.from_numpy(x).to(device)).cpu().numpy()
        msg = report(f"{name} {precision}", got, ref)
        print(msg, flush=True)
        assert got.shape == ref.shape
        assert np.isfinite(got).all(), msg
        if precision == "bf16":
            inherent = rel_l2(ref16, ref)
            print(f"{name} bf16: emulation vs float32 {inherent:.3e}, "
                  f"network vs emulation {rel_l2(got, ref16):.3e}", flush=True)
            if name == "tiny-plain":
                assert rel_l2(got, ref16) <= 1e-5, report(f"{name} bf16 vs emulation", got, ref16)
            assert rel_l2(got, ref) <= 1.25 * inherent, msg
        else:
            assert np.abs(got - ref).max() <= 1e-3, msg
            assert rel_l2(got, ref) <= 1e-5, msg
            agree = (got.argmax(-1) == ref.argmax(-1)).mean()
            assert agree >= 0.9999, f"{msg} label agreement {agree}"
        net.close()


def _random_topology(seed):
    """A seeded small network: plain or residual (BasicBlockD or BottleneckD), 2-4 stages,
    ragged widths, 3x3x3 or 1x3x3 kernels, isotropic or anisotropic strides, 1-4 input
    channels, 1-5 classes; residual patches divisible by the total stride (the residual
    encoder pools), plain ones of any size (the decoder crops)."""
    rng = np.random.default_rng(seed)
    stages = int(rng.integers(2, 5))
    feats = tuple(int(rng.choice([4, 8, 12, 16, 24, 32, 48])) for _ in range(stages))
    kernels = tuple((3, 3, 3) if rng.random() < 0.75 else (1, 3, 3) for _ in range(stages))
    strides = ((1, 1, 1),) + tuple(tuple(int(v) for v in rng.choice([1, 2, 2], 3))
                                   for _ in range(stages - 1))
    enc = tuple(int(rng.integers(1, 3)) for _ in range(stages))
    dec = tuple(int(rng.integers(1, 3)) for _ in range(stages - 1))
    cin, classes = int(rng.choice([1, 2, 3, 4])), int(rng.integers(1, 6))
    total = np.prod(np.array(strides), axis=0)
    if rng.random() < 0.5:
        bottleneck = tuple(max(2, f // 2) for f in feats) if rng.random() < 0.5 else None
        spec = ResidualEncoderUNetSpec(cin, classes, feats, kernels, strides, enc, dec,
                                       bottleneck_channels=bottleneck)
        patch = tuple(int(t * rng.integers(1, 4)) for t in total)
        patch = tuple(p * max(1, -(-4 // p)) for p in patch)  # at least 4 voxels an axis
    else:
        spec = PlainConvUNetSpec(cin, classes, feats, kernels, strides, enc, dec)
        patch = tuple(int(v) for v in rng.integers(4, 21, 3))
    return spec, patch, int(rng.integers(1, 3))


@pytest.mark.parametrize("seed", range(8))
def test_random_topologies_match_oracle(device, seed):
    """Seeded small topologies no hand-written case above covers, in the float32-product and
    the default fp16-split precision, at the float32 bar against the oracle."""
    spec, patch, batch = _random_topology(700 + seed)
    weights = random_weights(spec, seed=seed, random_affine=True)
    x = np.random.default_rng(seed).standard_normal((batch, *patch, spec.input_channels))
    x = x.astype(np.float32)
    residual = isinstance(spec, ResidualEncoderUNetSpec)
    ref = OracleNetwork(spec, weights, residual=residual)(x)
    for precision in ("fp32", "fp32-split"):
        print(f"random topology {seed}: {spec} patch={patch} batch={batch} precision={precision}",
              flush=True)
        net = build_network(spec, precision=precision)
        net.load_weights(weights)
        got = net(torch.from_numpy(x).to(device)).cpu().numpy()
        msg = report(f"random topology {seed} {precision}", got, ref)
        print(msg, flush=True)
        assert got.shape == ref.shape
        assert np.isfinite(got).all(), msg
        assert np.abs(got - ref).max() <= 1e-3, msg
        assert rel_l2(got, ref) <= 1e-5, msg
        assert (got.argmax(-1) == ref.argmax(-1)).mean() >= 0.9999, msg
        net.close()


@pytest.mark.parametrize("name", ["liver-32", "brats-4ch", "autopet-aniso", "resenc-L", "liver-128"])
def test_bf16_mixed_is_closer_than_bf16(device, name):
    """"bf16-mixed" keeps the full-resolution layers in fp16-split: its logits lie closer to
    the float32 oracle than the all-bf16 network's (both distances printed)."""
    spec, patch, batch, affine = CASES[name]
    weights = random_weights(spec, seed=1, random_affine=affine)
    x = np.random.default_rng(0).standard_normal((batch, *patch, spec.input_channels)).astype(np.float32)
    residual = isinstance(spec, ResidualEncoderUNetSpec)
    ref = OracleNetwork(spec, weights, residual=residual)(x)
    dist = {}
    for precision in ("bf16", "bf16-mixed"):
        print(f"network case {name} precision={precision}", flush=True)
        net = build_network(spec, precision=precision)
        net.load_weights(weights)
        got = net(torch.from_numpy(x).to(device)).cpu().numpy()
        net.close()
        assert np.isfinite(got).all()
        dist[precision] = rel_l2(got, ref)
    print(f"{name}: relative L2 to float32, bf16 {dist['bf16']:.3e}, bf16-mixed "
          f"{dist['bf16-mixed']:.3e}", flush=True)
    assert dist["bf16-mixed"] < dist["bf16"]


@pytest.mark.parametrize("algo", ["winograd", "direct"])
@pytest.mark.parametrize("name", ["liver-32", "brats-4ch", "autopet-aniso", "tiny-residual"])
def test_conv_route_matches_oracle(device, monkeypatch, name, algo):
    """The stride-1 3x3x3 split layers with 16-channel input blocks and C_out % 32 == 0 run
    on the Winograd kernel by default; NNX_CONV_ALGO=direct (read when the weights are
    packed) keeps them on the direct implicit GEMM.  Either route holds the float32 bar, and
    the kernel profile shows which one ran (tiny-residual has no eligible layer)."""
    from nnunet_mlx import _native

    spec, patch, batch, affine = CASES[name]
    weights = random_weights(spec, seed=3, random_affine=affine)
    x = np.random.default_rng(5).standard_normal((batch, *patch, spec.input_channels)).astype(np.float32)
    residual = isinstance(spec, ResidualEncoderUNetSpec)
    ref = OracleNetwork(spec, weights, residual=residual)(x)
    monkeypatch.setenv("NNX_CONV_ALGO", algo)
    print(f"{algo} network case {name} patch={patch} batch={batch}", flush=True)
    net = build_network(spec, precision="fp32-split")
    net.load_weights(weights)
    with _native.KernelProfile() as prof:
        got = net(torch.from_numpy(x).to(device)).cpu().numpy()
    net.close()
    wino = prof.classes.get("conv3d_wino", {}).get("launches", 0)
    direct = sum(c["launches"] for n, c in prof.classes.items() if n.startswith("conv3d_x3s"))
    if algo == "direct" or name == "tiny-residual":
        assert wino == 0, prof.classes.keys()
    else:
        assert wino > 0, prof.classes.keys()
    if algo == "direct" and name != "tiny-residual":
        assert direct > 0, prof.classes.keys()
    msg = report(f"{name} {algo}", got, ref)
    print(msg, f"winograd launches {wino}", flush=True)
    assert np.isfinite(got).all(), msg
    assert np.abs(got - ref).max() <= 1e-3, msg
    assert rel_l2(got, ref) <= 1e-5, msg


def test_persistent_winograd_forward_is_bit_identical(device, monkeypatch):
    """The persistent Winograd kernel runs the layers with at least four boxes a CU (here
    the 64^3 and 32^3 stages at batch 4) with the one-box kernel's arithmetic, including
    what the plain kernel tests do not reach: pending InstanceNorm + LeakyReLU on load
    (interior and border boxes, and the transposed convolution's half without one), the
    concatenated decoder input and the InstanceNorm partials of the epilogue.  The whole
    forward is therefore bit-identical with the persistent kernel switched off."""
    spec = liver_spec()
    weights = random_weights(spec, seed=7, random_affine=True)
    x = np.random.default_rng(11).standard_normal((4, 64, 64, 64, 1)).astype(np.float32)
    print("persistent vs one-box Winograd: liver network 64^3 batch 4", flush=True)
    outs = {}
    for flag in ("1", "0"):
        monkeypatch.setenv("NNX_WINO_PERSISTENT", flag)
        net = build_network(spec, precision="fp32-split")
        net.load_weights(weights)
        outs[flag] = net(torch.from_numpy(x).to(device)).cpu().numpy()
        net.close()
    assert np.isfinite(outs["1"]).all()
    assert np.array_equal(outs["1"].view(np.uint32), outs["0"].view(np.uint32)), \
        f"{int((outs['1'] != outs['0']).sum())} logits differ"


def test_forward_rejects_bad_input(device):
    from nnunet_mlx.errors import ContractError

    spec = CASES["tiny-plain"][0]
    net = build_network(spec)
    with pytest.raises(ContractError):
        net(torch.zeros((1, 8, 8, 8, 1), device=device))  # weights not loaded
    net.load_weights(random_weights(spec, seed=0))
    with pytest.raises(ContractError):
        net(torch.zeros((1, 8, 8, 8, 2), device=device))  # wrong channel count
    res_spec = CASES["tiny-residual"][0]
    res = build_network(res_spec)
    res.load_weights(random_weights(res_spec, seed=0))
    with pytest.raises(ContractError):
        # odd sizes: the stride-2 conv rounds up, the shortcut's average pool rounds down
        res(torch.zeros((1, 9, 8, 8, 1), device=device))


def test_forward_rejects_items_beyond_the_activation_limit(device):
    """A batch item whose full-resolution activation exceeds 2^31 elements (the kernels'
    per-item offsets are 32-bit) is refused while the workspace is planned, before any
    allocation or kernel; a batch of many items beyond 2^31 elements in total is fine (the
    real-shape workload tests run such batches)."""
    from nnunet_mlx.errors import ContractError

    spec = liver_spec()
    net = build_network(spec)
    net.load_weights(random_weights(spec, seed=0))
    x = torch.zeros((1, 288, 512, 512, 1), device=device)   # 288 * 512^2 * 32 > 2^31
    print("activation-limit case: one item of 288x512x512", flush=True)
    with pytest.raises(ContractError, match="2\\^31"):
        net(x)
    net.close()


def test_activations_beyond_the_split_range_name_the_layer():
    """A checkpoint whose activations leave the split-fp16 operand range (an InstanceNorm
    gamma of 1e4 after an outlier voxel: normalised activations near 1e5 at the input of the
    second convolution, beyond fp16's 65504) makes the fp32-split forward and sliding window
    raise a ContractError that names the first layer with non-finite output, never a silent
    result; the fp32 precision takes the same checkpoint and holds the float32 bar."""
    from nnunet_mlx.errors import ContractError
    from nnunet_mlx.prediction import sliding_window as sw

    spec = PlainConvUNetSpec(1, 2, (32, 64), K3 * 2, ((1, 1, 1), (2, 2, 2)), (2, 2), (2,))
    weights = random_weights(spec, seed=3)
    weights["enc0.block0.norm.weight"] = np.full(32, 1e4, dtype=np.float32)
    x = np.random.default_rng(5).standard_normal((2, 16, 16, 16, 1)).astype(np.float32)
    x[:, 8, 8, 8, 0] = 1e4
    print("split range: gamma 1e4 after an outlier voxel, 16^3 batch 2", flush=True)
    net = build_network(spec)  # fp32-split
    net.load_weights(weights)
    with pytest.raises(ContractError, match=r"enc0\.block1\.conv\.weight.*precision='fp32'"):
        net(torch.from_numpy(x).cuda())
    volume = np.ascontiguousarray(x[0].transpose(3, 0, 1, 2))
    with pytest.raises(ContractError, match=r"enc0\.block1\.conv\.weight"):
        sw.predict_device_logits(net, volume, patch_size=(16, 16, 16), num_classes=2)
    net.close()
    ref = OracleNetwork(spec, weights)(x)
    fp32 = build_network(spec, precision="fp32")
    fp32.load_weights(weights)
    got = fp32(torch.from_numpy(x).cuda()).cpu().numpy()
    fp32.close()
    msg = report("split range, fp32 precision", got, ref)
    print(msg, flush=True)
    assert np.isfinite(got).all() and rel_l2(got, ref) <= 1e-5, msg
    assert np.abs(got - ref).max() <= 1e-3 * max(1.0, np.abs(ref).max()), msg
