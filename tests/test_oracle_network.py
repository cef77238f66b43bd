"""Pinning of the network oracle on the CPU.

Convolutions and transposed convolutions are checked against float64 brute force (and
the reference's matmul + interleave formulation of the stride==kernel transposed conv),
the instance norm against torch's textbook ``F.instance_norm`` and its special cases, the
parameter naming against an independent count of the upstream network's parameters, and
the module composition (skip order, concat order, which seg head) against a float64
composition of the brute-force pieces.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from nnunet_mlx.model.topology import PlainConvUNetSpec, ResidualEncoderUNetSpec
from nnunet_mlx.storage.synthetic import parameter_shapes, random_weights
from oracle.network import (
    OracleNetwork,
    brute_force_conv3d,
    brute_force_tconv3d,
    conv_weight_to_torch,
    instance_norm,
    tconv_weight_to_torch,
)


@pytest.mark.parametrize("stride,kernel", [((1, 1, 1), (3, 3, 3)), ((2, 2, 2), (3, 3, 3)),
                                           ((1, 2, 2), (1, 3, 3)), ((1, 1, 1), (1, 1, 1))])
def test_torch_conv_usage_matches_brute_force(stride, kernel):
    rng = np.random.default_rng(0)
    x = rng.standard_normal((2, 5, 6, 7, 3)).astype(np.float32).astype(np.float64)
    w = rng.standard_normal((4, *kernel, 3)).astype(np.float32).astype(np.float64)
    ref = brute_force_conv3d(x, w, stride)
    xt = torch.from_numpy(x).permute(0, 4, 1, 2, 3)
    got = F.conv3d(xt, conv_weight_to_torch(w).double(), None, stride=stride,
                   padding=tuple(k // 2 for k in kernel))
    np.testing.assert_allclose(got.permute(0, 2, 3, 4, 1).numpy(), ref, rtol=1e-6, atol=1e-5)


def test_brute_force_conv_single_tap_known_answer():
    x = np.arange(27, dtype=np.float64).reshape(1, 3, 3, 3, 1)
    w = np.zeros((1, 3, 3, 3, 1))
    w[0, 2, 1, 1, 0] = 1.0  # picks the voxel one step ahead along z
    out = brute_force_conv3d(x, w, (1, 1, 1))
    np.testing.assert_array_equal(out[0, :2, :, :, 0], x[0, 1:, :, :, 0])
    np.testing.assert_array_equal(out[0, 2, :, :, 0], 0)


@pytest.mark.parametrize("k", [(2, 2, 2), (1, 2, 2), (2, 1, 2)])
def test_transposed_conv_matches_brute_force_and_matmul_interleave(k):
    rng = np.random.default_rng(1)
    # float32-representable values: the oracle's weight helpers hold float32 tensors
    x = rng.standard_normal((2, 3, 4, 2, 5)).astype(np.float32).astype(np.float64)
    w = rng.standard_normal((6, *k, 5)).astype(np.float32).astype(np.float64)  # (C_out, kD, kH, kW, C_in)
    ref = brute_force_tconv3d(x, w)
    xt = torch.from_numpy(x).permute(0, 4, 1, 2, 3)
    got = F.conv_transpose3d(xt, tconv_weight_to_torch(w).double(), None, stride=k)
    np.testing.assert_allclose(got.permute(0, 2, 3, 4, 1).numpy(), ref, rtol=1e-12, atol=1e-12)
    # the reference's formulation: matmul against (C_out*K, C_in), then transpose
    # (0, 1, 5, 2, 6, 3, 7, 4) to interleave the kernel offsets (network.py:139-174)
    b, d, h, wd, c = x.shape
    proj = x.reshape(-1, c) @ w.reshape(-1, c).T
    proj = proj.reshape(b, d, h, wd, 6, *k).transpose(0, 1, 5, 2, 6, 3, 7, 4)
    proj = proj.reshape(b, d * k[0], h * k[1], wd * k[2], 6)
    np.testing.assert_allclose(proj, ref, rtol=1e-12, atol=1e-12)


def test_instance_norm_matches_textbook():
    rng = np.random.default_rng(2)
    x = torch.from_numpy((rng.standard_normal((2, 5, 6, 7, 8)) * 2 + 3).astype(np.float32))
    bias = torch.from_numpy(rng.standard_normal(5).astype(np.float32))
    gamma = torch.from_numpy((1 + 0.3 * rng.standard_normal(5)).astype(np.float32))
    beta = torch.from_numpy(rng.standard_normal(5).astype(np.float32))
    got = instance_norm(x, gamma, beta, 1e-5, input_bias=bias, negative_slope=0.01)
    xb = (x + bias.view(1, -1, 1, 1, 1)).double()
    ref = F.instance_norm(xb, weight=gamma.double(), bias=beta.double(), eps=1e-5)
    ref = torch.maximum(0.01 * ref, ref)
    np.testing.assert_allclose(got.numpy(), ref.numpy(), rtol=1e-5, atol=2e-6)


def test_instance_norm_special_cases():
    x = torch.full((1, 2, 3, 3, 3), 0.7, dtype=torch.float32)
    x[0, 1] = torch.arange(27, dtype=torch.float32).view(3, 3, 3)
    beta = torch.tensor([0.25, 0.0])
    out = instance_norm(x, None, beta, 1e-5)
    assert torch.all(out[0, 0] == 0.25)  # constant channel: variance clamped, output = beta
    relu = instance_norm(x, None, None, 1e-5, negative_slope=0.0)
    assert torch.all(relu >= 0)
    ident = instance_norm(x, None, None, 1e-5, negative_slope=1.0)
    np.testing.assert_array_equal(ident.numpy(), instance_norm(x, None, None, 1e-5).numpy())


def _upstream_param_count(spec: PlainConvUNetSpec) -> int:
    """Independent count of dynamic-network-architectures' PlainConvUNet parameters with
    conv bias, affine instance norm and all deep-supervision seg layers."""
    total = 0
    cin = spec.input_channels
    for stage, f in enumerate(spec.features):
        for j in range(spec.encoder_convs[stage]):
            c = cin if j == 0 else f
            total += c * f * 27 + f + 2 * f
        cin = f
    for d in range(len(spec.features) - 1):
        below, skip = spec.features[-1 - d], spec.features[-2 - d]
        total += below * skip * 8 + skip
        for j in range(spec.decoder_convs[d]):
            c = 2 * skip if j == 0 else skip
            total += c * skip * 27 + skip + 2 * skip
        total += skip * spec.num_classes + spec.num_classes
    return total


def liver() -> PlainConvUNetSpec:
    return PlainConvUNetSpec(1, 3, (32, 64, 128, 256, 320, 320), ((3, 3, 3),) * 6,
                             ((1, 1, 1),) + ((2, 2, 2),) * 5, (2,) * 6, (2,) * 5)


def test_parameter_names_and_count():
    spec = liver()
    shapes = parameter_shapes(spec)
    assert sum(int(np.prod(s)) for s in shapes.values()) == _upstream_param_count(spec)
    assert shapes["enc0.block0.conv.weight"] == (32, 3, 3, 3, 1)
    assert shapes["up0.weight"] == (320, 2, 2, 2, 320)
    assert shapes["dec4.block0.conv.weight"] == (32, 3, 3, 3, 64)
    assert shapes["seg4.weight"] == (3, 1, 1, 1, 32)
    assert "seg0.bias" in shapes and len(shapes) == 108


def test_residual_parameter_names():
    spec = ResidualEncoderUNetSpec(1, 3, (4, 8), ((3, 3, 3),) * 2, ((1, 1, 1), (2, 2, 2)), (1, 2), (1,))
    shapes = parameter_shapes(spec)
    assert "stem.conv.weight" in shapes
    assert shapes["res1.block0.proj.conv.weight"] == (8, 1, 1, 1, 4)
    assert "res1.block0.proj.conv.bias" not in shapes  # projection conv has no bias
    assert "res1.block1.proj.conv.weight" not in shapes
    assert shapes["res1.block0.conv1.conv.weight"] == (8, 3, 3, 3, 4)


def _norm64(x, bias, gamma, beta, slope):
    v = x + bias
    mean = v.mean(axis=(1, 2, 3), keepdims=True)
    var = v.var(axis=(1, 2, 3), keepdims=True)
    r = (v - mean) / np.sqrt(var + 1e-5) * gamma + beta
    return np.maximum(slope * r, r) if slope is not None else r


def test_plain_network_composition_against_float64():
    """Tiny PlainConvUNet: oracle vs a float64 composition of brute-force pieces
    (decoder pops the deepest skip first, concatenates (up, skip), applies seg{n-1})."""
    spec = PlainConvUNetSpec(1, 3, (4, 8, 8), ((3, 3, 3),) * 3, ((1, 1, 1), (2, 2, 2), (2, 2, 2)),
                             (2, 1, 1), (1, 2))
    w = random_weights(spec, seed=3, random_affine=True)
    x = np.random.default_rng(4).standard_normal((1, 8, 8, 8, 1)).astype(np.float32)
    got = OracleNetwork(spec, w)(x)

    def cn(prefix, h, stride):
        y = brute_force_conv3d(h, w[f"{prefix}.conv.weight"], stride)
        return _norm64(y, w[f"{prefix}.conv.bias"], w[f"{prefix}.norm.weight"],
                       w[f"{prefix}.norm.bias"], 0.01)

    h = x.astype(np.float64)[0:1]
    skips = []
    h = cn("enc0.block0", h, (1, 1, 1))
    h = cn("enc0.block1", h, (1, 1, 1))
    skips.append(h)
    h = cn("enc1.block0", h, (2, 2, 2))
    skips.append(h)
    h = cn("enc2.block0", h, (2, 2, 2))
    for d, skip in enumerate(reversed(skips)):
        up = brute_force_tconv3d(h, w[f"up{d}.weight"]) + w[f"up{d}.bias"]
        h = np.concatenate([up, skip], axis=-1)
        for j in range(spec.decoder_convs[d]):
            h = cn(f"dec{d}.block{j}", h, (1, 1, 1))
    ref = np.einsum("nzyxc,oc->nzyxo", h, w["seg1.weight"][:, 0, 0, 0, :].astype(np.float64)) + w["seg1.bias"]
    np.testing.assert_allclose(got, ref, rtol=1e-4, atol=1e-4)


def _rne_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even to bf16 by integer arithmetic on the float32 bits (finite
    inputs): add 0x7FFF plus the lowest kept bit, truncate the low 16 bits."""
    u = x.astype(np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16 << 16
    return u.astype(np.uint32).view(np.float32)


def test_round_bf16_is_nearest_even():
    from oracle.network import round_bf16

    one = np.float32(1.0)
    cases = {
        1.0: 1.0,
        1 + 2.0**-8: 1.0,                    # tie -> even (mantissa 0)
        1 + 3 * 2.0**-8: 1 + 2.0**-6,        # tie -> even (mantissa 2)
        1 + 2.0**-8 + 2.0**-20: 1 + 2.0**-7,  # just above the tie
        -(1 + 3 * 2.0**-8): -(1 + 2.0**-6),
        65504.0: 65536.0,
    }
    got = round_bf16(torch.tensor(list(cases), dtype=torch.float32)).numpy()
    np.testing.assert_array_equal(got, np.array(list(cases.values()), dtype=np.float32))
    x = (np.random.default_rng(12).standard_normal(100_000) * 10.0 ** np.random.default_rng(13)
         .integers(-20, 20, 100_000)).astype(np.float32)
    np.testing.assert_array_equal(round_bf16(torch.from_numpy(x)).numpy(), _rne_bf16_bits(x))
    assert one == round_bf16(torch.tensor([one])).item()


def test_bf16_oracle_rounding_points():
    """bf16 mode rounds the operands of the 3-D convolutions with >= 8 taps except the one
    reading the network input, and of the transposed convolutions; nothing else.  The
    logits then move by a bf16-sized amount."""
    spec = PlainConvUNetSpec(1, 3, (4, 8), ((3, 3, 3), (3, 3, 3)), ((1, 1, 1), (2, 2, 2)), (2, 2), (2,))
    w = random_weights(spec, seed=5, random_affine=True)
    net = OracleNetwork(spec, w, bf16=True)
    x = torch.randn(1, 4, 6, 6, 6, generator=torch.Generator().manual_seed(0))
    k3 = torch.randn(8, 4, 3, 3, 3, generator=torch.Generator().manual_seed(1))
    k1 = torch.randn(8, 4, 1, 1, 1, generator=torch.Generator().manual_seed(2))
    from oracle.network import round_bf16

    for prefix, weight, rounded in (("enc0.block1", k3, True), ("dec0.block0", k3, True),
                                    ("up", k3, True), ("enc0.block0", k3, False),
                                    ("stem", k3, False), ("res1.block0.proj", k1, False)):
        xo, wo = net._bf16_operands(prefix, x, weight)
        assert torch.equal(xo, round_bf16(x) if rounded else x), prefix
        assert torch.equal(wo, round_bf16(weight) if rounded else weight), prefix
    xo, wo = OracleNetwork(spec, w)._bf16_operands("enc0.block1", x, k3)
    assert xo is x and wo is k3
    xs = np.random.default_rng(6).standard_normal((1, 8, 8, 8, 1)).astype(np.float32)
    full = OracleNetwork(spec, w)(xs)
    emulated = net(xs)
    rel = np.linalg.norm(emulated - full) / np.linalg.norm(full)
    assert 1e-5 < rel < 3e-2


def _pool64(h, stride):
    """float64 average pooling with kernel = stride (sizes divisible), channels-last."""
    n, d, hh, w, c = h.shape
    a, b, e = stride
    return h.reshape(n, d // a, a, hh // b, b, w // e, e, c).mean(axis=(2, 4, 6))


def _leaky64(v, slope=0.01):
    return np.maximum(slope * v, v)


def _residual_reference(spec, w, x, variant=None):
    """float64 composition of a ResidualEncoderUNet from brute-force pieces, written from
    the block definitions (src/nnunet_mlx/model/network.py:467-602): the shortcut is the
    input, average-pooled by the block's stride when it is not 1, then a bias-free 1x1
    ConvNorm when the channel count changes; the branch is ConvNormAct(stride) then ConvNorm
    (BasicBlockD) or 1x1 ConvNormAct, kxk ConvNormAct(stride), 1x1 ConvNorm (BottleneckD);
    the block output is LeakyReLU(branch + shortcut).  ``variant`` builds a deliberately
    wrong block ("act_before_add": LeakyReLU(LeakyReLU(branch) + shortcut);
    "pool_after_projection": the projection at full resolution, then the pooling)."""

    def cn(prefix, h, stride, act, bias=True):
        y = brute_force_conv3d(h, w[f"{prefix}.conv.weight"], stride)
        b = w[f"{prefix}.conv.bias"] if bias else np.zeros(y.shape[-1])
        return _norm64(y, b, w[f"{prefix}.norm.weight"], w[f"{prefix}.norm.bias"],
                       0.01 if act else None)

    h = cn("stem", x.astype(np.float64), (1, 1, 1), True)
    skips = []
    for s in range(len(spec.features)):
        for b in range(spec.encoder_blocks[s]):
            stride = tuple(spec.strides[s]) if b == 0 else (1, 1, 1)
            pre = f"res{s}.block{b}"
            pool_first = variant != "pool_after_projection"
            shortcut = h if stride == (1, 1, 1) or not pool_first else _pool64(h, stride)
            if f"{pre}.proj.conv.weight" in w:
                shortcut = cn(f"{pre}.proj", shortcut, (1, 1, 1), False, bias=False)
            if stride != (1, 1, 1) and not pool_first:
                shortcut = _pool64(shortcut, stride)
            if spec.bottleneck_channels is None:
                branch = cn(f"{pre}.conv2", cn(f"{pre}.conv1", h, stride, True), (1, 1, 1),
                            variant == "act_before_add")
            else:
                t = cn(f"{pre}.conv1", h, (1, 1, 1), True)
                t = cn(f"{pre}.conv2", t, stride, True)
                branch = cn(f"{pre}.conv3", t, (1, 1, 1), variant == "act_before_add")
            h = _leaky64(branch + shortcut)
        skips.append(h)
    h = skips.pop()
    for d in range(len(spec.features) - 1):
        skip = skips.pop()
        up = brute_force_tconv3d(h, w[f"up{d}.weight"]) + w[f"up{d}.bias"]
        h = np.concatenate([up, skip], axis=-1)
        for j in range(spec.decoder_convs[d]):
            h = cn(f"dec{d}.block{j}", h, (1, 1, 1), True)
    last = len(spec.features) - 2
    return (np.einsum("nzyxc,oc->nzyxo", h, w[f"seg{last}.weight"][:, 0, 0, 0, :].astype(np.float64))
            + w[f"seg{last}.bias"])


RESIDUAL_CASES = {
    # BasicBlockD: stride-1 first stage with a stem of its own width (projection without
    # pooling), strided stages with pooling + projection, two blocks in a stage
    "basic": ResidualEncoderUNetSpec(2, 3, (4, 8, 8), ((3, 3, 3),) * 3,
                                     ((1, 1, 1), (2, 2, 2), (1, 2, 2)), (1, 2, 1), (1, 2),
                                     stem_channels=6),
    # BottleneckD: 1x1 / kxk (stride) / 1x1 branch
    "bottleneck": ResidualEncoderUNetSpec(1, 2, (4, 8), ((3, 3, 3),) * 2, ((1, 1, 1), (2, 2, 2)),
                                          (2, 1), (1,), bottleneck_channels=(2, 3)),
}


@pytest.mark.parametrize("name", sorted(RESIDUAL_CASES))
def test_residual_network_composition_against_float64(name):
    """Tiny ResidualEncoderUNets: the oracle's residual path vs the float64 composition."""
    spec = RESIDUAL_CASES[name]
    w = random_weights(spec, seed=7, random_affine=True)
    x = np.random.default_rng(8).standard_normal((1, 8, 8, 8, spec.input_channels)).astype(np.float32)
    got = OracleNetwork(spec, w, residual=True)(x)
    ref = _residual_reference(spec, w, x)
    np.testing.assert_allclose(got, ref, rtol=1e-4, atol=1e-4)


def test_residual_composition_detects_misplaced_operations():
    """The composition tells the block variants apart: with LeakyReLU applied to the branch
    before the residual addition, or with the shortcut pooled after its projection, the
    logits move far beyond the tolerance the oracle is held to above, so an oracle with
    either mistake fails test_residual_network_composition_against_float64."""
    spec = RESIDUAL_CASES["basic"]
    w = random_weights(spec, seed=7, random_affine=True)
    x = np.random.default_rng(8).standard_normal((1, 8, 8, 8, spec.input_channels)).astype(np.float32)
    got = OracleNetwork(spec, w, residual=True)(x)
    for variant in ("act_before_add", "pool_after_projection"):
        wrong = _residual_reference(spec, w, x, variant=variant)
        assert np.abs(wrong - got).max() > 50 * 1e-4, variant
