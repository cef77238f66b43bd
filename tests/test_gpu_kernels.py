"""Per-kernel parity of the HIP path against float64 / numpy references.

Convolutions, transposed convolution and the seg head are compared with float64 torch-CPU
operators (rel-L2 <= 1e-5 and max-abs <= 1e-4 * max|ref|, float32 accumulation over up to
17,280 products); instance norm with a float64 restatement; the sliding-window kernels
(gather+flip, mirror-average + Gaussian accumulation, fold add, finalize) bit for bit with
numpy float32/float16 arithmetic in the reference's operation order.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from nnunet_mlx import _native
from tests.helpers import dev, host, rel_l2, report, stream

pytestmark = pytest.mark.gpu


def _conv_ref64(x, w, stride):
    xt = torch.from_numpy(x.astype(np.float64)).permute(0, 4, 1, 2, 3)
    wt = torch.from_numpy(w.astype(np.float64)).permute(0, 4, 1, 2, 3)
    pad = tuple(k // 2 for k in w.shape[1:4])
    y = F.conv3d(xt, wt, None, stride=tuple(stride), padding=pad)
    return y.permute(0, 2, 3, 4, 1).numpy()


CONV_CASES = [
    # batch, in_size, c1, c2, cout, kernel, stride
    (1, (8, 8, 8), 4, 0, 8, (3, 3, 3), (1, 1, 1)),
    (2, (16, 16, 16), 32, 0, 32, (3, 3, 3), (1, 1, 1)),
    (1, (17, 9, 20), 32, 0, 32, (3, 3, 3), (1, 1, 1)),
    (2, (16, 16, 16), 32, 32, 32, (3, 3, 3), (1, 1, 1)),
    (1, (16, 16, 16), 32, 0, 64, (3, 3, 3), (2, 2, 2)),
    (1, (15, 13, 17), 32, 0, 64, (3, 3, 3), (2, 2, 2)),
    (1, (12, 12, 12), 64, 0, 64, (3, 3, 3), (1, 1, 1)),
    (2, (8, 8, 8), 128, 0, 128, (3, 3, 3), (1, 1, 1)),
    (1, (24, 24, 32), 64, 0, 128, (3, 3, 3), (1, 1, 1)),
    (1, (4, 4, 4), 320, 320, 320, (3, 3, 3), (1, 1, 1)),
    (1, (8, 8, 8), 256, 0, 320, (3, 3, 3), (2, 2, 2)),
    (1, (7, 10, 8), 2, 0, 32, (3, 3, 3), (1, 2, 2)),
    (1, (6, 8, 8), 8, 0, 16, (1, 3, 3), (1, 1, 1)),
    (1, (8, 8, 8), 16, 0, 32, (1, 1, 1), (1, 1, 1)),
    (1, (9, 9, 9), 3, 0, 5, (3, 3, 3), (1, 1, 1)),
    (1, (5, 7, 6), 12, 20, 24, (3, 3, 3), (1, 1, 1)),
    # strided with two inputs of ragged channel counts; strided along y, x only with a
    # 1 x 3 x 3 kernel
    (2, (9, 12, 10), 12, 20, 24, (3, 3, 3), (2, 2, 2)),
    (1, (6, 14, 13), 8, 0, 16, (1, 3, 3), (1, 2, 2)),
    # strided with enough output tiles (1024 workgroups) for the 128-column split tiles
    (2, (32, 64, 64), 16, 0, 256, (3, 3, 3), (2, 2, 2)),
]


@pytest.mark.parametrize("case", CONV_CASES, ids=lambda c: f"b{c[0]}-{c[1]}-c{c[2]}+{c[3]}-o{c[4]}-k{c[5]}-s{c[6]}")
def test_conv3d_igemm_matches_float64(lib, case):
    batch, size, c1, c2, cout, kernel, stride = case
    print(f"conv case {case}", flush=True)
    rng = np.random.default_rng(hash(case) % 2**32)
    x1 = rng.standard_normal((batch, *size, c1)).astype(np.float32)
    x2 = rng.standard_normal((batch, *size, c2)).astype(np.float32) if c2 else None
    w = (rng.standard_normal((cout, *kernel, c1 + c2)) / np.sqrt((c1 + c2) * np.prod(kernel))).astype(np.float32)
    bias = rng.standard_normal(cout).astype(np.float32)
    out_size = [(s + 2 * (k // 2) - k) // st + 1 for s, k, st in zip(size, kernel, stride)]
    k_c = _native.ints(kernel)
    packed = torch.empty(lib.nnx_conv3d_packed_floats(cout, k_c, c1, c2), dtype=torch.float32, device="cuda")
    dw = dev(w)
    _native.check(lib.nnx_conv3d_pack_weight(dw.data_ptr(), cout, k_c, c1, c2, packed.data_ptr(), stream()))
    dx1 = dev(x1)
    dx2 = dev(x2) if c2 else None
    db = dev(bias)
    y = torch.full((batch, *out_size, cout), float("nan"), dtype=torch.float32, device="cuda")
    _native.check(lib.nnx_conv3d_igemm(
        dx1.data_ptr(), c1, dx2.data_ptr() if c2 else None, c2, packed.data_ptr(), db.data_ptr(),
        y.data_ptr(), batch, _native.ints(size), cout, k_c, _native.ints(stride), stream()))
    got = host(y)
    full = np.concatenate([x1, x2], axis=-1) if c2 else x1
    ref = _conv_ref64(full, w, stride) + bias.astype(np.float64)
    msg = report("conv", got, ref)
    assert np.isfinite(got).all(), msg
    assert rel_l2(got, ref) <= 1e-5, msg
    assert np.abs(got - ref).max() <= 1e-4 * max(1.0, np.abs(ref).max()), msg


def _random_conv_cases(seed, n):
    """Seeded shapes for the sweeps below: ragged channel counts, per-axis kernels of 1 or 3
    and strides of 1 or 2, volumes from one voxel to a few tiles."""
    rng = np.random.default_rng(seed)
    cases = []
    for _ in range(n):
        kernel = tuple(int(k) for k in rng.choice([1, 3], 3, p=[0.25, 0.75]))
        stride = tuple(int(t) for t in rng.choice([1, 2], 3))
        size = tuple(int(v) for v in rng.integers(1, 17, 3))
        c2 = int(rng.choice([0, 0, int(rng.integers(1, 25))]))
        cases.append((int(rng.integers(1, 4)), size, int(rng.integers(1, 49)), c2,
                      int(rng.integers(1, 73)), kernel, stride))
    return cases


@pytest.mark.parametrize("case", CONV_CASES, ids=lambda c: f"b{c[0]}-{c[1]}-c{c[2]}+{c[3]}-o{c[4]}-k{c[5]}-s{c[6]}")
def test_conv3d_split_matches_float64(lib, case):
    """Split-fp16 products (hi*hi + hi*lo + lo*hi) hold the same float32 bar as the fp32 kernel."""
    _check_split_conv(lib, case)


@pytest.mark.parametrize("case", _random_conv_cases(2026, 12),
                         ids=lambda c: f"b{c[0]}-{c[1]}-c{c[2]}+{c[3]}-o{c[4]}-k{c[5]}-s{c[6]}")
def test_conv3d_split_random_shapes_match_float64(lib, case):
    """The same bar over a seeded sweep of shapes no hand-picked case above covers."""
    _check_split_conv(lib, case)


def _check_split_conv(lib, case):
    batch, size, c1, c2, cout, kernel, stride = case
    print(f"split conv case {case}", flush=True)
    rng = np.random.default_rng((hash(case) + 7) % 2**32)
    x1 = rng.standard_normal((batch, *size, c1)).astype(np.float32)
    x2 = rng.standard_normal((batch, *size, c2)).astype(np.float32) if c2 else None
    w = (rng.standard_normal((cout, *kernel, c1 + c2)) / np.sqrt((c1 + c2) * np.prod(kernel))).astype(np.float32)
    # a few weights three decades below the rest exercise the low halves of small values
    w.reshape(-1)[:: 7] *= 1e-3
    bias = rng.standard_normal(cout).astype(np.float32)
    out_size = [(s + 2 * (k // 2) - k) // st + 1 for s, k, st in zip(size, kernel, stride)]
    k_c = _native.ints(kernel)
    scale = lib.nnx_split_weight_scale(float(np.abs(w).max()))
    assert scale > 0 and np.log2(scale) == int(np.log2(scale))
    assert 2.0**14 <= np.abs(w).max() * scale < 2.0**15
    nbytes = lib.nnx_conv3d_split_packed_bytes(cout, k_c, c1, c2)
    packed = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    dw = dev(w)
    _native.check(lib.nnx_conv3d_split_pack_weight(dw.data_ptr(), cout, k_c, c1, c2, scale,
                                                   packed.data_ptr(), stream()))
    dx1 = dev(x1)
    dx2 = dev(x2) if c2 else None
    db = dev(bias)
    y = torch.full((batch, *out_size, cout), float("nan"), dtype=torch.float32, device="cuda")
    _native.check(lib.nnx_conv3d_split(
        dx1.data_ptr(), c1, dx2.data_ptr() if c2 else None, c2, packed.data_ptr(), scale,
        db.data_ptr(), y.data_ptr(), batch, _native.ints(size), cout, k_c, _native.ints(stride),
        stream()))
    got = host(y)
    full = np.concatenate([x1, x2], axis=-1) if c2 else x1
    ref = _conv_ref64(full, w, stride) + bias.astype(np.float64)
    msg = report("split conv", got, ref)
    assert np.isfinite(got).all(), msg
    assert rel_l2(got, ref) <= 1e-5, msg
    assert np.abs(got - ref).max() <= 1e-4 * max(1.0, np.abs(ref).max()), msg


WINOGRAD_CASES = [
    # batch, in_size, c1, c2, cout
    (2, (16, 16, 16), 32, 0, 32),
    (1, (17, 9, 20), 32, 0, 32),     # ragged: partial 4 x 8 x 8 boxes on every axis
    (2, (16, 16, 16), 32, 32, 32),   # concat-free decoder input
    (1, (12, 12, 12), 64, 0, 64),
    (2, (8, 8, 8), 128, 0, 128),
    (1, (24, 24, 32), 64, 0, 128),
    (1, (4, 4, 4), 320, 320, 320),
    (1, (5, 7, 6), 16, 16, 32),      # smaller than one box
    (3, (9, 13, 11), 48, 16, 96),
]


def _random_winograd_cases(seed, n):
    """Seeded Winograd shapes: 16-channel input blocks on one or two inputs, 32-column output
    blocks, volumes from one voxel to several ragged 4 x 8 x 8 boxes."""
    rng = np.random.default_rng(seed)
    return [(int(rng.integers(1, 4)), tuple(int(v) for v in rng.integers(1, 21, 3)),
             16 * int(rng.integers(1, 5)), 16 * int(rng.choice([0, 0, 1, 2])),
             32 * int(rng.integers(1, 4))) for _ in range(n)]


@pytest.mark.parametrize("case", WINOGRAD_CASES, ids=lambda c: f"b{c[0]}-{c[1]}-c{c[2]}+{c[3]}-o{c[4]}")
def test_conv3d_winograd_matches_float64(lib, case):
    """Winograd F(2x2x2, 3x3x3) with split-fp16 products holds the float32 bar of the
    direct kernels against float64 (activations up to ~30, weights spanning three decades)."""
    _check_winograd_conv(lib, case)


@pytest.mark.parametrize("case", _random_winograd_cases(2027, 10),
                         ids=lambda c: f"b{c[0]}-{c[1]}-c{c[2]}+{c[3]}-o{c[4]}")
def test_conv3d_winograd_random_shapes_match_float64(lib, case):
    """The same bar over a seeded sweep of Winograd shapes."""
    _check_winograd_conv(lib, case)


def _check_winograd_conv(lib, case):
    batch, size, c1, c2, cout = case
    print(f"winograd conv case {case}", flush=True)
    rng = np.random.default_rng((hash(case) + 11) % 2**32)
    x1 = (rng.standard_normal((batch, *size, c1)) * rng.uniform(0.5, 8.0)).astype(np.float32)
    x2 = rng.standard_normal((batch, *size, c2)).astype(np.float32) if c2 else None
    w = (rng.standard_normal((cout, 3, 3, 3, c1 + c2)) / np.sqrt((c1 + c2) * 27)).astype(np.float32)
    w.reshape(-1)[:: 7] *= 1e-3
    bias = rng.standard_normal(cout).astype(np.float32)
    scale = lib.nnx_winograd_weight_scale(float(np.abs(w).max()))
    assert scale > 0 and np.log2(scale) == int(np.log2(scale))
    packed = torch.empty(lib.nnx_conv3d_winograd_packed_bytes(cout, c1, c2), dtype=torch.uint8,
                         device="cuda")
    dw = dev(w)
    _native.check(lib.nnx_conv3d_winograd_pack_weight(dw.data_ptr(), cout, c1, c2, scale,
                                                      packed.data_ptr(), stream()))
    dx1, db = dev(x1), dev(bias)
    dx2 = dev(x2) if c2 else None
    y = torch.full((batch, *size, cout), float("nan"), dtype=torch.float32, device="cuda")
    _native.check(lib.nnx_conv3d_winograd(
        dx1.data_ptr(), c1, dx2.data_ptr() if c2 else None, c2, packed.data_ptr(), scale,
        db.data_ptr(), y.data_ptr(), batch, _native.ints(size), cout, stream()))
    got = host(y)
    full = np.concatenate([x1, x2], axis=-1) if c2 else x1
    ref = _conv_ref64(full, w, (1, 1, 1)) + bias.astype(np.float64)
    msg = report("winograd conv", got, ref)
    print(msg, flush=True)
    assert np.isfinite(got).all(), msg
    assert rel_l2(got, ref) <= 1e-5, msg
    assert np.abs(got - ref).max() <= 1e-4 * max(1.0, np.abs(ref).max()), msg


PERSISTENT_CASES = [
    # batch, in_size, c1, c2, cout: at least 4 workgroups a CU (the persistent kernel's range)
    (2, (32, 64, 64), 32, 0, 32),
    (8, (20, 40, 36), 32, 32, 64),   # two inputs, two column blocks, ragged x boxes
    (4, (17, 33, 31), 64, 0, 96),    # ragged boxes on every axis, three column blocks
]


def _winograd_run(lib, case, persistent: bool, seed: int = 3):
    import os

    batch, size, c1, c2, cout = case
    rng = np.random.default_rng(seed)
    x1 = (rng.standard_normal((batch, *size, c1)) * 3.0).astype(np.float32)
    x2 = rng.standard_normal((batch, *size, c2)).astype(np.float32) if c2 else None
    w = (rng.standard_normal((cout, 3, 3, 3, c1 + c2)) / np.sqrt((c1 + c2) * 27)).astype(np.float32)
    bias = rng.standard_normal(cout).astype(np.float32)
    scale = lib.nnx_winograd_weight_scale(float(np.abs(w).max()))
    packed = torch.empty(lib.nnx_conv3d_winograd_packed_bytes(cout, c1, c2), dtype=torch.uint8,
                         device="cuda")
    _native.check(lib.nnx_conv3d_winograd_pack_weight(dev(w).data_ptr(), cout, c1, c2, scale,
                                                      packed.data_ptr(), stream()))
    dx1, db = dev(x1), dev(bias)
    dx2 = dev(x2) if c2 else None
    y = torch.full((batch, *size, cout), float("nan"), dtype=torch.float32, device="cuda")
    old = os.environ.get("NNX_WINO_PERSISTENT")
    os.environ["NNX_WINO_PERSISTENT"] = "1" if persistent else "0"
    try:
        _native.check(lib.nnx_conv3d_winograd(
            dx1.data_ptr(), c1, dx2.data_ptr() if c2 else None, c2, packed.data_ptr(), scale,
            db.data_ptr(), y.data_ptr(), batch, _native.ints(size), cout, stream()))
        torch.cuda.synchronize()
    finally:
        if old is None:
            del os.environ["NNX_WINO_PERSISTENT"]
        else:
            os.environ["NNX_WINO_PERSISTENT"] = old
    return host(y), x1, x2, w, bias


@pytest.mark.parametrize("case", PERSISTENT_CASES, ids=lambda c: f"b{c[0]}-{c[1]}-c{c[2]}+{c[3]}-o{c[4]}")
def test_conv3d_winograd_persistent_kernel_is_bit_identical(lib, case):
    """The persistent Winograd kernel (a workgroup a CU looping over boxes, the next box's
    halo and weights requested during the current box's last chunk) computes every box
    with the one-box kernel's arithmetic: its output equals that kernel's bit for bit, and
    holds the float32 bar against float64 on the first case."""
    print(f"winograd persistent case {case}", flush=True)
    got, x1, x2, w, bias = _winograd_run(lib, case, persistent=True)
    ref_kernel, *_ = _winograd_run(lib, case, persistent=False)
    assert np.isfinite(got).all()
    assert np.array_equal(got.view(np.uint32), ref_kernel.view(np.uint32)), \
        f"{int((got != ref_kernel).sum())} values differ"
    if case == PERSISTENT_CASES[0]:
        ref = _conv_ref64(x1, w, (1, 1, 1)) + bias.astype(np.float64)
        msg = report("winograd persistent", got, ref)
        print(msg, flush=True)
        assert rel_l2(got, ref) <= 1e-5, msg
        assert np.abs(got - ref).max() <= 1e-4 * max(1.0, np.abs(ref).max()), msg


def test_conv3d_winograd_rejects_unsupported_layers(lib):
    """Channel counts off the 16 / 32 grid, a second input off the grid and a bad weight
    scale are refused before any launch, with valid buffers so that the layer check (not a
    null pointer) is what refuses; the output keeps its contents."""
    x = torch.zeros((1, 8, 8, 8, 64), dtype=torch.float32, device="cuda")
    packed = torch.zeros(lib.nnx_conv3d_winograd_packed_bytes(64, 64, 64), dtype=torch.uint8,
                         device="cuda")
    y = torch.full((1, 8, 8, 8, 64), 7.0, dtype=torch.float32, device="cuda")
    size = _native.ints((8, 8, 8))
    for c1, c2, cout, scale, needle in [(12, 0, 32, 1.0, "multiples of 16"),
                                        (32, 0, 24, 1.0, "multiples of 16"),
                                        (32, 8, 32, 1.0, "multiples of 16"),
                                        # both inputs on the grid, 1040 channels in all: past
                                        # the kernel's 1024-channel parameter table
                                        (528, 512, 32, 1.0, "at most 1024"),
                                        (32, 0, 32, 0.0, "scale")]:
        rc = lib.nnx_conv3d_winograd(x.data_ptr(), c1, x.data_ptr() if c2 else None, c2,
                                     packed.data_ptr(), scale, None, y.data_ptr(), 1, size, cout,
                                     stream())
        assert rc == _native.NNX_ERR_INVALID, (c1, c2, cout)
        assert needle in _native.last_error(), _native.last_error()
    torch.cuda.synchronize()
    assert bool((y == 7.0).all())


@pytest.mark.parametrize("size,cout", [((16, 16, 16), 32), ((5, 7, 9), 8)])
def test_direct_single_channel_conv(lib, size, cout):
    print(f"direct conv {size} {cout}", flush=True)
    rng = np.random.default_rng(7)
    x = rng.standard_normal((2, *size, 1)).astype(np.float32)
    w = (rng.standard_normal((cout, 3, 3, 3, 1)) * 0.3).astype(np.float32)
    b = rng.standard_normal(cout).astype(np.float32)
    y = torch.empty((2, *size, cout), dtype=torch.float32, device="cuda")
    dx, dw, db = dev(x), dev(w), dev(b)  # keep device buffers alive across the launch
    _native.check(lib.nnx_conv3d_direct_small_cin(
        dx.data_ptr(), dw.data_ptr(), db.data_ptr(), y.data_ptr(), 2,
        _native.ints(size), cout, stream()))
    got = host(y)
    ref = _conv_ref64(x, w, (1, 1, 1)) + b
    assert rel_l2(got, ref) <= 1e-6, report("direct", got, ref)


@pytest.mark.parametrize("size,cout,amplitude,cin", [
    ((16, 16, 16), 32, 1.0, 1), ((5, 7, 9), 8, 1.0, 1), ((9, 20, 11), 12, 3e4, 1),
    ((4, 8, 8), 64, 1e-30, 1),
    # two channels: ragged tiles, and channel amplitudes 1 and 3e4 sharing one tile scale
    ((7, 9, 19), 32, (1.0, 3e4), 2), ((16, 16, 16), 32, 1.0, 2), ((3, 5, 33), 4, (3e4, 1e-3), 2),
    # four channels (two taps of four channels a K step, the last step padded), including
    # the 36..48-output and the >48-output builds
    ((16, 16, 16), 32, 1.0, 4), ((7, 9, 19), 48, (1.0, 3e4, 1e-3, 5.0), 4),
    ((5, 6, 17), 64, (2.0, 1.0, 1.0, 3e4), 4), ((3, 5, 33), 4, 1.0, 4)])
def test_direct_single_channel_conv_split(lib, size, cout, amplitude, cin):
    """Split products on MFMA hold the float32 bar of the split kernels at any input range
    (each tile scales its input by a power of two): raw CT-like magnitudes beyond the fp16
    range, tiny values, and tiles mixing both; with two or four input channels the channels
    of one tile share its scale."""
    print(f"direct split conv {size} {cout} {amplitude} cin={cin}", flush=True)
    rng = np.random.default_rng(11)
    amp = np.broadcast_to(np.asarray(amplitude, dtype=np.float64), (cin,))
    x = (rng.standard_normal((2, *size, cin)) * amp).astype(np.float32)
    x[0, : size[0] // 2] *= 1e-3  # tiles whose values span three decades
    w = (rng.standard_normal((cout, 3, 3, 3, cin)) * 0.3).astype(np.float32)
    w.reshape(-1)[::5] *= 1e-3
    b = (rng.standard_normal(cout) * amp.max() * 0.1).astype(np.float32)
    scale = lib.nnx_split_weight_scale(float(np.abs(w).max()))
    y = torch.full((2, *size, cout), float("nan"), dtype=torch.float32, device="cuda")
    dx, dw, db = dev(x), dev(w), dev(b)
    _native.check(lib.nnx_conv3d_direct_small_cin_split(
        dx.data_ptr(), cin, dw.data_ptr(), scale, db.data_ptr(), y.data_ptr(), 2,
        _native.ints(size), cout, stream()))
    got = host(y)
    ref = _conv_ref64(x, w, (1, 1, 1)) + b.astype(np.float64)
    msg = report("direct split", got, ref)
    assert np.isfinite(got).all(), msg
    assert rel_l2(got, ref) <= 1e-6, msg
    assert np.abs(got - ref).max() <= 1e-5 * np.abs(ref).max(), msg


def test_direct_split_conv_rejects_other_channel_counts(lib):
    """The split first convolution takes 1, 2 or 4 input channels; 3 is refused before any
    launch and the output keeps its contents."""
    x = torch.zeros((1, 8, 8, 8, 3), dtype=torch.float32, device="cuda")
    w = torch.zeros((32, 3, 3, 3, 3), dtype=torch.float32, device="cuda")
    y = torch.full((1, 8, 8, 8, 32), 7.0, dtype=torch.float32, device="cuda")
    rc = lib.nnx_conv3d_direct_small_cin_split(x.data_ptr(), 3, w.data_ptr(), 1.0, None,
                                               y.data_ptr(), 1, _native.ints((8, 8, 8)), 32,
                                               stream())
    assert rc == _native.NNX_ERR_INVALID
    assert "1, 2 or 4 input channels" in _native.last_error(), _native.last_error()
    torch.cuda.synchronize()
    assert bool((y == 7.0).all())


def _norm_ref64(x, in_bias, gamma, beta, eps, act, slope, residual):
    v = x.astype(np.float64)
    if in_bias is not None:
        v = v + in_bias
    axes = tuple(range(1, v.ndim - 1))
    mean = v.mean(axis=axes, keepdims=True)
    var = ((v - mean) ** 2).mean(axis=axes, keepdims=True)
    r = (v - mean) / np.sqrt(var + eps)
    if gamma is not None:
        r = r * gamma
    if beta is not None:
        r = r + beta
    if residual is not None:
        r = r + residual
    if act:
        r = np.maximum(slope * r, r)
    return r


NORM_CASES = [
    # batch, spatial, channels, affine, input_bias, act, residual
    (2, (16, 16, 16), 32, False, False, True, False),
    (1, (9, 11, 13), 32, True, True, True, False),
    (3, (4, 4, 4), 320, True, False, True, False),
    (1, (8, 8, 8), 64, True, True, False, True),
    (2, (5, 6, 7), 2, True, True, True, True),
    (1, (32, 32, 32), 128, False, True, True, False),
    # more than 16384 runs of 1024 vectors an item: workgroups loop over runs, the run's
    # first channel advancing by 64 modulo 320; a partial last run
    (1, (55, 61, 63), 320, True, False, True, True),
]


def _random_norm_cases(seed, n):
    """Seeded InstanceNorm shapes: channel counts with and without a 4-channel vector width,
    volumes from one voxel up, every combination of the optional parts."""
    rng = np.random.default_rng(seed)
    return [(int(rng.integers(1, 5)), tuple(int(v) for v in rng.integers(1, 24, 3)),
             int(rng.choice([int(rng.integers(1, 13)), 4 * int(rng.integers(1, 81))])),
             bool(rng.integers(0, 2)), bool(rng.integers(0, 2)), bool(rng.integers(0, 2)),
             bool(rng.integers(0, 2))) for _ in range(n)]


@pytest.mark.parametrize("case", NORM_CASES + _random_norm_cases(2029, 12), ids=str)
def test_instnorm_lrelu_matches_float64(lib, case):
    batch, spatial, c, affine, use_bias, act, use_res = case
    print(f"norm case {case}", flush=True)
    rng = np.random.default_rng(11)
    x = (rng.standard_normal((batch, *spatial, c)) * 3 + 1.5).astype(np.float32)
    in_bias = rng.standard_normal(c).astype(np.float32) if use_bias else None
    gamma = (1 + 0.2 * rng.standard_normal(c)).astype(np.float32) if affine else None
    beta = (0.3 * rng.standard_normal(c)).astype(np.float32) if affine else None
    res = rng.standard_normal(x.shape).astype(np.float32) if use_res else None
    S = int(np.prod(spatial))
    nbytes = lib.nnx_instnorm_workspace_bytes(batch, S, c)
    ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    dx = dev(x)
    y = torch.empty_like(dx)
    keep = [dev(a) if a is not None else None for a in (in_bias, gamma, beta, res)]
    ptrs = [k.data_ptr() if k is not None else None for k in keep]
    _native.check(lib.nnx_instnorm_lrelu(
        dx.data_ptr(), y.data_ptr(), batch, S, c, ptrs[0], ptrs[1], ptrs[2], 1e-5, int(act), 0.01,
        ptrs[3], ws.data_ptr(), nbytes, stream()))
    got = host(y)
    ref = _norm_ref64(x, in_bias, gamma, beta, 1e-5, act, 0.01, res)
    assert np.abs(got - ref).max() <= 2e-5, report("norm", got, ref)


def test_instnorm_in_place_and_constant_channel(lib):
    x = np.full((1, 6, 6, 6, 4), 0.1, dtype=np.float32)
    x[..., 1] = np.random.default_rng(0).standard_normal((1, 6, 6, 6))
    S = 216
    nbytes = lib.nnx_instnorm_workspace_bytes(1, S, 4)
    ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    dx = dev(x)
    _native.check(lib.nnx_instnorm_lrelu(dx.data_ptr(), dx.data_ptr(), 1, S, 4, None, None, None,
                                         1e-5, 1, 0.01, None, ws.data_ptr(), nbytes, stream()))
    got = host(dx)
    assert np.abs(got[..., 0]).max() < 1e-4  # variance clamped, output ~0
    ref = _norm_ref64(x, None, None, None, 1e-5, True, 0.01, None)
    assert np.abs(got[..., 1] - ref[..., 1]).max() < 2e-5


@pytest.mark.parametrize("case", [
    (2, (4, 4, 4), 64, 32, (2, 2, 2)),
    (1, (7, 5, 4), 320, 320, (1, 2, 2)),
    (1, (8, 8, 8), 128, 64, (2, 2, 2)),
    (1, (3, 5, 2), 6, 4, (2, 1, 2)),
], ids=str)
def test_tconv3d_gemm_matches_float64(lib, case):
    batch, size, cin, cout, k = case
    print(f"tconv case {case}", flush=True)
    rng = np.random.default_rng(3)
    x = rng.standard_normal((batch, *size, cin)).astype(np.float32)
    w = (rng.standard_normal((cout, *k, cin)) / np.sqrt(cin)).astype(np.float32)
    b = rng.standard_normal(cout).astype(np.float32)
    k_c = _native.ints(k)
    packed = torch.empty(lib.nnx_tconv3d_packed_floats(cout, k_c, cin), dtype=torch.float32, device="cuda")
    dx, dw, db = dev(x), dev(w), dev(b)
    _native.check(lib.nnx_tconv3d_pack_weight(dw.data_ptr(), cout, k_c, cin, packed.data_ptr(), stream()))
    out_size = [s * kk for s, kk in zip(size, k)]
    y = torch.full((batch, *out_size, cout), float("nan"), dtype=torch.float32, device="cuda")
    _native.check(lib.nnx_tconv3d_gemm(dx.data_ptr(), cin, packed.data_ptr(), db.data_ptr(),
                                       y.data_ptr(), batch, _native.ints(size), cout, k_c, stream()))
    got = host(y)
    xt = torch.from_numpy(x.astype(np.float64)).permute(0, 4, 1, 2, 3)
    wt = torch.from_numpy(w.astype(np.float64)).permute(4, 0, 1, 2, 3)
    ref = F.conv_transpose3d(xt, wt, torch.from_numpy(b.astype(np.float64)), stride=k)
    ref = ref.permute(0, 2, 3, 4, 1).numpy()
    assert np.isfinite(got).all()
    assert rel_l2(got, ref) <= 1e-6, report("tconv", got, ref)


@pytest.mark.parametrize("case", [
    (2, (4, 4, 4), 64, 32, (2, 2, 2)),
    (1, (7, 5, 4), 320, 320, (1, 2, 2)),
    (1, (8, 8, 8), 128, 64, (2, 2, 2)),
    (1, (3, 5, 2), 6, 4, (2, 1, 2)),
    (3, (5, 6, 7), 96, 24, (2, 2, 2)),
    # two row tiles a workgroup (the next one's lines requested during the current one)
    # and a partial last tile
    (2, (39, 41, 47), 64, 32, (2, 2, 2)),
], ids=str)
def test_tconv3d_split_matches_float64(lib, case):
    """Split-fp16 products hold the float32 bar (rel-L2 <= 1e-5) of the transposed conv."""
    _check_split_tconv(lib, case)


def _random_tconv_cases(seed, n):
    """Seeded transposed-convolution shapes: kernel = stride of 1 or 2 per axis, ragged
    input and output channel counts (scalar stores where C_out % 4 != 0)."""
    rng = np.random.default_rng(seed)
    return [(int(rng.integers(1, 4)), tuple(int(v) for v in rng.integers(1, 13, 3)),
             int(rng.integers(1, 97)), int(rng.integers(1, 65)),
             tuple(int(k) for k in rng.integers(1, 3, 3))) for _ in range(n)]


@pytest.mark.parametrize("case", _random_tconv_cases(2028, 10), ids=str)
def test_tconv3d_split_random_shapes_match_float64(lib, case):
    """The same bar over a seeded sweep of transposed-convolution shapes."""
    _check_split_tconv(lib, case)


def _check_split_tconv(lib, case):
    batch, size, cin, cout, k = case
    print(f"split tconv case {case}", flush=True)
    rng = np.random.default_rng(4)
    x = rng.standard_normal((batch, *size, cin)).astype(np.float32)
    w = (rng.standard_normal((cout, *k, cin)) / np.sqrt(cin)).astype(np.float32)
    w.reshape(-1)[::5] *= 1e-3
    b = rng.standard_normal(cout).astype(np.float32)
    k_c = _native.ints(k)
    scale = lib.nnx_split_weight_scale(float(np.abs(w).max()))
    packed = torch.empty(lib.nnx_tconv3d_split_packed_bytes(cout, k_c, cin), dtype=torch.uint8, device="cuda")
    dx, dw, db = dev(x), dev(w), dev(b)
    _native.check(lib.nnx_tconv3d_split_pack_weight(dw.data_ptr(), cout, k_c, cin, scale,
                                                    packed.data_ptr(), stream()))
    out_size = [s * kk for s, kk in zip(size, k)]
    y = torch.full((batch, *out_size, cout), float("nan"), dtype=torch.float32, device="cuda")
    _native.check(lib.nnx_tconv3d_split(dx.data_ptr(), cin, packed.data_ptr(), scale, db.data_ptr(),
                                        y.data_ptr(), batch, _native.ints(size), cout, k_c, stream()))
    got = host(y)
    xt = torch.from_numpy(x.astype(np.float64)).permute(0, 4, 1, 2, 3)
    wt = torch.from_numpy(w.astype(np.float64)).permute(4, 0, 1, 2, 3)
    ref = F.conv_transpose3d(xt, wt, torch.from_numpy(b.astype(np.float64)), stride=k)
    ref = ref.permute(0, 2, 3, 4, 1).numpy()
    msg = report("split tconv", got, ref)
    assert np.isfinite(got).all(), msg
    assert rel_l2(got, ref) <= 1e-5, msg
    assert np.abs(got - ref).max() <= 1e-4 * max(1.0, np.abs(ref).max()), msg


def _bf16(a: np.ndarray) -> np.ndarray:
    """Round to bf16 (nearest even), returned as float64."""
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(torch.bfloat16).double().numpy()


@pytest.mark.parametrize("case", CONV_CASES, ids=lambda c: f"b{c[0]}-{c[1]}-c{c[2]}+{c[3]}-o{c[4]}-k{c[5]}-s{c[6]}")
def test_conv3d_bf16_matches_rounded_float64(lib, case):
    """bf16 arithmetic: the float64 convolution of the bf16-rounded input and weights (each
    product is exact in float32) to float32 accumulation error, and the bf16 bar
    (relative L2 <= 1e-2) against the unrounded float64 convolution."""
    batch, size, c1, c2, cout, kernel, stride = case
    print(f"bf16 conv case {case}", flush=True)
    rng = np.random.default_rng((hash(case) + 11) % 2**32)
    x1 = rng.standard_normal((batch, *size, c1)).astype(np.float32)
    x2 = rng.standard_normal((batch, *size, c2)).astype(np.float32) if c2 else None
    w = (rng.standard_normal((cout, *kernel, c1 + c2)) / np.sqrt((c1 + c2) * np.prod(kernel))).astype(np.float32)
    bias = rng.standard_normal(cout).astype(np.float32)
    out_size = [(s + 2 * (k // 2) - k) // st + 1 for s, k, st in zip(size, kernel, stride)]
    k_c, s_c = _native.ints(kernel), _native.ints(stride)
    scale = lib.nnx_split_weight_scale(float(np.abs(w).max()))
    packed = torch.empty(lib.nnx_conv3d_split_packed_bytes(cout, k_c, c1, c2), dtype=torch.uint8, device="cuda")
    dw = dev(w)
    _native.check(lib.nnx_conv3d_bf16_pack_weight(dw.data_ptr(), cout, k_c, c1, c2, scale,
                                                  packed.data_ptr(), stream()))
    dx1 = dev(x1)
    dx2 = dev(x2) if c2 else None
    db = dev(bias)
    y = torch.full((batch, *out_size, cout), float("nan"), dtype=torch.float32, device="cuda")
    _native.check(lib.nnx_conv3d_bf16(
        dx1.data_ptr(), c1, dx2.data_ptr() if c2 else None, c2, packed.data_ptr(), scale,
        db.data_ptr(), y.data_ptr(), batch, _native.ints(size), cout, k_c, s_c, stream()))
    got = host(y)
    full = np.concatenate([x1, x2], axis=-1) if c2 else x1
    # scaling by a power of two commutes with the rounding: bf16(w * scale) / scale == bf16(w)
    ref_rounded = _conv_ref64(_bf16(full), _bf16(w), stride) + bias.astype(np.float64)
    ref = _conv_ref64(full, w, stride) + bias.astype(np.float64)
    msg = report("bf16 conv", got, ref_rounded)
    assert np.isfinite(got).all(), msg
    assert rel_l2(got, ref_rounded) <= 1e-5, msg
    assert rel_l2(got, ref) <= 1e-2, report("bf16 conv vs unrounded", got, ref)


@pytest.mark.parametrize("case", [
    (2, (4, 4, 4), 64, 32, (2, 2, 2)),
    (1, (7, 5, 4), 320, 320, (1, 2, 2)),
    (1, (3, 5, 2), 6, 4, (2, 1, 2)),
], ids=str)
def test_tconv3d_bf16_matches_rounded_float64(lib, case):
    batch, size, cin, cout, k = case
    print(f"bf16 tconv case {case}", flush=True)
    rng = np.random.default_rng(9)
    x = rng.standard_normal((batch, *size, cin)).astype(np.float32)
    w = (rng.standard_normal((cout, *k, cin)) / np.sqrt(cin)).astype(np.float32)
    b = rng.standard_normal(cout).astype(np.float32)
    k_c = _native.ints(k)
    scale = lib.nnx_split_weight_scale(float(np.abs(w).max()))
    packed = torch.empty(lib.nnx_tconv3d_split_packed_bytes(cout, k_c, cin), dtype=torch.uint8, device="cuda")
    dx, dw, db = dev(x), dev(w), dev(b)
    _native.check(lib.nnx_tconv3d_bf16_pack_weight(dw.data_ptr(), cout, k_c, cin, scale,
                                                   packed.data_ptr(), stream()))
    out_size = [s * kk for s, kk in zip(size, k)]
    y = torch.full((batch, *out_size, cout), float("nan"), dtype=torch.float32, device="cuda")
    _native.check(lib.nnx_tconv3d_bf16(dx.data_ptr(), cin, packed.data_ptr(), scale, db.data_ptr(),
                                       y.data_ptr(), batch, _native.ints(size), cout, k_c, stream()))
    got = host(y)

    def tconv64(xa, wa):
        xt = torch.from_numpy(xa).permute(0, 4, 1, 2, 3)
        wt = torch.from_numpy(wa).permute(4, 0, 1, 2, 3)
        r = F.conv_transpose3d(xt, wt, torch.from_numpy(b.astype(np.float64)), stride=k)
        return r.permute(0, 2, 3, 4, 1).numpy()

    ref_rounded = tconv64(_bf16(x), _bf16(w))
    ref = tconv64(x.astype(np.float64), w.astype(np.float64))
    msg = report("bf16 tconv", got, ref_rounded)
    assert np.isfinite(got).all(), msg
    assert rel_l2(got, ref_rounded) <= 1e-5, msg
    assert rel_l2(got, ref) <= 1e-2, report("bf16 tconv vs unrounded", got, ref)


def test_conv1x1_seg_head(lib):
    rng = np.random.default_rng(5)
    x = rng.standard_normal((2, 6, 7, 8, 32)).astype(np.float32)
    w = rng.standard_normal((3, 1, 1, 1, 32)).astype(np.float32)
    b = rng.standard_normal(3).astype(np.float32)
    y = torch.empty((2, 6, 7, 8, 3), dtype=torch.float32, device="cuda")
    dx, dw, db = dev(x), dev(w), dev(b)
    _native.check(lib.nnx_conv1x1(dx.data_ptr(), 32, dw.data_ptr(), db.data_ptr(),
                                  y.data_ptr(), 2 * 6 * 7 * 8, 3, stream()))
    ref = np.einsum("nzyxc,oc->nzyxo", x.astype(np.float64), w[:, 0, 0, 0, :].astype(np.float64)) + b
    assert rel_l2(host(y), ref) <= 1e-6


@pytest.mark.parametrize("channels,kernel,size", [
    (5, (2, 2, 2), (8, 6, 4)),        # one channel a thread
    (32, (2, 2, 2), (8, 12, 200)),    # 4-channel vectors, rows longer than a block
    (8, (2, 1, 1), (6, 5, 7)),        # anisotropic (the last ResEnc stage's stride)
])
def test_avgpool3d(lib, channels, kernel, size):
    rng = np.random.default_rng(6)
    x = rng.standard_normal((2, *size, channels)).astype(np.float32)
    out = [n // k for n, k in zip(size, kernel)]
    y = torch.full((2, *out, channels), float("nan"), dtype=torch.float32, device="cuda")
    dx = dev(x)
    _native.check(lib.nnx_avgpool3d(dx.data_ptr(), y.data_ptr(), 2, _native.ints(size), channels,
                                    _native.ints(kernel), stream()))
    ref = x.reshape(2, out[0], kernel[0], out[1], kernel[1], out[2], kernel[2],
                    channels).astype(np.float64).mean(axis=(2, 4, 6))
    assert np.abs(host(y) - ref).max() < 1e-6


# ---- sliding-window kernels: bitwise ------------------------------------------------

FLIPS_3AX = [0, 1, 2, 4, 3, 5, 6, 7]


def _unflip(view: np.ndarray, mask: int) -> np.ndarray:
    axes = tuple(a for a in range(3) if mask >> a & 1)
    return np.flip(view, axis=axes) if axes else view


# (channels, patch, output offset in floats): rows of a multiple of 4 floats into an aligned
# output take 16-byte runs; odd rows, a misaligned output and rows that do not fill the last
# workgroup take the single-float path or the row bound
GATHER_CASES = [
    (2, (12, 8, 10), 0),
    (3, (12, 11, 12), 0),
    (1, (12, 8, 7), 0),
    (2, (12, 8, 10), 1),
    (1, (5, 13, 200), 0),
]


@pytest.mark.parametrize("case", GATHER_CASES, ids=str)
def test_gather_flip_exact(lib, case):
    channels, patch, shift = case
    print(f"gather case {case}", flush=True)
    rng = np.random.default_rng(8)
    vol = rng.standard_normal((channels, 9, 11, 13)).astype(np.float32)
    pad = (2, 0, 1)
    offset = (0, 3, 4)
    after = [max(0, o + p - s - b) for o, p, s, b in zip(offset, patch, vol.shape[1:], pad)]
    padded = np.pad(vol, [(0, 0)] + [(b, a) for b, a in zip(pad, after)])
    n = 8 * int(np.prod(patch)) * channels
    buf = torch.full((n + shift,), float("nan"), dtype=torch.float32, device="cuda")
    dvol = dev(vol)
    _native.check(lib.nnx_sw_gather_flip(
        dvol.data_ptr(), channels, _native.i64s(vol.shape[1:]), _native.ints(pad),
        _native.ints(offset), _native.ints(patch), _native.ints(FLIPS_3AX), 8,
        buf.data_ptr() + 4 * shift, stream()))
    got = host(buf)[shift:].reshape(8, *patch, channels)
    sl = tuple(slice(o, o + p) for o, p in zip(offset, patch))
    tile = np.moveaxis(padded[(slice(None),) + sl], 0, -1)
    for v, mask in enumerate(FLIPS_3AX):
        np.testing.assert_array_equal(got[v], _unflip(tile, mask))


@pytest.mark.parametrize("seed", range(8))
def test_gather_flip_random_geometry_exact(lib, seed):
    """Seeded volumes, paddings, tile offsets, patches and view sets: every gathered view is
    the mirrored tile of the zero-padded volume, bit for bit."""
    rng = np.random.default_rng(300 + seed)
    channels = int(rng.integers(1, 5))
    size = tuple(int(v) for v in rng.integers(1, 16, 3))
    patch = tuple(int(v) for v in rng.integers(1, 20, 3))
    before = tuple(int(v) for v in rng.integers(0, 4, 3))
    padded = [max(s + b + int(rng.integers(0, 4)), p) for s, b, p in zip(size, before, patch)]
    offset = tuple(int(rng.integers(0, q - p + 1)) for q, p in zip(padded, patch))
    flips = [int(f) for f in rng.choice(8, int(rng.integers(1, 9)), replace=False)]
    print(f"gather seed {seed}: c {channels} size {size} patch {patch} before {before} "
          f"padded {padded} offset {offset} flips {flips}", flush=True)
    vol = rng.standard_normal((channels, *size)).astype(np.float32)
    after = [q - s - b for q, s, b in zip(padded, size, before)]
    full = np.pad(vol, [(0, 0)] + [(b, a) for b, a in zip(before, after)])
    n = len(flips) * int(np.prod(patch)) * channels
    buf = torch.full((n,), float("nan"), dtype=torch.float32, device="cuda")
    dvol = dev(vol)
    _native.check(lib.nnx_sw_gather_flip(
        dvol.data_ptr(), channels, _native.i64s(size), _native.ints(before), _native.ints(offset),
        _native.ints(patch), _native.ints(flips), len(flips), buf.data_ptr(), stream()))
    got = host(buf).reshape(len(flips), *patch, channels)
    sl = tuple(slice(o, o + p) for o, p in zip(offset, patch))
    tile = np.moveaxis(full[(slice(None),) + sl], 0, -1)
    for v, mask in enumerate(flips):
        np.testing.assert_array_equal(got[v], _unflip(tile, mask))


@pytest.mark.parametrize("fp16", [False, True])
def test_accumulate_fold_finalize_bitwise(lib, fp16):
    rng = np.random.default_rng(9)
    K, patch = 3, (6, 5, 4)
    padded = (10, 9, 7)
    g = rng.uniform(0.01, 1.0, patch).astype(np.float16 if fp16 else np.float32)
    acc = np.zeros((*padded, K), dtype=g.dtype)
    norm = np.zeros(padded, dtype=g.dtype)
    dacc, dnorm = dev(acc), dev(norm)
    dg = dev(g)
    offsets = [(0, 0, 0), (4, 4, 3), (2, 1, 0), (4, 0, 3)]
    accum = _native.NNX_ACCUM_NNUNET_F16 if fp16 else _native.NNX_ACCUM_F32
    for off in offsets:
        pred = (rng.standard_normal((8, *patch, K)) * 4).astype(np.float32)
        dpred = dev(pred)
        _native.check(lib.nnx_sw_accumulate(
            dpred.data_ptr(), 8, _native.ints(FLIPS_3AX), K, _native.ints(patch), dg.data_ptr(),
            _native.ints(off), _native.i64s(padded), accum, dacc.data_ptr(), dnorm.data_ptr(), stream()))
        s = pred[0]
        for v in range(1, 8):
            s = s + _unflip(pred[v], FLIPS_3AX[v])
        s = s / np.float32(8)
        sl = tuple(slice(o, o + p) for o, p in zip(off, patch))
        if fp16:
            acc[sl] = (acc[sl].astype(np.float32) + s * g.astype(np.float32)[..., None]).astype(np.float16)
            norm[sl] = norm[sl] + g
        else:
            acc[sl] += s * g[..., None]
            norm[sl] += g
    np.testing.assert_array_equal(host(dacc), acc)
    np.testing.assert_array_equal(host(dnorm), norm)
    # fold add (2 folds: the same accumulator twice) and finalize with crop
    crop_lo, crop = (1, 2, 1), (8, 6, 5)
    total = torch.empty((*crop, K), dtype=dacc.dtype, device="cuda")
    for first in (1, 0):
        _native.check(lib.nnx_sw_fold_add(dacc.data_ptr(), dnorm.data_ptr(), K, _native.i64s(padded),
                                          _native.ints(crop_lo), _native.i64s(crop), accum, first,
                                          total.data_ptr(), stream()))
    csl = tuple(slice(o, o + c) for o, c in zip(crop_lo, crop))
    dt = np.float16 if fp16 else np.float32
    with np.errstate(divide="ignore", invalid="ignore"):
        q = (acc.astype(np.float32) / norm.astype(np.float32)[..., None]).astype(dt)[csl]
    expected_total = (q + q).astype(dt)
    got_total = host(total)
    np.testing.assert_array_equal(got_total, expected_total)
    logits = torch.empty_like(total)
    labels = torch.empty(crop, dtype=torch.int16, device="cuda")
    invalid = torch.zeros(1, dtype=torch.int32, device="cuda")
    _native.check(lib.nnx_sw_fold_finalize(total.data_ptr(), K, int(np.prod(crop)), 2, accum,
                                           logits.data_ptr(), labels.data_ptr(), invalid.data_ptr(), stream()))
    avg = (expected_total.astype(np.float32) / np.float32(2)).astype(dt)
    np.testing.assert_array_equal(host(logits), avg)
    finite = np.isfinite(avg.astype(np.float32)).all(axis=-1)
    want = np.argmax(np.where(np.isfinite(avg), avg, -np.inf).astype(np.float32), axis=-1).astype(np.uint16)
    want[~finite] = 65535
    np.testing.assert_array_equal(host(labels).view(np.uint16), want)
    assert int(host(invalid)[0]) == int((~finite).sum())


@pytest.mark.parametrize("fp16", [False, True])
@pytest.mark.parametrize("seed", range(6))
def test_accumulate_fold_finalize_random_geometry_bitwise(lib, seed, fp16):
    """Seeded classes, patches, padded volumes, view sets, tile offsets, crops and fold counts:
    the accumulators, the fold total, the averaged logits and the labels equal the same
    float32 (or float16) operations in numpy, bit for bit (uncovered voxels give 0/0 and the
    invalid label)."""
    rng = np.random.default_rng(500 + seed)
    K = int(rng.integers(1, 6))
    patch = tuple(int(v) for v in rng.integers(1, 10, 3))
    padded = tuple(p + int(rng.integers(0, 6)) for p in patch)
    flips = [int(f) for f in rng.choice(8, int(rng.integers(1, 9)), replace=False)]
    offsets = [tuple(int(rng.integers(0, q - p + 1)) for q, p in zip(padded, patch))
               for _ in range(int(rng.integers(1, 6)))]
    crop_lo = tuple(int(rng.integers(0, q)) for q in padded)
    crop = tuple(int(rng.integers(1, q - lo + 1)) for q, lo in zip(padded, crop_lo))
    nfolds = int(rng.integers(1, 4))
    print(f"accumulate seed {seed} fp16 {fp16}: K {K} patch {patch} padded {padded} flips {flips} "
          f"offsets {offsets} crop {crop_lo}+{crop} folds {nfolds}", flush=True)
    dt = np.float16 if fp16 else np.float32
    accum = _native.NNX_ACCUM_NNUNET_F16 if fp16 else _native.NNX_ACCUM_F32
    g = rng.uniform(0.01, 1.0, patch).astype(dt)
    acc = np.zeros((*padded, K), dtype=dt)
    norm = np.zeros(padded, dtype=dt)
    dacc, dnorm, dg = dev(acc), dev(norm), dev(g)
    for off in offsets:
        pred = (rng.standard_normal((len(flips), *patch, K)) * 4).astype(np.float32)
        dpred = dev(pred)
        _native.check(lib.nnx_sw_accumulate(
            dpred.data_ptr(), len(flips), _native.ints(flips), K, _native.ints(patch), dg.data_ptr(),
            _native.ints(off), _native.i64s(padded), accum, dacc.data_ptr(), dnorm.data_ptr(),
            stream()))
        m = _unflip(pred[0], flips[0])
        for v in range(1, len(flips)):
            m = m + _unflip(pred[v], flips[v])
        if len(flips) > 1:
            m = m / np.float32(len(flips))
        sl = tuple(slice(o, o + p) for o, p in zip(off, patch))
        w = m * g.astype(np.float32)[..., None]
        acc[sl] = (acc[sl].astype(np.float32) + w).astype(dt)
        norm[sl] = (norm[sl].astype(np.float32) + g.astype(np.float32)).astype(dt)
    np.testing.assert_array_equal(host(dacc), acc)
    np.testing.assert_array_equal(host(dnorm), norm)
    total = torch.empty((*crop, K), dtype=dacc.dtype, device="cuda")
    csl = tuple(slice(o, o + c) for o, c in zip(crop_lo, crop))
    with np.errstate(divide="ignore", invalid="ignore"):
        q = (acc.astype(np.float32) / norm.astype(np.float32)[..., None]).astype(dt)[csl]
    expected = q
    for f in range(nfolds):
        _native.check(lib.nnx_sw_fold_add(dacc.data_ptr(), dnorm.data_ptr(), K, _native.i64s(padded),
                                          _native.ints(crop_lo), _native.i64s(crop), accum,
                                          int(f == 0), total.data_ptr(), stream()))
        if f:
            expected = (expected.astype(np.float32) + q.astype(np.float32)).astype(dt)
    np.testing.assert_array_equal(host(total), expected)
    logits = torch.empty_like(total)
    labels = torch.empty(crop, dtype=torch.int16, device="cuda")
    invalid = torch.zeros(1, dtype=torch.int32, device="cuda")
    _native.check(lib.nnx_sw_fold_finalize(total.data_ptr(), K, int(np.prod(crop)), nfolds, accum,
                                           logits.data_ptr(), labels.data_ptr(), invalid.data_ptr(),
                                           stream()))
    avg = expected if nfolds == 1 else \
        (expected.astype(np.float32) / np.float32(nfolds)).astype(dt)
    np.testing.assert_array_equal(host(logits), avg)
    finite = np.isfinite(avg.astype(np.float32)).all(axis=-1)
    want = np.argmax(np.where(np.isfinite(avg), avg, -np.inf).astype(np.float32), axis=-1)
    want = want.astype(np.uint16)
    want[~finite] = 65535
    np.testing.assert_array_equal(host(labels).view(np.uint16), want)
    assert int(host(invalid)[0]) == int((~finite).sum())


def test_finalize_ties_choose_earliest_and_flags_nonfinite(lib):
    total = np.array([[1.0, 1.0, 0.5], [0.2, 3.0, 3.0], [np.nan, 1.0, 2.0], [-np.inf, -1.0, -1.0]],
                     dtype=np.float32)
    labels = torch.empty(4, dtype=torch.int16, device="cuda")
    invalid = torch.zeros(1, dtype=torch.int32, device="cuda")
    dtotal = dev(total)
    _native.check(lib.nnx_sw_fold_finalize(dtotal.data_ptr(), 3, 4, 1, _native.NNX_ACCUM_F32, None,
                                           labels.data_ptr(), invalid.data_ptr(), stream()))
    np.testing.assert_array_equal(host(labels).view(np.uint16), [0, 1, 65535, 65535])
    assert int(host(invalid)[0]) == 2


def test_count_nonfinite(lib):
    x = np.zeros(100000, dtype=np.float32)
    x[[5, 77, 99999]] = [np.inf, np.nan, -np.inf]
    count = torch.empty(1, dtype=torch.int32, device="cuda")
    dx = dev(x)
    _native.check(lib.nnx_count_nonfinite(dx.data_ptr(), x.size, count.data_ptr(), stream()))
    assert int(host(count)[0]) == 3


def test_errors_are_reported(lib):
    from nnunet_mlx.errors import ContractError

    with pytest.raises(ContractError, match="odd"):
        _native.check(lib.nnx_conv3d_igemm(None, 1, None, 0, None, None, None, 1, _native.ints((4, 4, 4)), 4,
                                           _native.ints((2, 2, 2)), _native.ints((1, 1, 1)), stream()))
    assert lib.nnx_last_error()
