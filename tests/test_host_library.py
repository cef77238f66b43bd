"""CPU-only checks of the C-ABI library: it loads and exports every declared symbol."""

from __future__ import annotations

import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def _declared_symbols() -> set[str]:
    text = (ROOT / "include" / "nnx.h").read_text()
    return set(re.findall(r"\b(nnx_[a-z0-9_]+)\s*\(", text)) - {"nnx_forward_fn"}


def test_header_declarations_match_binding_table():
    from nnunet_mlx import _native

    assert _declared_symbols() == set(_native.EXPORTED_SYMBOLS)


def test_header_constants_match_the_binding():
    """Every NNX_* integer constant include/nnx.h defines has the same value in _native."""
    import re

    from nnunet_mlx import _native

    header = (Path(__file__).resolve().parents[1] / "include" / "nnx.h").read_text()
    defines = dict(re.findall(r"^#define (NNX_\w+) (-?\d+)\s*$", header, re.M))
    assert "NNX_PRECISION_BF16_MIXED" in defines
    for name, value in defines.items():
        assert getattr(_native, name) == int(value), name


def test_library_loads_and_exports_every_symbol():
    from nnunet_mlx import _native

    if not _native.library_path().is_file():
        pytest.fail("libnnunet_hip.so is not built; run __graft_entry__.build()")
    lib = _native.load()
    for name in _declared_symbols():
        assert getattr(lib, name) is not None, name
    assert b"gfx950" in lib.nnx_version()


def test_error_path_without_gpu():
    """Argument validation happens before any device call, so it works on a CPU host."""
    from nnunet_mlx import _native
    from nnunet_mlx.errors import ContractError

    lib = _native.load()
    rc = lib.nnx_conv3d_igemm(None, 1, None, 0, None, None, None, 1, _native.ints((4, 4, 4)), 4,
                              _native.ints((2, 2, 2)), _native.ints((1, 1, 1)), None)
    assert rc == _native.NNX_ERR_INVALID
    assert b"odd" in lib.nnx_last_error()
    with pytest.raises(ContractError):
        _native.check(rc)


def test_convolutions_refuse_items_beyond_32_bit_voxel_offsets():
    """The convolution kernels hold a voxel's offset inside its batch item in 32 bits: a
    batch item of 2^31 voxels or more is refused by every convolution entry point before
    any device call (so on a CPU host too); one voxel fewer passes that check (and fails
    the next one, the null buffers)."""
    from nnunet_mlx import _native

    lib = _native.load()
    k3, s1 = _native.ints((3, 3, 3)), _native.ints((1, 1, 1))
    calls = {
        "split": lambda size: lib.nnx_conv3d_split(None, 16, None, 0, None, 1.0, None, None, 1,
                                                   _native.ints(size), 32, k3, s1, None),
        "winograd": lambda size: lib.nnx_conv3d_winograd(None, 16, None, 0, None, 1.0, None, None,
                                                         1, _native.ints(size), 32, None),
        "igemm": lambda size: lib.nnx_conv3d_igemm(None, 16, None, 0, None, None, None, 1,
                                                   _native.ints(size), 32, k3, s1, None),
    }
    for name, call in calls.items():
        assert call((2048, 1024, 1024)) == _native.NNX_ERR_INVALID, name
        assert b"2^31 voxels" in lib.nnx_last_error(), name
        assert call((2047, 1024, 1024)) == _native.NNX_ERR_INVALID, name
        assert b"2^31 voxels" not in lib.nnx_last_error(), name


def test_instnorm_workspace_query_refuses_what_the_normalisation_refuses():
    """The workspace-size query answers 0 (instead of trapping on a division by a zero channel
    group count) for empty tensors and for the sizes the normalisation itself refuses."""
    from nnunet_mlx import _native

    lib = _native.load()
    assert lib.nnx_instnorm_workspace_bytes(2, 24 ** 3, 32) > 0
    for batch, spatial, channels in ((1, 10, 0), (0, 10, 4), (1, 0, 4), (-1, 10, 4), (1, -5, 4),
                                     (1, 10, -4), (65536, 10, 4), (1, 10, 1025)):
        assert lib.nnx_instnorm_workspace_bytes(batch, spatial, channels) == 0, (batch, spatial,
                                                                                channels)


def test_split_weight_scale_rules():
    """The split-fp16 weight scale is the power of two that puts max |w| in [2^14, 2^15)."""
    from nnunet_mlx import _native

    lib = _native.load()
    assert lib.nnx_split_weight_scale(0.0) == 1.0
    assert lib.nnx_split_weight_scale(1.0) == 2.0**14
    assert lib.nnx_split_weight_scale(0.75) == 2.0**15
    assert lib.nnx_split_weight_scale(6e4) == 0.5
    assert lib.nnx_split_weight_scale(2.0**-30) == 2.0**44
    assert lib.nnx_split_weight_scale(float("nan")) == 0.0
    assert lib.nnx_split_weight_scale(float("inf")) == 0.0
    assert lib.nnx_split_weight_scale(-1.0) == 0.0
    for m in (1e-4, 0.0123, 0.5, 3.0, 1000.0):
        s = lib.nnx_split_weight_scale(m)
        assert 2.0**14 <= m * s < 2.0**15
    # below 2^-113 the power of two would overflow float32: it stops at 2^127
    assert lib.nnx_split_weight_scale(2.0**-113) == 2.0**127
    assert lib.nnx_split_weight_scale(2.0**-114) == 2.0**127
    assert lib.nnx_split_weight_scale(1e-40) == 2.0**127


def test_winograd_weight_scale_rules():
    """The Winograd scale bounds the transformed weights (|U| <= 3.375 max |w|) the same way,
    and answers for every finite magnitude, including those whose bound overflows float32
    (it never throws across the C ABI)."""
    import numpy as np

    from nnunet_mlx import _native

    lib = _native.load()
    for m in (1e-4, 0.0123, 0.5, 3.0, 1000.0, 1e30, 1e38, float(np.finfo(np.float32).max)):
        s = lib.nnx_winograd_weight_scale(m)
        assert s > 0.0 and np.log2(s) == int(np.log2(s)), m
        assert 2.0**14 <= 3.375 * m * s < 2.0**15, m
    for bad in (float("nan"), float("inf"), -1.0):
        assert lib.nnx_winograd_weight_scale(bad) == 0.0
    assert lib.nnx_winograd_weight_scale(0.0) == 1.0


def test_model_create_bounds_every_spec_field():
    """nnx_model_create builds the graph on the host (no device call) and refuses a spec
    field outside its documented range before building anything."""
    import ctypes

    from nnunet_mlx import _native

    lib = _native.load()
    keep = []

    def spec(**over):
        S = over.pop("stages", 4)
        fields = dict(features=[32, 64, 128, 256][:S] + [256] * max(0, S - 4),
                      kernel_sizes=[3] * (3 * S), strides=[1, 1, 1] + [2] * (3 * (S - 1)),
                      encoder_convs=[2] * S, decoder_convs=[2] * (S - 1))
        fields.update({k: v for k, v in over.items() if k in fields})
        s = _native.NnxSpec()
        s.arch, s.spatial_dims = _native.NNX_ARCH_PLAIN, 3
        s.input_channels, s.num_classes, s.n_stages = over.get("cin", 1), over.get("classes", 3), S
        for name, values in fields.items():
            array = _native.ints(values)
            keep.append(array)
            setattr(s, name, ctypes.cast(array, _native.c_int_p))
        s.conv_bias, s.norm_affine, s.norm_eps, s.leaky_slope = 1, 1, 1e-5, 0.01
        s.precision = _native.NNX_PRECISION_FP32_SPLIT
        return s

    def create(s):
        handle = ctypes.c_void_p()
        rc = lib.nnx_model_create(ctypes.byref(s), ctypes.byref(handle))
        if handle.value:
            lib.nnx_model_destroy(handle)
        return rc

    assert create(spec()) == _native.NNX_OK
    assert create(spec(stages=16)) == _native.NNX_OK
    for bad in (dict(stages=17), dict(cin=1025), dict(classes=1025),
                dict(features=[32, 64, 128, 1025]), dict(kernel_sizes=[3] * 11 + [17]),
                dict(strides=[1] * 11 + [17]), dict(encoder_convs=[2, 2, 2, 65]),
                dict(decoder_convs=[2, 65, 2]), dict(stages=1 << 30, features=[32] * 4)):
        if bad.get("stages", 0) == 1 << 30:
            # the count alone is refused: the arrays are never read past their 4 entries
            s = spec()
            s.n_stages = 1 << 30
        else:
            s = spec(**bad)
        assert create(s) == _native.NNX_ERR_INVALID, bad


def test_sliding_window_config_limits_are_checked_before_any_device_call():
    """Sizes whose buffer byte counts would wrap, offsets whose sum with the patch would
    overflow 32 bits and a null config are refused while validating, on any host."""
    import ctypes

    from nnunet_mlx import _native

    lib = _native.load()
    keep = []

    def config(size=(4, 4, 4), padded=(4, 4, 4), patch=(4, 4, 4), offset=(0, 0, 0), classes=3):
        c = _native.NnxSwConfig()
        c.channels, c.num_classes = 1, classes
        c.size[:], c.pad_before[:], c.padded[:], c.patch[:] = size, (0, 0, 0), padded, patch
        offsets, flips = _native.ints(offset), _native.ints((0,))
        keep.extend((offsets, flips))
        c.ntiles, c.tile_offsets = 1, ctypes.cast(offsets, _native.c_int_p)
        c.nviews, c.view_flips = 1, ctypes.cast(flips, _native.c_int_p)
        c.accumulation, c.d_gaussian, c.tiles_per_batch = _native.NNX_ACCUM_F32, 4096, 1
        return c

    fns = (_native.FORWARD_FN * 1)(_native.FORWARD_FN())
    users = (ctypes.c_void_p * 1)(None)

    def run(c):
        return lib.nnx_sw_predict_custom(fns, users, 1, ctypes.byref(c), 4096, None, None, None)

    big = (65535, 65535, (1 << 31) - 1)
    for c, words in ((config(padded=big, patch=big), b"too large"),
                     (config(padded=(1 << 31, 4, 4)), b"2^31 - 1"),
                     (config(patch=(2, 2, 2), offset=((1 << 31) - 1, 0, 0)), b"tile offset"),
                     (config(classes=65536), b"65535")):
        assert run(c) == _native.NNX_ERR_INVALID
        assert words in lib.nnx_last_error(), lib.nnx_last_error()
    folds = (ctypes.c_void_p * 1)(None)
    assert lib.nnx_sw_predict(folds, 1, None, None, None, None, None) == _native.NNX_ERR_INVALID
    assert b"config must not be null" in lib.nnx_last_error()


def test_box_checks_do_not_wrap():
    """A box start near 2^63 whose sum with the extent would wrap negative is refused (the
    checks compare the extent with what is left of the axis instead of adding)."""
    import ctypes

    from nnunet_mlx import _native

    lib = _native.load()

    def i64(values):
        return (ctypes.c_int64 * len(values))(*values)

    size, far, one = i64((4, 4, 4)), i64(((1 << 63) - 1, 0, 0)), i64((1, 1, 1))
    fake = 4096  # never dereferenced: the box check fails first
    assert lib.nnx_zscore_stats(fake, 1, size, 0, far, one, None, fake, fake, None) == \
        _native.NNX_ERR_INVALID
    assert b"outside the volume" in lib.nnx_last_error()
    assert lib.nnx_channel_minmax(fake, 1, size, 0, far, one, fake, fake, None) == \
        _native.NNX_ERR_INVALID
    assert lib.nnx_nonzero_mask_filled(fake, 1, size, far, one, fake, fake, None) == \
        _native.NNX_ERR_INVALID
    crop_lo = _native.ints((1, 0, 0))
    huge = i64(((1 << 63) - 1, 1, 1))
    assert lib.nnx_sw_fold_add(fake, fake, 3, size, crop_lo, huge, _native.NNX_ACCUM_F32, 1, fake,
                               None) == _native.NNX_ERR_INVALID
    assert b"crop outside the volume" in lib.nnx_last_error()


def test_finalize_failed_part_way_leaves_the_model_refusing_retries():
    """A finalize that fails for missing parameters can be repeated; one that fails while
    uploading (here: no device on a CPU host, or any device error) releases host copies as
    it goes, so a retry is refused instead of reading the released copies."""
    import ctypes

    import numpy as np

    from nnunet_mlx import _native

    lib = _native.load()
    keep = []
    s = _native.NnxSpec()
    s.arch, s.spatial_dims, s.input_channels, s.num_classes, s.n_stages = (
        _native.NNX_ARCH_PLAIN, 3, 1, 2, 2)
    for name, values in dict(features=[4, 8], kernel_sizes=[3] * 6, strides=[1, 1, 1, 2, 2, 2],
                             encoder_convs=[1, 1], decoder_convs=[1]).items():
        array = _native.ints(values)
        keep.append(array)
        setattr(s, name, ctypes.cast(array, _native.c_int_p))
    s.conv_bias, s.norm_affine, s.norm_eps, s.leaky_slope = 1, 1, 1e-5, 0.01
    s.precision = _native.NNX_PRECISION_FP32_SPLIT
    handle = ctypes.c_void_p()
    _native.check(lib.nnx_model_create(ctypes.byref(s), ctypes.byref(handle)))
    try:
        count = ctypes.c_int()
        _native.check(lib.nnx_model_param_count(handle, ctypes.byref(count)))
        assert lib.nnx_model_finalize(handle) == _native.NNX_ERR_STATE  # nothing loaded yet
        for i in range(count.value):
            name, ndim = ctypes.c_char_p(), ctypes.c_int()
            shape = (ctypes.c_int64 * 5)()
            _native.check(lib.nnx_model_param_info(handle, i, ctypes.byref(name), ctypes.byref(ndim),
                                                   shape))
            dims = tuple(shape[:ndim.value])
            data = np.full(dims, 0.5, dtype=np.float32)
            _native.check(lib.nnx_model_load_param(handle, name.value, data.ctypes.data,
                                                   _native.i64s(dims), ndim.value))
        first = lib.nnx_model_finalize(handle)
        if first == _native.NNX_OK:
            pytest.skip("a device is present: the upload did not fail")
        assert lib.nnx_model_finalize(handle) == _native.NNX_ERR_INVALID
        assert b"failed part-way" in lib.nnx_last_error()
    finally:
        lib.nnx_model_destroy(handle)
