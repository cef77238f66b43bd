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
