"""The allocation-free InstanceNorm entry (nnx_instnorm_lrelu_noalloc) against the
workspace entry it varies (nnx_instnorm_lrelu): bit-identical outputs (the same kernels on
the same inputs), on two calls in a row with the second smaller, so the second call runs on
the scratch the first one left behind; sizes beyond the scratch are refused with an error
and launch nothing."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from nnunet_mlx import _native
from tests.helpers import dev, host, stream

pytestmark = pytest.mark.gpu


def _call_pair(lib, batch, spatial, channels, seed, bias, affine, act, residual):
    rng = np.random.default_rng(seed)
    S = int(np.prod(spatial))
    x = (rng.standard_normal((batch, S, channels)) * 3 + 1).astype(np.float32)
    b = rng.standard_normal(channels).astype(np.float32) if bias else None
    g = rng.uniform(0.5, 2, channels).astype(np.float32) if affine else None
    be = rng.standard_normal(channels).astype(np.float32) if affine else None
    r = rng.standard_normal((batch, S, channels)).astype(np.float32) if residual else None
    dx = dev(x)
    db, dg, dbe, dr = (dev(a) if a is not None else None for a in (b, g, be, r))
    ptr = lambda t: None if t is None else t.data_ptr()  # noqa: E731
    ws_bytes = lib.nnx_instnorm_workspace_bytes(batch, S, channels)
    assert 0 < ws_bytes <= lib.nnx_instnorm_noalloc_max_bytes()
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda")
    want = torch.full_like(dx, float("nan"))
    got = torch.full_like(dx, float("nan"))
    _native.check(lib.nnx_instnorm_lrelu(dx.data_ptr(), want.data_ptr(), batch, S, channels,
                                         ptr(db), ptr(dg), ptr(dbe), 1e-5, int(act), 0.01, ptr(dr),
                                         ws.data_ptr(), ws_bytes, stream()))
    _native.check(lib.nnx_instnorm_lrelu_noalloc(dx.data_ptr(), got.data_ptr(), batch, S, channels,
                                                 ptr(db), ptr(dg), ptr(dbe), 1e-5, int(act), 0.01,
                                                 ptr(dr), stream()))
    a, e = host(got), host(want)
    assert np.isfinite(e).all()
    np.testing.assert_array_equal(a, e)


def test_noalloc_instnorm_equals_workspace_entry(lib):
    print("no-alloc instnorm: batch 2, 24^3, 32 channels, then batch 1, 9x11x13, 12 channels",
          flush=True)
    _call_pair(lib, 2, (24, 24, 24), 32, 1, bias=True, affine=True, act=True, residual=False)
    _call_pair(lib, 1, (9, 11, 13), 12, 2, bias=False, affine=True, act=False, residual=True)


def test_noalloc_instnorm_rejects_sizes_beyond_the_scratch(lib):
    limit = lib.nnx_instnorm_noalloc_max_bytes()
    assert limit == 16 << 20
    batch, S, C = 64, 128 ** 3, 32
    assert lib.nnx_instnorm_workspace_bytes(batch, S, C) > limit
    x = torch.zeros(1, device="cuda")  # never read: the size check fails first
    rc = lib.nnx_instnorm_lrelu_noalloc(x.data_ptr(), x.data_ptr(), batch, S, C, None, None, None,
                                        1e-5, 1, 0.01, None, stream())
    assert rc == _native.NNX_ERR_INVALID
    assert b"scratch" in lib.nnx_last_error()
