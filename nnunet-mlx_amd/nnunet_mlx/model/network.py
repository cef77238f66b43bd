"""nnU-Net v2 PlainConvUNet and ResidualEncoderUNet running on the MI355X HIP path.

Same module names, parameter names and tensor layouts as the reference's
``nnunet_mlx.model.network`` (src/nnunet_mlx/model/network.py:413-732): channels-last
activations (B, D, H, W, C), convolution weights (C_out, kD, kH, kW, C_in), parameter
keys ``enc{i}.block{j}.conv.weight``, ``up{d}.weight``, ``seg{d}.bias``,
``res{s}.block{b}.conv1.norm.weight``, ...  Each instance owns one native model
(``nnx_model``) whose graph, weights and workspace live in libnnunet_hip.so; calling it
runs the whole forward on the GPU and returns only the highest-resolution logits
(upstream's ``deep_supervision=False``).
"""

from __future__ import annotations

import ctypes
from collections.abc import Mapping

import numpy as np
import torch

from nnunet_mlx import _native
from nnunet_mlx.errors import ContractError
from nnunet_mlx.model.topology import NetworkSpec, PlainConvUNetSpec, ResidualEncoderUNetSpec


# Convolution arithmetic of the HIP network.  "fp32" and "fp32-split" meet the float32
# logits tolerance (max-abs <= 1e-3, relative L2 <= 1e-5 against the float32 oracle):
# "fp32" multiplies in float32 on fp32 MFMA; "fp32-split" (the default, ~2.5x faster
# convolutions) computes the 3-D convolutions as hi*hi + hi*lo + lo*hi of fp16-split
# operands with float32 accumulation (a first convolution with 1, 2 or 4 input channels scales
# each input tile by a power of two before the split; other first convolutions keep float32
# products).  "bf16" rounds the hidden 3-D convolutions' (and the transposed convolutions')
# weights and inputs to bf16 and multiplies once, with float32 accumulation and float32 norm
# statistics; on random-init networks its logits land at relative L2 1.0e-2 to 2.3e-2 of the
# float32 logits (the bf16 rounding itself, emulated on the CPU, lands at the same distance),
# so relative L2 <= 1e-2 is not met in general.  "bf16-mixed" runs bf16 below full resolution
# and fp32-split at full resolution (the first encoder stage, the last decoder stage and the
# transposed convolution into it): on the pancreas ResEnc-L two thirds of the convolution
# FLOPs in bf16, logits at relative L2 7.6e-3 of the float32 logits.
PRECISIONS = {
    "fp32": _native.NNX_PRECISION_FP32,
    "fp32-split": _native.NNX_PRECISION_FP32_SPLIT,
    "bf16": _native.NNX_PRECISION_BF16,
    "bf16-mixed": _native.NNX_PRECISION_BF16_MIXED,
}
DEFAULT_PRECISION = "fp32-split"


def _spec_struct(spec: NetworkSpec, keep: list, precision: str = DEFAULT_PRECISION) -> _native.NnxSpec:
    residual = isinstance(spec, ResidualEncoderUNetSpec)
    if spec.spatial_dims != 3:
        raise ContractError("only three-dimensional networks run on the HIP path")
    stages = len(spec.features)
    arrays = {
        "features": _native.ints(spec.features),
        "kernel_sizes": _native.ints([v for row in spec.kernel_sizes for v in row]),
        "strides": _native.ints([v for row in spec.strides for v in row]),
        "encoder_convs": _native.ints(spec.encoder_blocks if residual else spec.encoder_convs),
        "decoder_convs": _native.ints(spec.decoder_convs),
    }
    bottleneck = None
    if residual and spec.bottleneck_channels is not None:
        bottleneck = _native.ints(spec.bottleneck_channels)
    keep.extend(arrays.values())
    keep.append(bottleneck)
    s = _native.NnxSpec()
    s.arch = _native.NNX_ARCH_RESIDUAL if residual else _native.NNX_ARCH_PLAIN
    s.spatial_dims = 3
    s.input_channels = spec.input_channels
    s.num_classes = spec.num_classes
    s.n_stages = stages
    for name, array in arrays.items():
        setattr(s, name, ctypes.cast(array, _native.c_int_p))
    s.conv_bias = int(spec.conv_bias)
    s.norm_affine = int(spec.norm_affine)
    s.norm_eps = float(spec.norm_eps)
    s.leaky_slope = float(spec.leaky_slope)
    s.stem_channels = int(spec.stem_channels or 0) if residual else 0
    s.bottleneck_channels = ctypes.cast(bottleneck, _native.c_int_p) if bottleneck is not None else None
    if precision not in PRECISIONS:
        raise ContractError(f"unsupported precision {precision!r}; expected one of {sorted(PRECISIONS)}")
    s.precision = PRECISIONS[precision]
    return s


class NativeNetwork:
    """Shared implementation of the two architectures (one ``nnx_model`` each)."""

    def __init__(self, spec: NetworkSpec, *, precision: str = DEFAULT_PRECISION) -> None:
        self.spec = spec
        self.training = False
        self.inference_arithmetic = "native"
        self.precision = precision
        self._lib = _native.load()
        keep: list = []
        struct = _spec_struct(spec, keep, precision)
        handle = ctypes.c_void_p()
        _native.check(self._lib.nnx_model_create(ctypes.byref(struct), ctypes.byref(handle)),
                      "nnx_model_create")
        self._handle = handle
        self._finalized = False

    # -- parameters ------------------------------------------------------------------
    @property
    def handle(self) -> ctypes.c_void_p:
        return self._handle

    def parameter_shapes(self) -> dict[str, tuple[int, ...]]:
        """Reference parameter names and MLX-layout shapes the network expects."""
        count = ctypes.c_int()
        _native.check(self._lib.nnx_model_param_count(self._handle, ctypes.byref(count)))
        shapes: dict[str, tuple[int, ...]] = {}
        for index in range(count.value):
            name = ctypes.c_char_p()
            ndim = ctypes.c_int()
            shape = (ctypes.c_int64 * 5)()
            _native.check(self._lib.nnx_model_param_info(
                self._handle, index, ctypes.byref(name), ctypes.byref(ndim), shape))
            shapes[name.value.decode()] = tuple(int(shape[i]) for i in range(ndim.value))
        return shapes

    def load_weights(self, weights: Mapping[str, np.ndarray], *, strict: bool = True) -> None:
        """Load float32 weights strictly by reference name, then repack them on the GPU.

        Mirrors ``Module.load_weights(strict=True)`` as used by
        load_inference_checkpoint (src/nnunet_mlx/storage/checkpoint.py:232-237):
        unexpected or missing keys and non-finite tensors raise ``ContractError``.
        """
        if self._finalized:
            raise ContractError("weights are already loaded")
        expected = self.parameter_shapes()
        provided = set(weights)
        missing = sorted(set(expected) - provided)
        unexpected = sorted(provided - set(expected))
        if strict and (missing or unexpected):
            raise ContractError(
                f"checkpoint parameters do not match the network: missing {missing[:8]}, "
                f"unexpected {unexpected[:8]}"
            )
        for name in expected:
            array = np.ascontiguousarray(np.asarray(weights[name]), dtype=np.float32)
            if tuple(array.shape) != expected[name]:
                raise ContractError(
                    f"parameter {name} has shape {array.shape}, expected {expected[name]}"
                )
            shape = _native.i64s(array.shape)
            _native.check(self._lib.nnx_model_load_param(
                self._handle, name.encode(), array.ctypes.data, shape, array.ndim), name)
        _native.check(self._lib.nnx_model_finalize(self._handle), "nnx_model_finalize")
        self._finalized = True

    def share_workspace(self, owner: NativeNetwork) -> None:
        """Use ``owner``'s activation buffers (folds run one at a time)."""
        _native.check(self._lib.nnx_model_share_workspace(self._handle, owner.handle))

    # -- forward -----------------------------------------------------------------------
    def forward_into(self, tiles: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
        """Run (n, D, H, W, C_in) device tiles into a preallocated (n, D, H, W, K) tensor."""
        if not self._finalized:
            raise ContractError("load_weights must be called before inference")
        if tiles.dtype != torch.float32 or tiles.ndim != 5:
            raise ContractError("network input must be float32 (n, D, H, W, C) channels-last")
        if tiles.shape[-1] != self.spec.input_channels:
            raise ContractError(
                f"network expects {self.spec.input_channels} input channels, got {tiles.shape[-1]}"
            )
        expected = (*tiles.shape[:-1], self.spec.num_classes)
        if tuple(out.shape) != expected or out.dtype != torch.float32:
            raise ContractError(f"output buffer must be float32 {expected}")
        spatial = _native.ints(tiles.shape[1:4])
        with torch.cuda.device(tiles.device):
            _native.check(self._lib.nnx_forward(
                self._handle, _native.ptr(tiles), _native.ptr(out), int(tiles.shape[0]), spatial,
                _native.stream_handle(tiles.device)), "nnx_forward")
        return out

    def __call__(self, values: torch.Tensor | np.ndarray) -> torch.Tensor:
        """Channels-last float32 tiles -> float32 logits on the same device."""
        if isinstance(values, np.ndarray):
            if values.dtype != np.float32:
                raise ContractError("network input must be float32")
            values = torch.from_numpy(np.ascontiguousarray(values)).cuda()
        tiles = values.contiguous()
        out = torch.empty((*tiles.shape[:-1], self.spec.num_classes), dtype=torch.float32,
                          device=tiles.device)
        self.forward_into(tiles, out)
        # non-finite logits from finite inputs and weights: name the layer where they arose
        count = torch.empty(1, dtype=torch.int32, device=tiles.device)
        _native.check(self._lib.nnx_count_nonfinite(
            _native.ptr(out), out.numel(), _native.ptr(count),
            _native.stream_handle(tiles.device)), "nnx_count_nonfinite")
        if int(count.item()) != 0:
            _native.name_nonfinite_layer(
                ContractError("the network forward produced non-finite logits"),
                lambda: self.forward_into(tiles, torch.empty_like(out)))
        return out

    def eval(self) -> NativeNetwork:
        return self

    def close(self) -> None:
        handle, self._handle = getattr(self, "_handle", None), None
        if handle is not None and handle.value:
            self._lib.nnx_model_destroy(handle)

    def __del__(self) -> None:
        try:
            self.close()
        except Exception:
            pass


class PlainConvUNet(NativeNetwork):
    """Plan-driven PlainConvUNet (dynamic-network-architectures v0.4.4 semantics)."""

    def __init__(self, spec: PlainConvUNetSpec, *, precision: str = DEFAULT_PRECISION) -> None:
        if not isinstance(spec, PlainConvUNetSpec):
            raise ContractError("PlainConvUNet needs a PlainConvUNetSpec")
        super().__init__(spec, precision=precision)


class ResidualEncoderUNet(NativeNetwork):
    """nnU-Net ResidualEncoderUNet: residual stem and stages, plain decoder."""

    def __init__(self, spec: ResidualEncoderUNetSpec, *, precision: str = DEFAULT_PRECISION) -> None:
        if not isinstance(spec, ResidualEncoderUNetSpec):
            raise ContractError("ResidualEncoderUNet needs a ResidualEncoderUNetSpec")
        super().__init__(spec, precision=precision)


def build_network(spec: NetworkSpec, *, precision: str = DEFAULT_PRECISION) -> NativeNetwork:
    if isinstance(spec, ResidualEncoderUNetSpec):
        return ResidualEncoderUNet(spec, precision=precision)
    return PlainConvUNet(spec, precision=precision)
