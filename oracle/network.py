"""Oracle network: torch-CPU float32 restatement of the reference's nnU-Net modules.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Follows, module by module:
  * ConvNorm / ConvNormAct: src/nnunet_mlx/model/network.py:177-356 — convolution with
    padding k//2 and *no* bias, then instance normalisation of (conv + bias), then
    LeakyReLU ``max(slope*r, r)``.
  * instance_norm: src/nnunet_mlx/kernels/metal_native_norm.py:92-168 — provisional mean
    m0 = sum(x)/S, centred sums D = sum(x-m0)/S and Q = sum((x-m0)^2)/S, mean = m0 + D,
    var = max(Q - D*D, 0), scale = gamma * rsqrt(var + eps), r = fma(x - mean, scale, beta).
  * NonOverlappingConvTranspose3d: src/nnunet_mlx/model/network.py:101-174 — stride ==
    kernel transposed convolution, + bias.
  * decoder: src/nnunet_mlx/model/network.py:771-877 — up{d}, concat((up, skip)),
    dec{d} blocks, only seg{n-1} applied (1x1x1 conv with bias).
  * residual encoder: src/nnunet_mlx/model/network.py:467-732 — stem ConvNormAct, per
    block conv1 (stride) ConvNormAct, conv2 ConvNorm, skip = AvgPool(stride) then 1x1
    ConvNorm (no bias) when channels change, out = leaky_relu(h + skip).

Pinned by tests/test_oracle_network.py against: float64 brute-force convolution and
transposed convolution on tiny shapes, torch.nn.functional.instance_norm (textbook),
the constant-channel and slope 0/1 special cases, and the reference's own parameter
naming (src/nnunet_mlx/storage/weights.py:48-123).
"""

from __future__ import annotations

from collections.abc import Mapping
from typing import Any

import numpy as np
import torch
import torch.nn.functional as F

Weights = Mapping[str, np.ndarray]


def _t(array: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(array, dtype=np.float32))


def conv_weight_to_torch(weight: np.ndarray) -> torch.Tensor:
    """(C_out, kD, kH, kW, C_in) -> torch (C_out, C_in, kD, kH, kW)."""
    return _t(weight).permute(0, 4, 1, 2, 3).contiguous()


def tconv_weight_to_torch(weight: np.ndarray) -> torch.Tensor:
    """(C_out, kD, kH, kW, C_in) -> torch ConvTranspose (C_in, C_out, kD, kH, kW)."""
    return _t(weight).permute(4, 0, 1, 2, 3).contiguous()


def round_bf16(x: torch.Tensor) -> torch.Tensor:
    """float32 -> nearest bf16 (ties to even) -> float32 (torch's bfloat16 cast)."""
    return x.to(torch.bfloat16).to(torch.float32)


def instance_norm(
    values: torch.Tensor,
    gamma: torch.Tensor | None,
    beta: torch.Tensor | None,
    eps: float,
    *,
    input_bias: torch.Tensor | None = None,
    negative_slope: float | None = None,
    residual: torch.Tensor | None = None,
) -> torch.Tensor:
    """Instance norm of NCDHW float32 ``values`` following metal_native_norm.py:92-168.

    ``residual`` (NCDHW) is added after the affine step and before the activation, as
    ResidualBlock.__call__ does (network.py:511-516).
    """
    x = values if input_bias is None else values + input_bias.view(1, -1, 1, 1, 1)
    dims = tuple(range(2, x.ndim))
    spatial = float(np.prod(x.shape[2:]))
    provisional = x.sum(dim=dims) / spatial
    centered = x - provisional.view(*provisional.shape, 1, 1, 1)
    correction = centered.sum(dim=dims) / spatial
    squares = (centered * centered).sum(dim=dims) / spatial
    mean = provisional + correction
    variance = torch.clamp(squares - correction * correction, min=0.0)
    scale = torch.rsqrt(variance + np.float32(eps))
    if gamma is not None:
        scale = gamma.view(1, -1) * scale
    shift = torch.zeros_like(scale[0]) if beta is None else beta
    # r = fma(x - mean, scale, shift): the float64 product of two float32 values is
    # exact, so one float64 addition then a float32 rounding restates the fused op.
    diff = (x - mean.view(*mean.shape, 1, 1, 1)).double()
    r = (diff * scale.double().view(*scale.shape, 1, 1, 1) + shift.double().view(1, -1, 1, 1, 1)).float()
    if residual is not None:
        r = r + residual
    if negative_slope is not None:
        r = torch.maximum(np.float32(negative_slope) * r, r)
    return r


class OracleNetwork:
    """Forward of a PlainConvUNet or ResidualEncoderUNet on the CPU in float32.

    ``bf16=True`` emulates the bf16 arithmetic (``_bf16_operands``): operands rounded to
    bf16 at the convolutions that run on bf16 MFMA, everything else float32.

    ``spec`` is any object with the PlainConvUNetSpec / ResidualEncoderUNetSpec fields
    (src/nnunet_mlx/model/topology.py:132-430); ``residual`` selects the architecture.
    ``weights`` maps reference parameter names to arrays in the reference layout.
    """

    def __init__(self, spec: Any, weights: Weights, *, residual: bool = False,
                 bf16: bool = False) -> None:
        self.spec = spec
        self.residual = residual
        self.bf16 = bf16
        self.w = {name: _t(np.asarray(value)) for name, value in weights.items()}

    def _bf16_operands(self, prefix: str, x: torch.Tensor, weight: torch.Tensor):
        """The bf16 arithmetic's rounding points: the inputs and weights of every 3-D
        convolution with >= 8 taps except the one reading the network input, and of the
        transposed convolutions, are rounded to bf16 (nearest even); products and sums
        stay float32."""
        taps = int(np.prod(weight.shape[2:]))
        first = prefix in ("enc0.block0", "stem")
        if not self.bf16 or (prefix != "up" and (taps < 8 or first)):
            return x, weight
        return round_bf16(x), round_bf16(weight)

    # -- building blocks -----------------------------------------------------------
    def conv_norm(
        self,
        prefix: str,
        x: torch.Tensor,
        *,
        stride: tuple[int, ...],
        act: bool,
        residual: torch.Tensor | None = None,
        bias: bool | None = None,
    ) -> torch.Tensor:
        spec = self.spec
        weight = conv_weight_to_torch(self.w[f"{prefix}.conv.weight"].numpy())
        kernel = weight.shape[2:]
        padding = tuple(k // 2 for k in kernel)
        x, weight = self._bf16_operands(prefix, x, weight)
        y = F.conv3d(x, weight, None, stride=tuple(stride), padding=padding)
        has_bias = spec.conv_bias if bias is None else bias
        conv_bias = self.w[f"{prefix}.conv.bias"] if has_bias else None
        gamma = self.w.get(f"{prefix}.norm.weight") if spec.norm_affine else None
        beta = self.w.get(f"{prefix}.norm.bias") if spec.norm_affine else None
        slope = spec.leaky_slope if act else None
        return instance_norm(
            y, gamma, beta, spec.norm_eps, input_bias=conv_bias, negative_slope=slope,
            residual=residual,
        )

    def upsample(self, index: int, x: torch.Tensor, stride: tuple[int, ...]) -> torch.Tensor:
        weight = tconv_weight_to_torch(self.w[f"up{index}.weight"].numpy())
        bias = self.w.get(f"up{index}.bias") if self.spec.conv_bias else None
        x, weight = self._bf16_operands("up", x, weight)
        return F.conv_transpose3d(x, weight, bias, stride=tuple(stride))

    @staticmethod
    def match_spatial(values: torch.Tensor, reference: torch.Tensor) -> torch.Tensor:
        """Centre crop / zero pad (network.py:898-916)."""
        for axis in range(2, values.ndim):
            delta = int(values.shape[axis] - reference.shape[axis])
            if delta > 0:
                start = delta // 2
                values = values.narrow(axis, start, int(reference.shape[axis]))
            elif delta < 0:
                before = (-delta) // 2
                pad = [0, 0] * (values.ndim - 2)
                index = (values.ndim - 1 - axis) * 2
                pad[index] = before
                pad[index + 1] = -delta - before
                values = F.pad(values, pad)
        return values

    # -- networks ------------------------------------------------------------------
    def _decode(self, skips: list[torch.Tensor]) -> torch.Tensor:
        spec = self.spec
        stages = len(spec.features)
        hidden = skips.pop()
        for index in range(stages - 1):
            source = stages - 1 - index
            skip = skips.pop()
            hidden = self.match_spatial(self.upsample(index, hidden, spec.strides[source]), skip)
            hidden = torch.cat((hidden, skip), dim=1)
            for block in range(spec.decoder_convs[index]):
                hidden = self.conv_norm(
                    f"dec{index}.block{block}", hidden, stride=(1, 1, 1), act=True
                )
        last = stages - 2
        weight = conv_weight_to_torch(self.w[f"seg{last}.weight"].numpy())
        return F.conv3d(hidden, weight, self.w[f"seg{last}.bias"])

    def _plain(self, x: torch.Tensor) -> torch.Tensor:
        spec = self.spec
        skips = []
        for stage in range(len(spec.features)):
            for block in range(spec.encoder_convs[stage]):
                stride = spec.strides[stage] if block == 0 else (1, 1, 1)
                x = self.conv_norm(f"enc{stage}.block{block}", x, stride=stride, act=True)
            skips.append(x)
        return self._decode(skips)

    def _residual(self, x: torch.Tensor) -> torch.Tensor:
        spec = self.spec
        x = self.conv_norm("stem", x, stride=(1, 1, 1), act=True)
        bottleneck = getattr(spec, "bottleneck_channels", None)
        skips = []
        for stage in range(len(spec.features)):
            for block in range(spec.encoder_blocks[stage]):
                stride = tuple(spec.strides[stage]) if block == 0 else (1, 1, 1)
                prefix = f"res{stage}.block{block}"
                skip = x
                if stride != (1, 1, 1):
                    skip = F.avg_pool3d(skip, kernel_size=stride, stride=stride)
                if f"{prefix}.proj.conv.weight" in self.w:
                    skip = self.conv_norm(
                        f"{prefix}.proj", skip, stride=(1, 1, 1), act=False, bias=False
                    )
                if bottleneck is None:
                    h = self.conv_norm(f"{prefix}.conv1", x, stride=stride, act=True)
                    x = self.conv_norm(
                        f"{prefix}.conv2", h, stride=(1, 1, 1), act=True, residual=skip
                    )
                else:
                    h = self.conv_norm(f"{prefix}.conv1", x, stride=(1, 1, 1), act=True)
                    h = self.conv_norm(f"{prefix}.conv2", h, stride=stride, act=True)
                    x = self.conv_norm(
                        f"{prefix}.conv3", h, stride=(1, 1, 1), act=True, residual=skip
                    )
            skips.append(x)
        return self._decode(skips)

    @torch.no_grad()
    def __call__(self, tile: np.ndarray) -> np.ndarray:
        """Channels-last (n, D, H, W, C_in) float32 -> (n, D, H, W, num_classes)."""
        x = _t(tile).permute(0, 4, 1, 2, 3).contiguous()
        y = self._residual(x) if self.residual else self._plain(x)
        return y.permute(0, 2, 3, 4, 1).contiguous().numpy()


def brute_force_conv3d(x: np.ndarray, weight: np.ndarray, stride: tuple[int, int, int]) -> np.ndarray:
    """float64 direct convolution, channels-last, padding k//2; for tiny shapes only."""
    x = np.asarray(x, dtype=np.float64)
    w = np.asarray(weight, dtype=np.float64)
    n, d, h, wd, c = x.shape
    cout, kd, kh, kw, cin = w.shape
    assert cin == c
    pd, ph, pw = kd // 2, kh // 2, kw // 2
    od = (d + 2 * pd - kd) // stride[0] + 1
    oh = (h + 2 * ph - kh) // stride[1] + 1
    ow = (wd + 2 * pw - kw) // stride[2] + 1
    xp = np.zeros((n, d + 2 * pd, h + 2 * ph, wd + 2 * pw, c))
    xp[:, pd : pd + d, ph : ph + h, pw : pw + wd] = x
    out = np.zeros((n, od, oh, ow, cout))
    for a in range(kd):
        for b in range(kh):
            for e in range(kw):
                patch = xp[
                    :,
                    a : a + stride[0] * (od - 1) + 1 : stride[0],
                    b : b + stride[1] * (oh - 1) + 1 : stride[1],
                    e : e + stride[2] * (ow - 1) + 1 : stride[2],
                ]
                out += np.einsum("nzyxc,oc->nzyxo", patch, w[:, a, b, e, :])
    return out


def brute_force_tconv3d(x: np.ndarray, weight: np.ndarray) -> np.ndarray:
    """float64 stride==kernel transposed convolution, channels-last, no bias."""
    x = np.asarray(x, dtype=np.float64)
    w = np.asarray(weight, dtype=np.float64)
    n, d, h, wd, _ = x.shape
    cout, kd, kh, kw, _ = w.shape
    out = np.zeros((n, d * kd, h * kh, wd * kw, cout))
    for a in range(kd):
        for b in range(kh):
            for e in range(kw):
                out[:, a::kd, b::kh, e::kw] = np.einsum("nzyxc,oc->nzyxo", x, w[:, a, b, e, :])
    return out
