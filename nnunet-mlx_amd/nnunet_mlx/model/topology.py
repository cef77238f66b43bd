"""Topology specs for the supported nnU-Net v2 networks, parsed from plans.

Same public surface as the reference's ``nnunet_mlx.model.topology``
(src/nnunet_mlx/model/topology.py:132-430): ``PlainConvUNetSpec`` and
``ResidualEncoderUNetSpec`` frozen dataclasses with ``from_plans``, ``spatial_dims``
and ``to_payload``.  A plans file describes the network in
``configurations.<name>.architecture`` as ``network_class_name`` plus ``arch_kwargs``
(upstream dynamic_network_architectures constructor arguments).  Only networks this
package computes exactly are admitted: Conv + InstanceNorm + LeakyReLU, activation after
the norm, no active dropout, no running statistics.  Anything else raises
``ContractError`` naming the offending ``arch_kwargs`` entry.
"""

from __future__ import annotations

import math
from collections.abc import Mapping, Sequence
from dataclasses import dataclass

from nnunet_mlx.errors import ContractError

SpatialShape = tuple[int, ...]

# Operation class paths must end with these names (torch registers the classes under
# several module paths, e.g. torch.nn.Conv3d and torch.nn.modules.conv.Conv3d).
_OPERATION_SUFFIXES = {"conv_op": "Conv{d}d", "norm_op": "InstanceNorm{d}d", "nonlin": "LeakyReLU"}
# Option keys of the norm, activation and dropout that carry no arithmetic of their own,
# or whose values are checked below.
_NORM_OPTIONS = frozenset({"eps", "affine", "momentum", "track_running_stats"})
_NONLIN_OPTIONS = frozenset({"negative_slope", "inplace"})
_DROPOUT_OPTIONS = frozenset({"p", "inplace"})
_DROPOUT_CLASSES = frozenset(
    f"torch.nn.{module}Dropout{suffix}" for module in ("", "modules.dropout.")
    for suffix in ("", "2d", "3d"))


class _ArchKwargs:
    """Typed access to one ``arch_kwargs`` mapping; every failure names its key."""

    def __init__(self, raw: object, where: str) -> None:
        if not isinstance(raw, Mapping):
            raise ContractError(f"{where}.arch_kwargs is not a mapping")
        self.raw = raw
        self.where = f"{where}.arch_kwargs"

    def error(self, key: str, problem: str) -> ContractError:
        return ContractError(f"plans {self.where}.{key} {problem}")

    def has(self, key: str) -> bool:
        return key in self.raw

    def section(self, key: str) -> Mapping[str, object]:
        value = self.raw.get(key)
        if value is None:
            return {}
        if not isinstance(value, Mapping):
            raise self.error(key, "is not a mapping")
        return value

    def flag(self, key: str, default: bool, source: Mapping[str, object] | None = None) -> bool:
        value = (self.raw if source is None else source).get(key, default)
        if type(value) is not bool:
            raise self.error(key, f"must be true or false, not {value!r}")
        return value

    def real(self, key: str, default: float, source: Mapping[str, object] | None = None) -> float:
        value = (self.raw if source is None else source).get(key, default)
        if type(value) is bool or not isinstance(value, (int, float)) or not math.isfinite(value):
            raise self.error(key, f"must be a finite number, not {value!r}")
        return float(value)

    def count(self, key: str, value: object = None) -> int:
        value = self.raw.get(key) if value is None else value
        if type(value) is not int or value < 1:
            raise self.error(key, f"must hold positive integers, found {value!r}")
        return value

    def counts(self, key: str) -> tuple[int, ...]:
        value = self.raw.get(key)
        if isinstance(value, (str, bytes)) or not isinstance(value, Sequence) or not value:
            raise self.error(key, "must be a non-empty list of positive integers")
        return tuple(self.count(key, item) for item in value)

    def per_stage(self, key: str, stages: int) -> tuple[int, ...]:
        """One positive count per stage; a single integer stands for every stage."""
        value = self.raw.get(key)
        if type(value) is int:
            return (self.count(key, value),) * stages
        values = self.counts(key)
        if len(values) != stages:
            raise self.error(key, f"has {len(values)} entries for {stages} encoder stages")
        return values

    def rows(self, key: str) -> tuple[SpatialShape, ...]:
        """Per-stage spatial rows (kernel sizes, strides): 2 or 3 positive integers each,
        the same number in every row."""
        value = self.raw.get(key)
        if isinstance(value, (str, bytes)) or not isinstance(value, Sequence) or not value:
            raise self.error(key, "must be a non-empty list of spatial rows")
        rows = []
        for row in value:
            if isinstance(row, (str, bytes)) or not isinstance(row, Sequence):
                raise self.error(key, f"row {row!r} is not a list")
            rows.append(tuple(self.count(key, v) for v in row))
        lengths = {len(r) for r in rows}
        if len(lengths) != 1 or lengths.pop() not in (2, 3):
            raise self.error(key, "rows must all hold 2 or all hold 3 integers")
        return tuple(rows)


def _read_architecture(plans: Mapping[str, object], configuration: str,
                       class_suffix: str) -> tuple[_ArchKwargs, int]:
    """The configuration's ``arch_kwargs`` after the checks every admitted network
    shares, and the number of spatial dimensions."""
    configurations = plans.get("configurations") if isinstance(plans, Mapping) else None
    if not isinstance(configurations, Mapping) or configuration not in configurations:
        raise ContractError(f"nnU-Net plans have no configuration {configuration!r}")
    entry = configurations[configuration]
    architecture = entry.get("architecture") if isinstance(entry, Mapping) else None
    if not isinstance(architecture, Mapping):
        raise ContractError(f"plans configuration {configuration!r} has no architecture")
    name = architecture.get("network_class_name")
    if not isinstance(name, str) or not name.endswith(class_suffix):
        raise ContractError(f"unsupported nnU-Net architecture {name!r}")
    args = _ArchKwargs(architecture.get("arch_kwargs"), f"configurations.{configuration}")
    dims = len(args.rows("kernel_sizes")[0])

    for key, suffix in _OPERATION_SUFFIXES.items():
        op = args.raw.get(key)
        wanted = suffix.format(d=dims)
        if not isinstance(op, str) or not op.endswith("." + wanted):
            raise ContractError(f"{dims}-D nnU-Net requires {wanted} for {key}, got {op!r}")

    # the activation must follow the norm
    if args.flag("nonlin_first", False):
        raise args.error("nonlin_first", "asks for the activation before the norm, which is "
                                         "not supported")
    stages = len(args.counts("features_per_stage"))
    if args.has("n_stages") and args.count("n_stages") != stages:
        raise args.error("n_stages", f"is {args.raw['n_stages']} but features_per_stage has "
                                     f"{stages} entries")

    norm = args.section("norm_op_kwargs")
    if set(norm) - _NORM_OPTIONS:
        raise args.error("norm_op_kwargs", f"has unsupported options {sorted(set(norm) - _NORM_OPTIONS)}")
    if args.flag("track_running_stats", False, norm):
        raise args.error("norm_op_kwargs", "uses running statistics, which are not supported")
    if norm.get("momentum") is not None and not 0.0 <= args.real("momentum", 0.1, norm) <= 1.0:
        raise args.error("norm_op_kwargs", "momentum lies outside [0, 1]")

    nonlin = args.section("nonlin_kwargs")
    if set(nonlin) - _NONLIN_OPTIONS:
        raise args.error("nonlin_kwargs", f"has unsupported options {sorted(set(nonlin) - _NONLIN_OPTIONS)}")

    dropout = args.raw.get("dropout_op")
    if dropout is not None:
        if dropout not in _DROPOUT_CLASSES:
            raise args.error("dropout_op", f"{dropout!r} is not a torch dropout class")
        options = args.section("dropout_op_kwargs")
        if set(options) - _DROPOUT_OPTIONS:
            raise args.error("dropout_op_kwargs", "has unsupported options")
        if args.real("p", 0.5, options) != 0.0:
            raise args.error("dropout_op_kwargs", "enables dropout at inference (p != 0)")
    return args, dims


def _norm_and_activation(args: _ArchKwargs) -> dict[str, object]:
    norm = args.section("norm_op_kwargs")
    nonlin = args.section("nonlin_kwargs")
    return dict(
        conv_bias=args.flag("conv_bias", False),
        norm_eps=args.real("eps", 1e-5, norm),
        norm_affine=args.flag("affine", False, norm),
        leaky_slope=args.real("negative_slope", 0.01, nonlin),
    )


def _validate_topology(spec, per_stage: tuple[int, ...], kind: str) -> None:
    """Shape rules both specs share, whether built from plans or directly."""
    n = len(spec.features)
    problems = []
    if spec.input_channels < 1 or spec.num_classes < 1:
        problems.append("needs input channels and at least one output")
    if n < 2:
        problems.append("needs at least two stages")
    if {len(spec.kernel_sizes), len(spec.strides), len(per_stage)} != {n}:
        problems.append("kernel sizes, strides and per-stage counts must have one entry per stage")
    if len(spec.decoder_convs) != n - 1:
        problems.append("needs one decoder entry per skip connection")
    widths = {len(row) for row in spec.kernel_sizes} | {len(row) for row in spec.strides}
    if len(widths) != 1 or not widths <= {2, 3}:
        problems.append("kernel and stride rows must all be 2-D or all 3-D")
    if any(k < 1 or k % 2 == 0 for row in spec.kernel_sizes for k in row):
        problems.append("convolution kernels must be positive and odd")
    if not spec.norm_eps > 0:
        problems.append("normalization epsilon must be positive")
    if not 0 <= spec.leaky_slope <= 1:
        problems.append("LeakyReLU negative_slope must lie in [0, 1]")
    if problems:
        raise ContractError(f"{kind}: " + "; ".join(problems))


@dataclass(frozen=True)
class PlainConvUNetSpec:
    """Topology of upstream's ``PlainConvUNet``; per-stage fields run from the highest
    resolution down to the bottleneck (src/nnunet_mlx/model/topology.py:132-254)."""

    input_channels: int
    num_classes: int
    features: tuple[int, ...]
    kernel_sizes: tuple[SpatialShape, ...]
    strides: tuple[SpatialShape, ...]
    encoder_convs: tuple[int, ...]
    decoder_convs: tuple[int, ...]
    conv_bias: bool = True
    norm_eps: float = 1e-5
    norm_affine: bool = True
    leaky_slope: float = 0.01

    def __post_init__(self) -> None:
        _validate_topology(self, self.encoder_convs, "PlainConvUNet")

    @property
    def spatial_dims(self) -> int:
        return len(self.kernel_sizes[0])

    @classmethod
    def from_plans(cls, plans: Mapping[str, object], *, configuration: str, input_channels: int,
                   num_classes: int) -> PlainConvUNetSpec:
        args, _ = _read_architecture(plans, configuration, ".PlainConvUNet")
        features = args.counts("features_per_stage")
        return cls(input_channels=input_channels, num_classes=num_classes, features=features,
                   kernel_sizes=args.rows("kernel_sizes"), strides=args.rows("strides"),
                   encoder_convs=args.per_stage("n_conv_per_stage", len(features)),
                   decoder_convs=args.counts("n_conv_per_stage_decoder"),
                   **_norm_and_activation(args))

    def to_payload(self) -> dict[str, object]:
        return {
            "input_channels": self.input_channels, "num_classes": self.num_classes,
            "features": self.features, "kernel_sizes": self.kernel_sizes, "strides": self.strides,
            "encoder_convs": self.encoder_convs, "decoder_convs": self.decoder_convs,
            "conv_bias": self.conv_bias, "norm_eps": self.norm_eps,
            "norm_affine": self.norm_affine, "leaky_slope": self.leaky_slope,
        }


@dataclass(frozen=True)
class ResidualEncoderUNetSpec:
    """Topology of upstream's ``ResidualEncoderUNet`` (BasicBlockD, or BottleneckD when
    ``bottleneck_channels`` is set) (src/nnunet_mlx/model/topology.py:257-430)."""

    input_channels: int
    num_classes: int
    features: tuple[int, ...]
    kernel_sizes: tuple[SpatialShape, ...]
    strides: tuple[SpatialShape, ...]
    encoder_blocks: tuple[int, ...]
    decoder_convs: tuple[int, ...]
    conv_bias: bool = True
    norm_eps: float = 1e-5
    norm_affine: bool = True
    leaky_slope: float = 0.01
    stem_channels: int | None = None
    bottleneck_channels: tuple[int, ...] | None = None

    def __post_init__(self) -> None:
        _validate_topology(self, self.encoder_blocks, "ResidualEncoderUNet")
        if self.stem_channels is not None and self.stem_channels < 1:
            raise ContractError("ResidualEncoderUNet: stem channels must be positive")
        if self.bottleneck_channels is not None and (
                len(self.bottleneck_channels) != len(self.features)
                or min(self.bottleneck_channels) < 1):
            raise ContractError("ResidualEncoderUNet: bottleneck channels need one positive "
                                "entry per encoder stage")

    @property
    def spatial_dims(self) -> int:
        return len(self.kernel_sizes[0])

    @property
    def effective_stem_channels(self) -> int:
        return self.stem_channels or self.features[0]

    @classmethod
    def from_plans(cls, plans: Mapping[str, object], *, configuration: str, input_channels: int,
                   num_classes: int) -> ResidualEncoderUNetSpec:
        args, _ = _read_architecture(plans, configuration, ".ResidualEncoderUNet")
        features = args.counts("features_per_stage")
        block = args.raw.get("block")
        # BasicBlockD (the default block) has no bottleneck width; BottleneckD needs one,
        # given once for every stage or per stage
        if block is None or (isinstance(block, str) and block.endswith(".BasicBlockD")):
            if args.raw.get("bottleneck_channels") is not None:
                raise args.error("bottleneck_channels", "is set for BasicBlockD blocks")
            bottleneck = None
        elif isinstance(block, str) and block.endswith(".BottleneckD"):
            if args.raw.get("bottleneck_channels") is None:
                raise args.error("bottleneck_channels", "is required for BottleneckD blocks")
            bottleneck = args.per_stage("bottleneck_channels", len(features))
        else:
            raise args.error("block", f"{block!r} is not BasicBlockD or BottleneckD")
        stem = args.raw.get("stem_channels")
        return cls(input_channels=input_channels, num_classes=num_classes, features=features,
                   kernel_sizes=args.rows("kernel_sizes"), strides=args.rows("strides"),
                   encoder_blocks=args.per_stage("n_blocks_per_stage", len(features)),
                   decoder_convs=args.counts("n_conv_per_stage_decoder"),
                   stem_channels=None if stem is None else args.count("stem_channels"),
                   bottleneck_channels=bottleneck, **_norm_and_activation(args))

    def to_payload(self) -> dict[str, object]:
        return {
            "input_channels": self.input_channels, "num_classes": self.num_classes,
            "features": self.features, "kernel_sizes": self.kernel_sizes, "strides": self.strides,
            "encoder_blocks": self.encoder_blocks, "decoder_convs": self.decoder_convs,
            "conv_bias": self.conv_bias, "norm_eps": self.norm_eps,
            "norm_affine": self.norm_affine, "leaky_slope": self.leaky_slope,
            "stem_channels": self.stem_channels, "bottleneck_channels": self.bottleneck_channels,
        }


NetworkSpec = PlainConvUNetSpec | ResidualEncoderUNetSpec
