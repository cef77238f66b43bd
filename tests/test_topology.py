"""Plans parsing of the network specs (host only): the plans the synthetic writer emits
read back to the same spec, and every unsupported network feature is refused with a
ContractError naming the plans entry."""

from __future__ import annotations

import copy

import pytest

from nnunet_mlx.errors import ContractError
from nnunet_mlx.model.factory import spec_from_plans
from nnunet_mlx.model.topology import PlainConvUNetSpec, ResidualEncoderUNetSpec
from nnunet_mlx.storage.synthetic import plans_payload

K3 = ((3, 3, 3),)
PLAIN = PlainConvUNetSpec(1, 3, (4, 8, 16), K3 * 3, ((1, 1, 1), (2, 2, 2), (1, 2, 2)), (2, 1, 2),
                          (1, 2), conv_bias=True, norm_eps=1e-4, norm_affine=True, leaky_slope=0.02)
BASIC = ResidualEncoderUNetSpec(2, 4, (4, 8, 16), K3 * 3, ((1, 1, 1), (2, 2, 2), (2, 2, 2)),
                                (1, 2, 2), (1, 1), stem_channels=6)
BOTTLENECK = ResidualEncoderUNetSpec(1, 2, (4, 8), K3 * 2, ((1, 1, 1), (2, 2, 2)), (2, 1), (1,),
                                     bottleneck_channels=(2, 3))


def _plans(spec):
    return plans_payload(spec, patch_size=(16, 16, 16))


def _args(plans):
    return plans["configurations"]["3d_fullres"]["architecture"]["arch_kwargs"]


@pytest.mark.parametrize("spec", [PLAIN, BASIC, BOTTLENECK], ids=["plain", "basic", "bottleneck"])
def test_plans_round_trip(spec):
    got = spec_from_plans(_plans(spec), configuration="3d_fullres",
                          input_channels=spec.input_channels, output_channels=spec.num_classes)
    assert got == spec


def test_single_counts_expand_to_every_stage():
    plans = _plans(PLAIN)
    _args(plans)["n_conv_per_stage"] = 2
    got = PlainConvUNetSpec.from_plans(plans, configuration="3d_fullres", input_channels=1,
                                       num_classes=3)
    assert got.encoder_convs == (2, 2, 2)
    plans = _plans(BOTTLENECK)
    _args(plans)["bottleneck_channels"] = 5
    got = ResidualEncoderUNetSpec.from_plans(plans, configuration="3d_fullres", input_channels=1,
                                             num_classes=2)
    assert got.bottleneck_channels == (5, 5)


def _refused(spec, edit, match, cls=None):
    plans = copy.deepcopy(_plans(spec))
    edit(_args(plans), plans)
    cls = cls or type(spec)
    with pytest.raises(ContractError, match=match):
        cls.from_plans(plans, configuration="3d_fullres", input_channels=spec.input_channels,
                       num_classes=spec.num_classes)


def _set(key, value):
    def edit(args, plans):
        args[key] = value
    return edit


def _set_in(section, key, value):
    def edit(args, plans):
        args[section] = dict(args.get(section) or {}, **{key: value})
    return edit


@pytest.mark.parametrize("edit,match", [
    (_set("nonlin_first", True), "nonlin_first"),
    (_set("n_stages", 4), "n_stages"),
    (_set("conv_op", "torch.nn.Conv2d"), "Conv3d"),
    (_set("norm_op", "torch.nn.BatchNorm3d"), "InstanceNorm3d"),
    (_set("nonlin", "torch.nn.ReLU"), "LeakyReLU"),
    (_set_in("norm_op_kwargs", "track_running_stats", True), "running statistics"),
    (_set_in("norm_op_kwargs", "momentum", 1.5), "momentum"),
    (_set_in("norm_op_kwargs", "weird", 1), "unsupported options"),
    (_set_in("nonlin_kwargs", "weird", 1), "unsupported options"),
    (_set("dropout_op", "torch.nn.Dropout3d"), "p != 0"),
    (_set("dropout_op", "my.Dropout"), "not a torch dropout"),
    (_set("kernel_sizes", [[3, 3, 3], [3, 3], [3, 3, 3]]), "kernel_sizes"),
    (_set("features_per_stage", [4, 8, True]), "features_per_stage"),
    (_set("conv_bias", 1), "conv_bias"),
    (_set("n_conv_per_stage", [2, 2]), "encoder stages"),
    (_set("strides", "222"), "strides"),
])
def test_unsupported_plain_plans(edit, match):
    _refused(PLAIN, edit, match)


def test_dropout_with_zero_probability_is_admitted():
    plans = _plans(PLAIN)
    _args(plans)["dropout_op"] = "torch.nn.modules.dropout.Dropout3d"
    _args(plans)["dropout_op_kwargs"] = {"p": 0.0, "inplace": True}
    assert PlainConvUNetSpec.from_plans(plans, configuration="3d_fullres", input_channels=1,
                                        num_classes=3) == PLAIN


@pytest.mark.parametrize("spec,edit,match", [
    (BASIC, _set("block", "dynamic_network_architectures.building_blocks.residual.Other"),
     "BasicBlockD or BottleneckD"),
    (BASIC, _set("bottleneck_channels", [1, 2, 3]), "BasicBlockD"),
    (BOTTLENECK, _set("bottleneck_channels", None), "required for BottleneckD"),
    (BOTTLENECK, _set("bottleneck_channels", [1, 2, 3]), "encoder stages"),
    (BASIC, _set("stem_channels", 0), "stem_channels"),
])
def test_unsupported_residual_plans(spec, edit, match):
    _refused(spec, edit, match)


def test_wrong_architecture_and_configuration():
    with pytest.raises(ContractError, match="unsupported nnU-Net architecture"):
        ResidualEncoderUNetSpec.from_plans(_plans(PLAIN), configuration="3d_fullres",
                                           input_channels=1, num_classes=3)
    with pytest.raises(ContractError, match="no configuration"):
        PlainConvUNetSpec.from_plans(_plans(PLAIN), configuration="2d", input_channels=1,
                                     num_classes=3)


def test_direct_construction_checks():
    with pytest.raises(ContractError, match="odd"):
        PlainConvUNetSpec(1, 3, (4, 8), ((3, 3, 3), (2, 2, 2)), ((1, 1, 1), (2, 2, 2)), (1, 1), (1,))
    with pytest.raises(ContractError, match="one decoder entry"):
        PlainConvUNetSpec(1, 3, (4, 8), K3 * 2, ((1, 1, 1), (2, 2, 2)), (1, 1), (1, 1))
    with pytest.raises(ContractError, match="negative_slope"):
        PlainConvUNetSpec(1, 3, (4, 8), K3 * 2, ((1, 1, 1), (2, 2, 2)), (1, 1), (1,),
                          leaky_slope=2.0)
    with pytest.raises(ContractError, match="bottleneck"):
        ResidualEncoderUNetSpec(1, 3, (4, 8), K3 * 2, ((1, 1, 1), (2, 2, 2)), (1, 1), (1,),
                                bottleneck_channels=(2,))
