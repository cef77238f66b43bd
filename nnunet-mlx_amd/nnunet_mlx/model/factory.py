"""Plan-bound construction of nnU-Net networks on the HIP path.

Reference: build_model_from_plans (src/nnunet_mlx/model/factory.py:17-65).
"""

from __future__ import annotations

from collections.abc import Mapping

from nnunet_mlx.errors import ContractError
from nnunet_mlx.model.topology import PlainConvUNetSpec, ResidualEncoderUNetSpec


def spec_from_plans(plans: Mapping[str, object], *, configuration: str, input_channels: int,
                    output_channels: int):
    configurations = plans.get("configurations")
    if not isinstance(configurations, Mapping) or configuration not in configurations:
        raise ContractError(f"nnU-Net plans lack configuration {configuration!r}")
    config = configurations[configuration]
    architecture = config.get("architecture") if isinstance(config, Mapping) else None
    name = architecture.get("network_class_name") if isinstance(architecture, Mapping) else None
    if not isinstance(name, str):
        raise ContractError("plans architecture lacks network_class_name")
    if name.endswith("PlainConvUNet"):
        return PlainConvUNetSpec.from_plans(plans, configuration=configuration,
                                            input_channels=input_channels, num_classes=output_channels)
    if name.endswith("ResidualEncoderUNet"):
        return ResidualEncoderUNetSpec.from_plans(plans, configuration=configuration,
                                                  input_channels=input_channels,
                                                  num_classes=output_channels)
    raise ContractError(f"unsupported nnU-Net architecture {name!r}")


def build_model_from_plans(plans: Mapping[str, object], *, configuration: str, input_channels: int,
                           output_channels: int):
    """Build the network named by a plans configuration, without weights."""
    from nnunet_mlx.model.network import build_network

    return build_network(spec_from_plans(plans, configuration=configuration,
                                         input_channels=input_channels,
                                         output_channels=output_channels))
