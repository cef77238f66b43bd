"""Random-initialised converted model folders for benchmarks and tests.

Writes the converted-checkpoint layout the loader reads (plans.json, dataset.json,
fold_<k>/checkpoint_final/{state.json, weights.safetensors}) for a PlainConvUNet or
ResidualEncoderUNet spec.  Weights follow nnU-Net's ``InitWeights_He(1e-2)``:
Kaiming-normal with std = sqrt(2 / (1 + 0.01^2)) / sqrt(fan_in), fan_in = C_in * prod(k)
for convolutions and C_out * prod(k) for transposed convolutions (torch's fan-in of a
ConvTranspose weight), biases 0, norm weight 1 and bias 0 — unless ``random_affine``
asks for random biases and affine parameters (to exercise those code paths).
Draws come from ``numpy.random.default_rng(SeedSequence(seed))``, one tensor at a time
in parameter-name order, so the same seed gives the same weights everywhere.
"""

from __future__ import annotations

import json
from collections.abc import Sequence
from pathlib import Path

import numpy as np

from nnunet_mlx.model.topology import NetworkSpec, PlainConvUNetSpec, ResidualEncoderUNetSpec
from nnunet_mlx.storage.checkpoint import (
    CheckpointIdentity,
    InferenceCheckpointState,
    save_inference_checkpoint,
)

_NEG_SLOPE = 1e-2


def parameter_shapes(spec: NetworkSpec) -> dict[str, tuple[int, ...]]:
    """Reference parameter names and MLX-layout shapes of ``spec`` (host-only helper)."""
    shapes: dict[str, tuple[int, ...]] = {}
    k = spec.kernel_sizes

    def convnorm(prefix: str, cin: int, cout: int, kernel, bias: bool) -> None:
        shapes[f"{prefix}.conv.weight"] = (cout, *kernel, cin)
        if bias:
            shapes[f"{prefix}.conv.bias"] = (cout,)
        if spec.norm_affine:
            shapes[f"{prefix}.norm.weight"] = (cout,)
            shapes[f"{prefix}.norm.bias"] = (cout,)

    stages = len(spec.features)
    if isinstance(spec, PlainConvUNetSpec):
        cin = spec.input_channels
        for s in range(stages):
            for j in range(spec.encoder_convs[s]):
                convnorm(f"enc{s}.block{j}", cin if j == 0 else spec.features[s], spec.features[s],
                         k[s], spec.conv_bias)
            cin = spec.features[s]
    else:
        stem = spec.effective_stem_channels
        convnorm("stem", spec.input_channels, stem, k[0], spec.conv_bias)
        cin = stem
        for s in range(stages):
            for b in range(spec.encoder_blocks[s]):
                bin_ = cin if b == 0 else spec.features[s]
                out = spec.features[s]
                pre = f"res{s}.block{b}"
                if spec.bottleneck_channels is None:
                    convnorm(f"{pre}.conv1", bin_, out, k[s], spec.conv_bias)
                    convnorm(f"{pre}.conv2", out, out, k[s], spec.conv_bias)
                else:
                    bc = spec.bottleneck_channels[s]
                    convnorm(f"{pre}.conv1", bin_, bc, (1, 1, 1), spec.conv_bias)
                    convnorm(f"{pre}.conv2", bc, bc, k[s], spec.conv_bias)
                    convnorm(f"{pre}.conv3", bc, out, (1, 1, 1), spec.conv_bias)
                if bin_ != out:
                    convnorm(f"{pre}.proj", bin_, out, (1, 1, 1), False)
            cin = spec.features[s]
    for d in range(stages - 1):
        src = stages - 1 - d
        below, skip = spec.features[src], spec.features[src - 1]
        stride = tuple(spec.strides[src])
        shapes[f"up{d}.weight"] = (skip, *stride, below)
        if spec.conv_bias:
            shapes[f"up{d}.bias"] = (skip,)
        for j in range(spec.decoder_convs[d]):
            convnorm(f"dec{d}.block{j}", 2 * skip if j == 0 else skip, skip, k[src - 1], spec.conv_bias)
        shapes[f"seg{d}.weight"] = (spec.num_classes, 1, 1, 1, skip)
        shapes[f"seg{d}.bias"] = (spec.num_classes,)
    return shapes


def random_weights(spec: NetworkSpec, seed: int, *, random_affine: bool = False) -> dict[str, np.ndarray]:
    rng = np.random.default_rng(np.random.SeedSequence(seed))
    gain = np.sqrt(2.0 / (1.0 + _NEG_SLOPE**2))
    weights: dict[str, np.ndarray] = {}
    for name in sorted(parameter_shapes(spec)):
        shape = parameter_shapes(spec)[name]
        if name.endswith(".weight") and len(shape) == 5:
            kernel = int(np.prod(shape[1:4]))
            fan_in = (shape[0] if name.startswith("up") else shape[4]) * kernel
            value = rng.standard_normal(shape) * (gain / np.sqrt(fan_in))
        elif name.endswith("norm.weight"):
            value = 1.0 + 0.1 * rng.standard_normal(shape) if random_affine else np.ones(shape)
        else:  # biases
            value = 0.1 * rng.standard_normal(shape) if random_affine else np.zeros(shape)
        weights[name] = value.astype(np.float32)
    return weights


def _class_name(spec: NetworkSpec) -> str:
    if isinstance(spec, ResidualEncoderUNetSpec):
        return "dynamic_network_architectures.architectures.unet.ResidualEncoderUNet"
    return "dynamic_network_architectures.architectures.unet.PlainConvUNet"


def plans_payload(spec: NetworkSpec, *, patch_size: Sequence[int], configuration: str = "3d_fullres",
                  normalization: str = "ZScoreNormalization") -> dict[str, object]:
    arch_kwargs: dict[str, object] = {
        "n_stages": len(spec.features),
        "features_per_stage": list(spec.features),
        "conv_op": "torch.nn.modules.conv.Conv3d",
        "kernel_sizes": [list(r) for r in spec.kernel_sizes],
        "strides": [list(r) for r in spec.strides],
        "n_conv_per_stage_decoder": list(spec.decoder_convs),
        "conv_bias": bool(spec.conv_bias),
        "norm_op": "torch.nn.modules.instancenorm.InstanceNorm3d",
        "norm_op_kwargs": {"eps": float(spec.norm_eps), "affine": bool(spec.norm_affine)},
        "dropout_op": None,
        "dropout_op_kwargs": None,
        "nonlin": "torch.nn.LeakyReLU",
        "nonlin_kwargs": {"inplace": True, "negative_slope": float(spec.leaky_slope)},
    }
    if isinstance(spec, ResidualEncoderUNetSpec):
        arch_kwargs["n_blocks_per_stage"] = list(spec.encoder_blocks)
        if spec.bottleneck_channels is not None:
            arch_kwargs["block"] = "dynamic_network_architectures.building_blocks.residual.BottleneckD"
            arch_kwargs["bottleneck_channels"] = list(spec.bottleneck_channels)
        if spec.stem_channels is not None:
            arch_kwargs["stem_channels"] = spec.stem_channels
    else:
        arch_kwargs["n_conv_per_stage"] = list(spec.encoder_convs)
    channels = spec.input_channels
    return {
        "dataset_name": "Dataset999_Synthetic",
        "plans_name": "nnUNetPlans",
        "original_median_spacing_after_transp": [1.0, 1.0, 1.0],
        "original_median_shape_after_transp": [int(v) for v in patch_size],
        "image_reader_writer": "SimpleITKIO",
        "transpose_forward": [0, 1, 2],
        "transpose_backward": [0, 1, 2],
        "configurations": {
            configuration: {
                "data_identifier": f"nnUNetPlans_{configuration}",
                "preprocessor_name": "DefaultPreprocessor",
                "batch_size": 2,
                "batch_dice": False,
                "patch_size": [int(v) for v in patch_size],
                "median_image_size_in_voxels": [int(v) for v in patch_size],
                "spacing": [1.0, 1.0, 1.0],
                "normalization_schemes": [normalization] * channels,
                "use_mask_for_norm": [False] * channels,
                "resampling_fn_data": "resample_data_or_seg_to_shape",
                "resampling_fn_seg": "resample_data_or_seg_to_shape",
                "resampling_fn_data_kwargs": {"is_seg": False, "order": 3, "order_z": 0, "force_separate_z": None},
                "resampling_fn_seg_kwargs": {"is_seg": True, "order": 1, "order_z": 0, "force_separate_z": None},
                "resampling_fn_probabilities": "resample_data_or_seg_to_shape",
                "resampling_fn_probabilities_kwargs": {"is_seg": False, "order": 1, "order_z": 0, "force_separate_z": None},
                "architecture": {
                    "network_class_name": _class_name(spec),
                    "arch_kwargs": arch_kwargs,
                    "_kw_requires_import": ["conv_op", "norm_op", "dropout_op", "nonlin"],
                },
                "batch_dice_": False,
            }
        },
        "experiment_planner_used": "ExperimentPlanner",
        "label_manager": "LabelManager",
        "foreground_intensity_properties_per_channel": {
            str(c): {"max": 1.0, "mean": 0.0, "median": 0.0, "min": -1.0,
                     "percentile_00_5": -1.0, "percentile_99_5": 1.0, "std": 1.0}
            for c in range(channels)
        },
    }


def dataset_payload(spec: NetworkSpec, labels: Sequence[str] | None = None) -> dict[str, object]:
    names = list(labels) if labels is not None else [f"class{i}" for i in range(1, spec.num_classes)]
    table = {"background": 0}
    for index, name in enumerate(names, start=1):
        table[name] = index
    return {
        "channel_names": {str(c): f"channel{c}" for c in range(spec.input_channels)},
        "labels": table,
        "numTraining": 1,
        "file_ending": ".nii.gz",
    }


def write_random_model_folder(
    folder: str | Path, spec: NetworkSpec, *, patch_size: Sequence[int], seeds: Sequence[int] = (0,),
    configuration: str = "3d_fullres", mirroring_axes: Sequence[int] = (0, 1, 2),
    trainer_name: str = "nnUNetTrainer", random_affine: bool = False,
    labels: Sequence[str] | None = None,
) -> Path:
    """Write one fold per seed (fold k uses seeds[k]); return the folder path."""
    root = Path(folder)
    root.mkdir(parents=True, exist_ok=True)
    (root / "plans.json").write_text(
        json.dumps(plans_payload(spec, patch_size=patch_size, configuration=configuration), indent=2) + "\n")
    (root / "dataset.json").write_text(json.dumps(dataset_payload(spec, labels), indent=2) + "\n")
    for fold, seed in enumerate(seeds):
        state = InferenceCheckpointState(
            identity=CheckpointIdentity(trainer_name=trainer_name, configuration=configuration, fold=fold),
            current_epoch=None,
            spatial_dims=3,
            inference_allowed_mirroring_axes=tuple(int(a) for a in mirroring_axes),
            dropped_source_keys=(),
        )
        save_inference_checkpoint(root / f"fold_{fold}" / "checkpoint_final",
                                  weights=random_weights(spec, seed, random_affine=random_affine),
                                  state=state)
    return root
