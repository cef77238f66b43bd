"""Upstream nnU-Net checkpoint conversion (host only).

The upstream names and layouts are built here from the network's own parameter list with
the upstream module naming (dynamic_network_architectures: ``encoder.stages.<s>.0.convs.<i>
.conv`` / ``.norm``, ``encoder.stem.convs.0``, ``encoder.stages.<s>.blocks.<b>.conv1|conv2``
and ``.skip.1``, ``decoder.stages.<s>.convs.<i>``, ``decoder.transpconvs.<s>``,
``decoder.seg_layers.<s>``; torch conv weights (C_out, C_in, *k), transposed (C_in, C_out,
*k)), so conversion must invert them exactly.
"""

from __future__ import annotations

import json

import numpy as np
import pytest
import torch

from nnunet_mlx.errors import ContractError
from nnunet_mlx.model.topology import PlainConvUNetSpec, ResidualEncoderUNetSpec
from nnunet_mlx.storage import checkpoint as ckpt
from nnunet_mlx.storage import upstream
from nnunet_mlx.storage.synthetic import dataset_payload, plans_payload, random_weights

K3 = ((3, 3, 3),)
PLAIN = PlainConvUNetSpec(1, 3, (4, 8, 16), K3 * 3, ((1, 1, 1), (2, 2, 2), (2, 2, 2)), (2, 2, 2), (2, 2))
RESENC = ResidualEncoderUNetSpec(2, 4, (4, 8, 16), K3 * 3, ((1, 1, 1), (2, 2, 2), (2, 2, 2)),
                                 (1, 2, 2), (1, 1))


def upstream_name(name: str) -> tuple[str, str]:
    """(upstream key, layout kind) of one converted name."""
    p = name.split(".")
    if p[0].startswith("enc"):
        return f"encoder.stages.{p[0][3:]}.0.convs.{p[1][5:]}.{p[2]}.{p[3]}", "conv"
    if p[0] == "stem":
        return f"encoder.stem.convs.0.{p[1]}.{p[2]}", "conv"
    if p[0].startswith("res"):
        s, b = p[0][3:], p[1][5:]
        if p[2] == "proj":
            return f"encoder.stages.{s}.blocks.{b}.skip.1.{p[3]}.{p[4]}", "conv"
        return f"encoder.stages.{s}.blocks.{b}.{p[2]}.{p[3]}.{p[4]}", "conv"
    if p[0].startswith("dec"):
        return f"decoder.stages.{p[0][3:]}.convs.{p[1][5:]}.{p[2]}.{p[3]}", "conv"
    if p[0].startswith("up"):
        return f"decoder.transpconvs.{p[0][2:]}.{p[1]}", "transposed"
    if p[0].startswith("seg"):
        return f"decoder.seg_layers.{p[0][3:]}.{p[1]}", "seg"
    raise AssertionError(name)


def to_upstream(weights: dict[str, np.ndarray]) -> dict[str, torch.Tensor]:
    state = {}
    for name, value in weights.items():
        key, kind = upstream_name(name)
        if name.endswith(".weight") and value.ndim == 5:
            # (C_out, *k, C_in) -> torch (C_out, C_in, *k) or transposed (C_in, C_out, *k)
            value = np.moveaxis(value, -1, 1) if kind != "transposed" else np.moveaxis(value, -1, 0)
        state[key] = torch.from_numpy(np.ascontiguousarray(value))
    return state


@pytest.mark.parametrize("spec", [PLAIN, RESENC], ids=["plain", "resenc"])
def test_state_dict_round_trip(spec):
    weights = random_weights(spec, seed=3, random_affine=True)
    state = to_upstream(weights)
    # aliases the upstream modules register a second time
    first = next(iter(state))
    state["decoder.encoder.stages.0.0.convs.0.conv.weight"] = state[first].clone()
    state["encoder.stages.0.0.convs.0.all_modules.0.weight"] = state[first].clone()
    converted = upstream.convert_state_dict(state)
    assert set(converted.weights) == set(weights)
    for name, value in weights.items():
        np.testing.assert_array_equal(converted.weights[name], value)
    assert converted.dropped_keys == ("decoder.encoder.stages.0.0.convs.0.conv.weight",
                                      "encoder.stages.0.0.convs.0.all_modules.0.weight")


def test_layouts_of_single_keys():
    w = np.arange(2 * 3 * 1 * 2 * 4, dtype=np.float32).reshape(2, 3, 1, 2, 4)
    name, out = upstream.map_key_and_layout("encoder.stages.1.0.convs.0.conv.weight", w)
    assert name == "enc1.block0.conv.weight" and out.shape == (2, 1, 2, 4, 3)
    assert out[1, 0, 1, 3, 2] == w[1, 2, 0, 1, 3]
    name, out = upstream.map_key_and_layout("decoder.transpconvs.0.weight", w)
    assert name == "up0.weight" and out.shape == (3, 1, 2, 4, 2)
    assert out[2, 0, 1, 3, 1] == w[1, 2, 0, 1, 3]
    name, out = upstream.map_key_and_layout("decoder.stages.2.convs.1.norm.bias", w[0, 0, 0, 0])
    assert name == "dec2.block1.norm.bias"
    assert upstream.map_key_and_layout("encoder.stages.0.0.convs.0.all_modules.1.weight", w) is None
    assert upstream.map_key_and_layout("decoder.deep_supervision.weight", w) is None


def test_state_dict_errors():
    good = {"decoder.seg_layers.0.bias": torch.zeros(3)}
    with pytest.raises(ContractError):
        upstream.convert_state_dict({"decoder.seg_layers.0.bias": torch.tensor([np.nan])})
    with pytest.raises(ContractError):
        upstream.convert_state_dict({"mystery.weight": torch.zeros(1)})
    with pytest.raises(ContractError):
        upstream.convert_state_dict({"decoder.seg_layers.0.bias": [0.0]})
    with pytest.raises(ContractError):
        upstream.convert_state_dict({"decoder.encoder.x": torch.zeros(1)})
    assert upstream.convert_state_dict(good).weights["seg0.bias"].dtype == np.float32
    # the auxiliary LesionTracer head: dropped only when asked, and only with 11 outputs
    aux = {"decoder.seg_layers.0.weight": torch.zeros(3, 4, 1, 1, 1),
           "decoder.organ_seg_layers.0.weight": torch.zeros(11, 4, 1, 1, 1)}
    with pytest.raises(ContractError):
        upstream.convert_state_dict(aux)
    assert upstream.convert_state_dict(aux, allow_lesiontracer_auxiliary_head=True).dropped_keys == (
        "decoder.organ_seg_layers.0.weight",)


def write_upstream_folder(root, spec, *, folds=(0, 1), trainer="nnUNetTrainer",
                          configuration="3d_fullres"):
    root.mkdir()
    (root / "plans.json").write_text(json.dumps(plans_payload(spec, patch_size=(16, 16, 16))))
    (root / "dataset.json").write_text(json.dumps(dataset_payload(spec)))
    originals = {}
    for k, fold in enumerate(folds):
        weights = random_weights(spec, seed=10 + k, random_affine=True)
        originals[fold] = weights
        (root / f"fold_{fold}").mkdir()
        torch.save({"network_weights": to_upstream(weights), "trainer_name": trainer,
                    "init_args": {"configuration": configuration, "fold": fold},
                    "inference_allowed_mirroring_axes": (0, 1, 2), "current_epoch": 999,
                    "logging": {"loss": [np.float32(0.5), np.float64(0.25)]}},
                   root / f"fold_{fold}" / "checkpoint_final.pth")
    return originals


def test_convert_trained_model_writes_a_loadable_folder(tmp_path):
    originals = write_upstream_folder(tmp_path / "upstream", PLAIN)
    result = upstream.convert_trained_model(tmp_path / "upstream", tmp_path / "converted")
    assert result.folds == (0, 1) and result.configuration == "3d_fullres"
    manifest = json.loads((tmp_path / "converted" / "conversion.json").read_text())
    assert manifest["schema_version"] == "nnunet-mlx.conversion.v1"
    assert [e["fold"] for e in manifest["folds"]] == [0, 1]
    for fold, weights in originals.items():
        directory = tmp_path / "converted" / f"fold_{fold}" / "checkpoint_final"
        state = ckpt.read_state(directory)
        assert state.identity.fold == fold and state.identity.trainer_name == "nnUNetTrainer"
        assert state.inference_allowed_mirroring_axes == (0, 1, 2)
        loaded = ckpt.read_weights(directory)
        assert set(loaded) == set(weights)
        for name, value in weights.items():
            np.testing.assert_array_equal(loaded[name], value)


def test_convert_trained_model_rejections(tmp_path):
    write_upstream_folder(tmp_path / "a", PLAIN, folds=(0,), trainer="nnUNetTrainerSomethingCustom")
    with pytest.raises(ContractError, match="not supported"):
        upstream.convert_trained_model(tmp_path / "a", tmp_path / "a_out")
    assert not (tmp_path / "a_out").exists()
    write_upstream_folder(tmp_path / "b", PLAIN, folds=(0,))
    (tmp_path / "exists").mkdir()
    with pytest.raises(ContractError, match="exists"):
        upstream.convert_trained_model(tmp_path / "b", tmp_path / "exists")
    # a checkpoint of another network does not fit the planned one
    write_upstream_folder(tmp_path / "c", PLAIN, folds=(0,))
    other = to_upstream(random_weights(RESENC, seed=1))
    torch.save({"network_weights": other, "trainer_name": "nnUNetTrainer",
                "init_args": {"configuration": "3d_fullres"},
                "inference_allowed_mirroring_axes": None, "current_epoch": 1},
               tmp_path / "c" / "fold_0" / "checkpoint_final.pth")
    with pytest.raises(ContractError, match="do not match"):
        upstream.convert_trained_model(tmp_path / "c", tmp_path / "c_out")
    assert not any(p.name.startswith(".c_out") for p in tmp_path.iterdir())
    assert upstream.detect_upstream_folds(tmp_path / "b") == (0,)


class _ConvNorm(torch.nn.Module):
    def __init__(self, cin, cout, kernel, stride, spec):
        super().__init__()
        self.conv = torch.nn.Conv3d(cin, cout, kernel, stride, tuple(k // 2 for k in kernel),
                                    bias=spec.conv_bias)
        self.norm = torch.nn.InstanceNorm3d(cout, eps=spec.norm_eps, affine=spec.norm_affine)
        self.slope = spec.leaky_slope

    def forward(self, x):
        return torch.nn.functional.leaky_relu(self.norm(self.conv(x)), self.slope)


class _Stage(torch.nn.Module):
    def __init__(self, blocks):
        super().__init__()
        self.convs = torch.nn.ModuleList(blocks)

    def forward(self, x):
        for block in self.convs:
            x = block(x)
        return x


class UpstreamPlainUNet(torch.nn.Module):
    """torch.nn modules named and laid out as upstream's PlainConvUNet, so its state dict
    is an upstream one and ``load_state_dict`` checks names and shapes."""

    def __init__(self, spec):
        super().__init__()
        f, k, s = spec.features, spec.kernel_sizes, spec.strides
        self.encoder = torch.nn.Module()
        cin, stages = spec.input_channels, []
        for i in range(len(f)):
            blocks = [_ConvNorm(cin if b == 0 else f[i], f[i], k[i], s[i] if b == 0 else 1, spec)
                      for b in range(spec.encoder_convs[i])]
            stages.append(torch.nn.Sequential(_Stage(blocks)))
            cin = f[i]
        self.encoder.stages = torch.nn.ModuleList(stages)
        self.decoder = torch.nn.Module()
        up, dec, seg = [], [], []
        for d in range(len(f) - 1):
            src, dst = len(f) - 1 - d, len(f) - 2 - d
            up.append(torch.nn.ConvTranspose3d(f[src], f[dst], s[src], s[src], bias=spec.conv_bias))
            dec.append(_Stage([_ConvNorm(2 * f[dst] if b == 0 else f[dst], f[dst], k[dst], 1, spec)
                               for b in range(spec.decoder_convs[d])]))
            seg.append(torch.nn.Conv3d(f[dst], spec.num_classes, 1, 1, 0, bias=True))
        self.decoder.transpconvs = torch.nn.ModuleList(up)
        self.decoder.stages = torch.nn.ModuleList(dec)
        self.decoder.seg_layers = torch.nn.ModuleList(seg)

    def forward(self, x):
        skips = []
        for stage in self.encoder.stages:
            x = stage(x)
            skips.append(x)
        x = skips.pop()
        for d in range(len(self.decoder.stages)):
            x = torch.cat((self.decoder.transpconvs[d](x), skips.pop()), 1)
            x = self.decoder.stages[d](x)
        return self.decoder.seg_layers[-1](x)


def test_converted_weights_compute_what_the_upstream_modules_compute():
    """An upstream state dict, converted, gives the oracle network the forward of the
    upstream torch modules it came from (a transposed operand or swapped name fails)."""
    from oracle.network import OracleNetwork

    torch.manual_seed(5)
    upstream_net = UpstreamPlainUNet(PLAIN).eval()
    with torch.no_grad():
        for p in upstream_net.parameters():
            p.copy_(torch.randn_like(p) * 0.3)
    state = upstream_net.state_dict()
    converted = upstream.convert_state_dict(state)
    assert set(converted.weights) == set(random_weights(PLAIN, seed=0))
    x = torch.randn(1, PLAIN.input_channels, 12, 16, 8)
    with torch.no_grad():
        want = upstream_net(x).permute(0, 2, 3, 4, 1).numpy()
    got = OracleNetwork(PLAIN, converted.weights)(x.permute(0, 2, 3, 4, 1).numpy())
    assert got.shape == want.shape
    np.testing.assert_allclose(got, want, rtol=1e-4, atol=1e-4)


class _ConvNormOnly(torch.nn.Module):
    """Upstream ConvDropoutNormReLU without its nonlinearity (conv, norm)."""

    def __init__(self, cin, cout, kernel, stride, spec, bias):
        super().__init__()
        self.conv = torch.nn.Conv3d(cin, cout, kernel, stride, tuple(k // 2 for k in kernel),
                                    bias=bias)
        self.norm = torch.nn.InstanceNorm3d(cout, eps=spec.norm_eps, affine=spec.norm_affine)

    def forward(self, x):
        return self.norm(self.conv(x))


class _UpstreamResidualBlock(torch.nn.Module):
    """Upstream BasicBlockD / BottleneckD: the branch, and ``skip`` = Sequential(AvgPool of
    the stride when it is not 1, bias-free 1x1 conv + norm when the channels change);
    LeakyReLU after the sum."""

    def __init__(self, cin, cout, kernel, stride, spec, bottleneck=None):
        super().__init__()
        stride = tuple(stride)
        self.slope = spec.leaky_slope
        if bottleneck is None:
            self.conv1 = _ConvNorm(cin, cout, kernel, stride, spec)
            self.conv2 = _ConvNormOnly(cout, cout, kernel, 1, spec, spec.conv_bias)
            self.branch = (self.conv1, self.conv2)
        else:
            self.conv1 = _ConvNorm(cin, bottleneck, (1, 1, 1), 1, spec)
            self.conv2 = _ConvNorm(bottleneck, bottleneck, kernel, stride, spec)
            self.conv3 = _ConvNormOnly(bottleneck, cout, (1, 1, 1), 1, spec, spec.conv_bias)
            self.branch = (self.conv1, self.conv2, self.conv3)
        ops = []
        if stride != (1, 1, 1):
            ops.append(torch.nn.AvgPool3d(stride, stride))
        if cin != cout:
            ops.append(_ConvNormOnly(cin, cout, (1, 1, 1), 1, spec, False))
        self.skip = torch.nn.Sequential(*ops) if ops else None

    def forward(self, x):
        residual = x if self.skip is None else self.skip(x)
        out = x
        for module in self.branch:
            out = module(out)
        return torch.nn.functional.leaky_relu(out + residual, self.slope)


class UpstreamResidualUNet(torch.nn.Module):
    """torch.nn modules named and laid out as upstream's ResidualEncoderUNet (stem,
    ``encoder.stages.<s>.blocks.<b>``, the plain decoder)."""

    def __init__(self, spec):
        super().__init__()
        f, k, s = spec.features, spec.kernel_sizes, spec.strides
        self.encoder = torch.nn.Module()
        stem_ch = spec.effective_stem_channels
        self.encoder.stem = _Stage([_ConvNorm(spec.input_channels, stem_ch, k[0], 1, spec)])
        cin, stages = stem_ch, []
        for i in range(len(f)):
            bottleneck = None if spec.bottleneck_channels is None else spec.bottleneck_channels[i]
            stage = torch.nn.Module()
            stage.blocks = torch.nn.Sequential(*[
                _UpstreamResidualBlock(cin if b == 0 else f[i], f[i], k[i],
                                       s[i] if b == 0 else (1, 1, 1), spec, bottleneck)
                for b in range(spec.encoder_blocks[i])])
            stages.append(stage)
            cin = f[i]
        self.encoder.stages = torch.nn.ModuleList(stages)
        self.decoder = torch.nn.Module()
        up, dec, seg = [], [], []
        for d in range(len(f) - 1):
            src, dst = len(f) - 1 - d, len(f) - 2 - d
            up.append(torch.nn.ConvTranspose3d(f[src], f[dst], s[src], s[src], bias=spec.conv_bias))
            dec.append(_Stage([_ConvNorm(2 * f[dst] if b == 0 else f[dst], f[dst], k[dst], 1, spec)
                               for b in range(spec.decoder_convs[d])]))
            seg.append(torch.nn.Conv3d(f[dst], spec.num_classes, 1, 1, 0, bias=True))
        self.decoder.transpconvs = torch.nn.ModuleList(up)
        self.decoder.stages = torch.nn.ModuleList(dec)
        self.decoder.seg_layers = torch.nn.ModuleList(seg)

    def forward(self, x):
        x = self.encoder.stem(x)
        skips = []
        for stage in self.encoder.stages:
            x = stage.blocks(x)
            skips.append(x)
        x = skips.pop()
        for d in range(len(self.decoder.stages)):
            x = torch.cat((self.decoder.transpconvs[d](x), skips.pop()), 1)
            x = self.decoder.stages[d](x)
        return self.decoder.seg_layers[-1](x)


RESIDUAL_NETS = {
    "basic": ResidualEncoderUNetSpec(2, 3, (4, 8, 16), K3 * 3, ((1, 1, 1), (2, 2, 2), (1, 2, 2)),
                                     (1, 2, 2), (1, 1), stem_channels=6),
    "bottleneck": ResidualEncoderUNetSpec(1, 2, (4, 8, 8), K3 * 3,
                                          ((1, 1, 1), (2, 2, 2), (2, 2, 2)), (2, 1, 2), (1, 1),
                                          bottleneck_channels=(2, 3, 4)),
}


@pytest.mark.parametrize("name", sorted(RESIDUAL_NETS))
def test_converted_residual_weights_compute_what_the_upstream_modules_compute(name):
    """An upstream residual-encoder state dict (stem, blocks with conv1/conv2[/conv3] and
    skip.<i>), converted, gives the oracle's residual path the upstream modules' forward."""
    from oracle.network import OracleNetwork

    spec = RESIDUAL_NETS[name]
    torch.manual_seed(11)
    upstream_net = UpstreamResidualUNet(spec).eval()
    with torch.no_grad():
        for p in upstream_net.parameters():
            p.copy_(torch.randn_like(p) * 0.3)
    state = upstream_net.state_dict()
    assert any(".skip.1.conv.weight" in key for key in state) or name == "bottleneck"
    converted = upstream.convert_state_dict(state)
    assert set(converted.weights) == set(random_weights(spec, seed=0))
    x = torch.randn(1, spec.input_channels, 8, 16, 12)
    with torch.no_grad():
        want = upstream_net(x).permute(0, 2, 3, 4, 1).numpy()
    got = OracleNetwork(spec, converted.weights, residual=True)(x.permute(0, 2, 3, 4, 1).numpy())
    assert got.shape == want.shape
    np.testing.assert_allclose(got, want, rtol=1e-4, atol=1e-4)


@pytest.mark.gpu
def test_converted_folder_runs_on_the_device(tmp_path):
    """A converted folder loads through the model-folder path and its resident fold gives
    the upstream modules' logits (float32 bar)."""
    from nnunet_mlx.model.folder import load_model_bundle

    torch.manual_seed(9)
    upstream_net = UpstreamPlainUNet(PLAIN).eval()
    with torch.no_grad():
        for p in upstream_net.parameters():
            p.copy_(torch.randn_like(p) * 0.3)
    root = tmp_path / "upstream"
    write_upstream_folder(root, PLAIN, folds=(0,))
    torch.save({"network_weights": upstream_net.state_dict(), "trainer_name": "nnUNetTrainer",
                "init_args": {"configuration": "3d_fullres"},
                "inference_allowed_mirroring_axes": (0, 1, 2), "current_epoch": 1},
               root / "fold_0" / "checkpoint_final.pth")
    upstream.convert_trained_model(root, tmp_path / "converted")
    print("converted folder: loading fold 0 on the device", flush=True)
    bundle = load_model_bundle(tmp_path / "converted", configuration="3d_fullres")
    x = torch.randn(2, PLAIN.input_channels, 16, 16, 16)
    with torch.no_grad():
        want = upstream_net(x).permute(0, 2, 3, 4, 1).numpy()
    got = bundle.models[0](x.permute(0, 2, 3, 4, 1).contiguous().cuda()).cpu().numpy()
    assert got.shape == want.shape
    assert np.abs(got - want).max() <= 1e-3
    assert bundle.mirroring_axes == (0, 1, 2) and bundle.folds == (0,)
    for model in bundle.models:
        model.close()


def test_resolve_results_folder(tmp_path, monkeypatch):
    model = tmp_path / "Dataset003_Liver" / "nnUNetTrainer__nnUNetPlans__3d_fullres"
    model.mkdir(parents=True)
    assert upstream.resolve_results_folder("3", configuration="3d_fullres", results=tmp_path) == model
    monkeypatch.setenv("nnUNet_results", str(tmp_path))
    assert upstream.resolve_results_folder("Dataset003_Liver", configuration="3d_fullres") == model
    with pytest.raises(ContractError, match="does not exist"):
        upstream.resolve_results_folder("3", configuration="2d")
    (tmp_path / "Dataset003_Other").mkdir()
    with pytest.raises(ContractError, match="expected one"):
        upstream.resolve_results_folder("3", configuration="3d_fullres")
    monkeypatch.delenv("nnUNet_results")
    with pytest.raises(ContractError, match="nnUNet_results"):
        upstream.resolve_results_folder("3", configuration="3d_fullres")


def test_cached_conversion_reuses_and_rebuilds(tmp_path):
    import os

    source = tmp_path / "results" / "Dataset003_Liver" / "nnUNetTrainer__nnUNetPlans__3d_fullres"
    source.parent.mkdir(parents=True)
    write_upstream_folder(source, PLAIN, folds=(0, 1))
    cache = tmp_path / "cache"
    entry = upstream.cached_conversion(source, folds=(1,), cache=cache)
    assert entry == cache / "converted" / "Dataset003_Liver" / source.name
    weights = entry / "fold_0" / "checkpoint_final" / "weights.safetensors"
    assert weights.is_file()          # every available fold is converted
    stamp = weights.stat().st_mtime_ns
    marker = (entry / ".source").read_text()
    assert upstream.cached_conversion(source, cache=cache) == entry
    assert weights.stat().st_mtime_ns == stamp and (entry / ".source").read_text() == marker
    # a retrained fold (new modification time) makes the entry stale
    ckpt_path = source / "fold_1" / "checkpoint_final.pth"
    st = ckpt_path.stat()
    os.utime(ckpt_path, ns=(st.st_atime_ns, st.st_mtime_ns + 10**9))
    assert not upstream.conversion_is_current(entry, source, (0, 1), "checkpoint_final.pth")
    upstream.cached_conversion(source, cache=cache)
    assert upstream.conversion_is_current(entry, source, (0, 1), "checkpoint_final.pth")
    # so does edited plans JSON, and a missing payload file
    plans = json.loads((source / "plans.json").read_text())
    plans["plans_name"] = "edited"
    (source / "plans.json").write_text(json.dumps(plans))
    assert not upstream.conversion_is_current(entry, source, (0, 1), "checkpoint_final.pth")
    upstream.cached_conversion(source, cache=cache)
    assert json.loads((entry / "plans.json").read_text())["plans_name"] == "edited"
    (entry / "fold_0" / "checkpoint_final" / "state.json").unlink()
    assert not upstream.conversion_is_current(entry, source, (0, 1), "checkpoint_final.pth")
    with pytest.raises(ContractError, match="have no"):
        upstream.cached_conversion(source, folds=(4,), cache=cache)
    # a symlinked entry is refused rather than deleted through
    elsewhere = tmp_path / "elsewhere"
    elsewhere.mkdir()
    os.symlink(elsewhere, cache / "converted" / "Dataset003_Liver" / "linked")
    linked_source = source.parent / "linked"
    write_upstream_folder(linked_source, PLAIN, folds=(0,))
    with pytest.raises(ContractError, match="symlink"):
        upstream.cached_conversion(linked_source, cache=cache)
    assert elsewhere.is_dir()
