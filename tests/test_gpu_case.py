"""Raw case -> label image on the GPU against the oracle composition of the same steps.

The oracle chain: nonzero crop, CT normalisation and spline resampling
(``oracle.preprocess``; Torch-grid plans: ``oracle.torch_resample``), the float32 network
(``oracle.network``) under the sliding window with float16 accumulation
(``oracle.sliding_window``), spline restoration with the first-maximum argmax
(``oracle.restore``; Torch-grid plans: the Torch-grid resampler and argmax), then uncrop.  The device path differs from it
only by float32 summation order inside the network, so labels may differ where two classes
are within a rounding of each other: the bar is 99.9 % identical voxels, identical outside
the crop box.
"""

from __future__ import annotations

import json

import numpy as np
import pytest
import torch

from nnunet_mlx.model.topology import PlainConvUNetSpec
from nnunet_mlx.storage import nifti
from nnunet_mlx.storage.synthetic import random_weights, write_random_model_folder
from oracle import preprocess as op
from oracle import sliding_window as osw
from oracle.network import OracleNetwork
from oracle.restore import restore_labels_spline

pytestmark = pytest.mark.gpu

SPEC = PlainConvUNetSpec(1, 3, (8, 16), ((3, 3, 3),) * 2, ((1, 1, 1), (2, 2, 2)), (2, 2), (2,))
PATCH = (16, 32, 32)
CT = {"mean": 60.0, "std": 80.0, "percentile_00_5": -150.0, "percentile_99_5": 250.0}
TARGET_SPACING = (2.0, 0.8, 0.8)
IMAGE_SPACING_XYZ = (0.9, 0.9, 3.0)


def ct_model_folder(root, seeds=(0,)):
    folder = write_random_model_folder(root, SPEC, patch_size=PATCH, seeds=seeds,
                                       random_affine=False, labels=("liver", "tumor"))
    plans = json.loads((folder / "plans.json").read_text())
    cfg = plans["configurations"]["3d_fullres"]
    cfg["spacing"] = list(TARGET_SPACING)
    cfg["normalization_schemes"] = ["CTNormalization"]
    plans["foreground_intensity_properties_per_channel"] = {"0": dict(CT)}
    (folder / "plans.json").write_text(json.dumps(plans))
    return folder


def synthetic_ct(path, seed):
    """(Z, Y, X) int16 CT with air outside a body box and two bright ellipsoids."""
    rng = np.random.default_rng(seed)
    z, y, x = np.mgrid[0:12, 0:40, 0:36]
    ct = np.zeros((12, 40, 36), dtype=np.int16)
    body = (y >= 4) & (y < 37) & (x >= 3) & (x < 33)
    ct[body] = (rng.standard_normal(body.sum()) * 40 + 30).astype(np.int16)
    blob = ((z - 6) / 4.0) ** 2 + ((y - 18) / 9.0) ** 2 + ((x - 14) / 7.0) ** 2 < 1
    ct[blob] = (rng.standard_normal(blob.sum()) * 20 + 160).astype(np.int16)
    nifti.write_nifti(path, ct, IMAGE_SPACING_XYZ)
    return ct


def oracle_case_labels(ct_zyx, seeds=(0,)):
    """The oracle chain for a one-channel CT on the (Z, Y, X) grid, identity transpose."""
    raw = ct_zyx.astype(np.float32)[None]
    bbox = op.nonzero_bbox(raw)
    crop = raw[(slice(None), *(slice(a, b) for a, b in bbox))]
    norm = op.ct_normalize(crop[0], CT["mean"], CT["std"], CT["percentile_00_5"],
                           CT["percentile_99_5"])[None]
    original = tuple(reversed(IMAGE_SPACING_XYZ))
    new_shape = tuple(round(o / n * s) for o, n, s in zip(original, TARGET_SPACING, crop.shape[1:]))
    data = op.resample_data(norm, new_shape, separate_axis=0)
    nets = [OracleNetwork(SPEC, random_weights(SPEC, s)) for s in seeds]
    logits, _ = osw.predict(nets, data, PATCH, num_classes=3, axes=(0, 1, 2),
                            step_fraction=0.5, accumulation="nnunet-fp16")
    labels, _ = restore_labels_spline(logits, crop.shape[1:], order=1, separate_axis=0)
    full = np.zeros(ct_zyx.shape, dtype=np.uint16)
    full[tuple(slice(a, b) for a, b in bbox)] = labels
    return full, bbox


def test_run_writes_the_oracle_labels(tmp_path):
    import nnunet_mlx

    folder = ct_model_folder(tmp_path / "model")
    ct = synthetic_ct(tmp_path / "case_0000.nii.gz", seed=3)
    print("raw case: run() on a 12x40x36 CT, separate-z plans", flush=True)
    result = nnunet_mlx.run(weights_path=folder, image_paths=[tmp_path / "case_0000.nii.gz"],
                            output_dir=tmp_path / "out")
    mask = nifti.read_nifti(result["outputs"]["mask"])
    want, bbox = oracle_case_labels(ct)
    assert mask.array.shape == ct.shape and mask.array.dtype == np.uint8
    assert mask.spacing == pytest.approx(IMAGE_SPACING_XYZ)
    agree = (mask.array == want).mean()
    print(f"label agreement {agree:.6f}, classes {np.bincount(want.ravel(), minlength=3)}",
          flush=True)
    assert agree >= 0.999
    outside = np.ones(ct.shape, dtype=bool)
    outside[tuple(slice(a, b) for a, b in bbox)] = False
    assert (mask.array[outside] == 0).all()
    details = result["details"]
    assert details["accumulation"] == "nnunet-fp16" and details["folds"] == [0]
    assert details["preprocessed_shape"][1:] == [18, 37, 34]
    assert result["artifacts"]["mask"]["labels"][1]["name"] == "liver"


TORCH_KWARGS = {"is_seg": False, "force_separate_z": None, "memefficient_seg_resampling": False}


def test_run_with_torch_grid_plans(tmp_path):
    """Plans with upstream's Torch-grid resampler for the image and the probabilities
    (linear in plane, nearest-exact along the separate axis): the device case path against
    the oracle chain with oracle.torch_resample in both places."""
    import nnunet_mlx
    from nnunet_mlx.data.resampling import separate_z_axis
    from oracle import torch_resample as otr

    folder = ct_model_folder(tmp_path / "model")
    plans = json.loads((folder / "plans.json").read_text())
    cfg = plans["configurations"]["3d_fullres"]
    for field in ("resampling_fn_data", "resampling_fn_probabilities"):
        cfg[field] = "resample_torch_fornnunet"
        cfg[f"{field}_kwargs"] = dict(TORCH_KWARGS)
    (folder / "plans.json").write_text(json.dumps(plans))
    ct = synthetic_ct(tmp_path / "case_0000.nii.gz", seed=5)
    print("raw case: run() on a 12x40x36 CT, Torch-grid plans", flush=True)
    result = nnunet_mlx.run(weights_path=folder, image_paths=[tmp_path / "case_0000.nii.gz"],
                            output_dir=tmp_path / "out")
    mask = nifti.read_nifti(result["outputs"]["mask"])

    raw = ct.astype(np.float32)[None]
    bbox = op.nonzero_bbox(raw)
    crop = raw[(slice(None), *(slice(a, b) for a, b in bbox))]
    norm = op.ct_normalize(crop[0], CT["mean"], CT["std"], CT["percentile_00_5"],
                           CT["percentile_99_5"])[None]
    original = tuple(reversed(IMAGE_SPACING_XYZ))
    new_shape = tuple(round(o / n * s) for o, n, s in zip(original, TARGET_SPACING, crop.shape[1:]))
    _, axis = separate_z_axis(original, TARGET_SPACING, force=None)
    data = otr.resample(norm, new_shape, axis=axis)
    nets = [OracleNetwork(SPEC, random_weights(SPEC, 0))]
    logits, _ = osw.predict(nets, data, PATCH, num_classes=3, axes=(0, 1, 2),
                            step_fraction=0.5, accumulation="nnunet-fp16")
    _, back_axis = separate_z_axis(TARGET_SPACING, original, force=None)
    values = otr.resample(np.moveaxis(np.asarray(logits, dtype=np.float32), -1, 0),
                          crop.shape[1:], axis=back_axis)
    want = np.zeros(ct.shape, dtype=np.uint16)
    want[tuple(slice(a, b) for a, b in bbox)] = values.argmax(axis=0)
    assert result["details"]["preprocessed_shape"][1:] == list(new_shape)
    agree = (mask.array == want).mean()
    print(f"label agreement {agree:.6f}, classes {np.bincount(want.ravel(), minlength=3)}, "
          f"axes {axis}/{back_axis}", flush=True)
    assert agree >= 0.999
    outside = np.ones(ct.shape, dtype=bool)
    outside[tuple(slice(a, b) for a, b in bbox)] = False
    assert (mask.array[outside] == 0).all()


def test_loaded_model_and_named_model_agree_with_run(tmp_path):
    from nnunet_mlx import medmlx
    from nnunet_mlx.named_models import liver

    folder = ct_model_folder(tmp_path / "model", seeds=(0, 1))
    synthetic_ct(tmp_path / "a.nii.gz", seed=4)
    synthetic_ct(tmp_path / "b.nii.gz", seed=5)
    print("raw case: two folds, loaded model over two cases", flush=True)
    first = medmlx.run(weights_path=folder, image_paths=[tmp_path / "a.nii.gz"],
                       output_dir=tmp_path / "run_a")
    with liver.load_model(weights_path=folder) as model:
        again = model.run(image_path=tmp_path / "a.nii.gz", output_dir=tmp_path / "model_a")
        other = model.run(image_path=tmp_path / "b.nii.gz", output_dir=tmp_path / "model_b")
        with pytest.raises(Exception, match="exists"):
            model.run(image_path=tmp_path / "a.nii.gz", output_dir=tmp_path / "model_a")
    a1 = nifti.read_nifti(first["outputs"]["mask"]).array
    a2 = nifti.read_nifti(again["outputs"]["mask"]).array
    np.testing.assert_array_equal(a1, a2)
    assert other["details"]["folds"] == [0, 1]
    named = liver.run(image_path=tmp_path / "b.nii.gz", output_dir=tmp_path / "named_b",
                      weights_path=folder)
    np.testing.assert_array_equal(nifti.read_nifti(named["outputs"]["mask"]).array,
                                  nifti.read_nifti(other["outputs"]["mask"]).array)
    with pytest.raises(RuntimeError, match="closed"):
        model.run(image_path=tmp_path / "b.nii.gz", output_dir=tmp_path / "closed")


@pytest.mark.parametrize("changed", ["plans.json", "fold_0/checkpoint_final/weights.safetensors"])
def test_loaded_model_rejects_changed_sources_and_a_reload_picks_them_up(tmp_path, changed):
    """A loaded model refuses to run once a file it was built from has been touched
    (src/nnunet_mlx/medmlx.py:534,565; tests/test_medmlx.py:369-391); loading again
    serves the folder as it now is."""
    import os

    from nnunet_mlx import medmlx
    from nnunet_mlx.errors import ContractError

    folder = ct_model_folder(tmp_path / "model")
    synthetic_ct(tmp_path / "a.nii.gz", seed=4)
    print(f"raw case: loaded model, then {changed} touched", flush=True)
    with medmlx.load_model(weights_path=folder) as model:
        model.run(image_paths=[tmp_path / "a.nii.gz"], output_dir=tmp_path / "before")
        target = folder / changed
        st = target.stat()
        os.utime(target, ns=(st.st_atime_ns, st.st_mtime_ns + 1_000_000_000))
        with pytest.raises(ContractError, match="changed"):
            model.run(image_paths=[tmp_path / "a.nii.gz"], output_dir=tmp_path / "stale")
    assert not (tmp_path / "stale").exists() or not any((tmp_path / "stale").iterdir())
    with medmlx.load_model(weights_path=folder) as model:
        result = model.run(image_paths=[tmp_path / "a.nii.gz"], output_dir=tmp_path / "fresh")
    assert (tmp_path / "fresh").is_dir() and nifti.read_nifti(result["outputs"]["mask"]).array.size


def test_cli_predicts_an_upstream_folder(tmp_path, monkeypatch):
    """``nnunet-mlx predict -m`` converts an upstream results folder (cached) and predicts
    the input folder; the labels equal run() on the converted folder."""
    from nnunet_mlx import medmlx
    from nnunet_mlx.cli import main
    from tests.test_upstream_conversion import to_upstream

    folder = ct_model_folder(tmp_path / "model")
    upstream = tmp_path / "results" / "Dataset001_Ct" / "nnUNetTrainer__nnUNetPlans__3d_fullres"
    (upstream / "fold_0").mkdir(parents=True)
    for name in ("plans.json", "dataset.json"):
        (upstream / name).write_text((folder / name).read_text())
    torch.save({"network_weights": to_upstream(random_weights(SPEC, 0)),
                "trainer_name": "nnUNetTrainer", "init_args": {"configuration": "3d_fullres"},
                "inference_allowed_mirroring_axes": (0, 1, 2), "current_epoch": 1000},
               upstream / "fold_0" / "checkpoint_final.pth")
    (tmp_path / "in").mkdir()
    synthetic_ct(tmp_path / "in" / "c1_0000.nii.gz", seed=6)
    synthetic_ct(tmp_path / "in" / "c2_0000.nii.gz", seed=7)
    monkeypatch.setenv("NNUNET_MLX_CACHE", str(tmp_path / "cache"))
    print("raw case: CLI predict -d over an upstream results folder", flush=True)
    monkeypatch.setenv("nnUNet_results", str(tmp_path / "results"))
    assert main(["predict", "-i", str(tmp_path / "in"), "-o", str(tmp_path / "out"), "-d", "1",
                 "-c", "3d_fullres", "-f", "0"]) == 0
    for case in ("c1", "c2"):   # cases read, predicted and written in overlapped order
        got = nifti.read_nifti(tmp_path / "out" / f"{case}.nii.gz").array
        ref = medmlx.run(weights_path=folder, image_paths=[tmp_path / "in" / f"{case}_0000.nii.gz"],
                         output_dir=tmp_path / f"ref_{case}")
        np.testing.assert_array_equal(got, nifti.read_nifti(ref["outputs"]["mask"]).array)
    # the installed console script, as a separate process: it reuses the conversion and
    # skips the finished case, then predicts a third case to another folder
    import os
    import subprocess

    from tests.helpers import install_package

    bin_dir = install_package(tmp_path / "site")
    env = dict(os.environ, PYTHONPATH=str(tmp_path / "site"))
    synthetic_ct(tmp_path / "in" / "c3_0000.nii.gz", seed=8)
    print("raw case: installed nnunet-mlx predict as a subprocess", flush=True)
    out = subprocess.run([str(bin_dir / "nnunet-mlx"), "predict", "-i", str(tmp_path / "in"),
                          "-o", str(tmp_path / "out"), "-d", "1", "-c", "3d_fullres", "-f", "0",
                          "--continue_prediction", "--json"], env=env, capture_output=True,
                         text=True, timeout=300)
    assert out.returncode == 0, out.stderr
    predicted = json.loads(out.stdout.strip().splitlines()[-1])["predicted"]
    assert any(p.endswith("c3.nii.gz") for p in predicted), predicted
    assert not any(p.endswith(("c1.nii.gz", "c2.nii.gz")) for p in predicted), predicted
    got = nifti.read_nifti(tmp_path / "out" / "c3.nii.gz").array
    ref = medmlx.run(weights_path=folder, image_paths=[tmp_path / "in" / "c3_0000.nii.gz"],
                     output_dir=tmp_path / "ref_c3")
    np.testing.assert_array_equal(got, nifti.read_nifti(ref["outputs"]["mask"]).array)


def test_brats_style_mri_case(tmp_path):
    """Four MRI channels, z-score normalisation inside the filled nonzero mask, isotropic
    1 mm plans, the five-fold ensemble the named BraTS entry runs: against the oracle chain."""
    from nnunet_mlx.named_models import brats

    spec = PlainConvUNetSpec(4, 5, (8, 16), ((3, 3, 3),) * 2, ((1, 1, 1), (2, 2, 2)), (2, 2), (2,))
    folder = write_random_model_folder(tmp_path / "model", spec, patch_size=(16, 24, 24),
                                       seeds=tuple(range(5)),
                                       labels=("edema", "nonenh", "empty", "enh"))
    plans = json.loads((folder / "plans.json").read_text())
    cfg = plans["configurations"]["3d_fullres"]
    cfg["use_mask_for_norm"] = [True] * 4
    cfg["spacing"] = [1.0, 1.0, 1.0]
    (folder / "plans.json").write_text(json.dumps(plans))
    rng = np.random.default_rng(12)
    z, y, x = np.mgrid[0:20, 0:30, 0:28]
    head = ((z - 10) / 8.0) ** 2 + ((y - 15) / 12.0) ** 2 + ((x - 14) / 11.0) ** 2 < 1
    ventricle = ((z - 10) / 2.0) ** 2 + ((y - 15) / 3.0) ** 2 + ((x - 14) / 3.0) ** 2 < 1
    images, channels = {}, []
    for c, name in enumerate(brats.CHANNELS):
        vol = np.zeros((20, 30, 28), dtype=np.float32)
        vol[head] = (rng.standard_normal(int(head.sum())) * 100 + 400 + 50 * c).astype(np.float32)
        vol[ventricle] = 0.0                       # a sealed zero cavity: inside the mask
        nifti.write_nifti(tmp_path / f"{name}.nii.gz", vol, (1.0, 1.0, 1.0))
        images[name] = tmp_path / f"{name}.nii.gz"
        channels.append(vol)
    print("raw case: BraTS-style 4-channel MRI, masked z-score", flush=True)
    result = brats.run(image_paths=images, output_dir=tmp_path / "out", weights_path=folder)
    mask = nifti.read_nifti(result["outputs"]["mask"]).array
    raw = np.stack(channels)
    bbox = op.nonzero_bbox(raw)
    sl = tuple(slice(a, b) for a, b in bbox)
    filled = op.filled_nonzero_mask(raw)[sl]
    assert filled.sum() > np.any(raw != 0, axis=0)[sl].sum()   # the cavity is filled
    data = np.stack([op.zscore_normalize(raw[c][sl], filled) for c in range(4)])
    nets = [OracleNetwork(spec, random_weights(spec, s)) for s in range(5)]
    logits, _ = osw.predict(nets, data, (16, 24, 24), num_classes=5, axes=(0, 1, 2),
                            step_fraction=0.5, accumulation="nnunet-fp16")
    labels = np.argmax(logits, axis=-1)
    want = np.zeros(raw.shape[1:], dtype=np.uint16)
    want[sl] = labels
    agree = (mask == want).mean()
    print(f"label agreement {agree:.6f}, classes {np.bincount(want.ravel(), minlength=5)}",
          flush=True)
    assert agree >= 0.999
    assert result["details"]["folds"] == [0, 1, 2, 3, 4]
