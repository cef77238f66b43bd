"""Host side of the raw-case path: NIfTI-1 reading/writing in SimpleITK's array layout,
case grouping, uncropping and the argument checks of the public API and the CLI."""

from __future__ import annotations

import gzip
import struct

import numpy as np
import pytest

from nnunet_mlx.errors import ContractError
from nnunet_mlx.storage import nifti


def handmade_nifti(path, values_xyz: np.ndarray, code: int, spacing, *, slope=1.0, inter=0.0,
                   endian="<", sform=None):
    """A NIfTI-1 file assembled field by field from the format specification (independent
    of the module's writer): voxels stored with x fastest."""
    header = bytearray(348)
    struct.pack_into(endian + "i", header, 0, 348)
    dims = values_xyz.shape
    struct.pack_into(endian + "8h", header, 40, len(dims), *dims, *([1] * (7 - len(dims))))
    struct.pack_into(endian + "2h", header, 70, code, values_xyz.dtype.itemsize * 8)
    struct.pack_into(endian + "8f", header, 76, 1.0, *spacing, *([1.0] * (7 - len(spacing))))
    struct.pack_into(endian + "f", header, 108, 352.0)
    struct.pack_into(endian + "2f", header, 112, slope, inter)
    if sform is not None:
        struct.pack_into(endian + "h", header, 254, 1)
        struct.pack_into(endian + "12f", header, 280, *np.asarray(sform, dtype=np.float32).ravel())
    header[344:348] = b"n+1\0"
    body = values_xyz.astype(values_xyz.dtype.newbyteorder(endian)).tobytes(order="F")
    payload = bytes(header) + b"\0" * 4 + body
    if str(path).endswith(".gz"):
        with gzip.open(path, "wb") as handle:
            handle.write(payload)
    else:
        path.write_bytes(payload)


def test_reader_layout_matches_simpleitk_arrays(tmp_path):
    """array[z, y, x] == voxel (x, y, z); spacing in (x, y, z) order."""
    rng = np.random.default_rng(0)
    xyz = rng.integers(-1000, 1000, size=(5, 4, 3)).astype(np.int16)
    handmade_nifti(tmp_path / "a.nii.gz", xyz, 4, (0.7, 0.8, 2.5))
    image = nifti.read_nifti(tmp_path / "a.nii.gz")
    assert image.array.shape == (3, 4, 5) and image.array.dtype == np.int16
    assert image.array[2, 1, 4] == xyz[4, 1, 2]
    np.testing.assert_array_equal(image.array, xyz.transpose(2, 1, 0))
    assert image.spacing == pytest.approx((0.7, 0.8, 2.5))


@pytest.mark.parametrize("endian", ["<", ">"])
def test_reader_scaling_and_byte_order(tmp_path, endian):
    xyz = np.arange(24, dtype=np.uint16).reshape(4, 3, 2)
    handmade_nifti(tmp_path / "s.nii", xyz, 512, (1.0, 1.0, 1.0), slope=0.5, inter=-1024.0,
                   endian=endian)
    image = nifti.read_nifti(tmp_path / "s.nii")
    assert image.array.dtype == np.float32
    np.testing.assert_array_equal(image.array, (xyz.transpose(2, 1, 0) * 0.5 - 1024).astype(np.float32))


def test_reader_rejects_bad_files(tmp_path):
    (tmp_path / "x.nii").write_bytes(b"\0" * 400)
    with pytest.raises(ContractError, match="348"):
        nifti.read_nifti(tmp_path / "x.nii")
    xyz = np.zeros((4, 4, 4), dtype=np.float32)
    handmade_nifti(tmp_path / "t.nii", xyz, 16, (1, 1, 1))
    raw = (tmp_path / "t.nii").read_bytes()
    (tmp_path / "t.nii").write_bytes(raw[:-10])
    with pytest.raises(ContractError, match="truncated"):
        nifti.read_nifti(tmp_path / "t.nii")
    with pytest.raises(ContractError, match="NIfTI"):
        nifti.read_nifti(tmp_path / "t.mha")
    handmade_nifti(tmp_path / "c.nii", xyz.astype(np.complex64).real.astype(np.float32), 32, (1, 1, 1))
    with pytest.raises(ContractError, match="datatype"):
        nifti.read_nifti(tmp_path / "c.nii")


def test_read_images_stacks_channels_and_reverses_spacing(tmp_path):
    rng = np.random.default_rng(1)
    a = rng.standard_normal((6, 5, 4)).astype(np.float32)
    b = rng.standard_normal((6, 5, 4)).astype(np.float32)
    handmade_nifti(tmp_path / "c_0000.nii.gz", a, 16, (0.8, 0.9, 3.0))
    handmade_nifti(tmp_path / "c_0001.nii.gz", b, 16, (0.8, 0.9, 3.0))
    data, props = nifti.read_images([tmp_path / "c_0000.nii.gz", tmp_path / "c_0001.nii.gz"])
    assert data.shape == (2, 4, 5, 6) and data.dtype == np.float32
    np.testing.assert_array_equal(data[1], b.transpose(2, 1, 0))
    assert props["spacing"] == pytest.approx((3.0, 0.9, 0.8))
    handmade_nifti(tmp_path / "d_0001.nii.gz", b, 16, (0.8, 0.9, 2.0))
    with pytest.raises(ContractError, match="spacing"):
        nifti.read_images([tmp_path / "c_0000.nii.gz", tmp_path / "d_0001.nii.gz"])
    handmade_nifti(tmp_path / "e.nii", a[:, :, 0], 16, (0.5, 0.25))
    data, props = nifti.read_images([tmp_path / "e.nii"])
    assert data.shape == (1, 1, 5, 6) and props["spacing"] == pytest.approx((999 * 0.5, 0.25, 0.5))


def test_write_segmentation_keeps_the_input_geometry(tmp_path):
    sform = [[-0.8, 0, 0, 10.5], [0, 0.9, 0, -3.0], [0, 0, 3.0, 7.25]]
    xyz = np.zeros((6, 5, 4), dtype=np.int16)
    handmade_nifti(tmp_path / "img.nii.gz", xyz, 4, (0.8, 0.9, 3.0), sform=sform)
    _, props = nifti.read_images([tmp_path / "img.nii.gz"])
    labels = np.zeros((4, 5, 6), dtype=np.uint16)
    labels[1, 2, 3] = 2
    nifti.write_segmentation(labels, tmp_path / "mask.nii.gz", props, overwrite=False)
    out = nifti.read_nifti(tmp_path / "mask.nii.gz")
    assert out.array.dtype == np.uint8 and out.array[1, 2, 3] == 2 and out.array.sum() == 2
    assert out.spacing == pytest.approx((0.8, 0.9, 3.0))
    np.testing.assert_allclose(out.affine[:3], np.asarray(sform), rtol=0, atol=1e-6)
    labels[0, 0, 0] = 300
    nifti.write_segmentation(labels, tmp_path / "mask.nii.gz", props, overwrite=True)
    assert nifti.read_nifti(tmp_path / "mask.nii.gz").array.dtype == np.uint16
    with pytest.raises(ContractError, match="exists"):
        nifti.write_segmentation(labels, tmp_path / "mask.nii.gz", props, overwrite=False)
    with pytest.raises(ContractError):
        nifti.write_segmentation(labels.astype(np.float32), tmp_path / "m2.nii", props,
                                 overwrite=False)


def test_writer_round_trip(tmp_path):
    values = np.random.default_rng(2).integers(-2000, 2000, size=(7, 9, 8)).astype(np.int16)
    nifti.write_nifti(tmp_path / "ct.nii.gz", values, (0.7, 0.7, 2.5))
    image = nifti.read_nifti(tmp_path / "ct.nii.gz")
    np.testing.assert_array_equal(image.array, values)
    assert image.spacing == pytest.approx((0.7, 0.7, 2.5))


def test_uncrop_and_case_grouping(tmp_path):
    from nnunet_mlx.prediction.pipeline import case_files, uncrop_segmentation

    cropped = np.arange(1, 1 + 2 * 3 * 4, dtype=np.uint16).reshape(2, 3, 4)
    out = uncrop_segmentation(cropped, (5, 6, 7), [(1, 3), (2, 5), (3, 7)], (1, 2, 0))
    full = np.zeros((5, 6, 7), dtype=np.uint16)
    full[1:3, 2:5, 3:7] = cropped
    np.testing.assert_array_equal(out, full.transpose(1, 2, 0))
    with pytest.raises(ContractError):
        uncrop_segmentation(cropped, (5, 6, 7), [(1, 3), (2, 5), (3, 6)], (0, 1, 2))
    for name in ("a_0000.nii.gz", "a_0001.nii.gz", "b_0000.nii.gz", "b_0001.nii.gz", "notes.txt"):
        (tmp_path / name).write_bytes(b"")
    cases = case_files(tmp_path, ".nii.gz", 2)
    assert list(cases) == ["a", "b"] and cases["b"][1].name == "b_0001.nii.gz"
    (tmp_path / "c_0000.nii.gz").write_bytes(b"")
    with pytest.raises(ContractError, match="case c"):
        case_files(tmp_path, ".nii.gz", 2)


def test_public_api_argument_checks(tmp_path):
    from nnunet_mlx import medmlx
    from nnunet_mlx.named_models import brats, liver

    image = tmp_path / "ct.nii.gz"
    nifti.write_nifti(image, np.zeros((4, 4, 4), dtype=np.int16), (1, 1, 1))
    with pytest.raises(ContractError, match="non-empty list"):
        medmlx.check_request(str(image), output_dir=tmp_path / "o")
    with pytest.raises(ContractError, match="Missing"):
        medmlx.check_request([tmp_path / "nope.nii.gz"], output_dir=tmp_path / "o")
    with pytest.raises(ContractError, match="step_fraction"):
        medmlx.check_request([image], output_dir=tmp_path / "o", step_fraction=0)
    with pytest.raises(ContractError, match="boolean"):
        medmlx.check_request([image], output_dir=tmp_path / "o", use_mirroring=1)
    with pytest.raises(ContractError, match="probability"):
        medmlx.check_request([image], output_dir=tmp_path / "o", save_probabilities=True)
    with pytest.raises(ContractError, match="download"):
        liver.run(image_path=image, output_dir=tmp_path / "o")
    with pytest.raises(ContractError, match="fold"):
        brats.run(image_paths={}, output_dir=tmp_path / "o", fold=7)
    with pytest.raises(ContractError, match="t1"):
        brats.run(image_paths={"t1": image}, output_dir=tmp_path / "o")
    with pytest.raises(ContractError, match="model folder does not exist"):
        medmlx.run(weights_path=tmp_path / "missing", image_paths=[image], output_dir=tmp_path / "o")


def test_cli_argument_errors(tmp_path, capsys):
    from nnunet_mlx.cli import main

    assert main(["predict", "-i", str(tmp_path), "-o", str(tmp_path / "o"), "-d", "3"]) == 2
    assert "-d and -c" in capsys.readouterr().err
    assert main(["predict", "-i", str(tmp_path), "-o", str(tmp_path / "o"), "-m", str(tmp_path),
                 "-d", "3", "-c", "3d_fullres"]) == 2
    assert main(["predict", "-i", str(tmp_path), "-o", str(tmp_path / "o"), "-m", str(tmp_path),
                 "-f", "x"]) == 2
    assert "invalid fold" in capsys.readouterr().err


def test_default_batch_respects_the_activation_limit():
    """Largest activation per view from the spec (input channels and classes included), and
    the default tiles per batch of the sliding window's own request: about 32 views, capped
    so a forward batch's largest activation stays within 2^31 elements (liver: 4 tiles x 8
    views = exactly 2^31; ResEnc-L 128x160x160 without mirroring: 20 tiles)."""
    from types import SimpleNamespace

    import torch

    from nnunet_mlx.model.topology import PlainConvUNetSpec, ResidualEncoderUNetSpec
    from nnunet_mlx.prediction import sliding_window as sw

    k3 = ((3, 3, 3),)
    liver = PlainConvUNetSpec(1, 3, (32, 64, 128, 256, 320, 320), k3 * 6,
                              ((1, 1, 1),) + ((2, 2, 2),) * 5, (2,) * 6, (2,) * 5)
    resenc = ResidualEncoderUNetSpec(1, 3, (32, 64, 128, 256, 320, 320, 320), k3 * 7,
                                     ((1, 1, 1),) + ((2, 2, 2),) * 5 + ((2, 1, 1),),
                                     (1, 3, 4, 6, 6, 6, 6), (1,) * 6)
    per = sw._activation_elements_per_view([SimpleNamespace(spec=liver)], (128, 128, 128))
    assert per == 128 ** 3 * 32 and 4 * 8 * per == sw.ACTIVATION_ELEMENT_LIMIT
    assert sw._activation_elements_per_view([object()], (8, 8, 8)) == 8 ** 3
    # classes (or input channels) wider than the first stage set the per-view size
    wide = sw._activation_elements_per_view([SimpleNamespace(spec=liver)], (8, 8, 8),
                                            num_classes=40)
    assert wide == 8 ** 3 * 40

    # the helper the sliding-window request calls when tiles_per_batch is None
    assert sw.default_tiles_per_batch([SimpleNamespace(spec=liver)], (128, 128, 128), 8) == 4
    assert sw.default_tiles_per_batch([SimpleNamespace(spec=resenc)], (128, 160, 160), 1) == 20
    assert sw.default_tiles_per_batch([SimpleNamespace(spec=liver)], (16, 16, 16), 1) == 32
    assert sw.default_tiles_per_batch([SimpleNamespace(spec=liver)], (16, 16, 16), 8) == 4
    # at least one tile, however large the patch
    assert sw.default_tiles_per_batch([SimpleNamespace(spec=liver)], (512, 512, 512), 8) == 1


def test_source_signature_tracks_every_model_file(tmp_path):
    """The loaded-model signature covers plans.json, dataset.json and each fold's state and
    weights (src/nnunet_mlx/medmlx.py:454-469): a touch of any one of them changes it, a
    missing one raises, and files outside that set do not count."""
    import os

    from nnunet_mlx.medmlx import source_signature

    folder = tmp_path / "model"
    files = ["plans.json", "dataset.json"]
    for fold in ("fold_0", "fold_all"):
        files += [f"{fold}/checkpoint_final/state.json",
                  f"{fold}/checkpoint_final/weights.safetensors"]
    for name in files:
        (folder / name).parent.mkdir(parents=True, exist_ok=True)
        (folder / name).write_text("x")
    (folder / "notes.txt").write_text("not a model file")
    (folder / "fold_0" / "checkpoint_best").mkdir()
    (folder / "fold_0" / "checkpoint_best" / "state.json").write_text("{}")
    base = source_signature(folder, "checkpoint_final")
    assert [r[0] for r in base] == files[:2] + sorted(files[2:])
    assert source_signature(folder, "checkpoint_final") == base
    (folder / "notes.txt").write_text("edited")
    os.utime(folder / "fold_0" / "checkpoint_best" / "state.json", ns=(1, 1))
    assert source_signature(folder, "checkpoint_final") == base
    for name in files:
        st = (folder / name).stat()
        os.utime(folder / name, ns=(st.st_atime_ns, st.st_mtime_ns + 10**9))
        now = source_signature(folder, "checkpoint_final")
        assert now != base, name
        base = now
    (folder / files[-1]).unlink()
    with pytest.raises(ContractError, match="missing"):
        source_signature(folder, "checkpoint_final")
