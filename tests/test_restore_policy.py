"""Host-side restoration policy: spacing validation, separate-axis choice, contract parsing."""

from __future__ import annotations

import pytest

from nnunet_mlx.data.resampling import separate_z_axis, validate_spacing
from nnunet_mlx.errors import ContractError
from nnunet_mlx.plans import ResamplingContract
from nnunet_mlx.prediction.restore import device_class_restore_supported


def test_separate_z_axis_rules():
    iso, aniso = (1.0, 1.0, 1.0), (3.5, 1.0, 1.0)
    assert separate_z_axis(iso, iso, force=None) == (False, None)
    assert separate_z_axis(aniso, iso, force=None) == (True, 0)      # current spacing decides
    assert separate_z_axis(iso, (1.0, 4.0, 1.0), force=None) == (True, 1)  # else the target
    assert separate_z_axis((3.5, 3.5, 1.0), iso, force=None) == (False, None)  # tied coarsest
    assert separate_z_axis(iso, aniso, force=False) == (False, None)
    assert separate_z_axis((1.0, 2.0, 1.0), iso, force=True) == (True, 1)
    assert separate_z_axis((3.0, 1.0, 1.0), iso, force=None) == (False, None)  # ratio == threshold
    with pytest.raises(ContractError):
        validate_spacing((1.0, 0.0, 1.0), name="s")
    with pytest.raises(ContractError):
        validate_spacing((1.0, True, 1.0), name="s")


def test_resampling_contract_parsing():
    cfg = {"resampling_fn_probabilities": "resample_data_or_seg_to_shape",
           "resampling_fn_probabilities_kwargs": {"is_seg": False, "order": 1, "order_z": 0,
                                                  "force_separate_z": None}}
    c = ResamplingContract.from_configuration(cfg, field="resampling_fn_probabilities",
                                              expected_is_seg=False)
    assert (c.function_name, c.order, c.order_z, c.force_separate_z) == (
        "resample_data_or_seg_to_shape", 1, 0, None)
    default = ResamplingContract.from_configuration(
        {"f": "resample_data_or_seg_to_shape", "f_kwargs": {}}, field="f", expected_is_seg=False)
    assert (default.order, default.order_z, default.force_separate_z) == (3, 0, False)
    torch_fn = ResamplingContract.from_configuration(
        {"f": "resample_torch_fornnunet", "f_kwargs": {}}, field="f", expected_is_seg=False)
    assert (torch_fn.order, torch_fn.force_separate_z) == (1, None)
    assert (torch_fn.mode, torch_fn.aniso_axis_mode, torch_fn.seg_tiebreak) == (
        "linear", "nearest-exact", "nearest")
    upstream = ResamplingContract.from_configuration(
        {"f": "resample_torch_fornnunet",
         "f_kwargs": {"is_seg": False, "force_separate_z": None, "memefficient_seg_resampling": True,
                      "seg_tiebreak": "lowest", "mode": "nearest", "aniso_axis_mode": "linear",
                      "num_threads": 8, "device": "cpu", "separate_z_anisotropy_threshold": 2}},
        field="f", expected_is_seg=False)
    assert (upstream.mode, upstream.aniso_axis_mode, upstream.seg_tiebreak,
            upstream.separate_z_anisotropy_threshold) == ("nearest", "linear", "lowest", 2.0)
    spline_tie = ResamplingContract.from_configuration(
        {"f": "resample_data_or_seg_to_shape", "f_kwargs": {"seg_tiebreak": "highest"}},
        field="f", expected_is_seg=False)
    assert spline_tie.seg_tiebreak == "highest"
    torch_kwargs = lambda **kw: {"f": "resample_torch_fornnunet", "f_kwargs": kw}  # noqa: E731
    for bad in ({"f": "other", "f_kwargs": {}},
                {"f": "resample_data_or_seg_to_shape", "f_kwargs": {"is_seg": True}},
                {"f": "resample_data_or_seg_to_shape", "f_kwargs": {"order": 7}},
                {"f": "resample_data_or_seg_to_shape", "f_kwargs": {"mode": "linear"}},
                {"f": "resample_data_or_seg_to_shape", "f_kwargs": {"seg_tiebreak": "first"}},
                torch_kwargs(order=1), torch_kwargs(mode="cubic"),
                torch_kwargs(aniso_axis_mode="area"), torch_kwargs(num_threads=0),
                torch_kwargs(num_threads=True), torch_kwargs(device="cuda"),
                torch_kwargs(memefficient_seg_resampling=1), torch_kwargs(seg_tiebreak=None)):
        with pytest.raises(ContractError):
            ResamplingContract.from_configuration(bad, field="f", expected_is_seg=False)


def test_device_support_decision():
    order1 = ResamplingContract("resample_data_or_seg_to_shape", 1, 0, False)
    torch_fn = ResamplingContract("resample_torch_fornnunet", 1, 0, None)
    iso = (1.0, 1.0, 1.0)
    assert device_class_restore_supported((4, 5, 6), (8, 5, 3), iso, iso, order1, classes=3)
    assert not device_class_restore_supported((4, 5, 6), (8, 5, 3), iso, iso, torch_fn, classes=3)
    assert device_class_restore_supported((4, 5, 6), (4, 5, 6), iso, iso, torch_fn, classes=3)
    assert not device_class_restore_supported((4, 5, 6), (8, 5, 3), iso, iso, order1, classes=70000)
    forced = ResamplingContract("resample_data_or_seg_to_shape", 1, 0, True)
    assert not device_class_restore_supported((4, 5, 6), (8, 5, 3), (2.0, 1.0, 1.0), iso, forced,
                                              classes=3)
