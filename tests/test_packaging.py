"""Packaging (host only): the repository installs offline as a distribution whose
``nnunet-mlx`` console script and ``medmlx.models`` entry points (the reference's
pyproject.toml:84-89) resolve to this package."""

from __future__ import annotations

import json
import os
import subprocess
import sys

import pytest

from tests.helpers import install_package


@pytest.fixture(scope="module")
def installed(tmp_path_factory):
    target = tmp_path_factory.mktemp("site")
    bin_dir = install_package(target)
    env = dict(os.environ, PYTHONPATH=str(target))
    return target, bin_dir, env


def test_console_script(installed, tmp_path):
    target, bin_dir, env = installed
    script = bin_dir / "nnunet-mlx"
    assert script.is_file()
    out = subprocess.run([str(script), "predict", "--help"], env=env, capture_output=True,
                         text=True, timeout=120)
    assert out.returncode == 0 and "-step_size" in out.stdout
    out = subprocess.run([str(script), "predict", "-i", str(tmp_path), "-o", str(tmp_path / "o"),
                          "-d", "3"], env=env, capture_output=True, text=True, timeout=120)
    assert out.returncode == 2 and "-d and -c" in out.stderr


def test_model_entry_points(installed):
    target, _, env = installed
    code = ("import json, importlib.metadata as m, nnunet_mlx\n"
            "eps = m.entry_points(group='medmlx.models')\n"
            "print(json.dumps({'models': {e.name: e.load()['id'] for e in eps},"
            " 'package': nnunet_mlx.__file__}))")
    out = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True,
                         timeout=120, cwd=str(target))
    assert out.returncode == 0, out.stderr
    got = json.loads(out.stdout)
    assert got["models"] == {name: name for name in ("nnunet-liver", "nnunet-brats2021",
                                                     "nnunet-autopet", "nnunet-pancreas")}
    assert got["package"].startswith(str(target))


def test_named_models_state_their_device_peak():
    """Every named model carries the registry's peak_memory_gb (the reference's MODEL key,
    src/nnunet_mlx/named_models/liver.py:18), here the measured MI355X device peak."""
    from nnunet_mlx.named_models import autopet, brats, liver, pancreas

    for module in (liver, brats, autopet, pancreas):
        peak = module.MODEL["peak_memory_gb"]
        assert isinstance(peak, float) and 0 < peak < 288, (module.__name__, peak)
