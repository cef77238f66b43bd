"""``nnunet-mlx predict``: nnUNetv2_predict's options over a trained upstream model folder.

Reference: ``predict_command`` (src/nnunet_mlx/commands/upstream.py:56-178) and the CLI
entry (src/nnunet_mlx/cli.py:17-76).  The trained PyTorch model is converted on first use
into the conversion cache (``nnunet_mlx.storage.upstream.cached_conversion``), loaded with
every fold resident on the GPU, and each case of the input folder runs through
``ModelFolderPredictor`` with float16 window accumulation.  Run as
``python -m nnunet_mlx predict -i IN -o OUT -d 3 -c 3d_fullres`` (or ``-m FOLDER``).
Multi-process preprocessing/export workers, cascades, probabilities and ``-num_parts``
splitting are not options here.
"""

from __future__ import annotations

import argparse
import json
import sys
from collections.abc import Sequence
from dataclasses import replace
from pathlib import Path

from nnunet_mlx.errors import ContractError


def _parser() -> argparse.ArgumentParser:
    parser = argparse.ArgumentParser(prog="nnunet-mlx")
    commands = parser.add_subparsers(dest="command", required=True)
    p = commands.add_parser("predict", help="Predict a folder from a trained nnU-Net model.")
    p.add_argument("-i", dest="input_folder", required=True, type=Path,
                   help="Input folder with nnU-Net-named images (case_0000.nii.gz).")
    p.add_argument("-o", dest="output_folder", required=True, type=Path, help="Output folder.")
    p.add_argument("-d", dest="dataset", help="Dataset ID or name under $nnUNet_results.")
    p.add_argument("-c", dest="configuration", help="Configuration, e.g. 3d_fullres.")
    p.add_argument("-p", dest="plans", default="nnUNetPlans", help="Plans identifier.")
    p.add_argument("-tr", dest="trainer", default="nnUNetTrainer", help="Trainer class name.")
    p.add_argument("-m", dest="model_folder", type=Path,
                   help="Trained model folder, instead of -d/-c/-tr/-p.")
    p.add_argument("-f", dest="folds", nargs="+",
                   help="Folds to ensemble (default: 0 1 2 3 4 with -d, every fold with -m).")
    p.add_argument("-chk", dest="checkpoint_name", default="checkpoint_final.pth",
                   help="Upstream checkpoint file in each fold folder.")
    p.add_argument("-step_size", dest="step_size", type=float, default=0.5,
                   help="Sliding-window step fraction.")
    p.add_argument("--disable_tta", action="store_true",
                   help="Skip mirroring test-time augmentation.")
    p.add_argument("--continue_prediction", action="store_true",
                   help="Skip cases already predicted.")
    p.add_argument("--json", dest="json_output", action="store_true")
    return parser


def _folds(values: Sequence[str] | None) -> tuple[int | str, ...] | None:
    if values is None:
        return None
    folds: list[int | str] = []
    for value in values:
        if value == "all":
            folds.append("all")
        elif value.isdigit():
            folds.append(int(value))
        else:
            raise ContractError(f"invalid fold {value!r}")
    return tuple(folds)


def predict(args: argparse.Namespace) -> dict[str, object]:
    from nnunet_mlx.medmlx import predictor
    from nnunet_mlx.model.folder import load_model_bundle
    from nnunet_mlx.plans import read_json_object
    from nnunet_mlx.storage.upstream import (CONVERSION_FILENAME, cached_conversion,
                                             resolve_results_folder)

    if not 0 < args.step_size <= 1:
        raise ContractError("-step_size must be in (0, 1]")
    folds = _folds(args.folds)
    if args.model_folder is not None:
        if args.dataset is not None or args.configuration is not None:
            raise ContractError("pass either -m or -d with -c, not both")
        trained = args.model_folder
    else:
        if args.dataset is None or args.configuration is None:
            raise ContractError("pass -d and -c, or a trained model folder with -m")
        trained = resolve_results_folder(args.dataset, configuration=args.configuration,
                                         trainer=args.trainer, plans=args.plans)
        if folds is None:
            folds = (0, 1, 2, 3, 4)
    converted = cached_conversion(trained, folds=folds, checkpoint_name=args.checkpoint_name)
    manifest = read_json_object(converted / CONVERSION_FILENAME)
    selected = folds if folds is not None else tuple(e["fold"] for e in manifest["folds"])
    bundle = load_model_bundle(converted, configuration=str(manifest["configuration"]),
                               folds=selected)
    if args.disable_tta:
        bundle = replace(bundle, mirroring_axes=())
    try:
        results = predictor(bundle, step_fraction=args.step_size).predict_folder(
            args.input_folder, args.output_folder, overwrite=not args.continue_prediction,
            continue_prediction=args.continue_prediction)
    finally:
        for model in bundle.models:
            model.close()
    return {"predicted": [str(f) for r in results for f in r.files],
            "conversion": str(converted), "folds": list(selected)}


def main(argv: Sequence[str] | None = None) -> int:
    args = _parser().parse_args(argv)
    try:
        payload = predict(args)
    except ContractError as error:
        print(f"error: {error}", file=sys.stderr)
        return 2
    if args.json_output:
        print(json.dumps(payload, sort_keys=True))
    else:
        print(f"predicted: {len(payload['predicted'])}")
    return 0
