"""GPU-resident Gaussian sliding-window inference for 3-D nnU-Net logits on MI355X.

Public names and contracts follow the reference's ``nnunet_mlx.prediction.sliding_window``
(src/nnunet_mlx/prediction/sliding_window.py:32-562).  The host computes what must be
bit-exact with the reference's numpy arithmetic — tile offsets (float64 stride, Python
half-to-even ``round``), the minimum padding, the mirror order and the float32/float16
Gaussian maps — and hands them to the HIP pipeline:

  gather+flip (all mirror views of a tile into one batch) -> network forward ->
  mirror average + Gaussian accumulation into a whole-volume HBM accumulator ->
  normalisation -> fold sum -> fold average + argmax.

For networks built by this package the whole tile loop runs inside
libnnunet_hip.so (``nnx_sw_predict``); any other callable mapping channels-last device
tiles to logits is driven from Python through the same HIP kernels.
"""

from __future__ import annotations

import ctypes
from collections.abc import Callable, Sequence
from functools import lru_cache
from itertools import combinations, product

import numpy as np
import torch

from nnunet_mlx import _native
from nnunet_mlx.errors import ContractError

FloatArray = np.ndarray
ACCUMULATIONS = ("float32", "nnunet-fp16")


def compute_steps(
    image_size: Sequence[int], patch_size: Sequence[int], *, step_fraction: float = 0.5
) -> tuple[tuple[int, ...], ...]:
    """Per-axis patch start offsets (upstream ``compute_steps_for_sliding_window``).

    Reference: src/nnunet_mlx/prediction/sliding_window.py:32-67.
    """
    if not 0 < step_fraction <= 1:
        raise ContractError(f"step_fraction must be in (0, 1], got {step_fraction}")
    if len(image_size) not in (2, 3) or len(patch_size) != len(image_size):
        raise ContractError("sliding-window inference requires matching 2-D or 3-D shapes")
    return tuple(
        _axis_steps(int(image), int(patch), step_fraction=step_fraction)
        for image, patch in zip(image_size, patch_size)
    )


def _axis_steps(image: int, patch: int, *, step_fraction: float) -> tuple[int, ...]:
    if image < patch:
        raise ContractError(f"padded image dimension {image} is smaller than patch {patch}")
    count = int(np.ceil((image - patch) / (patch * step_fraction))) + 1
    span = image - patch
    stride = span / (count - 1) if count > 1 else 0.0
    return tuple(round(stride * k) for k in range(count))


@lru_cache(maxsize=8)
def gaussian_importance(patch_size: tuple[int, ...]) -> FloatArray:
    """Float32 tile weights: separable Gaussian (centre size//2, sigma size/8), max 1,
    exact zeros replaced by the smallest normal float32 (sliding_window.py:70-93)."""
    if any(size < 1 for size in patch_size):
        raise ContractError(f"invalid patch size {patch_size}")
    exponent = np.zeros(patch_size, dtype=np.float32)
    for axis, size in enumerate(patch_size):
        coordinates = np.arange(size, dtype=np.float32)
        term = ((coordinates - (size // 2)) / (size / 8)) ** 2
        exponent += term.reshape(tuple(size if i == axis else 1 for i in range(len(patch_size))))
    values = np.exp(-0.5 * exponent).astype(np.float32, copy=False)
    values /= np.float32(values.max())
    values[values == 0] = np.finfo(np.float32).tiny
    values.setflags(write=False)
    return values


@lru_cache(maxsize=8)
def nnunet_fp16_gaussian(patch_size: tuple[int, ...]) -> np.ndarray:
    """nnU-Net's scaled float16 Gaussian: a filtered centred impulse (sigma size/8,
    constant mode), scaled to max 10, float16, zeros -> smallest nonzero
    (sliding_window.py:96-113)."""
    from scipy.ndimage import gaussian_filter

    impulse = np.zeros(patch_size)
    impulse[tuple(size // 2 for size in patch_size)] = 1
    weights = gaussian_filter(impulse, [size / 8 for size in patch_size], mode="constant")
    rounded = (weights / (weights.max() / 10)).astype(np.float16)
    rounded[rounded == 0] = rounded[rounded != 0].min()
    rounded.setflags(write=False)
    return rounded


def mirror_flip_masks(axes: Sequence[int]) -> tuple[int, ...]:
    """View order of mirrored_prediction (sliding_window.py:514-515) as axis bitmasks:
    identity, then ``combinations(axes, r)`` for r = 1..len(axes); bit a = spatial axis a."""
    masks = [0]
    for count in range(1, len(axes) + 1):
        for selected in combinations(tuple(axes), count):
            masks.append(sum(1 << a for a in selected))
    return tuple(masks)


def pad_minimum(shape: Sequence[int], patch: Sequence[int]):
    """Zero padding up to the patch, odd voxel after (sliding_window.py:542-562)."""
    before, crop = [], []
    for size, minimum in zip(shape, patch):
        total = max(0, minimum - size)
        before.append(total // 2)
        crop.append(slice(total // 2, total // 2 + size))
    padded = tuple(max(int(s), int(p)) for s, p in zip(shape, patch))
    return tuple(before), padded, tuple(crop)


def _validate_request(data, patch_size, num_classes, mirroring_axes, accumulation):
    if accumulation not in ACCUMULATIONS:
        raise ContractError(f"unsupported sliding-window accumulation {accumulation!r}")
    if data.ndim != 4:
        raise ContractError(
            f"expected finite float32 (C,*spatial) 3-D input, got {tuple(data.shape)}"
            " (two-dimensional inference does not run on the HIP path)"
        )
    is_float32 = data.dtype == (torch.float32 if isinstance(data, torch.Tensor) else np.float32)
    if not is_float32:
        raise ContractError(f"expected finite float32 (C,*spatial) 3-D input, got {data.dtype}")
    patch = tuple(int(v) for v in patch_size)
    if len(patch) != 3 or any(v < 1 for v in patch):
        raise ContractError(f"invalid patch size {patch}")
    if num_classes < 1:
        raise ContractError("sliding-window inference requires at least one output channel")
    axes = tuple(int(a) for a in mirroring_axes)
    if any(a not in range(3) for a in axes) or len(set(axes)) != len(axes):
        raise ContractError(f"invalid mirroring axes {axes}")
    return patch, axes


def _device_volume(data, device: torch.device) -> torch.Tensor:
    if isinstance(data, torch.Tensor):
        volume = data.to(device=device, dtype=torch.float32).contiguous()
    else:
        volume = torch.from_numpy(np.ascontiguousarray(data, dtype=np.float32)).to(device)
    lib = _native.load()
    count = torch.empty(1, dtype=torch.int32, device=device)
    _native.check(lib.nnx_count_nonfinite(_native.ptr(volume), volume.numel(), _native.ptr(count),
                                          _native.stream_handle(device)))
    if int(count.item()) != 0:
        raise ContractError(
            f"expected finite float32 (C,*spatial) 3-D input, got {tuple(volume.shape)}"
        )
    return volume


# Default memory budget of one forward batch: its largest single activation (elements).
# The network workspace keeps every activation of the batch resident (about 4 x the
# largest one for a plain network, more for residual encoders), so 2^31 float32 elements
# (8 GiB) keeps a default batch within a few tens of GB of HBM.  A memory budget only: the
# library handles batches of any size whose items stay below 2^31 elements.
ACTIVATION_ELEMENT_LIMIT = 1 << 31
# Views per forward batch the default aims at: enough workgroups for the 8^3 and 4^3 stages.
DEFAULT_VIEWS_PER_BATCH = 32


def _activation_elements_per_view(models, patch, *, channels: int = 1, num_classes: int = 1) -> int:
    """Largest tensor (elements) one view of ``patch`` creates in any of the networks: the
    input tile, the logits, the full-resolution stage or a deeper stage (stride-2 sizes
    round up)."""
    voxels = int(np.prod([int(v) for v in patch]))
    worst = voxels * max(int(channels), int(num_classes))
    for model in models:
        spec = getattr(model, "spec", None)
        if spec is None:
            continue
        size = [int(v) for v in patch]
        first = max(spec.features[0], getattr(spec, "stem_channels", None) or 0)
        worst = max(worst, voxels * first)
        for features, stride in zip(spec.features, spec.strides):
            size = [-(-n // int(st)) for n, st in zip(size, stride)]
            worst = max(worst, int(np.prod(size)) * int(features))
    return worst


def default_tiles_per_batch(models, patch, nviews: int, *, channels: int = 1,
                            num_classes: int = 1) -> int:
    """Tiles per forward batch when the caller does not choose: about
    ``DEFAULT_VIEWS_PER_BATCH`` views, fewer while the batch's largest activation exceeds
    ``ACTIVATION_ELEMENT_LIMIT``, at least one tile."""
    tiles = max(1, DEFAULT_VIEWS_PER_BATCH // max(1, int(nviews)))
    per_tile = _activation_elements_per_view(models, patch, channels=channels,
                                             num_classes=num_classes) * max(1, int(nviews))
    while tiles > 1 and tiles * per_tile > ACTIVATION_ELEMENT_LIMIT:
        tiles -= 1
    return tiles


class _Request:
    """Everything the HIP pipeline needs for one volume, kept alive across the call."""

    def __init__(self, data, *, patch_size, num_classes, mirroring_axes, step_fraction,
                 accumulation, device, tiles_per_batch, models=()):
        self.patch, self.axes = _validate_request(
            data, patch_size, num_classes, mirroring_axes, accumulation)
        self.accumulation = accumulation
        self.fp16 = accumulation == "nnunet-fp16"
        self.num_classes = int(num_classes)
        self.volume = _device_volume(data, device)
        self.channels = int(self.volume.shape[0])
        self.size = tuple(int(v) for v in self.volume.shape[1:])
        self.pad_before, self.padded, self.crop = pad_minimum(self.size, self.patch)
        steps = compute_steps(self.padded, self.patch, step_fraction=step_fraction)
        self.offsets = [tuple(o) for o in product(*steps)]
        self.flips = mirror_flip_masks(self.axes)
        gaussian = nnunet_fp16_gaussian(self.patch) if self.fp16 else gaussian_importance(self.patch)
        self.gaussian = torch.from_numpy(np.array(gaussian, copy=True)).to(device)
        self.device = device
        if tiles_per_batch is None:
            tiles_per_batch = default_tiles_per_batch(models, self.patch, len(self.flips),
                                                      channels=self.channels,
                                                      num_classes=self.num_classes)
        self.tiles_per_batch = int(tiles_per_batch)
        self._offsets_c = _native.ints([v for o in self.offsets for v in o])
        self._flips_c = _native.ints(self.flips)
        cfg = _native.NnxSwConfig()
        cfg.channels = self.channels
        cfg.num_classes = self.num_classes
        cfg.size[:] = self.size
        cfg.pad_before[:] = self.pad_before
        cfg.padded[:] = self.padded
        cfg.patch[:] = self.patch
        cfg.ntiles = len(self.offsets)
        cfg.tile_offsets = ctypes.cast(self._offsets_c, _native.c_int_p)
        cfg.nviews = len(self.flips)
        cfg.view_flips = ctypes.cast(self._flips_c, _native.c_int_p)
        cfg.accumulation = _native.NNX_ACCUM_NNUNET_F16 if self.fp16 else _native.NNX_ACCUM_F32
        cfg.d_gaussian = self.gaussian.data_ptr()
        cfg.tiles_per_batch = self.tiles_per_batch
        self.config = cfg

    def outputs(self, want_logits: bool, want_labels: bool):
        dtype = torch.float16 if self.fp16 else torch.float32
        logits = (torch.empty((*self.size, self.num_classes), dtype=dtype, device=self.device)
                  if want_logits else None)
        labels = (torch.empty(self.size, dtype=torch.int16, device=self.device)
                  if want_labels else None)
        return logits, labels


def _run(models, request: _Request, *, want_logits: bool, want_labels: bool):
    from nnunet_mlx.model.network import NativeNetwork

    if not models:
        raise ContractError("fold inference requires at least one model")
    logits, labels = request.outputs(want_logits, want_labels)
    lib = _native.load()
    stream = _native.stream_handle(request.device)
    if all(isinstance(m, NativeNetwork) for m in models):
        for m in models:
            if m.spec.input_channels != request.channels:
                raise ContractError("model input channels do not match the data")
            if m.spec.num_classes != request.num_classes:
                raise ContractError("model output channels do not match num_classes")
        handles = (ctypes.c_void_p * len(models))(*[m.handle.value for m in models])

        def native_loop() -> None:
            with torch.cuda.device(request.device):
                _native.check(lib.nnx_sw_predict(
                    handles, len(models), ctypes.byref(request.config),
                    _native.ptr(request.volume), _native.ptr(logits), _native.ptr(labels),
                    stream), "nnx_sw_predict")

        try:
            native_loop()
        except ContractError as error:
            if "non-finite logits" not in str(error):
                raise
            _native.name_nonfinite_layer(error, native_loop)
    else:
        _run_callables(models, request, logits, labels)
    return logits, labels


def _run_callables(models, request: _Request, logits, labels) -> None:
    """Tile loop driven from Python over the HIP kernels, for arbitrary callables."""
    lib = _native.load()
    stream = _native.stream_handle(request.device)
    dev = request.device
    K = request.num_classes
    dtype = torch.float16 if request.fp16 else torch.float32
    acc = torch.empty((*request.padded, K), dtype=dtype, device=dev)
    norm = torch.empty(request.padded, dtype=dtype, device=dev)
    total = torch.empty((*request.size, K), dtype=dtype, device=dev)
    nviews = len(request.flips)
    batch = torch.empty((nviews, *request.patch, request.channels), dtype=torch.float32, device=dev)
    size_c = _native.i64s(request.size)
    padded_c = _native.i64s(request.padded)
    pad_c = _native.ints(request.pad_before)
    patch_c = _native.ints(request.patch)
    accum = request.config.accumulation
    for fold, model in enumerate(models):
        acc.zero_()
        norm.zero_()
        for offset in request.offsets:
            off_c = _native.ints(offset)
            _native.check(lib.nnx_sw_gather_flip(
                _native.ptr(request.volume), request.channels, size_c, pad_c, off_c, patch_c,
                request._flips_c, nviews, _native.ptr(batch), stream), "nnx_sw_gather_flip")
            pred = model(batch)
            if not isinstance(pred, torch.Tensor) or pred.dtype != torch.float32:
                raise ContractError("model output must be a float32 device tensor")
            expected = (nviews, *request.patch, K)
            if tuple(pred.shape) != expected:
                raise ContractError(f"model output shape {tuple(pred.shape)} does not match {expected}")
            pred = pred.contiguous()
            _native.check(lib.nnx_sw_accumulate(
                _native.ptr(pred), nviews, request._flips_c, K, patch_c,
                _native.ptr(request.gaussian), off_c, padded_c, accum, _native.ptr(acc),
                _native.ptr(norm), stream), "nnx_sw_accumulate")
        _native.check(lib.nnx_sw_fold_add(
            _native.ptr(acc), _native.ptr(norm), K, padded_c, pad_c, size_c, accum,
            1 if fold == 0 else 0, _native.ptr(total), stream), "nnx_sw_fold_add")
    invalid = torch.empty(1, dtype=torch.int32, device=dev)
    voxels = int(np.prod(request.size))
    _native.check(lib.nnx_sw_fold_finalize(
        _native.ptr(total), K, voxels, len(models), accum, _native.ptr(logits),
        _native.ptr(labels), _native.ptr(invalid), stream), "nnx_sw_fold_finalize")
    if int(invalid.item()) != 0:
        raise ContractError("sliding-window inference produced non-finite logits")


def _device(models) -> torch.device:
    if not torch.cuda.is_available():
        raise _native.NativeUnavailable("the HIP sliding window needs a GPU")
    return torch.device("cuda", torch.cuda.current_device())


def predict_device_logits(
    model, data_channels_first, *, patch_size: Sequence[int], num_classes: int,
    mirroring_axes: Sequence[int] = (), step_fraction: float = 0.5,
    accumulation: str = "float32", tiles_per_batch: int | None = None,
) -> torch.Tensor:
    """Cropped channels-last ``(*spatial, K)`` normalised logits left on the GPU,
    float16 for ``nnunet-fp16`` (sliding_window.py:219-258)."""
    return average_fold_device_logits(
        (model,), data_channels_first, patch_size=patch_size, num_outputs=num_classes,
        mirroring_axes=mirroring_axes, step_fraction=step_fraction, accumulation=accumulation,
        tiles_per_batch=tiles_per_batch,
    )


def average_fold_device_logits(
    models, data_channels_first, *, patch_size: Sequence[int], num_outputs: int,
    mirroring_axes: Sequence[int] = (), step_fraction: float = 0.5,
    accumulation: str = "float32", tiles_per_batch: int | None = None,
) -> torch.Tensor:
    """Fold-averaged channels-last logits on the GPU (inference.py:93-149)."""
    request = _Request(
        data_channels_first, patch_size=patch_size, num_classes=num_outputs,
        mirroring_axes=mirroring_axes, step_fraction=step_fraction, accumulation=accumulation,
        device=_device(models), tiles_per_batch=tiles_per_batch, models=tuple(models),
    )
    logits, _ = _run(tuple(models), request, want_logits=True, want_labels=False)
    return logits


def predict_host_logits(
    model, data_channels_first, *, patch_size: Sequence[int], num_classes: int,
    mirroring_axes: Sequence[int] = (), step_fraction: float = 0.5,
    accumulation: str = "float32", tiles_per_batch: int | None = None,
) -> np.ndarray:
    """Host ``(K, *spatial)`` logits in the accumulation dtype (sliding_window.py:158-216)."""
    logits = predict_device_logits(
        model, data_channels_first, patch_size=patch_size, num_classes=num_classes,
        mirroring_axes=mirroring_axes, step_fraction=step_fraction, accumulation=accumulation,
        tiles_per_batch=tiles_per_batch,
    )
    return np.ascontiguousarray(np.moveaxis(logits.cpu().numpy(), -1, 0))


def predict_logits(
    model, data_channels_first, *, patch_size: Sequence[int], num_classes: int,
    mirroring_axes: Sequence[int] = (), step_fraction: float = 0.5,
    accumulation: str = "float32", tiles_per_batch: int | None = None,
) -> np.ndarray:
    """Finite host ``(K, *spatial)`` float32 logits (sliding_window.py:116-155)."""
    return np.asarray(predict_host_logits(
        model, data_channels_first, patch_size=patch_size, num_classes=num_classes,
        mirroring_axes=mirroring_axes, step_fraction=step_fraction, accumulation=accumulation,
        tiles_per_batch=tiles_per_batch,
    ), dtype=np.float32)


def predict_labels(
    model, data_channels_first, *, patch_size: Sequence[int], num_classes: int,
    mirroring_axes: Sequence[int] = (), step_fraction: float = 0.5,
    accumulation: str = "float32", tiles_per_batch: int | None = None,
) -> np.ndarray:
    """Cropped uint16 labels; only labels leave the GPU (sliding_window.py:312-356)."""
    return average_fold_labels(
        (model,), data_channels_first, patch_size=patch_size, num_outputs=num_classes,
        mirroring_axes=mirroring_axes, step_fraction=step_fraction, accumulation=accumulation,
        tiles_per_batch=tiles_per_batch,
    )


def average_fold_labels(
    models, data_channels_first, *, patch_size: Sequence[int], num_outputs: int,
    mirroring_axes: Sequence[int] = (), step_fraction: float = 0.5,
    accumulation: str = "float32", tiles_per_batch: int | None = None,
    return_device: bool = False,
):
    """Argmax labels of the fold-averaged logits, computed on the GPU."""
    request = _Request(
        data_channels_first, patch_size=patch_size, num_classes=num_outputs,
        mirroring_axes=mirroring_axes, step_fraction=step_fraction, accumulation=accumulation,
        device=_device(models), tiles_per_batch=tiles_per_batch, models=tuple(models),
    )
    _, labels = _run(tuple(models), request, want_logits=False, want_labels=True)
    if return_device:
        return labels
    return labels.cpu().numpy().view(np.uint16)
