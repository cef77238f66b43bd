"""ctypes binding of libnnunet_hip.so (include/nnx.h).

The HIP library is the only compute path: importing a compute entry point without
the built library raises ``NativeUnavailable`` — there is no CPU fallback.  torch is
imported first so that the library binds to the HIP runtime torch already loaded
(both name it libamdhip64.so.7); torch supplies device buffers and the current stream.
"""

from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path
from typing import Any

import torch  # noqa: F401  (loads the shared HIP runtime before the library)

from nnunet_mlx.errors import ContractError, NativeError

LIB_NAME = "libnnunet_hip.so"
LIB_PATH = Path(os.environ.get("NNX_LIB", Path(__file__).resolve().parent / "_lib" / LIB_NAME))

NNX_OK = 0
NNX_ERR_INVALID = -1
NNX_ERR_HIP = -2
NNX_ERR_NONFINITE = -3
NNX_ERR_STATE = -4
NNX_ERR_NOMEM = -5

NNX_ARCH_PLAIN = 0
NNX_ARCH_RESIDUAL = 1
NNX_PRECISION_FP32 = 0
NNX_PRECISION_FP32_SPLIT = 1
NNX_PRECISION_BF16 = 2
NNX_PRECISION_BF16_MIXED = 3
NNX_NORM_NONE = 0
NNX_NORM_CT = 1
NNX_NORM_ZSCORE = 2
NNX_NORM_ZSCORE_MASKED = 3
NNX_ACCUM_F32 = 0
NNX_ACCUM_NNUNET_F16 = 1

c_int_p = ctypes.POINTER(ctypes.c_int)
c_i64_p = ctypes.POINTER(ctypes.c_int64)
c_void_p = ctypes.c_void_p


class NativeUnavailable(NativeError):
    """libnnunet_hip.so is missing or cannot be loaded."""


class NnxSpec(ctypes.Structure):
    _fields_ = [
        ("arch", ctypes.c_int),
        ("spatial_dims", ctypes.c_int),
        ("input_channels", ctypes.c_int),
        ("num_classes", ctypes.c_int),
        ("n_stages", ctypes.c_int),
        ("features", c_int_p),
        ("kernel_sizes", c_int_p),
        ("strides", c_int_p),
        ("encoder_convs", c_int_p),
        ("decoder_convs", c_int_p),
        ("conv_bias", ctypes.c_int),
        ("norm_affine", ctypes.c_int),
        ("norm_eps", ctypes.c_float),
        ("leaky_slope", ctypes.c_float),
        ("stem_channels", ctypes.c_int),
        ("bottleneck_channels", c_int_p),
        ("precision", ctypes.c_int),
    ]


class NnxSwConfig(ctypes.Structure):
    _fields_ = [
        ("channels", ctypes.c_int),
        ("num_classes", ctypes.c_int),
        ("size", ctypes.c_int64 * 3),
        ("pad_before", ctypes.c_int * 3),
        ("padded", ctypes.c_int64 * 3),
        ("patch", ctypes.c_int * 3),
        ("ntiles", ctypes.c_int),
        ("tile_offsets", c_int_p),
        ("nviews", ctypes.c_int),
        ("view_flips", c_int_p),
        ("accumulation", ctypes.c_int),
        ("d_gaussian", c_void_p),
        ("tiles_per_batch", ctypes.c_int),
    ]


FORWARD_FN = ctypes.CFUNCTYPE(
    ctypes.c_int, c_void_p, c_void_p, c_void_p, ctypes.c_int, c_int_p, c_void_p
)

# name -> (restype, argtypes)
_SIGNATURES: dict[str, tuple[Any, list[Any]]] = {
    "nnx_last_error": (ctypes.c_char_p, []),
    "nnx_version": (ctypes.c_char_p, []),
    "nnx_model_create": (ctypes.c_int, [ctypes.POINTER(NnxSpec), ctypes.POINTER(c_void_p)]),
    "nnx_model_param_count": (ctypes.c_int, [c_void_p, c_int_p]),
    "nnx_model_param_info": (
        ctypes.c_int,
        [c_void_p, ctypes.c_int, ctypes.POINTER(ctypes.c_char_p), c_int_p, c_i64_p],
    ),
    "nnx_model_load_param": (ctypes.c_int, [c_void_p, ctypes.c_char_p, c_void_p, c_i64_p, ctypes.c_int]),
    "nnx_model_finalize": (ctypes.c_int, [c_void_p]),
    "nnx_model_share_workspace": (ctypes.c_int, [c_void_p, c_void_p]),
    "nnx_forward": (ctypes.c_int, [c_void_p, c_void_p, c_void_p, ctypes.c_int, c_int_p, c_void_p]),
    "nnx_model_destroy": (None, [c_void_p]),
    "nnx_sw_predict": (
        ctypes.c_int,
        [ctypes.POINTER(c_void_p), ctypes.c_int, ctypes.POINTER(NnxSwConfig), c_void_p, c_void_p, c_void_p, c_void_p],
    ),
    "nnx_sw_predict_custom": (
        ctypes.c_int,
        [ctypes.POINTER(FORWARD_FN), ctypes.POINTER(c_void_p), ctypes.c_int, ctypes.POINTER(NnxSwConfig),
         c_void_p, c_void_p, c_void_p, c_void_p],
    ),
    "nnx_sw_release": (None, []),
    "nnx_set_layer_checks": (ctypes.c_int, [ctypes.c_int]),
    "nnx_count_nonfinite": (ctypes.c_int, [c_void_p, ctypes.c_int64, c_void_p, c_void_p]),
    "nnx_instnorm_workspace_bytes": (ctypes.c_size_t, [ctypes.c_int, ctypes.c_int64, ctypes.c_int]),
    "nnx_instnorm_lrelu": (
        ctypes.c_int,
        [c_void_p, c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_int, c_void_p, c_void_p, c_void_p,
         ctypes.c_float, ctypes.c_int, ctypes.c_float, c_void_p, c_void_p, ctypes.c_size_t, c_void_p],
    ),
    "nnx_instnorm_noalloc_max_bytes": (ctypes.c_size_t, []),
    "nnx_instnorm_lrelu_noalloc": (
        ctypes.c_int,
        [c_void_p, c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_int, c_void_p, c_void_p, c_void_p,
         ctypes.c_float, ctypes.c_int, ctypes.c_float, c_void_p, c_void_p],
    ),
    "nnx_conv3d_packed_floats": (ctypes.c_size_t, [ctypes.c_int, c_int_p, ctypes.c_int, ctypes.c_int]),
    "nnx_conv3d_pack_weight": (
        ctypes.c_int, [c_void_p, ctypes.c_int, c_int_p, ctypes.c_int, ctypes.c_int, c_void_p, c_void_p]
    ),
    "nnx_conv3d_igemm": (
        ctypes.c_int,
        [c_void_p, ctypes.c_int, c_void_p, ctypes.c_int, c_void_p, c_void_p, c_void_p, ctypes.c_int,
         c_int_p, ctypes.c_int, c_int_p, c_int_p, c_void_p],
    ),
    "nnx_split_weight_scale": (ctypes.c_float, [ctypes.c_float]),
    "nnx_conv3d_split_packed_bytes": (ctypes.c_size_t, [ctypes.c_int, c_int_p, ctypes.c_int, ctypes.c_int]),
    "nnx_conv3d_split_pack_weight": (
        ctypes.c_int,
        [c_void_p, ctypes.c_int, c_int_p, ctypes.c_int, ctypes.c_int, ctypes.c_float, c_void_p, c_void_p],
    ),
    "nnx_conv3d_split": (
        ctypes.c_int,
        [c_void_p, ctypes.c_int, c_void_p, ctypes.c_int, c_void_p, ctypes.c_float, c_void_p, c_void_p,
         ctypes.c_int, c_int_p, ctypes.c_int, c_int_p, c_int_p, c_void_p],
    ),
    "nnx_winograd_weight_scale": (ctypes.c_float, [ctypes.c_float]),
    "nnx_conv3d_winograd_packed_bytes": (ctypes.c_size_t, [ctypes.c_int, ctypes.c_int, ctypes.c_int]),
    "nnx_conv3d_winograd_pack_weight": (
        ctypes.c_int,
        [c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_float, c_void_p, c_void_p],
    ),
    "nnx_conv3d_winograd": (
        ctypes.c_int,
        [c_void_p, ctypes.c_int, c_void_p, ctypes.c_int, c_void_p, ctypes.c_float, c_void_p, c_void_p,
         ctypes.c_int, c_int_p, ctypes.c_int, c_void_p],
    ),
    "nnx_conv3d_direct_small_cin": (
        ctypes.c_int, [c_void_p, c_void_p, c_void_p, c_void_p, ctypes.c_int, c_int_p, ctypes.c_int, c_void_p]
    ),
    "nnx_conv3d_direct_small_cin_split": (
        ctypes.c_int,
        [c_void_p, ctypes.c_int, c_void_p, ctypes.c_float, c_void_p, c_void_p, ctypes.c_int, c_int_p,
         ctypes.c_int, c_void_p],
    ),
    "nnx_tconv3d_packed_floats": (ctypes.c_size_t, [ctypes.c_int, c_int_p, ctypes.c_int]),
    "nnx_tconv3d_pack_weight": (
        ctypes.c_int, [c_void_p, ctypes.c_int, c_int_p, ctypes.c_int, c_void_p, c_void_p]
    ),
    "nnx_tconv3d_split_packed_bytes": (ctypes.c_size_t, [ctypes.c_int, c_int_p, ctypes.c_int]),
    "nnx_tconv3d_split_pack_weight": (
        ctypes.c_int, [c_void_p, ctypes.c_int, c_int_p, ctypes.c_int, ctypes.c_float, c_void_p, c_void_p]
    ),
    "nnx_tconv3d_split": (
        ctypes.c_int,
        [c_void_p, ctypes.c_int, c_void_p, ctypes.c_float, c_void_p, c_void_p, ctypes.c_int, c_int_p,
         ctypes.c_int, c_int_p, c_void_p],
    ),
    "nnx_conv3d_bf16_pack_weight": (
        ctypes.c_int,
        [c_void_p, ctypes.c_int, c_int_p, ctypes.c_int, ctypes.c_int, ctypes.c_float, c_void_p, c_void_p],
    ),
    "nnx_conv3d_bf16": (
        ctypes.c_int,
        [c_void_p, ctypes.c_int, c_void_p, ctypes.c_int, c_void_p, ctypes.c_float, c_void_p, c_void_p,
         ctypes.c_int, c_int_p, ctypes.c_int, c_int_p, c_int_p, c_void_p],
    ),
    "nnx_tconv3d_bf16_pack_weight": (
        ctypes.c_int, [c_void_p, ctypes.c_int, c_int_p, ctypes.c_int, ctypes.c_float, c_void_p, c_void_p]
    ),
    "nnx_tconv3d_bf16": (
        ctypes.c_int,
        [c_void_p, ctypes.c_int, c_void_p, ctypes.c_float, c_void_p, c_void_p, ctypes.c_int, c_int_p,
         ctypes.c_int, c_int_p, c_void_p],
    ),
    "nnx_restore_labels": (
        ctypes.c_int, [c_void_p, ctypes.c_int, ctypes.c_int, c_int_p, c_int_p, c_void_p, c_void_p]
    ),
    "nnx_restore_labels_spline_workspace": (ctypes.c_size_t, [c_int_p, c_int_p, ctypes.c_int]),
    "nnx_restore_labels_spline": (
        ctypes.c_int,
        [c_void_p, ctypes.c_int, ctypes.c_int, c_int_p, c_int_p, ctypes.c_int, ctypes.c_int,
         c_void_p, ctypes.c_size_t, c_void_p, c_void_p],
    ),
    "nnx_torch_resize": (
        ctypes.c_int,
        [c_void_p, ctypes.c_int, ctypes.c_int, c_int_p, c_i64_p, c_void_p, c_int_p, c_i64_p,
         ctypes.c_int, c_void_p],
    ),
    "nnx_torch_resize_argmax": (
        ctypes.c_int,
        [c_void_p, ctypes.c_int, ctypes.c_int, c_int_p, c_i64_p, c_int_p, ctypes.c_int, c_void_p,
         c_void_p],
    ),
    "nnx_nonzero_bbox": (ctypes.c_int, [c_void_p, ctypes.c_int, c_i64_p, c_void_p, c_void_p]),
    "nnx_nonzero_mask_filled": (
        ctypes.c_int, [c_void_p, ctypes.c_int, c_i64_p, c_i64_p, c_i64_p, c_void_p, c_void_p, c_void_p]
    ),
    "nnx_zscore_stats_workspace": (ctypes.c_size_t, []),
    "nnx_channel_minmax": (
        ctypes.c_int,
        [c_void_p, ctypes.c_int, c_i64_p, ctypes.c_int, c_i64_p, c_i64_p, c_void_p, c_void_p,
         c_void_p],
    ),
    "nnx_zscore_stats": (
        ctypes.c_int,
        [c_void_p, ctypes.c_int, c_i64_p, ctypes.c_int, c_i64_p, c_i64_p, c_void_p, c_void_p,
         c_void_p, c_void_p],
    ),
    "nnx_crop_normalize_masked": (
        ctypes.c_int,
        [c_void_p, ctypes.c_int, c_i64_p, c_int_p, c_i64_p, c_i64_p, c_int_p,
         ctypes.POINTER(ctypes.c_float), c_void_p, c_i64_p, c_i64_p, c_void_p, c_void_p],
    ),
    "nnx_crop_normalize": (
        ctypes.c_int,
        [c_void_p, ctypes.c_int, c_i64_p, c_int_p, c_i64_p, c_i64_p, c_int_p,
         ctypes.POINTER(ctypes.c_float), c_void_p, c_void_p],
    ),
    "nnx_resample_spline_workspace": (ctypes.c_size_t, [c_i64_p, c_i64_p, ctypes.c_int]),
    "nnx_resample_spline": (
        ctypes.c_int,
        [c_void_p, ctypes.c_int, c_i64_p, c_i64_p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
         c_void_p, ctypes.c_size_t, c_void_p, c_void_p],
    ),
    "nnx_tconv3d_gemm": (
        ctypes.c_int,
        [c_void_p, ctypes.c_int, c_void_p, c_void_p, c_void_p, ctypes.c_int, c_int_p, ctypes.c_int,
         c_int_p, c_void_p],
    ),
    "nnx_conv1x1": (
        ctypes.c_int, [c_void_p, ctypes.c_int, c_void_p, c_void_p, c_void_p, ctypes.c_int64, ctypes.c_int, c_void_p]
    ),
    "nnx_sw_gather_flip": (
        ctypes.c_int,
        [c_void_p, ctypes.c_int, c_i64_p, c_int_p, c_int_p, c_int_p, c_int_p, ctypes.c_int, c_void_p, c_void_p],
    ),
    "nnx_sw_accumulate": (
        ctypes.c_int,
        [c_void_p, ctypes.c_int, c_int_p, ctypes.c_int, c_int_p, c_void_p, c_int_p, c_i64_p, ctypes.c_int,
         c_void_p, c_void_p, c_void_p],
    ),
    "nnx_sw_fold_add": (
        ctypes.c_int,
        [c_void_p, c_void_p, ctypes.c_int, c_i64_p, c_int_p, c_i64_p, ctypes.c_int, ctypes.c_int, c_void_p,
         c_void_p],
    ),
    "nnx_sw_fold_finalize": (
        ctypes.c_int,
        [c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_int, ctypes.c_int, c_void_p, c_void_p, c_void_p,
         c_void_p],
    ),
    "nnx_profile_begin": (ctypes.c_int, []),
    "nnx_profile_end": (ctypes.c_int, [c_int_p]),
    "nnx_profile_read": (
        ctypes.c_int,
        [ctypes.c_int, ctypes.POINTER(ctypes.c_char_p), c_int_p, ctypes.POINTER(ctypes.c_double),
         ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double)],
    ),
    "nnx_avgpool3d": (
        ctypes.c_int, [c_void_p, c_void_p, ctypes.c_int, c_int_p, ctypes.c_int, c_int_p, c_void_p]
    ),
}

EXPORTED_SYMBOLS = tuple(_SIGNATURES)

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def library_path() -> Path:
    return LIB_PATH


def load() -> ctypes.CDLL:
    """Load (once) and return the HIP library; raise ``NativeUnavailable`` if absent."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.is_file():
            raise NativeUnavailable(
                f"{LIB_NAME} is not built at {LIB_PATH}; run __graft_entry__.build() "
                "(make -C nnunet-mlx_amd/csrc). There is no CPU fallback."
            )
        try:
            lib = ctypes.CDLL(str(LIB_PATH), mode=ctypes.RTLD_GLOBAL)
        except OSError as error:
            raise NativeUnavailable(f"cannot load {LIB_PATH}: {error}") from error
        for name, (restype, argtypes) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = lib
        return lib


def last_error() -> str:
    message = load().nnx_last_error()
    return message.decode("utf-8", "replace") if message else ""


def check(status: int, what: str = "") -> None:
    """Raise the Python error matching a library status code."""
    if status == NNX_OK:
        return
    message = last_error()
    if what:
        message = f"{what}: {message}"
    if status in (NNX_ERR_INVALID, NNX_ERR_NONFINITE):
        raise ContractError(message)
    raise NativeError(message)


def name_nonfinite_layer(error: ContractError, rerun) -> None:
    """A forward produced non-finite logits (``error``): run it again (``rerun``) with the
    library's layer checks on (nnx_set_layer_checks) and raise ContractError naming the first
    layer whose output held non-finite values.  With finite inputs and weights that is a layer
    whose input activations left the split-fp16 operand range.  Re-raises ``error`` when no
    layer check fires."""
    lib = load()
    check(lib.nnx_set_layer_checks(1), "nnx_set_layer_checks")
    try:
        rerun()
    except ContractError as located:
        if "layer check" not in str(located):
            raise
        raise ContractError(
            f"non-finite logits: {located}.  The split-fp16 precisions take layer inputs below "
            "65504 in magnitude (8188 at Winograd layers, whose input transform sums 8 of "
            "them); build this network with precision='fp32'") from error
    finally:
        lib.nnx_set_layer_checks(0)
    raise error


def ints(values) -> ctypes.Array:
    seq = [int(v) for v in values]
    return (ctypes.c_int * max(1, len(seq)))(*seq)


def i64s(values) -> ctypes.Array:
    seq = [int(v) for v in values]
    return (ctypes.c_int64 * max(1, len(seq)))(*seq)


def ptr(tensor: torch.Tensor | None) -> int | None:
    """Device pointer of a contiguous CUDA tensor (None stays NULL)."""
    if tensor is None:
        return None
    if not tensor.is_cuda:
        raise ContractError("the HIP path needs device tensors")
    if not tensor.is_contiguous():
        raise ContractError("the HIP path needs contiguous tensors")
    return tensor.data_ptr()


def stream_handle(device: torch.device | None = None) -> int:
    return torch.cuda.current_stream(device).cuda_stream


class KernelProfile:
    """Per-kernel-class HIP-event timings of library launches (nnx_profile_*)."""

    def __enter__(self) -> "KernelProfile":
        check(load().nnx_profile_begin(), "nnx_profile_begin")
        self.classes: dict[str, dict[str, float]] = {}
        return self

    def __exit__(self, *exc) -> None:
        lib = load()
        count = ctypes.c_int()
        check(lib.nnx_profile_end(ctypes.byref(count)), "nnx_profile_end")
        for index in range(count.value):
            name = ctypes.c_char_p()
            launches = ctypes.c_int()
            ms, flops, nbytes = ctypes.c_double(), ctypes.c_double(), ctypes.c_double()
            check(lib.nnx_profile_read(index, ctypes.byref(name), ctypes.byref(launches),
                                       ctypes.byref(ms), ctypes.byref(flops), ctypes.byref(nbytes)))
            self.classes[name.value.decode()] = {
                "launches": launches.value, "ms": ms.value, "flops": flops.value, "bytes": nbytes.value,
            }
