"""NIfTI-1 single-file images (``.nii`` / ``.nii.gz``) in nnU-Net's SimpleITK array layout.

The reference reads and writes NIfTI through SimpleITK
(src/nnunet_mlx/storage/imageio.py:214-320): ``GetArrayFromImage`` gives the voxels as a
C-order ``(Z, Y, X)`` array (X fastest, as stored on disk), nnU-Net's spacing is the
reversed image spacing ``(sz, sy, sx)``, 4-D files carry channels in the leading array
axis, and every channel file of a case must share shape and geometry.  Labels are written
as uint8 when the largest label is below 255, else uint16
(src/nnunet_mlx/storage/imageio.py:289-320, 647-666), with the input's geometry.

This module parses the 348-byte NIfTI-1 header itself (no SimpleITK or nibabel here):
stored values are scaled by ``scl_slope`` / ``scl_inter`` when the slope is nonzero and
the pair is not the identity, computed in float64 and returned as float32.  The output
label image reuses the input header's geometry fields (pixdim, qform, sform, units), so the
mask lies on exactly the input grid.
"""

from __future__ import annotations

import gzip
import struct
from collections.abc import Mapping, Sequence
from dataclasses import dataclass
from pathlib import Path

import numpy as np

from nnunet_mlx.errors import ContractError

NIFTI_ENDINGS = (".nii.gz", ".nii")
HEADER_BYTES = 348
DATA_OFFSET = 352

# NIfTI-1 datatype codes -> numpy element types
_DTYPES = {2: np.uint8, 4: np.int16, 8: np.int32, 16: np.float32, 64: np.float64,
           256: np.int8, 512: np.uint16, 768: np.uint32, 1024: np.int64, 1280: np.uint64}
_CODES = {np.dtype(v): k for k, v in _DTYPES.items()}


@dataclass(frozen=True)
class NiftiImage:
    """One image: ``array`` in SimpleITK layout ((Z, Y, X) or (C, Z, Y, X) for 4-D
    files), ``spacing`` in the image's (x, y, z) order, and the raw header."""

    array: np.ndarray
    spacing: tuple[float, ...]
    header: bytes

    @property
    def affine(self) -> np.ndarray:
        """The sform rows when ``sform_code`` > 0, else diag(spacing) — informational."""
        endian = _endian(self.header)
        sform_code = struct.unpack_from(endian + "h", self.header, 254)[0]
        if sform_code > 0:
            rows = struct.unpack_from(endian + "12f", self.header, 280)
            return np.vstack([np.asarray(rows, dtype=np.float64).reshape(3, 4), [0, 0, 0, 1]])
        return np.diag([*self.spacing[:3], 1.0])


def _endian(header: bytes) -> str:
    if struct.unpack_from("<i", header, 0)[0] == HEADER_BYTES:
        return "<"
    if struct.unpack_from(">i", header, 0)[0] == HEADER_BYTES:
        return ">"
    raise ContractError("not a NIfTI-1 file (sizeof_hdr is not 348)")


def _read_bytes(path: Path) -> bytes:
    opener = gzip.open if path.name.endswith(".gz") else open
    try:
        with opener(path, "rb") as handle:
            return handle.read()
    except (OSError, EOFError) as error:
        raise ContractError(f"cannot read NIfTI file {path}: {error}") from error


def read_nifti(path: str | Path) -> NiftiImage:
    """Read one single-file NIfTI-1 image (2-D to 4-D, scalar voxel types)."""
    source = Path(path)
    if not source.name.endswith(NIFTI_ENDINGS):
        raise ContractError(f"nnU-Net input must be a NIfTI image (.nii or .nii.gz): {source}")
    raw = _read_bytes(source)
    if len(raw) < DATA_OFFSET:
        raise ContractError(f"NIfTI file {source} is truncated")
    header = raw[:HEADER_BYTES]
    endian = _endian(header)
    if header[344:348] != b"n+1\0":
        raise ContractError(f"{source} is not a single-file NIfTI-1 image (magic n+1)")
    dim = struct.unpack_from(endian + "8h", header, 40)
    ndim = dim[0]
    if not 2 <= ndim <= 4 or any(d < 1 for d in dim[1:ndim + 1]):
        raise ContractError(f"{source}: NIfTI images must be 2-D, 3-D or 4-D with positive sizes")
    datatype = struct.unpack_from(endian + "h", header, 70)[0]
    if datatype not in _DTYPES:
        raise ContractError(f"{source}: unsupported NIfTI datatype code {datatype}")
    pixdim = struct.unpack_from(endian + "8f", header, 76)
    offset = int(struct.unpack_from(endian + "f", header, 108)[0])
    slope, inter = struct.unpack_from(endian + "2f", header, 112)
    dtype = np.dtype(_DTYPES[datatype]).newbyteorder(endian)
    sizes = dim[1:ndim + 1]
    count = int(np.prod(sizes))
    if offset < DATA_OFFSET or len(raw) < offset + count * dtype.itemsize:
        raise ContractError(f"NIfTI file {source} is truncated")
    values = np.frombuffer(raw, dtype=dtype, count=count, offset=offset)
    array = values.reshape(tuple(reversed(sizes))).astype(dtype.newbyteorder("="))
    if slope != 0 and not (slope == 1 and inter == 0):
        array = (array.astype(np.float64) * slope + inter).astype(np.float32)
    spacing = tuple(float(v) for v in pixdim[1:min(ndim, 3) + 1])
    if any(not np.isfinite(s) or s <= 0 for s in spacing):
        raise ContractError(f"{source}: voxel spacing must be positive")
    return NiftiImage(np.ascontiguousarray(array), spacing, header)


def read_images(image_files: Sequence[str | Path]) -> tuple[np.ndarray, dict[str, object]]:
    """Co-registered channel files -> ((C, Z, Y, X) float32, properties).

    ``properties["spacing"]`` is nnU-Net's (z, y, x) spacing; 2-D files become one channel
    with a singleton Z axis and the placeholder spacing (999 * max, sy, sx); 4-D files
    contribute their leading axis as channels.  Every file must share array shape and
    spacing; the first file's header is kept for writing the label image.
    Reference: src/nnunet_mlx/storage/imageio.py:227-286."""
    paths = tuple(Path(p) for p in image_files)
    if not paths:
        raise ContractError("raw prediction requires at least one image file")
    missing = [str(p) for p in paths if not p.is_file()]
    if missing:
        raise ContractError(f"input image files do not exist: {missing}")
    arrays, spacings, headers = [], [], []
    for path in paths:
        image = read_nifti(path)
        array = image.array
        if array.ndim == 2:
            array = array[None, None]
            spacing = (max(image.spacing) * 999, *reversed(image.spacing))
        elif array.ndim == 3:
            array = array[None]
            spacing = tuple(reversed(image.spacing))
        else:
            spacing = tuple(reversed(image.spacing))
        arrays.append(array)
        spacings.append(spacing)
        headers.append(image)
    shapes = {a.shape[1:] for a in arrays}
    if len(shapes) != 1:
        raise ContractError(f"channel images differ in shape: {sorted(shapes)}")
    if any(not np.allclose(s, spacings[0], rtol=0, atol=1e-6) for s in spacings[1:]):
        raise ContractError("channel images differ in voxel spacing")
    data = np.vstack([a.astype(np.float32, copy=False) for a in arrays])
    if not np.isfinite(data).all():
        raise ContractError("input images contain non-finite values")
    properties: dict[str, object] = {
        "spacing": tuple(float(v) for v in spacings[0]),
        "nifti_header": headers[0].header,
        "nifti_spatial_dims": min(headers[0].array.ndim, 3),
    }
    return data, properties


def label_dtype(labels: np.ndarray) -> type[np.uint8] | type[np.uint16]:
    """uint8 when the largest label is below 255, else uint16
    (src/nnunet_mlx/storage/imageio.py:661-665)."""
    return np.uint8 if int(np.max(labels, initial=0)) < 255 else np.uint16


def write_segmentation(segmentation: np.ndarray, output_file: str | Path,
                       properties: Mapping[str, object], *, overwrite: bool) -> None:
    """Write a (Z, Y, X) label map on the grid of the image whose header ``properties``
    holds (``read_images``); gzip-compressed for ``.nii.gz``.
    Reference: src/nnunet_mlx/storage/imageio.py:289-320."""
    target = Path(output_file)
    if not target.name.endswith(NIFTI_ENDINGS):
        raise ContractError(f"segmentation output must end in .nii or .nii.gz: {target}")
    if target.exists() and not overwrite:
        raise ContractError(f"segmentation output already exists: {target}")
    if target.exists() and not target.is_file():
        raise ContractError(f"segmentation output is not a file: {target}")
    labels = np.asarray(segmentation)
    if labels.ndim != 3 or not np.issubdtype(labels.dtype, np.integer):
        raise ContractError("export segmentation must be an integer (Z, Y, X) array")
    if labels.size and (labels.min() < 0 or labels.max() > np.iinfo(np.uint16).max):
        raise ContractError("export segmentation labels must lie in the uint16 range")
    source = properties.get("nifti_header")
    if not isinstance(source, bytes) or len(source) != HEADER_BYTES:
        raise ContractError("segmentation export needs the input image's NIfTI header")
    spatial = int(properties.get("nifti_spatial_dims", 3))
    if spatial == 2:
        if labels.shape[0] != 1:
            raise ContractError("2-D segmentation export requires singleton depth")
        sizes = (labels.shape[2], labels.shape[1])
    else:
        sizes = (labels.shape[2], labels.shape[1], labels.shape[0])
    dtype = np.dtype(label_dtype(labels))
    endian = _endian(source)
    header = bytearray(source)
    struct.pack_into(endian + "8h", header, 40, len(sizes), *sizes, *([1] * (7 - len(sizes))))
    struct.pack_into(endian + "2h", header, 70, _CODES[dtype], dtype.itemsize * 8)
    struct.pack_into(endian + "f", header, 108, float(DATA_OFFSET))
    struct.pack_into(endian + "2f", header, 112, 1.0, 0.0)   # no intensity scaling
    struct.pack_into(endian + "2f", header, 124, 0.0, 0.0)   # cal_max, cal_min
    body = np.ascontiguousarray(labels.astype(dtype.newbyteorder(endian))).tobytes()
    payload = bytes(header) + b"\0\0\0\0" + body
    target.parent.mkdir(parents=True, exist_ok=True)
    staging = target.with_name(f".{target.name}.partial")
    if target.name.endswith(".gz"):
        with gzip.open(staging, "wb", compresslevel=4) as handle:
            handle.write(payload)
    else:
        staging.write_bytes(payload)
    staging.replace(target)


def write_nifti(path: str | Path, array: np.ndarray, spacing: Sequence[float], *,
                affine: np.ndarray | None = None) -> None:
    """Write a (Z, Y, X) (or (Y, X)) array as a NIfTI-1 image with the given (x, y, z)
    spacing and optional 4x4 sform (used to build inputs for tests and benchmarks)."""
    values = np.asarray(array)
    if values.ndim not in (2, 3) or np.dtype(values.dtype) not in _CODES:
        raise ContractError("write_nifti takes a 2-D or 3-D array of a NIfTI scalar type")
    header = bytearray(HEADER_BYTES)
    struct.pack_into("<i", header, 0, HEADER_BYTES)
    sizes = tuple(reversed(values.shape))
    struct.pack_into("<8h", header, 40, len(sizes), *sizes, *([1] * (7 - len(sizes))))
    dtype = np.dtype(values.dtype)
    struct.pack_into("<2h", header, 70, _CODES[dtype], dtype.itemsize * 8)
    pix = [1.0] + [float(s) for s in spacing][:len(sizes)]
    pix += [1.0] * (8 - len(pix))
    struct.pack_into("<8f", header, 76, *pix)
    struct.pack_into("<f", header, 108, float(DATA_OFFSET))
    struct.pack_into("<2f", header, 112, 1.0, 0.0)
    header[123] = 2   # millimetres
    if affine is None:
        affine = np.diag([*[float(s) for s in spacing][:3], 1.0])
    struct.pack_into("<2h", header, 252, 0, 2)   # qform unknown, sform aligned
    struct.pack_into("<12f", header, 280, *np.asarray(affine, dtype=np.float64)[:3].reshape(-1))
    header[344:348] = b"n+1\0"
    body = np.ascontiguousarray(values.astype(dtype.newbyteorder("<"))).tobytes()
    payload = bytes(header) + b"\0\0\0\0" + body
    target = Path(path)
    target.parent.mkdir(parents=True, exist_ok=True)
    if target.name.endswith(".gz"):
        with gzip.open(target, "wb", compresslevel=1) as handle:
            handle.write(payload)
    else:
        target.write_bytes(payload)
