"""SE12 format types: host-side mirror of the reference's domain value objects.

Class and attribute names follow the reference (lws/domain/weights.py:22-37,
lws/domain/se12/tile.py:19-62, lws/domain/se12/codebook.py:19-30,
lws/domain/se12/codec.py:32-108, lws/domain/se12/container.py:7-27,
lws/domain/se12/summary.py:71-92), so an `Se12Tensor` built by the reference
encoder can be handed to this package's kernels unchanged (attribute access
only: `tensor.streams.primary.sm.value` and so on).

`Se12DeviceTensor` is this package's own addition: the same streams resident
in HBM as torch tensors, which is what the HIP library binds to.
"""

from __future__ import annotations

import dataclasses
from typing import Any

import numpy as np

TILE_ROWS = 16
TILE_COLS = 256
TILE_SIZE = TILE_ROWS * TILE_COLS
ESCAPE_BUDGET = 16
CODEBOOK_SIZE = 15
ESCAPE_CODE = 15
FORMAT_NAME = "SE12"
CURRENT_FORMAT_VERSION = 1
SUPPORTED_FORMAT_VERSIONS = (1,)
# per tile: 4096 sm + 2048 ec + 16 esc bytes
TILE_STREAM_BYTES = TILE_SIZE + TILE_SIZE // 2 + ESCAPE_BUDGET


class UnsupportedFormatVersionError(ValueError):
    """A packed file declares a format version this codec does not know (container.py:12)."""


@dataclasses.dataclass(frozen=True)
class FormatVersion:
    value: int


def validate_format_version(found: FormatVersion) -> None:
    """Refuses an unknown version, naming found and supported ones (container.py:21-27)."""
    if found.value in SUPPORTED_FORMAT_VERSIONS:
        return
    supported = ", ".join(str(v) for v in SUPPORTED_FORMAT_VERSIONS)
    raise UnsupportedFormatVersionError(f"found format version {found.value}, supported: {supported}")


@dataclasses.dataclass(frozen=True)
class Bf16Weights:
    """Flattened int16 bit pattern of a BF16 tensor (weights.py:22-37)."""

    bit_pattern: np.ndarray

    def __post_init__(self) -> None:
        if self.bit_pattern.dtype != np.int16:
            raise ValueError("Bf16Weights requires an int16 bit-pattern view")
        if self.bit_pattern.ndim != 1:
            raise ValueError("Bf16Weights requires a flattened 1-D array")


@dataclasses.dataclass(frozen=True)
class TileShape:
    rows: int
    cols: int


@dataclasses.dataclass(frozen=True)
class EscapeBudget:
    value: int


@dataclasses.dataclass(frozen=True)
class MatrixShape:
    rows: int
    cols: int


@dataclasses.dataclass(frozen=True)
class Codebook:
    """The 15 exponent byte values, most frequent first (codebook.py:19-30)."""

    exponents: tuple[int, ...]

    def __post_init__(self) -> None:
        if len(self.exponents) != CODEBOOK_SIZE:
            raise ValueError(f"Codebook needs exactly {CODEBOOK_SIZE} entries, got {len(self.exponents)}")


@dataclasses.dataclass(frozen=True)
class SignMantissaBytes:
    value: np.ndarray


@dataclasses.dataclass(frozen=True)
class EcBytes:
    value: np.ndarray


@dataclasses.dataclass(frozen=True)
class EscBytes:
    value: np.ndarray


@dataclasses.dataclass(frozen=True)
class FallbackBitmap:
    value: np.ndarray


@dataclasses.dataclass(frozen=True)
class FallbackRaw:
    value: np.ndarray


@dataclasses.dataclass(frozen=True)
class PrimaryStreams:
    sm: SignMantissaBytes
    ec: EcBytes


@dataclasses.dataclass(frozen=True)
class FallbackData:
    bitmap: FallbackBitmap
    raw: FallbackRaw


@dataclasses.dataclass(frozen=True)
class EscapeHandling:
    esc: EscBytes
    fallback: FallbackData


@dataclasses.dataclass(frozen=True)
class Se12Streams:
    primary: PrimaryStreams
    escape_handling: EscapeHandling


@dataclasses.dataclass(frozen=True)
class TilingParameters:
    tile_shape: TileShape
    escape_budget: EscapeBudget


@dataclasses.dataclass(frozen=True)
class Se12Geometry:
    shape: MatrixShape
    tiling: TilingParameters


@dataclasses.dataclass(frozen=True)
class Se12Metadata:
    codebook: Codebook
    geometry: Se12Geometry


@dataclasses.dataclass(frozen=True)
class Se12Tensor:
    """Every stream plus the metadata needed to decode it (codec.py:103-108)."""

    streams: Se12Streams
    metadata: Se12Metadata


def default_tile_shape() -> TileShape:
    return TileShape(rows=TILE_ROWS, cols=TILE_COLS)


def default_escape_budget() -> EscapeBudget:
    return EscapeBudget(value=ESCAPE_BUDGET)


def tile_grid(rows: int, cols: int) -> tuple[int, int]:
    """(tile rows, tile cols) of the padded matrix (lws/adapters/cuda/gemv.py:89-92)."""
    return -(-rows // TILE_ROWS), -(-cols // TILE_COLS)


def bitmap_bytes(tile_count: int) -> int:
    return -(-tile_count // 8)


def make_se12_tensor(sm, ec, esc, bitmap, raw, codebook, rows: int, cols: int) -> Se12Tensor:
    """Wraps host arrays in the reference's container layout."""
    return Se12Tensor(
        streams=Se12Streams(
            primary=PrimaryStreams(sm=SignMantissaBytes(np.asarray(sm)), ec=EcBytes(np.asarray(ec))),
            escape_handling=EscapeHandling(
                esc=EscBytes(np.asarray(esc)),
                fallback=FallbackData(bitmap=FallbackBitmap(np.asarray(bitmap)), raw=FallbackRaw(np.asarray(raw))),
            ),
        ),
        metadata=Se12Metadata(
            codebook=Codebook(tuple(int(c) for c in codebook)),
            geometry=Se12Geometry(
                shape=MatrixShape(rows=int(rows), cols=int(cols)),
                tiling=TilingParameters(tile_shape=default_tile_shape(), escape_budget=default_escape_budget()),
            ),
        ),
    )


def se12_tensor_byte_size(tensor: Any) -> int:
    """All five streams plus the 15 codebook bytes (summary.py:71-92): the
    algorithmic byte count of one pass over the weights."""
    s = tensor.streams
    total = (
        s.primary.sm.value.nbytes + s.primary.ec.value.nbytes + s.escape_handling.esc.value.nbytes
        + s.escape_handling.fallback.bitmap.value.nbytes + s.escape_handling.fallback.raw.value.nbytes
    )
    return int(total) + len(tensor.metadata.codebook.exponents)


def packed_byte_size(rows: int, cols: int, fallback_tiles: int) -> int:
    """Same count from the shape and the number of fallback tiles."""
    tr, tc = tile_grid(rows, cols)
    t = tr * tc
    return t * TILE_STREAM_BYTES + bitmap_bytes(t) + fallback_tiles * TILE_SIZE * 2 + CODEBOOK_SIZE


def validate_streams(tensor: Any) -> None:
    """Checks each stream's dtype and size against the shape (a malformed
    stream would otherwise make a kernel read out of bounds)."""
    shape = tensor.metadata.geometry.shape
    tiling = tensor.metadata.geometry.tiling
    if (tiling.tile_shape.rows, tiling.tile_shape.cols) != (TILE_ROWS, TILE_COLS):
        raise ValueError(f"unsupported tile shape {tiling.tile_shape}")
    if tiling.escape_budget.value != ESCAPE_BUDGET:
        raise ValueError(f"unsupported escape budget {tiling.escape_budget.value}")
    tr, tc = tile_grid(shape.rows, shape.cols)
    t = tr * tc
    s = tensor.streams
    expect = {
        "sm": (s.primary.sm.value, np.uint8, t * TILE_SIZE),
        "ec": (s.primary.ec.value, np.uint8, t * TILE_SIZE // 2),
        "esc": (s.escape_handling.esc.value, np.uint8, t * ESCAPE_BUDGET),
        "fallback_bitmap": (s.escape_handling.fallback.bitmap.value, np.uint8, bitmap_bytes(t)),
    }
    for name, (arr, dtype, size) in expect.items():
        if arr.dtype != dtype or arr.size != size:
            raise ValueError(f"stream {name}: expected {size} x {np.dtype(dtype).name}, got {arr.size} x {arr.dtype}")
    raw = s.escape_handling.fallback.raw.value
    if raw.dtype != np.int16 or raw.size % TILE_SIZE != 0:
        raise ValueError(f"stream fallback_raw: expected whole tiles of int16, got {raw.size} x {raw.dtype}")
    nfb = int(np.unpackbits(s.escape_handling.fallback.bitmap.value, count=t).sum())
    if raw.size != nfb * TILE_SIZE:
        raise ValueError(f"bitmap marks {nfb} fallback tiles but fallback_raw holds {raw.size // TILE_SIZE}")


def validate_device_streams(dt: "Se12DeviceTensor") -> None:
    """The device-side counterpart of `validate_streams`: every stream a torch
    tensor on one GPU, contiguous, of the right dtype and size for the shape
    (the library binds to these pointers and its kernels read every byte the
    shape implies). The fallback count against the bitmap is checked by the
    library at bind."""
    import torch

    if dt.rows <= 0 or dt.cols <= 0:
        raise ValueError(f"shape must be positive, got [{dt.rows}, {dt.cols}]")
    tr, tc = tile_grid(dt.rows, dt.cols)
    t = tr * tc
    expect = {
        "sm": (dt.sm, torch.uint8, t * TILE_SIZE),
        "ec": (dt.ec, torch.uint8, t * TILE_SIZE // 2),
        "esc": (dt.esc, torch.uint8, t * ESCAPE_BUDGET),
        "codebook": (dt.codebook, torch.uint8, CODEBOOK_SIZE),
        "fallback_bitmap": (dt.fallback_bitmap, torch.uint8, bitmap_bytes(t)),
    }
    device = dt.sm.device if isinstance(dt.sm, torch.Tensor) else None
    if device is None or device.type != "cuda":
        raise ValueError(f"SE12 streams must be device tensors, sm is on {device}")
    for name, (arr, dtype, size) in expect.items():
        if not isinstance(arr, torch.Tensor) or arr.device != device:
            raise ValueError(f"stream {name} must be a tensor on {device}")
        if arr.dtype != dtype or arr.numel() != size or not arr.is_contiguous():
            raise ValueError(f"stream {name}: expected {size} contiguous x {dtype}, got {arr.numel()} x {arr.dtype}")
    raw = dt.fallback_raw
    if not isinstance(raw, torch.Tensor) or raw.device != device or raw.dtype != torch.int16 \
            or raw.numel() % TILE_SIZE != 0 or not raw.is_contiguous():
        raise ValueError(f"stream fallback_raw must be whole contiguous int16 tiles on {device}")
    if tuple(int(c) for c in dt.codebook_host) != tuple(int(c) for c in dt.codebook.cpu().tolist()):
        raise ValueError("codebook_host differs from the device codebook")


@dataclasses.dataclass
class Se12DeviceTensor:
    """The SE12 streams resident on one GPU (torch tensors), plus metadata."""

    sm: Any
    ec: Any
    esc: Any
    codebook: Any             # uint8 [15] on the device
    fallback_bitmap: Any
    fallback_raw: Any         # int16 [fallback_tiles * 4096] (may be empty)
    rows: int
    cols: int
    codebook_host: tuple[int, ...]

    @property
    def tile_grid(self) -> tuple[int, int]:
        return tile_grid(self.rows, self.cols)

    @property
    def fallback_tiles(self) -> int:
        return int(self.fallback_raw.numel()) // TILE_SIZE

    def byte_size(self) -> int:
        """Algorithmic bytes of one pass (every stream + the codebook)."""
        return packed_byte_size(self.rows, self.cols, self.fallback_tiles)

    def clone(self) -> "Se12DeviceTensor":
        """A copy of every stream in new device memory."""
        return dataclasses.replace(self, sm=self.sm.clone(), ec=self.ec.clone(), esc=self.esc.clone(),
                                   codebook=self.codebook.clone(), fallback_bitmap=self.fallback_bitmap.clone(),
                                   fallback_raw=self.fallback_raw.clone())

    @classmethod
    def from_host(cls, tensor: Any, device=None) -> "Se12DeviceTensor":
        """Uploads a host `Se12Tensor` (the reference container layout)."""
        import torch

        validate_streams(tensor)
        dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
        s = tensor.streams
        shape = tensor.metadata.geometry.shape
        cb = tuple(int(c) for c in tensor.metadata.codebook.exponents)

        def up(a, dtype):
            return torch.from_numpy(np.ascontiguousarray(a).reshape(-1).view(dtype)).to(dev)

        return cls(
            sm=up(s.primary.sm.value, np.uint8),
            ec=up(s.primary.ec.value, np.uint8),
            esc=up(s.escape_handling.esc.value, np.uint8),
            codebook=torch.tensor(cb, dtype=torch.uint8, device=dev),
            fallback_bitmap=up(s.escape_handling.fallback.bitmap.value, np.uint8),
            fallback_raw=up(s.escape_handling.fallback.raw.value, np.int16),
            rows=int(shape.rows),
            cols=int(shape.cols),
            codebook_host=cb,
        )

    def to_host(self) -> Se12Tensor:
        """Downloads into the reference container layout (esc as [tiles, 16])."""
        t = self.tile_grid[0] * self.tile_grid[1]
        return make_se12_tensor(
            self.sm.cpu().numpy(),
            self.ec.cpu().numpy(),
            self.esc.cpu().numpy().reshape(t, ESCAPE_BUDGET),
            self.fallback_bitmap.cpu().numpy(),
            self.fallback_raw.cpu().numpy(),
            self.codebook_host,
            self.rows,
            self.cols,
        )
