"""The packed-model container written by `lws.pack`: SE12 streams and
pass-through tensors in safetensors files.

Layout (lws/adapters/safetensors/packed_store.py:41-141, kept byte-compatible
so that files move both ways between the two implementations):
  - an eligible tensor (BF16 and 2-D, lws/application/codec/pack_model.py:3-7)
    is stored as five tensors `<name>.se12.sm` (uint8), `.ec` (uint8), `.esc`
    (uint8 [tiles, 16]), `.fallback_bitmap` (uint8), `.fallback_raw` (int16);
  - every other tensor is stored under its own name, unchanged;
  - the file metadata holds one JSON blob under the key "se12":
    {"format": "SE12", "format_version": 1, "tensors": {name: {...}}} with, per
    eligible tensor, eligible/shape/dtype/tile_rows/tile_cols/escape_budget/
    codebook, and per pass-through tensor eligible/shape/dtype.
Reading validates the format name and version (lws/domain/se12/container.py:
21-27) and every stream's size against the shape before anything reaches a
kernel.
"""

from __future__ import annotations

import dataclasses
import json
import pathlib
from typing import Any, Iterable

import numpy as np
import torch

from .format import (
    ESCAPE_BUDGET,
    TILE_COLS,
    TILE_ROWS,
    FormatVersion,
    Se12Tensor,
    make_se12_tensor,
    tile_grid,
    validate_format_version,
    validate_streams,
)

FORMAT_NAME = "SE12"
CURRENT_FORMAT_VERSION = 1
METADATA_KEY = "se12"
STREAM_SUFFIXES = ("sm", "ec", "esc", "fallback_bitmap", "fallback_raw")

_DTYPES = {
    "torch.bfloat16": torch.bfloat16,
    "torch.float64": torch.float64,
    "torch.float32": torch.float32,
    "torch.float16": torch.float16,
    "torch.int64": torch.int64,
    "torch.int32": torch.int32,
    "torch.int16": torch.int16,
    "torch.int8": torch.int8,
    "torch.uint8": torch.uint8,
    "torch.bool": torch.bool,
}


class PackedFormatError(ValueError):
    """A packed file that is not a well-formed SE12 container."""


def is_eligible(tensor: torch.Tensor) -> bool:
    """The packer's rule: BF16 and 2-D tensors are SE12-encoded, all others pass
    through (pack_model.py:3-7)."""
    return tensor.dtype == torch.bfloat16 and tensor.dim() == 2


@dataclasses.dataclass
class PackedModel:
    """The tensors of one packed model (all files of a directory, or one file)."""

    se12: dict[str, Se12Tensor]
    passthrough: dict[str, torch.Tensor]
    files: tuple[pathlib.Path, ...]

    def names(self) -> list[str]:
        return sorted(set(self.se12) | set(self.passthrough))


def _se12_metadata(t: Se12Tensor) -> dict:
    g = t.metadata.geometry
    return {
        "eligible": True,
        "shape": [g.shape.rows, g.shape.cols],
        "dtype": "torch.bfloat16",
        "tile_rows": g.tiling.tile_shape.rows,
        "tile_cols": g.tiling.tile_shape.cols,
        "escape_budget": g.tiling.escape_budget.value,
        "codebook": [int(c) for c in t.metadata.codebook.exponents],
    }


def write_packed_file(path, se12: dict[str, Se12Tensor], passthrough: dict[str, torch.Tensor] | None = None) -> pathlib.Path:
    """Writes one container file: the streams of every SE12 tensor and the
    pass-through tensors unchanged (packed_store.py:47-55,71-141)."""
    import safetensors.torch

    path = pathlib.Path(path)
    path.parent.mkdir(parents=True, exist_ok=True)
    tensors: dict[str, torch.Tensor] = {}
    meta: dict[str, dict] = {}
    for name, t in se12.items():
        validate_streams(t)
        s = t.streams
        tr, tc = tile_grid(t.metadata.geometry.shape.rows, t.metadata.geometry.shape.cols)
        arrays = {
            "sm": np.ascontiguousarray(s.primary.sm.value, dtype=np.uint8).reshape(-1),
            "ec": np.ascontiguousarray(s.primary.ec.value, dtype=np.uint8).reshape(-1),
            "esc": np.ascontiguousarray(s.escape_handling.esc.value, dtype=np.uint8).reshape(tr * tc, ESCAPE_BUDGET),
            "fallback_bitmap": np.ascontiguousarray(s.escape_handling.fallback.bitmap.value, dtype=np.uint8).reshape(-1),
            "fallback_raw": np.ascontiguousarray(s.escape_handling.fallback.raw.value, dtype=np.int16).reshape(-1),
        }
        for suffix in STREAM_SUFFIXES:
            tensors[f"{name}.{METADATA_KEY}.{suffix}"] = torch.from_numpy(arrays[suffix])
        meta[name] = _se12_metadata(t)
    for name, t in (passthrough or {}).items():
        if name in meta:
            raise PackedFormatError(f"tensor {name!r} given both as SE12 and as pass-through")
        tensors[name] = t.detach().to("cpu").contiguous()
        meta[name] = {"eligible": False, "shape": list(t.shape), "dtype": str(t.dtype)}
    payload = {"format": FORMAT_NAME, "format_version": CURRENT_FORMAT_VERSION, "tensors": meta}
    safetensors.torch.save_file(tensors, str(path), metadata={METADATA_KEY: json.dumps(payload)})
    return path


def _file_payload(f, path: pathlib.Path) -> dict:
    raw = (f.metadata() or {}).get(METADATA_KEY)
    if raw is None:
        raise PackedFormatError(f"{path}: no {METADATA_KEY!r} metadata (not an SE12 container)")
    payload = json.loads(raw)
    if payload.get("format") != FORMAT_NAME:
        raise PackedFormatError(f"{path}: format {payload.get('format')!r}, expected {FORMAT_NAME!r}")
    validate_format_version(FormatVersion(int(payload.get("format_version", -1))))
    return payload


def read_packed_file(path, names: Iterable[str] | None = None) -> PackedModel:
    """Reads one container file (all tensors, or only `names`)."""
    from safetensors import safe_open

    path = pathlib.Path(path)
    se12: dict[str, Se12Tensor] = {}
    passthrough: dict[str, torch.Tensor] = {}
    with safe_open(str(path), framework="pt") as f:
        payload = _file_payload(f, path)
        keys = set(f.keys())
        wanted = None if names is None else set(names)
        for name, m in payload["tensors"].items():
            if wanted is not None and name not in wanted:
                continue
            if m.get("eligible"):
                if (m.get("tile_rows"), m.get("tile_cols"), m.get("escape_budget")) != (TILE_ROWS, TILE_COLS, ESCAPE_BUDGET):
                    raise PackedFormatError(f"{path}: {name}: unsupported tiling {m}")
                if m.get("dtype") != "torch.bfloat16":
                    raise PackedFormatError(f"{path}: {name}: SE12 tensor of dtype {m.get('dtype')}")
                rows, cols = (int(v) for v in m["shape"])
                streams = {}
                for suffix in STREAM_SUFFIXES:
                    key = f"{name}.{METADATA_KEY}.{suffix}"
                    if key not in keys:
                        raise PackedFormatError(f"{path}: {name}: missing stream {key!r}")
                    streams[suffix] = f.get_tensor(key).numpy()
                try:  # the codebook length and every stream size are checked here
                    t = make_se12_tensor(streams["sm"], streams["ec"], streams["esc"], streams["fallback_bitmap"],
                                         streams["fallback_raw"], m["codebook"], rows, cols)
                    validate_streams(t)
                except ValueError as e:
                    raise PackedFormatError(f"{path}: {name}: {e}") from None
                se12[name] = t
            else:
                if name not in keys:
                    raise PackedFormatError(f"{path}: pass-through tensor {name!r} missing")
                t = f.get_tensor(name)
                if list(t.shape) != list(m["shape"]) or str(t.dtype) != m["dtype"]:
                    raise PackedFormatError(f"{path}: {name}: stored {list(t.shape)} {t.dtype}, metadata says {m['shape']} {m['dtype']}")
                passthrough[name] = t
    return PackedModel(se12=se12, passthrough=passthrough, files=(path,))


def read_packed(path) -> PackedModel:
    """Reads a packed model: one file, or every `*.safetensors` file of a
    directory (one per shard, as the packer writes them)."""
    path = pathlib.Path(path)
    files = sorted(path.glob("*.safetensors")) if path.is_dir() else [path]
    if not files:
        raise PackedFormatError(f"{path}: no .safetensors files")
    out = PackedModel(se12={}, passthrough={}, files=tuple(files))
    for fp in files:
        part = read_packed_file(fp)
        for name in list(part.se12) + list(part.passthrough):
            if name in out.se12 or name in out.passthrough:
                raise PackedFormatError(f"{fp}: tensor {name!r} appears in two files")
        out.se12.update(part.se12)
        out.passthrough.update(part.passthrough)
    return out


def pack_state_dict(state_dict: dict[str, torch.Tensor], path, device=None) -> pathlib.Path:
    """Packs a model's tensors into one container file: eligible tensors are
    SE12-encoded on the GPU (the library's encoder, byte-identical to the
    reference packer's), the rest pass through."""
    from .hip import encode_on_device

    se12: dict[str, Se12Tensor] = {}
    passthrough: dict[str, torch.Tensor] = {}
    dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
    for name, t in state_dict.items():
        if is_eligible(t):
            se12[name] = encode_on_device(t.detach().to(dev)).to_host()
        else:
            passthrough[name] = t
    return write_packed_file(path, se12, passthrough)


def dtype_from_name(name: str) -> torch.dtype:
    if name not in _DTYPES:
        raise PackedFormatError(f"unknown dtype {name!r}")
    return _DTYPES[name]


def describe(model: PackedModel) -> dict[str, Any]:
    """Counts and byte totals of a packed model (the packer's summary terms)."""
    from .format import se12_tensor_byte_size

    se12_bytes = sum(se12_tensor_byte_size(t) for t in model.se12.values())
    bf16_bytes = sum(2 * t.metadata.geometry.shape.rows * t.metadata.geometry.shape.cols for t in model.se12.values())
    return {"se12_tensors": len(model.se12), "passthrough_tensors": len(model.passthrough),
            "se12_bytes": se12_bytes, "bf16_bytes": bf16_bytes,
            "ratio": se12_bytes / bf16_bytes if bf16_bytes else None}
