"""The packed-model container (lws.pack layout, packed_store.py:41-141):
round trip through safetensors, the metadata payload field by field, a file
written the way the reference packer writes it (keys and JSON built here
without the library's writer), and refusal of malformed files (format
version, AC-008; missing or short streams; wrong format name)."""

from __future__ import annotations

import json

import numpy as np
import pytest
import torch

from conftest import GOLDEN_NAMES, golden_as_encoding, load_golden
from oracle import se12_codec as o
from se12_amd import packed
from se12_amd.format import UnsupportedFormatVersionError, make_se12_tensor


def _tensor(enc: dict):
    rows, cols = enc["shape"]
    return make_se12_tensor(enc["sm"], enc["ec"], enc["esc"], enc["fallback_bitmap"], enc["fallback_raw"],
                            enc["codebook"], rows, cols)


def _streams_equal(a, b) -> bool:
    sa, sb = a.streams, b.streams
    pairs = [(sa.primary.sm.value, sb.primary.sm.value), (sa.primary.ec.value, sb.primary.ec.value),
             (sa.escape_handling.esc.value, sb.escape_handling.esc.value),
             (sa.escape_handling.fallback.bitmap.value, sb.escape_handling.fallback.bitmap.value),
             (sa.escape_handling.fallback.raw.value, sb.escape_handling.fallback.raw.value)]
    return all(np.array_equal(np.asarray(x).reshape(-1), np.asarray(y).reshape(-1)) for x, y in pairs) and \
        a.metadata == b.metadata


def test_eligibility_rule():
    assert packed.is_eligible(torch.zeros((4, 4), dtype=torch.bfloat16))
    assert not packed.is_eligible(torch.zeros((4,), dtype=torch.bfloat16))
    assert not packed.is_eligible(torch.zeros((4, 4), dtype=torch.float32))
    assert not packed.is_eligible(torch.zeros((2, 4, 4), dtype=torch.bfloat16))


def test_round_trip_keeps_every_stream_and_passthrough(tmp_path):
    encs = {f"layer.{i}.weight": golden_as_encoding(load_golden(n)) for i, n in enumerate(GOLDEN_NAMES)}
    se12 = {k: _tensor(e) for k, e in encs.items()}
    passthrough = {"norm.weight": torch.arange(7, dtype=torch.bfloat16), "step": torch.tensor([3], dtype=torch.int64),
                   "scale": torch.full((2, 3), 0.5, dtype=torch.float32)}
    path = packed.write_packed_file(tmp_path / "model-00001-of-00001.safetensors", se12, passthrough)
    back = packed.read_packed(tmp_path)
    assert back.files == (path,)
    assert set(back.se12) == set(se12) and set(back.passthrough) == set(passthrough)
    for k in se12:
        assert _streams_equal(se12[k], back.se12[k]), k
    for k, t in passthrough.items():
        assert back.passthrough[k].dtype == t.dtype and torch.equal(back.passthrough[k], t)
    # decoding what was read gives the original bits
    for k, e in encs.items():
        t = back.se12[k]
        s = t.streams
        enc = {"sm": s.primary.sm.value, "ec": s.primary.ec.value, "esc": s.escape_handling.esc.value,
               "fallback_bitmap": s.escape_handling.fallback.bitmap.value,
               "fallback_raw": s.escape_handling.fallback.raw.value,
               "codebook": np.array(t.metadata.codebook.exponents, dtype=np.uint8), "shape": e["shape"]}
        assert np.array_equal(o.decode(enc), o.decode(e))


def test_metadata_payload_matches_the_packer(tmp_path):
    from safetensors import safe_open

    g = load_golden("ragged_20x300")
    t = _tensor(golden_as_encoding(g))
    path = packed.write_packed_file(tmp_path / "m.safetensors", {"w": t}, {"b": torch.zeros(3, dtype=torch.float16)})
    with safe_open(str(path), framework="pt") as f:
        payload = json.loads(f.metadata()["se12"])
        keys = sorted(f.keys())
        esc = f.get_tensor("w.se12.esc")
        raw = f.get_tensor("w.se12.fallback_raw")
    assert payload["format"] == "SE12" and payload["format_version"] == 1
    assert payload["tensors"]["w"] == {"eligible": True, "shape": [20, 300], "dtype": "torch.bfloat16", "tile_rows": 16,
                                       "tile_cols": 256, "escape_budget": 16,
                                       "codebook": [int(c) for c in g["codebook"]]}
    assert payload["tensors"]["b"] == {"eligible": False, "shape": [3], "dtype": "torch.float16"}
    assert keys == ["b", "w.se12.ec", "w.se12.esc", "w.se12.fallback_bitmap", "w.se12.fallback_raw", "w.se12.sm"]
    assert esc.dtype == torch.uint8 and tuple(esc.shape) == (4, 16)   # [tiles, budget] as codec.py:342
    assert raw.dtype == torch.int16


def test_reads_a_file_laid_out_by_the_reference_packer(tmp_path):
    """Keys and metadata written here directly with safetensors, as
    packed_store.py:71-141 writes them (esc [tiles, 16], streams as numpy
    arrays, pass-through under its own name)."""
    import safetensors.torch

    g = load_golden("fallback_16x256")
    tensors = {
        "model.w.se12.sm": torch.from_numpy(g["sm"].astype(np.uint8)),
        "model.w.se12.ec": torch.from_numpy(g["ec"].astype(np.uint8)),
        "model.w.se12.esc": torch.from_numpy(g["esc"].astype(np.uint8).reshape(-1, 16)),
        "model.w.se12.fallback_bitmap": torch.from_numpy(g["fallback_bitmap"].astype(np.uint8)),
        "model.w.se12.fallback_raw": torch.from_numpy(g["fallback_raw"].astype(np.int16)),
        "model.norm": torch.ones(5, dtype=torch.bfloat16),
    }
    meta = {"format": "SE12", "format_version": 1, "tensors": {
        "model.w": {"eligible": True, "shape": [16, 256], "dtype": "torch.bfloat16", "tile_rows": 16, "tile_cols": 256,
                    "escape_budget": 16, "codebook": [int(c) for c in g["codebook"]]},
        "model.norm": {"eligible": False, "shape": [5], "dtype": "torch.bfloat16"}}}
    path = tmp_path / "ref.safetensors"
    safetensors.torch.save_file(tensors, str(path), metadata={"se12": json.dumps(meta)})
    back = packed.read_packed(path)
    enc = golden_as_encoding(g)
    assert _streams_equal(back.se12["model.w"], _tensor(enc))
    assert torch.equal(back.passthrough["model.norm"], torch.ones(5, dtype=torch.bfloat16))
    assert packed.describe(back)["se12_tensors"] == 1


def _rewrite(path, mutate_meta=None, drop=None, replace=None):
    import safetensors.torch
    from safetensors import safe_open

    with safe_open(str(path), framework="pt") as f:
        meta = json.loads(f.metadata()["se12"])
        tensors = {k: f.get_tensor(k) for k in f.keys()}
    if mutate_meta:
        mutate_meta(meta)
    if drop:
        tensors.pop(drop)
    if replace:
        tensors.update(replace)
    safetensors.torch.save_file(tensors, str(path), metadata={"se12": json.dumps(meta)})


@pytest.mark.parametrize("case", ["version", "format", "missing", "short", "codebook", "passthrough_dtype"])
def test_malformed_files_are_refused(tmp_path, case):
    g = load_golden("normal_32x512")
    path = packed.write_packed_file(tmp_path / "m.safetensors", {"w": _tensor(golden_as_encoding(g))},
                                    {"n": torch.ones(4, dtype=torch.float32)})
    if case == "version":
        _rewrite(path, mutate_meta=lambda m: m.update(format_version=2))
        with pytest.raises(UnsupportedFormatVersionError, match="found format version 2, supported: 1"):
            packed.read_packed(path)
        return
    if case == "format":
        _rewrite(path, mutate_meta=lambda m: m.update(format="SE13"))
    elif case == "missing":
        _rewrite(path, drop="w.se12.ec")
    elif case == "short":
        _rewrite(path, replace={"w.se12.sm": torch.zeros(100, dtype=torch.uint8)})
    elif case == "codebook":
        _rewrite(path, mutate_meta=lambda m: m["tensors"]["w"].update(codebook=[1, 2, 3]))
    elif case == "passthrough_dtype":
        _rewrite(path, mutate_meta=lambda m: m["tensors"]["n"].update(dtype="torch.float16"))
    with pytest.raises(packed.PackedFormatError):
        packed.read_packed(path)


def test_duplicate_names_across_files_are_refused(tmp_path):
    t = _tensor(golden_as_encoding(load_golden("normal_32x512")))
    packed.write_packed_file(tmp_path / "a.safetensors", {"w": t})
    packed.write_packed_file(tmp_path / "b.safetensors", {"w": t})
    with pytest.raises(packed.PackedFormatError, match="two files"):
        packed.read_packed(tmp_path)
