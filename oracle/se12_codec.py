"""CPU oracle for the SE12 path: a numpy restatement of the reference codec.

TEST INFRASTRUCTURE ONLY. This module is the checker the HIP path is compared
against. Only `tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of
`bench.py` may import it; the product package `se12_amd` never does.

Every function restates one step of the reference's algorithm and cites the
reference file:line it follows (paths relative to the reference repository).

How each function is pinned (checked against something other than itself):
  split_bits / join_bits     exhaustive over all 65,536 bit patterns (closed form
                             and round trip), tests/test_oracle_codec.py
  build_codebook             golden vectors written by the reference encoder
                             (tests/golden/*.npz) including a tie-heavy tensor,
                             plus a brute-force sort on tiny histograms
  encode                     byte equality with the golden vectors (every stream)
  decode                     round trip on the reference's own edge-case lists,
                             padding shapes and forced-fallback construction,
                             and decode(golden streams) == golden input bits
  fallback_ranks             brute-force prefix sum over random bitmaps
  packed_byte_size           arithmetic: 6,160 B per tile + bitmap + raw + 15
  gemv_reference             float64 brute force on small inputs
"""

from __future__ import annotations

import numpy as np

# Format constants: lws/domain/se12/tile.py:19-24 (16x256 tiles, escape budget
# 16, 15-entry codebook, escape code 15, padding bit pattern 0x0000).
TILE_ROWS = 16
TILE_COLS = 256
TILE_SIZE = TILE_ROWS * TILE_COLS
ESCAPE_BUDGET = 16
CODEBOOK_SIZE = 15
ESCAPE_CODE = 15


# ---------------------------------------------------------------------------
# BF16 bit split / join: lws/domain/weights.py:95-119
# ---------------------------------------------------------------------------


def split_bits(bits: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """(exponent byte, sign|mantissa byte) of each BF16 pattern (weights.py:95-106)."""
    u = bits.astype(np.uint16, copy=False)
    exponent = ((u >> 7) & 0xFF).astype(np.uint8)
    sm = (((u >> 8) & 0x80) | (u & 0x7F)).astype(np.uint8)
    return exponent, sm


def join_bits(exponent: np.ndarray, sm: np.ndarray) -> np.ndarray:
    """Inverse of split_bits, as int16 (weights.py:109-119)."""
    e = exponent.astype(np.uint16)
    s = sm.astype(np.uint16)
    return (((s & 0x80) << 8) | (e << 7) | (s & 0x7F)).astype(np.uint16).view(np.int16)


# ---------------------------------------------------------------------------
# geometry: lws/domain/se12/codec.py:210-282, lws/adapters/cuda/gemv.py:89-97
# ---------------------------------------------------------------------------


def tile_grid(rows: int, cols: int) -> tuple[int, int]:
    """(tile rows, tile cols) after padding up to whole tiles (gemv.py:89-92)."""
    return -(-rows // TILE_ROWS), -(-cols // TILE_COLS)


def padded_shape(rows: int, cols: int) -> tuple[int, int]:
    tr, tc = tile_grid(rows, cols)
    return tr * TILE_ROWS, tc * TILE_COLS


def to_tiles(a: np.ndarray) -> np.ndarray:
    """[Rp, Cp] -> [TR, TC, 4096]; tile t = tr*TC + tc, in-tile index lr*256 + lc (codec.py:265-273)."""
    rp, cp = a.shape
    tr, tc = rp // TILE_ROWS, cp // TILE_COLS
    return a.reshape(tr, TILE_ROWS, tc, TILE_COLS).transpose(0, 2, 1, 3).reshape(tr, tc, TILE_SIZE)


def from_tiles(t: np.ndarray) -> np.ndarray:
    """Inverse of to_tiles (codec.py:276-282)."""
    tr, tc, _ = t.shape
    return t.reshape(tr, tc, TILE_ROWS, TILE_COLS).transpose(0, 2, 1, 3).reshape(tr * TILE_ROWS, tc * TILE_COLS)


# ---------------------------------------------------------------------------
# codebook: lws/domain/se12/codebook.py:41-59
# ---------------------------------------------------------------------------


def build_codebook(exponent_2d: np.ndarray, valid_2d: np.ndarray) -> np.ndarray:
    """15 exponent values: by count over REAL weights, descending; equal counts
    go to the larger exponent value first; zero-count values fill the rest
    (codebook.py:55-58: reversed stable argsort of the 256-bin histogram)."""
    counts = np.bincount(exponent_2d[valid_2d].astype(np.int64), minlength=256)
    # Sort key (count desc, exponent desc) as one integer, so the rule is written
    # out directly instead of through argsort's stability.
    key = counts.astype(np.int64) * 256 + np.arange(256, dtype=np.int64)
    order = np.argsort(-key, kind="stable")
    return order[:CODEBOOK_SIZE].astype(np.uint8)


# ---------------------------------------------------------------------------
# encoder: lws/domain/se12/codec.py:111-141 and its helpers (:225-365)
# ---------------------------------------------------------------------------


def encode(bits: np.ndarray, rows: int, cols: int) -> dict:
    """SE12-encode a BF16 matrix given as int16/uint16 bits (codec.py:111-141).

    Returns the five streams plus metadata, named as the packed layout names
    them (lws/adapters/safetensors/packed_store.py:77-81): sm, ec, esc,
    fallback_bitmap, fallback_raw, and codebook, shape.
    """
    bits = np.asarray(bits).reshape(rows, cols).astype(np.uint16, copy=False).view(np.int16)
    rp, cp = padded_shape(rows, cols)
    padded = np.zeros((rp, cp), dtype=np.int16)  # padding = +0.0 (tile.py:1-10, codec.py:225-235)
    padded[:rows, :cols] = bits
    valid = np.zeros((rp, cp), dtype=bool)
    valid[:rows, :cols] = True

    exponent, sm = split_bits(padded)
    codebook = build_codebook(exponent, valid)
    lookup = np.full(256, ESCAPE_CODE, dtype=np.uint8)  # codec.py:297-302
    lookup[codebook] = np.arange(CODEBOOK_SIZE, dtype=np.uint8)
    code = lookup[exponent]
    real_escape = (code == ESCAPE_CODE) & valid
    code = np.where(valid, code, 0).astype(np.uint8)  # padding code pinned to 0 (codec.py:125)

    t_exp = to_tiles(exponent)
    t_esc = to_tiles(real_escape)
    t_code = to_tiles(code)
    t_sm = to_tiles(sm)
    t_raw = to_tiles(padded)

    rank = np.cumsum(t_esc, axis=-1, dtype=np.int32) - 1  # codec.py:131
    fallback = t_esc.sum(axis=-1) > ESCAPE_BUDGET  # codec.py:132-133

    flat_code = t_code.reshape(-1)
    ec = (flat_code[0::2] | (flat_code[1::2] << 4)).astype(np.uint8)  # codec.py:310-314

    ntr, ntc, _ = t_exp.shape
    esc = np.zeros((ntr, ntc, ESCAPE_BUDGET), dtype=np.uint8)  # codec.py:332-343
    keep = t_esc & (rank < ESCAPE_BUDGET) & ~fallback[:, :, None]
    i, j, k = np.nonzero(keep)
    esc[i, j, rank[i, j, k]] = t_exp[i, j, k]

    return {
        "sm": t_sm.reshape(-1).copy(),
        "ec": ec,
        "esc": esc.reshape(ntr * ntc, ESCAPE_BUDGET),
        "fallback_bitmap": np.packbits(fallback.reshape(-1)),  # MSB-first (codec.py:351-353)
        "fallback_raw": t_raw[fallback].reshape(-1).copy(),  # codec.py:363-365
        "codebook": codebook,
        "shape": (rows, cols),
    }


# ---------------------------------------------------------------------------
# decoder: lws/domain/se12/codec.py:144-186 and its helpers (:317-391)
# ---------------------------------------------------------------------------


def unpack_codes(ec: np.ndarray) -> np.ndarray:
    """Two 4-bit codes per byte, even index in the low nibble (codec.py:317-324)."""
    out = np.empty(ec.size * 2, dtype=np.uint8)
    out[0::2] = ec & 0x0F
    out[1::2] = (ec >> 4) & 0x0F
    return out


def unpack_bitmap(bitmap: np.ndarray, tile_count: int) -> np.ndarray:
    """One bit per tile, MSB first within each byte (codec.py:356-360)."""
    return np.unpackbits(bitmap, count=tile_count).astype(bool)


def decode_tiles(enc: dict) -> np.ndarray:
    """Tile-major decoded bit patterns [TR, TC, 4096] int16, fallback tiles restored."""
    rows, cols = enc["shape"]
    ntr, ntc = tile_grid(rows, cols)
    code = unpack_codes(enc["ec"]).reshape(ntr, ntc, TILE_SIZE)
    esc = enc["esc"].reshape(ntr, ntc, ESCAPE_BUDGET)
    is_esc = code == ESCAPE_CODE
    # rank of each escape among the tile's escapes, clipped like codec.py:384-385
    rank = np.clip(np.cumsum(is_esc, axis=-1, dtype=np.int32) - 1, 0, ESCAPE_BUDGET - 1)
    gathered = np.take_along_axis(esc, rank, axis=-1)
    cb = np.asarray(enc["codebook"], dtype=np.uint8)
    exponent = np.where(is_esc, gathered, cb[np.where(is_esc, 0, code)])  # codec.py:388-390
    sm = enc["sm"].reshape(ntr, ntc, TILE_SIZE)
    tiles = join_bits(exponent, sm)
    fallback = unpack_bitmap(enc["fallback_bitmap"], ntr * ntc).reshape(ntr, ntc)
    nfb = int(fallback.sum())
    if nfb:  # codec.py:368-376
        tiles = tiles.copy()
        tiles[fallback] = np.asarray(enc["fallback_raw"], dtype=np.int16).reshape(nfb, TILE_SIZE)
    return tiles


def decode(enc: dict) -> np.ndarray:
    """Decoded BF16 bits as int16 [rows, cols] (codec.py:144-186)."""
    rows, cols = enc["shape"]
    return np.ascontiguousarray(from_tiles(decode_tiles(enc))[:rows, :cols])


def fallback_tile_count(enc: dict) -> int:
    """Set bits of the bitmap (codec.py:189-202)."""
    return int(np.unpackbits(enc["fallback_bitmap"]).sum())


def fallback_ranks(bitmap: np.ndarray, tile_count: int) -> np.ndarray:
    """Each tile's rank among fallback tiles, cumsum(bits) - 1 (adapters/cuda/gemv.py:47-53)."""
    return (np.cumsum(unpack_bitmap(bitmap, tile_count).astype(np.int32)) - 1).astype(np.int32)


def packed_byte_size(enc: dict) -> int:
    """All five streams plus the 15 codebook bytes (domain/se12/summary.py:71-92)."""
    return int(
        enc["sm"].nbytes + enc["ec"].nbytes + enc["esc"].nbytes
        + enc["fallback_bitmap"].nbytes + np.asarray(enc["fallback_raw"]).nbytes + CODEBOOK_SIZE
    )


# ---------------------------------------------------------------------------
# data generation and the GEMV reference
# ---------------------------------------------------------------------------


def f32_to_bf16_bits(a: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even float32 -> BF16 bits as int16 (what torch's
    `.to(torch.bfloat16)` does in lws/bench/micro.py:143-145); NaN stays NaN."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)
    rounded = ((u + np.uint32(0x7FFF) + ((u >> 16) & np.uint32(1))) >> 16).astype(np.uint32)
    nan = (u & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)
    rounded = np.where(nan, (u >> 16) | np.uint32(0x40), rounded)
    return rounded.astype(np.uint16).view(np.int16)


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    """Exact BF16 -> float32 (`bits << 16`)."""
    return (np.asarray(bits).astype(np.uint16).astype(np.uint32) << 16).view(np.float32)


def normal_bf16(rows: int, cols: int, seed: int, std: float) -> np.ndarray:
    """default_rng(seed).standard_normal((rows, cols), float32) * std -> BF16 bits."""
    a = np.random.default_rng(seed).standard_normal((rows, cols), dtype=np.float32)
    if std != 1.0:
        a *= np.float32(std)
    return f32_to_bf16_bits(a)


def gemv_reference(enc: dict, x: np.ndarray, *, fp64: bool = False) -> np.ndarray:
    """y[b, n] = sum_k W[n, k] x[b, k] with W decoded by the oracle: float32
    matmul (numpy decode + matmul), or float64 for the brute-force check
    (lws/bench/micro.py:148-151 computes its reference in FP64)."""
    w = bf16_bits_to_f32(decode(enc))
    xf = np.asarray(x)
    if fp64:
        return xf.astype(np.float64) @ w.astype(np.float64).T
    return xf.astype(np.float32) @ w.T
