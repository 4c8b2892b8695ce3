"""A numpy model of the per-lane decode the HIP kernels run (se12_device.hpp),
checked against the oracle on the CPU: lane l of the wave owning a tile reads
sm bytes [1024*j + 16*l, +16) and ec bytes [512*j + 8*l, +8) for chunks
j = 0..3, looks up each ec byte in the 256-entry pair table (built at bind
time from the codebook; code 15 contributes exponent 0), duplicates sm bytes with the v_perm selectors 0x01010000 /
0x03030202, merges with the exponent mask 0x7F807F80, and ranks escapes by
(chunk, lane, position) - only in the chunks the per-tile sidecar word marks.
The reference checked its own warp-32 rank scheme the same way before writing
CUDA (tests/test_spec_fused_gemv.py:209-271)."""

from __future__ import annotations

import numpy as np
import pytest

from conftest import golden_as_encoding, load_golden
from oracle import se12_codec as o


def perm(hi: int, lo: int, sel: int) -> int:
    data = (hi << 32) | lo
    out = 0
    for i in range(4):
        s = (sel >> (8 * i)) & 0xFF
        assert s < 8
        out |= ((data >> (8 * s)) & 0xFF) << (8 * i)
    return out


def packed_codebook(codebook) -> list[int]:
    """The 15 codebook bytes as 4 little-endian words, byte 15 = 0."""
    b = list(int(c) for c in codebook) + [0]
    return [b[4 * k] | b[4 * k + 1] << 8 | b[4 * k + 2] << 16 | b[4 * k + 3] << 24 for k in range(4)]


def pair_lut(codebook) -> list[int]:
    """The pair table, built the way the kernels' table is laid out: entry
    4l + i holds high code l >> 2 and low code 4(l & 3) + i, read from the
    codebook packed into 4 little-endian words whose byte 15 is 0."""
    words = packed_codebook(codebook)

    def byte(c):
        return (words[c >> 2] >> (8 * (c & 3))) & 0xFF

    lut = [0] * 256
    for lane in range(64):
        hi = byte(lane >> 2) << 23
        lo = words[lane & 3]
        for i in range(4):
            lut[4 * lane + i] = (((lo >> (8 * i)) & 0xFF) << 7) | hi
    return lut


def tile_info_words(enc: dict) -> np.ndarray:
    """The bind-time sidecar: fallback tiles -> 0x80000000 | rank among
    fallback tiles; others -> bit j set iff chunk j (tile rows 4j..4j+3)
    holds an escape code."""
    rows, cols = enc["shape"]
    ntr, ntc = o.tile_grid(rows, cols)
    t = ntr * ntc
    fb = o.unpack_bitmap(enc["fallback_bitmap"], t)
    ranks = np.cumsum(fb) - 1
    codes = o.unpack_codes(enc["ec"]).reshape(t, 4, 1024)
    chunk_bits = ((codes == 15).any(axis=2) * (1 << np.arange(4))).sum(axis=1)
    return np.where(fb, 0x80000000 | ranks, chunk_bits).astype(np.uint64)


def lane_model_decode_tile(sm_tile: bytes, ec_tile: bytes, esc_tile, lut, info: int) -> np.ndarray:
    out = np.zeros(4096, dtype=np.uint16)
    run = 0
    for j in range(4):
        pats, escmasks = [], []
        for lane in range(64):
            ecb = ec_tile[512 * j + 8 * lane: 512 * j + 8 * lane + 8]
            pats.append([lut[b] for b in ecb])
            m = 0
            for p in range(16):
                if ((ecb[p >> 1] >> (4 * (p & 1))) & 15) == 15:
                    m |= 1 << p
            escmasks.append(m)
        if info >> j & 1:  # wave-uniform: only chunks the sidecar marks
            counts = [bin(m).count("1") for m in escmasks]
            incl = np.cumsum(counts)
            if max(counts) <= 1:  # the kernel's mask-count path gives the same ranks
                assert [sum(1 for c in counts[:lane] if c) for lane in range(64)] == [int(incl[i]) - counts[i] for i in range(64)]
            for lane in range(64):
                r = run + int(incl[lane]) - counts[lane]
                for p in range(16):
                    if escmasks[lane] >> p & 1:
                        e = int(esc_tile[min(r, 15)])
                        q, hi = p >> 1, p & 1
                        m = 0x7F800000 if hi else 0x00007F80
                        pats[lane][q] = (pats[lane][q] & ~m & 0xFFFFFFFF) | (e << (23 if hi else 7))
                        r += 1
            run += int(incl[-1])
        for lane in range(64):
            o_ = 1024 * j + 16 * lane
            words = [int.from_bytes(sm_tile[o_ + 4 * d: o_ + 4 * d + 4], "little") for d in range(4)]
            for q in range(8):
                w = words[q >> 1]
                dup = perm(w, w, 0x03030202 if q & 1 else 0x01010000)
                pair = (pats[lane][q] & 0x7F807F80) | (dup & ~0x7F807F80 & 0xFFFFFFFF)
                out[o_ + 2 * q] = pair & 0xFFFF
                out[o_ + 2 * q + 1] = pair >> 16
    return out


@pytest.mark.parametrize("name", ["normal_32x512", "mixed_48x768", "ragged_20x300", "edge_1x214"])
def test_lane_model_reproduces_the_oracle(name):
    g = load_golden(name)
    enc = golden_as_encoding(g)
    tiles = o.decode_tiles(enc)
    ntr, ntc, _ = tiles.shape
    lut = pair_lut(enc["codebook"])
    info = tile_info_words(enc)
    sm, ec = enc["sm"].tobytes(), enc["ec"].tobytes()
    for t in range(ntr * ntc):
        if info[t] >> 31:
            continue
        got = lane_model_decode_tile(sm[4096 * t: 4096 * (t + 1)], ec[2048 * t: 2048 * (t + 1)], enc["esc"][t], lut, int(info[t]))
        assert np.array_equal(got, tiles.reshape(-1, 4096)[t].view(np.uint16)), f"tile {t}"


def test_lane_model_on_escape_dense_tile():
    rng = np.random.default_rng(4)
    e = rng.choice(np.arange(110, 125, dtype=np.uint8), size=4096)
    pos = rng.choice(np.arange(3, 4096), size=13, replace=False)
    e[pos] = rng.integers(1, 100, size=13)
    e[:3] = [5, 6, 7]  # several escapes in one lane's chunk: 16 in all
    sign = rng.integers(0, 2, size=4096).astype(np.uint16)
    mant = rng.integers(0, 0x80, size=4096).astype(np.uint16)
    bits = ((sign << 15) | (e.astype(np.uint16) << 7) | mant).view(np.int16)
    enc = o.encode(bits, 16, 256)
    assert o.fallback_tile_count(enc) == 0
    info = int(tile_info_words(enc)[0])
    assert info == 0b1111 or info & 1  # escapes in chunk 0 at least
    got = lane_model_decode_tile(enc["sm"].tobytes(), enc["ec"].tobytes(), enc["esc"][0], pair_lut(enc["codebook"]), info)
    assert np.array_equal(got.view(np.int16), bits)


def test_pair_table_matches_the_codebook_rule():
    """Entry b = (codebook[b & 15] << 7) | (codebook[b >> 4] << 23), code 15 -> 0."""
    cb = np.array([122, 121, 120, 123, 119, 118, 124, 117, 116, 125, 115, 114, 126, 113, 255], dtype=np.uint8)
    lut = pair_lut(cb)
    for b in range(256):
        c0, c1 = b & 15, b >> 4
        e0 = int(cb[c0]) if c0 < 15 else 0
        e1 = int(cb[c1]) if c1 < 15 else 0
        assert lut[b] == (e0 << 7) | (e1 << 23), b


def test_tile_info_words_on_the_golden_vectors():
    """Fallback tiles carry their rank; other tiles mark exactly the chunks
    whose codes include 15 (checked tile by tile against the decoded codes)."""
    for name in ["mixed_48x768", "uniform_33x300", "fallback_16x256", "normal_32x512"]:
        enc = golden_as_encoding(load_golden(name))
        info = tile_info_words(enc)
        rows, cols = enc["shape"]
        ntr, ntc = o.tile_grid(rows, cols)
        fb = o.unpack_bitmap(enc["fallback_bitmap"], ntr * ntc)
        codes = o.unpack_codes(enc["ec"]).reshape(-1, 4096)
        rank = 0
        for t in range(ntr * ntc):
            if fb[t]:
                assert info[t] == 0x80000000 | rank
                rank += 1
            else:
                for j in range(4):
                    assert bool(info[t] >> j & 1) == bool((codes[t, 1024 * j:1024 * (j + 1)] == 15).any())


def listed_escapes(ec_tile: bytes) -> list[int]:
    """Tile positions (row * 256 + column) of a tile's escape codes in
    row-major order: the order in which they take the tile's esc slots."""
    codes = np.frombuffer(ec_tile, dtype=np.uint8)
    nib = np.stack([codes & 15, codes >> 4], axis=1).reshape(-1)
    return [int(p) for p in np.nonzero(nib == 15)[0]]


def half_layout_decode_tile(sm_tile: bytes, ec_tile: bytes, esc_tile, lut) -> np.ndarray:
    """The decode-only kernel's half layout (se12_decode.hip): part p = 0..7
    covers tile rows 2p, 2p + 1; lane l takes row 2p + l // 32 and columns
    8 (l % 32) .. + 7 (8 sm bytes at 512 p + 8 l, 4 ec bytes at 256 p + 4 l).
    Pattern word 4 p + k of a lane (k = column pair) comes from the pair
    table; escape k of the tile's listed escapes, at (row, col), is ORed into
    pattern word 4 (row // 2) + (col % 8) // 2 of lane 32 (row % 2) +
    col // 8 (patch_listed_escapes, kHalfLayout), then the merge."""
    pats = [[0] * 32 for _ in range(64)]
    for lane in range(64):
        for p in range(8):
            eb = ec_tile[256 * p + 4 * lane: 256 * p + 4 * lane + 4]
            for k in range(4):
                pats[lane][4 * p + k] = lut[eb[k]]
    for k, pos in enumerate(listed_escapes(ec_tile)):
        row, col = pos >> 8, pos & 255
        owner = ((row & 1) << 5) | (col >> 3)
        word = ((row >> 1) << 2) | ((col & 7) >> 1)
        pats[owner][word] |= int(esc_tile[k]) << (23 if col & 1 else 7)
    out = np.zeros(4096, dtype=np.uint16)
    for lane in range(64):
        for p in range(8):
            row, col = 2 * p + (lane >> 5), 8 * (lane & 31)
            o_ = 512 * p + 8 * lane
            words = [int.from_bytes(sm_tile[o_ + 4 * d: o_ + 4 * d + 4], "little") for d in range(2)]
            assert o_ == row * 256 + col   # sm's tile-local row-major order
            for k in range(4):
                w = words[k >> 1]
                dup = perm(w, w, 0x03030202 if k & 1 else 0x01010000)
                pair = (pats[lane][4 * p + k] & 0x7F807F80) | (dup & ~0x7F807F80 & 0xFFFFFFFF)
                out[row * 256 + col + 2 * k] = pair & 0xFFFF
                out[row * 256 + col + 2 * k + 1] = pair >> 16
    return out


@pytest.mark.parametrize("name", ["normal_32x512", "mixed_48x768", "ragged_20x300", "edge_1x214"])
def test_half_layout_reproduces_the_oracle(name):
    """Every tile the decode kernel decodes (not raw: at most 8 escapes, not
    a fallback tile) comes out of the half layout equal to the oracle."""
    g = load_golden(name)
    enc = golden_as_encoding(g)
    tiles = o.decode_tiles(enc)
    ntr, ntc, _ = tiles.shape
    lut = pair_lut(enc["codebook"])
    info = tile_info_words(enc)
    sm, ec = enc["sm"].tobytes(), enc["ec"].tobytes()
    checked = 0
    for t in range(ntr * ntc):
        ect = ec[2048 * t: 2048 * (t + 1)]
        if info[t] >> 31 or len(listed_escapes(ect)) > 8:
            continue
        got = half_layout_decode_tile(sm[4096 * t: 4096 * (t + 1)], ect, enc["esc"][t], lut)
        assert np.array_equal(got, tiles.reshape(-1, 4096)[t].view(np.uint16)), f"tile {t}"
        checked += 1
    assert checked > 0 or name == "edge_1x214"   # its one tile holds more than 8 escapes (read raw)


def test_half_layout_patches_escapes_in_both_rows_of_a_part():
    """Eight escapes spread over both rows of several parts, two in one
    lane's 8 columns, the first and last weight of the tile."""
    rng = np.random.default_rng(9)
    e = rng.choice(np.arange(110, 125, dtype=np.uint8), size=4096)
    pos = np.array([0, 257, 258, 1023, 1024 + 300, 2048 + 511, 3000, 4095])
    e[pos] = rng.integers(1, 100, size=len(pos))
    sign = rng.integers(0, 2, size=4096).astype(np.uint16)
    mant = rng.integers(0, 0x80, size=4096).astype(np.uint16)
    bits = ((sign << 15) | (e.astype(np.uint16) << 7) | mant).view(np.int16)
    enc = o.encode(bits, 16, 256)
    assert listed_escapes(enc["ec"].tobytes()) == sorted(pos.tolist())
    got = half_layout_decode_tile(enc["sm"].tobytes(), enc["ec"].tobytes(), enc["esc"][0], pair_lut(enc["codebook"]))
    assert np.array_equal(got.view(np.int16), bits)
    # swapped esc slots (a wrong rank) are caught
    wrong = enc["esc"][0].copy()
    wrong[[0, 1]] = wrong[[1, 0]]
    if wrong[0] != enc["esc"][0][0]:
        got2 = half_layout_decode_tile(enc["sm"].tobytes(), enc["ec"].tobytes(), wrong, pair_lut(enc["codebook"]))
        assert not np.array_equal(got2.view(np.int16), bits)
