"""A numpy model of the per-lane decode the HIP kernels run (se12_device.hpp),
checked against the oracle on the CPU: lane l of the wave owning a tile reads
sm bytes [1024*j + 16*l, +16) and ec bytes [512*j + 8*l, +8) for chunks
j = 0..3, looks up each ec byte in the 256-entry pair table, duplicates sm
bytes with the v_perm selectors 0x01010000 / 0x03030202, merges with the
exponent mask 0x7F807F80, and ranks escapes by (chunk, lane, position) with a
wave prefix sum. The reference checked its own warp-32 rank scheme the same
way before writing CUDA (tests/test_spec_fused_gemv.py:209-271)."""

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


def pair_lut(codebook) -> list[int]:
    lut = []
    for b in range(256):
        c0, c1 = b & 15, b >> 4
        p0 = (int(codebook[c0]) << 7) if c0 < 15 else 0
        p1 = (int(codebook[c1]) << 7) if c1 < 15 else 0
        lut.append(p0 | (p1 << 16) | (1 if 15 in (c0, c1) else 0))
    return lut


def lane_model_decode_tile(sm_tile: bytes, ec_tile: bytes, esc_tile, lut) -> np.ndarray:
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
        if any(p & 1 for lane_p in pats for p in lane_p):  # wave-uniform slow path
            counts = [bin(m).count("1") for m in escmasks]
            incl = np.cumsum(counts)
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
    fallback = o.unpack_bitmap(enc["fallback_bitmap"], ntr * ntc)
    sm, ec = enc["sm"].tobytes(), enc["ec"].tobytes()
    for t in range(ntr * ntc):
        if fallback[t]:
            continue
        got = lane_model_decode_tile(sm[4096 * t: 4096 * (t + 1)], ec[2048 * t: 2048 * (t + 1)], enc["esc"][t], lut)
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
    got = lane_model_decode_tile(enc["sm"].tobytes(), enc["ec"].tobytes(), enc["esc"][0], pair_lut(enc["codebook"]))
    assert np.array_equal(got.view(np.int16), bits)
