"""Pins the CPU oracle (oracle/se12_codec.py) before anything is checked
against it: golden vectors written by the reference encoder, exhaustive
closed forms, the reference tests' own edge cases
(tests/test_spec_se12_roundtrip.py:36-119, tests/test_spec_fused_gemv.py:46-128
in the reference), and brute force on small inputs."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import GOLDEN_NAMES, golden_as_encoding, load_golden
from oracle import se12_codec as o

STREAMS = ("sm", "ec", "esc", "fallback_bitmap", "fallback_raw", "codebook")


@pytest.mark.parametrize("name", GOLDEN_NAMES)
def test_encode_matches_reference_bytes(name):
    g = load_golden(name)
    enc = o.encode(g["bits"], g["rows"], g["cols"])
    for k in STREAMS:
        assert enc[k].dtype == g[k].dtype, k
        assert np.array_equal(enc[k], g[k]), f"{name}: stream {k} differs from the reference encoder"


@pytest.mark.parametrize("name", GOLDEN_NAMES)
def test_decode_of_reference_streams_is_the_input(name):
    g = load_golden(name)
    dec = o.decode(golden_as_encoding(g))
    assert np.array_equal(dec.reshape(-1), g["decoded"])
    assert np.array_equal(dec.reshape(-1), g["bits"].astype(np.int16))


def test_golden_set_covers_fallback_ties_padding_and_escapes():
    fb = {n: o.fallback_tile_count(golden_as_encoding(load_golden(n))) for n in GOLDEN_NAMES}
    assert fb["fallback_16x256"] == 1
    assert fb["mixed_48x768"] == 2
    assert fb["normal_32x512"] == 0
    ties = load_golden("ties_16x256")
    # 5 used exponents (3 of them tied at 820), then unused values from 255 down
    assert list(ties["codebook"]) == [131, 130, 90, 7, 200, 255, 254, 253, 252, 251, 250, 249, 248, 247, 246]
    mixed = golden_as_encoding(load_golden("mixed_48x768"))
    assert list(np.unpackbits(mixed["fallback_bitmap"], count=9)) == [0, 1, 0, 0, 0, 1, 0, 0, 0]


def test_split_and_join_are_exact_inverses_over_all_patterns():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.int16)
    e, sm = o.split_bits(bits)
    u = bits.view(np.uint16).astype(np.uint32)
    assert np.array_equal(e, ((u >> 7) & 0xFF).astype(np.uint8))
    assert np.array_equal(sm >> 7, (u >> 15).astype(np.uint8))
    assert np.array_equal(sm & 0x7F, (u & 0x7F).astype(np.uint8))
    assert np.array_equal(o.join_bits(e, sm), bits)


def _bits(sign, exponent, mantissa):
    return (sign << 15) | (exponent << 7) | mantissa


def test_round_trip_on_float_edge_cases():
    edge = [_bits(0, 0, 0), _bits(1, 0, 0), _bits(0, 0, 1), _bits(1, 0, 1), _bits(0, 0, 0x7F), _bits(0, 0xFF, 0),
            _bits(1, 0xFF, 0), _bits(0, 0xFF, 0x40), _bits(0, 0xFF, 0x7F), _bits(1, 0xFF, 0x01), _bits(0, 1, 0),
            _bits(1, 1, 0), _bits(0, 0xFE, 0x7F), _bits(1, 0xFE, 0x7F)]
    rng = np.random.default_rng(7)
    edge += [_bits(int(rng.integers(0, 2)), int(rng.integers(1, 0xFE)), int(rng.integers(0, 0x80))) for _ in range(200)]
    bits = np.array(edge, dtype=np.uint16).view(np.int16)
    assert np.array_equal(o.decode(o.encode(bits, 1, bits.size)).reshape(-1), bits)


@pytest.mark.parametrize("rows,cols", [(16, 256), (32, 256), (16, 512), (32, 512), (33, 300), (1, 1), (36, 1), (160, 2560)])
def test_round_trip_with_and_without_padding(rows, cols):
    rng = np.random.default_rng(rows * 1000 + cols)
    bits = rng.integers(0, 65536, size=rows * cols, dtype=np.uint32).astype(np.uint16).view(np.int16)
    assert np.array_equal(o.decode(o.encode(bits, rows, cols)).reshape(-1), bits)


def _compose(exponents, rng):
    n = exponents.size
    sign = rng.integers(0, 2, size=n).astype(np.uint16)
    mant = rng.integers(0, 0x80, size=n).astype(np.uint16)
    return ((sign << 15) | (exponents.astype(np.uint16) << 7) | mant).view(np.int16)


def test_forced_fallback_tile_is_raw_and_exact():
    rng = np.random.default_rng(3)
    e = np.zeros(4096, dtype=np.uint8)
    e[:4076] = np.tile(np.arange(15, dtype=np.uint8), 4076 // 15 + 1)[:4076]
    e[4076:] = np.arange(100, 120, dtype=np.uint8)
    bits = _compose(e, rng)
    enc = o.encode(bits, 16, 256)
    assert o.fallback_tile_count(enc) == 1
    assert np.array_equal(enc["fallback_raw"], bits)
    assert not enc["esc"].any()
    assert np.array_equal(o.decode(enc).reshape(-1), bits)


def test_concentrated_exponents_never_fall_back():
    rng = np.random.default_rng(5)
    e = rng.choice(np.arange(120, 135, dtype=np.uint8), size=160 * 2560)
    enc = o.encode(_compose(e, rng), 160, 2560)
    assert o.fallback_tile_count(enc) == 0
    assert not (o.unpack_codes(enc["ec"]) == 15).any()


def test_escape_budget_boundary_16_stays_17_falls_back():
    rng = np.random.default_rng(9)
    for count, fallback in ((16, 0), (17, 1)):
        e = np.full(4096, 120, dtype=np.uint8)
        e[:14 * 200] = np.repeat(np.arange(121, 135, dtype=np.uint8), 200)
        pos = rng.choice(4096, size=count, replace=False)
        e[pos] = np.arange(40, 40 + count, dtype=np.uint8)
        bits = _compose(e, rng)
        enc = o.encode(bits, 16, 256)
        assert o.fallback_tile_count(enc) == fallback
        if not fallback:
            # slots hold the escaped exponents in tile-local row-major order
            assert list(enc["esc"][0]) == [int(x) for x in e[np.sort(pos)]]
        assert np.array_equal(o.decode(enc).reshape(-1), bits)


def test_codebook_rule_against_brute_force_sort():
    rng = np.random.default_rng(11)
    for trial in range(50):
        distinct = int(rng.integers(1, 40))
        values = rng.choice(256, size=distinct, replace=False)
        counts = rng.integers(1, 4, size=distinct)  # small counts -> many ties
        e = np.repeat(values, counts).astype(np.uint8)
        cb = o.build_codebook(e.reshape(1, -1), np.ones((1, e.size), dtype=bool))
        hist = {v: 0 for v in range(256)}
        for v in e:
            hist[int(v)] += 1
        expect = sorted(range(256), key=lambda v: (-hist[v], -v))[:15]
        assert list(cb) == expect, trial


def test_codebook_ignores_padding():
    bits = np.full(3, _bits(0, 200, 0), dtype=np.uint16).view(np.int16)
    enc = o.encode(bits, 1, 3)  # 4093 padding zeros (exponent 0) must not count
    assert enc["codebook"][0] == 200
    assert enc["codebook"][1] == 255


def test_fallback_ranks_are_the_prefix_sum():
    rng = np.random.default_rng(0)
    mask = rng.integers(0, 2, size=37).astype(bool)
    ranks = o.fallback_ranks(np.packbits(mask), 37)
    running = 0
    for t in range(37):
        if mask[t]:
            assert ranks[t] == running
            running += 1


def test_tile_grid_and_byte_size():
    assert o.tile_grid(64, 512) == (4, 2)
    assert o.tile_grid(33, 300) == (3, 2)
    enc = o.encode(o.normal_bf16(32, 512, seed=0, std=0.02).reshape(-1), 32, 512)
    assert o.packed_byte_size(enc) == 4 * 6160 + 1 + 15
    g = golden_as_encoding(load_golden("mixed_48x768"))
    assert o.packed_byte_size(g) == 9 * 6160 + 2 + 2 * 4096 * 2 + 15


def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(1)
    a = np.concatenate([rng.standard_normal(100000).astype(np.float32) * 0.02,
                        np.array([0.0, -0.0, np.inf, -np.inf, 1e-40, 3.0e38], dtype=np.float32)])
    ours = o.f32_to_bf16_bits(a)
    ref = torch.from_numpy(a).to(torch.bfloat16).view(torch.int16).numpy()
    assert np.array_equal(ours, ref)


def test_gemv_reference_fp32_is_close_to_fp64_brute_force():
    enc = o.encode(o.normal_bf16(48, 700, seed=4, std=0.02).reshape(-1), 48, 700)
    x = o.bf16_bits_to_f32(o.normal_bf16(3, 700, seed=5, std=1.0))
    y32 = o.gemv_reference(enc, x)
    w = o.bf16_bits_to_f32(o.decode(enc)).astype(np.float64)
    brute = np.array([[sum(w[n, k] * float(x[b, k]) for k in range(700)) for n in range(48)] for b in range(3)])
    assert np.allclose(y32, brute, rtol=1e-5, atol=1e-5)


def test_a_planted_nibble_swap_is_caught_by_the_goldens():
    """The golden check is not vacuous: an oracle that packed ec nibbles the
    other way round would fail it."""
    g = load_golden("normal_32x512")
    enc = o.encode(g["bits"], 32, 512)
    swapped = ((enc["ec"] >> 4) | (enc["ec"] << 4)).astype(np.uint8)
    assert not np.array_equal(swapped, g["ec"])
