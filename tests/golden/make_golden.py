"""Writes the SE12 golden vectors in this directory from the reference encoder.

Run once, in a container where the reference repository is mounted read-only
at /root/reference (it is never present on a GPU machine):

    python tests/golden/make_golden.py

Each `<name>.npz` holds the input BF16 bits and shape, every stream the
reference `encode_tensor` wrote (lws/domain/se12/codec.py:111-141), its
codebook, and the reference `decode_tensor` output. The fixtures pin what only
running the reference can pin: the codebook tie-break and unused-slot order
(lws/domain/se12/codebook.py:55-58), the nibble order in `ec`, the escape slot
order in `esc`, the bitmap bit order and the fallback_raw tile order.
Nothing here is copied from the reference: it is called, and only its outputs
are kept.
"""

from __future__ import annotations

import pathlib
import sys

import numpy as np

REFERENCE_SRC = pathlib.Path("/root/reference/src")
HERE = pathlib.Path(__file__).resolve().parent


def _bits(sign: int, exponent: int, mantissa: int) -> int:
    return (sign << 15) | (exponent << 7) | mantissa


def _as_int16(values) -> np.ndarray:
    return np.asarray(values, dtype=np.uint16).view(np.int16)


def _compose(exponents: np.ndarray, rng: np.random.Generator) -> np.ndarray:
    n = exponents.size
    sign = rng.integers(0, 2, size=n).astype(np.uint16)
    mant = rng.integers(0, 0x80, size=n).astype(np.uint16)
    return ((sign << 15) | (exponents.astype(np.uint16) << 7) | mant).view(np.int16)


def cases() -> dict[str, tuple[np.ndarray, int, int]]:
    out: dict[str, tuple[np.ndarray, int, int]] = {}

    # float edge cases: zeros, subnormals, infinities, NaN payloads, extremes
    edge = [
        _bits(0, 0, 0), _bits(1, 0, 0), _bits(0, 0, 1), _bits(1, 0, 1), _bits(0, 0, 0x7F),
        _bits(0, 0xFF, 0), _bits(1, 0xFF, 0), _bits(0, 0xFF, 0x40), _bits(0, 0xFF, 0x7F),
        _bits(1, 0xFF, 0x01), _bits(0, 1, 0), _bits(1, 1, 0), _bits(0, 0xFE, 0x7F), _bits(1, 0xFE, 0x7F),
    ]
    rng = np.random.default_rng(101)
    edge += [_bits(int(rng.integers(0, 2)), int(rng.integers(1, 0xFE)), int(rng.integers(0, 0x80))) for _ in range(200)]
    out["edge_1x214"] = (_as_int16(edge), 1, len(edge))

    # uniform random bits, padded in both dimensions (most tiles fall back)
    rng = np.random.default_rng(102)
    out["uniform_33x300"] = (rng.integers(0, 65536, size=33 * 300, dtype=np.uint32).astype(np.uint16).view(np.int16), 33, 300)

    # one tile with 20 single-occurrence exponents: exactly one fallback tile
    rng = np.random.default_rng(103)
    e = np.zeros(4096, dtype=np.uint8)
    e[:4076] = np.tile(np.arange(15, dtype=np.uint8), 4076 // 15 + 1)[:4076]
    e[4076:] = np.arange(100, 120, dtype=np.uint8)
    out["fallback_16x256"] = (_compose(e, rng), 16, 256)

    # fewer than 15 distinct exponents with tied counts: pins tie-break and unused slots
    rng = np.random.default_rng(104)
    e = np.repeat(np.array([130, 90, 131, 7, 200], dtype=np.uint8), 4096 // 5 + 1)[:4096]
    e[-1] = 131
    rng.shuffle(e)
    out["ties_16x256"] = (_compose(e, rng), 16, 256)

    # BF16 N(0, 0.02) from seed 0, the synthetic weight distribution of the benchmarks
    a = np.random.default_rng(0).standard_normal((32, 512), dtype=np.float32) * np.float32(0.02)
    u = a.view(np.uint32)
    bf = ((u + np.uint32(0x7FFF) + ((u >> 16) & np.uint32(1))) >> 16).astype(np.uint16).view(np.int16)
    out["normal_32x512"] = (bf.reshape(-1), 32, 512)

    # 3x3 tiles: tiles 1 and 5 overflow the escape budget, the others carry 0..12 escapes
    rng = np.random.default_rng(105)
    ex = rng.choice(np.arange(115, 130, dtype=np.uint8), size=(48, 768))
    for t, count in enumerate([3, 30, 0, 12, 1, 17, 16, 5, 9]):
        tr, tc = divmod(t, 3)
        pos = rng.choice(4096, size=count, replace=False)
        rr, cc = divmod(pos, 256)
        ex[tr * 16 + rr, tc * 256 + cc] = rng.integers(60, 100, size=count).astype(np.uint8)
    out["mixed_48x768"] = (_compose(ex.reshape(-1), rng), 48, 768)

    # ragged 20x300 with escapes next to the padded region
    rng = np.random.default_rng(106)
    ex = rng.choice(np.arange(118, 133, dtype=np.uint8), size=(20, 300))
    ex[19, 290:300] = np.arange(40, 50, dtype=np.uint8)
    ex[3, 257] = 250
    ex[17, 0] = 0
    ex[0, 299] = 255
    out["ragged_20x300"] = (_compose(ex.reshape(-1), rng), 20, 300)
    return out


def main() -> int:
    sys.path.insert(0, str(REFERENCE_SRC))
    from lws.domain.se12.codec import decode_tensor, encode_tensor
    from lws.domain.se12.tile import MatrixShape
    from lws.domain.weights import Bf16Weights

    for name, (bits, rows, cols) in cases().items():
        enc = encode_tensor(Bf16Weights(bit_pattern=np.ascontiguousarray(bits, dtype=np.int16)), MatrixShape(rows=rows, cols=cols))
        dec = decode_tensor(enc)
        s = enc.streams
        np.savez_compressed(
            HERE / f"{name}.npz",
            bits=bits,
            shape=np.array([rows, cols], dtype=np.int64),
            sm=s.primary.sm.value,
            ec=s.primary.ec.value,
            esc=s.escape_handling.esc.value,
            fallback_bitmap=s.escape_handling.fallback.bitmap.value,
            fallback_raw=s.escape_handling.fallback.raw.value,
            codebook=np.array(enc.metadata.codebook.exponents, dtype=np.uint8),
            decoded=dec.bit_pattern,
        )
        print(name, rows, cols, "codebook", list(enc.metadata.codebook.exponents))
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
