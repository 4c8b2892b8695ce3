"""The GPU encoder writes byte-identical streams to the reference encoder
(golden vectors) and to the oracle on larger seeded inputs."""

from __future__ import annotations

import numpy as np
import pytest

from conftest import GOLDEN_NAMES, load_golden
from gpu_helpers import bf16_tensor, heavy_tailed_bf16, uniform_bits
from oracle import se12_codec as o

pytestmark = pytest.mark.gpu


def _encode(bits: np.ndarray, device):
    from se12_amd.hip import encode_on_device

    dt = encode_on_device(bf16_tensor(bits, device))
    h = dt.to_host()
    s = h.streams
    t = dt.tile_grid[0] * dt.tile_grid[1]
    return {
        "sm": s.primary.sm.value, "ec": s.primary.ec.value, "esc": s.escape_handling.esc.value.reshape(t, 16),
        "fallback_bitmap": s.escape_handling.fallback.bitmap.value, "fallback_raw": s.escape_handling.fallback.raw.value,
        "codebook": np.array(h.metadata.codebook.exponents, dtype=np.uint8),
    }


def _assert_same(got, expect):
    for k in ("sm", "ec", "esc", "fallback_bitmap", "fallback_raw", "codebook"):
        assert np.array_equal(np.asarray(got[k]).reshape(-1), np.asarray(expect[k]).reshape(-1)), k


@pytest.mark.parametrize("name", GOLDEN_NAMES)
def test_encoder_matches_reference_bytes(gpu, name):
    g = load_golden(name)
    _assert_same(_encode(g["bits"].reshape(g["rows"], g["cols"]), gpu), g)


@pytest.mark.parametrize("rows,cols,kind", [(2304, 9216, "normal"), (300, 1000, "uniform"), (129, 4700, "heavy")])
def test_encoder_matches_oracle(gpu, rows, cols, kind):
    if kind == "normal":
        bits = o.normal_bf16(rows, cols, seed=0, std=0.02)
    elif kind == "uniform":
        bits = uniform_bits(rows, cols, seed=1)
    else:
        bits = heavy_tailed_bf16(rows, cols, seed=2)
    _assert_same(_encode(bits, gpu), o.encode(bits.reshape(-1), rows, cols))
