"""HIP decode-only kernel vs the oracle: bit-exact (int16 compare), as the
reference's GPU decode test asks (tests/test_spec_gpu_decode.py:75-113 in the
reference), on the golden vectors, edge cases, ragged shapes, forced fallback
tiles, escape-heavy data and the 2304x9216 benchmark shape."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import GOLDEN_NAMES, golden_as_encoding, load_golden
from gpu_helpers import escape_count_bf16, heavy_tailed_bf16, normal_case, to_device, uniform_bits
from oracle import se12_codec as o

pytestmark = pytest.mark.gpu


def _decode(enc, device) -> np.ndarray:
    from se12_amd.hip import HipSe12WeightDecoder

    dt = to_device(enc, device)
    out = HipSe12WeightDecoder().decode_to_device(dt)
    torch.cuda.synchronize()
    return out.view(torch.int16).cpu().numpy()


@pytest.mark.parametrize("name", GOLDEN_NAMES)
def test_decode_golden_vectors_bit_exact(gpu, name):
    g = load_golden(name)
    got = _decode(golden_as_encoding(g), gpu)
    assert got.shape == (g["rows"], g["cols"])
    assert np.array_equal(got.reshape(-1), g["decoded"])


def test_decode_uniform_random_bits(gpu):
    bits = uniform_bits(64, 512, seed=7)
    enc = o.encode(bits.reshape(-1), 64, 512)
    assert o.fallback_tile_count(enc) > 0
    assert np.array_equal(_decode(enc, gpu), bits)


@pytest.mark.parametrize("rows,cols", [(1, 1), (36, 1), (33, 300), (17, 257), (16, 4096), (160, 2560), (5, 1030)])
def test_decode_ragged_shapes(gpu, rows, cols):
    bits = heavy_tailed_bf16(rows, cols, seed=rows + cols)
    enc = o.encode(bits.reshape(-1), rows, cols)
    assert np.array_equal(_decode(enc, gpu), bits)


def test_decode_benchmark_shape_bit_exact(gpu):
    bits, enc = normal_case(2304, 9216, seed=0)
    got = _decode(enc, gpu)
    assert np.array_equal(got, bits)


def test_decode_escape_heavy(gpu):
    bits = heavy_tailed_bf16(512, 4608, seed=3)
    enc = o.encode(bits.reshape(-1), 512, 4608)
    codes = o.unpack_codes(enc["ec"])
    assert (codes == 15).sum() > 100
    assert np.array_equal(_decode(enc, gpu), bits)


def test_decode_rows_in_request_order(gpu):
    from se12_amd.hip import HipSe12WeightDecoder, RowIndices

    bits = uniform_bits(48, 512, seed=4)
    enc = o.encode(bits.reshape(-1), 48, 512)
    dt = to_device(enc, gpu)
    dec = HipSe12WeightDecoder()
    got = dec.decode_rows(dt, RowIndices(values=(5, 0, 47, 12, 5)))
    assert np.array_equal(got.bit_pattern, bits[[5, 0, 47, 12, 5], :].reshape(-1))
    with pytest.raises(IndexError):
        dec.decode_rows(dt, RowIndices(values=(48,)))
    # device indices out of range give rows of zeros
    out = dec.decode_rows_to_device(dt, torch.tensor([3, -1, 99], device=gpu))
    torch.cuda.synchronize()
    o_np = out.view(torch.int16).cpu().numpy()
    assert np.array_equal(o_np[0], bits[3])
    assert not o_np[1:].any()


def test_decode_rows_ragged_and_fallback(gpu):
    from se12_amd.hip import HipSe12WeightDecoder, RowIndices

    g = load_golden("mixed_48x768")
    enc = golden_as_encoding(g)
    bits = g["bits"].reshape(48, 768)
    rows = tuple(range(47, -1, -5))
    got = HipSe12WeightDecoder().decode_rows(to_device(enc, gpu), RowIndices(values=rows))
    assert np.array_equal(got.bit_pattern, bits[list(rows)].reshape(-1))


def test_decode_every_escape_count(gpu):
    """Tiles with 0..16 escapes (listed in the bind-time sidecar up to 8, more
    decoded to raw tiles at bind) and a fallback tile: bit-exact, whole matrix
    and row subsets."""
    from se12_amd.hip import HipSe12WeightDecoder, RowIndices

    bits, counts = escape_count_bf16(seed=11)
    enc = o.encode(bits.reshape(-1), 64, 1024)
    codes = o.unpack_codes(enc["ec"]).reshape(16, 4096)
    assert (codes == 15).sum(axis=1).tolist() == counts
    assert o.fallback_tile_count(enc) == sum(1 for n in counts if n > 16)
    assert np.array_equal(_decode(enc, gpu), bits)
    dt = to_device(enc, gpu)
    rows = [63, 0, 17, 31, 40, 15, 48]
    got = HipSe12WeightDecoder().decode_rows(dt, RowIndices(tuple(rows)))
    assert np.array_equal(got.bit_pattern, bits[rows].reshape(-1))



def test_bind_stats_count_the_raw_decoded_tiles(gpu):
    """se12_handle_bind_stats: the tiles holding 9..16 escapes (more than a
    side record lists, fewer than a fallback tile) are the ones bind decodes
    to raw BF16; the sidecar bytes are 64 per tile, the 1 KiB pair table and
    8 KiB per such tile. A raw-twin handle derives nothing."""
    from se12_amd.hip import RawBf16MatVecKernel, Se12MatVecKernel

    bits, counts = escape_count_bf16(seed=11)
    enc = o.encode(bits.reshape(-1), 64, 1024)
    st = Se12MatVecKernel(to_device(enc, gpu), max_batch=1).bind_stats()
    raw = sum(1 for n in counts if 8 < n <= 16)
    assert raw == 5
    assert st == {"raw_tiles": raw, "sidecar_bytes": 16 * 64 + 1024 + raw * 8192}
    import ctypes

    from se12_amd import _native as nat

    w = torch.from_numpy(bits.astype(np.int16)).to(gpu).view(torch.bfloat16)
    rk = RawBf16MatVecKernel(w, max_batch=1)
    a, b = ctypes.c_int64(-1), ctypes.c_int64(-1)
    nat.check(nat.lib().se12_handle_bind_stats(rk.handle.raw, ctypes.byref(a), ctypes.byref(b)))
    assert (a.value, b.value) == (0, 0)
