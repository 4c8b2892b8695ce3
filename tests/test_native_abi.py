"""The C ABI without a GPU: the library loads, exports every symbol the header
declares with the signatures the binding uses, and its host-only entry points
(codebook rule, argument validation, error reporting) behave."""

from __future__ import annotations

import ctypes
import pathlib
import re

import numpy as np
import pytest

from conftest import ROOT
from oracle import se12_codec as o
from se12_amd import _native as nat

HEADER = ROOT / "include" / "se12_gfx950.h"


def header_functions() -> set[str]:
    text = "\n".join(h.read_text() for h in sorted(HEADER.parent.glob("*.h")))
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(se12_[a-z0-9_]+)\s*\(", text))


def test_library_is_built_in_tree():
    assert nat.LIB_PATH.exists(), "run python -m se12_amd.csrc.build"
    assert nat.LIB_PATH.parent.parent == ROOT / "se12_amd"


def test_every_declared_symbol_is_exported_and_bound():
    declared = header_functions()
    assert len(declared) >= 14
    lib = nat.lib()
    for name in declared:
        assert hasattr(lib, name), name
    assert declared == set(nat.SIGNATURES), declared ^ set(nat.SIGNATURES)


def test_version_names_the_target():
    assert "gfx950" in nat.version()


def test_codebook_rule_matches_the_oracle():
    from se12_amd.hip import codebook_from_histogram

    rng = np.random.default_rng(3)
    for _ in range(40):
        counts = np.zeros(256, dtype=np.int64)
        idx = rng.choice(256, size=int(rng.integers(1, 60)), replace=False)
        counts[idx] = rng.integers(1, 5, size=idx.size)
        e = np.repeat(np.arange(256), counts).astype(np.uint8)
        expect = o.build_codebook(e.reshape(1, -1), np.ones((1, e.size), dtype=bool))
        assert codebook_from_histogram(counts) == tuple(int(v) for v in expect)


def test_null_arguments_fail_with_a_message_and_no_gpu_call():
    lib = nat.lib()
    rc = lib.se12_bind(None, 16, 256, 1, None, None)
    assert rc == nat.SE12_E_INVALID
    assert "NULL" in nat.last_error()
    rc = lib.se12_gemv(None, None, 0, 1, None, None, None)
    assert rc == nat.SE12_E_INVALID
    assert "handle" in nat.last_error()
    with pytest.raises(nat.Se12Error):
        nat.check(lib.se12_decode(None, None, None))
    assert lib.se12_gemv_gelu_mul(None, None, 0, 1, None, None, None, None) == nat.SE12_E_INVALID
    assert "se12_gemv_gelu_mul" in nat.last_error()
    assert lib.se12_gemv_rmsnorm(None, None, 0, 1, None, None, None, None, None, 1e-6, None, None) == nat.SE12_E_INVALID
    assert "se12_gemv_rmsnorm" in nat.last_error()
    assert lib.se12_gemv_rowss(None, None, 0, 1, None, None, None, None) == nat.SE12_E_INVALID
    assert "se12_gemv_rowss" in nat.last_error()
    assert lib.se12_handle_bind_stats(None, None, None) == nat.SE12_E_INVALID
    assert "se12_handle_bind_stats" in nat.last_error()


def test_bind_rejects_bad_shapes_before_touching_the_device():
    lib = nat.lib()
    s = nat.Streams(sm_dev=16, ec_dev=16, esc_dev=16, codebook_dev=16, fallback_bitmap_dev=16,
                    fallback_raw_dev=None, fallback_raw_elems=0)
    h = ctypes.c_void_p()
    assert lib.se12_bind(ctypes.byref(s), 0, 256, 1, None, ctypes.byref(h)) == nat.SE12_E_INVALID
    assert lib.se12_bind(ctypes.byref(s), 16, 256, 33, None, ctypes.byref(h)) == nat.SE12_E_INVALID
    assert "max_batch" in nat.last_error()
    s.fallback_raw_elems = 100
    assert lib.se12_bind(ctypes.byref(s), 16, 256, 1, None, ctypes.byref(h)) == nat.SE12_E_INVALID
    assert "whole number of tiles" in nat.last_error()
    s.fallback_raw_elems = 0
    s.sm_dev = 17
    assert lib.se12_bind(ctypes.byref(s), 16, 256, 1, None, ctypes.byref(h)) == nat.SE12_E_INVALID
    assert "aligned" in nat.last_error()
    # 2^31 tiles or more (the decode kernel indexes tiles in 32 bits)
    s.sm_dev = 16
    assert lib.se12_bind(ctypes.byref(s), 16 << 17, 256 << 14, 1, None, ctypes.byref(h)) == nat.SE12_E_INVALID
    assert "too large" in nat.last_error()


def test_encoder_rejects_bad_shapes():
    lib = nat.lib()
    cb = (ctypes.c_uint8 * 15)()
    n = ctypes.c_int64()
    assert lib.se12_encode_prepare(None, 16, 256, 256, cb, ctypes.byref(n), None) == nat.SE12_E_INVALID
    assert lib.se12_encode_prepare(ctypes.c_void_p(16), 16, 256, 100, cb, ctypes.byref(n), None) == nat.SE12_E_INVALID


def test_launch_candidates_respect_each_kernels_limits():
    """BF16 batches of 5+ rows take the batched MFMA kernel (at most 8 waves
    per block, a multiple of batch / 8, and 16 K splits); FP32 x and smaller
    batches the dot2 kernel."""
    from se12_amd.launch import (candidate_configurations, configuration, max_waves_per_block, uses_mfma,
                                 waves_and_splits)

    assert not uses_mfma(4) and uses_mfma(5) and not uses_mfma(32, float32_activations=True)
    # MFMA blocks count row blocks of batch / 8 tile rows (rounded up, 4 in
    # place of 3); a block's waves are those rows times K groups
    from se12_amd.launch import mfma_min_waves

    assert [mfma_min_waves(b) for b in (5, 8, 9, 16, 17, 24, 25, 32)] == [1, 1, 2, 2, 4, 4, 4, 4]
    assert configuration(4, 3, 2304, batch=8).blocks.value == 144 * 3
    assert configuration(4, 3, 2304, batch=32).blocks.value == 36 * 3
    assert configuration(8, 1, 2304, batch=17).blocks.value == 36
    assert configuration(4, 3, 2304, batch=4).blocks.value == 144 * 3
    with pytest.raises(ValueError, match="multiple of 4"):
        waves_and_splits(configuration(6, 1, 2304, batch=17), 2304, batch=17)
    with pytest.raises(ValueError, match="multiple of 2"):
        waves_and_splits(configuration(3, 1, 2304, batch=9), 2304, batch=9)
    # (the x-slab kernel serves 4608x36864 at 24 and 32 rows: x's columns
    # would need 12 and 16 resident-x splits)
    assert all(waves_and_splits(c, 4608, batch=24, k=36864)[0] % 4 == 0 for c in candidate_configurations(4608, 36864, batch=24))
    assert min(waves_and_splits(c, 4608, batch=32, k=36864)[0] for c in candidate_configurations(4608, 36864, batch=32)) == 4
    assert max_waves_per_block(1) == 16 and max_waves_per_block(6) == 8
    for rows, k, batch, f32, max_s in ((2304, 9216, 1, False, 36), (4608, 36864, 32, False, 16), (2304, 9216, 6, True, 36)):
        cfgs = candidate_configurations(rows, k, batch=batch, float32_activations=f32)
        pairs = [waves_and_splits(c, rows, batch=batch, k=k, float32_activations=f32) for c in cfgs]
        assert max(s for _, s in pairs) == max_s
        assert max(w for w, _ in pairs) == max_waves_per_block(batch, f32)
    # 5 or more BF16 rows of x that fit a block's LDS (9 x 2304: 41 KiB): the
    # resident-x kernel, (waves 1..12, blocks 1..tile rows); 9 rows at K =
    # 9216 (162 KiB) do not fit, 6 (108 KiB) do, but rows of 32+ K tiles on
    # at most 160 tile rows (5/8 of 256 CUs) take the x-slab kernel
    from se12_amd.launch import rx_lds_bytes, uses_rx

    assert uses_rx(2304, 2304, 9) and not uses_rx(2304, 9216, 9) and not uses_rx(2304, 2304, 9, float32_activations=True)
    assert uses_rx(4608, 9216, 6) and uses_rx(4096, 14336, 5) and uses_rx(4096, 14336, 6) and uses_rx(256000, 2304, 5)
    assert not uses_rx(2304, 9216, 6) and not uses_rx(2560, 8192, 8) and uses_rx(2576, 8192, 8)
    assert uses_rx(2304, 6144, 8) and uses_rx(2304, 9216, 8, compute_units=128)  # 144 rows > 5/8 of 128 CUs
    assert uses_rx(14336, 3584, 8) and uses_rx(14336, 3584, 16) and uses_rx(14336, 3584, 24)
    # 17..32 rows whose first 16 fit, on at most one tile row per CU: 16 rows
    # in LDS, batch group 1 from global memory, at most 8 waves
    from se12_amd.launch import rx_max_waves, rx_splits, rx_staged_rows

    assert rx_staged_rows(4096, 3584, 32) == 16 and rx_staged_rows(4096, 3584, 16) == 16
    assert rx_staged_rows(4096, 3584, 24) == 16 and rx_staged_rows(4096, 2304, 32) == 32
    # past one tile row per CU, two K splits with all the rows of x
    assert rx_staged_rows(4112, 3584, 32) == 32 and rx_splits(4112, 3584, 32) == 2
    assert rx_staged_rows(4096, 14336, 17) == 17
    assert rx_staged_rows(4096, 3584, 32, compute_units=128) == 32 and rx_splits(4096, 3584, 32, compute_units=128) == 2
    assert rx_max_waves(4096, 3584, 32) == 8 and rx_max_waves(4096, 3584, 16) == 12 and rx_max_waves(14336, 3584, 16) == 12
    assert not uses_rx(2304, 2300, 9) and not uses_rx(2300, 2304, 9) and not uses_rx(256000, 2304, 4)
    assert rx_lds_bytes(9216, 6) == 6 * 1152 * 16 and rx_lds_bytes(2304, 5) == 1472 * 16
    pairs = [waves_and_splits(c, 2304, batch=9, k=2304) for c in candidate_configurations(2304, 2304, batch=9)]
    assert max(w for w, _ in pairs) == 12 and max(b for _, b in pairs) == 144 and min(b for _, b in pairs) >= 1


def test_resident_x_k_split_rule():
    """A single matrix whose x fits a block's LDS neither whole nor as its
    first 16 rows splits K into the fewest ranges whose columns of x fit
    (2..8; 2 at up to 16 rows only on launches of 8192+ tiles); the x-slab
    kernel serves the rest. Blocks then count K splits too."""
    from se12_amd.launch import (candidate_configurations, rx_configuration, rx_kgroups, rx_layout, rx_splits,
                                 waves_and_splits)

    assert rx_layout(3584, 14336, 16) == (16, 3)      # 19 K tiles of 56: 152 KiB of x per block
    assert rx_layout(3584, 14336, 24) == (24, 5) and rx_layout(3584, 14336, 32) == (32, 7)
    assert rx_layout(2304, 9216, 24) == (24, 3) and rx_layout(2304, 9216, 32) == (32, 4)
    assert rx_layout(4608, 36864, 9) == (9, 5) and rx_layout(4608, 36864, 16) == (16, 8)
    assert rx_layout(36864, 4608, 24) == (24, 2)      # 2304 tile rows x 18 K tiles
    assert rx_layout(3584, 14336, 9) == (9, 2)        # two splits at one batch group: 12,544 tiles
    assert rx_layout(2304, 9216, 16) == (0, 0)        # 5,184 tiles: the x-slab kernel
    assert rx_layout(14336, 3584, 32) == (32, 2) and rx_layout(14336, 3584, 23) == (23, 2)
    assert rx_layout(14336, 3584, 22) == (22, 1)      # x fits whole
    assert rx_layout(4608, 4096, 24) == (24, 2)       # two batch groups: two splits on any size
    assert rx_layout(4608, 36864, 24) == (0, 0)       # 12 splits: over the limit
    assert rx_layout(4096, 3584, 32) == (16, 1) and rx_layout(2304, 2304, 32) == (32, 1)
    assert rx_splits(2304, 9216, 4) == 0 and rx_splits(2304, 9216, 24, float32_activations=True) == 0
    assert rx_configuration(8, 85, splits=3).blocks.value == 255
    assert rx_kgroups(3584, 14336, 8, 85, splits=3) == 2   # 18 K tiles per split, 224 rows over 85 x 4 slots
    assert rx_kgroups(3584, 14336, 8, 32, splits=3) == 1
    for c in candidate_configurations(3584, 14336, batch=16):
        waves, blocks = waves_and_splits(c, 3584, batch=16, k=14336)
        assert blocks % 3 == 0 and 1 <= blocks // 3 <= 224 and blocks <= 3 * 256
    with pytest.raises(ValueError, match="3 K splits"):
        waves_and_splits(rx_configuration(8, 85), 3584, batch=16, k=14336)


def test_resident_x_kgroups_rule():
    """K groups of the resident-x kernel: powers of two dividing the waves,
    at least two K tiles per group, at most one row per row slot."""
    from se12_amd.launch import rx_kgroups

    assert rx_kgroups(2304, 9216, 8, 144) == 8         # 144 tile rows, 36 K tiles: one row per block
    assert rx_kgroups(2304, 9216, 8, 72) == 4
    assert rx_kgroups(14336, 3584, 8, 256) == 1        # 896 rows: 3+ per block keep the waves busy
    assert rx_kgroups(14336, 3584, 8, 320) == 2        # 2.8 rows per block over 4 slots each; 14 K tiles
    assert rx_kgroups(14336, 3584, 8, 512) == 4
    assert rx_kgroups(9216, 2304, 8, 256) == 2
    assert rx_kgroups(9216, 2304, 8, 576) == 4         # 9 K tiles: groups of 2..3 tiles
    assert rx_kgroups(256000, 2304, 8, 256) == 1       # rows far beyond the slots
    assert rx_kgroups(2304, 9216, 12, 144) == 4        # 12 waves: 4 divides, 8 does not
    assert rx_kgroups(2304, 9216, 3, 144) == 1
    for rows, k, w, p in ((2304, 9216, 12, 144), (14336, 3584, 8, 512), (9216, 2304, 8, 576), (272, 2304, 8, 17)):
        kg = rx_kgroups(rows, k, w, p)
        assert w % kg == 0 and -(-k // 256) >= 2 * kg
        assert kg == 1 or p * (w // kg) >= -(-rows // 16)


def test_step_kernels_reject_invalid_arguments():
    """Argument checks run before any HIP call, so this runs without a GPU
    (host pointers are never dereferenced)."""
    import torch

    x = torch.zeros((2, 8), dtype=torch.bfloat16)
    lib = nat.lib()
    s = ctypes.c_void_p(None)
    with pytest.raises(nat.Se12Error, match="mode 1"):
        nat.step_check(lib.se12_step_rmsnorm(nat.ptr(x), nat.STEP_BF16, 8, nat.ptr(x[0]), None, None, nat.ptr(x),
                                             2, 8, 1e-6, 0.0, 1, s))
    with pytest.raises(nat.Se12Error, match="mode must be"):
        nat.step_check(lib.se12_step_rmsnorm(nat.ptr(x), nat.STEP_BF16, 8, nat.ptr(x[0]), nat.ptr(x), nat.ptr(x[0]),
                                             nat.ptr(x), 2, 8, 1e-6, 0.0, 2, s))
    with pytest.raises(nat.Se12Error, match="bad argument"):
        nat.step_check(lib.se12_step_gelu_mul(nat.ptr(x), nat.ptr(x), 7, 8, nat.ptr(x), 2, 8, s))
    def attention(heads, kvh, d, L, ws, ws_bytes):
        return lib.se12_step_attention(nat.ptr(x), nat.ptr(x), nat.ptr(x), nat.STEP_BF16, heads * d, kvh * d,
                                       nat.ptr(x), nat.ptr(x), nat.ptr(x), nat.ptr(x), nat.ptr(x), 1, heads, kvh, d,
                                       L, 1.0, 0.0, 0, ws, ws_bytes, s)

    need = lib.se12_step_attention_workspace(1, 8, 4, 256, 640)
    # counters, scores, chunk statistics and partial sums, each section 256-byte aligned
    assert need == 256 + 8 * 10 * 64 * 4 + 768 + 8 * 10 * 256 * 4        # 640 B of statistics padded to 768
    assert lib.se12_step_attention_workspace(1, 6, 4, 256, 640) < 0      # 6 query heads over 4 KV heads
    assert lib.se12_step_attention_workspace(1, 24, 2, 64, 640) < 0      # groups of 12
    assert lib.se12_step_attention_workspace(1, 8, 4, 512, 640) < 0      # head_dim above 256
    assert lib.se12_step_attention_workspace(1, 8, 4, 100, 640) < 0      # head_dim not a multiple of 8
    assert lib.se12_step_attention_workspace(1, 8, 4, 256, 644) < 0      # cache length not a multiple of 8
    aligned = ctypes.c_void_p(1 << 20)                                     # never dereferenced
    with pytest.raises(nat.Se12Error, match="bad shape"):
        nat.step_check(attention(3, 2, 4, 4, aligned, 1 << 20))
    with pytest.raises(nat.Se12Error, match="workspace too small"):
        nat.step_check(attention(8, 4, 256, 640, aligned, need - 1))
    with pytest.raises(nat.Se12Error, match="aligned"):
        nat.step_check(attention(8, 4, 256, 640, ctypes.c_void_p((1 << 20) + 4), need))
    with pytest.raises(nat.Se12Error, match="NULL"):
        nat.step_check(attention(8, 4, 256, 640, None, need))
    ws = lib.se12_step_logits_workspace(2, 256000)
    assert ws == 256 + 1024 + 1024          # counters; 2 rows x 125 slices of 2,048 logits: values, indices
    assert lib.se12_step_logits_workspace(0, 10) < 0

    def argmax(rows, vocab, stride, wsp, ws_bytes):
        return lib.se12_step_logits_argmax(nat.ptr(x), nat.STEP_BF16, stride, rows, vocab, 0.0, None, nat.ptr(x),
                                           nat.ptr(x), 4, nat.ptr(x), wsp, ws_bytes, s)

    with pytest.raises(nat.Se12Error, match="bad argument"):
        nat.step_check(argmax(2, 8, 4, aligned, 1 << 20))                  # stride below vocab
    with pytest.raises(nat.Se12Error, match="workspace too small"):
        nat.step_check(argmax(2, 256000, 256000, aligned, ws - 1))
    with pytest.raises(nat.Se12Error, match="aligned"):
        nat.step_check(argmax(2, 256000, 256000, ctypes.c_void_p((1 << 20) + 16), ws))
    with pytest.raises(nat.Se12Error, match="hidden above 8192"):
        nat.step_check(lib.se12_step_rmsnorm(nat.ptr(x), nat.STEP_BF16, 9000, nat.ptr(x[0]), None, None, nat.ptr(x),
                                             2, 9000, 1e-6, 0.0, 0, s))
    with pytest.raises(nat.Se12Error, match="NULL"):
        nat.step_check(lib.se12_step_advance(None, nat.ptr(x), s))
    with pytest.raises(nat.Se12Error, match="NULL pos"):
        nat.step_check(lib.se12_step_logits_argmax_advance(nat.ptr(x), nat.STEP_BF16, 256000, 2, 256000, 0.0, None,
                                                           nat.ptr(x), nat.ptr(x), 4, nat.ptr(x), None, aligned, ws, s))
    with pytest.raises(nat.Se12Error, match="se12_step_logits_argmax_advance: workspace too small"):
        nat.step_check(lib.se12_step_logits_argmax_advance(nat.ptr(x), nat.STEP_BF16, 256000, 2, 256000, 0.0, None,
                                                           nat.ptr(x), nat.ptr(x), 4, nat.ptr(x), nat.ptr(x), aligned,
                                                           ws - 1, s))
    # the row-arrival counter after the per-row ones: 64 rows need a second 256-byte line
    assert lib.se12_step_logits_workspace(64, 2048) == 512 + 256 + 256
