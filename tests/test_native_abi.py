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
    text = HEADER.read_text()
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


def test_encoder_rejects_bad_shapes():
    lib = nat.lib()
    cb = (ctypes.c_uint8 * 15)()
    n = ctypes.c_int64()
    assert lib.se12_encode_prepare(None, 16, 256, 256, cb, ctypes.byref(n), None) == nat.SE12_E_INVALID
    assert lib.se12_encode_prepare(ctypes.c_void_p(16), 16, 256, 100, cb, ctypes.byref(n), None) == nat.SE12_E_INVALID


def test_launch_candidates_respect_each_kernels_limits():
    """BF16 batches of 5+ rows take the batched MFMA kernel (at most 8 waves
    per block and 16 K splits); FP32 x and smaller batches the dot2 kernel."""
    from se12_amd.launch import (candidate_configurations, configuration, max_waves_per_block, uses_mfma,
                                 waves_and_splits)

    assert not uses_mfma(4) and uses_mfma(5) and not uses_mfma(32, float32_activations=True)
    # MFMA blocks count row blocks of `waves` tile rows and need batch / 8 waves
    assert configuration(4, 3, 2304, batch=8).blocks.value == 36 * 3
    assert configuration(4, 3, 2304, batch=4).blocks.value == 144 * 3
    assert min(waves_and_splits(c, 2304, batch=32, k=9216)[0] for c in candidate_configurations(2304, 9216, batch=32)) == 4
    assert max_waves_per_block(1) == 16 and max_waves_per_block(6) == 8
    for batch, f32, max_s in ((1, False, 36), (6, False, 16), (32, False, 16), (6, True, 36)):
        cfgs = candidate_configurations(2304, 9216, batch=batch, float32_activations=f32)
        pairs = [waves_and_splits(c, 2304, batch=batch, k=9216, float32_activations=f32) for c in cfgs]
        assert max(s for _, s in pairs) == max_s
        assert max(w for w, _ in pairs) == max_waves_per_block(batch, f32)
