"""The tuner's orchestration and its cache file on the CPU, with fake
evaluators (the reference's tests/test_spec_tune.py:22-81 restated): each
kernel keeps its own fastest passing configuration, the order-matched one is
the best shared passing one, a shape where nothing passes is left out, the
file round-trips in the reference's JSON layout, other GPUs' files are
ignored, and the lookup the runtime calls returns the tuned entries."""

from __future__ import annotations

import json
import warnings

import pytest

from se12_amd import tune
from se12_amd.launch import TimingAndAccuracy, candidate_configurations, waves_and_splits


def _evals(raw_fn, fused_fn):
    return lambda req: (lambda c: raw_fn(req, c), lambda c: fused_fn(req, c))


def test_each_kernel_keeps_its_fastest_passing_configuration(tmp_path):
    req = tune.TuneRequest(2304, 9216, 1)
    cands = candidate_configurations(2304, 9216, batch=1)
    # raw fastest at the smallest block, fused at the largest, shared best at 4 waves 1 split
    raw = lambda r, c: TimingAndAccuracy(float(c.threads_per_block.value), True)
    fused = lambda r, c: TimingAndAccuracy(float(-c.threads_per_block.value), True)
    tf = tune.tune_launch("amd-test-gfx950", [req], _evals(raw, fused), directory=tmp_path)
    (e,) = tf.entries
    assert e.raw == min(cands, key=lambda c: c.threads_per_block.value)
    assert e.fused == max(cands, key=lambda c: c.threads_per_block.value)
    assert e.order_matched in cands
    assert (tmp_path / "tune-amd-test-gfx950.json").exists()


def test_order_matched_is_the_best_combined_passing_configuration(tmp_path):
    req = tune.TuneRequest(1024, 2304, 4)
    cands = candidate_configurations(1024, 2304, batch=4)
    target = cands[len(cands) // 2]
    raw = lambda r, c: TimingAndAccuracy(1.0 if c == target else 5.0, True)
    fused = lambda r, c: TimingAndAccuracy(2.0 if c == target else 1.5, c == target or c == cands[0])
    tf = tune.tune_launch("g", [req], _evals(raw, fused), save=False)
    assert tf.entries[0].order_matched == target


def test_a_shape_where_nothing_passes_is_left_out():
    req = tune.TuneRequest(256, 512, 1)
    fail = lambda r, c: TimingAndAccuracy(1.0, False)
    tf = tune.tune_launch("g", [req], _evals(fail, fail), save=False)
    assert tf.entries == ()


def test_file_round_trips_in_the_reference_layout_and_feeds_the_lookup(tmp_path):
    reqs = [tune.TuneRequest(2304, 9216, 1), tune.TuneRequest(2304, 9216, 16)]
    ok = lambda r, c: TimingAndAccuracy(float(c.blocks.value), True)
    tf = tune.tune_launch("amd-x-gfx950", reqs, _evals(ok, ok), directory=tmp_path)
    payload = json.loads((tmp_path / "tune-amd-x-gfx950.json").read_text())
    assert payload["gpu_slug"] == "amd-x-gfx950"
    assert set(payload["entries"][0]) == {"key", "configurations"}
    assert payload["entries"][0]["key"] == {"output_rows": 2304, "k": 9216, "batch": 1}
    assert set(payload["entries"][0]["configurations"]) == {"raw", "fused", "order_matched"}
    back = tune.load_tuning("amd-x-gfx950", tmp_path)
    assert back == tf
    look = back.lookup("order_matched")
    assert look(2304, 9216, 16) == tf.entries[1].order_matched
    assert look(2304, 9216, 2) is None
    # the batch-16 entry is an MFMA configuration (row blocks x splits)
    waves, splits = waves_and_splits(look(2304, 9216, 16), 2304, batch=16, k=9216)
    assert 2 <= waves <= 8 and 1 <= splits <= 16
    with pytest.raises(ValueError):
        back.lookup("best")


def test_other_gpus_files_are_ignored_with_a_warning(tmp_path):
    tune.save_tuning(tune.TuningFile("amd-other-gfx942", ()), tmp_path)
    with warnings.catch_warnings(record=True) as w:
        warnings.simplefilter("always")
        assert tune.load_tuning("amd-x-gfx950", tmp_path) is None
    assert any("another GPU" in str(x.message) for x in w)
