"""The tuner's orchestration and its cache on the CPU, driven the way the
reference drives its own (tests/test_spec_tune.py:22-140 restated): requests
with a weight shape and a batch, an evaluator factory returning a raw / fused
pair of CandidateEvaluators, and a TuningCache object. Each kernel keeps its
own fastest passing configuration, the order-matched one is the best shared
passing one, a shape where nothing passes is left out, the filesystem cache
round-trips in the reference's JSON layout and ignores other GPUs' files, and
the lookup the runtime calls returns the tuned entries.

The stand-ins below are plain objects with the reference's attribute names
(lws/application/gpu/tune_launch.py:31-40, lws/application/ports/gpu/
tuning_cache.py:20-79, lws/domain/launch/search_space.py:44-48), so the
tuner is shown to read nothing but those attributes."""

from __future__ import annotations

import dataclasses
import json
import warnings

import pytest

from se12_amd import tune
from se12_amd.launch import candidate_configurations, waves_and_splits


@dataclasses.dataclass(frozen=True)
class RefWeightShape:
    output_rows: int
    k: int


@dataclasses.dataclass(frozen=True)
class RefBatch:
    value: int


@dataclasses.dataclass(frozen=True)
class RefRequest:
    weight_shape: RefWeightShape
    batch: RefBatch


@dataclasses.dataclass(frozen=True)
class RefSlug:
    value: str


@dataclasses.dataclass(frozen=True)
class RefMeasurement:
    median_latency_microseconds: float
    passes_accuracy_check: bool


@dataclasses.dataclass(frozen=True)
class RefPair:
    raw: object
    fused: object


class StandInEvaluator:
    """CandidateEvaluator: evaluate(configuration) -> measurement."""

    def __init__(self, fn) -> None:
        self.fn = fn
        self.seen = []

    def evaluate(self, configuration):
        self.seen.append(configuration)
        return self.fn(configuration)


class MemoryCache:
    """TuningCache kept in memory."""

    def __init__(self) -> None:
        self.stored = None

    def load(self):
        return self.stored

    def save(self, tuning_file) -> None:
        self.stored = tuning_file


def request(rows, cols, batch) -> RefRequest:
    return RefRequest(RefWeightShape(rows, cols), RefBatch(batch))


def pair_of(raw_fn, fused_fn):
    return lambda req: RefPair(raw=StandInEvaluator(lambda c: raw_fn(req, c)),
                               fused=StandInEvaluator(lambda c: fused_fn(req, c)))


def test_each_kernel_keeps_its_fastest_passing_configuration():
    req = request(2304, 9216, 1)
    cands = tune.tuning_candidates(2304, 9216, 1)
    # raw fastest at the smallest block, fused at the largest
    raw = lambda r, c: RefMeasurement(float(c.threads_per_block.value), True)
    fused = lambda r, c: RefMeasurement(float(-c.threads_per_block.value), True)
    cache = MemoryCache()
    tf = tune.tune_launch(RefSlug("amd-test-gfx950"), [req], pair_of(raw, fused), cache)
    assert tf.gpu_slug.value == "amd-test-gfx950"
    (e,) = tf.entries.items
    assert (e.key.weight_shape.output_rows, e.key.weight_shape.k, e.key.batch.value) == (2304, 9216, 1)
    assert e.configurations.independent.raw == min(cands, key=lambda c: c.threads_per_block.value)
    assert e.configurations.independent.fused == max(cands, key=lambda c: c.threads_per_block.value)
    assert e.configurations.order_matched in cands
    assert cache.stored is tf


def test_every_candidate_is_evaluated_for_both_kernels():
    req = request(1024, 2304, 4)
    made = []

    def evaluators(r):
        p = RefPair(raw=StandInEvaluator(lambda c: RefMeasurement(1.0, True)),
                    fused=StandInEvaluator(lambda c: RefMeasurement(1.0, True)))
        made.append(p)
        return p

    tune.tune_launch("g", [req], evaluators, MemoryCache())
    cands = list(tune.tuning_candidates(1024, 2304, 4))
    assert made[0].raw.seen == cands and made[0].fused.seen == cands


def test_order_matched_is_the_best_combined_passing_configuration():
    req = request(1024, 2304, 4)
    cands = tune.tuning_candidates(1024, 2304, 4)
    target = cands[len(cands) // 2]
    raw = lambda r, c: RefMeasurement(1.0 if c == target else 5.0, True)
    fused = lambda r, c: RefMeasurement(2.0 if c == target else 1.5, c == target or c == cands[0])
    tf = tune.tune_launch("g", [req], pair_of(raw, fused), MemoryCache())
    assert tf.entries.items[0].configurations.order_matched == target


def test_a_shape_where_nothing_passes_is_left_out():
    fail = lambda r, c: RefMeasurement(1.0, False)
    cache = MemoryCache()
    tf = tune.tune_launch("g", [request(256, 512, 1)], pair_of(fail, fail), cache)
    assert tf.entries.items == () and cache.stored is tf


def test_file_round_trips_in_the_reference_layout_and_feeds_the_lookup(tmp_path):
    reqs = [request(2304, 9216, 1), request(2304, 9216, 16)]
    ok = lambda r, c: RefMeasurement(float(c.blocks.value), True)
    cache = tune.FilesystemTuningCache(tmp_path, RefSlug("amd-x-gfx950"))
    tf = tune.tune_launch(RefSlug("amd-x-gfx950"), reqs, pair_of(ok, ok), cache)
    payload = json.loads((tmp_path / "tune-amd-x-gfx950.json").read_text())
    assert payload["gpu_slug"] == "amd-x-gfx950"
    assert set(payload["entries"][0]) == {"key", "configurations"}
    assert payload["entries"][0]["key"] == {"output_rows": 2304, "k": 9216, "batch": 1}
    assert set(payload["entries"][0]["configurations"]) == {"raw", "fused", "order_matched"}
    assert set(payload["entries"][0]["configurations"]["raw"]) == {"threads_per_block", "blocks"}
    back = cache.load()
    assert back == tf
    look = tune.tuning_lookup(back, "order_matched")
    assert look(2304, 9216, 16) == tf.entries.items[1].configurations.order_matched
    assert look(2304, 9216, 2) is None
    assert tune.tuning_lookup(back, "raw")(2304, 9216, 1) == tf.entries.items[0].configurations.independent.raw
    # the batch-16 entry is an MFMA configuration (row blocks x splits)
    waves, splits = waves_and_splits(look(2304, 9216, 16), 2304, batch=16, k=9216)
    assert 2 <= waves <= 12 and 1 <= splits <= 16
    with pytest.raises(ValueError):
        tune.tuning_lookup(back, "best")


def test_a_file_written_by_the_reference_layout_loads(tmp_path):
    """A file as the reference's filesystem adapter writes it
    (tuning_cache.py:107-135) loads into the same structure."""
    payload = {"gpu_slug": "amd-x-gfx950", "entries": [
        {"key": {"output_rows": 2304, "k": 9216, "batch": 1},
         "configurations": {"raw": {"threads_per_block": 512, "blocks": 144},
                            "fused": {"threads_per_block": 512, "blocks": 144},
                            "order_matched": {"threads_per_block": 384, "blocks": 144}}}]}
    (tmp_path / "tune-amd-x-gfx950.json").write_text(json.dumps(payload))
    tf = tune.FilesystemTuningCache(tmp_path, "amd-x-gfx950").load()
    (e,) = tf.entries.items
    assert e.configurations.order_matched.threads_per_block.value == 384
    assert tune.to_json(tf) == payload


def test_other_gpus_files_are_ignored_with_a_warning(tmp_path):
    tune.FilesystemTuningCache(tmp_path, "amd-other-gfx942").save(
        tune.tune_launch("amd-other-gfx942", [], pair_of(None, None), MemoryCache()))
    with warnings.catch_warnings(record=True) as w:
        warnings.simplefilter("always")
        assert tune.FilesystemTuningCache(tmp_path, "amd-x-gfx950").load() is None
    assert any("amd-other-gfx942" in str(x.message) for x in w)
    # the matching file is found even beside another GPU's
    mine = tune.FilesystemTuningCache(tmp_path, "amd-x-gfx950")
    mine.save(tune.tune_launch("amd-x-gfx950", [], pair_of(None, None), MemoryCache()))
    assert mine.load().gpu_slug.value == "amd-x-gfx950"


def test_no_directory_means_no_file(tmp_path):
    assert tune.FilesystemTuningCache(tmp_path / "missing", "g").load() is None


def test_candidates_cover_bf16_and_fp32_activations():
    """At 16 rows BF16 activations run an MFMA kernel and FP32 ones the dot2
    kernel: the tuner offers both sets, BF16's first, without repeats."""
    bf16 = candidate_configurations(2304, 9216, batch=16)
    f32 = candidate_configurations(2304, 9216, batch=16, float32_activations=True)
    both = tune.tuning_candidates(2304, 9216, 16)
    assert both[:len(bf16)] == bf16 and set(both) == set(bf16) | set(f32) and len(set(both)) == len(both)


def test_refused_configurations_count_as_failing():
    """An evaluator whose kernel refuses a configuration (the library raises
    for a launch its activations cannot take; the reference's evaluator does
    not catch that) leaves the candidate failing, not the tuner crashing."""
    from se12_amd._native import Se12Error

    f32 = set(candidate_configurations(2304, 9216, batch=16, float32_activations=True))

    def fn(r, c):
        if c not in f32:
            raise ValueError("threads_per_block 448 must be a multiple of 64 in [128, 512]")
        if c.blocks.value % 7 == 0:
            raise Se12Error(-2, "launch refused")
        return RefMeasurement(float(c.threads_per_block.value + c.blocks.value), True)

    tf = tune.tune_launch("g", [request(2304, 9216, 16)], pair_of(fn, fn), MemoryCache())
    (e,) = tf.entries.items
    for cfg in (e.configurations.independent.raw, e.configurations.independent.fused, e.configurations.order_matched):
        assert cfg in f32 and cfg.blocks.value % 7 != 0
