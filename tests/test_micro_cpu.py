"""The microbenchmark's decision rules without a GPU: the faster lossless
baseline, GO / NO-GO / INCONCLUSIVE per shape (lws/domain/benchmark/
verdict.py:11-85, lws/application/gpu/run_microbenchmark.py:78-117), the
per-batch aggregation, the reference's byte count and accuracy bound, and
the sysfs readers' tolerance of machines that expose nothing."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from se12_amd import micro, runtime
from se12_amd.hip import latency_stats


def timed(name: str, median_us: float, gbps: float) -> micro.VariantResult:
    return micro.VariantResult(name, True, 1e-6, latency_stats([median_us] * 3), gbps)


def rejected(name: str) -> micro.VariantResult:
    return micro.VariantResult(name, False, 0.5)


PEAK = 5000.0


@pytest.mark.parametrize("fused_us,raw,blas,expect", [
    (8.0, (10.0, 4000.0), (12.0, 3400.0), ("GO", micro.RAW, 0.8)),
    (9.6, (10.0, 4000.0), (12.0, 3400.0), ("NO-GO", micro.RAW, 0.96)),
    (9.5, (10.0, 4000.0), (12.0, 3400.0), ("GO", micro.RAW, 0.95)),          # the threshold is inclusive
    (8.0, (12.0, 3300.0), (10.0, 4000.0), ("GO", micro.BLAS, 0.8)),          # hipBLASLt the faster baseline
    (8.0, (10.0, 3400.0), (12.0, 3000.0), ("INCONCLUSIVE", micro.RAW, 0.8)),  # 68% of the copy peak
    (8.0, (10.0, 3500.0), (12.0, 3000.0), ("GO", micro.RAW, 0.8)),           # exactly 70%: valid
])
def test_shape_verdict_against_the_faster_baseline(fused_us, raw, blas, expect):
    res = {micro.FUSED: timed(micro.FUSED, fused_us, 1.0), micro.RAW: timed(micro.RAW, *raw),
           micro.BLAS: timed(micro.BLAS, *blas)}
    v = micro.decide_shape_verdict(res, PEAK)
    assert (v["verdict"], v["baseline"]) == expect[:2]
    assert v["ratio"] == pytest.approx(expect[2])
    assert v["baseline_fraction_of_peak"] == pytest.approx(res[expect[1]].bandwidth_gbps / PEAK)


def test_rejected_variants_are_never_the_baseline_and_block_a_verdict():
    base = {micro.RAW: timed(micro.RAW, 10.0, 4000.0), micro.BLAS: timed(micro.BLAS, 9.0, 4400.0)}
    assert micro.decide_shape_verdict({micro.FUSED: rejected(micro.FUSED), **base}, PEAK) is None
    v = micro.decide_shape_verdict({micro.FUSED: timed(micro.FUSED, 8.0, 1), micro.RAW: timed(micro.RAW, 10.0, 4000.0),
                                    micro.BLAS: rejected(micro.BLAS)}, PEAK)
    assert v["baseline"] == micro.RAW
    assert micro.decide_shape_verdict({micro.FUSED: timed(micro.FUSED, 8.0, 1), micro.RAW: rejected(micro.RAW),
                                       micro.BLAS: rejected(micro.BLAS)}, PEAK) is None


def test_payload_aggregates_per_batch_with_inconclusive_first():
    ratios = {1: [((2304, 9216), 0.8, 0.9), ((256000, 2304), 0.7, 0.95)],
              4: [((2304, 9216), 0.8, 0.9), ((256000, 2304), 0.97, 0.95)],
              16: [((2304, 9216), 0.5, 0.4), ((256000, 2304), 1.2, 0.95)]}
    p = runtime.verdict_payload("gpu-gfx950", "gfx950", ratios)
    assert {b: e["verdict"] for b, e in p["per_batch"].items()} == {"1": "GO", "4": "NO-GO", "16": "INCONCLUSIVE"}
    assert p["verdict"] == "GO" and p["compute_capability"] == "gfx950"
    assert p["per_batch"]["16"]["per_shape"][0] == {"shape": [2304, 9216], "ratio": 0.5, "verdict": "INCONCLUSIVE",
                                                    "baseline_fraction_of_peak": 0.4}
    policy = runtime.FusedPolicy(frozenset({int(b) for b, e in p["per_batch"].items() if e["verdict"] == "GO"}))
    assert [policy.fused_for(b) for b in (1, 2, 4, 16)] == [True, False, False, False]


def test_byte_count_and_accuracy_bound_are_the_reference_s():
    assert micro.bytes_moved(2304, 9216, 1) == 2304 * 9216 * 2 + 9216 * 4 == 42_504_192
    ref = torch.tensor([[0.5, 100.0]], dtype=torch.float64)
    ok, err = micro.within_tolerance(torch.tensor([[0.509, 100.9]]), ref)     # |d| / max(|r|, 1)
    assert ok and err == pytest.approx(0.009, rel=1e-3)
    ok, _ = micro.within_tolerance(torch.tensor([[0.511, 100.0]]), ref)
    assert not ok


def test_sysfs_readers_tolerate_missing_files(tmp_path):
    facts = micro.sysfs_facts("ffff:ff:1f.0")
    for k in ("temperature_celsius", "power_limit_watts", "sm_clock_mhz_current", "compute_partition"):
        assert facts[k] is None
    table = tmp_path / "pp_dpm_sclk"
    table.write_text("0: 500Mhz\n1: 1400Mhz *\n2: 2400Mhz\n")
    assert micro._current_level(str(table)) == 1400.0
    table.write_text("0: 500Mhz\n")
    assert micro._current_level(str(table)) is None


# Medians (us) of one full MI355X microbenchmark run: (rows, cols, batch,
# fused, raw twin, hipBLASLt). Its copy of 1 GiB moved 4,628.4 GB/s of HBM
# traffic, i.e. 2,314.2 GB/s with the copied bytes counted once.
MEASURED_ROWS = [
    (2304, 9216, 1, 9.259, 10.246, 14.789),
    (2304, 9216, 4, 11.482, 13.502, 14.854),
    (2304, 9216, 16, 17.063, 17.936, 15.260),
    (9216, 2304, 1, 8.619, 11.190, 15.050),
    (9216, 2304, 4, 10.762, 11.859, 15.337),
    (9216, 2304, 16, 13.920, 15.453, 15.480),
    (256000, 2304, 1, 141.660, 184.914, 193.561),
    (256000, 2304, 4, 159.098, 193.506, 196.643),
    (256000, 2304, 16, 183.955, 291.371, 201.955),
]
COPY_TRAFFIC_GBPS = 4628.4


def _replay(peak_gbps: float) -> dict:
    ratios: dict = {}
    for rows, cols, b, fused, raw, blas in MEASURED_ROWS:
        moved = micro.bytes_moved(rows, cols, b)
        res = {n: timed(n, us, moved / (us * 1e-6) / 1e9)
               for n, us in ((micro.FUSED, fused), (micro.RAW, raw), (micro.BLAS, blas))}
        v = micro.decide_shape_verdict(res, peak_gbps)
        ratios.setdefault(b, []).append(((rows, cols), v["ratio"], v["baseline_fraction_of_peak"]))
    p = runtime.verdict_payload("gpu-gfx950", "gfx950", ratios)
    return {b: e["verdict"] for b, e in p["per_batch"].items()}


def test_measured_rows_give_the_reference_verdicts_with_the_copy_counted_once():
    """The reference's 70% bar divides the baseline's BF16-equivalent rate by
    a copy whose bytes are counted once (lws/adapters/cuda/benchmark_timer.py:
    55-66, verdict.py:40-47). On these rows every baseline clears it, so batch
    1 and 4 are GO (every ratio <= 0.95) and batch 16 is NO-GO (2304x9216 at
    1.118 against hipBLASLt)."""
    assert _replay(COPY_TRAFFIC_GBPS / 2) == {"1": "GO", "4": "GO", "16": "NO-GO"}
    # a copy counted twice (read + write) halves every fraction and turns the
    # same timings INCONCLUSIVE at batch 4 and 16
    assert _replay(COPY_TRAFFIC_GBPS) == {"1": "GO", "4": "INCONCLUSIVE", "16": "INCONCLUSIVE"}


def test_auto_policy_follows_the_replayed_verdict(tmp_path):
    ratios: dict = {}
    for rows, cols, b, fused, raw, blas in MEASURED_ROWS:
        moved = micro.bytes_moved(rows, cols, b)
        res = {n: timed(n, us, moved / (us * 1e-6) / 1e9)
               for n, us in ((micro.FUSED, fused), (micro.RAW, raw), (micro.BLAS, blas))}
        v = micro.decide_shape_verdict(res, COPY_TRAFFIC_GBPS / 2)
        ratios.setdefault(b, []).append(((rows, cols), v["ratio"], v["baseline_fraction_of_peak"]))
    runtime.write_verdict(runtime.verdict_payload("gpu-gfx950", "gfx950", ratios), tmp_path)
    pol = runtime.load_policy("gpu-gfx950", tmp_path)
    assert [pol.fused_for(b) for b in (1, 2, 4, 5, 16, 17)] == [True, True, True, False, False, False]
