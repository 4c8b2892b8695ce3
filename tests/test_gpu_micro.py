"""The microbenchmark on the GPU at small shapes: both reports are written
with every metadata field the reference's report check requires
(lws/domain/benchmark/summary.py:14-41), each (shape, batch) row carries
consistent timings and a verdict that follows the rules, and
`load_packed(mode="auto")` then takes the fused path exactly for the batch
sizes the written verdict file calls GO (AC-025)."""

from __future__ import annotations

import json

import pytest
import torch

from se12_amd import micro, runtime

pytestmark = pytest.mark.gpu

# lws/domain/benchmark/summary.py:14-41
REQUIRED_METADATA_FIELDS = (
    "gpu_name", "gpu_slug", "compute_capability", "sm_count", "vram_bytes", "l2_size_bytes",
    "peak_copy_bandwidth_gbps", "driver_version", "cuda_runtime_version", "nvrtc_version", "torch_version",
    "cupy_version", "compile_target", "compute_profile", "sm_clock_mhz", "memory_clock_mhz", "temperature_celsius",
    "power_limit_watts", "ecc_enabled", "mig_enabled", "display_attached", "cuda_graphs_enabled", "shape",
    "batch_size", "warmup_runs", "timed_runs", "median_microseconds", "p10_microseconds", "p90_microseconds",
)


def test_micro_reports_and_auto_mode_follow_the_measurement(gpu, tmp_path):
    from test_gpu_runtime import _tiny_gemma

    shapes = ((512, 256), (2304, 2304))
    micro_rep, verdict = micro.run(shapes, (1, 4, 16), device=gpu, warmup=3, timed=10, log=None)
    mp, vp = micro.write_reports(micro_rep, verdict, tmp_path / "reports")
    m = json.loads(mp.read_text())
    v = json.loads(vp.read_text())
    assert not [f for f in REQUIRED_METADATA_FIELDS if f not in m]
    assert m["gpu_slug"] == runtime.current_gpu_slug(gpu) == v["gpu_slug"]
    assert m["compute_capability"].startswith("gfx") and m["sm_count"] > 0 and m["peak_copy_bandwidth_gbps"] > 100
    assert len(m["results"]) == len(shapes) * 3
    for row in m["results"]:
        res = row["results"]
        assert set(res) == {micro.FUSED, micro.RAW, micro.BLAS}
        for r in res.values():
            assert not r["rejected"], r
            assert 0 < r["p10_microseconds"] <= r["median_microseconds"] <= r["p90_microseconds"]
        sv = row["shape_verdict"]
        base = min((micro.RAW, micro.BLAS), key=lambda n: res[n]["median_microseconds"])
        assert sv["baseline"] == base
        assert sv["ratio"] == pytest.approx(res[micro.FUSED]["median_microseconds"] / res[base]["median_microseconds"])
        assert sv["verdict"] == runtime.shape_verdict(sv["ratio"], sv["baseline_fraction_of_peak"])
    for b in ("1", "4", "16"):
        per = [row["shape_verdict"]["verdict"] for row in m["results"] if str(row["batch_size"]) == b]
        assert v["per_batch"][b]["verdict"] == runtime.aggregate_verdict(per)

    model, cfg = _tiny_gemma(gpu, seed=13, layers=1)
    runtime.pack_pretrained(model, tmp_path / "packed")
    auto = runtime.load_packed(tmp_path / "packed", mode="auto", device=gpu, verdict_dir=tmp_path / "reports", log=None)
    lin = auto.lm_head
    assert lin.policy.source == str(vp)
    for b, want in ((1, "1"), (2, "4"), (4, "4"), (9, "16"), (16, "16")):
        assert lin.uses_fused(b, False) == (v["per_batch"][want]["verdict"] == "GO"), b
    assert not lin.uses_fused(17, False) and not lin.uses_fused(1, True)
    ids = torch.randint(0, cfg.vocab_size, (1, 6), device=gpu)
    with torch.no_grad():
        out = auto.generate(ids, max_new_tokens=3, do_sample=False)
    assert out.shape == (1, 9)


def test_micro_cli_writes_both_files(gpu, tmp_path):
    rc = micro.main(["--out", str(tmp_path / "micro-x.json"), "--shapes", "256x512", "--batches", "1",
                     "--warmup", "2", "--timed", "5"])
    assert rc == 0
    slug = runtime.current_gpu_slug(gpu)
    assert (tmp_path / f"micro-{slug}.json").exists() and (tmp_path / f"verdict-{slug}.json").exists()
