"""Microbenchmark and per-GPU verdict: fused SE12 vs the lossless baselines.

    python -m se12_amd.micro --out reports/micro-<gpu-slug>.json

The reference's microbenchmark (lws/bench/micro.py:50-85,105-125) times the
raw-BF16 kernel and the fused SE12 kernel per (shape, batch) after an
accuracy pre-check against an FP64 product, reports median / p10 / p90 and
BF16-equivalent bandwidth, and decides a verdict per shape
(lws/application/gpu/run_microbenchmark.py:78-117,
lws/domain/benchmark/verdict.py:11-85): the ratio of the fused median to
the faster lossless baseline's, GO at <= 0.95, NO-GO above, INCONCLUSIVE
when that baseline reaches less than 70% of the measured copy bandwidth;
GO for the GPU only when every shape is GO. It writes `micro-<slug>.json`
and `verdict-<slug>.json` (lws/adapters/filesystem/report_store.py:13-44).

Here the same rules run over three variants: the fused kernel, its
same-skeleton raw-BF16 twin, and hipBLASLt's BF16 product (`F.linear`),
the baseline being the faster of the two lossless ones. Differences, each
deliberate:
- the verdict is recorded per batch size (1, 4 and 16), since the runtime's
  auto mode picks the path per batch (the reference records batch 1 only);
- activations are BF16, as a decode step feeds them (the reference passes
  FP32, which its kernels upcast to anyway);
- the cache flush before each sample covers L2 and the 256 MB Infinity
  Cache;
- each variant runs over a rotation of cold copies of the matrix captured
  back to back in one HIP graph, as a decode step issues its products, and
  a sample is one replay over its launches (timed eagerly, every variant
  pays ~2 us of host dispatch, a fifth of a launch at the 2B shapes, which
  alone pushes a bandwidth-bound baseline under the 70% bar; a graph of a
  single launch pays ~10 us per replay instead); the p10 / p90 are those of
  these per-replay means;
- the report carries the reference's metadata fields
  (lws/domain/benchmark/summary.py:11-41) with AMD facts under the
  reference's names (compute_capability = gfx architecture, sm_count =
  compute units, cuda_runtime_version = HIP runtime, nvrtc_version = the
  ahead-of-time library's build string, mig_enabled = a compute partition
  other than SPX), plus AMD-only fields; a fact the machine does not expose
  is null.
"""

from __future__ import annotations

import argparse
import dataclasses
import glob
import json
import os
import pathlib
import platform
import sys
from typing import Any, Callable

import numpy as np
import torch
import torch.nn.functional as F

from . import _native as nat
from .hip import (
    INFINITY_CACHE_BYTES,
    HipBenchmarkTimer,
    HipGpuProbe,
    LatencyStats,
    RawBf16MatVecKernel,
    Se12MatVecKernel,
    encode_on_device,
)
from .runtime import PEAK_BANDWIDTH_FRACTION, shape_verdict, verdict_payload

DEFAULT_SHAPES = ((2304, 9216), (9216, 2304), (256000, 2304))
DEFAULT_BATCHES = (1, 4, 16)
WARMUP_RUNS = 25
TIMED_RUNS = 100
RELATIVE_ACCURACY_TOLERANCE = 1e-2
FUSED = "fused_se12"
RAW = "raw_bf16"
BLAS = "hipblaslt_bf16"
BASELINES = (RAW, BLAS)


@dataclasses.dataclass(frozen=True)
class VariantResult:
    """One variant at one (shape, batch): rejected by the accuracy check
    (never timed), or timed."""

    name: str
    accuracy_passed: bool
    max_relative_error: float
    stats: LatencyStats | None = None
    bandwidth_gbps: float | None = None

    def as_dict(self) -> dict:
        if not self.accuracy_passed:
            return {"rejected": True, "reason": "failed accuracy/exactness check",
                    "max_relative_error": self.max_relative_error}
        return {"rejected": False, "median_microseconds": self.stats.median_us,
                "p10_microseconds": self.stats.p10_us, "p90_microseconds": self.stats.p90_us,
                "bandwidth_gbps": self.bandwidth_gbps, "max_relative_error": self.max_relative_error}


def bytes_moved(rows: int, cols: int, batch: int) -> int:
    """BF16-equivalent bytes of one product, the reference's count
    (micro.py:162-165): the weights as BF16 plus FP32 activations."""
    return rows * cols * 2 + batch * cols * 4


def within_tolerance(y: torch.Tensor, reference: torch.Tensor) -> tuple[bool, float]:
    """Max |y - ref| / max(|ref|, 1) <= 1e-2 against the FP64 product
    (micro.py:154-159)."""
    rel = ((y.double() - reference).abs() / reference.abs().clamp_min(1.0)).max().item()
    return rel <= RELATIVE_ACCURACY_TOLERANCE, float(rel)


def faster_baseline(results: dict[str, VariantResult]) -> VariantResult | None:
    """The faster timed lossless baseline (run_microbenchmark.py:78-94)."""
    timed = [results[n] for n in BASELINES if n in results and results[n].accuracy_passed]
    return min(timed, key=lambda r: r.stats.median_us) if timed else None


def decide_shape_verdict(results: dict[str, VariantResult], peak_gbps: float) -> dict | None:
    """None unless the fused kernel and a baseline were both timed
    (run_microbenchmark.py:102-117). `peak_gbps` is the copy peak as the
    reference measures it, the copied bytes counted once
    (HipBenchmarkTimer.measure_peak_copy_bandwidth;
    lws/adapters/cuda/benchmark_timer.py:55-66), and the baseline's rate is
    its BF16-equivalent bandwidth (bytes_moved / median), so
    `baseline_fraction_of_peak` is the reference's ratio
    (verdict.py:40-47)."""
    fused = results.get(FUSED)
    base = faster_baseline(results)
    if fused is None or not fused.accuracy_passed or base is None:
        return None
    ratio = fused.stats.median_us / base.stats.median_us
    fraction = base.bandwidth_gbps / peak_gbps
    return {"ratio": ratio, "baseline": base.name, "baseline_fraction_of_peak": fraction,
            "verdict": shape_verdict(ratio, fraction)}


def synthetic_weights(rows: int, cols: int, device) -> torch.Tensor:
    """numpy default_rng(0) N(0, 1) float32 rounded to BF16 (micro.py:143-145)."""
    a = np.random.default_rng(0).standard_normal((rows, cols), dtype=np.float32)
    return torch.from_numpy(a).to(device).to(torch.bfloat16)


def synthetic_activations(batch: int, cols: int, device, seed: int = 1) -> torch.Tensor:
    a = np.random.default_rng(seed).standard_normal((batch, cols), dtype=np.float32)
    return torch.from_numpy(a).to(device).to(torch.bfloat16)


def cold_copies(nbytes: int, minimum: int = 8) -> int:
    """Copies of one matrix to rotate through: together over 1.1 GB (4x the
    Infinity Cache), so that every launch reads HBM, and at least `minimum`
    launches per graph replay, over which the replay's fixed cost spreads."""
    return max(minimum, -(-int(1.1e9) // nbytes))


def benchmark_shape(rows: int, cols: int, batches, timer: HipBenchmarkTimer, peak_gbps: float, device,
                    warmup: int = WARMUP_RUNS, timed: int = TIMED_RUNS) -> list[dict]:
    """Every batch of one shape: accuracy pre-check of each variant on the
    first copy, then each passing variant timed over a rotation of cold
    copies (HipBenchmarkTimer.time_cold_rotation), then the shape's verdict
    at that batch."""
    w = synthetic_weights(rows, cols, device)
    dt = encode_on_device(w)
    copies = cold_copies(2 * rows * cols)
    ws = [w] + [w.clone() for _ in range(copies - 1)]
    fused = [Se12MatVecKernel(d) for d in [dt] + [dt.clone() for _ in range(copies - 1)]]
    raw = [RawBf16MatVecKernel(m) for m in ws]
    stream_bytes = dt.byte_size()
    rows_out = []
    for b in batches:
        x = synthetic_activations(b, cols, device, seed=1 + b)
        y_f = [torch.empty((b, rows), dtype=torch.float32, device=device) for _ in range(copies)]
        y_r = [torch.empty((b, rows), dtype=torch.float32, device=device) for _ in range(copies)]
        ops = {
            FUSED: [lambda k=k, y=y: k.multiply(x, out=y) for k, y in zip(fused, y_f)],
            RAW: [lambda k=k, y=y: k.multiply(x, out=y) for k, y in zip(raw, y_r)],
            BLAS: [lambda m=m: F.linear(x, m) for m in ws],
        }
        reference = F.linear(x.double(), w.double())
        moved = bytes_moved(rows, cols, b)
        results: dict[str, VariantResult] = {}
        for name, rotation in ops.items():
            ok, err = within_tolerance(rotation[0](), reference)
            if not ok:
                results[name] = VariantResult(name, False, err)
                continue
            st = timer.time_cold_rotation(rotation, warmup=warmup, timed=timed)
            results[name] = VariantResult(name, True, err, st, moved / (st.median_us * 1e-6) / 1e9)
        del reference
        row = {"shape": [rows, cols], "batch_size": b, "bytes_moved": moved, "se12_stream_bytes": stream_bytes,
               "cold_copies": copies, "results": {n: r.as_dict() for n, r in results.items()},
               "shape_verdict": decide_shape_verdict(results, peak_gbps)}
        if results.get(FUSED) is not None and results[FUSED].accuracy_passed:
            row["fused_stream_gbps"] = (stream_bytes + b * cols * 2 + b * rows * 4) / (results[FUSED].stats.median_us * 1e3)
        rows_out.append(row)
    del fused, raw, ws, w, dt
    torch.cuda.empty_cache()
    return rows_out


def _read(path: str) -> str | None:
    try:
        with open(path) as f:
            return f.read().strip()
    except OSError:
        return None


def _current_level(path: str) -> float | None:
    """The starred level of a pp_dpm_* table, in MHz."""
    text = _read(path)
    if not text:
        return None
    for line in text.splitlines():
        if line.strip().endswith("*"):
            digits = "".join(ch for ch in line.split(":", 1)[-1] if ch.isdigit() or ch == ".")
            return float(digits) if digits else None
    return None


def sysfs_facts(pci_address: str) -> dict:
    """What amdgpu's sysfs says about the device at `pci_address` (temperature,
    power cap, clocks, partitions, driver version); None where unreadable."""
    base = f"/sys/bus/pci/devices/{pci_address}"
    hwmon = sorted(glob.glob(f"{base}/hwmon/hwmon*"))
    h = hwmon[0] if hwmon else None
    temp = _read(f"{h}/temp1_input") if h else None
    power = (_read(f"{h}/power1_cap") if h else None)
    part = _read(f"{base}/current_compute_partition")
    return {
        "temperature_celsius": int(temp) / 1000.0 if temp and temp.lstrip("-").isdigit() else None,
        "power_limit_watts": int(power) / 1e6 if power and power.isdigit() else None,
        "sm_clock_mhz_current": _current_level(f"{base}/pp_dpm_sclk"),
        "memory_clock_mhz_current": _current_level(f"{base}/pp_dpm_mclk"),
        "compute_partition": part,
        "memory_partition": _read(f"{base}/current_memory_partition"),
        "amdgpu_driver_version": _read("/sys/module/amdgpu/version"),
    }


def _rocm_version() -> str | None:
    for path in ("/opt/rocm/.info/version", "/opt/rocm/.info/version-dev"):
        v = _read(path)
        if v:
            return v
    return None


def device_metadata(device, peak_gbps: float, warmup: int, timed: int) -> dict:
    """The reference's report metadata (lws/domain/benchmark/summary.py:
    14-41), AMD facts under its names, plus AMD-only fields."""
    props = HipGpuProbe(device.index).facts()
    fs = sysfs_facts(props.pci_address)
    part = fs["compute_partition"]
    return {
        "gpu_name": props.name,
        "gpu_slug": props.slug,
        "compute_capability": props.arch.split(":")[0],
        "sm_count": props.compute_units,
        "vram_bytes": props.total_memory_bytes,
        "l2_size_bytes": props.l2_bytes,
        "peak_copy_bandwidth_gbps": peak_gbps,
        "driver_version": fs["amdgpu_driver_version"] or props.driver_version,
        "cuda_runtime_version": props.runtime_version,
        "nvrtc_version": nat.version(),
        "torch_version": torch.__version__,
        "cupy_version": None,
        "compile_target": f"code-object {props.arch.split(':')[0]}",
        "compute_profile": "bf16-native",
        "sm_clock_mhz": props.clock_khz / 1000.0,
        "memory_clock_mhz": props.memory_clock_khz / 1000.0,
        "temperature_celsius": fs["temperature_celsius"],
        "power_limit_watts": fs["power_limit_watts"],
        "ecc_enabled": props.ecc_enabled,
        "mig_enabled": None if part is None else part.upper() != "SPX",
        "display_attached": props.kernel_timeout,
        "cuda_graphs_enabled": True,
        "warmup_runs": warmup,
        "timed_runs": timed,
        # AMD-only
        "gfx_arch": props.arch,
        "compute_units": props.compute_units,
        "infinity_cache_bytes": INFINITY_CACHE_BYTES,
        "memory_bus_width_bits": props.memory_bus_width_bits,
        "hbm_peak_gbps_from_clock": props.hbm_peak_gbps,
        "hip_runtime_version": props.runtime_version,
        "hip_driver_version": props.driver_version,
        "rocm_version": _rocm_version(),
        "torch_hip_version": getattr(torch.version, "hip", None),
        "compute_partition": part,
        "memory_partition": fs["memory_partition"],
        "sm_clock_mhz_current": fs["sm_clock_mhz_current"],
        "memory_clock_mhz_current": fs["memory_clock_mhz_current"],
        "pci_address": props.pci_address,
        "host": platform.node(),
        "activations": "bf16",
        "flush_bytes": int(timer_flush_bytes(props.l2_bytes)),
    }


def timer_flush_bytes(l2_bytes: int) -> int:
    return 2 * (int(l2_bytes) + INFINITY_CACHE_BYTES)


def run(shapes=DEFAULT_SHAPES, batches=DEFAULT_BATCHES, device=None, warmup: int = WARMUP_RUNS,
        timed: int = TIMED_RUNS, log: Callable[[str], None] | None = print) -> tuple[dict, dict]:
    """Measures every (shape, batch) and returns (micro report, verdict file)."""
    dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
    timer = HipBenchmarkTimer(dev.index)
    # the verdict's peak: the reference's copy figure (bytes counted once);
    # the copy's physical traffic (read + write) is reported beside it
    peak = float(timer.measure_peak_copy_bandwidth().value)
    traffic = timer.measure_copy_traffic_gbps()
    rows = []
    for r, c in shapes:
        got = benchmark_shape(r, c, batches, timer, peak, dev, warmup=warmup, timed=timed)
        for row in got:
            if log:
                v = row["shape_verdict"]
                med = {n: (d.get("median_microseconds")) for n, d in row["results"].items()}
                log(f"[micro] {r}x{c} B={row['batch_size']}: " +
                    ", ".join(f"{n} {m:.2f} us" if m is not None else f"{n} rejected" for n, m in med.items()) +
                    (f" -> ratio {v['ratio']:.3f} vs {v['baseline']} ({v['baseline_fraction_of_peak']:.0%} of copy peak): "
                     f"{v['verdict']}" if v else " -> no verdict"))
        rows.extend(got)
    meta = device_metadata(dev, peak, warmup, timed)
    ratios: dict[int, list[tuple]] = {}
    for row in rows:
        v = row["shape_verdict"]
        if v is not None:
            ratios.setdefault(row["batch_size"], []).append((tuple(row["shape"]), v["ratio"], v["baseline_fraction_of_peak"]))
    verdict = verdict_payload(meta["gpu_slug"], meta["compute_capability"], ratios)
    verdict["peak_copy_bandwidth_gbps"] = peak
    verdict["copy_traffic_gbps"] = traffic
    verdict["peak_bandwidth_fraction"] = PEAK_BANDWIDTH_FRACTION
    # the headline row (first shape, batch 1) carries the reference's
    # per-row metadata fields at the top level
    head = next((row for row in rows if row["batch_size"] == min(batches)), rows[0])
    fr = head["results"].get(FUSED, {})
    raw_rows = [row for row in rows if row["results"].get(RAW, {}).get("bandwidth_gbps")]
    micro = dict(meta)
    micro["copy_traffic_gbps"] = traffic
    micro.update({
        "shape": head["shape"], "batch_size": head["batch_size"],
        "median_microseconds": fr.get("median_microseconds"), "p10_microseconds": fr.get("p10_microseconds"),
        "p90_microseconds": fr.get("p90_microseconds"),
        "raw_bandwidth_fraction_of_peak": (min(row["results"][RAW]["bandwidth_gbps"] for row in raw_rows) / peak
                                           if raw_rows else None),
        "verdict": verdict["verdict"],
        "verdict_per_batch": {b: e["verdict"] for b, e in verdict["per_batch"].items()},
        "results": rows,
    })
    return micro, verdict


def write_reports(micro: dict, verdict: dict, out_dir) -> tuple[pathlib.Path, pathlib.Path]:
    """micro-<slug>.json and verdict-<slug>.json in `out_dir`
    (report_store.py:13-44)."""
    d = pathlib.Path(out_dir)
    d.mkdir(parents=True, exist_ok=True)
    mp = d / f"micro-{micro['gpu_slug']}.json"
    vp = d / f"verdict-{verdict['gpu_slug']}.json"
    mp.write_text(json.dumps(micro, indent=1))
    vp.write_text(json.dumps(verdict, indent=1))
    return mp, vp


def _shape(text: str) -> tuple[int, int]:
    r, c = text.lower().replace(",", "x").split("x")
    return int(r), int(c)


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser(prog="python -m se12_amd.micro")
    ap.add_argument("--out", default=None, help="micro-<slug>.json path or a directory (default: reports/)")
    ap.add_argument("--shapes", default=None, help="e.g. 2304x9216,9216x2304 (default: the reference's three)")
    ap.add_argument("--batches", default=None, help="e.g. 1,4,16")
    ap.add_argument("--warmup", type=int, default=WARMUP_RUNS)
    ap.add_argument("--timed", type=int, default=TIMED_RUNS)
    a = ap.parse_args(argv)
    if not torch.cuda.is_available():
        print("se12_amd.micro needs a HIP GPU", file=sys.stderr)
        return 2
    shapes = tuple(_shape(s) for s in a.shapes.split(",")) if a.shapes else DEFAULT_SHAPES
    batches = tuple(int(b) for b in a.batches.split(",")) if a.batches else DEFAULT_BATCHES
    micro, verdict = run(shapes, batches, warmup=a.warmup, timed=a.timed)
    out = pathlib.Path(a.out) if a.out else pathlib.Path(os.environ.get("LWS_VERDICT_DIR", "reports"))
    out_dir = out.parent if out.suffix == ".json" else out
    mp, vp = write_reports(micro, verdict, out_dir)
    print(f"verdict for GPU '{verdict['gpu_slug']}': {verdict['verdict']} (per batch: {micro['verdict_per_batch']}); "
          f"wrote {mp} and {vp}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
