"""The roofline model of the fused product, fed by the device and by
measurement.

Same formulas as the reference (lws/domain/performance/roofline.py:52-146,
weight-codec design.md):

    t_mem(format)     = bytes_per_weight(format) . W / BW
    t_compute(format) = W . c(format, B)
    t(format)         = max(t_mem, t_compute) + (1 - eta) . min(t_mem, t_compute)
    ratio             = t(SE12) / t(raw BF16)

with eta (overlap efficiency) fitted from a measured raw-kernel latency only,
so the fused kernel's predicted ratio is an out-of-sample test
(roofline.py:1-12,77-91). Where the inputs come from here:

- BW: the HBM traffic of a device-to-device copy (read + write counted).
  The reference calibrates with its copy bandwidth with the copied bytes
  counted once (adapters/cuda/calibration_probe.py:38-40, benchmark_timer.py:
  55-66), about a third of what a read-only pass streams here; with the
  traffic figure the fitted model predicts the fused / raw ratios of the
  Gemma-2-2B shapes within 5-20%, with the fastest streaming read (6.4 TB/s)
  it puts every shape compute-bound and misses by up to 44%. The streaming
  read bandwidth, the larger of a grid-stride read probe and the fused
  product's own stream over a cold LM head, is measured beside it and bounds
  each launch from below (launch_floor_us);
- c(format, B): each kernel's time per weight on cache-resident data, as the
  reference defines it (calibration_probe.py:44-63), but as the slope
  between two matrices that fill the GPU and stay in the 256 MB Infinity
  Cache (2304x2304 and 4608x2304: 8 / 16 MB of SE12 streams, 10.6 / 21 MB of
  BF16), each timed as back-to-back launches in a graph; the reference's one
  16x256 tile would time a single launch's fixed cost, which on this GPU
  (~1.7 us per graph node) outweighs the per-weight work of a whole 2B
  projection and made both kernels look compute-bound;
- t(format) gains that fixed cost as its own term, t_launch + max + (1 -
  eta) min, with t_launch measured as one small kernel node of a graph;
- peak: hipDeviceProp's memory clock x bus width (the device's own figure,
  `DeviceFacts.hbm_peak_gbps`) beside the published 8.0 TB/s.

SE12 bytes per weight come from the exact stream sizes of the shape (6,160 B
per 16x256 tile + bitmap + codebook + fallback tiles, the reference's
summary.py:71-92 byte count) instead of the nominal 12.03/8.
"""

from __future__ import annotations

import dataclasses
import enum

from .format import packed_byte_size

SE12_BYTES_PER_WEIGHT_NOMINAL = 12.03 / 8
RAW_BYTES_PER_WEIGHT = 2.0
BYTES_PER_US_PER_GBPS = 1000.0          # 1 GB/s = 1e3 bytes per microsecond
HBM_PEAK_PUBLISHED_GBPS = 8000.0         # MI355X HBM3E, AMD's published figure
# the cache-resident calibration shapes (see the module docstring)
CALIBRATION_SHAPES = ((2304, 2304), (4608, 2304))


class WeightFormat(enum.Enum):
    RAW_BF16 = "raw_bf16"
    SE12 = "se12"


@dataclasses.dataclass(frozen=True)
class DeviceFacts:
    """One GPU's inputs to the model: the peak derived from hipDeviceProp and
    what was measured on it."""

    hbm_peak_gbps: float          # memory clock x transfers per clock x bus width
    copy_gbps: float              # device-to-device copy, read + write counted
    stream_read_gbps: float       # the fastest streaming read measured (cold, over 4x L2 + Infinity Cache)
    launch_us: float              # one small kernel node of a HIP graph


def bytes_per_weight(fmt: WeightFormat, rows: int | None = None, cols: int | None = None,
                     fallback_tiles: int = 0) -> float:
    """Bytes per weight of one pass; SE12 exact for a shape when given."""
    if fmt is WeightFormat.RAW_BF16:
        return RAW_BYTES_PER_WEIGHT
    if rows is None or cols is None:
        return SE12_BYTES_PER_WEIGHT_NOMINAL
    return packed_byte_size(rows, cols, fallback_tiles) / (rows * cols)


def memory_time(weights: int, bytes_per_weight_: float, bandwidth_gbps: float) -> float:
    """Microseconds to stream `weights` at `bytes_per_weight_` (roofline.py:52-60)."""
    return weights * bytes_per_weight_ / (bandwidth_gbps * BYTES_PER_US_PER_GBPS)


def compute_time(weights: int, cost_us_per_weight: float) -> float:
    """Microseconds of compute-bound time (roofline.py:63-67)."""
    return weights * cost_us_per_weight


def fit_overlap_efficiency(measured_us: float, mem_us: float, compute_us: float, launch_us: float = 0.0) -> float:
    """eta from measured = launch + max + (1 - eta) min, clamped to [0, 1]
    (roofline.py:77-91)."""
    larger, smaller = max(mem_us, compute_us), min(mem_us, compute_us)
    if smaller <= 0:
        return 1.0
    eta = 1.0 - (measured_us - launch_us - larger) / smaller
    return min(max(eta, 0.0), 1.0)


def predicted_latency(mem_us: float, compute_us: float, eta: float, launch_us: float = 0.0) -> float:
    """launch + max + (1 - eta) min (roofline.py:94-102, plus the fixed
    per-launch cost)."""
    return launch_us + max(mem_us, compute_us) + (1.0 - eta) * min(mem_us, compute_us)


@dataclasses.dataclass(frozen=True)
class Calibration:
    """One GPU at one batch size: the bandwidth, each kernel's compute cost
    per weight (cache-resident) and the fixed cost of a launch."""

    bandwidth_gbps: float
    raw_cost_us_per_weight: float
    se12_cost_us_per_weight: float
    launch_us: float = 0.0


def calibrate(bandwidth_gbps: float, raw_hot_us: tuple[float, float], se12_hot_us: tuple[float, float],
              launch_us: float = 0.0, shapes=CALIBRATION_SHAPES) -> Calibration:
    """Costs per weight as the slope of each kernel's cache-resident time
    between the two calibration shapes (the fixed per-launch part cancels)."""
    dw = shapes[1][0] * shapes[1][1] - shapes[0][0] * shapes[0][1]
    return Calibration(bandwidth_gbps, max(raw_hot_us[1] - raw_hot_us[0], 0.0) / dw,
                       max(se12_hot_us[1] - se12_hot_us[0], 0.0) / dw, launch_us)


def fit_eta_from_raw(raw_measured_us: float, rows: int, cols: int, cal: Calibration) -> float:
    """eta from the raw twin's measured (cold) latency at one shape, the
    model's own t_mem, t_compute and launch cost for the raw kernel there."""
    w = rows * cols
    return fit_overlap_efficiency(raw_measured_us, memory_time(w, RAW_BYTES_PER_WEIGHT, cal.bandwidth_gbps),
                                  compute_time(w, cal.raw_cost_us_per_weight), cal.launch_us)


def predict_latencies(rows: int, cols: int, cal: Calibration, eta: float, exact: bool = True,
                      fallback_tiles: int = 0) -> tuple[float, float]:
    """(raw, SE12) predicted microseconds for one shape."""
    w = rows * cols
    se12_b = bytes_per_weight(WeightFormat.SE12, rows, cols, fallback_tiles) if exact else SE12_BYTES_PER_WEIGHT_NOMINAL
    raw = predicted_latency(memory_time(w, RAW_BYTES_PER_WEIGHT, cal.bandwidth_gbps),
                            compute_time(w, cal.raw_cost_us_per_weight), eta, cal.launch_us)
    se12 = predicted_latency(memory_time(w, se12_b, cal.bandwidth_gbps),
                             compute_time(w, cal.se12_cost_us_per_weight), eta, cal.launch_us)
    return raw, se12


def predict_shape_ratio(rows: int, cols: int, cal: Calibration, eta: float, exact: bool = True,
                        fallback_tiles: int = 0) -> float:
    """Predicted fused / raw-BF16 latency ratio for one shape (roofline.py:
    130-146), with the shape's exact SE12 bytes unless `exact` is False."""
    raw, se12 = predict_latencies(rows, cols, cal, eta, exact, fallback_tiles)
    return se12 / raw


def launch_floor_us(rows: int, cols: int, facts: DeviceFacts, batch: int = 1) -> float:
    """Lower bound of one fused launch on this GPU: the streams, x and y at
    the fastest streaming-read bandwidth measured on it, plus one graph
    launch."""
    nbytes = packed_byte_size(rows, cols, 0) + batch * cols * 2 + batch * rows * 4
    return facts.launch_us + nbytes / (facts.stream_read_gbps * BYTES_PER_US_PER_GBPS)


def achieved(nbytes: int, microseconds: float, peak_gbps: float) -> dict:
    """GB/s of algorithmic bytes and the fraction of peak (bench.py's roofline)."""
    gbps = nbytes / (microseconds * 1e-6) / 1e9
    return {"achieved": gbps, "peak": peak_gbps, "frac": gbps / peak_gbps}


def shape_report(rows: int, cols: int, cal: Calibration, eta: float, fused_us: float, raw_us: float,
                 fallback_tiles: int = 0) -> dict:
    """Predicted against measured for one shape: latencies and the fused /
    raw ratio."""
    p_raw, p_se12 = predict_latencies(rows, cols, cal, eta, True, fallback_tiles)
    measured = fused_us / raw_us
    predicted = p_se12 / p_raw
    return {"predicted_raw_us": p_raw, "predicted_se12_us": p_se12, "predicted_ratio": predicted,
            "measured_ratio": measured, "measured_over_predicted": measured / predicted}
