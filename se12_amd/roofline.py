"""The roofline model of the fused product, re-derived for MI355X.

Same formulas as the reference (lws/domain/performance/roofline.py:52-146,
weight-codec design.md):

    t_mem(format)     = bytes_per_weight(format) . W / BW
    t_compute(format) = W . c(format, B)
    t(format)         = max(t_mem, t_compute) + (1 - eta) . min(t_mem, t_compute)
    ratio             = t(SE12) / t(raw BF16)

with eta (overlap efficiency) fitted from a measured raw-kernel latency only.
Two changes: SE12 bytes per weight come from the exact stream sizes of the
shape (6,160 B per 16x256 tile + bitmap + codebook + fallback tiles, the
reference's summary.py:71-92 byte count) instead of the nominal 12.03/8,
and the device facts are MI355X's (8 TB/s HBM3E peak; 6.5 TB/s streaming
read measured here on weight-matrix-sized cold reads; ~1.7 us per launch in
a HIP graph, also measured here). `launch_floor_us` adds that launch cost,
which dominates small matrices.
"""

from __future__ import annotations

import dataclasses
import enum

from .format import packed_byte_size

SE12_BYTES_PER_WEIGHT_NOMINAL = 12.03 / 8
RAW_BYTES_PER_WEIGHT = 2.0
BYTES_PER_US_PER_GBPS = 1000.0          # 1 GB/s = 1e3 bytes per microsecond

HBM_PEAK_GBPS = 8000.0                   # MI355X HBM3E, published
STREAM_READ_GBPS = 6500.0                # measured: cold streaming read >= 128 MB
GRAPH_LAUNCH_US = 1.7                    # measured: one kernel node in a HIP graph


class WeightFormat(enum.Enum):
    RAW_BF16 = "raw_bf16"
    SE12 = "se12"


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


def fit_overlap_efficiency(measured_us: float, mem_us: float, compute_us: float) -> float:
    """eta from measured = max + (1 - eta) min, clamped to [0, 1] (roofline.py:77-91)."""
    larger, smaller = max(mem_us, compute_us), min(mem_us, compute_us)
    if smaller <= 0:
        return 1.0
    eta = 1.0 - (measured_us - larger) / smaller
    return min(max(eta, 0.0), 1.0)


def predicted_latency(mem_us: float, compute_us: float, eta: float) -> float:
    """max + (1 - eta) min (roofline.py:94-102)."""
    return max(mem_us, compute_us) + (1.0 - eta) * min(mem_us, compute_us)


@dataclasses.dataclass(frozen=True)
class Calibration:
    """One GPU: streaming bandwidth and compute cost per weight of each kernel
    at one batch size (cache-resident time / weights)."""

    bandwidth_gbps: float
    raw_cost_us_per_weight: float
    se12_cost_us_per_weight: float


def predict_shape_ratio(rows: int, cols: int, cal: Calibration, eta: float, exact: bool = True) -> float:
    """Predicted fused / raw-BF16 latency ratio for one shape (roofline.py:
    130-146), with the shape's exact SE12 bytes unless `exact` is False."""
    w = rows * cols
    se12_b = bytes_per_weight(WeightFormat.SE12, rows, cols) if exact else SE12_BYTES_PER_WEIGHT_NOMINAL
    raw = predicted_latency(memory_time(w, RAW_BYTES_PER_WEIGHT, cal.bandwidth_gbps),
                            compute_time(w, cal.raw_cost_us_per_weight), eta)
    se12 = predicted_latency(memory_time(w, se12_b, cal.bandwidth_gbps),
                             compute_time(w, cal.se12_cost_us_per_weight), eta)
    return se12 / raw


def launch_floor_us(rows: int, cols: int, batch: int = 1, bandwidth_gbps: float = STREAM_READ_GBPS,
                    launch_us: float = GRAPH_LAUNCH_US) -> float:
    """Lower bound of one fused launch on this GPU: the streams, x and y at the
    streaming bandwidth plus one graph launch."""
    nbytes = packed_byte_size(rows, cols, 0) + batch * cols * 2 + batch * rows * 4
    return launch_us + nbytes / (bandwidth_gbps * BYTES_PER_US_PER_GBPS)


def achieved(nbytes: int, microseconds: float, peak_gbps: float = HBM_PEAK_GBPS) -> dict:
    """GB/s of algorithmic bytes and the fraction of peak (bench.py's roofline)."""
    gbps = nbytes / (microseconds * 1e-6) / 1e9
    return {"achieved": gbps, "peak": peak_gbps, "frac": gbps / peak_gbps}
