"""The roofline model (se12_amd/roofline.py) against closed forms: the
reference's known answers (tests/test_spec_performance_model.py:30-121,
restated with their numbers), the exact SE12 byte count per shape, and the
crossing of ratio 1 as the decode cost grows."""

from __future__ import annotations

import dataclasses

import pytest

from se12_amd import roofline as r


def test_bytes_per_weight():
    assert r.bytes_per_weight(r.WeightFormat.RAW_BF16) == 2.0
    assert r.bytes_per_weight(r.WeightFormat.SE12) == pytest.approx(12.03 / 8)
    # exact: 5,184 tiles x 6,160 B + 648 B bitmap + 15 B codebook over 21,233,664 weights
    assert r.bytes_per_weight(r.WeightFormat.SE12, 2304, 9216) == pytest.approx((5184 * 6160 + 648 + 15) / (2304 * 9216))
    # a fallback tile adds 8,192 raw bytes
    assert r.bytes_per_weight(r.WeightFormat.SE12, 16, 256, fallback_tiles=1) == pytest.approx((6160 + 1 + 15 + 8192) / 4096)


def test_memory_and_compute_time():
    # 1e9 weights x 2 B at 1000 GB/s = 1e6 B/us -> 2000 us
    assert r.memory_time(10**9, 2.0, 1000.0) == pytest.approx(2000.0)
    assert r.compute_time(1000, 0.01) == pytest.approx(10.0)


@pytest.mark.parametrize("measured,eta", [(100.0, 1.0), (120.0, 0.0), (110.0, 0.5), (50.0, 1.0), (500.0, 0.0)])
def test_fit_overlap_efficiency(measured, eta):
    assert r.fit_overlap_efficiency(measured, 100.0, 20.0) == pytest.approx(eta)


def test_predicted_latency_extremes():
    assert r.predicted_latency(100.0, 20.0, 1.0) == pytest.approx(100.0)
    assert r.predicted_latency(100.0, 20.0, 0.0) == pytest.approx(120.0)
    # the fit inverts the prediction
    for eta in (0.0, 0.3, 1.0):
        assert r.fit_overlap_efficiency(r.predicted_latency(100.0, 20.0, eta), 100.0, 20.0) == pytest.approx(eta)


def test_ratio_tends_to_the_byte_ratio_when_compute_is_negligible():
    cal = r.Calibration(bandwidth_gbps=6500.0, raw_cost_us_per_weight=1e-12, se12_cost_us_per_weight=1e-12)
    exact = r.predict_shape_ratio(2304, 9216, cal, eta=0.0)
    assert exact == pytest.approx(r.bytes_per_weight(r.WeightFormat.SE12, 2304, 9216) / 2.0, rel=1e-5)
    assert r.predict_shape_ratio(2304, 9216, cal, eta=0.0, exact=False) == pytest.approx(12.03 / 16, rel=1e-5)


def test_ratio_crosses_one_as_the_decode_cost_grows():
    ratios = []
    for k in (1e-7, 1e-6, 1e-5, 1e-4, 1e-3):
        cal = r.Calibration(bandwidth_gbps=320.0, raw_cost_us_per_weight=1e-7, se12_cost_us_per_weight=k)
        ratios.append(r.predict_shape_ratio(2304, 9216, cal, eta=0.5))
    assert ratios == sorted(ratios) and ratios[0] < 1.0 < ratios[-1]


def test_launch_floor_and_achieved():
    facts = r.DeviceFacts(hbm_peak_gbps=8192.0, copy_gbps=5000.0, stream_read_gbps=6500.0, launch_us=1.7)
    # down_proj: 31,961,751 algorithmic bytes at 6.5 TB/s + one launch
    assert r.launch_floor_us(2304, 9216, facts) == pytest.approx(1.7 + 31961751 / 6.5e6)
    a = r.achieved(31961751, 10.0, 8000.0)
    assert a["achieved"] == pytest.approx(3196.1751) and a["frac"] == pytest.approx(3196.1751 / 8000.0)


def test_calibration_and_eta_fit_from_the_raw_kernel():
    # cache-resident 2304x2304 / 4608x2304: raw 3 / 4.5 us, SE12 4 / 6 us -> slopes per weight
    cal = r.calibrate(5000.0, raw_hot_us=(3.0, 4.5), se12_hot_us=(4.0, 6.0), launch_us=1.5)
    dw = 4608 * 2304 - 2304 * 2304
    assert cal.raw_cost_us_per_weight == pytest.approx(1.5 / dw) and cal.se12_cost_us_per_weight == pytest.approx(2.0 / dw)
    # raw twin at 2304x9216: t_mem = 42,467,328 B / 5e3 B/us = 8.493 us, t_compute = 4 x 1.5 = 6 us
    mem, comp = 2304 * 9216 * 2 / 5000e3, 4 * 1.5
    for eta in (0.0, 0.4, 1.0):
        measured = r.predicted_latency(mem, comp, eta, 1.5)
        assert measured == pytest.approx(1.5 + mem + (1 - eta) * comp)
        assert r.fit_eta_from_raw(measured, 2304, 9216, cal) == pytest.approx(eta)
    # the fitted eta reproduces the raw measurement; the fused prediction is out of sample
    eta = r.fit_eta_from_raw(12.0, 2304, 9216, cal)
    rep = r.shape_report(2304, 9216, cal, eta, fused_us=9.0, raw_us=12.0)
    assert rep["predicted_raw_us"] == pytest.approx(12.0)
    assert rep["measured_ratio"] == pytest.approx(9.0 / 12.0)
    assert rep["measured_over_predicted"] == pytest.approx(rep["measured_ratio"] / rep["predicted_ratio"])
    # a slower cache-resident kernel at the larger size never gives a negative cost
    assert r.calibrate(5000.0, (3.0, 2.0), (4.0, 3.0)).raw_cost_us_per_weight == 0.0


def test_peak_from_hip_device_properties():
    from se12_amd.hip import DeviceFacts

    p = DeviceFacts(name="x", arch="gfx950:sramecc+:xnack-", compute_units=256, wavefront_size=64, l2_bytes=4 << 20,
                    lds_bytes_per_cu=160 << 10, lds_bytes_per_block=160 << 10, total_memory_bytes=288 << 30,
                    clock_khz=2_400_000, memory_clock_khz=2_000_000, memory_bus_width_bits=8192)
    # MI355X: 2.0 GHz x 4 transfers x 8192 bits / 8 = 8,192 GB/s (published: 8.0 TB/s)
    assert p.hbm_peak_gbps == pytest.approx(8192.0)
    assert abs(p.hbm_peak_gbps / r.HBM_PEAK_PUBLISHED_GBPS - 1) < 0.03
    # HIP's major / minor of the gfx architecture (gfx950 -> 9.5, gfx942 -> 9.4, gfx90a -> 9.0)
    assert p.capability == (9, 5)
    assert dataclasses.replace(p, arch="gfx942").capability == (9, 4)
    assert dataclasses.replace(p, arch="gfx90a").capability == (9, 0)
    assert dataclasses.replace(p, arch="gfx1100").capability == (11, 0)
