"""The roofline model (se12_amd/roofline.py) against closed forms: the
reference's known answers (tests/test_spec_performance_model.py:30-121,
restated with their numbers), the exact SE12 byte count per shape, and the
crossing of ratio 1 as the decode cost grows."""

from __future__ import annotations

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
    cal = r.Calibration(bandwidth_gbps=r.STREAM_READ_GBPS, raw_cost_us_per_weight=1e-12, se12_cost_us_per_weight=1e-12)
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
    # down_proj: 31,961,751 algorithmic bytes at 6.5 TB/s + one launch
    assert r.launch_floor_us(2304, 9216) == pytest.approx(1.7 + 31961751 / 6.5e6)
    a = r.achieved(31961751, 10.0)
    assert a["achieved"] == pytest.approx(3196.1751) and a["frac"] == pytest.approx(3196.1751 / 8000.0)
