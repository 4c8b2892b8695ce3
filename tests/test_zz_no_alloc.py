"""se12_gemv_noalloc through the C ABI: the product with the library's
static per-GPU scratch gives exactly what se12_gemv gives on the same handle
and launch (split-K partial sums and arrival counters in use, dot2 and MFMA
kernels), on two calls in a row of which the second has a smaller input,
and within REL_TOL of the oracle; shapes and launches beyond the scratch are
refused before any launch."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from gpu_helpers import REL_TOL, bf16_tensor, max_rel_error, normal_case, to_device
from oracle import se12_codec as o
from se12_amd import _native as nat

pytestmark = pytest.mark.gpu


def _call(fn, kern, x, y, launch):
    xd = nat.X_BF16 if x.dtype == torch.bfloat16 else nat.X_F32
    lc = None if launch is None else ctypes.byref(nat.Launch(launch.threads_per_block.value, launch.blocks.value))
    return fn(kern.handle.raw, nat.ptr(x), xd, x.shape[0], nat.ptr(y), lc, nat.stream_ptr())


def _both(kern, x, launch):
    lib = nat.lib()
    y_ref = torch.full((x.shape[0], kern.rows), float("nan"), dtype=torch.float32, device=x.device)
    y_na = torch.full_like(y_ref, float("nan"))
    nat.check(_call(lib.se12_gemv, kern, x, y_ref, launch))
    nat.check(_call(lib.se12_gemv_noalloc, kern, x, y_na, launch))
    torch.cuda.synchronize()
    return y_ref, y_na


def test_noalloc_equals_the_allocating_product_twice_in_a_row(gpu):
    from se12_amd.hip import Se12MatVecKernel
    from se12_amd.launch import configuration, rx_configuration, rx_layout, uses_rx

    assert rx_layout(4608, 9216, 16) == (16, 2) and not uses_rx(1040, 9216, 9) and uses_rx(1040, 2304, 9)
    assert rx_layout(1040, 9216, 24) == (24, 3)
    big_bits, big_enc = normal_case(4608, 9216, seed=41)
    small_bits, small_enc = normal_case(1040, 2304, seed=42)
    long_bits, long_enc = normal_case(1040, 9216, seed=43)
    big = Se12MatVecKernel(to_device(big_enc, gpu))
    small = Se12MatVecKernel(to_device(small_enc, gpu))
    long = Se12MatVecKernel(to_device(long_enc, gpu))
    cases = [
        (big, big_enc, 4, configuration(4, 9, 4608, 4)),       # dot2, 9 K splits over 4 batch rows
        (small, small_enc, 2, configuration(3, 3, 1040, 2)),   # a smaller input after it
        (big, big_enc, 16, rx_configuration(8, 128, splits=2)),  # resident-x (x over a block's LDS), 2 K splits
        (long, long_enc, 9, configuration(2, 3, 1040, 9)),     # smaller again, x-slab MFMA, 3 K splits
        (long, long_enc, 24, rx_configuration(8, 32, splits=3)),  # resident-x kernel, 3 K splits
        (small, small_enc, 9, rx_configuration(4, 7)),         # resident-x kernel (no split-K scratch)
        (small, small_enc, 1, None),                            # the default launch
        (big, big_enc, 1, None),
    ]
    for i, (kern, enc, batch, launch) in enumerate(cases):
        xb = o.normal_bf16(batch, kern.cols, seed=50 + i, std=1.0)
        x = bf16_tensor(xb, gpu)
        y_ref, y_na = _both(kern, x, launch)
        assert torch.equal(y_na, y_ref), (i, batch, launch)
        assert max_rel_error(y_na, o.gemv_reference(enc, o.bf16_bits_to_f32(xb))) <= REL_TOL, i
    # FP32 activations (the dot2 kernel, several launches of 4 rows) through the Python wrapper
    xf = torch.randn((6, small.cols), device=gpu)
    out = torch.empty((6, small.rows), dtype=torch.float32, device=gpu)
    launch = configuration(3, 9, small.rows, 6, float32_activations=True)
    small.multiply_noalloc(xf, out, launch=launch)
    assert torch.equal(out, small.multiply(xf, launch=launch))


def test_noalloc_refuses_what_the_scratch_cannot_hold(gpu):
    from se12_amd.hip import Se12MatVecKernel, encode_on_device
    from se12_amd.launch import configuration

    lib = nat.lib()
    # dot2: 35 pair slots x 4 batch rows x 16384 rows = 2,293,760 > 262,144
    w = torch.randn((16384, 9216), device=gpu).mul_(0.02).to(torch.bfloat16)
    kern = Se12MatVecKernel(encode_on_device(w), max_batch=32)
    del w
    x = torch.randn((4, 9216), device=gpu).to(torch.bfloat16)
    y = torch.zeros((4, 16384), dtype=torch.float32, device=gpu)
    rc = _call(lib.se12_gemv_noalloc, kern, x, y, configuration(4, 36, 16384, 4))
    assert rc == nat.SE12_E_CAPACITY and "pair slots" in nat.last_error()
    assert torch.count_nonzero(y).item() == 0           # nothing launched
    # MFMA (resident-x, 4 K splits): 4 x 32 batch rows x 16384 rows =
    # 2,097,152 partial sums > 1,507,328
    x32 = torch.randn((32, 9216), device=gpu).to(torch.bfloat16)
    y32 = torch.zeros((32, 16384), dtype=torch.float32, device=gpu)
    rc = _call(lib.se12_gemv_noalloc, kern, x32, y32, None)
    assert rc == nat.SE12_E_CAPACITY and "partial sums" in nat.last_error()
    assert torch.count_nonzero(y32).item() == 0
    # 32,768 tile rows need 65,537 arrival counters > 65,536
    w = torch.randn((32768 * 16, 256), device=gpu).mul_(0.02).to(torch.bfloat16)
    tall = Se12MatVecKernel(encode_on_device(w), max_batch=1)
    del w
    x1 = torch.randn((1, 256), device=gpu).to(torch.bfloat16)
    y1 = torch.zeros((1, 32768 * 16), dtype=torch.float32, device=gpu)
    rc = _call(lib.se12_gemv_noalloc, tall, x1, y1, None)
    assert rc == nat.SE12_E_CAPACITY and "arrival counters" in nat.last_error()
    assert torch.count_nonzero(y1).item() == 0
    # the same calls through se12_gemv still work (its workspace is the handle's)
    nat.check(_call(lib.se12_gemv, tall, x1, y1, None))
    torch.cuda.synchronize()
    assert torch.isfinite(y1).all()
