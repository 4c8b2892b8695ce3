"""The adapters built with the reference's positional constructor arguments
(lws/adapters/cuda/gemv.py:146,183; lws/adapters/cuda/se12_decoder.py:48) on
the GPU: a compile target from the device, the ahead-of-time compiler,
multiply with no launch, with this kernel's configuration and with every
candidate the reference's tuner would time (its own launch semantics), each
within REL_TOL of the oracle, fused and raw twin bit-identical under each;
the decoder's decode / decode_rows / decode_to_device bit-exact."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gpu_helpers import REL_TOL, bf16_tensor, heavy_tailed_bf16, max_rel_error, normal_case
from oracle import se12_codec as o
from se12_amd.format import make_se12_tensor
from test_adapters_cpu import ref_candidates, ref_default

pytestmark = pytest.mark.gpu


def _host_tensor(enc):
    rows, cols = enc["shape"]
    return make_se12_tensor(enc["sm"], enc["ec"], enc["esc"], enc["fallback_bitmap"], enc["fallback_raw"],
                            enc["codebook"], rows, cols)


def _setup(gpu):
    from se12_amd.compiler import AotKernelCompiler, device_compile_target
    from se12_amd.hip import HipGpuProbe

    compiler = AotKernelCompiler()
    target = device_compile_target(gpu.index)
    sm_count = HipGpuProbe(gpu.index).facts().compute_units
    return compiler, target, sm_count


@pytest.mark.parametrize("batch", [1, 4, 5, 16])
def test_reference_constructed_kernels_multiply(gpu, batch):
    from se12_amd.adapters import RawBf16MatVecKernel, Se12MatVecKernel
    from se12_amd.launch import configuration

    compiler, target, sm_count = _setup(gpu)
    rows, cols = 448, 2304
    bits, enc = normal_case(rows, cols, seed=21)
    fused = Se12MatVecKernel(compiler, target, _host_tensor(enc), sm_count)
    raw = RawBf16MatVecKernel(compiler, target, bf16_tensor(bits, gpu), sm_count)
    xb = o.normal_bf16(batch, cols, seed=22 + batch, std=1.0)
    ref = o.gemv_reference(enc, o.bf16_bits_to_f32(xb))
    for x in (bf16_tensor(xb, gpu), bf16_tensor(xb, gpu).float()):   # the reference passes FP32 activations
        launches = [None] + ref_candidates(rows, batch) + [ref_default(sm_count, rows, batch)]
        if batch < 5 or x.dtype == torch.float32:
            launches.append(configuration(2, 3, rows, batch, x.dtype == torch.float32))
        for launch in launches:
            yf = fused.multiply(x, launch)
            yr = raw.multiply(x, launch)
            torch.cuda.synchronize()
            assert max_rel_error(yf, ref) <= REL_TOL, (launch, x.dtype)
            assert torch.equal(yf, yr), (launch, x.dtype)


def test_sm_count_feeds_the_default_launch(gpu):
    from se12_amd.adapters import Se12MatVecKernel

    compiler, target, sm_count = _setup(gpu)
    # 2304x2304 (144 x 9 tiles): one wave per K tile on 256 CUs, 6 waves
    # when 8 CUs share 1,296 tiles
    bits, enc = normal_case(2304, 2304, seed=3)
    host = _host_tensor(enc)
    full = Se12MatVecKernel(compiler, target, host, sm_count)
    small = Se12MatVecKernel(compiler, target, full.tensor, 8)
    assert full.default_launch(1) != small.default_launch(1)
    xb = o.normal_bf16(1, 2304, seed=4, std=1.0)
    ref = o.gemv_reference(enc, o.bf16_bits_to_f32(xb))
    assert max_rel_error(small.multiply(bf16_tensor(xb, gpu)), ref) <= REL_TOL


def test_reference_constructed_decoder(gpu):
    from se12_amd.adapters import Se12WeightDecoder
    from se12_amd.hip import RowIndices

    compiler, target, _ = _setup(gpu)
    dec = Se12WeightDecoder(compiler, target)
    rows, cols = 64, 512
    bits = heavy_tailed_bf16(rows, cols, seed=7)
    host = _host_tensor(o.encode(bits.reshape(-1), rows, cols))
    assert np.array_equal(dec.decode(host).bit_pattern, bits.reshape(-1))
    assert np.array_equal(dec.decode_to_device(host).view(torch.int16).cpu().numpy(), bits)
    order = (63, 0, 17, 17, 40)
    got = dec.decode_rows(host, RowIndices(order)).bit_pattern.reshape(len(order), cols)
    assert np.array_equal(got, bits[list(order)])
