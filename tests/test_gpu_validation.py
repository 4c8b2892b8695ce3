"""Caller-supplied tensors are checked before their pointers reach a kernel:
a host tensor, a wrong shape or dtype, or a short stream raises ValueError
and nothing is launched (each case here fails in the Python layer)."""

from __future__ import annotations

import dataclasses

import pytest
import torch

from gpu_helpers import bf16_tensor, normal_case, to_device
from oracle import se12_codec as o

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def small(gpu):
    from se12_amd.hip import Se12MatVecKernel

    bits, enc = normal_case(64, 512, seed=31)
    dt = to_device(enc, gpu)
    return Se12MatVecKernel(dt), dt


def test_host_and_misshapen_outputs_are_refused(gpu, small):
    from se12_amd import hip

    k, dt = small
    x = bf16_tensor(o.normal_bf16(2, 512, seed=1, std=1.0), gpu)
    cases = [
        lambda: k.multiply(x, out=torch.empty((2, 64), dtype=torch.float32)),
        lambda: k.multiply(x, out=torch.empty((2, 63), dtype=torch.float32, device=gpu)),
        lambda: k.multiply(x, out=torch.empty((2, 64), dtype=torch.bfloat16, device=gpu)),
        lambda: k.multiply(x, out=torch.empty((64, 2), dtype=torch.float32, device=gpu).t()),
        lambda: k.multiply(x.cpu()),
        lambda: k.multiply_rowss(x, torch.empty((2, 4), dtype=torch.float32)),
        lambda: k.multiply_rowss(x, torch.empty((2, 4), dtype=torch.float32, device=gpu),
                                 y=torch.empty((2, 64), dtype=torch.float32)),
        lambda: k.decode_into(torch.empty((64, 512), dtype=torch.bfloat16)),
        lambda: k.decode_rows_into(torch.tensor([0, 1]), torch.empty((2, 512), dtype=torch.bfloat16, device=gpu)),
        lambda: k.decode_rows_into(torch.tensor([0, 1], device=gpu), torch.empty((2, 512), dtype=torch.bfloat16)),
        lambda: hip.multiply_grouped([k, k], x, outs=[torch.empty((2, 64), dtype=torch.float32, device=gpu),
                                                       torch.empty((2, 64), dtype=torch.float32)]),
        lambda: hip.multiply_grouped([k], x, outs=[]),
    ]
    for i, case in enumerate(cases):
        with pytest.raises(ValueError):
            case()
        torch.cuda.synchronize()


def test_host_tensors_for_the_fused_heads_and_tails_are_refused(gpu):
    from se12_amd import hip

    bits, enc = normal_case(512, 512, seed=32)
    k = hip.Se12MatVecKernel(to_device(enc, gpu))
    b, n = 1, 512
    ok = dict(y_prev=torch.zeros((b, n), dtype=torch.float32, device=gpu),
              w1=torch.zeros(n, dtype=torch.bfloat16, device=gpu), w2=torch.zeros(n, dtype=torch.bfloat16, device=gpu),
              residual_in=torch.zeros((b, n), dtype=torch.bfloat16, device=gpu),
              residual_out=torch.zeros((b, n), dtype=torch.bfloat16, device=gpu),
              h_out=torch.zeros((b, n), dtype=torch.bfloat16, device=gpu))
    for name in ok:
        args = dict(ok)
        args[name] = args[name].cpu()
        with pytest.raises(ValueError, match=name):
            hip.multiply_prenorm([k], eps=1e-6, **args)
    x = torch.zeros((b, n), dtype=torch.bfloat16, device=gpu)
    with pytest.raises(ValueError):
        k.multiply_rmsnorm(x, ok["w1"], ok["w2"], ok["residual_in"], ok["h_out"].cpu(), 1e-6)
    with pytest.raises(ValueError):
        hip.multiply_gelu_mul(k, k, x, torch.zeros((b, n), dtype=torch.bfloat16))


def test_short_or_host_streams_are_refused_before_bind(gpu, small):
    from se12_amd.hip import Se12MatVecKernel

    _, dt = small
    bad = [
        dataclasses.replace(dt, sm=dt.sm[:-16]),
        dataclasses.replace(dt, ec=dt.ec[:-1]),
        dataclasses.replace(dt, esc=dt.esc.cpu()),
        dataclasses.replace(dt, fallback_bitmap=dt.fallback_bitmap.to(torch.int8)),
        dataclasses.replace(dt, fallback_raw=torch.zeros(100, dtype=torch.int16, device=gpu)),
        dataclasses.replace(dt, codebook=dt.codebook[:14]),
        dataclasses.replace(dt, codebook_host=tuple(reversed(dt.codebook_host))),
        dataclasses.replace(dt, rows=dt.rows + 16),
    ]
    for t in bad:
        with pytest.raises(ValueError):
            Se12MatVecKernel(t)
