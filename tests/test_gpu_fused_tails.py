"""Products with a decode-step tail (se12_gemv_gelu_mul, se12_gemv_rmsnorm)
or head (se12_gemv_prenorm) against the same product with the separate step
kernel (se12_step_gelu_mul, se12_step_rmsnorm mode 1):

- the FP32 products are bit-identical (same kernel, same launch shape);
- the MLP gate is element-wise with the same arithmetic: bit-identical;
- the norm's sum of squares runs over the GEMV block's threads instead of
  the norm kernel's, so its FP32 sum may round differently, and a one-ulp
  change of a normalised value can move the BF16 residual sum further where
  it cancels: residual and output bit-identical on >= 99% of elements and
  within 2^-7 of the row's largest magnitude everywhere;
- both stay right over repeated calls and graph replays (their arrival
  counters reset themselves), for the SE12 kernel and the raw twin, FAST and
  edge-handling variants, batch rows split over several dot2 launches, and
  where the step runs as its own kernel (MFMA batches, rows % 4 != 0)."""

from __future__ import annotations

import pytest
import torch

from gpu_helpers import to_device
from oracle import se12_codec as o
from se12_amd import _native as nat

pytestmark = pytest.mark.gpu


def _gen(gpu, seed):
    g = torch.Generator(device=gpu)
    g.manual_seed(seed)
    return g


def _norm_close(got: torch.Tensor, want: torch.Tensor, min_exact: float = 0.99) -> None:
    assert got.dtype == torch.bfloat16 and want.dtype == torch.bfloat16 and got.shape == want.shape
    same = got.view(torch.int16) == want.view(torch.int16)
    assert same.float().mean().item() >= min_exact
    err = (got.float() - want.float()).abs().amax(dim=1)
    scale = want.float().abs().amax(dim=1)
    assert bool((err <= scale * 2.0 ** -7).all()), (err, scale)


def _kernel(rows, cols, seed, fmt, gpu):
    from se12_amd.hip import RawBf16MatVecKernel, Se12MatVecKernel

    bits = o.normal_bf16(rows, cols, seed=seed, std=0.02)
    if fmt == "raw":
        return RawBf16MatVecKernel(torch.from_numpy(bits).to(gpu).view(torch.bfloat16), max_batch=8)
    enc = o.encode(bits.reshape(-1), rows, cols)
    return Se12MatVecKernel(to_device(enc, gpu), max_batch=8)


def _x(batch, cols, gpu, seed, dtype=torch.bfloat16):
    return torch.randn((batch, cols), generator=_gen(gpu, seed), device=gpu).to(dtype)


@pytest.mark.parametrize("fmt", ["se12", "raw"])
@pytest.mark.parametrize("rows,cols,batch,dtype", [
    (512, 768, 1, torch.bfloat16),      # FAST, one launch
    (9216, 2304, 1, torch.bfloat16),    # Gemma-2-2B gate / up
    (200, 300, 3, torch.bfloat16),      # edge-handling variant, ragged rows
    (256, 512, 6, torch.float32),       # FP32 x: two dot2 launches (4 + 2 rows)
    (384, 512, 8, torch.bfloat16),      # MFMA product, then the separate kernel
])
def test_gelu_mul_tail_equals_the_separate_kernel(gpu, fmt, rows, cols, batch, dtype):
    from se12_amd.hip import multiply_gelu_mul, multiply_grouped

    gate, up = _kernel(rows, cols, 1, fmt, gpu), _kernel(rows, cols, 2, fmt, gpu)
    x = _x(batch, cols, gpu, 3, dtype)
    want_y = multiply_grouped([gate, up], x)
    want = torch.empty((batch, rows), dtype=torch.bfloat16, device=gpu)
    nat.step_check(nat.lib().se12_step_gelu_mul(nat.ptr(want_y[0]), nat.ptr(want_y[1]), nat.STEP_F32, rows,
                                                nat.ptr(want), batch, rows, nat.stream_ptr()))
    for call in range(3):  # the pair counters reset themselves
        out = torch.full((batch, rows), float("nan"), dtype=torch.bfloat16, device=gpu)
        ys = multiply_gelu_mul(gate, up, x, out)
        torch.cuda.synchronize()
        assert torch.equal(ys[0], want_y[0]) and torch.equal(ys[1], want_y[1]), call
        assert torch.equal(out.view(torch.int16), want.view(torch.int16)), call


def _norm_inputs(batch, rows, gpu, seed):
    g = _gen(gpu, seed)
    w1 = (torch.randn(rows, generator=g, device=gpu) * 0.1).to(torch.bfloat16)
    w2 = (torch.randn(rows, generator=g, device=gpu) * 0.1).to(torch.bfloat16)
    res = torch.randn((batch, rows), generator=g, device=gpu).to(torch.bfloat16)
    return w1, w2, res


def _separate_norm(y, w1, w2, res, eps):
    batch, rows = y.shape
    res = res.clone()
    out = torch.empty_like(res)
    nat.step_check(nat.lib().se12_step_rmsnorm(nat.ptr(y), nat.STEP_F32, rows, nat.ptr(w1), nat.ptr(res), nat.ptr(w2),
                                               nat.ptr(out), batch, rows, eps, 0.0, 1, nat.stream_ptr()))
    return res, out


@pytest.mark.parametrize("fmt", ["se12", "raw"])
@pytest.mark.parametrize("rows,cols,batch,dtype", [
    (2304, 9216, 1, torch.bfloat16),    # Gemma-2-2B down_proj
    (2304, 2048, 1, torch.bfloat16),    # Gemma-2-2B o_proj
    (100, 256, 2, torch.bfloat16),      # one K tile: no split-K
    (300, 700, 3, torch.bfloat16),      # edge-handling variant, ragged rows
    (298, 512, 1, torch.bfloat16),      # rows % 4 != 0: separate kernel
    (256, 1024, 5, torch.float32),      # FP32 x: two dot2 launches (4 + 1 rows)
    (512, 512, 8, torch.bfloat16),      # MFMA product, then the separate kernel
    (8192, 256, 1, torch.bfloat16),     # 80 KiB of LDS for the tail (gfx950 blocks may take 160 KiB)
])
def test_rmsnorm_tail_matches_the_separate_kernel(gpu, fmt, rows, cols, batch, dtype):
    k = _kernel(rows, cols, 5, fmt, gpu)
    x = _x(batch, cols, gpu, 6, dtype)
    w1, w2, res0 = _norm_inputs(batch, rows, gpu, 7)
    eps = 1e-6
    want_y = k.multiply(x)
    want_res, want_out = _separate_norm(want_y, w1, w2, res0, eps)
    res = res0.clone()
    for call in range(3):  # the matrix counter resets itself; the residual accumulates
        out = torch.full((batch, rows), float("nan"), dtype=torch.bfloat16, device=gpu)
        y = k.multiply_rmsnorm(x, w1, w2, res, out, eps)
        torch.cuda.synchronize()
        assert torch.equal(y, want_y), call
        _norm_close(res, want_res)
        _norm_close(out, want_out)
        if call < 2:
            want_res, want_out = _separate_norm(want_y, w1, w2, res, eps)


def test_tails_replay_in_a_graph(gpu):
    """Five replays of a captured gate/up + down product pair with their tails,
    each checked against eager calls on the same inputs."""
    from se12_amd.hip import multiply_gelu_mul

    gate, up = _kernel(1024, 512, 11, "se12", gpu), _kernel(1024, 512, 12, "se12", gpu)
    down = _kernel(512, 1024, 13, "se12", gpu)
    x = _x(1, 512, gpu, 14)
    w1, w2, res0 = _norm_inputs(1, 512, gpu, 15)
    m = torch.empty((1, 1024), dtype=torch.bfloat16, device=gpu)
    gu = [torch.empty((1, 1024), dtype=torch.float32, device=gpu) for _ in range(2)]
    yd = torch.empty((1, 512), dtype=torch.float32, device=gpu)
    res = res0.clone()
    h = torch.empty((1, 512), dtype=torch.bfloat16, device=gpu)

    def step():
        multiply_gelu_mul(gate, up, x, m, ys=gu)
        down.multiply_rmsnorm(m, w1, w2, res, h, 1e-6, y=yd)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    torch.cuda.synchronize()
    for rep in range(5):
        res.copy_(res0)
        g.replay()
        torch.cuda.synchronize()
        got = (m.clone(), res.clone(), h.clone())
        res.copy_(res0)
        step()
        torch.cuda.synchronize()
        assert torch.equal(got[0], m) and torch.equal(got[1], res) and torch.equal(got[2], h), rep


def test_tail_arguments_are_checked(gpu):
    from se12_amd.hip import multiply_gelu_mul

    gate, up = _kernel(256, 512, 1, "se12", gpu), _kernel(128, 512, 2, "se12", gpu)
    x = _x(1, 512, gpu, 3)
    with pytest.raises(ValueError):
        multiply_gelu_mul(gate, up, x, torch.empty((1, 256), dtype=torch.bfloat16, device=gpu))
    k = _kernel(256, 512, 4, "se12", gpu)
    w1, w2, res = _norm_inputs(1, 256, gpu, 5)
    with pytest.raises(ValueError):
        k.multiply_rmsnorm(x, w1[:128], w2, res, torch.empty_like(res), 1e-6)


def _prenorm_case(gpu, kernels, batch, seed, same_residual=False, launch=None):
    from se12_amd.hip import multiply_grouped, multiply_prenorm

    K = kernels[0].cols
    g = _gen(gpu, seed)
    y_prev = torch.randn((batch, K), generator=g, device=gpu) * 3.0
    w1, w2, res0 = _norm_inputs(batch, K, gpu, seed + 1)
    eps = 1e-6
    want_res, want_h = _separate_norm(y_prev, w1, w2, res0, eps)
    res_in = res0.clone()
    res_out = res_in if same_residual else torch.full_like(res0, float("nan"))
    h = torch.full_like(res0, float("nan"))
    ys = multiply_prenorm(kernels, y_prev, w1, w2, res_in, res_out, h, eps, launch=launch)
    torch.cuda.synchronize()
    _norm_close(res_out, want_res)
    _norm_close(h, want_h)
    if not same_residual:
        assert torch.equal(res_in, res0)
    # the products are those of the h the launch wrote: bit for bit under one
    # launch shape; the default launches of the two calls may differ (a head
    # launch can take one wave fewer), which only reorders the FP32 K sums
    for got, want in zip(ys, multiply_grouped(kernels, h, launch=launch)):
        if launch is None:
            torch.testing.assert_close(got, want, rtol=1e-5, atol=1e-5)
        else:
            assert torch.equal(got, want)
    return ys, h


@pytest.mark.parametrize("fmt", ["se12", "raw"])
@pytest.mark.parametrize("batch", [1, 2, 4])
def test_prenorm_qkv_shapes(gpu, fmt, batch):
    """Gemma-2-2B q/k/v (2048/1024/1024 x 2304) from the previous down_proj output."""
    kernels = [_kernel(2048, 2304, 21, fmt, gpu), _kernel(1024, 2304, 22, fmt, gpu), _kernel(1024, 2304, 23, fmt, gpu)]
    for call in range(2):
        _prenorm_case(gpu, kernels, batch, 30 + call)


@pytest.mark.parametrize("fmt", ["se12", "raw"])
def test_prenorm_gate_up_with_the_mlp_gate(gpu, fmt):
    from se12_amd.hip import multiply_prenorm

    gate, up = _kernel(9216, 2304, 24, fmt, gpu), _kernel(9216, 2304, 25, fmt, gpu)
    ys, h = _prenorm_case(gpu, [gate, up], 1, 40)
    g = _gen(gpu, 40)
    y_prev = torch.randn((1, 2304), generator=g, device=gpu) * 3.0
    w1, w2, res0 = _norm_inputs(1, 2304, gpu, 41)
    m = torch.empty((1, 9216), dtype=torch.bfloat16, device=gpu)
    res_out, h = torch.empty_like(res0), torch.empty_like(res0)
    ys = multiply_prenorm([gate, up], y_prev, w1, w2, res0, res_out, h, 1e-6, gelu_out=m)
    want = torch.empty_like(m)
    nat.step_check(nat.lib().se12_step_gelu_mul(nat.ptr(ys[0]), nat.ptr(ys[1]), nat.STEP_F32, 9216, nat.ptr(want), 1,
                                                9216, nat.stream_ptr()))
    torch.cuda.synchronize()
    assert torch.equal(m, want)


@pytest.mark.parametrize("rows,cols,batch,same,waves", [
    (512, 2304, 1, True, None),    # one residual tensor: the norm runs as its own kernel
    (256, 1024, 6, False, None),   # MFMA product
    (200, 700, 2, False, None),    # edge-handling product
    (512, 2304, 1, False, 1),      # one wave per block
    (64, 8192, 1, False, None),    # the longest row the norm takes
    (64, 8192, 4, False, None),    # 4 rows of 8192: more than a block's LDS, separate kernel
])
def test_prenorm_separate_kernel_paths(gpu, rows, cols, batch, same, waves):
    from se12_amd.launch import configuration

    k = _kernel(rows, cols, 50, "se12", gpu)
    launch = None if waves is None else configuration(waves, 1, rows, batch)
    _prenorm_case(gpu, [k], batch, 51, same_residual=same, launch=launch)


def test_prenorm_replays_in_a_graph(gpu):
    """Ping-pong residuals over two products (q/k/v then gate/up), captured
    once and replayed five times against eager calls."""
    from se12_amd.hip import multiply_prenorm

    qkv = [_kernel(512, 1024, 61, "se12", gpu), _kernel(256, 1024, 62, "se12", gpu)]
    gu = [_kernel(2048, 1024, 63, "se12", gpu), _kernel(2048, 1024, 64, "se12", gpu)]
    g = _gen(gpu, 65)
    y1 = torch.randn((1, 1024), generator=g, device=gpu)
    y2 = torch.randn((1, 1024), generator=g, device=gpu)
    w = [(torch.randn(1024, generator=g, device=gpu) * 0.1).to(torch.bfloat16) for _ in range(4)]
    r0 = torch.randn((1, 1024), generator=g, device=gpu).to(torch.bfloat16)
    ra, rb, h = r0.clone(), torch.empty_like(r0), torch.empty_like(r0)
    m = torch.empty((1, 2048), dtype=torch.bfloat16, device=gpu)
    outs = [[torch.empty((1, k.rows), device=gpu) for k in ks] for ks in (qkv, gu)]

    def step():
        multiply_prenorm(qkv, y1, w[0], w[1], ra, rb, h, 1e-6, ys=outs[0])
        multiply_prenorm(gu, y2, w[2], w[3], rb, ra, h, 1e-6, ys=outs[1], gelu_out=m)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()
    torch.cuda.current_stream().wait_stream(s)
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr):
        step()
    torch.cuda.synchronize()
    for rep in range(5):
        ra.copy_(r0)
        gr.replay()
        torch.cuda.synchronize()
        got = [t.clone() for t in (ra, rb, h, m, *outs[0], *outs[1])]
        ra.copy_(r0)
        step()
        torch.cuda.synchronize()
        for a, b in zip(got, (ra, rb, h, m, *outs[0], *outs[1])):
            assert torch.equal(a, b), rep


def _want_row_ss(y: torch.Tensor) -> torch.Tensor:
    b, n = y.shape
    tr = (n + 15) // 16
    t = torch.zeros((b, tr * 16), dtype=torch.float32, device=y.device)
    t[:, :n] = y.to(torch.bfloat16).float() ** 2
    return t.view(b, tr, 16).sum(-1)


@pytest.mark.parametrize("fmt", ["se12", "raw"])
@pytest.mark.parametrize("rows,cols,batch,dtype", [
    (2304, 2048, 1, torch.bfloat16),    # Gemma-2-2B o_proj
    (2304, 9216, 1, torch.bfloat16),    # down_proj, split-K
    (2304, 9216, 4, torch.bfloat16),
    (300, 512, 3, torch.bfloat16),      # a partial last tile row
    (256, 1024, 6, torch.bfloat16),     # MFMA product, row sums after it
    (512, 768, 2, torch.float32),       # FP32 x
])
def test_rowss_sums_the_tile_rows_of_the_output(gpu, fmt, rows, cols, batch, dtype):
    k = _kernel(rows, cols, 70, fmt, gpu)
    tr = (rows + 15) // 16
    for call in range(2):
        x = _x(batch, cols, gpu, 71 + call, dtype)
        ss = torch.full((batch, tr), float("nan"), device=gpu)
        y = k.multiply_rowss(x, ss)
        torch.cuda.synchronize()
        assert torch.equal(y, k.multiply(x))
        torch.testing.assert_close(ss, _want_row_ss(y), rtol=1e-5, atol=1e-30)


@pytest.mark.parametrize("batch", [1, 2, 4])
@pytest.mark.parametrize("consumer_rows", [(2048, 1024, 1024), (9216, 9216)])
def test_prenorm_from_producer_row_sums(gpu, batch, consumer_rows):
    """The norm's first mean from the producer's row sums gives the norm of
    the separate step kernels (Gemma-2-2B o_proj -> gate/up, down -> q/k/v)."""
    from se12_amd.hip import multiply_grouped, multiply_prenorm

    producer = _kernel(2304, 2048, 80, "se12", gpu)
    kernels = [_kernel(r, 2304, 81 + i, "se12", gpu) for i, r in enumerate(consumer_rows)]
    x = _x(batch, 2048, gpu, 85)
    ss = torch.empty((batch, 144), device=gpu)
    y_prev = producer.multiply_rowss(x, ss)
    w1, w2, res0 = _norm_inputs(batch, 2304, gpu, 86)
    want_res, want_h = _separate_norm(y_prev, w1, w2, res0, 1e-6)
    res_out, h = torch.full_like(res0, float("nan")), torch.full_like(res0, float("nan"))
    ys = multiply_prenorm(kernels, y_prev, w1, w2, res0, res_out, h, 1e-6, y_prev_ss=ss)
    torch.cuda.synchronize()
    _norm_close(res_out, want_res)
    _norm_close(h, want_h)
    for got, want in zip(ys, multiply_grouped(kernels, h)):
        torch.testing.assert_close(got, want, rtol=1e-5, atol=1e-5)


def test_row_sums_replay_in_a_graph(gpu):
    """o_proj with row sums, then gate/up with the norm from them, captured
    once and replayed five times against eager calls."""
    from se12_amd.hip import multiply_prenorm

    o_k = _kernel(1024, 512, 90, "se12", gpu)
    gu = [_kernel(2048, 1024, 91, "se12", gpu), _kernel(2048, 1024, 92, "se12", gpu)]
    g = _gen(gpu, 93)
    x = torch.randn((1, 512), generator=g, device=gpu).to(torch.bfloat16)
    w = [(torch.randn(1024, generator=g, device=gpu) * 0.1).to(torch.bfloat16) for _ in range(2)]
    r0 = torch.randn((1, 1024), generator=g, device=gpu).to(torch.bfloat16)
    ra, rb, h = r0.clone(), torch.empty_like(r0), torch.empty_like(r0)
    y_o, ss = torch.empty((1, 1024), device=gpu), torch.empty((1, 64), device=gpu)
    m = torch.empty((1, 2048), dtype=torch.bfloat16, device=gpu)
    outs = [torch.empty((1, 2048), device=gpu) for _ in gu]

    def step():
        o_k.multiply_rowss(x, ss, y=y_o)
        multiply_prenorm(gu, y_o, w[0], w[1], ra, rb, h, 1e-6, ys=outs, gelu_out=m, y_prev_ss=ss)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()
    torch.cuda.current_stream().wait_stream(s)
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr):
        step()
    torch.cuda.synchronize()
    for rep in range(5):
        ss.fill_(float("nan"))
        gr.replay()
        torch.cuda.synchronize()
        got = [t.clone() for t in (ss, y_o, rb, h, m, *outs)]
        ss.fill_(float("nan"))
        step()
        torch.cuda.synchronize()
        for a, b in zip(got, (ss, y_o, rb, h, m, *outs)):
            assert torch.equal(a, b), rep


def test_row_sum_arguments_are_checked(gpu):
    from se12_amd.hip import multiply_prenorm

    k = _kernel(256, 512, 95, "se12", gpu)
    x = _x(2, 512, gpu, 96)
    with pytest.raises(ValueError):
        k.multiply_rowss(x, torch.empty((2, 15), device=gpu))
    with pytest.raises(ValueError):
        k.multiply_rowss(x, torch.empty((2, 16), device=gpu, dtype=torch.float64))
    c = _kernel(128, 256, 97, "se12", gpu)
    y = torch.randn((1, 256), device=gpu)
    w1, w2, r = _norm_inputs(1, 256, gpu, 98)
    with pytest.raises(ValueError):
        multiply_prenorm([c], y, w1, w2, r, torch.empty_like(r), torch.empty_like(r), 1e-6,
                         y_prev_ss=torch.empty((1, 15), device=gpu))
