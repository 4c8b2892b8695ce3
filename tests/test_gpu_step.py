"""The decode-step kernels (include/se12_step.h) against the framework op
sequences they replace (the eager Gemma-2 step in se12_amd/gemma2.py), on
random inputs. Each framework BF16 op rounds its FP32 result to BF16; the
kernels do the same op by op, so results agree to the last BF16 bit except
where an FP32 sum runs in another order or a transcendental differs in its
last FP32 bit: the bar is at most one BF16 ulp on any element and at least
99% of elements bit-identical. Index work (argmax ids, the token slot, the
KV-cache slot, the counters) is exact."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from se12_amd import _native as nat
from se12_amd.gemma2 import rms_norm, rotate_half

pytestmark = pytest.mark.gpu


def _gen(gpu, seed):
    g = torch.Generator(device=gpu)
    g.manual_seed(seed)
    return g


def _ulp_close(got: torch.Tensor, want: torch.Tensor, min_exact: float = 0.99) -> None:
    """At most one BF16 ulp apart everywhere, bit-identical on `min_exact` of
    the elements."""
    assert got.dtype == torch.bfloat16 and want.dtype == torch.bfloat16 and got.shape == want.shape
    a = got.view(torch.int16).to(torch.int32)
    b = want.view(torch.int16).to(torch.int32)
    same = a == b
    # adjacent BF16 values of one sign differ by 1 in their bit pattern
    near = ((a - b).abs() <= 1) & ((a < 0) == (b < 0))
    assert bool((same | near).all()), f"{int((~(same | near)).sum())} elements more than one ulp apart"
    assert same.float().mean().item() >= min_exact


def _rmsnorm(x, w1, residual, w2, out, hidden, eps, in_scale, mode, in_stride=None):
    dtype = nat.STEP_F32 if x.dtype == torch.float32 else nat.STEP_BF16
    nat.step_check(nat.lib().se12_step_rmsnorm(
        nat.ptr(x), dtype, in_stride or x.shape[1], nat.ptr(w1), nat.ptr(residual), nat.ptr(w2), nat.ptr(out),
        out.shape[0], hidden, eps, in_scale, mode, nat.stream_ptr()))


@pytest.mark.parametrize("rows,hidden", [(1, 2304), (5, 256), (3, 100)])
def test_rmsnorm_mode0_scaled_embedding(gpu, rows, hidden):
    g = _gen(gpu, rows * 1000 + hidden)
    emb = (torch.randn((rows, hidden), generator=g, device=gpu) * 0.02).to(torch.bfloat16)
    w = (torch.randn(hidden, generator=g, device=gpu) * 0.1).to(torch.bfloat16)
    scale = torch.tensor(math.sqrt(hidden), dtype=torch.bfloat16, device=gpu)
    x = torch.empty_like(emb)
    h = torch.empty_like(emb)
    _rmsnorm(emb, w, x, None, h, hidden, 1e-6, float(scale.float().item()), 0)
    x_ref = emb * scale
    assert torch.equal(x, x_ref)
    _ulp_close(h, rms_norm(x_ref, w, 1e-6))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_rmsnorm_mode1_residual_and_next_norm(gpu, dtype):
    rows, hidden = 4, 2304
    g = _gen(gpu, 7)
    y = torch.randn((rows, hidden + 64), generator=g, device=gpu).to(dtype)[:, :hidden]   # strided input
    x0 = torch.randn((rows, hidden), generator=g, device=gpu).to(torch.bfloat16)
    w1 = (torch.randn(hidden, generator=g, device=gpu) * 0.1).to(torch.bfloat16)
    w2 = (torch.randn(hidden, generator=g, device=gpu) * 0.1).to(torch.bfloat16)
    x = x0.clone()
    h = torch.empty_like(x0)
    _rmsnorm(y, w1, x, w2, h, hidden, 1e-6, 0.0, 1, in_stride=hidden + 64)
    x_ref = x0 + rms_norm(y.to(torch.bfloat16), w1, 1e-6)
    _ulp_close(x, x_ref)
    _ulp_close(h, rms_norm(x, w2, 1e-6))     # the second norm of the kernel's own residual


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_gelu_mul(gpu, dtype):
    rows, cols, stride = 3, 9216, 2 * 9216
    g = _gen(gpu, 11)
    gu = (torch.randn((rows, stride), generator=g, device=gpu) * 2).to(dtype)
    out = torch.empty((rows, cols), dtype=torch.bfloat16, device=gpu)
    gate, up = gu[:, :cols], gu[:, cols:]
    d = nat.STEP_F32 if dtype == torch.float32 else nat.STEP_BF16
    nat.step_check(nat.lib().se12_step_gelu_mul(nat.ptr(gate), nat.ptr(up), d, stride, nat.ptr(out), rows, cols,
                                                nat.stream_ptr()))
    ref = F.gelu(gate.to(torch.bfloat16), approximate="tanh") * up.to(torch.bfloat16)
    _ulp_close(out, ref)


def _attention_ref(q, k, v, kt, vc, inv_freq, pos, heads, kvh, d, scaling, softcap, window):
    """The eager step's attention at one position (gemma2.Gemma2Decoder._step)."""
    B = q.shape[0]
    freqs = torch.tensor([float(pos)], device=q.device)[..., None] * inv_freq
    emb = torch.cat((freqs, freqs), dim=-1)
    cos, sin = emb.cos().to(torch.bfloat16), emb.sin().to(torch.bfloat16)
    q = q.to(torch.bfloat16).view(B, heads, d)
    k = k.to(torch.bfloat16).view(B, kvh, d)
    v = v.to(torch.bfloat16)
    q = q * cos + rotate_half(q) * sin
    k = k * cos + rotate_half(k) * sin
    L = kt.shape[-1]
    kt = kt.clone()
    vc = vc.clone()
    kt[:, :, :, pos] = k
    vc[:, :, pos, :] = v.view(B, kvh, d)
    j = torch.arange(L, device=q.device)
    allowed = j <= pos
    if window:
        allowed = allowed & (pos - j < window)
    g = heads // kvh
    sc = torch.matmul(q.view(B, kvh, g, d), kt) * scaling
    sc = torch.tanh(sc / softcap) * softcap
    sc = sc.masked_fill(~allowed, float("-inf"))
    p = F.softmax(sc.float(), dim=-1).to(torch.bfloat16)
    return torch.matmul(p, vc).reshape(B, heads * d), kt, vc


def _workspace(gpu, batch, heads, kvh, d, L):
    n = nat.lib().se12_step_attention_workspace(batch, heads, kvh, d, L)
    assert n > 0
    return torch.zeros(n, dtype=torch.uint8, device=gpu)


def _attention(q, k, v, dtype, q_stride, kv_stride, kt, vc, inv_freq, pos_t, out, batch, heads, kvh, d, L, scaling,
               softcap, window, ws):
    dd = nat.STEP_F32 if dtype == torch.float32 else nat.STEP_BF16
    nat.step_check(nat.lib().se12_step_attention(
        nat.ptr(q), nat.ptr(k), nat.ptr(v), dd, q_stride, kv_stride, nat.ptr(kt), nat.ptr(vc), nat.ptr(inv_freq),
        nat.ptr(pos_t), nat.ptr(out), batch, heads, kvh, d, L, scaling, softcap, window, nat.ptr(ws), ws.numel(),
        nat.stream_ptr()))


# (batch, heads, kv heads, head dim, cache length, position, window, input dtype): one chunk of 64 positions,
# several chunks, a window starting inside a chunk, a cache length off the chunk size, every query-group size
ATTN_CASES = [
    (1, 8, 4, 256, 64, 0, 0, torch.float32),
    (2, 8, 4, 256, 64, 37, 0, torch.float32),
    (3, 8, 4, 256, 128, 90, 16, torch.float32),
    (2, 8, 4, 256, 64, 63, 0, torch.bfloat16),
    (1, 8, 4, 256, 640, 575, 0, torch.float32),
    (2, 8, 4, 256, 160, 150, 100, torch.float32),
    (1, 8, 4, 256, 304, 128, 0, torch.bfloat16),
    (2, 4, 4, 128, 200, 199, 0, torch.float32),
    (1, 8, 2, 64, 256, 130, 0, torch.float32),
    (2, 16, 2, 128, 96, 70, 0, torch.float32),
    (1, 8, 4, 256, 1024, 1023, 0, torch.float32),
    (1, 8, 4, 256, 1024, 1000, 300, torch.bfloat16),
    (2, 8, 4, 256, 1280, 1100, 0, torch.float32),
    (1, 8, 4, 256, 1280, 1279, 512, torch.bfloat16),
    (1, 8, 8, 64, 1096, 777, 0, torch.float32),
    (1, 16, 2, 128, 600, 590, 0, torch.float32),        # 8 query heads per KV head over 3 spans
    (2, 16, 4, 64, 520, 519, 200, torch.bfloat16),      # 4 per KV head over 2 spans, windowed
]


@pytest.mark.parametrize("batch,heads,kvh,d,L,pos,window,dtype", ATTN_CASES)
def test_attention_step(gpu, batch, heads, kvh, d, L, pos, window, dtype):
    g = _gen(gpu, 100 + pos + L)
    q = torch.randn((batch, heads * d), generator=g, device=gpu).to(dtype)
    kv = torch.randn((batch, 2 * kvh * d), generator=g, device=gpu).to(dtype)   # k and v side by side
    k, v = kv[:, : kvh * d], kv[:, kvh * d:]
    kt = (torch.randn((batch, kvh, d, L), generator=g, device=gpu)).to(torch.bfloat16)
    vc = (torch.randn((batch, kvh, L, d), generator=g, device=gpu)).to(torch.bfloat16)
    inv_freq = 1.0 / (10000.0 ** (torch.arange(0, d, 2, dtype=torch.int64, device=gpu).float() / d))
    scaling, softcap = 256.0 ** -0.5, 50.0
    want, kt_ref, vc_ref = _attention_ref(q, k, v, kt, vc, inv_freq, pos, heads, kvh, d, scaling, softcap, window)
    out = torch.empty((batch, heads * d), dtype=torch.bfloat16, device=gpu)
    pos_t = torch.tensor(pos, dtype=torch.int64, device=gpu)
    ws = _workspace(gpu, batch, heads, kvh, d, L)
    _attention(q, k, v, dtype, heads * d, 2 * kvh * d, kt, vc, inv_freq, pos_t, out, batch, heads, kvh, d, L, scaling,
               softcap, window, ws)
    torch.cuda.synchronize()
    # the caches change only at `pos`, the value slot exactly
    assert torch.equal(vc, vc_ref)
    mask = torch.ones(L, dtype=torch.bool, device=gpu)
    mask[pos] = False
    assert torch.equal(kt[..., mask], kt_ref[..., mask])
    _ulp_close(kt[..., pos].contiguous(), kt_ref[..., pos].contiguous(), min_exact=0.98)
    diff = (out.float() - want.float()).abs()
    assert diff.max().item() <= 2 ** -7 * want.float().abs().max().item() + 1e-3
    assert (out == want).float().mean().item() >= 0.9
    # the arrival counters are back at zero: a second call on the same workspace gives the same result
    out2 = torch.empty_like(out)
    _attention(q, k, v, dtype, heads * d, 2 * kvh * d, kt, vc, inv_freq, pos_t, out2, batch, heads, kvh, d, L,
               scaling, softcap, window, ws)
    torch.cuda.synchronize()
    assert torch.equal(out, out2)


@pytest.mark.parametrize("L", [80, 1096])
def test_attention_position_outside_the_cache_touches_nothing(gpu, L):
    batch, heads, kvh, d = 1, 4, 2, 64
    q = torch.ones((batch, heads * d), device=gpu)
    k = torch.ones((batch, kvh * d), device=gpu)
    kt = torch.full((batch, kvh, d, L), 3.0, device=gpu).to(torch.bfloat16)
    vc = torch.full((batch, kvh, L, d), 5.0, device=gpu).to(torch.bfloat16)
    inv_freq = torch.ones(d // 2, device=gpu)
    out = torch.full((batch, heads * d), 7.0, device=gpu).to(torch.bfloat16)
    ws = _workspace(gpu, batch, heads, kvh, d, L)
    for p in (L, -1):
        pos_t = torch.tensor(p, dtype=torch.int64, device=gpu)
        _attention(q, k, k, torch.float32, heads * d, kvh * d, kt, vc, inv_freq, pos_t, out, batch, heads, kvh, d, L,
                   1.0, 0.0, 0, ws)
        torch.cuda.synchronize()
        assert bool((out == 0).all()) and bool((kt == 3).all()) and bool((vc == 5).all())
    assert bool((ws[:8] == 0).all())


def _argmax(logits, dtype, stride, rows, vocab, softcap, out, ids, tokens, max_len, step, ws):
    d = nat.STEP_F32 if dtype == torch.float32 else nat.STEP_BF16
    nat.step_check(nat.lib().se12_step_logits_argmax(nat.ptr(logits), d, stride, rows, vocab, softcap, nat.ptr(out),
                                                     nat.ptr(ids), nat.ptr(tokens), max_len, nat.ptr(step),
                                                     nat.ptr(ws), ws.numel(), nat.stream_ptr()))


@pytest.mark.parametrize("dtype,vocab", [(torch.float32, 256000), (torch.bfloat16, 256000), (torch.float32, 3000)])
def test_logits_argmax_and_token_slot(gpu, dtype, vocab):
    rows, max_len = 3, 40
    stride = vocab + 32
    g = _gen(gpu, 17)
    z = (torch.randn((rows, stride), generator=g, device=gpu) * 5).to(dtype)
    z[1, vocab - 7] = 1000.0             # soft-capped to 30: ties with nothing else
    z[2, 7] = z[2, vocab // 2 + 1] = 2000.0   # an exact tie across vocabulary slices: the first index wins
    logits = z[:, :vocab]
    out = torch.empty((rows, vocab), dtype=torch.bfloat16, device=gpu)
    ids = torch.full((rows,), -1, dtype=torch.int64, device=gpu)
    tokens = torch.full((rows, max_len), -1, dtype=torch.int64, device=gpu)
    step = torch.tensor(5, dtype=torch.int64, device=gpu)
    ws = torch.zeros(nat.lib().se12_step_logits_workspace(rows, vocab), dtype=torch.uint8, device=gpu)
    _argmax(logits, dtype, stride, rows, vocab, 30.0, out, ids, tokens, max_len, step, ws)
    torch.cuda.synchronize()
    lb = logits.to(torch.bfloat16)
    _ulp_close(out, torch.tanh(lb / 30.0) * 30.0)
    # ids are the first maximum of the kernel's own capped logits
    mx = out.float().max(dim=1, keepdim=True).values
    first = (out.float() == mx).float().argmax(dim=1)
    assert torch.equal(ids, first)
    assert int(ids[1]) == vocab - 7 and int(ids[2]) == 7
    assert torch.equal(tokens[:, 5], ids) and int((tokens != -1).sum()) == rows
    # a step outside the token buffer writes ids only; the workspace's counters were left at zero
    step.fill_(max_len)
    tokens.fill_(-1)
    ids.fill_(-1)
    _argmax(logits, dtype, stride, rows, vocab, 30.0, None, ids, tokens, max_len, step, ws)
    torch.cuda.synchronize()
    assert bool((tokens == -1).all()) and torch.equal(ids, first)
    assert bool((ws[: 4 * rows] == 0).all())


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_logits_argmax_with_nan_logits(gpu, dtype):
    """NaN ranks above every number, as in torch.argmax: a row with NaNs
    gives its first NaN (across vocabulary slices too), a row of NaNs its
    first index, so the token id always indexes the vocabulary."""
    rows, vocab, max_len = 3, 256000, 8
    g = _gen(gpu, 23)
    z = torch.randn((rows, vocab), generator=g, device=gpu) * 5
    z[0, 100] = 1000.0
    z[0, vocab - 5] = float("nan")
    z[0, vocab // 2 + 3] = float("nan")
    z[1].fill_(float("nan"))
    z[2, 1] = float("nan")
    logits = z.to(dtype)
    ids = torch.full((rows,), -1, dtype=torch.int64, device=gpu)
    tokens = torch.full((rows, max_len), -1, dtype=torch.int64, device=gpu)
    step = torch.tensor(0, dtype=torch.int64, device=gpu)
    ws = torch.zeros(nat.lib().se12_step_logits_workspace(rows, vocab), dtype=torch.uint8, device=gpu)
    _argmax(logits, dtype, vocab, rows, vocab, 30.0, None, ids, tokens, max_len, step, ws)
    torch.cuda.synchronize()
    assert ids.tolist() == [vocab // 2 + 3, 0, 1]
    assert torch.equal(ids, torch.argmax(logits.float(), dim=1))
    assert torch.equal(tokens[:, 0], ids)
    assert bool((ws[: 4 * rows] == 0).all())


def test_bf16_rounding_of_fp32_inputs(gpu):
    """The step kernels round FP32 inputs to BF16 with the hardware
    conversion; it must give the integer round-to-nearest-even form, a NaN its
    top 16 bits with the quiet bit set. Through the logits kernel (soft cap
    off: its BF16 logits are the inputs rounded): ties, subnormals, the
    overflow to infinity, signalling and quiet NaNs, and 2^20 random bit
    patterns."""
    special = np.array([0x00000000, 0x80000000, 0x00000001, 0x007FFFFF, 0x00008000, 0x00018000, 0x3F808000,
                        0x3F818000, 0x3F80FFFF, 0x7F7FFFFF, 0x7F7F8000, 0x7F7F7FFF, 0x7F800000, 0xFF800000,
                        0x7F800001, 0x7FBFFFFF, 0x7FC00000, 0xFFC12345, 0xFF800001, 0x7FFFFFFF], dtype=np.uint32)
    rng = np.random.default_rng(7)
    u = np.concatenate([special, rng.integers(0, 2 ** 32, size=1 << 20, dtype=np.uint64).astype(np.uint32)])
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    want = np.where(nan, (u >> 16) | 0x40, (u.astype(np.uint64) + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    vocab = int(u.size)
    logits = torch.from_numpy(u.view(np.float32).copy()).to(gpu).view(1, vocab)
    out = torch.empty((1, vocab), dtype=torch.bfloat16, device=gpu)
    ids = torch.full((1,), -1, dtype=torch.int64, device=gpu)
    tokens = torch.full((1, 4), -1, dtype=torch.int64, device=gpu)
    step = torch.tensor(0, dtype=torch.int64, device=gpu)
    ws = torch.zeros(nat.lib().se12_step_logits_workspace(1, vocab), dtype=torch.uint8, device=gpu)
    _argmax(logits, torch.float32, vocab, 1, vocab, 0.0, out, ids, tokens, 4, step, ws)
    torch.cuda.synchronize()
    got = out.view(torch.int16).cpu().numpy().view(np.uint16).reshape(-1)
    assert np.array_equal(got, want), int((got != want).sum())
    assert 0 <= int(ids[0]) < vocab


@pytest.mark.parametrize("rows,vocab", [(1, 256000), (3, 256000), (2, 1000)])
def test_logits_argmax_advance_equals_argmax_then_advance(gpu, rows, vocab):
    """The one-launch pick-and-advance gives the ids, tokens, logits, pos
    and step of argmax followed by advance, on consecutive calls (its
    counters return to zero), across rows and with a single block per row."""
    max_len = 16
    g = _gen(gpu, 31)
    want, got = {}, {}
    for name, res in (("two", want), ("one", got)):
        ids = torch.full((rows,), -1, dtype=torch.int64, device=gpu)
        tokens = torch.full((rows, max_len), -1, dtype=torch.int64, device=gpu)
        out = torch.empty((rows, vocab), dtype=torch.bfloat16, device=gpu)
        step = torch.tensor(3, dtype=torch.int64, device=gpu)
        pos = torch.tensor(100, dtype=torch.int64, device=gpu)
        ws = torch.zeros(nat.lib().se12_step_logits_workspace(rows, vocab), dtype=torch.uint8, device=gpu)
        g.manual_seed(31)
        for _ in range(4):
            z = torch.randn((rows, vocab), generator=g, device=gpu) * 5
            if name == "two":
                _argmax(z, torch.float32, vocab, rows, vocab, 30.0, out, ids, tokens, max_len, step, ws)
                nat.step_check(nat.lib().se12_step_advance(nat.ptr(pos), nat.ptr(step), nat.stream_ptr()))
            else:
                nat.step_check(nat.lib().se12_step_logits_argmax_advance(
                    nat.ptr(z), nat.STEP_F32, vocab, rows, vocab, 30.0, nat.ptr(out), nat.ptr(ids), nat.ptr(tokens),
                    max_len, nat.ptr(step), nat.ptr(pos), nat.ptr(ws), ws.numel(), nat.stream_ptr()))
        torch.cuda.synchronize()
        res.update(ids=ids.cpu(), tokens=tokens.cpu(), out=out.view(torch.int16).cpu(), step=int(step), pos=int(pos))
        assert bool((ws[: 4 * (rows + 1)] == 0).all())
    assert got["step"] == want["step"] == 7 and got["pos"] == want["pos"] == 104
    assert torch.equal(got["ids"], want["ids"]) and torch.equal(got["tokens"], want["tokens"])
    assert torch.equal(got["out"], want["out"])
    assert int((got["tokens"] != -1).sum()) == 4 * rows and bool((got["tokens"][:, 3:7] != -1).all())


def test_logits_argmax_advance_graph_replays(gpu):
    """Captured in a HIP graph and replayed with new logits copied in
    between (eager work and synchronisations between replays), every
    replay picks the eager argmax, stores it at the current step and
    advances pos and step by one."""
    rows, vocab, max_len = 2, 256000, 8
    g = _gen(gpu, 37)
    z = torch.zeros((rows, vocab), device=gpu)
    ids = torch.full((rows,), -1, dtype=torch.int64, device=gpu)
    tokens = torch.full((rows, max_len), -1, dtype=torch.int64, device=gpu)
    step = torch.tensor(1, dtype=torch.int64, device=gpu)
    pos = torch.tensor(50, dtype=torch.int64, device=gpu)
    ws = torch.zeros(nat.lib().se12_step_logits_workspace(rows, vocab), dtype=torch.uint8, device=gpu)

    def pick():
        nat.step_check(nat.lib().se12_step_logits_argmax_advance(
            nat.ptr(z), nat.STEP_F32, vocab, rows, vocab, 0.0, None, nat.ptr(ids), nat.ptr(tokens), max_len,
            nat.ptr(step), nat.ptr(pos), nat.ptr(ws), ws.numel(), nat.stream_ptr()))

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=s):
            pick()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    assert int(step) == 1 and int(pos) == 50      # capture launches nothing
    want_tokens = []
    for rep in range(4):
        z.copy_(torch.randn((rows, vocab), generator=g, device=gpu) * 5)
        zb = z.to(torch.bfloat16).float()
        first = torch.arange(vocab, device=gpu).expand(rows, -1)
        want = torch.where(zb == zb.max(dim=1, keepdim=True).values, first, vocab).min(dim=1).values
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(ids, want), rep
        assert int(step) == 2 + rep and int(pos) == 51 + rep
        want_tokens.append(want)
        assert torch.equal(tokens[:, 1:2 + rep], torch.stack(want_tokens, dim=1))
        assert bool((ws[: 4 * (rows + 1)] == 0).all())


def test_advance(gpu):
    pos = torch.tensor(41, dtype=torch.int64, device=gpu)
    step = torch.tensor(2, dtype=torch.int64, device=gpu)
    for _ in range(3):
        nat.step_check(nat.lib().se12_step_advance(nat.ptr(pos), nat.ptr(step), nat.stream_ptr()))
    torch.cuda.synchronize()
    assert int(pos) == 44 and int(step) == 5
