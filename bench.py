"""Benchmark: fused SE12 decode + GEMV at batch 1 on one MI355X.

Workload (one "step"): every linear of a 26-layer Gemma-2-2B at batch 1 -
per layer q 2048x2304, k 1024x2304, v 1024x2304, o 2304x2048, gate 9216x2304,
up 9216x2304, down 2304x9216 - i.e. 182 fused SE12 GEMVs over 3.04 GB of SE12
streams (2.02 G weights), far beyond the 256 MB Infinity Cache, so every step
streams from HBM. The step runs the way a decode runtime issues it: the
projections that read the same input share one launch (q/k/v, then gate/up),
so 4 launches per layer; the same step with one launch per GEMV (7 per layer)
is reported beside it, and the hipBLASLt BF16 comparison gets the same
grouping (one GEMV over the concatenated q/k/v and gate/up weights). Weights are BF16 N(0, 0.02) drawn on the device (torch
generator seeded per layer and projection) and SE12-encoded on the GPU;
activations are BF16 N(0, 1) seeded per layer. The step is captured once in a
HIP graph and replayed; the timed region is bracketed by synchronizations and
HIP events on the replay stream. Every GEMV uses the library's default launch.

Printed JSON (one line on stdout): value = BF16-equivalent weight GB/s of the
whole step (2 bytes x weights / step time, the reference's convention,
lws/bench/micro.py:162-165); the same step with one launch per GEMV; the
step through hipBLASLt BF16 (torch.nn.functional.linear) and through the
raw-BF16 twin kernel; per-shape microseconds; a roofline object for the dominant kernel - the fused GEMV at
the 2304x9216 down_proj shape, timed live as 26 back-to-back launches over the
26 layers' (cold) matrices; and the oracle's numpy decode + matmul timed on
the host as the CPU baseline. More objects: the batch sweep B = 1..32 at
the Gemma-2-9B gate_proj shape 14336x3584 against hipBLASLt BF16 and the raw
twin (the crossover from the dot2 kernel to the MFMA kernels), the
decode-only kernel (SE12 -> BF16) at three shapes, batch-1 stress shapes
with heavy-tailed weights (tied LM head 256000x2304, Gemma-2-27B down_proj
4608x36864), and a random-init Gemma-2-2B greedy decode (prompt 512, 128
tokens) whose decode tokens/s is the `decode_tok_s` field.
"""

from __future__ import annotations

import argparse
import dataclasses
import json
import os
import sys
import time

import torch

METRIC = "BF16-equiv weight GB/s + us per fused SE12 GEMV at batch 1; decode tok/s"
HBM_PEAK_GBPS = 8000.0
# HBM bytes per launch of the dominant kernel, measured with two rocprofv3
# counter runs (FETCH_SIZE, WRITE_SIZE) scaled by the same counters' reading
# of a 256 MiB device copy; null in the output when the file is absent
TRAFFIC_FILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "gemv_fused_b1_down_proj_traffic.json")
LAYERS = 26
HIDDEN, INTER, QDIM, KVDIM = 2304, 9216, 2048, 1024
# (name, rows N, cols K, input vector)
PROJECTIONS = (
    ("q", QDIM, HIDDEN, "h"),
    ("k", KVDIM, HIDDEN, "h"),
    ("v", KVDIM, HIDDEN, "h"),
    ("o", HIDDEN, QDIM, "a"),
    ("gate", INTER, HIDDEN, "h"),
    ("up", INTER, HIDDEN, "h"),
    ("down", HIDDEN, INTER, "m"),
)


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def parse_args(argv=None):
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--layers", type=int, default=LAYERS, help="layers in the stack (26 = Gemma-2-2B)")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-per-shape", action="store_true")
    p.add_argument("--no-batch-sweep", action="store_true")
    p.add_argument("--no-stress", action="store_true")
    p.add_argument("--no-decode", action="store_true", help="skip the decode-only kernel timings")
    p.add_argument("--no-e2e", action="store_true", help="skip the Gemma-2-2B greedy decode")
    p.add_argument("--no-micro", action="store_true", help="skip the microbenchmark / verdict files")
    p.add_argument("--no-model", action="store_true", help="skip the roofline model's calibration")
    p.add_argument("--reports", default=os.environ.get("LWS_VERDICT_DIR", "reports"),
                   help="directory for micro-<slug>.json and verdict-<slug>.json")
    p.add_argument("--only-fused", action="store_true", help="skip the BF16 and raw-twin comparisons (profiling)")
    p.add_argument("--profile-down", action="store_true",
                   help="only the dominant kernel (26 down_proj launches per step) and a 256 MiB device copy of known "
                        "size, for hardware-counter runs")
    p.add_argument("--profile-batch", type=int, default=None, metavar="B",
                   help="only the batch sweep's 14336x3584 product at batch B (cold rotation of matrices), for "
                        "hardware-counter runs of one kernel")
    p.add_argument("--profile-shape", default="14336x3584", metavar="NxK",
                   help="the matrix shape of --profile-batch (default 14336x3584)")
    p.add_argument("--profile-blas", default=None, metavar="NxK",
                   help="only hipBLASLt's BF16 product (F.linear) at batch 1 on an NxK matrix (rotation of cold "
                        "matrices), then a 256 MiB device copy of known size, for hardware-counter runs of the baseline")
    p.add_argument("--profile-e2e", choices=("se12", "raw", "bf16"), default=None,
                   help="only the Gemma-2-2B decode of one backend: prefill 512, capture, a 0.5 s pause, 32 graph-"
                        "replayed steps (kernel traces of the decode step)")
    return p.parse_args(argv)


def profile_e2e(backend: str, device, steps: int = 32) -> int:
    """The Gemma-2-2B greedy decode of `e2e_decode` for one backend, with a
    0.5 s pause between capture and the timed steps so that a kernel trace
    can cut the decode steps from prefill and capture."""
    from se12_amd.gemma2 import GEMMA2_2B, PROJECTIONS, Gemma2Decoder, Gemma2Weights
    from se12_amd.hip import encode_on_device

    w = Gemma2Weights.random(GEMMA2_2B, device)
    enc = None
    if backend == "se12":
        enc = {(li, n): encode_on_device(lw[n]) for li, lw in enumerate(w.layers) for n in PROJECTIONS}
        enc["embed"] = encode_on_device(w.embed)
    gen = torch.Generator(device=device)
    gen.manual_seed(4242)
    prompt = torch.randint(0, GEMMA2_2B.vocab, (1, 512), generator=gen, device=device)
    dec = Gemma2Decoder(w, backend, batch=1, max_len=512 + 128, encoded=enc)
    dec.prefill(prompt)
    dec.capture()
    torch.cuda.synchronize()
    time.sleep(0.5)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    dec.decode(steps)
    end.record()
    end.synchronize()
    ms = start.elapsed_time(end)
    print(json.dumps({"profile": f"gemma-2-2b decode, {backend}", "steps": steps, "ms_per_step": round(ms / steps, 4)}),
          flush=True)
    return 0


def profile_down(args, device) -> int:
    """The dominant kernel alone: the 26 layers' 2304x9216 down_proj GEMVs
    (cold: 830 MB of streams), then a 256 MiB device-to-device copy whose byte
    counts calibrate the FETCH_SIZE / WRITE_SIZE counters."""
    from se12_amd.hip import Se12MatVecKernel, encode_on_device

    gen = torch.Generator(device=device)
    n, k = 2304, 9216
    down = []
    for layer in range(args.layers):
        gen.manual_seed(layer * 100 + 6)
        w = (torch.randn((n, k), generator=gen, device=device, dtype=torch.float32) * 0.02).to(torch.bfloat16)
        gen.manual_seed(1_000_000 + layer * 10 + 2)
        x = torch.randn((1, k), generator=gen, device=device, dtype=torch.float32).to(torch.bfloat16)
        kern = Se12MatVecKernel(encode_on_device(w), max_batch=1)
        down.append({"kern": kern, "x": x, "y": torch.empty((1, n), dtype=torch.float32, device=device)})
        del w
    g = capture(lambda: [e["kern"].multiply(e["x"], out=e["y"]) for e in down])
    ms = time_graph(g, args.steps, args.warmup)
    src = torch.empty(64 << 20, dtype=torch.float32, device=device)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"profile": "down_proj 2304x9216 fused GEMV", "us_per_launch": round(ms * 1e3 / len(down), 3),
                      "launches": len(down) * (args.steps + args.warmup + 2), "copy_bytes": src.numel() * 4,
                      "copies": 3}), flush=True)
    return 0


def profile_blas(args, device) -> int:
    """hipBLASLt's BF16 product (F.linear, batch 1) alone at one shape, over a
    rotation of distinct BF16 matrices of more than 1 GB so that every launch
    streams from HBM, then the 256 MiB device copy that calibrates the
    FETCH_SIZE / WRITE_SIZE counters (as --profile-down)."""
    n, k = (int(v) for v in args.profile_blas.split("x"))
    gen = torch.Generator(device=device)
    ws = []
    for r in range(cold_rotation(2 * n * k)):
        gen.manual_seed(r)
        ws.append((torch.randn((n, k), generator=gen, device=device) * 0.02).to(torch.bfloat16))
    gen.manual_seed(99)
    x = torch.randn((1, k), generator=gen, device=device).to(torch.bfloat16)
    g = capture(lambda: [torch.nn.functional.linear(x, w) for w in ws])
    ms = time_graph(g, args.steps, args.warmup)
    src = torch.empty(64 << 20, dtype=torch.float32, device=device)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"profile": f"hipBLASLt BF16 product {n}x{k} at batch 1", "us_per_launch": round(ms * 1e3 / len(ws), 3),
                      "launches": len(ws) * (args.steps + args.warmup + 2), "bf16_bytes": 2 * n * k,
                      "copy_bytes": src.numel() * 4, "copies": 3}), flush=True)
    return 0


def profile_batch(args, device, batch: int) -> int:
    """The batch sweep's product alone at one batch: 14336x3584 (a Gemma-2-9B
    MLP shape) or --profile-shape, a rotation of distinct matrices over more
    than 1 GB so that every launch streams from HBM, default launch."""
    from se12_amd.hip import Se12MatVecKernel, encode_on_device

    n, k = (int(v) for v in args.profile_shape.split("x"))
    gen = torch.Generator(device=device)
    kerns = []
    for r in range(cold_rotation(int(n * k * 1.504))):
        gen.manual_seed(r)
        w = (torch.randn((n, k), generator=gen, device=device) * 0.02).to(torch.bfloat16)
        kerns.append(Se12MatVecKernel(encode_on_device(w), max_batch=batch))
        del w
    gen.manual_seed(99)
    x = torch.randn((batch, k), generator=gen, device=device).to(torch.bfloat16)
    y = torch.empty((batch, n), dtype=torch.float32, device=device)
    g = capture(lambda: [kk.multiply(x, out=y) for kk in kerns])
    ms = time_graph(g, args.steps, args.warmup)
    launch = kerns[0].default_launch(batch)
    print(json.dumps({"profile": f"fused SE12 product {n}x{k} at batch {batch}",
                      "us_per_launch": round(ms * 1e3 / len(kerns), 3),
                      "launch": [launch.threads_per_block.value, launch.blocks.value]}), flush=True)
    return 0


def build_stack(layers: int, device):
    from se12_amd.hip import Se12MatVecKernel, encode_on_device

    gen = torch.Generator(device=device)
    stack = []
    for layer in range(layers):
        xs = {}
        for key, dim in (("h", HIDDEN), ("a", QDIM), ("m", INTER)):
            gen.manual_seed(1_000_000 + layer * 10 + len(xs))
            xs[key] = torch.randn((1, dim), generator=gen, device=device, dtype=torch.float32).to(torch.bfloat16)
        entries = []
        for pi, (name, n, k, xin) in enumerate(PROJECTIONS):
            gen.manual_seed(layer * 100 + pi)
            w = (torch.randn((n, k), generator=gen, device=device, dtype=torch.float32) * 0.02).to(torch.bfloat16)
            enc = encode_on_device(w)
            kern = Se12MatVecKernel(enc, max_batch=1)
            y = torch.empty((1, n), dtype=torch.float32, device=device)
            entries.append({"name": name, "n": n, "k": k, "w": w, "enc": enc, "kern": kern, "x": xs[xin], "y": y})
        stack.append(entries)
        if layer == 0 or (layer + 1) % 13 == 0:
            log(f"[bench] layer {layer + 1}/{layers} encoded")
    return stack


def capture(fn):
    """Captures fn() (a sequence of launches on the current stream) in a graph."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    torch.cuda.synchronize()
    return g


def evict_caches(buf: torch.Tensor) -> None:
    """Reads `buf` (1 GiB, over 4x L2 + Infinity Cache) so that the next
    launch finds its weights in HBM only. A read, not a fill: a fill leaves
    the caches full of dirty lines whose write-back would compete with the
    timed launch's reads."""
    torch.sum(buf)


class Timing(float):
    """Mean ms per replay (the float value), with the median, p10 and p90 of
    the per-replay times (the reference's statistics,
    lws/domain/benchmark/statistics.py:46-53)."""

    def __new__(cls, samples_ms):
        import numpy as np

        arr = np.asarray(samples_ms, dtype=np.float64)
        obj = super().__new__(cls, float(arr.mean()))
        obj.median = float(np.median(arr))
        obj.p10 = float(np.percentile(arr, 10))
        obj.p90 = float(np.percentile(arr, 90))
        return obj

    def stats_us(self, per: int = 1) -> dict:
        """Median / p10 / p90 in microseconds per launch (`per` launches per replay)."""
        return {"median_us": round(self.median * 1e3 / per, 3), "p10_us": round(self.p10 * 1e3 / per, 3),
                "p90_us": round(self.p90 * 1e3 / per, 3)}


def time_graph(g, steps: int, warmup: int, flush=None) -> Timing:
    """ms per replay over `steps` replays, events on the replay stream. Without
    a flush the replays run back to back between one pair of
    synchronizations, an event between consecutive replays; with one, the
    flush runs before each replay, outside its event pair."""
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    if flush is None:
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
        ev[0].record()
        for i in range(steps):
            g.replay()
            ev[i + 1].record()
        ev[-1].synchronize()
        return Timing([ev[i].elapsed_time(ev[i + 1]) for i in range(steps)])
    samples = []
    for _ in range(steps):
        flush()
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record()
        g.replay()
        end.record()
        end.synchronize()
        samples.append(start.elapsed_time(end))
    return Timing(samples)


def settled_us(g, launches: int, runs: int = 3) -> float:
    """us per launch of a graph of `launches` launches: the median of `runs`
    time_graph calls (each 5 warm-up and 10 timed replays). A single call
    right after capture reads up to 10% high: successive calls on a fresh
    graph settle (14336x3584 B = 24: 24.7, 23.9, 23.3 us)."""
    import statistics

    return statistics.median(time_graph(g, 10, 5) * 1e3 / launches for _ in range(runs))


def cold_rotation(nbytes: int) -> int:
    """Matrices to rotate through so that a pass streams from HBM (>= 1.1 GB,
    over 4x the 256 MB Infinity Cache)."""
    return max(2, -(-int(1.1e9) // nbytes))


def batch_sweep(device, batches=(1, 2, 4, 5, 6, 7, 8, 16, 24, 32), n=14336, k=3584, seed=9_000) -> dict:
    """Gemma-2-9B gate_proj 14336x3584 (or another n x k), BF16 N(0, 0.02):
    the fused product at each batch (the dot2 kernel up to 4 rows, an MFMA
    kernel from 5; one pass over the weights either way) against hipBLASLt
    BF16 and the raw twin at the same batch, each timed per launch over a
    rotation of cold matrices. B = 5..7 show the MFMA kernel where the dot2
    kernel, 4 batch rows per pass, would need a second pass over the
    weights."""
    from se12_amd.hip import RawBf16MatVecKernel, Se12MatVecKernel, encode_on_device
    from se12_amd.launch import rx_splits, uses_mfma, uses_rx

    gen = torch.Generator(device=device)
    ws, kerns = [], []
    r_se12 = cold_rotation(int(n * k * 1.504))
    r_bf16 = cold_rotation(2 * n * k)
    for r in range(max(r_se12, r_bf16)):
        gen.manual_seed(seed + r)
        w = (torch.randn((n, k), generator=gen, device=device, dtype=torch.float32) * 0.02).to(torch.bfloat16)
        if r < r_se12:
            kerns.append(Se12MatVecKernel(encode_on_device(w), max_batch=max(batches)))
        if r < r_bf16:
            ws.append(w)
    out = {"shape": [n, k], "rotation": {"se12": r_se12, "bf16": r_bf16}, "points": []}
    for b in batches:
        gen.manual_seed(seed + 999 + b)
        x = torch.randn((b, k), generator=gen, device=device, dtype=torch.float32).to(torch.bfloat16)
        y = torch.empty((b, n), dtype=torch.float32, device=device)
        g = capture(lambda x=x, y=y: [kk.multiply(x, out=y) for kk in kerns])
        us = settled_us(g, len(kerns))
        gb = capture(lambda x=x: [torch.nn.functional.linear(x, w) for w in ws])
        us_b = settled_us(gb, len(ws))
        raws = [RawBf16MatVecKernel(w, max_batch=b) for w in ws]
        yr = [torch.empty((b, n), dtype=torch.float32, device=device) for _ in raws]
        gr = capture(lambda x=x: [r.multiply(x, out=y) for r, y in zip(raws, yr)])
        us_r = settled_us(gr, len(raws))
        del g, gb, gr, raws, yr
        lc = kerns[0].default_launch(b)
        kernel = ("mfma_resident_x" if uses_rx(n, k, b) else "mfma_x_slab") if uses_mfma(b) else "dot2"
        if uses_rx(n, k, b) and rx_splits(n, k, b) > 1:
            kernel += f"_{rx_splits(n, k, b)}_k_splits"
        pt = {"batch": b, "kernel": kernel, "us": round(us, 3),
              "bf16_equiv_gbps": round(2 * n * k / (us * 1e-6) / 1e9, 1),
              "se12_gbps": round(kerns[0].tensor.byte_size() / (us * 1e-6) / 1e9, 1),
              "bf16_hipblaslt_us": round(us_b, 3), "speedup_of_se12": round(us_b / us, 4),
              "raw_twin_us": round(us_r, 3), "speedup_vs_faster_baseline": round(min(us_b, us_r) / us, 4),
              "launch": [lc.threads_per_block.value, lc.blocks.value]}
        out["points"].append(pt)
        log(f"[bench] batch sweep {pt}")
    return out


def decode_only(device, shapes=((2304, 9216), (9216, 2304), (256000, 2304))) -> dict:
    """The decode-only kernel (SE12 -> row-major BF16, the path of prefill and
    mode="exact"; lws/adapters/cuda/kernels/se12_decode.cu:12-43 is the
    reference's) on BF16 N(0, 0.02) matrices, timed per launch over a rotation
    of cold copies in one graph, beside a device copy of the same BF16 matrix
    (2 bytes read + 2 written per weight; the decode reads the streams, about
    1.5 bytes, and writes 2). Algorithmic bytes per launch: the streams plus
    the BF16 output."""
    from se12_amd.hip import HipBenchmarkTimer, Se12MatVecKernel, encode_on_device
    from se12_amd.micro import cold_copies

    timer = HipBenchmarkTimer(device.index)
    out = {}
    for n, k in shapes:
        gen = torch.Generator(device=device)
        gen.manual_seed(n + k)
        w = (torch.randn((n, k), generator=gen, device=device, dtype=torch.float32) * 0.02).to(torch.bfloat16)
        enc = encode_on_device(w)
        copies = cold_copies(enc.byte_size() + 2 * n * k)
        kerns = [Se12MatVecKernel(e, max_batch=1) for e in [enc] + [enc.clone() for _ in range(copies - 1)]]
        dst = [torch.empty((n, k), dtype=torch.bfloat16, device=device) for _ in range(copies)]
        st = timer.time_cold_rotation([lambda kk=kk, d=d: kk.decode_into(d) for kk, d in zip(kerns, dst)], 3, 10)
        exact = bool(torch.equal(dst[0], w))
        del kerns
        srcs = [w] + [w.clone() for _ in range(copies - 1)]
        st_c = timer.time_cold_rotation([lambda s_=s_, d=d: d.copy_(s_) for s_, d in zip(srcs, dst)], 3, 10)
        del srcs, dst
        alg = enc.byte_size() + 2 * n * k
        us = st.median_us
        out[f"{n}x{k}"] = {"us": round(us, 3), "p10_us": round(st.p10_us, 3), "p90_us": round(st.p90_us, 3),
                           "algorithmic_bytes": alg, "gbps": round(alg / (us * 1e-6) / 1e9, 1),
                           "frac_of_hbm_peak": round(alg / (us * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4),
                           "bf16_copy_us": round(st_c.median_us, 3),
                           "bf16_copy_gbps": round(4 * n * k / (st_c.median_us * 1e-6) / 1e9, 1),
                           "cold_copies": copies, "bit_exact": exact}
        log(f"[bench] decode only {n}x{k}: {out[f'{n}x{k}']}")
        del enc, w
        torch.cuda.empty_cache()
    return out


def heavy_tailed(n: int, k: int, seed: int, device) -> torch.Tensor:
    """Student-t (df 3) scaled to std 0.02 with 0.1% outliers at +-8 sigma, BF16."""
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    z = torch.randn((n, k), generator=gen, device=device)
    chi2 = torch.randn((3, n, k), generator=gen, device=device).square().sum(0)
    w = z / torch.sqrt(chi2 / 3.0) / (3.0 ** 0.5) * 0.02
    flat = w.view(-1)
    n_out = max(1, flat.numel() // 1000)
    idx = torch.randint(0, flat.numel(), (n_out,), generator=gen, device=device)
    sign = torch.randint(0, 2, (n_out,), generator=gen, device=device).float() * 2 - 1
    flat[idx] = sign * 0.16
    return w.to(torch.bfloat16)


def stress(device) -> dict:
    """Batch-1 products at the tied LM head 256000x2304 and the Gemma-2-27B
    down_proj 4608x36864 with heavy-tailed weights (escape and fallback
    paths), against hipBLASLt BF16 and the raw twin: each timed over a
    rotation of cold copies in one graph (at least 8 launches per replay, so
    the replay's fixed cost of ~10 us spreads; HipBenchmarkTimer.
    time_cold_rotation), median / p10 / p90 per launch of the run whose
    median is the median of three runs (the first run over freshly written
    copies read up to 10% high: 4608x36864 48.4 against 43.4 us)."""
    from se12_amd.hip import HipBenchmarkTimer, RawBf16MatVecKernel, Se12MatVecKernel, encode_on_device
    from se12_amd.micro import cold_copies

    timer = HipBenchmarkTimer(device.index)

    def settled(ops):
        runs = sorted((timer.time_cold_rotation(ops, 3, 10) for _ in range(3)), key=lambda r: r.median_us)
        return runs[1]

    out = {}
    for name, n, k, seed in (("lm_head", 256000, 2304, 11), ("down_27b", 4608, 36864, 12)):
        w = heavy_tailed(n, k, seed, device)
        enc = encode_on_device(w)
        copies = cold_copies(2 * n * k)
        ws = [w] + [w.clone() for _ in range(copies - 1)]
        kerns = [Se12MatVecKernel(e, max_batch=1) for e in [enc] + [enc.clone() for _ in range(copies - 1)]]
        gen = torch.Generator(device=device)
        gen.manual_seed(seed + 100)
        x = torch.randn((1, k), generator=gen, device=device).to(torch.bfloat16)
        ys = [torch.empty((1, n), dtype=torch.float32, device=device) for _ in range(copies)]
        st = settled([lambda kk=kk, y=y: kk.multiply(x, out=y) for kk, y in zip(kerns, ys)])
        del kerns
        st_b = settled([lambda m=m: torch.nn.functional.linear(x, m) for m in ws])
        raws = [RawBf16MatVecKernel(m, max_batch=1) for m in ws]
        st_r = settled([lambda kk=kk, y=y: kk.multiply(x, out=y) for kk, y in zip(raws, ys)])
        del raws
        us, us_b, us_r = st.median_us, st_b.median_us, st_r.median_us
        k0 = Se12MatVecKernel(enc, max_batch=1)
        lc = k0.default_launch(1)
        bs = k0.bind_stats()
        # the kernel's reads besides the format's bytes: tiles bind decoded to
        # raw BF16 (more escapes than a side record lists) add 8,192 bytes each
        streamed = enc.byte_size() + bs["raw_tiles"] * 8192
        out[name] = {"shape": [n, k], "us": round(us, 3), "p10_us": round(st.p10_us, 3), "p90_us": round(st.p90_us, 3),
                     "cold_copies": copies, "se12_bytes": enc.byte_size(),
                     "bytes_per_weight": round(enc.byte_size() / (n * k), 4),
                     "se12_gbps": round(enc.byte_size() / (us * 1e-6) / 1e9, 1),
                     "bind_decoded_raw_tiles": bs["raw_tiles"],
                     "bind_decoded_raw_bytes": bs["raw_tiles"] * 8192,
                     "streamed_bytes": streamed,
                     "streamed_gbps": round(streamed / (us * 1e-6) / 1e9, 1),
                     "sidecar_bytes": bs["sidecar_bytes"],
                     "bf16_equiv_gbps": round(2 * n * k / (us * 1e-6) / 1e9, 1),
                     "bf16_hipblaslt_us": round(us_b, 3), "raw_twin_us": round(us_r, 3),
                     "speedup_of_se12": round(us_b / us, 4), "speedup_vs_faster_baseline": round(min(us_b, us_r) / us, 4),
                     "fallback_tiles": enc.fallback_tiles, "tiles": enc.tile_grid[0] * enc.tile_grid[1],
                     "launch": [lc.threads_per_block.value, lc.blocks.value]}
        log(f"[bench] stress {name}: {out[name]}")
        del ws, enc, w, ys
        torch.cuda.empty_cache()
    return out


def e2e_decode(device, prompt_len: int = 512, new_tokens: int = 128) -> dict:
    """Random-init Gemma-2-2B (26 layers, hidden 2304, 8 query / 4 KV heads of
    256, intermediate 9216, vocab 256000; BF16 N(0, 0.02)) greedy decode at
    batch 1: a random prompt of `prompt_len` tokens, `new_tokens` generated.
    Every linear goes through the SE12 kernels (prefill decodes each layer and
    runs F.linear, exact); the same model through the order-matched raw-BF16
    twin and through hipBLASLt BF16 gives the comparison. Each decode step is
    one HIP graph replay; tokens/s counts the decode steps after prefill."""
    from se12_amd.gemma2 import GEMMA2_2B, PROJECTIONS, Gemma2Decoder, Gemma2Weights
    from se12_amd.hip import encode_on_device

    shape = GEMMA2_2B
    w = Gemma2Weights.random(shape, device)
    encoded = {(li, n): encode_on_device(lw[n]) for li, lw in enumerate(w.layers) for n in PROJECTIONS}
    encoded["embed"] = encode_on_device(w.embed)
    se12_bytes = sum(e.byte_size() for e in encoded.values())
    bf16_bytes = 2 * sum(lw[n].numel() for lw in w.layers for n in PROJECTIONS) + 2 * w.embed.numel()
    gen = torch.Generator(device=device)
    gen.manual_seed(4242)
    prompt = torch.randint(0, shape.vocab, (1, prompt_len), generator=gen, device=device)
    out = {"workload": f"gemma-2-2b random init, batch 1, prompt {prompt_len}, {new_tokens} greedy tokens",
           "se12_weight_bytes": se12_bytes, "bf16_weight_bytes": bf16_bytes}
    tokens = {}
    for name, backend in (("se12", "se12"), ("raw_bf16_twin", "raw"), ("bf16_hipblaslt", "bf16")):
        dec = Gemma2Decoder(w, backend, batch=1, max_len=prompt_len + new_tokens, encoded=encoded)
        dec.prefill(prompt)          # warm-up (library and GEMM selection), untimed
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        dec.prefill(prompt)
        torch.cuda.synchronize()
        prefill_ms = (time.perf_counter() - t0) * 1e3
        dec.capture()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        dec.decode(new_tokens - 1)
        end.record()
        end.synchronize()
        decode_ms = start.elapsed_time(end)
        tokens[name] = dec.tokens[0, :new_tokens].cpu()
        out[name] = {"prefill_ms": round(prefill_ms, 3), "decode_ms": round(decode_ms, 3),
                     "ms_per_token": round(decode_ms / (new_tokens - 1), 4),
                     "decode_tok_s": round((new_tokens - 1) / (decode_ms * 1e-3), 2),
                     "e2e_tok_s": round(new_tokens / ((prefill_ms + decode_ms) * 1e-3), 2)}
        log(f"[bench] e2e {name}: {out[name]}")
        del dec
        torch.cuda.empty_cache()
    same = tokens["se12"] == tokens["bf16_hipblaslt"]
    out["tokens_identical_se12_vs_raw_twin"] = bool(torch.equal(tokens["se12"], tokens["raw_bf16_twin"]))
    out["tokens_matching_se12_vs_bf16"] = int(same.sum())
    out["first_divergence_se12_vs_bf16"] = None if bool(same.all()) else int((~same).nonzero()[0, 0])
    out["decode_speedup_vs_bf16"] = round(out["se12"]["decode_tok_s"] / out["bf16_hipblaslt"]["decode_tok_s"], 4)
    del w, encoded
    torch.cuda.empty_cache()
    return out


def roofline_model(device, props, per_shape: dict) -> dict:
    """The reference's performance model (lws/domain/performance/roofline.py:
    52-146) fed by this device: peak from hipDeviceProp (memory clock x bus
    width), bandwidths and the graph launch cost measured here, each
    kernel's cost per weight from cache-resident launches (a 2304x2304
    matrix, 32 back-to-back launches in one graph), eta fitted from the raw
    twin's cold latency at the 2304x9216 down_proj shape, and the predicted
    fused / raw ratio against the measured one at every Gemma-2-2B shape."""
    from se12_amd import roofline as rl
    from se12_amd.hip import HipBenchmarkTimer, RawBf16MatVecKernel, Se12MatVecKernel, encode_on_device

    timer = HipBenchmarkTimer(device.index)
    gen = torch.Generator(device=device)
    # the streaming-read bandwidth: the faster of the library's grid-stride
    # read probe and the fused product's own stream over a cold 256000x2304
    # matrix at batch 1 (its tile-order reads go faster than any grid-stride
    # form), so that no product launch can beat the model's bandwidth
    probe_gbps = timer.measure_stream_read_bandwidth()
    gen.manual_seed(78)
    n_lm, k_lm = 256000, 2304
    lm = []
    for _ in range(2):
        w = (torch.randn((n_lm, k_lm), generator=gen, device=device) * 0.02).to(torch.bfloat16)
        lm.append(Se12MatVecKernel(encode_on_device(w), max_batch=1))
        del w
    x_lm = torch.randn((1, k_lm), generator=gen, device=device).to(torch.bfloat16)
    y_lm = torch.empty((1, n_lm), dtype=torch.float32, device=device)
    st_lm = timer.time_cold_rotation([lambda kk=kk: kk.multiply(x_lm, out=y_lm) for kk in lm], 3, 10)
    lm_gbps = (lm[0].tensor.byte_size() + k_lm * 2 + n_lm * 4) / (st_lm.median_us * 1e-6) / 1e9
    del lm, y_lm
    torch.cuda.empty_cache()
    facts = rl.DeviceFacts(hbm_peak_gbps=props.hbm_peak_gbps, copy_gbps=timer.measure_copy_traffic_gbps(),
                           stream_read_gbps=max(probe_gbps, lm_gbps), launch_us=timer.measure_graph_launch_us())
    gen.manual_seed(77)
    hot = {"raw": [], "se12": []}
    for n, k in rl.CALIBRATION_SHAPES:
        w = (torch.randn((n, k), generator=gen, device=device) * 0.02).to(torch.bfloat16)
        x = torch.randn((1, k), generator=gen, device=device).to(torch.bfloat16)
        y = torch.empty((1, n), dtype=torch.float32, device=device)
        for name, kern in (("raw", RawBf16MatVecKernel(w, max_batch=1)),
                           ("se12", Se12MatVecKernel(encode_on_device(w), max_batch=1))):
            g = capture(lambda kern=kern: [kern.multiply(x, out=y) for _ in range(32)])
            hot[name].append(time_graph(g, 20, 5).median * 1e3 / 32)
            del g
    cal = rl.calibrate(facts.copy_gbps, tuple(hot["raw"]), tuple(hot["se12"]), facts.launch_us)
    fit = per_shape["down"]
    eta = rl.fit_eta_from_raw(fit["raw_twin_us"], *fit["shape"], cal)
    shapes = {}
    for name, e in per_shape.items():
        rep = rl.shape_report(*e["shape"], cal, eta, e["us"], e["raw_twin_us"])
        shapes[name] = {kk: round(v, 4) for kk, v in rep.items()}
        shapes[name]["launch_floor_us"] = round(rl.launch_floor_us(*e["shape"], facts), 3)
    out = {"facts": {kk: round(v, 3) for kk, v in dataclasses.asdict(facts).items()},
           "stream_read": {"probe_gbps": round(probe_gbps, 1), "fused_lm_head_256000x2304_gbps": round(lm_gbps, 1),
                           "fused_lm_head_us": round(st_lm.median_us, 3)},
           "hbm_peak_published_gbps": rl.HBM_PEAK_PUBLISHED_GBPS,
           "calibration": {"shapes": [list(sh) for sh in rl.CALIBRATION_SHAPES], "batch": 1,
                           "raw_hot_us": [round(v, 3) for v in hot["raw"]],
                           "se12_hot_us": [round(v, 3) for v in hot["se12"]], "launch_us": round(cal.launch_us, 3),
                           "bandwidth_gbps": round(cal.bandwidth_gbps, 1),
                           "raw_cost_ps_per_weight": round(cal.raw_cost_us_per_weight * 1e6, 4),
                           "se12_cost_ps_per_weight": round(cal.se12_cost_us_per_weight * 1e6, 4)},
           "eta": round(eta, 4), "eta_fit": "raw twin, 2304x9216 (down_proj), cold",
           "per_shape": shapes}
    log(f"[bench] model: {out['facts']} eta {eta:.3f}")
    return out


def cpu_model() -> str | None:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def cpu_baseline(budget_s: float = 12.0) -> dict:
    """The oracle's numpy decode + float32 matmul of one 2304x9216 GEMV (the
    Gemma-2-2B down_proj shape, N(0, 0.02) seed 0) on the host: decode alone
    and decode + matmul, each timed with the BLAS pool limited to one thread
    (the value) and with every core the process may use; medians of at
    least 5 runs within the time budget."""
    import numpy as np
    from threadpoolctl import threadpool_info, threadpool_limits

    from oracle import se12_codec as o

    n, k = 2304, 9216
    bits = o.normal_bf16(n, k, seed=0, std=0.02)
    enc = o.encode(bits.reshape(-1), n, k)
    x = o.bf16_bits_to_f32(o.normal_bf16(1, k, seed=1, std=1.0))
    cores = len(os.sched_getaffinity(0))

    def med(fn, budget):
        times, t_end = [], time.perf_counter() + budget
        while len(times) < 5 or (time.perf_counter() < t_end and len(times) < 30):
            t0 = time.perf_counter()
            fn()
            times.append(time.perf_counter() - t0)
        return float(np.median(times)), len(times)

    with threadpool_limits(limits=1):
        dec_s, n_dec = med(lambda: o.decode(enc), budget_s / 4)
        gemv_s, n_gemv = med(lambda: o.gemv_reference(enc, x), budget_s / 2)
    with threadpool_limits(limits=cores):
        gemv_mt_s, n_mt = med(lambda: o.gemv_reference(enc, x), budget_s / 4)
    blas = [{"api": d.get("internal_api"), "version": d.get("version"), "threads": d.get("num_threads")}
            for d in threadpool_info() if d.get("user_api") == "blas"]
    return {
        "value": round(2.0 * n * k / gemv_s / 1e9, 4),
        "unit": "GB/s",
        "cores": 1,
        "kind": "port",
        "sample": f"one 2304x9216 GEMV at batch 1 (numpy decode + float32 matmul, 1 thread), median of {n_gemv} runs, "
                  f"{gemv_s * 1e3:.1f} ms each",
        "decode_only_ms": round(dec_s * 1e3, 3),
        "decode_only_runs": n_dec,
        "decode_gemv_ms": round(gemv_s * 1e3, 3),
        "decode_gemv_all_cores_ms": round(gemv_mt_s * 1e3, 3),
        "decode_gemv_all_cores_runs": n_mt,
        "decode_gemv_all_cores_gbps": round(2.0 * n * k / gemv_mt_s / 1e9, 4),
        "affinity_cores": cores,
        "cpu_model": cpu_model(),
        "blas": blas,
    }


def main(argv=None) -> int:
    args = parse_args(argv)
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); the SE12 path has no multi-GPU mode", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a HIP GPU", file=sys.stderr)
        return 2
    from se12_amd import _native
    from se12_amd.hip import HipGpuProbe, RawBf16MatVecKernel

    _native.lib()
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    if args.profile_down:
        return profile_down(args, dev)
    if args.profile_blas:
        return profile_blas(args, dev)
    if args.profile_batch is not None:
        if not 1 <= args.profile_batch <= 32:
            raise SystemExit("--profile-batch takes a batch in 1..32")
        return profile_batch(args, dev, args.profile_batch)
    if args.profile_e2e:
        return profile_e2e(args.profile_e2e, dev)
    props = HipGpuProbe(0).facts()
    log(f"[bench] device {props.name} {props.arch} CUs={props.compute_units}")
    t0 = time.perf_counter()
    stack = build_stack(args.layers, dev)
    torch.cuda.synchronize()
    log(f"[bench] stack built in {time.perf_counter() - t0:.1f}s")

    flat = [e for layer in stack for e in layer]
    weights = sum(e["n"] * e["k"] for e in flat)
    se12_bytes = sum(e["enc"].byte_size() for e in flat)
    act_bytes = sum(e["k"] * 2 + e["n"] * 4 for e in flat)
    bf16_bytes = 2 * weights

    from se12_amd.hip import multiply_grouped

    # per layer: [q, k, v] | o | [gate, up] | down
    GROUPS = ((0, 1, 2), (3,), (4, 5), (6,))

    def fused_step():
        for layer in stack:
            for grp in GROUPS:
                if len(grp) == 1:
                    e = layer[grp[0]]
                    e["kern"].multiply(e["x"], out=e["y"])
                else:
                    es = [layer[i] for i in grp]
                    multiply_grouped([e["kern"] for e in es], es[0]["x"], outs=[e["y"] for e in es])

    def separate_step():
        for e in flat:
            e["kern"].multiply(e["x"], out=e["y"])

    g_fused = capture(fused_step)
    ms = time_graph(g_fused, args.steps, args.warmup)
    value = bf16_bytes / (ms * 1e-3) / 1e9
    log(f"[bench] fused step (grouped launches) {ms:.3f} ms -> {value:.1f} GB/s BF16-equivalent")
    del g_fused
    g_sep = capture(separate_step)
    ms_sep = time_graph(g_sep, args.steps, args.warmup)
    log(f"[bench] fused step (one launch per GEMV) {ms_sep:.3f} ms -> {bf16_bytes / (ms_sep * 1e-3) / 1e9:.1f} GB/s")
    del g_sep

    result = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "ms_per_step_median": round(ms.median, 4),
        "ms_per_step_p10": round(ms.p10, 4),
        "ms_per_step_p90": round(ms.p90, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": f"gemma-2-2b linear stack: {args.layers} layers x 7 projections, batch 1",
            "gemvs_per_step": len(flat),
            "launches_per_step": len(stack) * len(GROUPS),
            "weights_per_step": weights,
            "se12_bytes_per_step": se12_bytes,
            "bf16_bytes_per_step": bf16_bytes,
            "batch": 1,
        },
    }

    result["one_launch_per_gemv"] = {"ms_per_step": round(ms_sep, 4), "gbps": round(bf16_bytes / (ms_sep * 1e-3) / 1e9, 1),
                                     "launches_per_step": len(flat)}

    # dominant kernel: the 26 down_proj GEMVs (2304x9216, 31.9 MB of streams
    # each, 830 MB in all: every launch reads cold HBM), timed on the replay
    # stream with HIP events around `steps` replays of a 26-launch graph
    down = [layer[6] for layer in stack]
    g_down = capture(lambda: [e["kern"].multiply(e["x"], out=e["y"]) for e in down])
    ms_down = time_graph(g_down, args.steps, args.warmup)
    us_launch = ms_down * 1e3 / len(down)
    bytes_launch = down[0]["enc"].byte_size() + down[0]["k"] * 2 + down[0]["n"] * 4
    achieved = bytes_launch / (us_launch * 1e-6) / 1e9
    launch = down[0]["kern"].default_launch(1)
    traffic = None
    if os.path.exists(TRAFFIC_FILE):
        with open(TRAFFIC_FILE) as f:
            traffic = json.load(f).get("traffic_bytes_per_launch")
    result["roofline"] = {
        "bound": "hbm",
        "achieved": round(achieved, 1),
        "peak": HBM_PEAK_GBPS,
        "unit": "GB/s",
        "frac": round(achieved / HBM_PEAK_GBPS, 4),
        "traffic": traffic,
        "kernel": "se12::gemv_kernel (fused SE12 decode + GEMV, batch 1)",
        "shape": [down[0]["n"], down[0]["k"]],
        "launch": {"threads_per_block": launch.threads_per_block.value, "blocks": launch.blocks.value},
        "avg_launch_us": round(us_launch, 3),
        "launch_stats": ms_down.stats_us(len(down)),
        "peak_published": HBM_PEAK_GBPS,
        "peak_from_device": round(props.hbm_peak_gbps, 1),
        "frac_of_device_peak": round(achieved / props.hbm_peak_gbps, 4),
        "algorithmic_bytes_per_launch": bytes_launch,
        "bf16_equiv_gbps": round(2 * down[0]["n"] * down[0]["k"] / (us_launch * 1e-6) / 1e9, 1),
    }
    log(f"[bench] down_proj launches: {us_launch:.2f} us each -> {achieved:.0f} GB/s of SE12 streams")
    del g_down

    # the launch that takes the largest share of the step: the grouped gate/up
    # product (2 x 9216x2304, 63.9 MB of streams per launch), timed the same
    # way over its 26 layers and reported beside the down_proj roofline
    gu = [[layer[4], layer[5]] for layer in stack]
    g_gu = capture(lambda: [multiply_grouped([e["kern"] for e in es], es[0]["x"], outs=[e["y"] for e in es])
                            for es in gu])
    ms_gu = time_graph(g_gu, args.steps, args.warmup)
    del g_gu
    us_gu = ms_gu * 1e3 / len(gu)
    bytes_gu = sum(e["enc"].byte_size() + e["n"] * 4 for e in gu[0]) + gu[0][0]["k"] * 2
    result["roofline_step_dominant"] = {
        "kernel": "se12::gemv_kernel, grouped gate/up (2 matrices per launch, batch 1)",
        "shape": [[e["n"], e["k"]] for e in gu[0]],
        "avg_launch_us": round(us_gu, 3),
        "algorithmic_bytes_per_launch": bytes_gu,
        "achieved": round(bytes_gu / (us_gu * 1e-6) / 1e9, 1),
        "peak": HBM_PEAK_GBPS,
        "frac": round(bytes_gu / (us_gu * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4),
        "share_of_step": round(us_gu * len(gu) / (ms * 1e3), 4),
    }
    log(f"[bench] gate/up launches: {us_gu:.2f} us each -> {bytes_gu / (us_gu * 1e-6) / 1e9:.0f} GB/s")

    if not args.only_fused:
        # hipBLASLt BF16 with the same grouping: one GEMV over concatenated weights
        cat = []
        for layer in stack:
            cat.append([(torch.cat([layer[i]["w"] for i in grp]) if len(grp) > 1 else layer[grp[0]]["w"], layer[grp[0]]["x"])
                        for grp in GROUPS])

        def bf16_step():
            for layer in cat:
                for w, x in layer:
                    torch.nn.functional.linear(x, w)

        def bf16_separate_step():
            for e in flat:
                torch.nn.functional.linear(e["x"], e["w"])

        g_bf16 = capture(bf16_step)
        ms_bf16 = time_graph(g_bf16, args.steps, args.warmup)
        del g_bf16
        g_bf16s = capture(bf16_separate_step)
        ms_bf16_sep = time_graph(g_bf16s, args.steps, args.warmup)
        del g_bf16s, cat
        raw = [[RawBf16MatVecKernel(e["w"], max_batch=1) for e in layer] for layer in stack]

        def raw_step():
            for layer, rl in zip(stack, raw):
                for grp in GROUPS:
                    multiply_grouped([rl[i] for i in grp], layer[grp[0]]["x"], outs=[layer[i]["y"] for i in grp])

        g_raw = capture(raw_step)
        ms_raw = time_graph(g_raw, args.steps, args.warmup)
        result["bf16_hipblaslt"] = {"ms_per_step": round(ms_bf16, 4), "gbps": round(bf16_bytes / (ms_bf16 * 1e-3) / 1e9, 1),
                                   "speedup_of_se12": round(ms_bf16 / ms, 4),
                                   "one_launch_per_gemv_ms": round(ms_bf16_sep, 4),
                                   "one_launch_per_gemv_speedup_of_se12": round(ms_bf16_sep / ms_sep, 4)}
        result["raw_bf16_twin"] = {"ms_per_step": round(ms_raw, 4), "gbps": round(bf16_bytes / (ms_raw * 1e-3) / 1e9, 1),
                                  "speedup_of_se12": round(ms_raw / ms, 4)}
        log(f"[bench] hipBLASLt bf16 {ms_bf16:.3f} ms (one launch per GEMV {ms_bf16_sep:.3f} ms), raw twin {ms_raw:.3f} ms")
        del g_raw, raw

    if not args.no_per_shape:
        flush_buf = torch.zeros(1 << 28, dtype=torch.float32, device=dev)  # 1 GiB > 4 x (L2 + MALL)

        def flush():
            evict_caches(flush_buf)

        per_shape = {}
        for pi, (name, n, k, _) in enumerate(PROJECTIONS):
            col = [layer[pi] for layer in stack]
            g = capture(lambda col=col: [e["kern"].multiply(e["x"], out=e["y"]) for e in col])
            ms_s = time_graph(g, 10, 3, flush=flush)
            us = ms_s * 1e3 / len(col)
            lc = col[0]["kern"].default_launch(1)
            per_shape[name] = {"shape": [n, k], "us": round(us, 3), "bf16_equiv_gbps": round(2 * n * k / (us * 1e-6) / 1e9, 1),
                               "se12_gbps": round(col[0]["enc"].byte_size() / (us * 1e-6) / 1e9, 1),
                               "launch": [lc.threads_per_block.value, lc.blocks.value]}
            per_shape[name].update(ms_s.stats_us(len(col)))
            if not args.only_fused:
                gb = capture(lambda col=col: [torch.nn.functional.linear(e["x"], e["w"]) for e in col])
                us_b = time_graph(gb, 10, 3, flush=flush) * 1e3 / len(col)
                rk = [RawBf16MatVecKernel(e["w"], max_batch=1) for e in col]
                yr = [torch.empty_like(e["y"]) for e in col]
                gr = capture(lambda col=col, rk=rk, yr=yr: [r.multiply(e["x"], out=y) for r, e, y in zip(rk, col, yr)])
                us_r = time_graph(gr, 10, 3, flush=flush) * 1e3 / len(col)
                del gb, gr, rk, yr
                per_shape[name]["bf16_hipblaslt_us"] = round(us_b, 3)
                per_shape[name]["raw_twin_us"] = round(us_r, 3)
                per_shape[name]["speedup_vs_faster_baseline"] = round(min(us_b, us_r) / us, 4)
            log(f"[bench] {name} {n}x{k}: {per_shape[name]}")
        result["per_shape"] = per_shape
        del flush_buf
        if not args.only_fused and not args.no_model:
            result["model"] = roofline_model(dev, props, per_shape)

    if not args.no_batch_sweep:
        del stack, flat
        torch.cuda.empty_cache()
        result["batch_sweep"] = batch_sweep(dev)
        torch.cuda.empty_cache()
        # the step's own dominant shape, Gemma-2-2B down_proj 2304x9216, from
        # the batches whose x no longer fits a block's LDS whole (9+)
        result["batch_sweep_down_proj"] = batch_sweep(dev, batches=(8, 9, 16, 24, 32), n=2304, k=9216, seed=19_000)
        torch.cuda.empty_cache()
    if not args.no_decode:
        result["decode_only"] = decode_only(dev)
    if not args.no_stress:
        result["stress"] = stress(dev)
    if not args.no_e2e:
        result["e2e"] = e2e_decode(dev)
        result["decode_tok_s"] = result["e2e"]["se12"]["decode_tok_s"]

    if not args.no_micro:
        from se12_amd import micro

        m, v = micro.run(device=dev, log=log)
        paths = micro.write_reports(m, v, args.reports)
        result["micro"] = {
            "verdict": v["verdict"], "per_batch": {b: e["verdict"] for b, e in v["per_batch"].items()},
            "peak_copy_bandwidth_gbps": round(v["peak_copy_bandwidth_gbps"], 1),
            "copy_traffic_gbps": round(v["copy_traffic_gbps"], 1),
            "rows": [{"shape": row["shape"], "batch": row["batch_size"],
                      **{n: r.get("median_microseconds") and round(r["median_microseconds"], 3)
                         for n, r in row["results"].items()},
                      **({"ratio": round(row["shape_verdict"]["ratio"], 4),
                          "baseline": row["shape_verdict"]["baseline"],
                          "baseline_fraction_of_peak": round(row["shape_verdict"]["baseline_fraction_of_peak"], 3),
                          "verdict": row["shape_verdict"]["verdict"]} if row["shape_verdict"] else {})}
                     for row in m["results"]],
            "files": [str(x) for x in paths],
        }
    if not args.no_cpu_baseline:
        log("[bench] cpu baseline ...")
        result["cpu_baseline"] = cpu_baseline()
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
