"""The device, timer and tuning-cache ports on the GPU, driven in the call
pattern of the reference's composition roots (lws/bench/micro.py:50-66,
lws/tune.py:38-56, lws/application/gpu/run_microbenchmark.py:54-117):

    properties = probe.properties()
    sm_count = properties.identity_and_compute.compute.sm_count
    l2_size  = properties.memory_and_nvrtc.memory.characteristics.l2_size
    target   = choose_compile_target(capability, nvrtc_targets, ForcePtx(False))
    timer    = CudaBenchmarkTimer(0, l2_size)
    peak     = timer.measure_peak_copy_bandwidth()
    samples  = timer.time_operation(operation, RunCounts(warmup, timed))
    tune_launch(gpu_slug, requests, evaluators, cache)

The reference's own value types are restated below as plain stand-ins (the
ports read attributes only). The compile-target rule is the reference's
(lws/domain/device/decisions.py:63-103) restated in a few lines."""

from __future__ import annotations

import dataclasses

import numpy as np
import pytest
import torch

from gpu_helpers import REL_TOL, max_rel_error, normal_case, to_device
from oracle import se12_codec as o

pytestmark = pytest.mark.gpu


@dataclasses.dataclass(frozen=True)
class RunCounts:
    warmup: int
    timed: int


@dataclasses.dataclass(frozen=True)
class Kind:
    value: str


@dataclasses.dataclass(frozen=True)
class ComputeArch:
    value: int


@dataclasses.dataclass(frozen=True)
class CompileTarget:
    kind: Kind
    arch: ComputeArch


def reference_compile_target(capability, nvrtc_targets) -> CompileTarget:
    """SASS for the device's own arch when the targets list it, else PTX for
    the highest listed arch below it (decisions.py:70-103, force_ptx off)."""
    arch = capability.major * 10 + capability.minor
    if arch in nvrtc_targets.values:
        return CompileTarget(Kind("sass"), ComputeArch(arch))
    below = [t for t in nvrtc_targets.values if t <= arch]
    if not below:
        raise ValueError("unsupported device")
    return CompileTarget(Kind("ptx"), ComputeArch(max(below)))


@dataclasses.dataclass(frozen=True)
class WeightShape:
    output_rows: int
    k: int


@dataclasses.dataclass(frozen=True)
class BatchSize:
    value: int


@dataclasses.dataclass(frozen=True)
class TuneRequest:
    weight_shape: WeightShape
    batch: BatchSize


def median_us(samples) -> float:
    return float(np.median(np.asarray(samples.values, dtype=np.float64)))


def test_probe_reports_the_reference_properties(gpu):
    from se12_amd.adapters import HipGpuProbe

    probe = HipGpuProbe(gpu.index)
    facts = probe.facts()
    props = probe.properties()
    ic, mn = props.identity_and_compute, props.memory_and_nvrtc
    assert ic.identity.name.value == facts.name and ic.identity.slug.value == facts.slug
    assert ic.compute.sm_count.value == facts.compute_units == torch.cuda.get_device_properties(gpu).multi_processor_count
    cap = ic.compute.capability
    tp = torch.cuda.get_device_properties(gpu)
    assert (cap.major, cap.minor) == (tp.major, tp.minor) == facts.capability
    assert mn.memory.characteristics.l2_size.value == facts.l2_bytes > 0
    assert mn.memory.characteristics.bandwidth.value == pytest.approx(facts.hbm_peak_gbps)
    assert 0 < mn.memory.vram.free.value <= mn.memory.vram.total.value
    assert mn.nvrtc_targets.values == (cap.major * 10 + cap.minor,)
    sv = probe.software_versions()
    assert sv.core.torch_and_cupy.torch.version == torch.__version__
    assert sv.nvrtc.targets == mn.nvrtc_targets and sv.nvrtc.version
    assert isinstance(sv.core.toolchain.driver, str) and isinstance(sv.core.toolchain.cuda_runtime, str)
    assert probe.smoke_test().supported is True


def test_reference_compile_target_builds_the_adapters(gpu):
    """The target the reference's rule picks from these properties compiles,
    and the adapters built from it multiply within REL_TOL of the oracle."""
    from se12_amd.adapters import HipGpuProbe, Se12MatVecKernel
    from se12_amd.compiler import AotKernelCompiler

    props = HipGpuProbe(gpu.index).properties()
    compute = props.identity_and_compute.compute
    target = reference_compile_target(compute.capability, props.memory_and_nvrtc.nvrtc_targets)
    assert target.kind.value == "sass"
    rows, cols = 256, 2304
    bits, enc = normal_case(rows, cols, seed=5)
    kern = Se12MatVecKernel(AotKernelCompiler(), target, to_device(enc, gpu), compute.sm_count)
    xb = o.normal_bf16(1, cols, seed=6, std=1.0)
    y = kern.multiply(torch.from_numpy(o.bf16_bits_to_f32(xb)).to(gpu))
    assert max_rel_error(y, o.gemv_reference(enc, o.bf16_bits_to_f32(xb))) <= REL_TOL


def test_timer_times_operations_and_counts_the_copy_once(gpu):
    from se12_amd.adapters import HipBenchmarkTimer, HipGpuProbe
    from se12_amd.hip import RawBf16MatVecKernel, Se12MatVecKernel

    props = HipGpuProbe(gpu.index).properties()
    timer = HipBenchmarkTimer(gpu.index, props.memory_and_nvrtc.memory.characteristics.l2_size)
    assert timer.l2_size == props.memory_and_nvrtc.memory.characteristics.l2_size.value
    peak = timer.measure_peak_copy_bandwidth()
    traffic = timer.measure_copy_traffic_gbps()
    # the port's peak counts the copied bytes once, the traffic figure twice
    assert 0.8 < 2 * peak.value / traffic < 1.25, (peak.value, traffic)
    assert peak.value < props.memory_and_nvrtc.memory.characteristics.bandwidth.value

    rows, cols = 2304, 9216
    bits, enc = normal_case(rows, cols, seed=0)
    fused = Se12MatVecKernel(to_device(enc, gpu), max_batch=1)
    raw = RawBf16MatVecKernel(torch.from_numpy(bits.astype(np.int16)).to(gpu).view(torch.bfloat16), max_batch=1)
    x = torch.from_numpy(o.bf16_bits_to_f32(o.normal_bf16(1, cols, seed=1, std=1.0))).to(gpu)
    counts = RunCounts(warmup=3, timed=12)
    s_fused = timer.time_operation(lambda: fused.multiply(x), counts)
    s_raw = timer.time_operation(lambda: raw.multiply(x), counts)
    assert len(s_fused.values) == 12 and len(s_raw.values) == 12
    assert all(v > 0 for v in s_fused.values + s_raw.values)
    # the reference's verdict arithmetic over these samples
    # (run_microbenchmark.py:66-117, statistics.py:54-62, verdict.py:40-62)
    moved = rows * cols * 2 + 1 * cols * 4
    base_gbps = moved / (median_us(s_raw) * 1e-6) / 1e9
    fraction = base_gbps / peak.value
    ratio = median_us(s_fused) / median_us(s_raw)
    verdict = "INCONCLUSIVE" if fraction < 0.70 else ("GO" if ratio <= 0.95 else "NO-GO")
    assert verdict in ("GO", "NO-GO", "INCONCLUSIVE") and fraction > 0


class DefaultMatchEvaluator:
    """A CandidateEvaluator in the manner of the reference's tuner
    (lws/adapters/cuda/candidate_evaluator.py:31-60): a kernel bound to its
    weights, timed over repeated launches with a configuration, passing when
    its output is within 1e-4 x max(|ref|, 1) of the kernel's own
    default-launch output."""

    def __init__(self, kernel, activations: torch.Tensor) -> None:
        self.kernel, self.activations = kernel, activations
        self.reference = kernel.multiply(activations)

    def evaluate(self, configuration):
        import time

        for _ in range(2):
            self.kernel.multiply(self.activations, configuration)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(5):
            out = self.kernel.multiply(self.activations, configuration)
        torch.cuda.synchronize()
        us = (time.perf_counter() - t0) / 5 * 1e6
        rel = ((out - self.reference).abs() / self.reference.abs().clamp_min(1.0)).max().item()

        @dataclasses.dataclass(frozen=True)
        class TimingAndAccuracy:
            median_latency_microseconds: float
            passes_accuracy_check: bool

        return TimingAndAccuracy(us, rel <= 1e-4)


@dataclasses.dataclass(frozen=True)
class EvaluatorPair:
    raw: object
    fused: object


def test_tuner_with_reference_style_evaluators_over_the_adapters(gpu, tmp_path):
    """The tuner's composition as lws.tune builds it (lws/tune.py:38-99):
    adapters built with the reference's constructor arguments, one evaluator
    per kernel, the cache port; every tuned configuration then runs through
    the adapter within REL_TOL of the oracle, raw and fused bit-identical
    under the order-matched one."""
    from se12_amd.adapters import (FilesystemTuningCache, HipGpuProbe, RawBf16MatVecKernel, Se12MatVecKernel,
                                   tune_launch)
    from se12_amd.compiler import AotKernelCompiler

    props = HipGpuProbe(gpu.index).properties()
    compute = props.identity_and_compute.compute
    target = reference_compile_target(compute.capability, props.memory_and_nvrtc.nvrtc_targets)
    compiler = AotKernelCompiler()
    rows, cols = 768, 2304
    bits, enc = normal_case(rows, cols, seed=71)
    fused = Se12MatVecKernel(compiler, target, to_device(enc, gpu), compute.sm_count)
    raw = RawBf16MatVecKernel(compiler, target, torch.from_numpy(bits.astype(np.int16)).to(gpu).view(torch.bfloat16),
                              compute.sm_count)
    xs = {b: torch.from_numpy(o.bf16_bits_to_f32(o.normal_bf16(b, cols, seed=72 + b, std=1.0))).to(gpu)
          for b in (1, 4, 8)}   # FP32, as lws.tune feeds them: at 8 rows the dot2 kernel, MFMA configurations refused

    def evaluators(req):
        x = xs[req.batch.value]
        return EvaluatorPair(raw=DefaultMatchEvaluator(raw, x), fused=DefaultMatchEvaluator(fused, x))

    slug = props.identity_and_compute.identity.slug
    cache = FilesystemTuningCache(tmp_path, slug)
    reqs = [TuneRequest(WeightShape(rows, cols), BatchSize(b)) for b in (1, 4, 8)]
    tf = tune_launch(slug, reqs, evaluators, cache)
    assert cache.load() == tf and len(tf.entries.items) == 3
    for e in tf.entries.items:
        x = xs[e.key.batch.value]
        ref = o.gemv_reference(enc, x.cpu().numpy())
        c = e.configurations
        for cfg in (c.independent.fused, c.order_matched):
            assert max_rel_error(fused.multiply(x, cfg), ref) <= REL_TOL
        assert torch.equal(fused.multiply(x, c.order_matched), raw.multiply(x, c.order_matched))


def test_tuner_writes_through_the_cache_port(gpu, tmp_path):
    from se12_amd.adapters import FilesystemTuningCache, HipGpuProbe, tune_launch
    from se12_amd.tune import gpu_evaluators, tuning_lookup
    from se12_amd.hip import Se12MatVecKernel, encode_on_device

    props = HipGpuProbe(gpu.index).properties()
    slug = props.identity_and_compute.identity.slug
    cache = FilesystemTuningCache(tmp_path, slug)
    reqs = [TuneRequest(WeightShape(512, 2304), BatchSize(b)) for b in (1, 8)]
    tf = tune_launch(slug, reqs, gpu_evaluators(gpu, samples=2), cache)
    assert len(tf.entries.items) == 2
    back = cache.load()
    assert back == tf
    # the tuned order-matched launch runs and stays within REL_TOL
    w = (torch.randn((512, 2304), device=gpu, generator=torch.Generator(device=gpu).manual_seed(3)) * 0.02).to(torch.bfloat16)
    kern = Se12MatVecKernel(encode_on_device(w))
    for b in (1, 8):
        cfg = tuning_lookup(back, "order_matched")(512, 2304, b)
        assert cfg is not None
        x = torch.randn((b, 2304), device=gpu).to(torch.bfloat16)
        y = kern.multiply(x, launch=cfg)
        ref = (x.float() @ w.float().t()).double()
        assert float(((y.double() - ref).abs() / ref.abs().clamp_min(1.0)).max()) <= REL_TOL


@pytest.mark.parametrize("batch", [24, 32])
def test_reference_launch_on_a_smaller_gpu_count(gpu, batch):
    """An adapter told of 132 compute units runs the library's kernel choice
    for 132 (at 4096x3584, batch 24 / 32: the resident-x kernel with two K
    splits, where 256 CUs keep 16 rows of x unsplit) and translates reference
    launches for that choice."""
    from test_adapters_cpu import RefBlocks, RefLaunch, RefThreads

    from se12_amd.adapters import Se12MatVecKernel
    from se12_amd.compiler import AotKernelCompiler, device_compile_target

    rows, cols = 4096, 3584
    bits, enc = normal_case(rows, cols, seed=40)
    kern = Se12MatVecKernel(AotKernelCompiler(), device_compile_target(gpu.index), to_device(enc, gpu), 132)
    xb = o.normal_bf16(batch, cols, seed=41, std=1.0)
    x = torch.from_numpy(xb.astype(np.int16)).to(gpu).view(torch.bfloat16)
    ref = o.gemv_reference(enc, o.bf16_bits_to_f32(xb))
    for launch in (None, RefLaunch(RefThreads(256), RefBlocks(-(-rows * batch // 8))),
                   RefLaunch(RefThreads(512), RefBlocks(-(-rows * batch // 16)))):
        y = kern.multiply(x, launch)
        torch.cuda.synchronize()
        assert max_rel_error(y, ref) <= REL_TOL, launch
