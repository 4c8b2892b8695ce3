"""The GPU adapters with the reference's constructor signatures.

The reference's composition roots (its microbenchmark, tuner and
calibration probe: lws/bench/micro.py:110-113, lws/tune.py:92-104,
lws/adapters/cuda/calibration_probe.py:47,78) and its GPU tests
(tests/test_spec_gpu_decode.py:101-102) build the adapters as

    RawBf16MatVecKernel(compiler, target, weights, sm_count)
    Se12MatVecKernel(compiler, target, tensor, sm_count, extra_decode_ops=0)
    CudaSe12WeightDecoder(compiler, target)

(lws/adapters/cuda/gemv.py:146,183; lws/adapters/cuda/se12_decoder.py:48).
The classes here take exactly those arguments and run the library's
kernels: `compiler` is an `AotKernelCompiler` (any object with the port's
`compile(source, target)`), `target` a `CompileTarget` from
`choose_compile_target`, and `sm_count` (an int or the reference's
`SmCount`) becomes the compute-unit count of the default launch.

`multiply(activations, launch=None)` keeps the port's meaning
(lws/application/ports/gpu/matvec_kernel.py:18-23). A `launch` built with
this package's `se12_amd.launch.LaunchConfiguration` is this kernel's
configuration (waves per block, tile rows x K splits); any other object with
`threads_per_block.value` and `blocks.value` - the reference's own
`LaunchConfiguration`, as its tuner and heuristic build them - carries the
reference's meaning and is translated by
`se12_amd.launch.from_reference_configuration`, with this adapter's
`sm_count` as the compute-unit count the library's kernel choice uses.

The reference's other GPU ports are built the same way:

    CudaGpuProbe(device_index=None)             -> HipGpuProbe
    CudaBenchmarkTimer(device_index, l2_size)   -> HipBenchmarkTimer
    FilesystemTuningCache(directory, gpu_slug)  -> FilesystemTuningCache

(lws/adapters/cuda/gpu_probe.py:59-80, lws/adapters/cuda/benchmark_timer.py:
20-66, lws/adapters/filesystem/tuning_cache.py:31-59). They return the port's
value objects (se12_amd.ports), and `tune_launch(gpu_slug, requests,
evaluators, cache)` takes the reference's arguments
(lws/application/gpu/tune_launch.py:43-48).
"""

from __future__ import annotations

from typing import Any

import torch

from . import _native as nat
from . import hip
from .compiler import KernelSource
from .launch import LaunchConfiguration, from_reference_configuration
from .tune import FilesystemTuningCache, tune_launch  # noqa: F401  (re-exported ports)

HipGpuProbe = hip.HipGpuProbe
HipBenchmarkTimer = hip.HipBenchmarkTimer


def _count(sm_count: Any) -> int:
    value = getattr(sm_count, "value", sm_count)
    if isinstance(value, bool) or not isinstance(value, int) or value < 1:
        raise ValueError(f"sm_count must be a positive count, got {sm_count!r}")
    return value


def _native_launch(kernel: hip._GemvBase, activations: torch.Tensor, launch: Any):
    if launch is None or isinstance(launch, LaunchConfiguration):
        return launch
    x = activations.unsqueeze(0) if activations.dim() == 1 else activations
    return from_reference_configuration(launch, kernel.rows, kernel.cols, x.shape[0],
                                        float32_activations=x.dtype == torch.float32,
                                        aligned_x=x.is_contiguous() and x.data_ptr() % 16 == 0,
                                        compute_units=kernel.sm_count)


class _ReferenceSignature:
    """The compile step and the launch translation both adapters share."""

    _entry = ""

    def _compile(self, compiler: Any, target: Any, sm_count: Any) -> None:
        self.compiled = compiler.compile(KernelSource(self._entry), target)
        self.kernel_function = self.compiled.function(self._entry)
        self.target = target
        self.sm_count = _count(sm_count)

    def _set_compute_units(self) -> None:
        nat.check(nat.lib().se12_set_compute_units(self.handle.raw, self.sm_count))

    def multiply(self, activations: torch.Tensor, launch: Any = None, out: torch.Tensor | None = None) -> torch.Tensor:
        return super().multiply(activations, launch=_native_launch(self, activations, launch), out=out)


class Se12MatVecKernel(_ReferenceSignature, hip.Se12MatVecKernel):
    """Fused SE12 decode + GEMV bound to one SE12 matrix, built as the
    reference builds it (gemv.py:180-194). `tensor` is the reference
    container (`Se12Tensor`, uploaded once) or an `Se12DeviceTensor`.
    `extra_decode_ops` is the reference's decode-cost calibration knob
    (extra ALU work per weight, kernels/gemv_se12.cu:24-45); this library
    ships no such variant, so only 0 is accepted."""

    _entry = "lws_gemv_se12"

    def __init__(self, compiler: Any, target: Any, tensor: Any, sm_count: Any, extra_decode_ops: int = 0,
                 max_batch: int = nat.MAX_BATCH) -> None:
        if extra_decode_ops != 0:
            raise ValueError("extra_decode_ops: the library has no decode-cost calibration variant (only 0)")
        self._compile(compiler, target, sm_count)
        hip.Se12MatVecKernel.__init__(self, tensor, max_batch=max_batch)
        self._set_compute_units()


class RawBf16MatVecKernel(_ReferenceSignature, hip.RawBf16MatVecKernel):
    """The raw-BF16 twin bound to a [N, K] BF16 device matrix, built as the
    reference builds it (gemv.py:143-155)."""

    _entry = "lws_gemv_raw_bf16"

    def __init__(self, compiler: Any, target: Any, weights: torch.Tensor, sm_count: Any,
                 max_batch: int = nat.MAX_BATCH) -> None:
        self._compile(compiler, target, sm_count)
        hip.RawBf16MatVecKernel.__init__(self, weights, max_batch=max_batch)
        self._set_compute_units()


class Se12WeightDecoder(hip.HipSe12WeightDecoder):
    """WeightDecoder built as the reference's CudaSe12WeightDecoder(compiler,
    target) (se12_decoder.py:45-76): decode, decode_rows, decode_to_device."""

    def __init__(self, compiler: Any, target: Any) -> None:
        super().__init__()
        self.compiled = compiler.compile(KernelSource("lws_se12_decode"), target)
        self.kernel_function = self.compiled.function("lws_se12_decode")
        self.target = target
