"""KernelCompiler behind the reference's port, as an ahead-of-time loader.

The reference compiles CUDA C at run time: `KernelCompiler.compile(CudaSource,
CompileTarget) -> CompiledKernelHandle` (lws/application/ports/gpu/
kernel_compiler.py:16-27), implemented with NVRTC, whose handle's
`function(name)` returns a kernel to launch (lws/adapters/cuda/
nvrtc_compiler.py:31-55). The target is SASS or PTX for an sm_XY number,
chosen from the device's compute capability (lws/domain/device/
decisions.py:70-84).

Here every kernel is compiled ahead of time by hipcc into
libse12_gfx950.so, for gfx950 code objects only. `AotKernelCompiler.compile`
therefore compiles nothing: it checks that the library holds code for the
target, loads it, and returns a handle whose `function(name)` gives the
library's C entry point that replaces the named reference kernel
(`lws_gemv_se12` -> `se12_gemv`, ...). The source text the reference passes
is accepted and kept for inspection, never compiled.
"""

from __future__ import annotations

import dataclasses
import enum
import os
import pathlib
from typing import Any

# gfx targets the library holds code objects for (se12_amd/csrc/build.py)
LIBRARY_ARCHES = ("gfx950",)


def arch_number(arch: str) -> int:
    """A gfx architecture as HIP's major * 10 + minor: gfx950 -> 95."""
    d = arch.split(":", 1)[0].strip().removeprefix("gfx")
    return int(d[:-2]) * 10 + int(d[-2], 16)


# the reference's integer compile-target arch -> the library's gfx target
ARCH_BY_NUMBER = {arch_number(a): a for a in LIBRARY_ARCHES}
CACHE_DIR_ENV_VAR = "LWS_CACHE_DIR"

# reference kernel name -> the C entry point that replaces it
KERNEL_ENTRY_POINTS = {
    "lws_gemv_se12": "se12_gemv",          # kernels/gemv_se12.cu:50-64
    "lws_gemv_raw_bf16": "se12_gemv",      # kernels/gemv_raw_bf16.cu:18-25 (a handle bound with se12_bind_raw_bf16)
    "lws_se12_decode": "se12_decode",      # kernels/se12_decode.cu:12-22
}


class UnsupportedDeviceError(ValueError):
    """The device cannot be targeted: the library holds no code object for
    its architecture (the reference's error of the same name,
    lws/domain/device/decisions.py:29-31)."""


class CompileTargetKind(enum.Enum):
    """gfx code objects built ahead of time (the reference's SASS / PTX,
    decisions.py:44-46, have no counterpart: no intermediate form is shipped)."""

    CODE_OBJECT = "code-object"


@dataclasses.dataclass(frozen=True)
class GfxArch:
    """A gfx target name without its feature suffixes, e.g. "gfx950"."""

    value: str


@dataclasses.dataclass(frozen=True)
class CompileTarget:
    kind: CompileTargetKind
    arch: GfxArch


@dataclasses.dataclass(frozen=True)
class KernelSource:
    """What a caller asks `compile` for. The reference passes CUDA C source
    text (`CudaSource`, kernel_compiler.py:16-18); any object with a `value`
    is accepted and kept, none is compiled."""

    value: str


def base_arch(arch_name: str) -> str:
    """"gfx950:sramecc+:xnack-" -> "gfx950"."""
    return arch_name.split(":", 1)[0].strip()


def choose_compile_target(arch_name: str) -> CompileTarget:
    """The code-object target for a device's gfx architecture (hipDeviceProp's
    gcnArchName); raises UnsupportedDeviceError when the library holds no
    code for it (decisions.py:70-84 refuses an unsupported device the same
    way)."""
    arch = base_arch(arch_name)
    if arch not in LIBRARY_ARCHES:
        raise UnsupportedDeviceError(
            f"the SE12 library holds code objects for {', '.join(LIBRARY_ARCHES)} only, not {arch or arch_name!r}")
    return CompileTarget(kind=CompileTargetKind.CODE_OBJECT, arch=GfxArch(arch))


def device_compile_target(device: int | None = None) -> CompileTarget:
    """choose_compile_target for a HIP device (default: the current one)."""
    from .hip import HipGpuProbe

    return choose_compile_target(HipGpuProbe(device).facts().arch)


class AotCompiledKernelHandle:
    """CompiledKernelHandle over the loaded library (nvrtc_compiler.py:31-40)."""

    def __init__(self, library: Any, target: CompileTarget, source: Any) -> None:
        self.library = library
        self.target = target
        self.source = source

    def function(self, name: str):
        """The C entry point that replaces reference kernel `name`, or the
        library symbol `name` itself."""
        symbol = KERNEL_ENTRY_POINTS.get(name, name)
        fn = getattr(self.library, symbol, None)
        if fn is None:
            raise KeyError(f"the SE12 library exports no {symbol!r} (asked for {name!r})")
        return fn


class AotKernelCompiler:
    """KernelCompiler port: loads libse12_gfx950.so for a supported target.

    `cache_directory` keeps the reference's meaning for the callers that
    store per-GPU files beside compiled kernels ($LWS_CACHE_DIR, default
    ~/.cache/lws; nvrtc_compiler.py:43-49,63-69); nothing is cached here."""

    def __init__(self) -> None:
        raw = os.environ.get(CACHE_DIR_ENV_VAR)
        self.cache_directory = pathlib.Path(raw) if raw else pathlib.Path.home() / ".cache" / "lws"

    def compile(self, source: Any, target: Any) -> AotCompiledKernelHandle:
        """`target` is this module's CompileTarget, or the reference's SASS
        target (kind value "sass", integer arch) that its
        `choose_compile_target(capability, nvrtc_targets, ForcePtx(False))`
        (decisions.py:70-84) picks from HipGpuProbe.properties(): the
        capability and targets there encode gfx950 as 95. A PTX target, or an
        architecture the library holds no code object for, is refused."""
        kind = getattr(target, "kind", None)
        arch = getattr(getattr(target, "arch", None), "value", None)
        if getattr(kind, "value", None) == "sass" and isinstance(arch, int):
            arch = ARCH_BY_NUMBER.get(arch)
            if arch is None:
                raise UnsupportedDeviceError(f"the SE12 library holds no code object for sm_{target.arch.value}")
        elif kind is not CompileTargetKind.CODE_OBJECT or not isinstance(arch, str):
            raise UnsupportedDeviceError(
                f"target {target!r} is not a gfx code-object target (use se12_amd.compiler.choose_compile_target)")
        if base_arch(arch) not in LIBRARY_ARCHES:
            raise UnsupportedDeviceError(f"the SE12 library holds no code object for {arch}")
        from . import _native

        return AotCompiledKernelHandle(_native.lib(), target, source)
