"""Value types of the reference's GPU ports, so that the HIP adapters hand the
reference's composition roots exactly the objects they read.

The reference's ports (lws/application/ports/gpu/*.py) exchange small frozen
value objects. Its entry points read them by attribute path, e.g.

    properties.identity_and_compute.compute.sm_count.value
    properties.memory_and_nvrtc.memory.characteristics.l2_size.value
    timer.time_operation(op, RunCounts(warmup, timed)).values
    timer.measure_peak_copy_bandwidth().value

(lws/bench/micro.py:50-66, lws/tune.py:38-56). The classes below have the
same names, fields and nesting as the reference's:

    DeviceProperties and its parts   lws/domain/device/properties.py:11-107
    SoftwareVersions and its parts   lws/domain/device/properties.py:110-165
    SupportVerdict                   lws/domain/device/decisions.py:228-231
    LatencySamples, RunCounts        lws/domain/benchmark/statistics.py:27-32,70-73
    TuningFile and its parts         lws/application/ports/gpu/tuning_cache.py:20-68

Any object with the same attributes works in their place (the reference's
own instances included): the adapters read attributes, never types.

AMD facts fill the NVIDIA-named fields:
- `ComputeCapability(major, minor)` is the gfx architecture's major and minor
  digits as HIP reports them (gfx950 -> 9, 5), so the reference's
  `arch_number` gives 95;
- `NvrtcTargets` holds the architecture numbers, in that encoding, that the
  ahead-of-time library has code objects for (gfx950 -> 95);
- `MemoryCharacteristics.bandwidth` is the peak from the memory clock and bus
  width (hipDeviceProp), as the reference computes it from the CUDA
  attributes (lws/adapters/cuda/gpu_probe.py:131-138), with HBM3E's
  transfers per reported clock;
- `ToolchainVersions(driver, cuda_runtime)` hold the HIP driver and runtime
  versions, `TorchAndCupy.cupy_version` the library's build string (there is
  no CuPy), `NvrtcInfo` the library version and its targets.
"""

from __future__ import annotations

import dataclasses

# ---------------------------------------------------------------------------
# device properties (lws/domain/device/properties.py)
# ---------------------------------------------------------------------------


@dataclasses.dataclass(frozen=True)
class DeviceName:
    value: str


@dataclasses.dataclass(frozen=True)
class GpuSlug:
    value: str


@dataclasses.dataclass(frozen=True)
class ComputeCapability:
    major: int
    minor: int


@dataclasses.dataclass(frozen=True)
class SmCount:
    value: int


@dataclasses.dataclass(frozen=True)
class Bytes:
    value: int

    def __post_init__(self) -> None:
        if self.value < 0:
            raise ValueError("Bytes cannot be negative")


@dataclasses.dataclass(frozen=True)
class GigabytesPerSecond:
    value: float


@dataclasses.dataclass(frozen=True)
class NvrtcTargets:
    values: tuple[int, ...]


@dataclasses.dataclass(frozen=True)
class DeviceIdentity:
    name: DeviceName
    slug: GpuSlug


@dataclasses.dataclass(frozen=True)
class ComputeHardware:
    capability: ComputeCapability
    sm_count: SmCount


@dataclasses.dataclass(frozen=True)
class IdentityAndCompute:
    identity: DeviceIdentity
    compute: ComputeHardware


@dataclasses.dataclass(frozen=True)
class VramSizes:
    total: Bytes
    free: Bytes


@dataclasses.dataclass(frozen=True)
class MemoryCharacteristics:
    l2_size: Bytes
    bandwidth: GigabytesPerSecond


@dataclasses.dataclass(frozen=True)
class MemoryProfile:
    vram: VramSizes
    characteristics: MemoryCharacteristics


@dataclasses.dataclass(frozen=True)
class MemoryAndNvrtc:
    memory: MemoryProfile
    nvrtc_targets: NvrtcTargets


@dataclasses.dataclass(frozen=True)
class DeviceProperties:
    identity_and_compute: IdentityAndCompute
    memory_and_nvrtc: MemoryAndNvrtc


# ---------------------------------------------------------------------------
# software versions (report only)
# ---------------------------------------------------------------------------


@dataclasses.dataclass(frozen=True)
class TorchArchList:
    values: tuple[str, ...]


@dataclasses.dataclass(frozen=True)
class TorchInfo:
    version: str
    arch_list: TorchArchList


@dataclasses.dataclass(frozen=True)
class NvrtcInfo:
    version: str
    targets: NvrtcTargets


@dataclasses.dataclass(frozen=True)
class ToolchainVersions:
    driver: str
    cuda_runtime: str


@dataclasses.dataclass(frozen=True)
class TorchAndCupy:
    torch: TorchInfo
    cupy_version: str


@dataclasses.dataclass(frozen=True)
class VersionsCore:
    toolchain: ToolchainVersions
    torch_and_cupy: TorchAndCupy


@dataclasses.dataclass(frozen=True)
class SoftwareVersions:
    core: VersionsCore
    nvrtc: NvrtcInfo


@dataclasses.dataclass(frozen=True)
class SupportVerdict:
    supported: bool


# ---------------------------------------------------------------------------
# benchmark timing (lws/domain/benchmark/statistics.py)
# ---------------------------------------------------------------------------


@dataclasses.dataclass(frozen=True)
class LatencySamples:
    """One run's per-sample latencies in microseconds."""

    values: tuple[float, ...]


@dataclasses.dataclass(frozen=True)
class RunCounts:
    warmup: int
    timed: int


# ---------------------------------------------------------------------------
# the tuning cache file (lws/application/ports/gpu/tuning_cache.py)
# ---------------------------------------------------------------------------


@dataclasses.dataclass(frozen=True)
class BatchSize:
    value: int


@dataclasses.dataclass(frozen=True)
class WeightShape:
    output_rows: int
    k: int


@dataclasses.dataclass(frozen=True)
class ShapeKey:
    weight_shape: WeightShape
    batch: BatchSize


@dataclasses.dataclass(frozen=True)
class KernelConfigurations:
    raw: object
    fused: object


@dataclasses.dataclass(frozen=True)
class ConfigurationSet:
    independent: KernelConfigurations
    order_matched: object


@dataclasses.dataclass(frozen=True)
class TunedEntry:
    key: ShapeKey
    configurations: ConfigurationSet


@dataclasses.dataclass(frozen=True)
class TunedEntries:
    items: tuple[TunedEntry, ...]


@dataclasses.dataclass(frozen=True)
class TuningFile:
    gpu_slug: GpuSlug
    entries: TunedEntries


def value_of(x) -> object:
    """`x.value` for a reference value object, else `x` itself (a plain int,
    float or str standing for it)."""
    return getattr(x, "value", x)
