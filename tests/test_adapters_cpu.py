"""The reference-signature boundary without a GPU: the compile target rule,
the ahead-of-time KernelCompiler, the translation of reference-semantics
launch configurations, and the adapters' constructor signatures."""

from __future__ import annotations

import dataclasses
import inspect

import pytest
import torch

from se12_amd import adapters, compiler, launch


# The reference's launch value types and the two rules that build them
# (lws/domain/launch/heuristic.py:24-87, search_space.py:14-36), restated as
# test inputs: distinct classes from se12_amd.launch's, as the reference's are.
@dataclasses.dataclass(frozen=True)
class RefThreads:
    value: int


@dataclasses.dataclass(frozen=True)
class RefBlocks:
    value: int


@dataclasses.dataclass(frozen=True)
class RefLaunch:
    threads_per_block: RefThreads
    blocks: RefBlocks


def ref_candidates(rows: int, batch: int) -> list[RefLaunch]:
    need = rows * batch
    return [RefLaunch(RefThreads(t), RefBlocks(-(-need // (t // 32)))) for t in (32, 64, 128, 256, 512)]


def ref_default(sm_count: int, rows: int, batch: int) -> RefLaunch:
    need = rows * batch
    fitting = [t for t in (256, 128, 64, 32) if -(-need // (t // 32)) >= 4 * sm_count]
    t = max(fitting) if fitting else 32
    return RefLaunch(RefThreads(t), RefBlocks(-(-need // (t // 32))))


def test_compile_target_from_the_device_arch():
    t = compiler.choose_compile_target("gfx950:sramecc+:xnack-")
    assert t.kind is compiler.CompileTargetKind.CODE_OBJECT and t.arch.value == "gfx950"
    for other in ("gfx942:sramecc+:xnack-", "gfx90a", "sm_90", ""):
        with pytest.raises(compiler.UnsupportedDeviceError):
            compiler.choose_compile_target(other)
    assert issubclass(compiler.UnsupportedDeviceError, ValueError)


def test_aot_compiler_checks_the_target_and_maps_reference_kernels():
    c = compiler.AotKernelCompiler()
    target = compiler.choose_compile_target("gfx950")
    h = c.compile(compiler.KernelSource("// CUDA source text is kept, never compiled"), target)
    assert h.target == target
    lib = h.library
    assert h.function("lws_gemv_se12") is lib.se12_gemv
    assert h.function("lws_gemv_raw_bf16") is lib.se12_gemv
    assert h.function("lws_se12_decode") is lib.se12_decode
    assert h.function("se12_decode_rows") is lib.se12_decode_rows
    with pytest.raises(KeyError):
        h.function("lws_calibration_kernel")
    bad = compiler.CompileTarget(kind=compiler.CompileTargetKind.CODE_OBJECT, arch=compiler.GfxArch("gfx942"))
    with pytest.raises(compiler.UnsupportedDeviceError):
        c.compile(compiler.KernelSource(""), bad)
    with pytest.raises(compiler.UnsupportedDeviceError):
        c.compile(compiler.KernelSource(""), object())


def test_cache_directory_follows_the_reference_variable(monkeypatch, tmp_path):
    monkeypatch.setenv("LWS_CACHE_DIR", str(tmp_path))
    assert compiler.AotKernelCompiler().cache_directory == tmp_path


@pytest.mark.parametrize("rows,k", [(2304, 9216), (9216, 2304), (14336, 3584), (1000, 300), (256000, 2304)])
@pytest.mark.parametrize("batch", [1, 2, 4, 5, 8, 9, 16, 17, 24, 32])
def test_reference_launches_translate_to_valid_configurations(rows, k, batch):
    cands = ref_candidates(rows, batch) + [ref_default(sm, rows, batch) for sm in (28, 132, 256)]
    for f32 in (False, True):
        for ref in cands:
            cfg = launch.from_reference_configuration(ref, rows, k, batch, float32_activations=f32)
            waves, splits = launch.waves_and_splits(cfg, rows, batch, k, float32_activations=f32)
            if launch.uses_rx(rows, k, batch, f32):
                # the resident-x kernel: the block's threads (at most 12 waves,
                # 8 with batch group 1's x from global memory), one tile row
                # per wave slot in each of the K splits the shape fixes
                # (`splits` here counts blocks)
                assert waves == min(-(-ref.threads_per_block.value // 64), launch.rx_max_waves(rows, k, batch))
                sp = launch.rx_splits(rows, k, batch, f32)
                assert splits == -(-launch.tile_rows(rows) // waves) * sp
                continue
            assert splits == 1
            # the block's threads in whole wave64s, a whole number of the MFMA
            # kernel's tile rows per block, within the variant's limit
            lo = launch.mfma_min_waves(batch) if launch.uses_mfma(batch, f32) else 1
            hi = launch.max_waves_per_block(batch, f32, launch.runs_generic(rows, k, f32)) // lo * lo
            assert waves == min(-(-ref.threads_per_block.value // (64 * lo)) * lo, hi)
        # misaligned x takes the edge-handling variants, whose limit is lower
        for ref in cands:
            cfg = launch.from_reference_configuration(ref, rows, k, batch, aligned_x=False)
            launch.waves_and_splits(cfg, rows, batch, k=k + (1 if k % 256 == 0 else 0))


def test_translation_keeps_the_block_and_refuses_uncovered_launches():
    cfg = launch.from_reference_configuration(RefLaunch(RefThreads(256), RefBlocks(288)), 2304, 9216, 1)
    assert launch.waves_and_splits(cfg, 2304, 1, 9216) == (4, 1)
    cfg = launch.from_reference_configuration(RefLaunch(RefThreads(32), RefBlocks(2304)), 2304, 9216, 1)
    assert launch.waves_and_splits(cfg, 2304, 1, 9216) == (1, 1)
    # B = 24 on the x-slab MFMA kernel (4608x36864: x's columns would need 12
    # resident-x splits): 4 tile rows per block, 448 threads (7 waves) -> 8 waves
    cfg = launch.from_reference_configuration(RefLaunch(RefThreads(448), RefBlocks(25000)), 4608, 36864, 24)
    assert launch.waves_and_splits(cfg, 4608, 24, 36864) == (8, 1)
    # B = 24 at 14336x3584 on the resident-x kernel with 2 K splits: 7 waves,
    # 896 tile rows over 128 blocks of 7 row slots in each split
    cfg = launch.from_reference_configuration(RefLaunch(RefThreads(448), RefBlocks(25000)), 14336, 3584, 24)
    assert launch.waves_and_splits(cfg, 14336, 24, 3584) == (7, 128 * 2)
    # B = 24 at K = 9216 on the resident-x kernel with 3 K splits: 7 waves,
    # one tile row per slot, in each split
    cfg = launch.from_reference_configuration(RefLaunch(RefThreads(448), RefBlocks(4000)), 2304, 9216, 24)
    assert launch.waves_and_splits(cfg, 2304, 24, 9216) == (7, 21 * 3)
    with pytest.raises(ValueError, match="do not cover"):
        launch.from_reference_configuration(RefLaunch(RefThreads(256), RefBlocks(287)), 2304, 9216, 1)
    for t in (0, 16, 48 + 1, 2048):
        with pytest.raises(ValueError):
            launch.from_reference_configuration(RefLaunch(RefThreads(t), RefBlocks(10**6)), 2304, 9216, 1)


def test_adapters_take_the_reference_constructor_arguments():
    def names(cls):
        return list(inspect.signature(cls.__init__).parameters)[1:]

    # lws/adapters/cuda/gemv.py:146,183; lws/adapters/cuda/se12_decoder.py:48
    assert names(adapters.RawBf16MatVecKernel)[:4] == ["compiler", "target", "weights", "sm_count"]
    assert names(adapters.Se12MatVecKernel)[:5] == ["compiler", "target", "tensor", "sm_count", "extra_decode_ops"]
    assert names(adapters.Se12WeightDecoder) == ["compiler", "target"]
    assert inspect.signature(adapters.Se12MatVecKernel.__init__).parameters["extra_decode_ops"].default == 0
    for cls in (adapters.Se12MatVecKernel, adapters.RawBf16MatVecKernel):
        assert list(inspect.signature(cls.multiply).parameters)[1:3] == ["activations", "launch"]


def test_adapter_arguments_are_checked_before_any_gpu_call():
    c = compiler.AotKernelCompiler()
    t = compiler.choose_compile_target("gfx950")
    with pytest.raises(ValueError, match="extra_decode_ops"):
        adapters.Se12MatVecKernel(c, t, None, 256, extra_decode_ops=4)
    for bad in (0, -3, True, 2.5, "256"):
        with pytest.raises(ValueError, match="sm_count"):
            adapters.Se12MatVecKernel(c, t, None, bad)
    with pytest.raises(compiler.UnsupportedDeviceError):
        adapters.RawBf16MatVecKernel(c, object(), None, 256)


@pytest.mark.parametrize("batch", [24, 32])
def test_translation_follows_the_adapters_compute_units(batch):
    """A matrix of 256 tile rows at K = 3584: x of 24 or 32 rows does not fit
    a block's LDS but its first 16 rows do, and on a GPU of 256+ CUs (one
    tile row per CU) such batches run the resident-x kernel with batch group
    1's x from global memory; with 132 compute units the library splits K
    in two instead and keeps every row of x. The translation must follow the
    count the library was given."""
    rows, k = 4096, 3584
    ref = RefLaunch(RefThreads(256), RefBlocks(-(-rows * batch // 8)))
    cfg256 = launch.from_reference_configuration(ref, rows, k, batch, compute_units=256)
    assert launch.rx_layout(rows, k, batch, compute_units=256) == (16, 1)
    assert launch.waves_and_splits(cfg256, rows, batch, k, compute_units=256) == (4, 64)
    assert launch.rx_layout(rows, k, batch, compute_units=132) == (batch, 2)
    # the rows whose x fits whole run the resident-x kernel unsplit on either GPU
    assert launch.rx_layout(rows, k, 20, compute_units=132) == (20, 1) == launch.rx_layout(rows, k, 20, compute_units=256)
    cfg132 = launch.from_reference_configuration(ref, rows, k, batch, compute_units=132)
    # 4 row slots per block: 64 blocks in each of the 2 K splits
    assert launch.waves_and_splits(cfg132, rows, batch, k, compute_units=132) == (4, 64 * 2)
    assert cfg132.blocks.value == 64 * 2
    # and the candidates the tuner would time follow the same rule
    c132 = launch.candidate_configurations(rows, k, batch, compute_units=132)
    for c in c132:
        launch.waves_and_splits(c, rows, batch, k, compute_units=132)


def test_adapter_translation_passes_its_sm_count(monkeypatch):
    seen = {}

    def fake(launch_cfg, rows, k, batch, **kw):
        seen.update(kw)
        return "translated"

    monkeypatch.setattr(adapters, "from_reference_configuration", fake)

    class K:
        rows, cols, sm_count = 4096, 3584, 132

    x = torch.zeros((24, 3584), dtype=torch.bfloat16)
    assert adapters._native_launch(K(), x, RefLaunch(RefThreads(256), RefBlocks(12288))) == "translated"
    assert seen["compute_units"] == 132


def test_aot_compiler_takes_the_reference_sass_target():
    """The reference's choose_compile_target gives CompileTarget(SASS,
    ComputeArch(95)) from the probe's capability (9, 5) and targets (95,)
    (lws/domain/device/decisions.py:70-103); the compiler accepts that for
    gfx950 and refuses PTX or another architecture."""

    @dataclasses.dataclass(frozen=True)
    class Kind:
        value: str

    @dataclasses.dataclass(frozen=True)
    class Arch:
        value: int

    @dataclasses.dataclass(frozen=True)
    class RefTarget:
        kind: Kind
        arch: Arch

    c = compiler.AotKernelCompiler()
    h = c.compile(compiler.KernelSource(""), RefTarget(Kind("sass"), Arch(95)))
    assert h.function("lws_gemv_se12") is h.library.se12_gemv
    for bad in (RefTarget(Kind("sass"), Arch(94)), RefTarget(Kind("ptx"), Arch(95))):
        with pytest.raises(compiler.UnsupportedDeviceError):
            c.compile(compiler.KernelSource(""), bad)
    assert compiler.arch_number("gfx950:sramecc+:xnack-") == 95


def test_port_adapters_take_the_reference_constructor_arguments():
    # lws/adapters/cuda/gpu_probe.py:62, benchmark_timer.py:24,
    # lws/adapters/filesystem/tuning_cache.py:44
    def names(cls):
        return list(inspect.signature(cls.__init__).parameters)[1:]

    assert len(names(adapters.HipGpuProbe)) == 1
    assert names(adapters.HipBenchmarkTimer) == ["device_index", "l2_size"]
    assert names(adapters.FilesystemTuningCache) == ["directory", "gpu_slug"]
    assert list(inspect.signature(adapters.HipBenchmarkTimer.time_operation).parameters)[1:] == ["operation", "counts"]
    assert list(inspect.signature(adapters.tune_launch).parameters) == ["gpu_slug", "requests", "evaluators", "cache"]
    for m in ("properties", "software_versions", "smoke_test"):
        assert list(inspect.signature(getattr(adapters.HipGpuProbe, m)).parameters) == ["self"]
