"""Fused SE12 decode + GEMV on the GPU vs the oracle's numpy decode + float32
matmul on the same seeded inputs, within REL_TOL (1e-3 relative, scale
clamped at 1). Also: the raw-BF16 twin gives bit-identical outputs under the
same launch configuration (the reference's AC-032,
tests/test_spec_fused_gemv.py:313-320), every launch configuration is
deterministic, and a captured HIP graph replays to the eager result."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from conftest import GOLDEN_NAMES, golden_as_encoding, load_golden
from gpu_helpers import (REL_TOL, bf16_tensor, escape_count_bf16, heavy_tailed_bf16, max_rel_error, normal_case, to_device,
                         uniform_bits)
from oracle import se12_codec as o

pytestmark = pytest.mark.gpu


def _x(batch: int, cols: int, seed: int) -> np.ndarray:
    return o.normal_bf16(batch, cols, seed=seed, std=1.0)


def _check(kernel, enc, xbits, device, launch=None, f32=False):
    x = bf16_tensor(xbits, device)
    if f32:
        x = x.float()
    y = kernel.multiply(x, launch=launch)
    torch.cuda.synchronize()
    ref = o.gemv_reference(enc, o.bf16_bits_to_f32(xbits))
    err = max_rel_error(y, ref)
    assert err <= REL_TOL, f"max relative error {err:.3e}"
    return y


@pytest.mark.parametrize("name", GOLDEN_NAMES)
@pytest.mark.parametrize("batch", [1, 3, 8])
def test_gemv_golden_vectors(gpu, name, batch):
    from se12_amd.hip import Se12MatVecKernel

    g = load_golden(name)
    enc = golden_as_encoding(g)
    w = o.bf16_bits_to_f32(o.decode(enc))
    if not np.isfinite(w).all() or np.abs(w).max() > 1e30:
        # inf/NaN/huge weights: a row with a NaN weight must give NaN; rows of
        # finite weights whose sum is finite in float64 and float32 must match
        k = Se12MatVecKernel(to_device(enc, gpu))
        xb = _x(batch, g["cols"], seed=1)
        y = k.multiply(bf16_tensor(xb, gpu)).cpu().numpy()
        ref = o.gemv_reference(enc, o.bf16_bits_to_f32(xb))
        ref64 = o.gemv_reference(enc, o.bf16_bits_to_f32(xb), fp64=True)
        nan_rows = np.isnan(w).any(axis=1)
        assert np.all(np.isnan(y[:, nan_rows]))
        ok = (~np.isinf(w).any(axis=1)) & ~nan_rows & (np.abs(w).max(axis=1) < 1e30)
        ok = ok[None, :] & np.isfinite(ref) & np.isfinite(ref64)
        assert np.all(np.abs(y[ok] - ref[ok]) <= REL_TOL * np.maximum(np.abs(ref[ok]), 1.0))
        return
    k = Se12MatVecKernel(to_device(enc, gpu))
    _check(k, enc, _x(batch, g["cols"], seed=batch), gpu)


def test_gemv_benchmark_shape_batch1(gpu):
    from se12_amd.hip import Se12MatVecKernel

    bits, enc = normal_case(2304, 9216, seed=0)
    k = Se12MatVecKernel(to_device(enc, gpu))
    _check(k, enc, _x(1, 9216, seed=1), gpu)


@pytest.mark.parametrize("batch", [1, 2, 3, 4, 5, 8, 16, 32])
def test_gemv_batch_sweep(gpu, batch):
    from se12_amd.hip import Se12MatVecKernel

    bits, enc = normal_case(448, 3584, seed=11)
    k = Se12MatVecKernel(to_device(enc, gpu))
    _check(k, enc, _x(batch, 3584, seed=100 + batch), gpu)


@pytest.mark.parametrize("batch", [1, 4, 7])
def test_gemv_float32_activations(gpu, batch):
    from se12_amd.hip import Se12MatVecKernel

    bits, enc = normal_case(300, 1000, seed=12)
    k = Se12MatVecKernel(to_device(enc, gpu))
    rng = np.random.default_rng(batch)
    x = rng.standard_normal((batch, 1000)).astype(np.float32)
    y = k.multiply(torch.from_numpy(x).to(gpu))
    ref = o.gemv_reference(enc, x)
    assert max_rel_error(y, ref) <= REL_TOL


@pytest.mark.parametrize("batch", [2, 4])
def test_float32_activations_through_the_pair_tree(gpu, batch):
    """FP32 activations (the edge-handling dot2 variants) at 2304x9216 and 2-4
    batch rows, whose default launch splits K in 3 (4 waves x 432 blocks) and
    adds the splits in the pair tree: within REL_TOL of the oracle, run to run
    identical, the raw twin bit-identical."""
    from se12_amd.hip import RawBf16MatVecKernel, Se12MatVecKernel

    bits, enc = normal_case(2304, 9216, seed=14)
    k = Se12MatVecKernel(to_device(enc, gpu))
    r = RawBf16MatVecKernel(bf16_tensor(bits, gpu))
    lc = k.default_launch(batch)
    assert (lc.threads_per_block.value, lc.blocks.value) == (256, 432)
    rng = np.random.default_rng(100 + batch)
    xf = rng.standard_normal((batch, 9216)).astype(np.float32)
    x = torch.from_numpy(xf).to(gpu)
    y1 = k.multiply(x).clone()
    y2 = k.multiply(x)
    yr = r.multiply(x, launch=lc)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2) and torch.equal(y1, yr)
    assert max_rel_error(y1, o.gemv_reference(enc, xf)) <= REL_TOL


@pytest.mark.parametrize("rows,cols", [(1, 1), (17, 257), (33, 300), (100, 2304), (2048, 2304), (64, 9216)])
def test_gemv_ragged_and_escape_heavy(gpu, rows, cols):
    from se12_amd.hip import Se12MatVecKernel

    bits = heavy_tailed_bf16(rows, cols, seed=rows * 7 + cols)
    enc = o.encode(bits.reshape(-1), rows, cols)
    k = Se12MatVecKernel(to_device(enc, gpu))
    _check(k, enc, _x(2, cols, seed=rows), gpu)


@pytest.mark.parametrize("batch", [5, 17])
@pytest.mark.parametrize("rows,cols", [(1, 1), (17, 257), (33, 300), (2048, 2304), (64, 9216)])
def test_batched_ragged_and_escape_heavy(gpu, rows, cols, batch):
    """The batched MFMA kernel (BF16 x, 5..32 rows) on ragged and escape-heavy
    matrices, padding rows of the 16-row batch groups included."""
    from se12_amd.hip import Se12MatVecKernel

    bits = heavy_tailed_bf16(rows, cols, seed=rows * 5 + cols)
    enc = o.encode(bits.reshape(-1), rows, cols)
    k = Se12MatVecKernel(to_device(enc, gpu))
    _check(k, enc, _x(batch, cols, seed=rows + batch), gpu)


@pytest.mark.parametrize("batch", [3, 9])
def test_gemv_fallback_tiles(gpu, batch):
    from se12_amd.hip import Se12MatVecKernel

    # concentrated exponents with random escapes; a third of the tiles overflow
    rng = np.random.default_rng(21)
    e = rng.choice(np.arange(118, 126, dtype=np.uint8), size=(64, 1024))
    for t in range(16):
        if t % 3 == 0:
            tr, tc = divmod(t, 4)
            pos = rng.choice(4096, size=40, replace=False)
            e[tr * 16 + pos // 256, tc * 256 + pos % 256] = rng.integers(100, 118, size=40)
    sign = rng.integers(0, 2, size=e.shape).astype(np.uint16)
    mant = rng.integers(0, 0x80, size=e.shape).astype(np.uint16)
    bits = ((sign << 15) | (e.astype(np.uint16) << 7) | mant).view(np.int16)
    enc = o.encode(bits.reshape(-1), 64, 1024)
    assert o.fallback_tile_count(enc) == 6
    k = Se12MatVecKernel(to_device(enc, gpu))
    _check(k, enc, _x(batch, 1024, seed=5), gpu)


@pytest.mark.parametrize("batch", [1, 6])
def test_gemv_padding_of_an_infinite_codebook0_is_masked(gpu, batch):
    """codebook[0] = 255: padding columns decode to +inf; rows whose real
    weights are finite must still give finite, correct outputs."""
    from se12_amd.hip import Se12MatVecKernel

    rows, cols = 32, 300
    rng = np.random.default_rng(8)
    bits = o.normal_bf16(rows, cols, seed=9, std=0.02)
    bits[:16] = np.uint16(0x7F80).view(np.int16)  # +inf rows make 255 the top exponent
    enc = o.encode(bits.reshape(-1), rows, cols)
    assert enc["codebook"][0] == 255
    k = Se12MatVecKernel(to_device(enc, gpu))
    xb = _x(batch, cols, seed=int(rng.integers(100)))
    y = k.multiply(bf16_tensor(xb, gpu)).cpu().numpy()
    ref = o.gemv_reference(enc, o.bf16_bits_to_f32(xb))
    assert np.all(np.isfinite(y[:, 16:]))
    assert np.all(np.abs(y[:, 16:] - ref[:, 16:]) <= REL_TOL * np.maximum(np.abs(ref[:, 16:]), 1.0))
    assert np.array_equal(np.isnan(y[:, :16]), np.isnan(ref[:, :16]))


def _configs(rows, cols, batch=1):
    from se12_amd.launch import candidate_configurations

    return candidate_configurations(rows, cols, batch=batch)


@pytest.mark.parametrize("rows,cols,batch", [(272, 2800, 2), (272, 2800, 6), (272, 2800, 20), (448, 3584, 32)])
def test_every_launch_configuration_is_correct_and_deterministic(gpu, rows, cols, batch):
    from se12_amd.hip import Se12MatVecKernel

    bits = heavy_tailed_bf16(rows, cols, seed=31)
    enc = o.encode(bits.reshape(-1), rows, cols)
    k = Se12MatVecKernel(to_device(enc, gpu))
    xb = _x(batch, cols, seed=32)
    x = bf16_tensor(xb, gpu)
    ref = o.gemv_reference(enc, o.bf16_bits_to_f32(xb))
    for cfg in _configs(rows, cols, batch=batch):
        y1 = k.multiply(x, launch=cfg).clone()
        y2 = k.multiply(x, launch=cfg)
        torch.cuda.synchronize()
        assert torch.equal(y1, y2), cfg
        assert max_rel_error(y1, ref) <= REL_TOL, cfg


@pytest.mark.parametrize("batch", [14, 16])
def test_x_slab_launches_with_and_without_the_slab_ring(gpu, batch):
    """The x-slab kernel under every launch the tuner would try, on a library
    told of 132 compute units (the x-slab kernel then serves 2128x6144 at 14
    and 16 batch rows: 133 tile rows, x does not fit whole, and two K splits
    at one batch group are refused below 8,192 tiles).
    Long launches (12+ steps per wave) whose ring of 8 slabs fits LDS keep
    their slabs in it with a block barrier every 4 steps, the others a
    barrier per step: every launch within REL_TOL of the oracle, run to run
    identical, the raw twin bit-identical."""
    from se12_amd import _native as nat
    from se12_amd.hip import RawBf16MatVecKernel, Se12MatVecKernel
    from se12_amd.launch import candidate_configurations, grid_rows, k_tiles, mfma_min_waves, uses_rx

    rows, cols, cus = 2128, 6144, 132
    assert not uses_rx(rows, cols, batch, compute_units=cus)
    bits = heavy_tailed_bf16(rows, cols, seed=35)
    enc = o.encode(bits.reshape(-1), rows, cols)
    k = Se12MatVecKernel(to_device(enc, gpu))
    r = RawBf16MatVecKernel(bf16_tensor(bits, gpu))
    for kern in (k, r):
        nat.check(nat.lib().se12_set_compute_units(kern.handle.raw, cus))
    xb = _x(batch, cols, seed=36)
    x = bf16_tensor(xb, gpu)
    ref = o.gemv_reference(enc, o.bf16_bits_to_f32(xb))
    cfgs = candidate_configurations(rows, cols, batch=batch, compute_units=cus)
    steps = set()
    for cfg in cfgs:
        waves = cfg.threads_per_block.value // 64
        splits = cfg.blocks.value // grid_rows(rows, waves, batch)
        share = -(-k_tiles(cols) // splits)                        # K tiles per split
        steps.add(-(-share // (waves // mfma_min_waves(batch))))  # per K group
        y1 = k.multiply(x, launch=cfg).clone()
        y2 = k.multiply(x, launch=cfg)
        yr = r.multiply(x, launch=cfg)
        torch.cuda.synchronize()
        assert torch.equal(y1, y2), cfg
        assert torch.equal(y1, yr), cfg
        assert max_rel_error(y1, ref) <= REL_TOL, cfg
    # one K group over 24 and 12 steps and two over 12 (ring of 8) and short
    # launches (a barrier per step) all ran
    assert 24 in steps and 12 in steps and min(steps) < 12, sorted(steps)


def test_every_batch1_launch_configuration(gpu):
    from se12_amd.hip import Se12MatVecKernel

    bits = heavy_tailed_bf16(2304, 9216, seed=33)
    enc = o.encode(bits.reshape(-1), 2304, 9216)
    k = Se12MatVecKernel(to_device(enc, gpu))
    xb = _x(1, 9216, seed=34)
    x = bf16_tensor(xb, gpu)
    ref = o.gemv_reference(enc, o.bf16_bits_to_f32(xb))
    cfgs = _configs(2304, 9216, batch=1)
    assert any(c.threads_per_block.value == 1024 for c in cfgs)
    for cfg in cfgs:
        y = k.multiply(x, launch=cfg)
        assert max_rel_error(y, ref) <= REL_TOL, cfg


@pytest.mark.parametrize("shape", [(2304, 9216), (272, 2800), (48, 768)])
def test_raw_twin_is_bit_identical_under_one_launch(gpu, shape):
    from se12_amd.hip import RawBf16MatVecKernel, Se12MatVecKernel

    rows, cols = shape
    if shape == (48, 768):
        g = load_golden("mixed_48x768")
        bits, enc = g["bits"].reshape(rows, cols), golden_as_encoding(g)
    else:
        bits = heavy_tailed_bf16(rows, cols, seed=rows)
        enc = o.encode(bits.reshape(-1), rows, cols)
    fused = Se12MatVecKernel(to_device(enc, gpu))
    raw = RawBf16MatVecKernel(bf16_tensor(bits, gpu))
    for batch in (1, 4, 6, 17, 32):
        x = bf16_tensor(_x(batch, cols, seed=batch), gpu)
        all_cfgs = list(_configs(rows, cols, batch=batch))
        cfgs = [None] + all_cfgs[:: max(1, len(all_cfgs) // 6)] + all_cfgs[-2:]
        for cfg in cfgs:
            assert torch.equal(fused.multiply(x, launch=cfg), raw.multiply(x, launch=cfg)), (batch, cfg)


@pytest.mark.parametrize("batch", [1, 2, 8, 16, 24])
def test_graph_replay_matches_eager(gpu, batch):
    """Replays of a captured product equal the eager result, with eager work
    between replays, at 2304x9216: the dot2 kernel (B = 1), the dot2 kernel
    with 3 K splits meeting in the pair tree (2), the x-slab kernel with K
    splits (8: one-wave blocks, 6 splits; 16) and the resident-x kernel with K
    splits (24), whose pair slots and arrival counters must be back at zero
    after every launch."""
    from se12_amd.hip import Se12MatVecKernel

    bits, enc = normal_case(2304, 9216, seed=0)
    k = Se12MatVecKernel(to_device(enc, gpu))
    x = bf16_tensor(_x(batch, 9216, seed=1), gpu)
    out = torch.empty((batch, 2304), dtype=torch.float32, device=gpu)
    eager = k.multiply(x).clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        k.multiply(x, out=out)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        k.multiply(x, out=out)
    for i in range(4):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), i
        _ = k.multiply(x)  # eager work between replays
        torch.cuda.synchronize()


def test_bad_arguments_raise(gpu):
    from se12_amd import _native as nat
    from se12_amd.hip import Se12MatVecKernel
    from se12_amd.launch import BlockCount, LaunchConfiguration, ThreadsPerBlock

    bits, enc = normal_case(64, 512, seed=2)
    k = Se12MatVecKernel(to_device(enc, gpu), max_batch=4)
    with pytest.raises(ValueError):
        k.multiply(torch.zeros((1, 511), dtype=torch.bfloat16, device=gpu))
    with pytest.raises(nat.Se12Error):
        k.multiply(torch.zeros((5, 512), dtype=torch.bfloat16, device=gpu))
    with pytest.raises(nat.Se12Error):
        k.multiply(torch.zeros((1, 512), dtype=torch.bfloat16, device=gpu),
                   launch=LaunchConfiguration(ThreadsPerBlock(96), BlockCount(4)))
    with pytest.raises(nat.Se12Error):
        k.multiply(torch.zeros((1, 512), dtype=torch.bfloat16, device=gpu),
                   launch=LaunchConfiguration(ThreadsPerBlock(64), BlockCount(5)))


def test_grouped_launch_equals_separate_launches(gpu):
    """q/k/v-like matrices sharing x in one launch: bit-identical to separate
    launches under the same waves per block and K splits, and within the
    tolerance of the oracle under the default launch."""
    from se12_amd.hip import RawBf16MatVecKernel, Se12MatVecKernel, multiply_grouped
    from se12_amd.launch import (BlockCount, LaunchConfiguration, ThreadsPerBlock, configuration, grid_rows,
                                 mfma_min_waves, rx_configuration, rx_kgroups, uses_rx)

    cols = 2304
    shapes = [(272, cols), (128, cols), (48, cols)]
    bits = [heavy_tailed_bf16(r, c, seed=40 + i) for i, (r, c) in enumerate(shapes)]
    encs = [o.encode(b.reshape(-1), r, c) for b, (r, c) in zip(bits, shapes)]
    kerns = [Se12MatVecKernel(to_device(e, gpu), max_batch=20) for e in encs]
    raws = [RawBf16MatVecKernel(bf16_tensor(b, gpu), max_batch=20) for b in bits]
    for batch in (1, 3, 6, 20):
        xb = _x(batch, cols, seed=50 + batch)
        x = bf16_tensor(xb, gpu)
        ys = multiply_grouped(kerns, x)
        for y, e in zip(ys, encs):
            ref = o.gemv_reference(e, o.bf16_bits_to_f32(xb))
            assert max_rel_error(y, ref) <= REL_TOL
        if uses_rx(272, cols, batch):
            # the resident-x kernel: (waves, blocks per matrix), which fix each
            # matrix's K groups; the same groups give the same sums, grouped or
            # single, whichever blocks hold the rows
            for waves, per in ((3, 1), (8, 17), (4, 5), (1, 3), (12, 3), (12, 17), (8, 1)):
                ys = multiply_grouped(kerns, x, launch=rx_configuration(waves, per, len(shapes)))
                ysr = multiply_grouped(raws, x, launch=rx_configuration(waves, per, len(shapes)))
                for k, r, y, yr, (rows, _), e in zip(kerns, raws, ys, ysr, shapes, encs):
                    tr = -(-rows // 16)
                    kg = rx_kgroups(rows, cols, waves, per)
                    assert kg == rx_kgroups(rows, cols, waves, min(per, tr))
                    assert torch.equal(y, k.multiply(x, launch=rx_configuration(waves, min(per, tr)))), (batch, waves, per)
                    assert torch.equal(yr, y), (batch, waves, per)
                    ref = o.gemv_reference(e, o.bf16_bits_to_f32(xb))
                    assert max_rel_error(y, ref) <= REL_TOL, (batch, waves, per, kg)
                    # another block count with the same K groups: the rows move
                    # to other blocks, the sums stay
                    for other in range(1, tr + 1):
                        if other != min(per, tr) and rx_kgroups(rows, cols, waves, other) == kg:
                            assert torch.equal(y, k.multiply(x, launch=rx_configuration(waves, other))), \
                                (batch, waves, per, other)
                            break
            continue
        for waves, splits in ((3, 1), (9, 1), (4, 3), (6, 2)):
            if batch >= 4 and waves > 8:
                continue
            if batch >= 5 and waves % mfma_min_waves(batch):  # MFMA: tile rows per block x K groups
                continue
            rows_total = sum(grid_rows(r, waves, batch) for r, _ in shapes)
            grouped = LaunchConfiguration(ThreadsPerBlock(64 * waves), BlockCount(rows_total * splits))
            ys = multiply_grouped(kerns, x, launch=grouped)
            ysr = multiply_grouped(raws, x, launch=grouped)
            for k, r, y, yr, (rows, _) in zip(kerns, raws, ys, ysr, shapes):
                single = configuration(waves, splits, rows, batch)
                assert torch.equal(y, k.multiply(x, launch=single)), (batch, waves, splits)
                assert torch.equal(yr, y), (batch, waves, splits)


def test_grouped_launch_with_x_partly_from_global(gpu):
    """q/k/v-like matrices at K = 3584 and 23..32 batch rows: x fits a block's
    LDS only up to 22 rows and the group has at most one tile row per CU, so
    the grouped launch keeps rows 0..15 of x in LDS and loads batch group 1's
    operands from global memory. Within the tolerance of the oracle; the raw
    twin bit-identical; each matrix bit-identical to its own launch under the
    same waves and K groups."""
    from se12_amd.hip import RawBf16MatVecKernel, Se12MatVecKernel, multiply_grouped
    from se12_amd.launch import rx_configuration, rx_kgroups, rx_staged_rows

    cols = 3584
    shapes = [(1024, cols), (512, cols), (512, cols)]
    bits = [heavy_tailed_bf16(r, c, seed=70 + i) for i, (r, c) in enumerate(shapes)]
    encs = [o.encode(b.reshape(-1), r, c) for b, (r, c) in zip(bits, shapes)]
    kerns = [Se12MatVecKernel(to_device(e, gpu), max_batch=32) for e in encs]
    raws = [RawBf16MatVecKernel(bf16_tensor(b, gpu), max_batch=32) for b in bits]
    total_rows = sum(r for r, _ in shapes)
    for batch in (23, 24, 32):
        assert rx_staged_rows(total_rows, cols, batch) == 16
        xb = _x(batch, cols, seed=80 + batch)
        x = bf16_tensor(xb, gpu)
        refs = [o.gemv_reference(e, o.bf16_bits_to_f32(xb)) for e in encs]
        ys, ysr = multiply_grouped(kerns, x), multiply_grouped(raws, x)
        for y, yr, ref in zip(ys, ysr, refs):
            assert max_rel_error(y, ref) <= REL_TOL, batch
            assert torch.equal(y, yr), batch
        for waves, per in ((8, 64), (4, 32), (6, 21)):
            ys = multiply_grouped(kerns, x, launch=rx_configuration(waves, per, len(shapes)))
            ysr = multiply_grouped(raws, x, launch=rx_configuration(waves, per, len(shapes)))
            for k, y, yr, (rows, _), ref in zip(kerns, ys, ysr, shapes, refs):
                tr = rows // 16
                assert rx_kgroups(rows, cols, waves, per) == rx_kgroups(rows, cols, waves, min(per, tr))
                assert torch.equal(y, k.multiply(x, launch=rx_configuration(waves, min(per, tr)))), (batch, waves, per)
                assert torch.equal(yr, y), (batch, waves, per)
                assert max_rel_error(y, ref) <= REL_TOL, (batch, waves, per)


@pytest.mark.parametrize("batch", [12, 16, 24, 32])
def test_resident_x_k_splits(gpu, batch):
    """x of 12..32 rows at K = 14336 fits a block's LDS only as a share of its
    columns: the resident-x kernel splits K (3 to 7 splits, each block holding
    its split's columns of x) and the last block of a row to arrive adds the
    splits' partial sums in split order. Heavy-tailed weights (listed
    escapes); against the oracle under the default and other launches (K
    groups; several rows per row slot; one slot holding all 65 rows), the raw
    twin bit-identical and a repeated launch bit-identical under each; a block
    count that is not a multiple of the splits refused."""
    from se12_amd import _native as nat
    from se12_amd.hip import RawBf16MatVecKernel, Se12MatVecKernel
    from se12_amd.launch import rx_configuration, rx_layout

    rows, cols = 1040, 14336
    staged, splits = rx_layout(rows, cols, batch)
    assert staged == batch and splits == {12: 3, 16: 3, 24: 5, 32: 7}[batch]
    bits = heavy_tailed_bf16(rows, cols, seed=90)
    enc = o.encode(bits.reshape(-1), rows, cols)
    fused = Se12MatVecKernel(to_device(enc, gpu))
    raw = RawBf16MatVecKernel(bf16_tensor(bits, gpu))
    xb = _x(batch, cols, seed=91 + batch)
    x = bf16_tensor(xb, gpu)
    ref = o.gemv_reference(enc, o.bf16_bits_to_f32(xb))
    for launch in (None, rx_configuration(12, 32, splits=splits), rx_configuration(4, 8, splits=splits),
                   rx_configuration(1, 1, splits=splits), rx_configuration(6, 65, splits=splits)):
        y = fused.multiply(x, launch=launch).clone()
        y2 = fused.multiply(x, launch=launch)
        yr = raw.multiply(x, launch=launch)
        torch.cuda.synchronize()
        assert max_rel_error(y, ref) <= REL_TOL, launch
        assert torch.equal(y, y2), launch
        assert torch.equal(y, yr), launch
    with pytest.raises(nat.Se12Error, match="K splits"):
        fused.multiply(x, launch=rx_configuration(8, 32 * splits + 1))


def test_grouped_launch_rejects_mixed_groups(gpu):
    from se12_amd import _native as nat
    from se12_amd.hip import RawBf16MatVecKernel, Se12MatVecKernel, multiply_grouped

    _, e1 = normal_case(64, 512, seed=3)
    _, e2 = normal_case(64, 768, seed=4)
    k1 = Se12MatVecKernel(to_device(e1, gpu))
    k2 = Se12MatVecKernel(to_device(e2, gpu))
    r1 = RawBf16MatVecKernel(bf16_tensor(o.decode(e1), gpu))
    x = torch.zeros((1, 512), dtype=torch.bfloat16, device=gpu)
    with pytest.raises(ValueError):
        multiply_grouped([k1, k2], x)
    with pytest.raises(ValueError):
        multiply_grouped([k1, r1], x)
    with pytest.raises(ValueError):
        multiply_grouped([k1] * 5, x)
    hs = (ctypes.c_void_p * 2)(k1.handle.raw.value, k2.handle.raw.value)
    y = torch.empty((1, 64), dtype=torch.float32, device=gpu)
    ys = (ctypes.c_void_p * 2)(y.data_ptr(), y.data_ptr())
    assert nat.lib().se12_gemv_grouped(hs, 2, nat.ptr(x), nat.X_BF16, 1, ys, None, nat.stream_ptr()) == nat.SE12_E_INVALID
    assert "one K" in nat.last_error()


@pytest.mark.parametrize("batch", [1, 2, 4, 6, 17])
def test_every_escape_count_matches_oracle_and_raw_twin(gpu, batch):
    """Tiles with 0..16 escapes (listed escapes up to 8, raw tiles decoded at
    bind beyond) and a fallback tile, through the dot2 (B <= 4) and MFMA
    kernels: within REL_TOL of the oracle, and bit-identical to the raw-BF16
    twin under each launch shape."""
    from se12_amd.hip import RawBf16MatVecKernel, Se12MatVecKernel

    bits, _ = escape_count_bf16(seed=12)
    enc = o.encode(bits.reshape(-1), 64, 1024)
    fused = Se12MatVecKernel(to_device(enc, gpu))
    raw = RawBf16MatVecKernel(bf16_tensor(bits, gpu))
    xb = _x(batch, 1024, seed=batch)
    _check(fused, enc, xb, gpu)
    x = bf16_tensor(xb, gpu)
    for cfg in [None] + list(_configs(64, 1024, batch=batch))[::3]:
        assert torch.equal(fused.multiply(x, launch=cfg), raw.multiply(x, launch=cfg)), cfg

