"""Launch configurations for the SE12 GEMV on MI355X, and the tuner's rules.

Mirrors lws/domain/launch/heuristic.py:24-51 (LaunchConfiguration =
threads_per_block + blocks) and lws/domain/launch/search_space.py:14-75
(candidate set, best configuration, order-matched configuration), re-derived
for this kernel's grid: a block is 1..16 wave64s working on one 16-row tile
row, and `blocks` = tile_rows x k_splits, where the K tiles of a tile row are
cut into `k_splits` contiguous ranges (the last block of a tile row to finish
adds the splits in order). BF16 batches of MFMA_MIN_BATCH or more rows run
the batched MFMA kernel instead, whose block is 1..8 wave64s each owning one
tile row: there `blocks` = ceil(tile_rows / waves) x k_splits, and a block
needs batch / 8 waves, 4 in place of 3 (each thread loads at most 4 x pieces per K
tile). The launch shape fixes the order of every sum, so the fused kernel and
its raw twin agree bit for bit under one configuration. The default
configuration itself is computed by the library (se12_default_launch) from
the device's CU count.
"""

from __future__ import annotations

import dataclasses

WAVE_SIZE = 64
WAVES_PER_BLOCK_CANDIDATES = (1, 2, 3, 4, 6, 8, 9, 12, 16)
K_SPLIT_CANDIDATES = (1, 2, 3, 4, 6, 8, 9, 12, 16, 18, 24, 32, 36, 48, 64)
MAX_K_SPLITS = 64
# BF16 activations with this many rows or more take the batched MFMA kernel:
# one launch over all rows, at most 8 waves per block and 16 K splits
MFMA_MIN_BATCH = 5
MFMA_MAX_K_SPLITS = 16
MFMA_MAX_WAVES = 8
MFMA_MAX_WAVES_GENERIC = 4   # the edge-handling MFMA variants (K % 256 != 0 or unaligned x)
# The resident-x MFMA kernel: every MFMA batch (MFMA_MIN_BATCH BF16 rows or
# more) on FAST shapes whose x (batch x K BF16, in whole 1 KiB loads) fits a
# block's LDS (gfx950: 160 KiB) beside the 1 KiB pair table; and 17..32 rows
# whose first 16 fit, on matrices of at most one tile row per CU (batch group
# 1's x then comes from global memory, at most RX_MAX_WAVES_XG waves per
# block). A single matrix whose x fits neither way can split K: split s of S
# takes K tiles [s TC / S, (s + 1) TC / S) of every row and holds only their
# columns of x (the fewest splits that fit, 2..RX_MAX_SPLITS, but 2 at 16 or
# fewer batch rows only on 8192+ tiles; the library adds the splits'
# partial sums in split order). Its launch is (waves per block 1..12, blocks
# per matrix and split 1..tile rows) with blocks = that count x splits x
# matrices; the launch fixes the K groups (rx_kgroups) and with them the order
# of every sum.
RX_MAX_WAVES = 12
RX_MAX_WAVES_XG = 8
RX_MAX_SPLITS = 8
COMPUTE_UNITS = 256  # MI355X; the library uses the device's count
LDS_PER_BLOCK = 160 * 1024
LUT_BYTES = 1024
RX_BLOCK_CANDIDATES = (32, 64, 128, 192, 256, 384, 512, 768, 1024)


@dataclasses.dataclass(frozen=True)
class ThreadsPerBlock:
    value: int


@dataclasses.dataclass(frozen=True)
class BlockCount:
    value: int


@dataclasses.dataclass(frozen=True)
class LaunchConfiguration:
    threads_per_block: ThreadsPerBlock
    blocks: BlockCount


@dataclasses.dataclass(frozen=True)
class GemvShape:
    output_rows: int
    batch_size: int


def tile_rows(output_rows: int) -> int:
    return -(-output_rows // 16)


def k_tiles(k: int) -> int:
    return -(-k // 256)


def uses_mfma(batch: int, float32_activations: bool = False) -> bool:
    return not float32_activations and batch >= MFMA_MIN_BATCH


def mfma_min_waves(batch: int) -> int:
    """Tile rows (waves) per block of the x-slab MFMA kernel: batch / 8
    rounded up, and 4 in place of 3."""
    r = -(-batch // 8)
    return 4 if r == 3 else r


def rx_lds_bytes(k: int, batch: int) -> int:
    """LDS of the resident x: batch x K BF16 in whole 64-piece loads of 16 bytes."""
    return -(-(batch * (k // 8)) // 64) * 64 * 16


def rx_layout(output_rows: int, k: int, batch: int, float32_activations: bool = False, aligned_x: bool = True,
              compute_units: int = COMPUTE_UNITS) -> tuple[int, int]:
    """(rows of x the resident-x kernel keeps in LDS, K splits) of a launch
    over one matrix (the library's rule): (batch, 1) where x fits, except
    on rows of 32+ K tiles with at most 5/8 of the CUs' worth of tile rows;
    (16, 1) for 17..32 rows whose first 16 fit on a matrix of at most one
    tile row per CU; (batch, S) with the fewest K splits S whose share of x's
    columns fits, except S = 2 at 16 or fewer rows on fewer than 8192 tiles;
    else (0, 0), the x-slab kernel."""
    if not (uses_mfma(batch, float32_activations) and aligned_x
            and not runs_generic(output_rows, k, float32_activations)):
        return 0, 0
    if rx_lds_bytes(k, batch) + LUT_BYTES <= LDS_PER_BLOCK:
        if 8 * tile_rows(output_rows) <= 5 * compute_units and k_tiles(k) >= 32:
            return 0, 0
        return batch, 1
    if batch > 16 and rx_lds_bytes(k, 16) + LUT_BYTES <= LDS_PER_BLOCK and tile_rows(output_rows) <= compute_units:
        return 16, 1
    tc = k_tiles(k)
    for s in range(2, min(RX_MAX_SPLITS, tc) + 1):
        if rx_lds_bytes(-(-tc // s) * 256, batch) + LUT_BYTES <= LDS_PER_BLOCK:
            if s == 2 and batch <= 16 and tile_rows(output_rows) * tc < 8192:
                return 0, 0
            return batch, s
    return 0, 0


def rx_staged_rows(output_rows: int, k: int, batch: int, float32_activations: bool = False, aligned_x: bool = True,
                   compute_units: int = COMPUTE_UNITS) -> int:
    """Rows of x the resident-x kernel keeps in LDS (rx_layout); 0 where the
    x-slab kernel serves the launch."""
    return rx_layout(output_rows, k, batch, float32_activations, aligned_x, compute_units)[0]


def rx_splits(output_rows: int, k: int, batch: int, float32_activations: bool = False, aligned_x: bool = True,
              compute_units: int = COMPUTE_UNITS) -> int:
    """K splits of a resident-x launch over one matrix (rx_layout); 0 where
    the x-slab kernel serves the launch."""
    return rx_layout(output_rows, k, batch, float32_activations, aligned_x, compute_units)[1]


def uses_rx(output_rows: int, k: int, batch: int, float32_activations: bool = False, aligned_x: bool = True,
            compute_units: int = COMPUTE_UNITS) -> bool:
    """Whether a launch runs the resident-x MFMA kernel (the library's rule)."""
    return rx_staged_rows(output_rows, k, batch, float32_activations, aligned_x, compute_units) > 0


def rx_max_waves(output_rows: int, k: int, batch: int, compute_units: int = COMPUTE_UNITS) -> int:
    """Waves per block of the resident-x kernel: 12, or 8 where batch group
    1's x comes from global memory."""
    staged = rx_staged_rows(output_rows, k, batch, compute_units=compute_units)
    return RX_MAX_WAVES_XG if 0 < staged < batch else RX_MAX_WAVES


def rx_kgroups(output_rows: int, k: int, waves: int, blocks_per_matrix: int, splits: int = 1) -> int:
    """K groups of a resident-x launch (the library's rule): the largest power
    of two that divides the waves per block, leaves every group at least two
    of its split's K tiles and keeps each row slot (blocks per matrix and
    split x waves / groups) to one row; one group from 3 tile rows per
    block."""
    tr, tc, kg = tile_rows(output_rows), k_tiles(k) // splits, 1
    if tr >= 3 * blocks_per_matrix:
        return kg
    while waves % (2 * kg) == 0 and tc >= 4 * kg and blocks_per_matrix * (waves // (2 * kg)) >= tr:
        kg *= 2
    return kg


def rx_configuration(waves: int, blocks_per_matrix: int, matrices: int = 1, splits: int = 1) -> LaunchConfiguration:
    """A resident-x launch: `blocks_per_matrix` blocks per matrix and K split."""
    return LaunchConfiguration(threads_per_block=ThreadsPerBlock(waves * WAVE_SIZE),
                               blocks=BlockCount(blocks_per_matrix * splits * matrices))


def grid_rows(output_rows: int, waves: int, batch: int = 1, float32_activations: bool = False) -> int:
    """Blocks per K split: one per tile row, or (MFMA) one per
    mfma_min_waves(batch) tile rows, whatever the waves per block (a block's
    waves are its tile rows times its K groups)."""
    tr = tile_rows(output_rows)
    return -(-tr // mfma_min_waves(batch)) if uses_mfma(batch, float32_activations) else tr


def configuration(waves: int, k_splits: int, output_rows: int, batch: int = 1,
                  float32_activations: bool = False) -> LaunchConfiguration:
    return LaunchConfiguration(
        threads_per_block=ThreadsPerBlock(waves * WAVE_SIZE),
        blocks=BlockCount(grid_rows(output_rows, waves, batch, float32_activations) * k_splits),
    )


def runs_generic(output_rows: int, k: int, float32_activations: bool = False) -> bool:
    """Whether the kernels take their edge-handling variants: FP32 x, K not a
    whole number of 256-column tiles, or (for the raw twin) output rows not a
    whole number of 16-row tiles."""
    return float32_activations or k % 256 != 0 or output_rows % 16 != 0


def max_k_splits(batch: int, float32_activations: bool = False) -> int:
    return MFMA_MAX_K_SPLITS if uses_mfma(batch, float32_activations) else MAX_K_SPLITS


def max_waves_per_block(batch: int, float32_activations: bool = False, generic: bool = False) -> int:
    """16 wave64s (1024 threads), or 8 where a launch needs more registers per
    lane: 4 batch rows per launch, 2-4 rows in the edge-handling variants, or
    the batched MFMA kernel."""
    if uses_mfma(batch, float32_activations):
        return MFMA_MAX_WAVES_GENERIC if generic else MFMA_MAX_WAVES
    b = min(batch, 4)
    if generic or float32_activations:
        return 8 if b >= 2 else 16
    return 8 if b >= 4 else 16


def waves_and_splits(launch: LaunchConfiguration, output_rows: int, batch: int = 1, k: int | None = None,
                     float32_activations: bool = False, compute_units: int = COMPUTE_UNITS) -> tuple[int, int]:
    """(waves per block, K splits) of a configuration for a matrix with
    `output_rows` rows; for the resident-x kernel (K given), (waves per
    block, blocks), whose K splits the shape fixes (rx_splits)."""
    tpb = launch.threads_per_block.value
    blocks = launch.blocks.value
    if k is not None and uses_rx(output_rows, k, batch, float32_activations, compute_units=compute_units):
        mw = rx_max_waves(output_rows, k, batch, compute_units)
        if tpb % WAVE_SIZE or not WAVE_SIZE <= tpb <= WAVE_SIZE * mw:
            raise ValueError(f"threads_per_block {tpb} must be a multiple of 64 in [64, {WAVE_SIZE * mw}]")
        sp = rx_splits(output_rows, k, batch, float32_activations, compute_units=compute_units)
        if blocks % sp or not 1 <= blocks // sp <= tile_rows(output_rows):
            raise ValueError(f"blocks {blocks} must be {sp} K splits x 1..{tile_rows(output_rows)}")
        return tpb // WAVE_SIZE, blocks
    generic = runs_generic(output_rows, k, float32_activations) if k is not None else float32_activations
    hi = WAVE_SIZE * max_waves_per_block(batch, float32_activations, generic)
    lo = WAVE_SIZE * (mfma_min_waves(batch) if uses_mfma(batch, float32_activations) else 1)
    if tpb % WAVE_SIZE or not lo <= tpb <= hi:
        raise ValueError(f"threads_per_block {tpb} must be a multiple of 64 in [{lo}, {hi}]")
    if uses_mfma(batch, float32_activations) and (tpb // WAVE_SIZE) % mfma_min_waves(batch):
        raise ValueError(f"the MFMA kernel takes a multiple of {mfma_min_waves(batch)} waves per block at batch {batch}")
    rows = grid_rows(output_rows, tpb // WAVE_SIZE, batch, float32_activations)
    if blocks <= 0 or blocks % rows:
        raise ValueError(f"blocks {blocks} must be a positive multiple of {rows}")
    return tpb // WAVE_SIZE, blocks // rows


def from_reference_configuration(launch, output_rows: int, k: int, batch: int = 1, float32_activations: bool = False,
                                 aligned_x: bool = True, compute_units: int = COMPUTE_UNITS) -> LaunchConfiguration:
    """This kernel's configuration for a launch built with the reference's
    meaning: one 32-lane warp per output element, `threads_per_block` in
    32..1024, and `blocks` x warps per block covering rows x batch
    (lws/domain/launch/heuristic.py:46-87; the tuner's candidates,
    search_space.py:14-36). The translation keeps the block's threads
    (rounded up to whole wave64s, and for the MFMA kernel to a multiple of the
    batch's tile rows per block, within the variant's limit) and splits no K
    tiles, as the reference kernel never does. A launch that leaves outputs
    uncovered, which the reference kernel would leave unwritten, is refused.
    `compute_units` is the count the library's kernel choice uses (the
    adapter's sm_count)."""
    tpb = int(launch.threads_per_block.value)
    blocks = int(launch.blocks.value)
    if tpb % 32 or not 32 <= tpb <= 1024:
        raise ValueError(f"threads_per_block {tpb} must be a multiple of 32 in [32, 1024]")
    if blocks <= 0 or blocks * (tpb // 32) < output_rows * batch:
        raise ValueError(f"{blocks} blocks of {tpb // 32} warps do not cover {output_rows} rows x batch {batch}")
    if uses_rx(output_rows, k, batch, float32_activations, aligned_x, compute_units):
        waves = min(-(-tpb // WAVE_SIZE), rx_max_waves(output_rows, k, batch, compute_units))
        return rx_configuration(waves, -(-tile_rows(output_rows) // waves),
                                splits=rx_splits(output_rows, k, batch, float32_activations, aligned_x, compute_units))
    mfma = uses_mfma(batch, float32_activations)
    generic = runs_generic(output_rows, k, float32_activations) or not aligned_x
    hi = max_waves_per_block(batch, float32_activations, generic)
    waves = -(-tpb // WAVE_SIZE)
    if mfma:
        lo = mfma_min_waves(batch)
        waves = -(-waves // lo) * lo
        hi = hi // lo * lo
    return configuration(min(waves, hi), 1, output_rows, batch, float32_activations)


def candidate_configurations(output_rows: int, k: int, batch: int = 1, float32_activations: bool = False,
                             compute_units: int = COMPUTE_UNITS) -> tuple[LaunchConfiguration, ...]:
    """Every (waves, splits) worth timing: waves per block up to the batch's
    limit (valid for the fused kernel and its raw twin alike), K splits up to
    the K tiles; for the dot2 kernel never more waves than tiles per split
    (search_space.py:17-19 enumerates threads per block the same way)."""
    tc = k_tiles(k)
    if uses_rx(output_rows, k, batch, float32_activations, compute_units=compute_units):
        tr = tile_rows(output_rows)
        sp = rx_splits(output_rows, k, batch, float32_activations, compute_units=compute_units)
        out = []
        for waves in (w for w in (1, 2, 3, 4, 6, 8, 12) if w <= rx_max_waves(output_rows, k, batch, compute_units)):
            # every candidate block count up to the tile rows, the tile rows
            # themselves (one row slot per block holds them all: the default
            # where they are fewer than the CUs) and one row per slot; with K
            # splits (one block per CU: each holds most of the LDS) up to the
            # CUs' share of a split
            ps = {b for b in RX_BLOCK_CANDIDATES if b <= tr} | {tr, -(-tr // waves)}
            if sp > 1:
                ps = {p for p in ps if p * sp <= compute_units} | {min(tr, compute_units // sp)}
            for p in sorted(ps):
                out.append(rx_configuration(waves, p, splits=sp))
        return tuple(out)
    mfma = uses_mfma(batch, float32_activations)
    mw = max_waves_per_block(batch, float32_activations, runs_generic(output_rows, k, float32_activations))
    lo = mfma_min_waves(batch) if mfma else 1
    splits = [s for s in K_SPLIT_CANDIDATES if s <= min(tc, max_k_splits(batch, float32_activations))]
    out = []
    for waves in WAVES_PER_BLOCK_CANDIDATES:
        if not lo <= waves <= mw or (mfma and waves % lo):
            continue
        for s in splits:
            if mfma or waves <= -(-tc // s):
                out.append(configuration(waves, s, output_rows, batch, float32_activations))
    return tuple(out)


@dataclasses.dataclass(frozen=True)
class TimingAndAccuracy:
    median_latency_microseconds: float
    passes_accuracy_check: bool


@dataclasses.dataclass(frozen=True)
class TimedCandidate:
    configuration: LaunchConfiguration
    measurement: TimingAndAccuracy


def best_configuration(timed: tuple[TimedCandidate, ...]) -> LaunchConfiguration | None:
    """Fastest configuration that passed the accuracy check (search_space.py:51-58)."""
    passing = [c for c in timed if c.measurement.passes_accuracy_check]
    if not passing:
        return None
    return min(passing, key=lambda c: c.measurement.median_latency_microseconds).configuration


def order_matched_configuration(raw_timed: tuple[TimedCandidate, ...], fused_timed: tuple[TimedCandidate, ...]) -> LaunchConfiguration | None:
    """One configuration shared by the raw twin and the fused kernel with the
    best combined time, both passing accuracy (search_space.py:61-75): with
    one launch shape the two give bit-identical FP32 outputs."""
    raw_ok = {c.configuration: c.measurement.median_latency_microseconds for c in raw_timed if c.measurement.passes_accuracy_check}
    fused_ok = {c.configuration: c.measurement.median_latency_microseconds for c in fused_timed if c.measurement.passes_accuracy_check}
    shared = [cfg for cfg in raw_ok if cfg in fused_ok]
    if not shared:
        return None
    return min(shared, key=lambda cfg: raw_ok[cfg] + fused_ok[cfg])
