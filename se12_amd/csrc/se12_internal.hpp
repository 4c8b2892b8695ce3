// Kernel argument blocks and launch entry points shared between the kernel
// translation units and the C ABI (se12_abi.hip). Host and device code.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace se12 {

struct GemvArgs {
    const uint8_t* sm;
    const uint8_t* ec;
    const uint32_t* lut;      // [256] pair table built at bind time
    const uint32_t* side;     // [T, 16] per-tile side records
    const int16_t* fb_raw;
    const int16_t* ovf_raw;   // tiles with too many escapes, decoded at bind
    const uint16_t* wraw;     // raw twin: row-major [N, K] BF16 bits
    const void* x;            // [B, K] BF16 or FP32
    float* y;                 // [B, N]
    float* partial;           // [S, B, Np] split-K partial sums
    int32_t* counters;        // [TR] arrival counters (zero between launches)
    uint64_t* pairs;          // [S - 1, B, Np] split-K pair slots (zero between launches)
    int64_t N, K, Np;
    int32_t TR, TC;
    int32_t S;                // K splits per tile row
};

// One launch over up to kMaxGroup matrices that share x (same K): the
// kernels take the matrix from blockIdx.z; tr_start[i] counts the grid rows
// (tile rows, or MFMA row blocks) of the matrices before i, tr_start[count]
// their total (the launch's `blocks` = that total x K splits).
constexpr int kMaxGroup = 4;

// Decode-step work done at the tail of a dot2 GEMV launch by the block that
// completes its inputs (arrival counters after the matrix's split-K
// counters: [TR, 2 TR) per tile row pair, [2 TR] for the whole matrix):
//   kEpiGeluMul  two matrices of one N (gate, up): the block completing a
//                tile row pair writes out = bf16(gelu_tanh(bf16(y0)) * bf16(y1))
//                for its 16 rows;
//   kEpiRmsNorm  one matrix with rows % 4 == 0 and 8-byte aligned y, w1,
//                w2, residual and out: the block completing the last tile
//                row runs, per batch row, residual = bf16(residual +
//                norm(bf16(y), w1)), out = norm(residual, w2).
constexpr int kEpiNone = 0;
constexpr int kEpiGeluMul = 1;
constexpr int kEpiRmsNorm = 2;

struct GemvEpilogue {
    int32_t kind;
    float eps;
    const uint16_t* w1;       // [N] BF16
    const uint16_t* w2;       // [N] BF16
    uint16_t* residual;       // [B, N] BF16
    uint16_t* out;            // [B, N] BF16
    // any kind, single-matrix dot2 launches: when not NULL, the block that
    // completes tile row t also writes row_ss[b, t] = the sum over its 16
    // rows n < N of bf16(y[b, n])^2 (a 16-lane DPP tree), the first sum of
    // squares of the decoder's next norm
    float* row_ss;            // [B, TR]
};

// Decode-step work done at the head of a dot2 GEMV launch (the XN kernel
// variants): instead of reading x, every block rebuilds it from the previous
// product's FP32 output y_prev, for each batch row,
//   r = bf16(residual_in + norm(bf16(y_prev), w1)),  x = norm(r, w2)
// (norm(t, w) = t * rsqrt(mean(t^2) + eps) * (1 + w)), into LDS; block
// (0, 0) also writes r to residual_out and x to h_out. residual_in and
// residual_out must not overlap (the launch's other blocks still read
// residual_in).
struct GemvPrologue {
    const float* y_prev;      // [B, K]
    const float* y_prev_ss;   // [B, ceil(K / 16)] row_ss of y_prev's product, or NULL
    const uint16_t* w1;       // [K] BF16
    const uint16_t* w2;       // [K] BF16
    const uint16_t* res_in;   // [B, K] BF16
    uint16_t* res_out;        // [B, K] BF16
    uint16_t* h_out;          // [B, K] BF16
    float eps;
};

struct GemvGroupArgs {
    GemvArgs m[kMaxGroup];
    int32_t tr_start[kMaxGroup + 1];
    int32_t count;
    int32_t rows_per_block;   // MFMA: tile rows per block (waves = rows x K groups)
    GemvEpilogue epi;         // dot2 launches only
    GemvPrologue pro;         // XN variants only
};

// The launch grid of a group: x = the tallest matrix's tile rows (row blocks
// for the MFMA kernel), y = K splits, z = matrix.
inline int32_t group_grid_x(const GemvGroupArgs& a) {
    int32_t x = 0;
    for (int i = 0; i < a.count; ++i) x = a.tr_start[i + 1] - a.tr_start[i] > x ? a.tr_start[i + 1] - a.tr_start[i] : x;
    return x;
}

// Dynamic LDS of an XN launch, in 16-byte aligned pieces: the cross-wave
// reduction, the prologue's staged inputs (y_prev FP32 and residual_in BF16
// per batch row, w1 and w2), and x of the batch rows (BF16).
constexpr size_t lds_align16(size_t n) { return (n + 15) / 16 * 16; }
constexpr size_t gemv_pro_x_bytes(int64_t k, int batch) { return (size_t)k * batch * 2; }
constexpr size_t gemv_pro_ss_bytes(int64_t k, int batch) { return lds_align16((size_t)batch * ((k + 15) / 16) * 4); }
constexpr size_t gemv_pro_stage_bytes(int64_t k, int batch) {
    return (size_t)k * (batch * 4 + batch * 2 + 4) + gemv_pro_ss_bytes(k, batch);
}
inline size_t gemv_xn_lds_bytes(int64_t k, int batch, int waves) {
    return lds_align16(gemv_pro_x_bytes(k, batch)) + lds_align16((size_t)waves * batch * 16 * sizeof(float)) +
           gemv_pro_stage_bytes(k, batch);
}

// arrival counters a handle holds: split-K per tile row, the epilogues' per
// tile row pair and per matrix
constexpr int64_t gemv_counter_count(int64_t tr) { return 2 * tr + 1; }
// dynamic LDS of the kEpiRmsNorm tail: the row in FP32, w1 / residual / w2
// as BF16, 32 floats for the block sums
constexpr size_t gemv_norm_lds_bytes(int64_t n) { return (size_t)n * 10 + 32 * sizeof(float); }

// How one GEMV launch runs: the launch shape (waves per block, blocks =
// tile rows x splits) fixes the results; the variant (tiles per round `g`,
// prefetch `pf`, `generic` edge handling) only changes speed.
struct GemvPlan {
    int batch;
    bool xf32;
    bool raw;
    bool generic;
    bool xn;  // x rebuilt by the prologue (GemvPrologue)
    int g;
    int pf;  // rounds in flight ahead of the decoded one (0 or 1)
    int waves;
    int blocks;
    size_t lds;
    int xg;       // resident-x kernel: batch group 1's x from global memory (0 / 1)
    int ksplits;  // resident-x kernel: K splits (grid y), each holding its columns of x
    int slab_ring;  // x-slab kernel: steps between block barriers (0: one per step)
};

struct DecodeArgs {
    const uint8_t* sm;
    const uint8_t* ec;
    const uint8_t* esc;
    const uint8_t* codebook;
    const uint8_t* bitmap;
    const uint32_t* lut;      // [256] pair table built at bind time
    const uint32_t* info;     // [T] per-tile sidecar word
    const uint4* escpos;      // [T] listed escape positions
    const uint32_t* side;     // [T, 16] per-tile side records
    const int16_t* fb_raw;
    const int16_t* ovf_raw;
    const int64_t* rows;      // decode_rows only
    uint16_t* out;
    int64_t N, K, T, nrows, items;
    int32_t TR, TC;
    int32_t out_vec_ok;
};

struct EncodeArgs {
    const uint16_t* w;
    int64_t N, K, ld;
    int32_t TR, TC;
    int64_t T;
    uint32_t codebook[4];     // 15 bytes, little-endian packed
    uint64_t* histogram;      // [256]
    int32_t* tile_escapes;    // [T]
    int32_t* fb_rank;         // [T]
    int64_t* totals;          // [1] fallback tile count
    uint8_t* sm;
    uint8_t* ec;
    uint8_t* esc;
    uint8_t* bitmap;
    int16_t* raw;
    int32_t w_vec_ok;
};

constexpr int kGemvMaxBatchPerLaunch = 4;
constexpr int kLutBytes = 1024;

// Largest block (threads) of a GEMV kernel variant, from its VGPR demand
// (512 VGPRs per SIMD lane: 1024 threads = 4 waves per SIMD = 128 VGPRs
// each, 512 threads = 256). The FAST estimates are fitted to hipcc's
// allocation (per round: a tile's streams + its x slice, 37 VGPRs at batch 1,
// 40 for the raw twin; 8 more per extra batch row; the fused batch-1 kernel
// takes 85 / 122 without / with prefetch, so its prefetching variant fits
// 1,024 threads); the GENERIC variants run one tile per round without
// prefetch. The build fails if any variant spills.
// `pf` = rounds kept in flight ahead of the one being decoded (0 or 1).
constexpr int gemv_vgpr_estimate(int batch, bool raw, int g, int pf) {
    return raw          ? 24 + 4 * (batch - 1) + (pf + 1) * g * (40 + 8 * (batch - 1))
           : batch == 1 ? 48 + (pf + 1) * g * 37
                        : 57 + 4 * (batch - 1) + (pf + 1) * g * (37 + 8 * (batch - 1));
}
constexpr int gemv_max_threads(int batch, bool xf32, bool raw, int g, int pf, bool generic) {
    return generic ? (batch >= 2 ? 512 : 1024)
                   : gemv_vgpr_estimate(batch, raw, g, pf) <= 128 ? 1024
                   : gemv_vgpr_estimate(batch, raw, g, pf) <= 256 ? 512 : 256;
}

// Minimum waves per SIMD the compiler must leave room for (register
// allocation target) for the variants whose occupancy sits on a VGPR
// granule boundary: the batch-1 single-tile rounds at 5 waves (96 VGPRs),
// two tiles per round at 4 (128). 1 = no target.
constexpr int gemv_waves_per_simd(int batch, bool raw, int g, int pf, bool generic) {
    return (raw || generic || batch != 1 || pf) ? 1 : g == 1 ? 5 : g == 2 ? 4 : 1;
}

// bytes of dynamic LDS a GEMV launch needs (the cross-wave reduction; the
// 1 KiB pair table is static)
inline size_t gemv_lds_bytes(int waves, int batch) { return (size_t)waves * batch * 16 * sizeof(float); }

hipError_t launch_gemv(const GemvGroupArgs& a, const GemvPlan& p, hipStream_t stream);
hipError_t launch_row_sumsq(const float* y, int64_t N, int32_t TR, int32_t batch, float* row_ss, hipStream_t stream);

// Batched path (se12_gemm.hip): BF16 x with kGemmMinBatch..32 rows runs one
// MFMA launch over all rows (one pass over the weights) instead of one
// dot2 launch per 4 rows. A block is 1..8 waves, one tile row each, and
// loads each x slab (batch x 256 BF16) with at most kGemmXPieces 16-byte
// pieces per thread, so it needs at least batch / 8 waves; at most
// kGemmMaxSplits K splits. The grid's x dimension counts row blocks
// (ceil(tile rows / rows per block) per matrix), and tr_start is in those
// units.
constexpr int kGemmMinBatch = 5;
constexpr int kGemmMaxThreads = 512;
// the edge-handling (GENERIC) MFMA variants, whose element-wise loads need
// more registers, take at most 4 waves per block (enough for 32 batch rows)
constexpr int kGemmMaxThreadsGeneric = 256;

constexpr int kGemmMaxSplits = 16;
constexpr int kGemmXPieces = 4;
// tile rows per block: the fewest waves whose threads load a batch x 256 x
// slab (batch / 8, rounded up), rounded up to a power of two (3 waves leave a
// SIMD of the CU without a row: 14336x3584 at B = 24 took 32.4 us with 3,
// B = 32 26.2 with 4)
constexpr int gemm_min_waves(int batch) {
    return (batch * 32 + 64 * kGemmXPieces - 1) / (64 * kGemmXPieces) == 3 ? 4
                                                                            : (batch * 32 + 64 * kGemmXPieces - 1) /
                                                                                  (64 * kGemmXPieces);
}
// The FAST variants' x slabs on launches of kGemmSlabRingMinSteps or more
// steps, where LDS allows: a ring of 2 M buffers per K group (M =
// kGemmSlabRing), each step's slab stored M steps before its use and one
// block barrier every M steps (se12_gemm.hip); otherwise two buffers and a
// barrier per step (slab_ring 0). Shorter launches keep the short prologue
// (2304x9216 B = 16, 6 steps: 17.0 us with a barrier per step against 17.8
// with the ring), and so do launches whose ring of 8 does not fit (a ring of
// 4 with two K groups was slower than a barrier per step: 4608x36864 B = 24
// / 32 78.4 / 81.5 us against 76.3 / 79.8).
constexpr int kGemmSlabRing = 4;
constexpr int kGemmSlabRingMinSteps = 12;
size_t gemm_lds_bytes(int waves, int batch, int slab_ring);
hipError_t launch_gemm(const GemvGroupArgs& a, int batch, const GemvPlan& p, hipStream_t stream);

// Resident-x batched path (se12_gemm_rx.hip): BF16 x with up to 32 rows on
// FAST shapes whose x (batch x K BF16, in whole 64-piece loads of 16 bytes)
// fits a block's LDS beside the pair table (se12_abi.hip's rx_fits). Blocks
// of 1..12 waves, any block count per matrix (blocks = that count x
// matrices); each row's K groups (GemvArgs::S holds them on this path) are
// fixed by the launch shape
// (rx_kgroups). kRxDepth tiles in flight per wave, up to 3 waves per SIMD
// (168 VGPRs: the decode, a tile in flight and the transposed tile in use).
constexpr int kRxMaxThreads = 768;
// with batch group 1's x from global memory: 2 waves per SIMD (210 VGPRs)
constexpr int kRxMaxThreadsXG = 512;
constexpr int kRxDepth = 2;
// K splits of a resident-x launch whose x does not fit (each split holds its
// share of x's columns): more splits measured slower than the x-slab kernel
constexpr int kRxMaxSplits = 8;
// K groups of the resident-x kernel for one matrix: the largest power of two
// that divides the waves per block, leaves each group at least two K tiles,
// and keeps every row slot (blocks x waves / KG of them) to at most one row;
// one group from 3 tile rows per block, where the rows already keep the
// waves busy (14336x3584 B = 16, 12 waves x 256 blocks: 20.7 us with one
// group against 22.6 with two).
constexpr int rx_kgroups(int64_t tile_rows, int32_t tile_cols, int32_t waves, int64_t blocks) {
    int kg = 1;
    if (tile_rows >= 3 * blocks) return kg;
    while (waves % (2 * kg) == 0 && tile_cols >= 4 * kg && blocks * (waves / (2 * kg)) >= tile_rows) kg *= 2;
    return kg;
}
constexpr size_t rx_lds_bytes(int64_t k, int batch) {
    return (size_t)(((int64_t)batch * (k / 8) + 63) / 64 * 64) * 16;
}
// dynamic LDS: x, or (the same memory, after the main loop) the K groups'
// sums, whichever is larger
// (staged = the rows of x held in LDS: all of the batch, or 16)
constexpr size_t rx_lds_total(int64_t k, int staged, int batch, int waves, int kgroups) {
    const size_t sums = kgroups > 1 ? (size_t)(waves - waves / kgroups) * (batch > 16 ? 2 : 1) * 1024 : 0;
    return rx_lds_bytes(k, staged) > sums ? rx_lds_bytes(k, staged) : sums;
}
hipError_t launch_gemm_rx(const GemvGroupArgs& a, int batch, const GemvPlan& p, hipStream_t stream);
hipError_t launch_decode(const DecodeArgs& a, bool rows, hipStream_t stream, int cu_count);
// Bind-time sidecar: one word per tile (fallback rank, or the chunks holding
// escape codes) and the fallback tile count.
// total[0] = fallback tiles, total[1] = tiles with more than the listed escapes
hipError_t launch_tile_info(const uint8_t* bitmap, const uint8_t* ec, int64_t T, uint32_t* info, uint4* escpos, int64_t* total,
                            hipStream_t stream);
hipError_t launch_overflow_decode(const DecodeArgs& a, int16_t* raw, hipStream_t stream);
hipError_t launch_side_records(const uint32_t* info, const uint8_t* esc, const uint4* escpos, int64_t T, uint32_t* side,
                               hipStream_t stream);
hipError_t launch_encode_histogram(const EncodeArgs& a, hipStream_t stream);
hipError_t launch_encode_count(const EncodeArgs& a, hipStream_t stream);
hipError_t launch_encode_scan(const EncodeArgs& a, hipStream_t stream);
hipError_t launch_encode_write(const EncodeArgs& a, hipStream_t stream);
// Streaming-read probe (se12_probe.hip): its grid for a device and the launch.
int64_t read_probe_blocks(int32_t compute_units);
hipError_t launch_read_probe(const void* buf, int64_t n16, uint32_t* out, int64_t blocks, hipStream_t stream);

}  // namespace se12
