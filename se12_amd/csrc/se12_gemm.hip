// Batched fused SE12 decode + matrix product for gfx950: Y[b, n] =
// sum_k W[n, k] X[b, k] for up to 32 BF16 batch rows in ONE pass over the
// weights (the dot2 kernel in se12_gemv.hip takes 4 rows per launch and so
// re-reads W once per 4 rows). Same semantics as the reference kernel
// lws/adapters/cuda/kernels/gemv_se12.cu:50-142 at batch B, which runs one
// warp per (row, batch) element and reads W B times.
//
// Grid: block = R x KG wave64s: R consecutive tile rows (R = ceil(batch / 8), 4 in place of 3,
// the fewest waves whose threads load an x slab in one go) times KG K groups;
// wave w owns tile row R * row_block + w % R and, of the split's K tiles, the
// ones of K group w / R (every KG-th tile). blockIdx.y = K split s covering
// the K tiles [s*TC/S, (s+1)*TC/S). A grouped launch serves up to 4 matrices
// with the same K: blockIdx.z = matrix, blockIdx.x = row block (the grid's x
// spans the tallest matrix; blocks past a shorter one's rows leave at once).
//
// Per step each K group's waves share one copy of their x slab (batch rows x
// 256 columns, BF16) in LDS: every thread requests up to 4 pieces of 16
// bytes of a later step's slabs while its wave decodes tile i and writes
// them to LDS after its MFMAs. Double-buffered with a block barrier per step
// (slabs of step i + 1 written during step i), or, on launches of 12 or more
// steps where LDS holds it, a ring of 8 slabs written 4 steps ahead with a
// barrier every 4 steps. Each wave requests its tile streams two tiles ahead
// of the decode (the edge-handling variants load and use in turn).
//
// FAST variants load each tile whole-line (a kilobyte of sm holding 4 tile
// rows per load instruction, as the resident-x kernel does) and move it into
// the block layout with DPP exchanges: lane l holds, in part p, the 16
// columns 16 (4 (l / 16) + p) .. + 15 of row l % 16, decoded through the
// pair table with listed escapes and raw tiles. Each part's first and second
// 8 columns are the A operands of two v_mfma_f32_16x16x32_bf16 (MFMA row =
// tile row); their K positions differ between lane groups, and the B
// operands (lane l: batch row 16 g + l % 16) read the same 8 columns of the
// x slab. GENERIC variants load row-wise: lane l takes row l % 16 and the 16
// columns 64 p + 16 (l / 16) .. + 15 of part p, and two lane-row swaps
// (v_permlane16_swap, v_permlane32_swap) leave each lane holding its A
// operands for the part's two 32-column slices s (lane l: columns 32 s + 8
// (l / 16) .. + 7). Either way the decoded tile never goes through memory;
// 8 MFMAs per tile and group of 16 batch rows, FP32 accumulate, in a fixed
// order. Rows of the LDS x slabs are padded to 528 bytes so that the 16-byte
// reads of 8 lanes per cycle hit distinct banks. Batch rows past the batch
// in a 16-row group read stale LDS: MFMA output column n depends on B column
// n only, and those columns are not stored.
//
// A wave adds its K tiles in ascending order; the K groups of a tile row are
// added in LDS in ascending group order by the group-0 wave, and for S > 1
// the last wave of a tile row to finish (device-scope arrival counter, reset
// by that wave) adds the S partials in ascending split order. The launch
// shape (W, S) fixes every sum: the raw-BF16 twin (same kernel, RAW) is
// bit-identical under one shape.
//
// FAST variants need K % 256 == 0 and 16-byte aligned x rows (and, for the
// raw twin, N % 16 == 0 and an aligned W); GENERIC variants guard loads by
// the matrix edges and zero weights and x past K (padding can decode to
// +inf when codebook[0] = 255).
#include <algorithm>

#include "se12_device.hpp"
#include "se12_internal.hpp"

namespace se12 {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float floatx4_t __attribute__((ext_vector_type(4)));

constexpr int kRowBytes = 528;                    // 512 B of BF16 + 16 B of padding

template <int BG>
constexpr int x_slab_bytes() {
    return 16 * BG * kRowBytes;
}

// the 16-byte pieces p = tid + k * threads (k < kGemmXPieces) of an x slab:
// batch row p / 32, columns 8 (p % 32) .. + 7
struct XPieces {
    uint4 v[kGemmXPieces];
};

// Every load here and below is issued unconditionally (indexes clamped into
// the matrix): a load skipped on some path leaves the compiler unable to
// count the loads in flight, and it then waits for all of them - the
// prefetched tiles included - before the next decode.
// The slabs of one step: K group g's slab is x at K tile kb + g + KG i
// (clamped into the split; a clamped slab is loaded but not used). Piece p
// of the step: group p / (batch * 32), batch row (p % (batch * 32)) / 32,
// columns 8 (p % 32) .. + 7.
template <bool GENERIC>
__device__ __forceinline__ XPieces load_x_slab(const GemvArgs& a, int batch, int kb, int n, int KG, int i, int tid,
                                               int threads) {
    XPieces xr;
    const int per = batch * 32;
#pragma unroll
    for (int k = 0; k < kGemmXPieces; ++k) {
        const int p = min(tid + k * threads, KG * per - 1);
        const int g = p / per, q = p - g * per;
        const int t = g + KG * i;
        const int kt = kb + (t < n ? t : n - 1);
        const uint16_t* row = static_cast<const uint16_t*>(a.x) + (int64_t)(q >> 5) * a.K;
        const int64_t col = (int64_t)kt * kTileCols + 8 * (q & 31);
        if constexpr (!GENERIC) {
            xr.v[k] = *reinterpret_cast<const uint4*>(row + col);
        } else {
            uint32_t e[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const uint32_t lo = row[min(col + 2 * t, a.K - 1)];
                const uint32_t hi = row[min(col + 2 * t + 1, a.K - 1)];
                e[t] = (col + 2 * t < a.K ? lo : 0u) | (col + 2 * t + 1 < a.K ? hi << 16 : 0u);
            }
            xr.v[k] = make_uint4(e[0], e[1], e[2], e[3]);
        }
    }
    return xr;
}

// pieces past the step's slabs repeat the last piece: the same bytes to the
// same address as the thread that owns it. Group g's slab sits at xb + g *
// slab_bytes.
__device__ __forceinline__ void store_x_slab(char* xb, int slab_bytes, const XPieces& xr, int batch, int KG, int tid,
                                             int threads) {
    const int per = batch * 32;
#pragma unroll
    for (int k = 0; k < kGemmXPieces; ++k) {
        const int p = min(tid + k * threads, KG * per - 1);
        const int g = p / per, q = p - g * per;
        *reinterpret_cast<uint4*>(xb + g * slab_bytes + (q >> 5) * kRowBytes + 16 * (q & 31)) = xr.v[k];
    }
}

// The row layout: lane l holds row l % 16 and, in part p, the 16 columns
// 64 p + 16 (l / 16) .. + 15 of the tile.
__device__ __forceinline__ int row_layout_col(int p, uint32_t lane) { return 64 * p + 16 * (int)(lane >> 4); }

// One tile's sm and ec bytes in the row layout (per part: 16 sm bytes, 8 ec
// bytes of the lane's row).
__device__ __forceinline__ void load_tile_rows(TileLoads& t, const uint8_t* sm, const uint8_t* ec, int64_t tile,
                                               uint32_t lane) {
    const uint8_t* smt = sm + tile * kTile + (lane & 15u) * kTileCols + 16u * (lane >> 4);
    const uint8_t* ect = ec + tile * (kTile / 2) + (lane & 15u) * (kTileCols / 2) + 8u * (lane >> 4);
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        t.sm[p] = *reinterpret_cast<const uint4*>(smt + 64 * p);
        t.ec[p] = *reinterpret_cast<const uint2*>(ect + 32 * p);
    }
}

// Raw BF16 of part p of a raw tile (tile-local row-major) in the row layout.
__device__ __forceinline__ void load_raw_part(const int16_t* tile_raw, int p, uint32_t lane, uint32_t w[8]) {
    const uint4* q = reinterpret_cast<const uint4*>(tile_raw + (lane & 15u) * kTileCols + row_layout_col(p, lane));
    const uint4 a = q[0], b = q[1];
    w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
    w[4] = b.x; w[5] = b.y; w[6] = b.z; w[7] = b.w;
}

// The lane's 16 decoded weights of a part (8 BF16 pairs: w[0..3] columns
// c..c+7, w[4..7] columns c+8..c+15) become the A operands of the part's two
// slices: a v_permlane16_swap (odd rows of the first register with even rows
// of the second) and a v_permlane32_swap (upper half of the first with lower
// half of the second) per register pair.
__device__ __forceinline__ void rows_to_operands(const uint32_t w[8], bf16x8_t& a0, bf16x8_t& a1) {
    uint32_t u[4], v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const auto s16 = __builtin_amdgcn_permlane16_swap(w[i], w[4 + i], false, false);
        const auto s32 = __builtin_amdgcn_permlane32_swap(s16[0], s16[1], false, false);
        u[i] = s32[0];
        v[i] = s32[1];
    }
    a0 = __builtin_bit_cast(bf16x8_t, make_uint4(u[0], u[1], u[2], u[3]));
    a1 = __builtin_bit_cast(bf16x8_t, make_uint4(v[0], v[1], v[2], v[3]));
}

// Raw-twin rows in the row layout (per part: the lane's 16 columns).
template <bool GENERIC>
__device__ __forceinline__ void load_raw_rows(uint4 r[4][2], const GemvArgs& a, int tr, int kt, uint32_t lane) {
    const int64_t row = (int64_t)tr * kTileRows + (lane & 15u);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int64_t col = (int64_t)kt * kTileCols + row_layout_col(j, lane);
        if constexpr (!GENERIC) {
            const uint16_t* p = a.wraw + row * a.K + col;
            r[j][0] = reinterpret_cast<const uint4*>(p)[0];
            r[j][1] = reinterpret_cast<const uint4*>(p)[1];
        } else {
            const uint16_t* p = a.wraw + min(row, a.N - 1) * a.K;
            uint32_t h[8];
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const int64_t c = col + 2 * q;
                const uint32_t lo = p[min(c, a.K - 1)];
                const uint32_t hi = p[min(c + 1, a.K - 1)];
                h[q] = row < a.N ? ((c < a.K ? lo : 0u) | (c + 1 < a.K ? hi << 16 : 0u)) : 0u;
            }
            r[j][0] = make_uint4(h[0], h[1], h[2], h[3]);
            r[j][1] = make_uint4(h[4], h[5], h[6], h[7]);
        }
    }
}

// weights at columns >= lim of the tile are zeroed
__device__ __forceinline__ void zero_past_k(uint32_t w[8], int c0, int lim) {
#pragma unroll
    for (int q = 0; q < 8; ++q) {
        const int c = c0 + 2 * q;
        w[q] = (c >= lim) ? 0u : ((c + 1 >= lim) ? (w[q] & 0xFFFFu) : w[q]);
    }
}

// The MFMAs of part p (slices 2p and 2p + 1) for every batch group, the x
// slab (B operands) read from LDS.
template <int BG>
__device__ __forceinline__ void mfma_part(const bf16x8_t& a0, const bf16x8_t& a1, const char* xb, int p, uint32_t lane,
                                          floatx4_t acc[BG]) {
    const int off = (int)(lane & 15u) * kRowBytes + 16 * (int)(lane >> 4);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int s = 2 * p + h;
#pragma unroll
        for (int g = 0; g < BG; ++g) {
            const uint4 bv = *reinterpret_cast<const uint4*>(xb + g * 16 * kRowBytes + off + 64 * s);
            acc[g] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(h ? a1 : a0, __builtin_bit_cast(bf16x8_t, bv), acc[g], 0, 0,
                                                              0);
        }
    }
}

// The MFMAs of part p of a tile in the block layout (FAST variants; lane l
// holds row l % 16, columns 16 (4 (l / 16) + p) .. + 15 as 8 BF16 pairs):
// its first and second 8 columns are the A operands of two MFMAs whose B
// operands are the same 8 columns of the x slab (batch row 16 g + l % 16).
// The MFMA's K positions differ between lane groups; A and B agree on them.
template <int BG>
__device__ __forceinline__ void mfma_block_part(const uint32_t w[8], const char* xb, int p, uint32_t lane,
                                                floatx4_t acc[BG]) {
    const int off = (int)(lane & 15u) * kRowBytes + 128 * (int)(lane >> 4) + 32 * p;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const bf16x8_t av = __builtin_bit_cast(bf16x8_t, make_uint4(w[4 * h], w[4 * h + 1], w[4 * h + 2], w[4 * h + 3]));
#pragma unroll
        for (int g = 0; g < BG; ++g) {
            const uint4 bv = *reinterpret_cast<const uint4*>(xb + g * 16 * kRowBytes + off + 16 * h);
            acc[g] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, __builtin_bit_cast(bf16x8_t, bv), acc[g], 0, 0, 0);
        }
    }
}

template <bool RAW>
struct GemmTile {
    TileSide side;
    TileLoads t;
    uint4 r[RAW ? 4 : 1][2];
};

template <int BG, bool RAW, bool GENERIC, int M>
__global__ __launch_bounds__(GENERIC ? kGemmMaxThreadsGeneric : kGemmMaxThreads) void gemm_kernel(GemvGroupArgs ga,
                                                                                                  int batch) {
    static_assert(M == 0 || (!GENERIC && M >= 1), "the slab ring serves the FAST variants");
    SE12_DECLARE_LUT(lut);
    extern __shared__ __attribute__((aligned(16))) char gsm[];
    // the matrix comes from the grid; every argument the block needs goes out
    // in one batch of scalar loads (issued where first used, each would wait
    // behind the one before)
    const GemvArgs a = ga.m[blockIdx.z];
    const int threads = blockDim.x;
    const int R = ga.rows_per_block;
    asm volatile("" ::"s"(a.sm), "s"(a.ec), "s"(a.lut), "s"(a.side), "s"(a.wraw), "s"(a.x), "s"(a.y), "s"(a.K),
                 "s"(a.TR), "s"(a.TC), "s"(a.S), "s"(R), "s"(threads), "s"(batch));
    const int W = threads >> 6;
    const int KG = W / R;
    const int tid = threadIdx.x;
    const uint32_t lane = threadIdx.x & 63u;
    const int w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int kg = w / R;
    if ((int)blockIdx.x * R >= a.TR) return;  // past a shorter matrix of a grouped launch
    const int tr = (int)blockIdx.x * R + (w - kg * R);
    const bool active = tr < a.TR;
    const int trl = active ? tr : a.TR - 1;  // row the loads of an idle wave use
    const int S = a.S;
    const int s = blockIdx.y;
    const int kb = (int)(((uint32_t)s * (uint32_t)a.TC) / (uint32_t)S);
    const int ke = (int)(((uint32_t)(s + 1) * (uint32_t)a.TC) / (uint32_t)S);
    const int n = ke - kb;
    const int steps = (n + KG - 1) / KG;  // K group kg takes the split's tiles kg, kg + KG, ...
    const int64_t row_tiles = (int64_t)trl * a.TC;
    const int slab_bytes = x_slab_bytes<BG>();
    // [NB buffers][KG slabs] of x: two with a block barrier per step, or a
    // ring of 2 M with a barrier every M steps
    constexpr int NB = M > 0 ? 2 * M : 2;
    char* xbuf = gsm;

    floatx4_t acc[BG];
#pragma unroll
    for (int g = 0; g < BG; ++g) acc[g] = floatx4_t{0.0f, 0.0f, 0.0f, 0.0f};

    auto load_tile_i = [&](GemmTile<RAW>& t, int i) {
        const int j = kg + KG * i;
        const int kt = kb + (j < n ? j : n - 1);
        if constexpr (RAW && GENERIC) {
            load_raw_rows<true>(t.r, a, trl, kt, lane);
        } else if constexpr (RAW) {
            load_raw_blocks(t.r, a.wraw, a.K, trl, kt, lane);
        } else if constexpr (GENERIC) {
            load_side(t.side, a.side, row_tiles + kt, lane);
            load_tile_rows(t.t, a.sm, a.ec, row_tiles + kt, lane);
        } else {
            load_tile_block_order(t.t, t.side, a.sm, a.ec, a.side, row_tiles + kt, lane);
        }
    };
    auto use_tile = [&](GemmTile<RAW>& t, int i) {
        const int kt = kb + kg + KG * i;
        const char* xb = xbuf + ((i % NB) * KG + kg) * slab_bytes;
        if constexpr (GENERIC) {
            const int lim = (int)(a.K - (int64_t)kt * kTileCols);
            // one part: weights (row layout) -> A operands -> the part's MFMAs
            auto part = [&](int p, uint32_t wv[8]) {
                zero_past_k(wv, row_layout_col(p, lane), lim);
                bf16x8_t a0, a1;
                rows_to_operands(wv, a0, a1);
                mfma_part<BG>(a0, a1, xb, p, lane, acc);
            };
            if constexpr (RAW) {
#pragma unroll
                for (int p = 0; p < 4; ++p) {
                    uint32_t wv[8] = {t.r[p][0].x, t.r[p][0].y, t.r[p][0].z, t.r[p][0].w,
                                      t.r[p][1].x, t.r[p][1].y, t.r[p][1].z, t.r[p][1].w};
                    part(p, wv);
                }
            } else {
                const uint32_t info = side_info(t.side, 0);
                if (info_is_fallback(info)) {
                    const int16_t* raw = raw_tile_ptr(info, a.fb_raw, a.ovf_raw);
                    uint32_t wv[4][8];
#pragma unroll
                    for (int p = 0; p < 4; ++p) load_raw_part(raw, p, lane, wv[p]);
                    wait_vector_loads();  // rare path: keeps the common path's waits exact
#pragma unroll
                    for (int p = 0; p < 4; ++p) part(p, wv[p]);
                } else {
                    uint32_t pat[4][8];
                    lookup_tile(lut, t.t, pat);
                    patch_tile_escapes<kRowLayout>(pat, info, t.side, 0, lane);
#pragma unroll
                    for (int p = 0; p < 4; ++p) {
                        uint32_t wv[8];
                        merge_chunk(pat[p], t.t.sm[p], wv);
                        part(p, wv);
                    }
                }
            }
        } else if constexpr (RAW) {
            // block layout: each part's 16 columns are the A operands as loaded
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                const uint32_t wv[8] = {t.r[p][0].x, t.r[p][0].y, t.r[p][0].z, t.r[p][0].w,
                                        t.r[p][1].x, t.r[p][1].y, t.r[p][1].z, t.r[p][1].w};
                mfma_block_part<BG>(wv, xb, p, lane, acc);
            }
        } else {
            const uint32_t info = side_info(t.side, 0);
            if (info_is_fallback(info)) {
                const int16_t* raw = raw_tile_ptr(info, a.fb_raw, a.ovf_raw);
                uint32_t wv[4][8];
#pragma unroll
                for (int p = 0; p < 4; ++p) raw_block_part(raw, p, lane, wv[p]);
                wait_vector_loads();  // rare path: keeps the common path's waits exact
#pragma unroll
                for (int p = 0; p < 4; ++p) mfma_block_part<BG>(wv[p], xb, p, lane, acc);
            } else {
                // whole-line loads (4 tile rows per instruction) into the block
                // layout, in place (the slot is reloaded next); each part's
                // patterns merged with its sm bytes as soon as looked up;
                // escapes only set exponent bits, which the merge takes from
                // the patterns, so they patch the merged words
                chunks_to_blocks(t.t);
                uint32_t wv[4][8];
#pragma unroll
                for (int p = 0; p < 4; ++p) {
                    uint32_t pat[8];
                    lookup_chunk(lut, t.t.ec[p], pat);
                    merge_chunk(pat, t.t.sm[p], wv[p]);
                }
                patch_tile_escapes<kBlockLayout>(wv, info, t.side, 0, lane);
#pragma unroll
                for (int p = 0; p < 4; ++p) mfma_block_part<BG>(wv[p], xb, p, lane, acc);
            }
        }
    };

    uint4 lutv;
    if constexpr (!RAW) lutv = reinterpret_cast<const uint4*>(a.lut)[lane];
    __builtin_amdgcn_sched_barrier(0);
    // rings of three: tile i's streams are requested two steps before its
    // decode, x slab i's pieces two steps before they are stored to LDS
    // Tile streams and x pieces are requested D - 1 steps ahead of their
    // use (D = 3; the GENERIC variants, whose element-wise loads are packed
    // as they arrive, load and use in turn): under a full-bandwidth stream
    // even the L2 hits of x take about a step to return. The loop body holds
    // D steps so that every step's loads are issued on every path that goes
    // on (loads past the last tile reload it): a load skipped on some path
    // would make the compiler wait for all loads in flight. Slab i + 1 is
    // stored to LDS at the end of step i.
    constexpr int D = GENERIC ? 1 : 3;
    auto x_step = [&](int i) { return load_x_slab<GENERIC>(a, batch, kb, n, KG, i, tid, threads); };
    auto has_tile = [&](int i) { return kg + KG * i < n; };
    if constexpr (M > 0) {
        // Slab ring: the slabs of step j sit in buffer j % NB (NB = 2 M);
        // every thread stores its pieces of the slabs of step j during step
        // j - M (pieces requested one step before; the prologue stores steps
        // 0 .. M - 1), and the block meets only before steps M, 2 M, ...
        // Slab j is read at step j after the meeting before the multiple of M
        // in (j - M, j], so after every wave's store of it; storing slab j
        // during step j - M overwrites slab j - 2 M, which every wave read
        // before the meeting before the multiple of M in (j - 2 M, j - M].
        // Fewer meetings let the waves' tile
        // arrivals even out (14336x3584 B = 32: 24.5 us against 26.0 with one
        // per step).
        constexpr int L = M;
        auto buf = [&](int j) { return xbuf + (j % NB) * KG * slab_bytes; };
        GemmTile<RAW> t0, t1, t2;
        load_tile_i(t0, 0);
        load_tile_i(t1, 1);
        XPieces xp[L];
#pragma unroll
        for (int j = 0; j < L; ++j) xp[j] = x_step(j);
        XPieces x0 = x_step(L), x1, x2;
        if constexpr (!RAW) store_block_lut(lut, lutv, lane);
#pragma unroll
        for (int j = 0; j < L; ++j) store_x_slab(buf(j), slab_bytes, xp[j], batch, KG, tid, threads);
        lds_barrier();  // the pair table and the slabs of steps 0 .. L - 1 are in LDS
        auto step = [&](GemmTile<RAW>& cur, GemmTile<RAW>& ahead, const XPieces& x_next, XPieces& x_ahead, int i) {
            x_ahead = x_step(i + L + 1);
            load_tile_i(ahead, i + 2);
            if (i > 0 && i % M == 0) lds_barrier();
            if (has_tile(i)) use_tile(cur, i);  // an idle wave decodes row trl; its sums are dropped
            store_x_slab(buf(i + L), slab_bytes, x_next, batch, KG, tid, threads);
        };
        int i = 0;
        while (true) {
            step(t0, t2, x0, x1, i);
            if (++i >= steps) break;
            step(t1, t0, x1, x2, i);
            if (++i >= steps) break;
            step(t2, t1, x2, x0, i);
            if (++i >= steps) break;
        }
    } else if constexpr (D == 3) {
        GemmTile<RAW> t0, t1, t2;
        load_tile_i(t0, 0);
        XPieces x0 = x_step(0);
        load_tile_i(t1, 1);
        XPieces x1 = x_step(1);
        XPieces x2;
        if constexpr (!RAW) store_block_lut(lut, lutv, lane);
        store_x_slab(xbuf, slab_bytes, x0, batch, KG, tid, threads);
        lds_barrier();
        auto step = [&](GemmTile<RAW>& cur, GemmTile<RAW>& ahead, const XPieces& x_next, XPieces& x_ahead,
                        int i) {
            x_ahead = x_step(i + 2);
            load_tile_i(ahead, i + 2);
            if (has_tile(i)) use_tile(cur, i);  // an idle wave decodes row trl; its sums are dropped
            store_x_slab(xbuf + ((i + 1) & 1) * KG * slab_bytes, slab_bytes, x_next, batch, KG, tid, threads);
            lds_barrier();
        };
        // the loop leaves after the last step (not after a group of three):
        // past it nothing waits on the loads it issued
        int i = 0;
        while (true) {
            step(t0, t2, x1, x2, i);
            if (++i >= steps) break;
            step(t1, t0, x2, x0, i);
            if (++i >= steps) break;
            step(t2, t1, x0, x1, i);
            if (++i >= steps) break;
        }
    } else {
        GemmTile<RAW> t0;
        XPieces xr = x_step(0);
        if constexpr (!RAW) store_block_lut(lut, lutv, lane);
        store_x_slab(xbuf, slab_bytes, xr, batch, KG, tid, threads);
        lds_barrier();
        for (int i = 0; i < steps; ++i) {
            xr = x_step(i + 1);
            load_tile_i(t0, i);
            if (has_tile(i)) use_tile(t0, i);
            store_x_slab(xbuf + ((i + 1) & 1) * KG * slab_bytes, slab_bytes, xr, batch, KG, tid, threads);
            lds_barrier();
        }
    }
    // the K groups of a tile row: groups 1..KG-1 hand their sums to group 0
    // through LDS (the x slabs are no longer read: every wave passed the
    // last step's barrier), which adds them in ascending group order
    if (KG > 1) {
        // [KG - 1][R][64 lanes][BG][4]: over the x slabs, which every wave
        // has passed the last barrier of, or past the slab ring, whose last
        // slabs other waves may still read
        float* red = reinterpret_cast<float*>(gsm + (M > 0 ? NB * KG * slab_bytes : 0));
        const int rw = w - kg * R;
        if (kg > 0) {
#pragma unroll
            for (int g = 0; g < BG; ++g)
                *reinterpret_cast<floatx4_t*>(red + ((((kg - 1) * R + rw) * 64 + (int)lane) * BG + g) * 4) = acc[g];
        }
        lds_barrier();
        if (kg > 0) return;
        for (int k = 1; k < KG; ++k)
#pragma unroll
            for (int g = 0; g < BG; ++g)
                acc[g] += *reinterpret_cast<const floatx4_t*>(red + ((((k - 1) * R + rw) * 64 + (int)lane) * BG + g) * 4);
    }
    if (!active) return;

    // accumulator layout: lane l holds D[4 * (l / 16) + e][l % 16] of each
    // batch group: tile row 4 * (l / 16) + e, batch row 16 * g + l % 16
    const int64_t n0 = (int64_t)tr * kTileRows + 4 * (int)(lane >> 4);
    if (S == 1) {
#pragma unroll
        for (int g = 0; g < BG; ++g) {
            const int b = 16 * g + (int)(lane & 15u);
            if (b < batch)
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (n0 + e < a.N) a.y[(int64_t)b * a.N + n0 + e] = acc[g][e];
        }
        return;
    }
    // split-K: device-scope partial stores, then the wave's arrival on the
    // tile row's counter; the last of the S waves adds the partials in order
#pragma unroll
    for (int g = 0; g < BG; ++g) {
        const int b = 16 * g + (int)(lane & 15u);
        if (b < batch) {
            const float v[4] = {acc[g][0], acc[g][1], acc[g][2], acc[g][3]};
            store_partial4(&a.partial[((int64_t)s * batch + b) * a.Np + n0], v);
        }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    int old = 0;
    if (lane == 0) old = __hip_atomic_fetch_add(&a.counters[tr], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    old = __builtin_amdgcn_readfirstlane(old);
    if (old != S - 1) return;
#pragma unroll
    for (int g = 0; g < BG; ++g) {
        const int b = 16 * g + (int)(lane & 15u);
        if (b < batch) {
            // every split's loads first (in groups of 8), then the adds in
            // ascending split order
            float sum[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            for (int s0 = 0; s0 < S; s0 += 8) {
                uint64_t lo[8], hi[8];
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    lo[k] = hi[k] = 0;
                    if (s0 + k < S) {
                        const float* pp = &a.partial[((int64_t)(s0 + k) * batch + b) * a.Np + n0];
                        lo[k] = load_partial2(pp);
                        hi[k] = load_partial2(pp + 2);
                    }
                }
#pragma unroll
                for (int k = 0; k < 8; ++k)
                    if (s0 + k < S) {
                        sum[0] += partial_lo(lo[k]);
                        sum[1] += partial_hi(lo[k]);
                        sum[2] += partial_lo(hi[k]);
                        sum[3] += partial_hi(hi[k]);
                    }
            }
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (n0 + e < a.N) a.y[(int64_t)b * a.N + n0 + e] = sum[e];
        }
    }
    if (lane == 0) __hip_atomic_store(&a.counters[tr], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

namespace {

template <int BG, bool RAW>
hipError_t gemm_b(const GemvGroupArgs& a, int batch, const GemvPlan& p, hipStream_t stream) {
    const dim3 grid(group_grid_x(a), a.m[0].S, a.count), block(p.waves * 64);
    if (p.generic)
        hipLaunchKernelGGL((gemm_kernel<BG, RAW, true, 0>), grid, block, p.lds, stream, a, batch);
    else if (p.slab_ring == kGemmSlabRing)
        hipLaunchKernelGGL((gemm_kernel<BG, RAW, false, kGemmSlabRing>), grid, block, p.lds, stream, a, batch);
    else
        hipLaunchKernelGGL((gemm_kernel<BG, RAW, false, 0>), grid, block, p.lds, stream, a, batch);
    return hipGetLastError();
}

}  // namespace

size_t gemm_lds_bytes(int waves, int batch, int slab_ring) {
    const int bg = batch > 16 ? 2 : 1;
    const int rows = gemm_min_waves(batch), kgroups = std::max(1, waves / rows);
    const size_t sums = (size_t)(kgroups - 1) * rows * 64 * bg * 4 * sizeof(float);
    if (slab_ring > 0) return (size_t)2 * slab_ring * kgroups * 16 * bg * kRowBytes + sums;
    const size_t slabs = (size_t)2 * kgroups * 16 * bg * kRowBytes;
    return std::max(slabs, sums);
}

hipError_t launch_gemm(const GemvGroupArgs& a, int batch, const GemvPlan& p, hipStream_t stream) {
    const int rows = gemm_min_waves(batch);
    if (batch < 1 || batch > 32 || p.waves % rows != 0 || a.rows_per_block != rows) return hipErrorInvalidValue;
    if (batch > 16) return p.raw ? gemm_b<2, true>(a, batch, p, stream) : gemm_b<2, false>(a, batch, p, stream);
    return p.raw ? gemm_b<1, true>(a, batch, p, stream) : gemm_b<1, false>(a, batch, p, stream);
}

}  // namespace se12
