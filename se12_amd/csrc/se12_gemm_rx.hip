// Batched fused SE12 decode + matrix product for gfx950 with x resident in
// LDS: Y[b, n] = sum_k W[n, k] X[b, k] for up to 32 BF16 batch rows in one
// pass over the weights. Same semantics as the reference kernel
// lws/adapters/cuda/kernels/gemv_se12.cu:50-142 at batch B (one warp per
// (row, batch) element, W read B times there).
//
// For shapes whose x fits a block's LDS (batch x K x 2 bytes): every block
// first copies all of x into LDS with direct-to-LDS loads (no registers
// held); then its waves run without a barrier. A block of W waves holds
// W / KG row slots times KG K groups: slot j of the launch (j = slot * P +
// block, P blocks) takes tile rows j, j + P W / KG, ... (the rows in flight
// at a time are adjacent, so the chip reads a moving window of the
// tile-major streams, and where rows are fewer than slots they spread over
// all blocks), and K group g of the slot takes the K tiles g, g + KG, ... of
// each row, in ascending order. A wave keeps its next kRxDepth tiles
// in flight in a ring of registers, across row boundaries. With one K group
// a wave stores each row as soon as its last K tile is done; with KG > 1
// (the host picks it where rows are few, and then no slot holds more than
// one row) the groups' sums meet once at the end, through LDS, and are added
// in ascending group order. The launch shape (W, P) fixes KG and so every
// sum; the raw-BF16 twin (same kernel, RAW) is bit-identical to the fused
// kernel under one shape.
//
// Per tile: each 1 KB of sm (512 B of ec) holding 4 tile rows is read whole
// by one load instruction (full cache lines in order; a layout with one row
// per lane measured 2 us slower at 14336 x 3584), then two DPP exchanges
// between the 4 parts and lane bits 3 and 2 bring the tile into the block
// layout: lane l holds, in part p, the 16 columns 16 (4 (l / 16) + p) .. +
// 15 of row l % 16. It is rebuilt through the pair table with listed
// escapes and raw tiles, and each part's first and second 8 columns are the
// A operands of two v_mfma_f32_16x16x32_bf16 (MFMA row = tile row l % 16).
// Their K positions differ between lane groups, and the B operands (lane l:
// batch row 16 g + l % 16) read the same 8 x columns from the resident x.
// x rows are stored as 16-byte pieces, piece q of row b at piece index b *
// (K / 8) + (q ^ (b & 7)): the 16 rows an MFMA reads at one column land in 8
// distinct 4-bank groups per 8 lanes (no bank conflicts; rows would
// otherwise be a multiple of 512 bytes apart, all in one bank).
// Batch rows past the batch in a 16-row group read row 0: MFMA output
// column n depends on B column n only, and those columns are not stored.
//
// Where only 16 rows of x fit (17..32 rows at K = 3584..4608), LDS holds
// rows 0..15 and each ring slot also loads batch group 1's B operands from
// global memory (x stays in L2): 8 more 16-byte loads per lane per tile, 32
// more VGPRs per slot, so at most 2 waves per SIMD (XG).
//
// Where x fits neither way, the launch splits K (grid y = S splits): split s
// takes K tiles [s TC / S, (s + 1) TC / S) of every row and its blocks hold
// only those columns of x. A row's sum over a split goes to the partial sums
// [S][batch][Np] with device-scope stores as the row ends; at its end the
// wave waits for those stores and arrives on each of its rows' counters (one
// lane per row); the last of a row's S arrivals adds the partial sums in
// ascending split order, stores the row and resets the counter.
//
// FAST only: K % 256 == 0, 16-byte aligned x rows, and for the raw twin
// N % 16 == 0 and an aligned W (the other cases run se12_gemm.hip).
#include "se12_device.hpp"
#include "se12_internal.hpp"

namespace se12 {

typedef __bf16 rx_bf16x8_t __attribute__((ext_vector_type(8)));
typedef float rx_floatx4_t __attribute__((ext_vector_type(4)));

namespace {

// One tile's loads: sm / ec in the block layout once transposed (below), or
// raw BF16 column blocks for the twin; the side record of the tile.
template <bool RAW, bool XG>
struct RxTile {
    TileSide side;
    TileLoads t;
    uint4 r[RAW ? 4 : 1][2];
    uint4 xg[XG ? 8 : 1];  // batch group 1's B operands (x from global memory)
};

}  // namespace

// byte offset in the resident x of piece q (8 columns) of batch row b
__device__ __forceinline__ int rx_piece(int b, int q, int pieces_per_row) {
    return (b * pieces_per_row + (q ^ (b & 7))) * 16;
}

template <int BG, bool RAW, bool XG>
__global__ __launch_bounds__(XG ? kRxMaxThreadsXG : kRxMaxThreads)
__attribute__((amdgpu_waves_per_eu(XG ? 2 : 3))) void gemm_rx_kernel(GemvGroupArgs ga, int batch) {
    static_assert(!XG || BG == 2, "x from global memory serves batch group 1");
    SE12_DECLARE_LUT(lut);
    extern __shared__ __attribute__((aligned(16))) char xs[];
    const GemvArgs a = ga.m[blockIdx.z];
    const int threads = blockDim.x;
    asm volatile("" ::"s"(a.sm), "s"(a.ec), "s"(a.lut), "s"(a.side), "s"(a.wraw), "s"(a.x), "s"(a.y), "s"(a.K),
                 "s"(a.N), "s"(a.TR), "s"(a.TC), "s"(a.S), "s"(threads), "s"(batch));
    const int W = threads >> 6;
    const uint32_t lane = threadIdx.x & 63u;
    const int w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int TC = a.TC;
    // K groups: the host sets KG (in S) so that it divides W, every wave has
    // K tiles, and with KG > 1 every row slot holds at most one row
    const int KG = a.S;
    // K splits (grid y): split s takes K tiles [kb0, ke0) of every row and
    // holds only their columns of x
    const int S = (int)gridDim.y, s = (int)blockIdx.y;
    const int kb0 = (int)((int64_t)s * TC / S), ke0 = (int)((int64_t)(s + 1) * TC / S);
    const int RW = W / KG;                                     // row slots per block
    const int kg = w / RW, rw = w - kg * RW;
    const int nw = (int)gridDim.x * RW;                        // row slots of this matrix
    const int j0 = rw * (int)gridDim.x + (int)blockIdx.x;      // this slot's first row
    const int rows = a.TR > j0 ? (a.TR - 1 - j0) / nw + 1 : 0; // rows j0, j0 + nw, ...
    const int ppr = (ke0 - kb0) * (kTileCols / 8);             // 16-byte pieces per x row in LDS
    // this group's K tiles: kb, kb + ks, ... below ke
    const int kb = kb0 + kg, ks = KG, ke = ke0;

    // The wave's tiles in order: its slot's r-th row (j0 + r nw), its K
    // tiles in ascending order. A cursor (r, kt) walks them; the load cursor
    // stops at the wave's last tile (a one-tile wave's second ring slot
    // re-loads that tile).
    const int per_row = (ke - kb + ks - 1) / ks;               // K tiles per row of this group
    const int n_tiles = rows * per_row;
    struct Cursor {
        int r, kt;
    };
    auto advance = [&](Cursor& c) {
        c.kt += ks;
        if (c.kt >= ke) {
            c.kt = kb;
            ++c.r;
        }
    };
    auto advance_clamped = [&](Cursor& c) {
        Cursor n = c;
        advance(n);
        if (n.r < rows) c = n;
    };
    auto row_of = [&](const Cursor& c) { return j0 + c.r * nw; };
    // batch group 1's x row of this lane when x comes from global memory
    // (rows past the batch read the last row; their outputs are not stored)
    const int xg_row = min(16 + (int)(lane & 15u), batch - 1);
    auto load = [&](RxTile<RAW, XG>& t, const Cursor& c) {
        const int tr = row_of(c), kt = c.kt;
        if constexpr (RAW) {
            load_raw_blocks(t.r, a.wraw, a.K, tr, kt, lane);
        } else {
            load_tile_block_order(t.t, t.side, a.sm, a.ec, a.side, (int64_t)tr * TC + kt, lane);
        }
        if constexpr (XG) {
            // pieces 2 p + h (8 columns each) of this lane's 32-column slice
            const uint4* xr = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(a.x) + (int64_t)xg_row * a.K) +
                              32 * kt + 8 * (int)(lane >> 4);
#pragma unroll
            for (int i = 0; i < 8; ++i) t.xg[i] = xr[i];
        }
    };

    // The first kRxDepth tiles, then all of x and the pair table straight to
    // LDS (direct-to-LDS loads: no registers held); the block meets once
    // everything has landed. (x first, with the barrier waiting for x only,
    // measured no faster: the tiles' loads then start later.) The LDS loads
    // are inline asm, which the compiler's wait counting does not see: with
    // its own direct-to-LDS loads it waits for every load in flight (vmcnt(0))
    // at each step of the ring below, the other slot's included.
    RxTile<RAW, XG> ring[kRxDepth];
    Cursor ld{0, kb};
    constexpr int kLoadsPerTile = (RAW ? 8 : 9) + (XG ? 8 : 0);
    if (n_tiles > 0) {
#pragma unroll
        for (int d = 0; d < kRxDepth; ++d) {
            load(ring[d], ld);
            advance_clamped(ld);
        }
    }
    {
        const int total = (XG ? 16 : batch) * ppr;             // pieces of x in LDS
        const int rounds = (total + threads - 1) / threads;
        const uint16_t* x = static_cast<const uint16_t*>(a.x);
        // block b starts at round b mod rounds, so that the blocks, which all
        // read the same x from L2 at the same time, spread over its channels
        int r = (int)(blockIdx.x % (unsigned)rounds);
        for (int i = 0; i < rounds; ++i) {
            const int base = r * threads + w * 64;
            if (base < total) {
                const int p = min(base + (int)lane, total - 1);  // a lane past the end re-loads the last piece
                const int b = p / ppr, e = p - b * ppr;
                const int q = e ^ (b & 7);                       // LDS piece p holds x piece q of row b
                lds_load16(x + (int64_t)b * a.K + 8 * (q + 32 * kb0), lds_address(xs + 16 * base));
            }
            r = r + 1 == rounds ? 0 : r + 1;
        }
    }
    // the 1 KB pair table: lane l's 16 bytes to LDS bytes 16 l .. + 15
    if (!RAW && w == 0) lds_load16(reinterpret_cast<const uint4*>(a.lut) + lane, lds_address(lut));
    wait_vector_loads();
    lds_barrier();

    rx_floatx4_t acc[BG];
#pragma unroll
    for (int g = 0; g < BG; ++g) acc[g] = rx_floatx4_t{0.0f, 0.0f, 0.0f, 0.0f};
    // B-operand row of this lane in each batch group (rows past the batch
    // read row 0; their outputs are never stored)
    int xrow[BG];
#pragma unroll
    for (int g = 0; g < BG; ++g) {
        const int b = 16 * g + (int)(lane & 15u);
        xrow[g] = b < batch ? b : 0;
    }
    // y as 16-byte pieces: N % 16 == 0 on this path, so a 16-byte aligned y
    // keeps every batch row aligned
    const bool y_vec = (reinterpret_cast<uintptr_t>(a.y) & 15u) == 0u;

    // The row's outputs: lane l holds D[4 (l / 16) + e][l % 16] of each batch
    // group (tile row 4 (l / 16) + e, batch row 16 g + l % 16). Lane l takes
    // those of lane 16 (l % 4) + l / 4, i.e. batch row 16 g + l / 4, tile
    // rows 4 (l % 4) .. + 3, and stores them as one 16-byte piece: each
    // batch row's 16 outputs are 64 contiguous bytes from 4 lanes.
    auto store_row = [&](int tr) {
        const int src = (int)((((lane & 3u) << 4) | (lane >> 2)) << 2);
#pragma unroll
        for (int g = 0; g < BG; ++g) {
            float v[4];
#pragma unroll
            for (int e = 0; e < 4; ++e)
                v[e] = __int_as_float(__builtin_amdgcn_ds_bpermute(src, __float_as_int(acc[g][e])));
            const int b = 16 * g + (int)(lane >> 2);
            if (b < batch) {
                float* yp = a.y + (int64_t)b * a.N + (int64_t)tr * kTileRows + 4 * (int)(lane & 3u);
                if (y_vec) {
                    *reinterpret_cast<float4*>(yp) = make_float4(v[0], v[1], v[2], v[3]);
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e) yp[e] = v[e];
                }
            }
        }
    };

    // With K splits, a row's sum over this split's K tiles goes to the
    // partial sums [S][batch][Np] (device-scope stores, no wait), in
    // store_row's lane layout; the wave arrives on its rows' counters at its
    // end (finish_splits).
    auto store_partial = [&](int tr) {
        const int src = (int)((((lane & 3u) << 4) | (lane >> 2)) << 2);
#pragma unroll
        for (int g = 0; g < BG; ++g) {
            float v[4];
#pragma unroll
            for (int e = 0; e < 4; ++e)
                v[e] = __int_as_float(__builtin_amdgcn_ds_bpermute(src, __float_as_int(acc[g][e])));
            const int b = 16 * g + (int)(lane >> 2);
            if (b < batch)
                store_partial4(a.partial + ((int64_t)s * batch + b) * a.Np + (int64_t)tr * kTileRows + 4 * (int)(lane & 3u), v);
        }
    };
    // Once the wave's partial stores have completed, one lane per row arrives
    // on the row's counter (device scope); the last of the S arrivals adds
    // the S partial sums in ascending split order, stores the row and resets
    // the counter for the next launch.
    auto finish_splits = [&](int n_rows) {
        // the wait for this wave's partial stores is also a compiler barrier
        // (memory clobber): no store sinks below it and no counter update
        // rises above it (the builtin wait is not modelled as touching
        // memory, so it would order nothing)
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        for (int r0 = 0; r0 < n_rows; r0 += 64) {
            const int r = r0 + (int)lane;
            int old = -1;
            if (r < n_rows) old = __hip_atomic_fetch_add(&a.counters[j0 + r * nw], 1, __ATOMIC_RELAXED,
                                                         __HIP_MEMORY_SCOPE_AGENT);
            uint64_t last = __ballot(old == S - 1);
            // the other splits' partial sums are read only after the arrival
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
            while (last) {
                const int tr = j0 + (r0 + __builtin_ctzll(last)) * nw;
                last &= last - 1;
#pragma unroll
                for (int g = 0; g < BG; ++g) {
                    const int b = 16 * g + (int)(lane >> 2);
                    if (b < batch) {
                        const int64_t n = (int64_t)tr * kTileRows + 4 * (int)(lane & 3u);
                        float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
                        uint64_t lo[kRxMaxSplits], hi[kRxMaxSplits];
#pragma unroll
                        for (int ss = 0; ss < kRxMaxSplits; ++ss) {
                            lo[ss] = hi[ss] = 0;
                            if (ss < S) {
                                const float* pp = a.partial + ((int64_t)ss * batch + b) * a.Np + n;
                                lo[ss] = load_partial2(pp);
                                hi[ss] = load_partial2(pp + 2);
                            }
                        }
#pragma unroll
                        for (int ss = 0; ss < kRxMaxSplits; ++ss)
                            if (ss < S) {
                                v[0] += partial_lo(lo[ss]);
                                v[1] += partial_hi(lo[ss]);
                                v[2] += partial_lo(hi[ss]);
                                v[3] += partial_hi(hi[ss]);
                            }
                        float* yp = a.y + (int64_t)b * a.N + n;
                        if (y_vec) {
                            *reinterpret_cast<float4*>(yp) = make_float4(v[0], v[1], v[2], v[3]);
                        } else {
#pragma unroll
                            for (int e = 0; e < 4; ++e) yp[e] = v[e];
                        }
                    }
                }
                if (lane == 0) __hip_atomic_store(&a.counters[tr], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
    };

    // part p of a tile in the block layout: lane l holds columns 16 (4 (l /
    // 16) + p) .. + 15 of row l % 16, as 8 BF16 pairs; its first and second
    // 8 columns are the A operands of two MFMAs, whose B operands are the x
    // pieces (8 columns) 2 (4 (l / 16) + p) and the next
    auto mfma_part = [&](const uint32_t wv[8], int kt, int p, const uint4* xg) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const rx_bf16x8_t av =
                __builtin_bit_cast(rx_bf16x8_t, make_uint4(wv[4 * h], wv[4 * h + 1], wv[4 * h + 2], wv[4 * h + 3]));
            const int q = 32 * (kt - kb0) + 8 * (int)(lane >> 4) + 2 * p + h;
#pragma unroll
            for (int g = 0; g < BG; ++g) {
                const uint4 bv =
                    (XG && g == 1) ? xg[2 * p + h] : *reinterpret_cast<const uint4*>(xs + rx_piece(xrow[g], q, ppr));
                acc[g] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, __builtin_bit_cast(rx_bf16x8_t, bv), acc[g], 0, 0, 0);
            }
        }
    };
    auto use = [&](RxTile<RAW, XG>& t, const Cursor& c) {
        const int kt = c.kt;
        if constexpr (RAW) {
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                const uint32_t wv[8] = {t.r[p][0].x, t.r[p][0].y, t.r[p][0].z, t.r[p][0].w,
                                        t.r[p][1].x, t.r[p][1].y, t.r[p][1].z, t.r[p][1].w};
                mfma_part(wv, kt, p, t.xg);
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
                for (int p = 0; p < 4; ++p) mfma_part(wv[p], kt, p, t.xg);
            } else {
                chunks_to_blocks(t.t);  // in place: the slot is reloaded next
                // each part's patterns merged with its sm bytes as soon as
                // looked up; escapes only set exponent bits, which the merge
                // takes from the patterns, so they patch the merged words
                uint32_t wv[4][8];
#pragma unroll
                for (int p = 0; p < 4; ++p) {
                    uint32_t pat[8];
                    lookup_chunk(lut, t.t.ec[p], pat);
                    merge_chunk(pat, t.t.sm[p], wv[p]);
                }
                patch_tile_escapes<kBlockLayout>(wv, info, t.side, 0, lane);
#pragma unroll
                for (int p = 0; p < 4; ++p) mfma_part(wv[p], kt, p, t.xg);
            }
        }
        // the row's last K tile of this wave: with one K group the row is
        // done; with more, its single row waits for the combine below
        if (KG == 1 && kt + ks >= ke) {
            if (S == 1)
                store_row(row_of(c));
            else
                store_partial(row_of(c));
#pragma unroll
            for (int g = 0; g < BG; ++g) acc[g] = rx_floatx4_t{0.0f, 0.0f, 0.0f, 0.0f};
        }
    };
    // The ring (two slots): while tiles remain to load, a step uses one slot
    // and reloads it with the tile two ahead; the last two tiles are used
    // without reloads (a load past the wave's last tile would hold the wave,
    // and the end of the kernel, for one more memory latency). Inside the
    // loop every load is issued on every path, so the compiler's wait counts
    // stay exact (a load skipped on one path would merge into a wait for all
    // loads in flight, the other slot's included).
    static_assert(kRxDepth == 2, "the ring below has two slots");
    Cursor cu{0, kb};
    auto step = [&](RxTile<RAW, XG>& t) {
        use(t, cu);
        advance(cu);
        __builtin_amdgcn_sched_barrier(0);  // no work of the next step above this one's
    };
    auto step_reload = [&](RxTile<RAW, XG>& t) {
        step(t);
        // the slot's next loads after its use: hoisted above it, they would
        // hold a third tile's registers
        __builtin_amdgcn_sched_barrier(0);
        load(t, ld);
        advance_clamped(ld);
    };
    if (n_tiles > 0) {
        // pair j uses tiles 2j, 2j + 1 and loads 2j + 2, 2j + 3
        int j = 0;
        for (; 2 * j + 3 < n_tiles; ++j) {
            step_reload(ring[0]);
            step_reload(ring[1]);
        }
        // the last two or three tiles: a third is loaded into the first
        // slot once it is used; the waits are explicit so that the second
        // slot's use does not also wait for that load
        const int left = n_tiles - 2 * j;  // 1 (a one-tile wave), 2 or 3
        step(ring[0]);
        if (left == 3) {
            load(ring[0], ld);
            wait_vector_loads_to<kLoadsPerTile>();
        } else {
            wait_vector_loads();
        }
        if (left >= 2) step(ring[1]);
        if (left == 3) step(ring[0]);
    }
    if (KG == 1) {
        if (S > 1 && rows > 0) finish_splits(rows);
        return;
    }
    // K groups: every wave is past its last MFMA (x is no longer read), the
    // groups 1.. of each slot leave their sums in LDS over x, and group 0
    // adds them in ascending group order and stores the row
    __syncthreads();
    const bool has_row = n_tiles > 0;
    rx_floatx4_t* part = reinterpret_cast<rx_floatx4_t*>(xs);  // [KG - 1][RW][64 lanes][BG]
    if (kg > 0) {
#pragma unroll
        for (int g = 0; g < BG; ++g)
            part[(((kg - 1) * RW + rw) * 64 + (int)lane) * BG + g] =
                has_row ? acc[g] : rx_floatx4_t{0.0f, 0.0f, 0.0f, 0.0f};
    }
    __syncthreads();
    if (kg > 0 || rows == 0) return;
    for (int k = 1; k < KG; ++k)
#pragma unroll
        for (int g = 0; g < BG; ++g) acc[g] += part[(((k - 1) * RW + rw) * 64 + (int)lane) * BG + g];
    if (S == 1) {
        store_row(j0);
        return;
    }
    store_partial(j0);
    finish_splits(1);
}

namespace {

template <int BG, bool RAW, bool XG = false>
hipError_t rx_go(const GemvGroupArgs& a, int batch, const GemvPlan& p, hipStream_t stream) {
    const dim3 grid(p.blocks / (a.count * p.ksplits), p.ksplits, a.count), block(p.waves * 64);
    hipLaunchKernelGGL((gemm_rx_kernel<BG, RAW, XG>), grid, block, p.lds, stream, a, batch);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_gemm_rx(const GemvGroupArgs& a, int batch, const GemvPlan& p, hipStream_t stream) {
    if (batch < 1 || batch > 32 || p.waves < 1 || p.waves * 64 > kRxMaxThreads || p.ksplits < 1 ||
        p.blocks % (a.count * p.ksplits) != 0 || (p.xg && p.ksplits != 1))
        return hipErrorInvalidValue;
    for (int i = 0; i < a.count; ++i)
        if (a.m[i].S < 1 || p.waves % a.m[i].S != 0) return hipErrorInvalidValue;
    if (p.xg) {
        if (batch <= 16 || p.waves * 64 > kRxMaxThreadsXG) return hipErrorInvalidValue;
        return p.raw ? rx_go<2, true, true>(a, batch, p, stream) : rx_go<2, false, true>(a, batch, p, stream);
    }
    if (batch > 16) return p.raw ? rx_go<2, true>(a, batch, p, stream) : rx_go<2, false>(a, batch, p, stream);
    return p.raw ? rx_go<1, true>(a, batch, p, stream) : rx_go<1, false>(a, batch, p, stream);
}

}  // namespace se12
