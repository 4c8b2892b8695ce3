// Fused SE12 decode + GEMV for gfx950, batch 1..4 per launch, and its raw-BF16
// twin (same grid, same per-lane order, same reductions: the two give
// bit-identical FP32 outputs for one launch shape, since decode is lossless).
//
// What it computes: y[b, n] = sum_k W[n, k] * x[b, k] in FP32, W rebuilt from
// the SE12 streams in registers (never written to memory) - the semantics of
// the reference kernel lws/adapters/cuda/kernels/gemv_se12.cu:50-142 and its
// raw twin gemv_raw_bf16.cu:18-56, laid out for wave64 instead of one warp per
// (row, batch) element.
//
// Grid: block = `waves` x 64 threads, one (tile row, K split) per block:
// blockIdx = tile_row * S + split, split s covering K tiles
// [s*TC/S, (s+1)*TC/S). The block's waves take that range round-robin, one
// 16x256 tile at a time, with the next tile's loads in flight while the
// current one is decoded. x for the block's K range is staged once in LDS
// (zero past K) and W is read once for all batch rows of the launch.
// Reductions, all in a fixed order: DPP over the 16 lanes of a tile row,
// LDS over the block's waves (ascending), and for S > 1 the last block of a
// tile row to finish (device-scope arrival counter) sums the S partials in
// ascending split order. The counter is reset by that block, so no memset is
// needed between launches (graph-capture friendly).
#include "se12_device.hpp"
#include "se12_internal.hpp"

namespace se12 {

struct RawLoads {
    uint4 v[4][2];
};

__device__ __forceinline__ void load_raw_tile(RawLoads& t, const uint16_t* w, int64_t N, int64_t K, int tr, int kt,
                                              uint32_t lane, bool vec_ok) {
    const int64_t col = (int64_t)kt * kTileCols + 16 * (lane & 15u);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int64_t row = (int64_t)tr * kTileRows + 4 * j + (lane >> 4);
        const uint16_t* p = w + row * K + col;
        if (vec_ok && row < N && col + 16 <= K) {
            t.v[j][0] = reinterpret_cast<const uint4*>(p)[0];
            t.v[j][1] = reinterpret_cast<const uint4*>(p)[1];
        } else {
            uint32_t h[8];
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                uint32_t lo = (row < N && col + 2 * q < K) ? (uint32_t)p[2 * q] : 0u;
                uint32_t hi = (row < N && col + 2 * q + 1 < K) ? (uint32_t)p[2 * q + 1] : 0u;
                h[q] = lo | (hi << 16);
            }
            t.v[j][0] = make_uint4(h[0], h[1], h[2], h[3]);
            t.v[j][1] = make_uint4(h[4], h[5], h[6], h[7]);
        }
    }
}

// Stages x[b, kb*256 .. ke*256) (zero past K) into LDS. Each thread issues up
// to kStageUnroll 16-byte loads before its first LDS store, so a block pays
// one memory round trip per kStageUnroll * threads items, not one per item.
constexpr int kStageUnroll = 8;

template <int B, bool XF32>
__device__ __forceinline__ void stage_x(void* xs_raw, const GemvArgs& a, int kb, int ke, int tid, int nthreads) {
    constexpr int EPI = XF32 ? 4 : 8;  // elements per 16-byte item
    const int ncols = (ke - kb) * kTileCols;
    const int per_row = ncols / EPI;
    const int total = B * per_row;
    const int64_t c0 = (int64_t)kb * kTileCols;
    for (int base = 0; base < total; base += nthreads * kStageUnroll) {
        uint4 v[kStageUnroll];
#pragma unroll
        for (int u = 0; u < kStageUnroll; ++u) {
            const int i = base + u * nthreads + tid;
            if (i < total) {
                const int b = i / per_row;
                const int c = (i - b * per_row) * EPI;
                const int64_t g = c0 + c;
                if constexpr (XF32) {
                    const float* x = static_cast<const float*>(a.x) + (int64_t)b * a.K;
                    if (a.x_vec_ok && g + EPI <= a.K) {
                        v[u] = *reinterpret_cast<const uint4*>(x + g);
                    } else {
                        uint32_t e[4];
#pragma unroll
                        for (int q = 0; q < 4; ++q) e[q] = (g + q < a.K) ? __float_as_uint(x[g + q]) : 0u;
                        v[u] = make_uint4(e[0], e[1], e[2], e[3]);
                    }
                } else {
                    const uint16_t* x = static_cast<const uint16_t*>(a.x) + (int64_t)b * a.K;
                    if (a.x_vec_ok && g + EPI <= a.K) {
                        v[u] = *reinterpret_cast<const uint4*>(x + g);
                    } else {
                        uint32_t e[4];
#pragma unroll
                        for (int q = 0; q < 4; ++q) {
                            const uint32_t lo = (g + 2 * q < a.K) ? (uint32_t)x[g + 2 * q] : 0u;
                            const uint32_t hi = (g + 2 * q + 1 < a.K) ? (uint32_t)x[g + 2 * q + 1] : 0u;
                            e[q] = lo | (hi << 16);
                        }
                        v[u] = make_uint4(e[0], e[1], e[2], e[3]);
                    }
                }
            }
        }
#pragma unroll
        for (int u = 0; u < kStageUnroll; ++u) {
            const int i = base + u * nthreads + tid;
            if (i < total) {
                const int b = i / per_row;
                const int c = (i - b * per_row) * EPI;
                char* dst = static_cast<char*>(xs_raw) + ((int64_t)b * a.xstride + c) * (XF32 ? 4 : 2);
                *reinterpret_cast<uint4*>(dst) = v[u];
            }
        }
    }
}

// multiply-accumulate 8 BF16 weight pairs with the lane's x pairs of batch b
template <bool XF32>
__device__ __forceinline__ float mac8(const uint32_t w[8], const uint32_t* xp, float acc) {
    if constexpr (XF32) {
        const float* xf = reinterpret_cast<const float*>(xp);
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            acc = fmaf(__uint_as_float(w[q] << 16), xf[2 * q], acc);
            acc = fmaf(__uint_as_float(w[q] & 0xFFFF0000u), xf[2 * q + 1], acc);
        }
    } else {
#pragma unroll
        for (int q = 0; q < 8; ++q) acc = dot2_bf16(w[q], xp[q], acc);
    }
    return acc;
}

// zero the weights of tile columns >= lim (the valid columns of the last K tile)
__device__ __forceinline__ void mask_tail(uint32_t w[8], int c0, int lim) {
#pragma unroll
    for (int q = 0; q < 8; ++q) {
        const int c = c0 + 2 * q;
        w[q] = (c >= lim) ? 0u : ((c + 1 >= lim) ? (w[q] & 0xFFFFu) : w[q]);
    }
}

template <int B, bool XF32>
__device__ __forceinline__ void load_x_pairs(uint32_t xp[B][XF32 ? 16 : 8], const void* xs_raw, int xstride,
                                             int kk, uint32_t lane) {
    constexpr int NX = XF32 ? 16 : 8;
#pragma unroll
    for (int b = 0; b < B; ++b) {
        const uint4* p;
        if constexpr (XF32)
            p = reinterpret_cast<const uint4*>(static_cast<const float*>(xs_raw) + (int64_t)b * xstride + kk +
                                               16 * (lane & 15u));
        else
            p = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(xs_raw) + (int64_t)b * xstride + kk +
                                               16 * (lane & 15u));
#pragma unroll
        for (int v = 0; v < NX / 4; ++v) {
            uint4 u = p[v];
            xp[b][4 * v + 0] = u.x;
            xp[b][4 * v + 1] = u.y;
            xp[b][4 * v + 2] = u.z;
            xp[b][4 * v + 3] = u.w;
        }
    }
}

// TAIL: the last K tile of a matrix whose K is not a multiple of 256 and
// whose codebook[0] is 255: there the padding decodes to +inf, which the zero
// x padding would turn into NaN, so those weights are zeroed. Any other
// padding weight is finite and meets x = 0, adding nothing.
template <int B, bool XF32, bool TAIL>
__device__ __forceinline__ void se12_tile(const GemvArgs& a, const TileLoads& t, const uint32_t* lut,
                                          const void* xs_raw, int kb, int kt, uint32_t lane, float acc[4][B]) {
    constexpr int NX = XF32 ? 16 : 8;
    uint32_t xp[B][NX];
    load_x_pairs<B, XF32>(xp, xs_raw, a.xstride, (kt - kb) * kTileCols, lane);
    constexpr bool tail = TAIL;
    const int lim = (int)(a.K - (int64_t)kt * kTileCols);
    const int c0 = 16 * (int)(lane & 15u);
    const int32_t frank = uniform_rank(t);
    if (frank >= 0) {
        const int16_t* raw = a.fb_raw + (int64_t)frank * kTile;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            uint32_t w[8];
            load_raw_chunk(raw, j, lane, w);
            if (tail) mask_tail(w, c0, lim);
#pragma unroll
            for (int b = 0; b < B; ++b) acc[j][b] = mac8<XF32>(w, xp[b], acc[j][b]);
        }
    } else {
        uint32_t run = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            uint32_t w[8];
            decode_chunk(lut, t.sm[j], t.ec[j], t.esc, run, lane, w);
            if (tail) mask_tail(w, c0, lim);
#pragma unroll
            for (int b = 0; b < B; ++b) acc[j][b] = mac8<XF32>(w, xp[b], acc[j][b]);
        }
    }
}

template <int B, bool XF32>
__device__ __forceinline__ void raw_tile(const GemvArgs& a, const RawLoads& t, const void* xs_raw, int kb, int kt,
                                         uint32_t lane, float acc[4][B]) {
    constexpr int NX = XF32 ? 16 : 8;
    uint32_t xp[B][NX];
    load_x_pairs<B, XF32>(xp, xs_raw, a.xstride, (kt - kb) * kTileCols, lane);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        uint32_t w[8] = {t.v[j][0].x, t.v[j][0].y, t.v[j][0].z, t.v[j][0].w,
                         t.v[j][1].x, t.v[j][1].y, t.v[j][1].z, t.v[j][1].w};
#pragma unroll
        for (int b = 0; b < B; ++b) acc[j][b] = mac8<XF32>(w, xp[b], acc[j][b]);
    }
}

// PF: keep the next tile's loads in flight while the current one is used
// (two load buffers); launches with one tile per wave use PF = false.
template <int B, bool XF32, bool RAW, bool PF>
__global__ __launch_bounds__(64 * gemv_max_waves(B, XF32)) void gemv_kernel(GemvArgs a) {
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    const int nthreads = blockDim.x;
    const int W = nthreads >> 6;
    const int tid = threadIdx.x;
    const uint32_t lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int S = a.S;
    const int tr = blockIdx.x / S;
    const int s = blockIdx.x - tr * S;
    const int kb = (int)(((int64_t)s * a.TC) / S);
    const int ke = (int)(((int64_t)(s + 1) * a.TC) / S);

    uint32_t* lut = reinterpret_cast<uint32_t*>(smem);
    float* red = reinterpret_cast<float*>(smem + kLutBytes);
    void* xs = smem + kLutBytes + W * B * 16 * sizeof(float);

    float acc[4][B];
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int b = 0; b < B; ++b) acc[j][b] = 0.0f;

    // The prefetch is issued unconditionally (the last iteration re-reads the
    // current tile) so the compiler's wait counts stay exact: a conditional
    // prefetch makes it wait for every outstanding load at the merge point.
    int kt = kb + w;
    if constexpr (RAW) {
        RawLoads t0, t1;
        const bool has = kt < ke;
        if (has) load_raw_tile(t0, a.wraw, a.N, a.K, tr, kt, lane, a.w_vec_ok);
        stage_x<B, XF32>(xs, a, kb, ke, tid, nthreads);
        lds_barrier();
        if (has) {
            if constexpr (PF) {
                while (true) {
                    int kn = kt + W;
                    bool more = kn < ke;
                    load_raw_tile(t1, a.wraw, a.N, a.K, tr, more ? kn : kt, lane, a.w_vec_ok);
                    raw_tile<B, XF32>(a, t0, xs, kb, kt, lane, acc);
                    if (!more) break;
                    kt = kn;
                    kn = kt + W;
                    more = kn < ke;
                    load_raw_tile(t0, a.wraw, a.N, a.K, tr, more ? kn : kt, lane, a.w_vec_ok);
                    raw_tile<B, XF32>(a, t1, xs, kb, kt, lane, acc);
                    if (!more) break;
                    kt = kn;
                }
            } else {
                while (true) {
                    raw_tile<B, XF32>(a, t0, xs, kb, kt, lane, acc);
                    kt += W;
                    if (kt >= ke) break;
                    load_raw_tile(t0, a.wraw, a.N, a.K, tr, kt, lane, a.w_vec_ok);
                }
            }
        }
    } else {
        // the masked tail tile, if any, is peeled off the main loop
        const bool peel = a.mask_tail && ke == a.TC;
        const int kem = peel ? ke - 1 : ke;
        TileLoads t0, t1;
        const int64_t row_tiles = (int64_t)tr * a.TC;
        const bool has = kt < kem;
        if (has) load_tile(t0, a.sm, a.ec, a.esc, a.fb_rank, row_tiles + kt, lane);
        build_pair_lut(lut, a.codebook, tid, nthreads);
        stage_x<B, XF32>(xs, a, kb, ke, tid, nthreads);
        lds_barrier();
        if (has) {
            if constexpr (PF) {
                while (true) {
                    int kn = kt + W;
                    bool more = kn < kem;
                    load_tile(t1, a.sm, a.ec, a.esc, a.fb_rank, row_tiles + (more ? kn : kt), lane);
                    se12_tile<B, XF32, false>(a, t0, lut, xs, kb, kt, lane, acc);
                    if (!more) break;
                    kt = kn;
                    kn = kt + W;
                    more = kn < kem;
                    load_tile(t0, a.sm, a.ec, a.esc, a.fb_rank, row_tiles + (more ? kn : kt), lane);
                    se12_tile<B, XF32, false>(a, t1, lut, xs, kb, kt, lane, acc);
                    if (!more) break;
                    kt = kn;
                }
            } else {
                while (true) {
                    se12_tile<B, XF32, false>(a, t0, lut, xs, kb, kt, lane, acc);
                    kt += W;
                    if (kt >= kem) break;
                    load_tile(t0, a.sm, a.ec, a.esc, a.fb_rank, row_tiles + kt, lane);
                }
            }
        }
        if (peel && (a.TC - 1 - kb) % W == w) {
            load_tile(t0, a.sm, a.ec, a.esc, a.fb_rank, row_tiles + a.TC - 1, lane);
            se12_tile<B, XF32, true>(a, t0, lut, xs, kb, a.TC - 1, lane, acc);
        }
    }

    // 16-lane row sums; lane 16*g of each row group holds tile rows 4*j + g
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int b = 0; b < B; ++b) {
            const float v = row16_sum(acc[j][b]);
            if ((lane & 15u) == 0u) red[(w * B + b) * 16 + 4 * j + (lane >> 4)] = v;
        }
    lds_barrier();

    const int b = tid >> 4;
    const int r = tid & 15;
    const int64_t n = (int64_t)tr * kTileRows + r;
    float v = 0.0f;
    if (tid < 16 * B) {
        for (int ww = 0; ww < W; ++ww) v += red[(ww * B + b) * 16 + r];
    }
    if (S == 1) {
        if (tid < 16 * B && n < a.N) a.y[(int64_t)b * a.N + n] = v;
        return;
    }
    // Cross-block reduction without cache-wide maintenance: the partials are
    // written with device-scope (sc1) stores, each thread waits for its stores
    // to complete before the block's arrival is counted, and the last block
    // reads them back with device-scope loads. (A __threadfence() here would
    // write back and invalidate the whole L2 of the XCD for every block.)
    if (tid < 16 * B)
        __hip_atomic_store(&a.partial[((int64_t)s * B + b) * a.Np + n], v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    int* last = reinterpret_cast<int*>(red);
    if (tid == 0) {
        const int old = __hip_atomic_fetch_add(&a.counters[tr], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *last = (old == S - 1) ? 1 : 0;
    }
    __syncthreads();
    if (*last) {
        if (tid < 16 * B) {
            float sum = 0.0f;
            for (int ss = 0; ss < S; ++ss)
                sum += __hip_atomic_load(&a.partial[((int64_t)ss * B + b) * a.Np + n], __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
            if (n < a.N) a.y[(int64_t)b * a.N + n] = sum;
        }
        if (tid == 0) __hip_atomic_store(&a.counters[tr], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

template <int B, bool PF>
static hipError_t launch_bp(const GemvArgs& a, bool xf32, bool raw, int threads, int blocks, size_t lds,
                            hipStream_t stream) {
    if (xf32) {
        if (raw)
            hipLaunchKernelGGL((gemv_kernel<B, true, true, PF>), dim3(blocks), dim3(threads), lds, stream, a);
        else
            hipLaunchKernelGGL((gemv_kernel<B, true, false, PF>), dim3(blocks), dim3(threads), lds, stream, a);
    } else {
        if (raw)
            hipLaunchKernelGGL((gemv_kernel<B, false, true, PF>), dim3(blocks), dim3(threads), lds, stream, a);
        else
            hipLaunchKernelGGL((gemv_kernel<B, false, false, PF>), dim3(blocks), dim3(threads), lds, stream, a);
    }
    return hipGetLastError();
}

template <int B>
static hipError_t launch_b(const GemvArgs& a, bool xf32, bool raw, bool pf, int threads, int blocks, size_t lds,
                           hipStream_t stream) {
    return pf ? launch_bp<B, true>(a, xf32, raw, threads, blocks, lds, stream)
              : launch_bp<B, false>(a, xf32, raw, threads, blocks, lds, stream);
}

hipError_t launch_gemv(const GemvArgs& a, int batch, bool xf32, bool raw, int threads, int blocks, size_t lds,
                       hipStream_t stream) {
    // more than one tile per wave in some block -> the prefetching variant
    const int waves = threads / 64;
    const int max_tiles = (a.TC + a.S - 1) / a.S;
    const bool pf = max_tiles > waves;
    switch (batch) {
        case 1: return launch_b<1>(a, xf32, raw, pf, threads, blocks, lds, stream);
        case 2: return launch_b<2>(a, xf32, raw, pf, threads, blocks, lds, stream);
        case 3: return launch_b<3>(a, xf32, raw, pf, threads, blocks, lds, stream);
        case 4: return launch_b<4>(a, xf32, raw, pf, threads, blocks, lds, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace se12
