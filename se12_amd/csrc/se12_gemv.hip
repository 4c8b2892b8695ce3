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
// Grid: block = W wave64s, one (tile row, K split) per block: blockIdx.x =
// tile row, blockIdx.y = split s, covering the K tiles [s*TC/S, (s+1)*TC/S).
// A grouped launch serves up to 4 matrices with the same K (q/k/v, gate/up)
// that share x: blockIdx.z = matrix, and the grid's x spans the tallest one
// (blocks past a shorter matrix's tile rows leave at once).
// Wave w of a block takes the split's tiles w, w + W, w + 2W, ... so in each
// round the block's waves read W consecutive tiles (contiguous HBM). The
// launch shape (W, S) alone fixes every accumulation order.
//
// Memory pipeline: a wave takes its tiles one round at a time (G tiles per
// round; the library launches G = 1) and reads the matching x slices
// straight from L2. A wave that owns 4 or more tiles keeps the next round's
// loads in flight while it decodes the current one (PF); with fewer, it
// loads, waits and decodes in turn, which staggers the chip's requests so
// that decode work overlaps the rest of the pass instead of piling up after
// its last byte (measured on MI355X: issuing every tile at once was slower). The block's waves meet once before decoding, after wave 0 has copied
// the bind-time pair table into LDS, and once for the final reduction.
//
// Reductions, all in a fixed order: DPP over the 16 lanes of a tile row,
// LDS over the block's waves (ascending), and for S > 1 the last block of a
// tile row to finish (device-scope arrival counter) sums the S partials in
// ascending split order. The counter is reset by that block, so no memset is
// needed between launches (graph-capture friendly).
//
// Optional decode-step tail (GemvEpilogue): the final y is then stored with
// device-scope stores and the block completing a gate/up tile row pair, or
// the whole matrix, applies the MLP gate or the residual RMSNorm in place of
// a separate launch.
//
// FAST variants need K % 256 == 0, 16-byte aligned BF16 x rows, and for the
// raw twin N % 16 == 0 and an aligned W; every other case runs the GENERIC
// variants (element loads guarded by the matrix edges, weights past K zeroed).
#include "se12_device.hpp"
#include "se12_internal.hpp"
#include "se12_step_math.hpp"

namespace se12 {

// x of one tile for one lane: B rows x 16 columns (BF16 pairs, or FP32).
template <int B, bool XF32>
struct XTile {
    uint32_t v[B][XF32 ? 16 : 8];
};

template <int B, bool XF32, bool GENERIC, bool XN>
__device__ __forceinline__ void load_x(XTile<B, XF32>& x, const GemvArgs& a, int kt, uint32_t lane, const uint16_t* xs) {
    const int64_t col = (int64_t)kt * kTileCols + 16 * (lane & 15u);
#pragma unroll
    for (int b = 0; b < B; ++b) {
        if constexpr (XN) {  // x rebuilt by the prologue, in LDS
            const uint4* p = reinterpret_cast<const uint4*>(xs + b * (int)a.K + (int)col);
            const uint4 u0 = p[0], u1 = p[1];
            x.v[b][0] = u0.x; x.v[b][1] = u0.y; x.v[b][2] = u0.z; x.v[b][3] = u0.w;
            x.v[b][4] = u1.x; x.v[b][5] = u1.y; x.v[b][6] = u1.z; x.v[b][7] = u1.w;
        } else if constexpr (!GENERIC) {
            const uint4* p = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(a.x) + b * a.K + col);
            const uint4 u0 = p[0], u1 = p[1];
            x.v[b][0] = u0.x; x.v[b][1] = u0.y; x.v[b][2] = u0.z; x.v[b][3] = u0.w;
            x.v[b][4] = u1.x; x.v[b][5] = u1.y; x.v[b][6] = u1.z; x.v[b][7] = u1.w;
        } else if constexpr (XF32) {
            const float* p = static_cast<const float*>(a.x) + b * a.K;
#pragma unroll
            for (int q = 0; q < 16; ++q) x.v[b][q] = (col + q < a.K) ? __float_as_uint(p[col + q]) : 0u;
        } else {
            const uint16_t* p = static_cast<const uint16_t*>(a.x) + b * a.K;
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const uint32_t lo = (col + 2 * q < a.K) ? (uint32_t)p[col + 2 * q] : 0u;
                const uint32_t hi = (col + 2 * q + 1 < a.K) ? (uint32_t)p[col + 2 * q + 1] : 0u;
                x.v[b][q] = lo | (hi << 16);
            }
        }
    }
}

// device-scope load / store of FP32 results that another block of the same
// launch wrote / will read
__device__ __forceinline__ float load_dev(const float* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_dev(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// GemvPrologue: every block rebuilds x (the decoder's next normalised input)
// from the previous product's FP32 output into LDS, with the arithmetic of
// se12_step_rmsnorm mode 1 (sums of squares over this block's threads).
// Its inputs are staged into LDS by direct-to-LDS loads (no registers held,
// so the first round's weights go out at the same time); the passes then
// run out of LDS. Block (0, 0) writes the new residual and x.
//
// LDS (after the kernel's reduction area; 16-byte aligned pieces,
// K % 256 == 0): y [B][K] FP32, residual [B][K] BF16, w1 [K], w2 [K], then
// x [B][K] BF16 (the new residual, then the kernel's x).
// bytes [0, n) of src into LDS at dst (16-byte aligned, n % 16 == 0), one
// KiB per wave instruction (lane i: bytes 16 i .. 16 i + 15 of the KiB)
__device__ __forceinline__ void stage_to_lds(const void* src, void* dst, int n, int w, int W, uint32_t lane) {
    for (int c = w * 1024; c < n; c += W * 1024) {
        const int off = c + (int)lane * 16;
        if (off < n)
            __builtin_amdgcn_global_load_lds(static_cast<const char*>(src) + off, static_cast<char*>(dst) + c, 16, 0, 0);
    }
}

template <int B>
__device__ __forceinline__ void gemv_prologue_stage(const GemvPrologue& pr, int64_t K, char* stage, int w, int W,
                                                    uint32_t lane) {
    const int k = (int)K;
    char* ys = stage;
    char* rs = ys + (size_t)B * k * 4;
    char* w1s = rs + (size_t)B * k * 2;
    char* w2s = w1s + (size_t)k * 2;
    stage_to_lds(pr.y_prev, ys, B * k * 4, w, W, lane);
    stage_to_lds(pr.res_in, rs, B * k * 2, w, W, lane);
    stage_to_lds(pr.w1, w1s, k * 2, w, W, lane);
    stage_to_lds(pr.w2, w2s, k * 2, w, W, lane);
    if (pr.y_prev_ss) {
        // the producer's per-tile-row sums of squares, 4 bytes per lane
        const int n = B * ((k + 15) / 16) * 4;
        char* ss = w2s + (size_t)k * 2;
        for (int c = w * 256; c < n; c += W * 256) {
            const int off = c + (int)lane * 4;
            if (off < n)
                __builtin_amdgcn_global_load_lds(reinterpret_cast<const char*>(pr.y_prev_ss) + off, ss + c, 4, 0, 0);
        }
    }
}

// after the staged loads have landed (the caller waits and meets the block)
template <int B>
__device__ void gemv_prologue_compute(const GemvPrologue& pr, int64_t K, char* stage, uint16_t* xs, float* sh) {
    using namespace se12step;
    const int tid = threadIdx.x, nt = blockDim.x;
    const int k = (int)K, n4 = k >> 2;
    const float4* ys = reinterpret_cast<const float4*>(stage);
    const uint2* rs = reinterpret_cast<const uint2*>(stage + (size_t)B * k * 4);
    const uint2* w1s = reinterpret_cast<const uint2*>(stage + (size_t)B * k * 6);
    const uint2* w2s = w1s + n4;
    const bool writer = blockIdx.x == 0 && blockIdx.y == 0 && blockIdx.z == 0;
    auto lo = [](uint32_t u) { return bf16_to_f(u & 0xFFFFu); };
    auto hi = [](uint32_t u) { return bf16_to_f(u >> 16); };
    auto pack = [](float a, float c) { return f_to_bf16x2(a, c); };
    const int trp = (k + 15) / 16;
    const float* row_ss = reinterpret_cast<const float*>(stage + (size_t)B * k * 6 + (size_t)k * 4);
    for (int b = 0; b < B; ++b) {
        const float4* yb = ys + (size_t)b * n4;
        const uint2* rb = rs + (size_t)b * n4;
        float inv;
        if (pr.y_prev_ss) {
            // from the producer's tile-row sums: lane l adds rows l, l + 64,
            // ... in order, then the wave's DPP tree; every wave gets the
            // same value, so no block barrier
            float ss = 0.0f;
            for (int i = (int)(tid & 63); i < trp; i += 64) ss += row_ss[b * trp + i];
            inv = rms_inv(wave_sum(ss), k, pr.eps);
        } else {
            float ss = 0.0f;
            for (int g = tid; g < n4; g += nt) {
                const float4 v = yb[g];
                const float4 t = make_float4(round_bf16(v.x), round_bf16(v.y), round_bf16(v.z), round_bf16(v.w));
                ss += t.x * t.x;
                ss += t.y * t.y;
                ss += t.z * t.z;
                ss += t.w * t.w;
            }
            inv = rms_inv(block_sum(ss, sh), k, pr.eps);
        }
        // the new residual (BF16-exact) goes to x's place in LDS, where the
        // same thread turns it into x
        uint2* xb = reinterpret_cast<uint2*>(xs + (size_t)b * k);
        // 4-element groups a thread holds in registers between the passes
        // (batch 1: at 2..4 rows the registers of the weights in flight
        // leave no room)
        constexpr int U = B == 1 ? 4 : 1;
        if (B == 1 && n4 <= U * nt) {
            // every LDS read of a pass issued at once (one latency per pass),
            // the residual kept in registers; the same arithmetic, in the
            // same order, as the loops below
            float4 v[U];
            uint2 c1[U], c2[U], c3[U], rp[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int g = tid + u * nt;
                if (g < n4) {
                    v[u] = yb[g];
                    c1[u] = w1s[g];
                    c2[u] = rb[g];
                    c3[u] = w2s[g];
                }
            }
            float ss2 = 0.0f;
#pragma unroll
            for (int u = 0; u < U; ++u) {
                if (tid + u * nt < n4) {
                    float4 r;
                    r.x = round_bf16(lo(c2[u].x) + round_bf16(rms_scale(round_bf16(v[u].x), inv, lo(c1[u].x))));
                    r.y = round_bf16(hi(c2[u].x) + round_bf16(rms_scale(round_bf16(v[u].y), inv, hi(c1[u].x))));
                    r.z = round_bf16(lo(c2[u].y) + round_bf16(rms_scale(round_bf16(v[u].z), inv, lo(c1[u].y))));
                    r.w = round_bf16(hi(c2[u].y) + round_bf16(rms_scale(round_bf16(v[u].w), inv, hi(c1[u].y))));
                    rp[u] = make_uint2(pack(r.x, r.y), pack(r.z, r.w));
                    ss2 += r.x * r.x;
                    ss2 += r.y * r.y;
                    ss2 += r.z * r.z;
                    ss2 += r.w * r.w;
                }
            }
            const float inv2 = rms_inv(block_sum(ss2, sh), k, pr.eps);
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int g = tid + u * nt;
                if (g < n4) {
                    const float4 r = make_float4(lo(rp[u].x), hi(rp[u].x), lo(rp[u].y), hi(rp[u].y));
                    const uint2 h = make_uint2(pack(rms_scale(r.x, inv2, lo(c3[u].x)), rms_scale(r.y, inv2, hi(c3[u].x))),
                                               pack(rms_scale(r.z, inv2, lo(c3[u].y)), rms_scale(r.w, inv2, hi(c3[u].y))));
                    xb[g] = h;
                    if (writer) {
                        reinterpret_cast<uint2*>(pr.res_out + (int64_t)b * K)[g] = rp[u];
                        reinterpret_cast<uint2*>(pr.h_out + (int64_t)b * K)[g] = h;
                    }
                }
            }
            continue;
        }
        float ss2 = 0.0f;
        for (int g = tid; g < n4; g += nt) {
            const float4 v = yb[g];
            const uint2 c1 = w1s[g], c2 = rb[g];
            float4 r;
            r.x = round_bf16(lo(c2.x) + round_bf16(rms_scale(round_bf16(v.x), inv, lo(c1.x))));
            r.y = round_bf16(hi(c2.x) + round_bf16(rms_scale(round_bf16(v.y), inv, hi(c1.x))));
            r.z = round_bf16(lo(c2.y) + round_bf16(rms_scale(round_bf16(v.z), inv, lo(c1.y))));
            r.w = round_bf16(hi(c2.y) + round_bf16(rms_scale(round_bf16(v.w), inv, hi(c1.y))));
            xb[g] = make_uint2(pack(r.x, r.y), pack(r.z, r.w));
            ss2 += r.x * r.x;
            ss2 += r.y * r.y;
            ss2 += r.z * r.z;
            ss2 += r.w * r.w;
        }
        const float inv2 = rms_inv(block_sum(ss2, sh), k, pr.eps);
        for (int g = tid; g < n4; g += nt) {
            const uint2 rp = xb[g];
            const float4 r = make_float4(lo(rp.x), hi(rp.x), lo(rp.y), hi(rp.y));
            const uint2 c3 = w2s[g];
            const uint2 h = make_uint2(pack(rms_scale(r.x, inv2, lo(c3.x)), rms_scale(r.y, inv2, hi(c3.x))),
                                       pack(rms_scale(r.z, inv2, lo(c3.y)), rms_scale(r.w, inv2, hi(c3.y))));
            xb[g] = h;
            if (writer) {
                reinterpret_cast<uint2*>(pr.res_out + (int64_t)b * K)[g] = rp;
                reinterpret_cast<uint2*>(pr.h_out + (int64_t)b * K)[g] = h;
            }
        }
    }
    __syncthreads();
}

// The decode-step work of GemvEpilogue, run by the block that has just
// written the final y of tile row `tr` (device-scope stores): it counts its
// arrival, and the block completing a tile row pair (kEpiGeluMul) or the
// matrix (kEpiRmsNorm) reads the results back and finishes the step. The
// arithmetic is that of se12_step_gelu_mul / se12_step_rmsnorm mode 1; the
// norm's sum of squares runs over this block's threads.
template <int B>
__device__ void gemv_epilogue(const GemvGroupArgs& ga, int tr, float* lds) {
    using namespace se12step;
    __shared__ int doer;
    const GemvEpilogue& e = ga.epi;
    const GemvArgs& a0 = ga.m[0];
    const int tid = threadIdx.x, nt = blockDim.x;
    const bool pair = e.kind == kEpiGeluMul;
    int32_t* cnt = a0.counters + (pair ? (int64_t)a0.TR + tr : 2 * (int64_t)a0.TR);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this block's y stores are complete
    __syncthreads();
    if (tid == 0) {
        const int old = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        doer = old == (pair ? 1 : a0.TR - 1);
    }
    __syncthreads();
    if (!doer) return;
    if (tid == 0) __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int64_t N = a0.N;
    if (pair) {
        if (tid < 16 * B) {
            const int64_t o = (int64_t)(tid >> 4) * N + (int64_t)tr * kTileRows + (tid & 15);
            if ((int64_t)tr * kTileRows + (tid & 15) < N)
                e.out[o] = gelu_mul_bf16(round_bf16(load_dev(a0.y + o)), round_bf16(load_dev(ga.m[1].y + o)));
        }
        return;
    }
    // RMSNorm of each batch row, four elements per step (the host asks for
    // rows % 4 == 0 and 8-byte aligned tensors): the row rounded to BF16, its
    // weights and residual are staged in LDS with every load of a pass
    // issued first; the passes then run out of LDS
    const int n = (int)N, n4 = n >> 2;
    float4* buf = reinterpret_cast<float4*>(lds);
    uint2* w1s = reinterpret_cast<uint2*>(lds + n);
    uint2* rs = w1s + n4;
    uint2* w2s = rs + n4;
    float* sh = reinterpret_cast<float*>(reinterpret_cast<char*>(lds) + ((10 * (size_t)n + 15) & ~(size_t)15));
    const uint2* w1g = reinterpret_cast<const uint2*>(e.w1);
    const uint2* w2g = reinterpret_cast<const uint2*>(e.w2);
    for (int b = 0; b < B; ++b) {
        const uint64_t* yr = reinterpret_cast<const uint64_t*>(a0.y + (int64_t)b * N);
        uint2* res = reinterpret_cast<uint2*>(e.residual + (int64_t)b * N);
        float ss = 0.0f;
        for (int g0 = 0; g0 < n4; g0 += 2 * nt) {
            uint64_t y01[2], y23[2];
            uint2 c1[2], c2[2], c3[2];
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                const int g = g0 + tid + k * nt;
                const int gc = g < n4 ? g : n4 - 1;  // clamped: every load is issued unconditionally
                y01[k] = __hip_atomic_load(yr + 2 * gc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                y23[k] = __hip_atomic_load(yr + 2 * gc + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                c1[k] = w1g[gc];
                c2[k] = res[gc];
                c3[k] = w2g[gc];
            }
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                const int g = g0 + tid + k * nt;
                if (g < n4) {
                    const float4 x = make_float4(round_bf16(__uint_as_float((uint32_t)y01[k])),
                                                 round_bf16(__uint_as_float((uint32_t)(y01[k] >> 32))),
                                                 round_bf16(__uint_as_float((uint32_t)y23[k])),
                                                 round_bf16(__uint_as_float((uint32_t)(y23[k] >> 32))));
                    buf[g] = x;
                    w1s[g] = c1[k];
                    rs[g] = c2[k];
                    w2s[g] = c3[k];
                    ss += x.x * x.x;
                    ss += x.y * x.y;
                    ss += x.z * x.z;
                    ss += x.w * x.w;
                }
            }
        }
        const float inv = rms_inv(block_sum(ss, sh), n, e.eps);
        float ss2 = 0.0f;
        auto lo = [](uint32_t u) { return bf16_to_f(u & 0xFFFFu); };
        auto hi = [](uint32_t u) { return bf16_to_f(u >> 16); };
        for (int g = tid; g < n4; g += nt) {
            const float4 x = buf[g];
            const uint2 w = w1s[g], r0 = rs[g];
            float4 r;
            r.x = round_bf16(lo(r0.x) + round_bf16(rms_scale(x.x, inv, lo(w.x))));
            r.y = round_bf16(hi(r0.x) + round_bf16(rms_scale(x.y, inv, hi(w.x))));
            r.z = round_bf16(lo(r0.y) + round_bf16(rms_scale(x.z, inv, lo(w.y))));
            r.w = round_bf16(hi(r0.y) + round_bf16(rms_scale(x.w, inv, hi(w.y))));
            buf[g] = r;
            ss2 += r.x * r.x;
            ss2 += r.y * r.y;
            ss2 += r.z * r.z;
            ss2 += r.w * r.w;
        }
        const float inv2 = rms_inv(block_sum(ss2, sh), n, e.eps);
        uint2* out = reinterpret_cast<uint2*>(e.out + (int64_t)b * N);
        for (int g = tid; g < n4; g += nt) {
            const float4 r = buf[g];
            const uint2 w = w2s[g];
            auto pack = [](float a, float c) { return f_to_bf16x2(a, c); };
            res[g] = make_uint2(pack(r.x, r.y), pack(r.z, r.w));
            out[g] = make_uint2(pack(rms_scale(r.x, inv2, lo(w.x)), rms_scale(r.y, inv2, hi(w.x))),
                                pack(rms_scale(r.z, inv2, lo(w.y)), rms_scale(r.w, inv2, hi(w.y))));
        }
        __syncthreads();  // the next row reuses the LDS
    }
}

struct RawLoads {
    uint4 v[4][2];
};

template <bool GENERIC>
__device__ __forceinline__ void load_raw_tile(RawLoads& t, const GemvArgs& a, int tr, int kt, uint32_t lane) {
    const int64_t col = (int64_t)kt * kTileCols + 16 * (lane & 15u);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int64_t row = (int64_t)tr * kTileRows + 4 * j + (lane >> 4);
        const uint16_t* p = a.wraw + row * a.K + col;
        if constexpr (!GENERIC) {
            t.v[j][0] = reinterpret_cast<const uint4*>(p)[0];
            t.v[j][1] = reinterpret_cast<const uint4*>(p)[1];
        } else {
            uint32_t h[8];
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const uint32_t lo = (row < a.N && col + 2 * q < a.K) ? (uint32_t)p[2 * q] : 0u;
                const uint32_t hi = (row < a.N && col + 2 * q + 1 < a.K) ? (uint32_t)p[2 * q + 1] : 0u;
                h[q] = lo | (hi << 16);
            }
            t.v[j][0] = make_uint4(h[0], h[1], h[2], h[3]);
            t.v[j][1] = make_uint4(h[4], h[5], h[6], h[7]);
        }
    }
}

// multiply-accumulate 8 BF16 weight pairs with the lane's x pairs of one row
template <bool XF32>
__device__ __forceinline__ float mac8(const uint32_t w[8], const uint32_t* xp, float acc) {
    if constexpr (XF32) {
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            acc = fmaf(__uint_as_float(w[q] << 16), __uint_as_float(xp[2 * q]), acc);
            acc = fmaf(__uint_as_float(w[q] & 0xFFFF0000u), __uint_as_float(xp[2 * q + 1]), acc);
        }
    } else {
#pragma unroll
        for (int q = 0; q < 8; ++q) acc = dot2_bf16(w[q], xp[q], acc);
    }
    return acc;
}

// zero the weights of tile columns >= lim (the valid columns of this K tile);
// in the GENERIC variants this keeps padding weights (codebook[0] << 7, which
// is +inf when codebook[0] == 255) from meeting the zero x padding
__device__ __forceinline__ void mask_cols(uint32_t w[8], int c0, int lim) {
#pragma unroll
    for (int q = 0; q < 8; ++q) {
        const int c = c0 + 2 * q;
        w[q] = (c >= lim) ? 0u : ((c + 1 >= lim) ? (w[q] & 0xFFFFu) : w[q]);
    }
}

// One SE12 tile: `info` / `esc` are the tile's wave-uniform side data. All
// 32 lookups are issued first, the escape patch (rare) runs behind one
// uniform branch, then the merges feed the dot products.
template <int B, bool XF32, bool GENERIC>
__device__ __forceinline__ void se12_tile(const GemvArgs& a, const TileLoads& t, uint32_t info, const TileSide& side,
                                          int g, const XTile<B, XF32>& x, const uint32_t* lut, int kt, uint32_t lane,
                                          float acc[4][B]) {
    const int c0 = 16 * (int)(lane & 15u);
    const int lim = GENERIC ? (int)(a.K - (int64_t)kt * kTileCols) : kTileCols;
    if (info_is_fallback(info)) {
        const int16_t* raw = raw_tile_ptr(info, a.fb_raw, a.ovf_raw);
        uint32_t w[4][8];
#pragma unroll
        for (int j = 0; j < 4; ++j) load_raw_chunk(raw, j, lane, w[j]);
        wait_vector_loads();  // rare path: keeps the common path's waits exact
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if constexpr (GENERIC) mask_cols(w[j], c0, lim);
#pragma unroll
            for (int b = 0; b < B; ++b) acc[j][b] = mac8<XF32>(w[j], x.v[b], acc[j][b]);
        }
    } else {
        uint32_t pat[4][8];
        lookup_tile(lut, t, pat);
        patch_tile_escapes(pat, info, side, g, lane);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            uint32_t w[8];
            merge_chunk(pat[j], t.sm[j], w);
            if constexpr (GENERIC) mask_cols(w, c0, lim);
#pragma unroll
            for (int b = 0; b < B; ++b) acc[j][b] = mac8<XF32>(w, x.v[b], acc[j][b]);
        }
    }
}

template <int B, bool XF32>
__device__ __forceinline__ void raw_tile(const RawLoads& t, const XTile<B, XF32>& x, float acc[4][B]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t w[8] = {t.v[j][0].x, t.v[j][0].y, t.v[j][0].z, t.v[j][0].w,
                               t.v[j][1].x, t.v[j][1].y, t.v[j][1].z, t.v[j][1].w};
#pragma unroll
        for (int b = 0; b < B; ++b) acc[j][b] = mac8<XF32>(w, x.v[b], acc[j][b]);
    }
}

// The loads of one round: G tiles (clamped to a valid tile of the split when
// the wave owns fewer, so every load is unconditional and the compiler's wait
// counts stay exact), their x slices and their side data (lane g: tile g).
template <int B, bool XF32, bool RAW, int G>
struct Round {
    XTile<B, XF32> x[G];
    TileSide side;
    TileLoads t[RAW ? 1 : G];
    RawLoads r[RAW ? G : 1];
};

// The leading arguments hold matrix 0's hot arguments (the weight stream
// pointer: sm, or W for the raw twin; ec, side records, pair table, x; tile
// columns, K splits, tile rows; waves per block). The library is built with
// those 9 arguments preloaded into SGPRs by the dispatch, so a block of
// matrix 0 issues its first tile loads without waiting for a kernel-argument
// load; the rest of the arguments (and every argument of matrices 1..3)
// arrive by scalar loads.
template <int B, bool XF32, bool RAW, int G, bool PF, bool GENERIC, bool XN>
__global__ __launch_bounds__(gemv_max_threads(B, XF32, RAW, G, PF, GENERIC))
__attribute__((amdgpu_waves_per_eu(gemv_waves_per_simd(B, RAW, G, PF, GENERIC)))) void gemv_kernel(
    const void* w0, const uint8_t* ec0, const uint32_t* side0, const uint32_t* lut0, const void* x0, int32_t TC0,
    int32_t S0, int32_t TR0, int32_t W, GemvGroupArgs ga) {
    SE12_DECLARE_LUT(lut);
    extern __shared__ __attribute__((aligned(16))) float dyn[];
    // the block's matrix and tile row come from the grid
    const int z = blockIdx.z;
    const GemvArgs& m = ga.m[z];
    GemvArgs a = {};
    if (z == 0) {
        if constexpr (RAW)
            a.wraw = static_cast<const uint16_t*>(w0);
        else
            a.sm = static_cast<const uint8_t*>(w0);
        a.ec = ec0;
        a.side = side0;
        a.lut = lut0;
        a.x = x0;
        a.TC = TC0;
        a.S = S0;
        a.TR = TR0;
    } else {
        // one batch of scalar loads (issued where first used, each would wait
        // behind the one before)
        a.sm = m.sm;
        a.wraw = m.wraw;
        a.ec = m.ec;
        a.side = m.side;
        a.lut = m.lut;
        a.x = m.x;
        a.TC = m.TC;
        a.S = m.S;
        a.TR = m.TR;
        asm volatile("" ::"s"(a.sm), "s"(a.wraw), "s"(a.ec), "s"(a.side), "s"(a.lut), "s"(a.x), "s"(a.TC), "s"(a.S),
                     "s"(a.TR));
    }
    // the other arguments: loaded once the first tiles are in flight, except
    // where the first loads' addresses need K and N (raw twin, edge handling)
    auto load_cold = [&]() {
        a.fb_raw = m.fb_raw;
        a.ovf_raw = m.ovf_raw;
        a.y = m.y;
        a.partial = m.partial;
        a.counters = m.counters;
        a.pairs = m.pairs;
        a.N = m.N;
        a.K = m.K;
        a.Np = m.Np;
    };
    constexpr bool kEarlyCold = RAW || GENERIC || B > 1;
    if constexpr (kEarlyCold) load_cold();
    const int tr = (int)blockIdx.x;
    if (tr >= a.TR) return;  // past a shorter matrix of a grouped launch
    // dynamic LDS: [x of the prologue (XN), 16-byte aligned] then the reductions
    // dynamic LDS: the reductions, then (XN) the prologue's staged inputs and
    // x, whose offsets depend on K (a scalar load): computed where first used
    float* red = dyn;
    char* const stage = reinterpret_cast<char*>(dyn) + lds_align16((size_t)W * B * 16 * sizeof(float));
    auto x_lds = [&]() { return reinterpret_cast<uint16_t*>(stage + gemv_pro_stage_bytes(a.K, B)); };
    uint16_t* xs = nullptr;
    const uint32_t lane = threadIdx.x & 63u;
    const int w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int S = a.S;
    const int s = blockIdx.y;
    const int kb = (int)(((uint32_t)s * (uint32_t)a.TC) / (uint32_t)S);
    const int ke = (int)(((uint32_t)(s + 1) * (uint32_t)a.TC) / (uint32_t)S);
    const int mine = (ke - kb - w + W - 1) / W;  // tiles of this wave (may be <= 0)
    const int last = mine > 0 ? kb + w + W * (mine - 1) : kb;
    const int rounds = mine > 0 ? (mine + G - 1) / G : 1;
    const int64_t row_tiles = (int64_t)tr * a.TC;

    float acc[4][B];
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int b = 0; b < B; ++b) acc[j][b] = 0.0f;

    auto tile_at = [&](int i) {
        const int kt = kb + w + W * i;
        return kt <= last ? kt : last;
    };
    auto load_round = [&](Round<B, XF32, RAW, G>& rd, int r) {
        if constexpr (!RAW) {
            // lane g: side data of tile g (lanes past G read the next round's
            // tiles, clamped, which keeps the addresses lane-dependent)
            // slot s = lane / 16 reads round tile s (clamped: slots past G
            // re-read the last one)
            load_side(rd.side, a.side, row_tiles + tile_at(r * G + ((int)(lane >> 4) < G ? (int)(lane >> 4) : G - 1)), lane);
        }
#pragma unroll
        for (int g = 0; g < G; ++g) load_x<B, XF32, GENERIC, XN>(rd.x[g], a, tile_at(r * G + g), lane, xs);
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const int kt = tile_at(r * G + g);
            if constexpr (RAW)
                load_raw_tile<GENERIC>(rd.r[g], a, tr, kt, lane);
            else
                load_tile(rd.t[g], a.sm, a.ec, row_tiles + kt, lane);
        }
    };
    // the first round of an XN launch: weights before the prologue, x after it
    auto load_round_w = [&](Round<B, XF32, RAW, G>& rd, int r) {
        if constexpr (!RAW)
            load_side(rd.side, a.side, row_tiles + tile_at(r * G + ((int)(lane >> 4) < G ? (int)(lane >> 4) : G - 1)), lane);
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const int kt = tile_at(r * G + g);
            if constexpr (RAW)
                load_raw_tile<GENERIC>(rd.r[g], a, tr, kt, lane);
            else
                load_tile(rd.t[g], a.sm, a.ec, row_tiles + kt, lane);
        }
    };
    auto load_round_x = [&](Round<B, XF32, RAW, G>& rd, int r) {
#pragma unroll
        for (int g = 0; g < G; ++g) load_x<B, XF32, GENERIC, XN>(rd.x[g], a, tile_at(r * G + g), lane, xs);
    };
    auto use_round = [&](const Round<B, XF32, RAW, G>& rd, int r) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const int i = r * G + g;
            if (i < mine) {
                if constexpr (RAW)
                    raw_tile<B, XF32>(rd.r[g], rd.x[g], acc);
                else
                    se12_tile<B, XF32, GENERIC>(a, rd.t[g], side_info(rd.side, g), rd.side, g, rd.x[g], lut,
                                                kb + w + W * i, lane, acc);
            }
        }
    };

    uint4 lutv;
    if constexpr (!RAW) lutv = reinterpret_cast<const uint4*>(a.lut)[lane];
    __builtin_amdgcn_sched_barrier(0);  // the table load goes out first
    Round<B, XF32, RAW, G> r0, r1;
    if constexpr (XN) {
        // the prologue's inputs (straight to LDS) and the first round's
        // weights go out together; x of the first round after the prologue
        // the first round's weights from the preloaded arguments, then the
        // prologue's inputs once their pointers (scalar loads) are in
        load_round_w(r0, 0);
        if constexpr (!kEarlyCold) load_cold();
        const GemvPrologue pro = ga.pro;
        gemv_prologue_stage<B>(pro, a.K, stage, w, W, lane);
        if constexpr (!RAW) store_block_lut(lut, lutv, lane);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the staged inputs have landed
        __syncthreads();
        xs = x_lds();
        gemv_prologue_compute<B>(pro, a.K, stage, xs, red);  // ends with a barrier
        load_round_x(r0, 0);
    } else {
        load_round(r0, 0);
        if constexpr (!kEarlyCold) load_cold();
        if constexpr (!RAW) {
            store_block_lut(lut, lutv, lane);
            lds_barrier();
        }
    }
    // the arguments of the tail, loaded while the first tiles are in flight
    // (a scalar load issued at the tail would hold the last stores)
    const int epi_kind = ga.epi.kind;
    float* const row_ss = ga.epi.row_ss;
    asm volatile("" ::"s"(a.y), "s"(a.N), "s"(epi_kind), "s"(row_ss));
    if constexpr (PF) {
        // one round in flight while a round decodes, waited for at the end of
        // that round (two rounds in flight measured slower: 4608x36864 at
        // batch 1 53.7 against 50.6 us, 2304x9216 9.1 against 8.7 us). The
        // last round loads nothing: a wave cannot end before its loads land,
        // so a dummy load there would hold the end of the kernel. The full
        // waits (seen by the compiler) keep every path's wait counts exact.
        // Inside the loop every load is issued on every path (a load skipped
        // on one path would merge into a wait for all loads in flight); the
        // last round is decoded after it.
        int r = 0;
        while (true) {
            if (r + 1 >= rounds) {
                use_round(r0, r);
                break;
            }
            load_round(r1, r + 1);
            use_round(r0, r);
            wait_vector_loads();
            if (++r + 1 >= rounds) {
                use_round(r1, r);
                break;
            }
            load_round(r0, r + 1);
            use_round(r1, r);
            wait_vector_loads();
            ++r;
        }
    } else {
        for (int r = 0; r < rounds; ++r) {
            if (r > 0) load_round(r0, r);
            use_round(r0, r);
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

    const int tid = threadIdx.x;
    const int b = tid >> 4;
    const int rr = tid & 15;
    const int64_t n = (int64_t)tr * kTileRows + rr;
    float v = 0.0f;
    if (tid < 16 * B) {
        for (int ww = 0; ww < W; ++ww) v += red[(ww * B + b) * 16 + rr];
    }
    const bool epi = epi_kind != kEpiNone;
    if (S > 1 && !epi && !row_ss) {
        // each output's S partials meet in the pair tree; the split holding
        // the total stores it
        if (tid < 16 * B && pair_tree_sum(a.pairs + (int64_t)b * a.Np + n, (int64_t)B * a.Np, s, S, v) && n < a.N)
            a.y[(int64_t)b * a.N + n] = v;
        return;
    }
    if (S > 1) {
        // Cross-block reduction without cache-wide maintenance: the partials
        // are written with device-scope stores, each thread waits for its
        // stores to complete before the block's arrival is counted, and the
        // last block reads them back with device-scope loads. (A
        // __threadfence() here would write back and invalidate the whole L2
        // of the XCD for every block.)
        if (tid < 16 * B) store_dev(&a.partial[((int64_t)s * B + b) * a.Np + n], v);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        int* flag = reinterpret_cast<int*>(red);
        if (tid == 0) {
            const int old = __hip_atomic_fetch_add(&a.counters[tr], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            *flag = (old == S - 1) ? 1 : 0;
        }
        __syncthreads();
        if (!*flag) return;
        if (tid < 16 * B) {
            // the splits' partials in ascending split order, one load per add:
            // this path serves only launches with a decode-step tail (split
            // launches without one meet in the pair tree above), and the
            // smaller code keeps the cold-cache batch-1 launches short (the 2B
            // q and k alone, 26 launches after an eviction: 5.11 / 4.92 us
            // with 8 loads in flight here, 4.71 / 4.52 with one)
            v = 0.0f;
            for (int ss = 0; ss < S; ++ss) v += load_dev(&a.partial[((int64_t)ss * B + b) * a.Np + n]);
        }
        if (tid == 0) __hip_atomic_store(&a.counters[tr], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (tid < 16 * B && n < a.N) {
        if (epi)
            store_dev(&a.y[(int64_t)b * a.N + n], v);  // read back by the block that runs the epilogue
        else
            a.y[(int64_t)b * a.N + n] = v;
    }
    if (row_ss && tid < 64) {  // wave 0, all lanes: the 16-lane trees of the batch rows
        const float t = (tid < 16 * B && n < a.N) ? se12step::round_bf16(v) : 0.0f;
        const float q = row16_sum(t * t);
        if (tid < 16 * B && (tid & 15) == 0) row_ss[(int64_t)b * a.TR + tr] = q;
    }
    if (epi) gemv_epilogue<B>(ga, tr, red);
}

namespace {

template <int B, bool XF32, bool RAW, int G, bool PF, bool GENERIC, bool XN = false>
hipError_t go(const GemvGroupArgs& a, int threads, int blocks, size_t lds, hipStream_t stream) {
    (void)blocks;
    const GemvArgs& m0 = a.m[0];
    const void* w0 = RAW ? static_cast<const void*>(m0.wraw) : static_cast<const void*>(m0.sm);
    hipLaunchKernelGGL((gemv_kernel<B, XF32, RAW, G, PF, GENERIC, XN>), dim3(group_grid_x(a), m0.S, a.count), dim3(threads), lds,
                       stream, w0, m0.ec, m0.side, m0.lut, m0.x, m0.TC, m0.S, m0.TR, threads / 64, a);
    return hipGetLastError();
}

template <int B, bool RAW>
hipError_t launch_b(const GemvGroupArgs& a, const GemvPlan& p, hipStream_t stream) {
    const int threads = p.waves * 64;
    if (p.xn)
        return p.pf ? go<B, false, RAW, 1, true, false, true>(a, threads, p.blocks, p.lds, stream)
                    : go<B, false, RAW, 1, false, false, true>(a, threads, p.blocks, p.lds, stream);
    if (p.generic)
        return p.xf32 ? go<B, true, RAW, 1, false, true>(a, threads, p.blocks, p.lds, stream)
                      : go<B, false, RAW, 1, false, true>(a, threads, p.blocks, p.lds, stream);
    return p.pf ? go<B, false, RAW, 1, true, false>(a, threads, p.blocks, p.lds, stream)
                : go<B, false, RAW, 1, false, false>(a, threads, p.blocks, p.lds, stream);
}

}  // namespace

// row_ss of a product whose launch did not write it (the MFMA kernel): the
// same 16-lane tree over bf16(y)^2 as the dot2 tail, so the values agree
// wherever y does. Grid (tile rows, batch rows), one wave per block.
__global__ __launch_bounds__(64) void row_sumsq_kernel(const float* y, int64_t N, int32_t TR, float* row_ss) {
    const int tr = blockIdx.x, b = blockIdx.y, lane = threadIdx.x;
    const int64_t n = (int64_t)tr * kTileRows + (lane & 15);
    const float t = (lane < 16 && n < N) ? se12step::round_bf16(y[(int64_t)b * N + n]) : 0.0f;
    const float q = row16_sum(t * t);
    if (lane == 0) row_ss[(int64_t)b * TR + tr] = q;
}

hipError_t launch_row_sumsq(const float* y, int64_t N, int32_t TR, int32_t batch, float* row_ss, hipStream_t stream) {
    hipLaunchKernelGGL(row_sumsq_kernel, dim3(TR, batch), dim3(64), 0, stream, y, N, TR, row_ss);
    return hipGetLastError();
}

hipError_t launch_gemv(const GemvGroupArgs& a, const GemvPlan& p, hipStream_t stream) {
    switch (p.batch * 2 + (p.raw ? 1 : 0)) {
        case 2: return launch_b<1, false>(a, p, stream);
        case 3: return launch_b<1, true>(a, p, stream);
        case 4: return launch_b<2, false>(a, p, stream);
        case 5: return launch_b<2, true>(a, p, stream);
        case 6: return launch_b<3, false>(a, p, stream);
        case 7: return launch_b<3, true>(a, p, stream);
        case 8: return launch_b<4, false>(a, p, stream);
        case 9: return launch_b<4, true>(a, p, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace se12
