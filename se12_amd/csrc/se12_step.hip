// Decode-step kernels of a Gemma-2 style decoder (one new token per
// sequence), so that a step is a handful of launches around the fused
// products instead of ~80 small framework kernels per layer. They take the
// products' FP32 outputs (or BF16, for a BF16 baseline) and reproduce the
// rounding sequence of the eager step: every framework BF16 op rounds its
// FP32 result to BF16 (round to nearest even), so do these, op by op.
//
//   rmsnorm        norm(x) = x * rsqrt(mean(x^2) + eps) * (1 + w), FP32 math,
//                  BF16 result; mode 1 fuses t = bf16(y), x = bf16(x + norm(t, w1)),
//                  h = norm(x, w2) (post-norm, residual add, next pre-norm)
//   attention      two launches over (sequence, KV head, 64-position chunk):
//                  q/k/v to BF16, rotary embedding, K/V written to the caches
//                  at `pos`, scores against positions 0..pos (or the sliding
//                  window), scaling, tanh soft-capping; then softmax in FP32
//                  and the weighted sum of V, chunk partials added in order
//   gelu_mul       bf16(gelu_tanh(bf16(g)) * bf16(u))
//   logits_argmax  final soft-capping of the logits and the greedy token,
//                  blocks over vocabulary slices, the last one picks
//   advance        pos += 1, step += 1
//
// Every kernel is latency-bound at decode sizes (a few KB to a few MB per
// launch): each thread issues all its loads before using any of them, and
// the caches are read 16 bytes per lane.
//
// The caches: K transposed [batch, kv_heads, head_dim, max_len] (so that a
// framework batched product can read it as a contiguous right operand), V
// [batch, kv_heads, max_len, head_dim], both BF16.
//
// Cross-block results (attention partials, argmax partials) are written with
// device-scope stores and counted in per-row arrival counters; the last block
// reads them back with device-scope loads in a fixed order and resets its
// counter, so results are deterministic and no memset is needed between calls.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "se12_step.h"
#include "se12_step_math.hpp"

namespace se12step {

// element i of an FP32 or BF16 tensor, rounded to BF16 (the framework's
// `.to(torch.bfloat16)` of a product output)
template <int DT>
__device__ __forceinline__ float load_as_bf16(const void* p, int64_t i) {
    if constexpr (DT == SE12_STEP_F32)
        return round_bf16(static_cast<const float*>(p)[i]);
    else
        return bf16_to_f(static_cast<const uint16_t*>(p)[i]);
}

__device__ __forceinline__ float load_as_bf16(const void* p, int dtype, int64_t i) {
    return dtype == SE12_STEP_F32 ? load_as_bf16<SE12_STEP_F32>(p, i) : load_as_bf16<SE12_STEP_BF16>(p, i);
}

// 8 BF16 values from 16 bytes
__device__ __forceinline__ void unpack8(const uint4 r, float* v) {
    const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        v[2 * i] = __uint_as_float(w[i] << 16);
        v[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
    }
}

// (value, index) with the larger value, the smaller index on a tie; NaN
// ranks above every number (torch.argmax's order), so a row of NaNs still
// gives an index in the vocabulary (its first NaN) and never the initial one
__device__ __forceinline__ void keep_first_max(float& bv, int& bi, float v, int i) {
    const bool vn = v != v, bn = bv != bv;
    if (vn ? (!bn || i < bi) : (!bn && (v > bv || (v == bv && i < bi)))) {
        bv = v;
        bi = i;
    }
}

// ---------------------------------------------------------------------------
// rmsnorm: one block per row, kNormPer elements per thread, all loads first
// ---------------------------------------------------------------------------

constexpr int kNormPer = 8;
constexpr int kNormMaxThreads = 1024;

struct NormArgs {
    const void* in;
    int64_t in_stride;
    const uint16_t* w1;
    uint16_t* residual;
    const uint16_t* w2;
    uint16_t* out;
    int hidden;
    float eps, in_scale;
};

template <int DT, int MODE>
__global__ __launch_bounds__(kNormMaxThreads) void rmsnorm_kernel(NormArgs a) {
    __shared__ float sh[17];
    const int r = blockIdx.x, t = threadIdx.x, nt = blockDim.x;
    const int64_t base = (int64_t)r * a.in_stride, rbase = (int64_t)r * a.hidden;
    float x[kNormPer], w1[kNormPer], res[kNormPer], w2[kNormPer];
#pragma unroll
    for (int k = 0; k < kNormPer; ++k) {
        const int i = t + k * nt;
        const int ic = i < a.hidden ? i : a.hidden - 1;  // clamped: every load is issued unconditionally
        x[k] = load_as_bf16<DT>(a.in, base + ic);
        w1[k] = bf16_to_f(a.w1[ic]);
        if constexpr (MODE == 1) {
            res[k] = bf16_to_f(a.residual[rbase + ic]);
            w2[k] = bf16_to_f(a.w2[ic]);
        }
    }
    float ss = 0.0f;
#pragma unroll
    for (int k = 0; k < kNormPer; ++k) {
        if constexpr (MODE == 0)
            if (a.in_scale != 0.0f) x[k] = round_bf16(x[k] * a.in_scale);  // scaled embedding row
        if (t + k * nt < a.hidden) ss += x[k] * x[k];
    }
    const float inv = rms_inv(block_sum(ss, sh), a.hidden, a.eps);
    if constexpr (MODE == 0) {
#pragma unroll
        for (int k = 0; k < kNormPer; ++k) {
            const int i = t + k * nt;
            if (i < a.hidden) {
                if (a.residual) a.residual[rbase + i] = f_to_bf16(x[k]);
                a.out[rbase + i] = f_to_bf16(rms_scale(x[k], inv, w1[k]));
            }
        }
        return;
    }
    // mode 1: residual += norm(bf16(in), w1); out = norm(residual, w2)
    float ss2 = 0.0f;
#pragma unroll
    for (int k = 0; k < kNormPer; ++k) {
        const float n1 = round_bf16(rms_scale(x[k], inv, w1[k]));
        res[k] = round_bf16(res[k] + n1);
        if (t + k * nt < a.hidden) ss2 += res[k] * res[k];
    }
    const float inv2 = rms_inv(block_sum(ss2, sh), a.hidden, a.eps);
#pragma unroll
    for (int k = 0; k < kNormPer; ++k) {
        const int i = t + k * nt;
        if (i < a.hidden) {
            a.residual[rbase + i] = f_to_bf16(res[k]);
            a.out[rbase + i] = f_to_bf16(rms_scale(res[k], inv2, w2[k]));
        }
    }
}

// ---------------------------------------------------------------------------
// attention: the positions 0..pos are cut into chunks of 64; one block per
// (sequence, KV head, chunk) in each of two launches:
//   scores  rotary embedding of q (and of k, in the block holding pos, which
//           also writes the new K/V slot), the chunk's scores for the G query
//           heads of the KV head, the chunk's max m_c and sum l_c of
//           exp(s - m_c);
//   pv      one block per (sequence, KV head, 32 head-dim columns, span of
//           positions): the global max M = max m_c and sum S =
//           sum l_c exp(m_c - M), the probabilities p = bf16(exp(s - M) / S)
//           (softmax in FP32, rounded as the framework rounds it) and the
//           sum p . V of its columns over its span in FP32. A span covers
//           1024 positions (256 x G query heads of registers per thread),
//           so caches up to that need one span and write the output
//           directly; longer ones write partial sums that the last block of
//           a (sequence, KV head, columns) adds in span order. Splitting
//           the columns instead of the positions keeps a short cache's
//           blocks free of that cross-block reduction.
// ---------------------------------------------------------------------------

constexpr int kChunk = 64;
constexpr int kAttnThreads = 256;
constexpr int kMaxHeadDim = 256;

struct AttnArgs {
    const void* q;
    const void* k;
    const void* v;
    int dtype;
    int64_t q_stride, kv_stride;
    uint16_t* kt;            // [B, kvh, d, L]
    uint16_t* vc;            // [B, kvh, L, d]
    const float* inv_freq;   // [d / 2]
    const int64_t* pos;
    uint16_t* out;           // [B, heads * d]
    float* scores;           // [B, heads, chunks * 64]
    float* stats;            // [B, heads, chunks, 2]: m_c, l_c
    float* partial;          // [B, heads, spans <= chunks, d]
    int* counters;           // [B * kvh * column blocks], zero between launches
    int heads, kvh, d, max_len, chunks;
    float scaling, softcap;
    int window;
};

__device__ __forceinline__ int window_lo(int p, int window) {
    return window > 0 ? (p - window + 1 > 0 ? p - window + 1 : 0) : 0;
}

// a wave-uniform 64-bit value held in a vector register, as a scalar
__device__ __forceinline__ int64_t uniform_i64(int64_t v) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)((uint64_t)v >> 32));
    return (int64_t)(((uint64_t)hi << 32) | lo);
}

// Makes the wave wait for a loaded value here: issued before a branch on the
// position, loads would otherwise be sunk past it and wait for it.
__device__ __forceinline__ void pin(float v) { asm volatile("" ::"v"(v)); }
__device__ __forceinline__ void pin(const uint4& v) { asm volatile("" ::"v"(v.x), "v"(v.y), "v"(v.z), "v"(v.w)); }

// Rotary embedding, with the framework's roundings, of the G queries and
// the key whose element t thread t < d holds in x[0..G]; the rotated values
// land in y and in qk ([G + 1][d] in LDS). Every thread of the block calls
// it (two barriers).
template <int G>
__device__ __forceinline__ void rotate_qk(float* qk, const float (&x)[G + 1], float fr, int p, int d, int t,
                                          float (&y)[G + 1]) {
    const int half = d / 2;
    if (t < d) {
#pragma unroll
        for (int h = 0; h <= G; ++h) qk[h * d + t] = x[h];
    }
    __syncthreads();
    if (t < d) {
        const float freq = (float)p * fr;
        const float cs = round_bf16(cosf(freq)), sn = round_bf16(sinf(freq));
#pragma unroll
        for (int h = 0; h <= G; ++h) {
            const float* xv = qk + h * d;
            const float rot = t < half ? -xv[t + half] : xv[t - half];
            y[h] = round_bf16(round_bf16(xv[t] * cs) + round_bf16(rot * sn));
        }
    }
    __syncthreads();
    if (t < d) {
#pragma unroll
        for (int h = 0; h <= G; ++h) qk[h * d + t] = y[h];
    }
}

// One 64-position chunk of keys against the G rotated queries in qk, for a
// team of 4 waves (tt = thread in the team): lane group pg = tt % 8 takes 8
// consecutive positions jgl.. (one 16-byte load per head-dim element), the
// 32 slices es = tt / 8 every 32nd element. The key at position p comes from
// qk (its cache slot is written in the same launch). The wave's 8 slices
// are summed (lane bits 3..5) and lanes 0..7 write the wave's sums to red
// ([4 waves][G][64]).
template <int G>
__device__ __forceinline__ void chunk_key_dots(const uint4 (&raw)[kMaxHeadDim / 32], const float* qk, int d, int tt,
                                               int jgl, int p, float* red) {
    const int pg = tt & 7, es = tt >> 3, tw = tt >> 6;
    float acc[8][G];
#pragma unroll
    for (int m = 0; m < 8; ++m)
#pragma unroll
        for (int h = 0; h < G; ++h) acc[m][h] = 0.0f;
#pragma unroll
    for (int i = 0; i < kMaxHeadDim / 32; ++i) {
        const int e = es + 32 * i;
        if (e < d) {
            float kv[8];
            unpack8(raw[i], kv);
#pragma unroll
            for (int m = 0; m < 8; ++m)
                if (jgl + m == p) kv[m] = qk[G * d + e];
#pragma unroll
            for (int h = 0; h < G; ++h) {
                const float qv = qk[h * d + e];
#pragma unroll
                for (int m = 0; m < 8; ++m) acc[m][h] += qv * kv[m];
            }
        }
    }
#pragma unroll
    for (int m = 0; m < 8; ++m)
#pragma unroll
        for (int h = 0; h < G; ++h) {
            float v = acc[m][h];
            v += __shfl_xor(v, 8, 64);
            v += __shfl_xor(v, 16, 64);
            v += __shfl_xor(v, 32, 64);
            acc[m][h] = v;
        }
    if ((tt & 63) < 8) {
#pragma unroll
        for (int h = 0; h < G; ++h)
#pragma unroll
            for (int m = 0; m < 8; ++m) red[(tw * G + h) * kChunk + 8 * pg + m] = acc[m][h];
    }
}

// For thread t < 64 (one wave): the score of position j0 + t for each head
// (the 4 waves' dots in order, scaling, soft-capping, -inf outside
// [lo, p]) and the chunk's max m and sum l of exp(score - m).
template <int G>
__device__ __forceinline__ void chunk_scores(const float* red, const AttnArgs& a, int t, int j0, int p, int lo,
                                             float (&sc)[G], float (&m)[G], float (&l)[G]) {
    const int jq = j0 + t;
    const bool valid = jq <= p && jq >= lo;
#pragma unroll
    for (int h = 0; h < G; ++h) {
        const float dot = red[(0 * G + h) * kChunk + t] + red[(1 * G + h) * kChunk + t] +
                          red[(2 * G + h) * kChunk + t] + red[(3 * G + h) * kChunk + t];
        float v = round_bf16(round_bf16(dot) * a.scaling);
        if (a.softcap > 0.0f) v = round_bf16(round_bf16(tanhf(round_bf16(v / a.softcap))) * a.softcap);
        if (!valid) v = -INFINITY;
        sc[h] = v;
        m[h] = wave_max(v);                      // >= 1 valid position per chunk
        l[h] = wave_sum(valid ? expf(v - m[h]) : 0.0f);
    }
}

template <int G, int DT>
__global__ __launch_bounds__(kAttnThreads) void attn_scores_kernel(const int64_t* pos, const void* q, const void* k,
                                                                   uint16_t* kt, int32_t d_, int32_t L_, int32_t kvh,
                                                                   int32_t q_stride, int32_t kv_stride, AttnArgs ga) {
    // the leading arguments (preloaded into SGPRs by the dispatch) are the
    // ones the first loads need; the rest arrive by scalar loads meanwhile
    AttnArgs a = ga;
    a.pos = pos;
    a.q = q;
    a.k = k;
    a.kt = kt;
    a.d = d_;
    a.max_len = L_;
    a.kvh = kvh;
    a.q_stride = q_stride;
    a.kv_stride = kv_stride;
    __shared__ float qk[(G + 1) * kMaxHeadDim];   // rotated q of the G heads, then k
    __shared__ float red[4 * G * kChunk];         // per wave: G x 64 partial dot products
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const int kvb = blockIdx.x;                    // b * kvh + kh
    const int b = kvb / a.kvh, kh = kvb % a.kvh;
    const int c = blockIdx.y, j0 = c * kChunk;
    const int d = a.d, half = d / 2;
    const int L = a.max_len;

    // Every load whose address does not depend on the position goes out
    // together with the position's: q and k of the new token (to BF16) and
    // the chunk of the key cache, all from preloaded arguments; then v and
    // the rotary frequency, whose pointers are scalar loads. The position is
    // a vector load, so that waiting for those scalar loads does not wait for
    // it. Lane group pg = 8 consecutive positions read as one 16-byte load
    // per head-dim element; the 32 slices es take every 32nd element.
    const int64_t p64v = __hip_atomic_load(a.pos, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    float xq[G], xk = 0.0f, vv = 0.0f, fr = 0.0f;
    const int tc = t < d ? t : d - 1;
#pragma unroll
    for (int h = 0; h < G; ++h)
        xq[h] = load_as_bf16<DT>(a.q, (int64_t)b * a.q_stride + (int64_t)(kh * G + h) * d + tc);
    xk = load_as_bf16<DT>(a.k, (int64_t)b * a.kv_stride + (int64_t)kh * d + tc);
    const int pg = t & 7, es = t >> 3;
    const int jg = j0 + 8 * pg;
    const int jgl = jg + 8 <= L ? jg : L - 8;     // L % 8 == 0: a group is wholly in or out
    const uint16_t* kb = a.kt + (int64_t)kvb * d * L + jgl;
    uint4 raw[kMaxHeadDim / 32];
#pragma unroll
    for (int i = 0; i < kMaxHeadDim / 32; ++i) {
        const int e = es + 32 * i;
        raw[i] = *reinterpret_cast<const uint4*>(kb + (int64_t)(e < d ? e : d - 1) * L);
    }
    __builtin_amdgcn_sched_barrier(0);  // the loads above go out first
    vv = load_as_bf16<DT>(a.v, (int64_t)b * a.kv_stride + (int64_t)kh * d + tc);
    fr = a.inv_freq[tc % half];
#pragma unroll
    for (int h = 0; h < G; ++h) pin(xq[h]);
    pin(xk);
#pragma unroll
    for (int i = 0; i < kMaxHeadDim / 32; ++i) pin(raw[i]);
    const int64_t p64 = uniform_i64(p64v);

    if (p64 < 0 || p64 >= a.max_len) return;
    const int p = (int)p64, lo = window_lo(p, a.window);
    if (j0 > p || j0 + kChunk <= lo) return;
    const bool holds_p = p < j0 + kChunk;

    float x[G + 1], y[G + 1];
#pragma unroll
    for (int h = 0; h < G; ++h) x[h] = xq[h];
    x[G] = xk;
    rotate_qk<G>(qk, x, fr, p, d, t, y);
    if (t < d && holds_p) {
        a.kt[((int64_t)kvb * d + t) * L + p] = f_to_bf16(y[G]);
        a.vc[((int64_t)kvb * L + p) * d + t] = f_to_bf16(vv);
    }
    __syncthreads();
    chunk_key_dots<G>(raw, qk, d, t, jgl, p, red);
    __syncthreads();
    if (t < kChunk) {
        float sc[G], m[G], l[G];
        chunk_scores<G>(red, a, t, j0, p, lo, sc, m, l);
        const int64_t lp = (int64_t)a.chunks * kChunk;
#pragma unroll
        for (int h = 0; h < G; ++h) {
            const int64_t row = (int64_t)b * a.kvh * G + kh * G + h;
            a.scores[row * lp + j0 + t] = sc[h];
            if (t == 0) {
                a.stats[(row * a.chunks + c) * 2 + 0] = m[h];
                a.stats[(row * a.chunks + c) * 2 + 1] = l[h];
            }
        }
    }
}

// weighted V: positions per thread (all loads in flight at once) and the
// span of positions of one block
constexpr int kPvCols = 32;
template <int G>
constexpr int pv_per_thread() { return G <= 2 ? 16 : 32 / G; }
template <int G>
constexpr int pv_span() { return (kAttnThreads / (kPvCols / 8)) * pv_per_thread<G>(); }

template <int G>
__global__ __launch_bounds__(kAttnThreads) void attn_pv_kernel(const int64_t* pos, const float* stats, const float* scores,
                                                               const uint16_t* vc, int32_t d_, int32_t L_, int32_t kvh,
                                                               int32_t chunks, AttnArgs ga) {
    // the leading arguments (preloaded into SGPRs by the dispatch) are the
    // ones the first loads need; the rest arrive by scalar loads meanwhile
    AttnArgs a = ga;
    a.pos = pos;
    a.stats = const_cast<float*>(stats);
    a.scores = const_cast<float*>(scores);
    a.vc = const_cast<uint16_t*>(vc);
    a.d = d_;
    a.max_len = L_;
    a.kvh = kvh;
    a.chunks = chunks;
    constexpr int P = pv_per_thread<G>();
    constexpr int kSpan = pv_span<G>();
    __shared__ float ms[2 * G];
    __shared__ float red[4 * G * kPvCols];        // per wave: G x 32 column sums
    __shared__ int flag;
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const int kvb = blockIdx.x;
    const int b = kvb / a.kvh, kh = kvb % a.kvh;
    const int cb = blockIdx.y, sp = blockIdx.z;
    const int d = a.d, L = a.max_len;
    const int64_t obase = (int64_t)b * a.kvh * G * d + (int64_t)kh * G * d;
    const int64_t row0 = (int64_t)b * a.kvh * G + kh * G;
    const int64_t lp = (int64_t)a.chunks * kChunk;
    // thread: 8-column group cq of the block's 32 columns, position slice ps
    const int cq = t & 3, ps = t >> 2;
    const int e0 = cb * kPvCols + 8 * cq;
    const uint16_t* vb = a.vc + (int64_t)kvb * L * d + (e0 < d ? e0 : d - 8);
    const int jb = sp * kSpan;

    // Every load whose address does not depend on the position goes out
    // together with the position's: the statistics of the first 64 chunks of
    // the wave's heads (lane = chunk), and the span's V rows and scores.
    const int64_t p64v = __hip_atomic_load(a.pos, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // a vector load
    constexpr int kHeadsPerWave = (G + 3) / 4;
    float sm[kHeadsPerWave], sl[kHeadsPerWave];
    const int cl = lane < a.chunks ? lane : a.chunks - 1;
#pragma unroll
    for (int k = 0; k < kHeadsPerWave; ++k) {
        const int h = w + 4 * k < G ? w + 4 * k : G - 1;
        const float* st = a.stats + (row0 + h) * a.chunks * 2;
        sm[k] = st[cl * 2];
        sl[k] = st[cl * 2 + 1];
    }
    uint4 vr[P];
    float sc[P][G];
#pragma unroll
    for (int i = 0; i < P; ++i) {
        const int j = jb + ps + 64 * i;
        const int jc = j < L ? j : L - 1;
        vr[i] = *reinterpret_cast<const uint4*>(vb + (int64_t)jc * d);
#pragma unroll
        for (int h = 0; h < G; ++h) sc[i][h] = a.scores[(row0 + h) * lp + jc];
    }
#pragma unroll
    for (int k = 0; k < kHeadsPerWave; ++k) {
        pin(sm[k]);
        pin(sl[k]);
    }
#pragma unroll
    for (int i = 0; i < P; ++i) {
        pin(vr[i]);
#pragma unroll
        for (int h = 0; h < G; ++h) pin(sc[i][h]);
    }

    const int64_t p64 = uniform_i64(p64v);
    if (p64 < 0 || p64 >= L) {  // no cache slot: zeros, no cache or counter touched
        if (cb == 0 && sp == 0)
            for (int i = t; i < G * d; i += kAttnThreads) a.out[obase + i] = 0;
        return;
    }
    const int p = (int)p64, lo = window_lo(p, a.window);
    const int s_lo = lo / kSpan, s_hi = p / kSpan;
    if (sp < s_lo || sp > s_hi) return;
    const int c_lo = lo / kChunk, c_hi = p / kChunk;
    // global max and sum of each head over its chunks (one wave per head)
#pragma unroll
    for (int k = 0; k < kHeadsPerWave; ++k) {
        const int h = w + 4 * k;
        if (h >= G) break;
        const float* st = a.stats + (row0 + h) * a.chunks * 2;
        const bool mine = lane >= c_lo && lane <= c_hi;
        float m = mine ? sm[k] : -INFINITY;
        for (int cc = lane + 64; cc <= c_hi; cc += 64)
            if (cc >= c_lo) m = fmaxf(m, st[cc * 2]);
        m = wave_max(m);
        float s = mine ? sl[k] * expf(sm[k] - m) : 0.0f;
        for (int cc = lane + 64; cc <= c_hi; cc += 64)
            if (cc >= c_lo) s += st[cc * 2 + 1] * expf(st[cc * 2] - m);
        s = wave_sum(s);
        if (lane == 0) {
            ms[2 * h] = m;
            ms[2 * h + 1] = s;
        }
    }
    __syncthreads();
    float acc[8][G];
#pragma unroll
    for (int m = 0; m < 8; ++m)
#pragma unroll
        for (int h = 0; h < G; ++h) acc[m][h] = 0.0f;
#pragma unroll
    for (int i = 0; i < P; ++i) {
        const int j = jb + ps + 64 * i;
        if (j >= lo && j <= p) {   // V past pos may hold anything (0 x NaN)
            float v[8];
            unpack8(vr[i], v);
#pragma unroll
            for (int h = 0; h < G; ++h) {
                const float pr = round_bf16(expf(sc[i][h] - ms[2 * h]) / ms[2 * h + 1]);
#pragma unroll
                for (int m = 0; m < 8; ++m) acc[m][h] += pr * v[m];
            }
        }
    }
    // the 16 position slices of a wave (lane bits 2..5), then the 4 waves in order
#pragma unroll
    for (int m = 0; m < 8; ++m)
#pragma unroll
        for (int h = 0; h < G; ++h) {
            float v = acc[m][h];
            v += __shfl_xor(v, 4, 64);
            v += __shfl_xor(v, 8, 64);
            v += __shfl_xor(v, 16, 64);
            v += __shfl_xor(v, 32, 64);
            acc[m][h] = v;
        }
    if (lane < 4) {
#pragma unroll
        for (int h = 0; h < G; ++h)
#pragma unroll
            for (int m = 0; m < 8; ++m) red[(w * G + h) * kPvCols + 8 * cq + m] = acc[m][h];
    }
    __syncthreads();
    const int nspans = s_hi - s_lo + 1;
    const int h = t / kPvCols, e = cb * kPvCols + t % kPvCols;
    const bool owner = t < G * kPvCols && e < d;
    float o = 0.0f;
    if (owner)
        o = red[(0 * G + h) * kPvCols + t % kPvCols] + red[(1 * G + h) * kPvCols + t % kPvCols] +
            red[(2 * G + h) * kPvCols + t % kPvCols] + red[(3 * G + h) * kPvCols + t % kPvCols];
    if (nspans == 1) {
        if (owner) a.out[obase + h * d + e] = f_to_bf16(o);
        return;
    }
    // several spans: partial sums [row][span][d], the last block of the
    // (sequence, KV head, columns) adds them in span order
    float* part = a.partial + (row0 + h) * (int64_t)a.chunks * d;
    if (owner) __hip_atomic_store(&part[(int64_t)sp * d + e], o, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    int* counter = &a.counters[(int64_t)kvb * gridDim.y + cb];
    if (t == 0) {
        const int old = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        flag = old == nspans - 1;
    }
    __syncthreads();
    if (!flag) return;
    if (owner) {
        float sum = 0.0f;
        for (int ss = s_lo; ss <= s_hi; ++ss)
            sum += __hip_atomic_load(&part[(int64_t)ss * d + e], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        a.out[obase + h * d + e] = f_to_bf16(sum);
    }
    if (t == 0) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------
// gelu(tanh) x up
// ---------------------------------------------------------------------------

template <int DT>
__global__ void gelu_mul_kernel(const void* gate, const void* up, int64_t stride, uint16_t* out, int rows, int cols) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)rows * cols) return;
    const int64_t r = i / cols, c = i - r * cols;
    out[i] = gelu_mul_bf16(load_as_bf16<DT>(gate, r * stride + c), load_as_bf16<DT>(up, r * stride + c));
}

// ---------------------------------------------------------------------------
// logits: blocks over vocabulary slices of kArgmaxPer x 256 logits per row
// ---------------------------------------------------------------------------

constexpr int kArgmaxThreads = 256;
constexpr int kArgmaxPer = 8;
constexpr int kArgmaxSlice = kArgmaxThreads * kArgmaxPer;

struct ArgmaxArgs {
    const void* logits;
    int64_t stride;
    int vocab;
    float softcap;
    uint16_t* logits_out;   // [rows, vocab] or NULL
    int64_t* ids;
    int64_t* tokens;
    int64_t token_stride;
    int64_t* step;          // read only unless pos is set
    int64_t* pos;           // NULL, or advance pos and step once every row's pick is stored
    float* part_v;          // [rows, blocks]
    int* part_i;            // [rows, blocks]
    int* counters;          // [rows + 1]: per-row block arrivals, then row arrivals; zero between launches
};

template <int DT>
__global__ __launch_bounds__(kArgmaxThreads) void logits_argmax_kernel(ArgmaxArgs a) {
    __shared__ float wv[kArgmaxThreads / 64];
    __shared__ int wi[kArgmaxThreads / 64];
    __shared__ int flag;
    const int r = blockIdx.y, blk = blockIdx.x, nblk = gridDim.x;
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const int s0 = blk * kArgmaxSlice;
    float z[kArgmaxPer];
#pragma unroll
    for (int k = 0; k < kArgmaxPer; ++k) {
        const int i = s0 + t + k * kArgmaxThreads;
        z[k] = load_as_bf16<DT>(a.logits, (int64_t)r * a.stride + (i < a.vocab ? i : a.vocab - 1));
    }
    float bv = -INFINITY;
    int bi = 0x7FFFFFFF;
#pragma unroll
    for (int k = 0; k < kArgmaxPer; ++k) {
        const int i = s0 + t + k * kArgmaxThreads;
        float v = z[k];
        if (a.softcap > 0.0f) v = round_bf16(round_bf16(tanhf(round_bf16(v / a.softcap))) * a.softcap);
        if (i < a.vocab) {
            if (a.logits_out) a.logits_out[(int64_t)r * a.vocab + i] = f_to_bf16(v);
            keep_first_max(bv, bi, v, i);
        }
    }
    for (int o = 32; o > 0; o >>= 1) keep_first_max(bv, bi, __shfl_xor(bv, o, 64), __shfl_xor(bi, o, 64));
    if (lane == 0) {
        wv[w] = bv;
        wi[w] = bi;
    }
    __syncthreads();
    if (t == 0) {
        for (int k = 1; k < kArgmaxThreads / 64; ++k) keep_first_max(bv, bi, wv[k], wi[k]);
        if (nblk > 1) {
            __hip_atomic_store(&a.part_v[(int64_t)r * nblk + blk], bv, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(&a.part_i[(int64_t)r * nblk + blk], bi, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            const int old = __hip_atomic_fetch_add(&a.counters[r], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            flag = old == nblk - 1;
        } else {
            flag = 1;
        }
    }
    __syncthreads();
    if (!flag) return;
    if (nblk > 1) {
        bv = -INFINITY;
        bi = 0x7FFFFFFF;
        for (int k = t; k < nblk; k += kArgmaxThreads)
            keep_first_max(bv, bi,
                           __hip_atomic_load(&a.part_v[(int64_t)r * nblk + k], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT),
                           __hip_atomic_load(&a.part_i[(int64_t)r * nblk + k], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
        for (int o = 32; o > 0; o >>= 1) keep_first_max(bv, bi, __shfl_xor(bv, o, 64), __shfl_xor(bi, o, 64));
        __syncthreads();
        if (lane == 0) {
            wv[w] = bv;
            wi[w] = bi;
        }
        __syncthreads();
        if (t == 0)
            for (int k = 1; k < kArgmaxThreads / 64; ++k) keep_first_max(bv, bi, wv[k], wi[k]);
    }
    if (t == 0) {
        a.ids[r] = bi;
        const int64_t st = *a.step;
        if (st >= 0 && st < a.token_stride) a.tokens[(int64_t)r * a.token_stride + st] = bi;
        if (nblk > 1) __hip_atomic_store(&a.counters[r], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (a.pos) {
            // every row has read the step before the last row's block moves
            // it: a row arrives only once its step load has returned (the
            // wait is also a compiler barrier)
            bool last = true;
            const int rows = (int)gridDim.y;
            if (rows > 1) {
                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
                last = __hip_atomic_fetch_add(&a.counters[rows], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == rows - 1;
            }
            if (last) {
                if (rows > 1) __hip_atomic_store(&a.counters[rows], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                *a.pos += 1;
                *a.step = st + 1;
            }
        }
    }
}

__global__ void advance_kernel(int64_t* pos, int64_t* step) {
    if (threadIdx.x == 0) {
        *pos += 1;
        *step += 1;
    }
}

}  // namespace se12step

using namespace se12step;

namespace {

thread_local char g_step_err[256] = "";

int step_fail(const char* msg) {
    snprintf(g_step_err, sizeof g_step_err, "%s", msg);
    return SE12_STEP_E_INVALID;
}

int step_fail(const char* who, const char* msg) {
    snprintf(g_step_err, sizeof g_step_err, "%s: %s", who, msg);
    return SE12_STEP_E_INVALID;
}

int step_launched() {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        snprintf(g_step_err, sizeof g_step_err, "launch: %s", hipGetErrorString(e));
        return SE12_STEP_E_HIP;
    }
    return SE12_STEP_OK;
}

bool dtype_ok(int32_t d) { return d == SE12_STEP_F32 || d == SE12_STEP_BF16; }

bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

int64_t up256(int64_t x) { return (x + 255) & ~(int64_t)255; }

struct AttnLayout {
    int64_t chunks, counters, scores, stats, partial, total;  // byte offsets
};

AttnLayout attn_layout(int32_t batch, int32_t heads, int32_t kv_heads, int32_t head_dim, int32_t max_len) {
    AttnLayout l;
    l.chunks = (max_len + kChunk - 1) / kChunk;
    l.counters = 0;
    l.scores = up256((int64_t)batch * kv_heads * (kMaxHeadDim / kPvCols) * sizeof(int));
    l.stats = l.scores + up256((int64_t)batch * heads * l.chunks * kChunk * sizeof(float));
    l.partial = l.stats + up256((int64_t)batch * heads * l.chunks * 2 * sizeof(float));
    l.total = l.partial + up256((int64_t)batch * heads * l.chunks * head_dim * sizeof(float));
    return l;
}

bool attn_shape_ok(int32_t batch, int32_t heads, int32_t kv_heads, int32_t head_dim, int32_t max_len) {
    if (batch <= 0 || kv_heads <= 0 || heads <= 0 || heads % kv_heads != 0 || head_dim < 8 ||
        head_dim > kMaxHeadDim || head_dim % 8 || max_len < 8 || max_len % 8 || (max_len + kChunk - 1) / kChunk > 65535)
        return false;
    const int g = heads / kv_heads;
    return g == 1 || g == 2 || g == 4 || g == 8;
}

template <int G>
void launch_attention(const AttnArgs& a, int blocks_x, hipStream_t stream) {
    const dim3 grid(blocks_x, a.chunks);
    const int32_t qs = (int32_t)a.q_stride, kvs = (int32_t)a.kv_stride;
    if (a.dtype == SE12_STEP_F32)
        hipLaunchKernelGGL((attn_scores_kernel<G, SE12_STEP_F32>), grid, dim3(kAttnThreads), 0, stream, a.pos, a.q, a.k, a.kt,
                           a.d, a.max_len, a.kvh, qs, kvs, a);
    else
        hipLaunchKernelGGL((attn_scores_kernel<G, SE12_STEP_BF16>), grid, dim3(kAttnThreads), 0, stream, a.pos, a.q, a.k,
                           a.kt, a.d, a.max_len, a.kvh, qs, kvs, a);
    const dim3 pv_grid(blocks_x, (a.d + kPvCols - 1) / kPvCols, (a.max_len + pv_span<G>() - 1) / pv_span<G>());
    hipLaunchKernelGGL(attn_pv_kernel<G>, pv_grid, dim3(kAttnThreads), 0, stream, a.pos, a.stats, a.scores, a.vc, a.d,
                       a.max_len, a.kvh, a.chunks, a);
}

struct ArgmaxLayout {
    int64_t blocks, counters, part_v, part_i, total;
};

ArgmaxLayout argmax_layout(int32_t rows, int32_t vocab) {
    ArgmaxLayout l;
    l.blocks = (vocab + kArgmaxSlice - 1) / kArgmaxSlice;
    l.counters = 0;
    l.part_v = up256((int64_t)(rows + 1) * sizeof(int));
    l.part_i = l.part_v + up256((int64_t)rows * l.blocks * sizeof(float));
    l.total = l.part_i + up256((int64_t)rows * l.blocks * sizeof(int));
    return l;
}

}  // namespace

extern "C" {

const char* se12_step_last_error(void) { return g_step_err; }

int se12_step_rmsnorm(const void* in, int32_t in_dtype, int64_t in_stride, const uint16_t* w1, uint16_t* residual,
                      const uint16_t* w2, uint16_t* out, int32_t rows, int32_t hidden, float eps, float in_scale,
                      int32_t mode, void* stream) {
    if (!in || !w1 || !out || rows <= 0 || hidden <= 0 || !dtype_ok(in_dtype) || in_stride < hidden)
        return step_fail("se12_step_rmsnorm: bad argument");
    if (mode == 1 && (!residual || !w2)) return step_fail("se12_step_rmsnorm: mode 1 needs residual and w2");
    if (mode != 0 && mode != 1) return step_fail("se12_step_rmsnorm: mode must be 0 or 1");
    if (hidden > kNormPer * kNormMaxThreads) return step_fail("se12_step_rmsnorm: hidden above 8192");
    NormArgs a{in, in_stride, w1, residual, w2, out, hidden, eps, in_scale};
    const int threads = ((hidden + kNormPer - 1) / kNormPer + 63) / 64 * 64;
    const hipStream_t st = static_cast<hipStream_t>(stream);
    const bool f32 = in_dtype == SE12_STEP_F32;
    if (mode == 0) {
        if (f32)
            hipLaunchKernelGGL((rmsnorm_kernel<SE12_STEP_F32, 0>), dim3(rows), dim3(threads), 0, st, a);
        else
            hipLaunchKernelGGL((rmsnorm_kernel<SE12_STEP_BF16, 0>), dim3(rows), dim3(threads), 0, st, a);
    } else {
        if (f32)
            hipLaunchKernelGGL((rmsnorm_kernel<SE12_STEP_F32, 1>), dim3(rows), dim3(threads), 0, st, a);
        else
            hipLaunchKernelGGL((rmsnorm_kernel<SE12_STEP_BF16, 1>), dim3(rows), dim3(threads), 0, st, a);
    }
    return step_launched();
}

int64_t se12_step_attention_workspace(int32_t batch, int32_t heads, int32_t kv_heads, int32_t head_dim,
                                      int32_t max_len) {
    if (!attn_shape_ok(batch, heads, kv_heads, head_dim, max_len)) {
        step_fail("se12_step_attention_workspace: bad shape");
        return SE12_STEP_E_INVALID;
    }
    return attn_layout(batch, heads, kv_heads, head_dim, max_len).total;
}

int se12_step_attention(const void* q, const void* k, const void* v, int32_t dtype, int64_t q_stride, int64_t kv_stride,
                        uint16_t* k_cache_t, uint16_t* v_cache, const float* inv_freq, const int64_t* pos, uint16_t* out,
                        int32_t batch, int32_t heads, int32_t kv_heads, int32_t head_dim, int32_t max_len, float scaling,
                        float softcap, int32_t window, void* workspace, int64_t workspace_bytes, void* stream) {
    if (!q || !k || !v || !k_cache_t || !v_cache || !inv_freq || !pos || !out || !workspace || !dtype_ok(dtype))
        return step_fail("se12_step_attention: NULL argument or bad dtype");
    if (!attn_shape_ok(batch, heads, kv_heads, head_dim, max_len) || q_stride < (int64_t)heads * head_dim ||
        kv_stride < (int64_t)kv_heads * head_dim || q_stride > INT32_MAX || kv_stride > INT32_MAX)
        return step_fail("se12_step_attention: bad shape");
    if (!aligned16(k_cache_t) || !aligned16(v_cache)) return step_fail("se12_step_attention: caches not 16-byte aligned");
    const AttnLayout l = attn_layout(batch, heads, kv_heads, head_dim, max_len);
    if (workspace_bytes < l.total) return step_fail("se12_step_attention: workspace too small");
    if (reinterpret_cast<uintptr_t>(workspace) % 256) return step_fail("se12_step_attention: workspace not 256-byte aligned");
    char* ws = static_cast<char*>(workspace);
    AttnArgs a;
    a.q = q;
    a.k = k;
    a.v = v;
    a.dtype = dtype;
    a.q_stride = q_stride;
    a.kv_stride = kv_stride;
    a.kt = k_cache_t;
    a.vc = v_cache;
    a.inv_freq = inv_freq;
    a.pos = pos;
    a.out = out;
    a.counters = reinterpret_cast<int*>(ws + l.counters);
    a.scores = reinterpret_cast<float*>(ws + l.scores);
    a.stats = reinterpret_cast<float*>(ws + l.stats);
    a.partial = reinterpret_cast<float*>(ws + l.partial);
    a.heads = heads;
    a.kvh = kv_heads;
    a.d = head_dim;
    a.max_len = max_len;
    a.chunks = (int)l.chunks;
    a.scaling = scaling;
    a.softcap = softcap;
    a.window = window;
    const hipStream_t st = static_cast<hipStream_t>(stream);
    switch (heads / kv_heads) {
        case 1: launch_attention<1>(a, batch * kv_heads, st); break;
        case 2: launch_attention<2>(a, batch * kv_heads, st); break;
        case 4: launch_attention<4>(a, batch * kv_heads, st); break;
        default: launch_attention<8>(a, batch * kv_heads, st); break;
    }
    return step_launched();
}

int se12_step_gelu_mul(const void* gate, const void* up, int32_t dtype, int64_t stride, uint16_t* out, int32_t rows,
                       int32_t cols, void* stream) {
    if (!gate || !up || !out || rows <= 0 || cols <= 0 || stride < cols || !dtype_ok(dtype))
        return step_fail("se12_step_gelu_mul: bad argument");
    const int64_t n = (int64_t)rows * cols;
    const dim3 grid((unsigned)((n + 255) / 256));
    const hipStream_t st = static_cast<hipStream_t>(stream);
    if (dtype == SE12_STEP_F32)
        hipLaunchKernelGGL(gelu_mul_kernel<SE12_STEP_F32>, grid, dim3(256), 0, st, gate, up, stride, out, rows, cols);
    else
        hipLaunchKernelGGL(gelu_mul_kernel<SE12_STEP_BF16>, grid, dim3(256), 0, st, gate, up, stride, out, rows, cols);
    return step_launched();
}

int64_t se12_step_logits_workspace(int32_t rows, int32_t vocab) {
    if (rows <= 0 || vocab <= 0 || rows > 65535) {
        step_fail("se12_step_logits_workspace: bad shape");
        return SE12_STEP_E_INVALID;
    }
    return argmax_layout(rows, vocab).total;
}

}  // extern "C"

namespace {

int launch_argmax(const char* who, const void* logits, int32_t dtype, int64_t stride, int32_t rows, int32_t vocab,
                  float softcap, uint16_t* logits_out, int64_t* ids, int64_t* tokens, int64_t token_stride,
                  int64_t* step, int64_t* pos, void* workspace, int64_t workspace_bytes, void* stream) {
    if (!logits || !ids || !tokens || !step || !workspace || rows <= 0 || rows > 65535 || vocab <= 0 || stride < vocab ||
        !dtype_ok(dtype))
        return step_fail(who, "bad argument");
    const ArgmaxLayout l = argmax_layout(rows, vocab);
    if (workspace_bytes < l.total) return step_fail(who, "workspace too small");
    if (reinterpret_cast<uintptr_t>(workspace) % 256) return step_fail(who, "workspace not 256-byte aligned");
    char* ws = static_cast<char*>(workspace);
    ArgmaxArgs a{logits, stride, vocab, softcap, logits_out, ids, tokens, token_stride, step, pos,
                 reinterpret_cast<float*>(ws + l.part_v), reinterpret_cast<int*>(ws + l.part_i),
                 reinterpret_cast<int*>(ws + l.counters)};
    const dim3 grid((unsigned)l.blocks, rows);
    const hipStream_t st = static_cast<hipStream_t>(stream);
    if (dtype == SE12_STEP_F32)
        hipLaunchKernelGGL(logits_argmax_kernel<SE12_STEP_F32>, grid, dim3(kArgmaxThreads), 0, st, a);
    else
        hipLaunchKernelGGL(logits_argmax_kernel<SE12_STEP_BF16>, grid, dim3(kArgmaxThreads), 0, st, a);
    return step_launched();
}

}  // namespace

extern "C" {

int se12_step_logits_argmax(const void* logits, int32_t dtype, int64_t stride, int32_t rows, int32_t vocab, float softcap,
                            uint16_t* logits_out, int64_t* ids, int64_t* tokens, int64_t token_stride,
                            const int64_t* step, void* workspace, int64_t workspace_bytes, void* stream) {
    // the kernel writes the step only when it is given pos
    return launch_argmax("se12_step_logits_argmax", logits, dtype, stride, rows, vocab, softcap, logits_out, ids, tokens,
                         token_stride, const_cast<int64_t*>(step), nullptr, workspace, workspace_bytes, stream);
}

int se12_step_logits_argmax_advance(const void* logits, int32_t dtype, int64_t stride, int32_t rows, int32_t vocab,
                                    float softcap, uint16_t* logits_out, int64_t* ids, int64_t* tokens,
                                    int64_t token_stride, int64_t* step, int64_t* pos, void* workspace,
                                    int64_t workspace_bytes, void* stream) {
    if (!pos) return step_fail("se12_step_logits_argmax_advance: NULL pos");
    return launch_argmax("se12_step_logits_argmax_advance", logits, dtype, stride, rows, vocab, softcap, logits_out, ids,
                         tokens, token_stride, step, pos, workspace, workspace_bytes, stream);
}

int se12_step_advance(int64_t* pos, int64_t* step, void* stream) {
    if (!pos || !step) return step_fail("se12_step_advance: NULL argument");
    hipLaunchKernelGGL(advance_kernel, dim3(1), dim3(64), 0, static_cast<hipStream_t>(stream), pos, step);
    return step_launched();
}

}  // extern "C"
