// SE12 encoder on the GPU, byte-identical to the reference encoder
// lws/domain/se12/codec.py:111-141 (which runs numpy on the host at pack time,
// lws/application/codec/pack_model.py:113-120). Four kernels:
//   histogram  - 256-bin exponent histogram over the real weights
//                (the host then picks the codebook, codebook.py:41-59)
//   count      - escapes per tile (weights whose exponent is not in the
//                codebook; padding never escapes, codec.py:119-125)
//   scan       - fallback flag (count > 16, codec.py:132-133), rank among
//                fallback tiles, MSB-first bitmap (codec.py:351-353)
//   write      - sm / ec / esc / fallback_raw, one wave per tile with the same
//                lane mapping as the decoder: escapes take slots in tile-local
//                row-major order (codec.py:131,332-343); fallback tiles keep
//                their padded bits raw (codec.py:363-365) and zero esc slots.
#include "se12_device.hpp"
#include "se12_internal.hpp"

namespace se12 {

constexpr int kEncWaves = 4;
constexpr int kHistThreads = 256;

__device__ __forceinline__ uint32_t cb_byte(const EncodeArgs& a, int i) {
    return (a.codebook[i >> 2] >> (8 * (i & 3))) & 0xFFu;
}

// code of each exponent value (15 = escape)
__device__ __forceinline__ void build_code_lut(uint8_t* code_of, const EncodeArgs& a, int tid, int nthreads) {
    for (int e = tid; e < 256; e += nthreads) {
        uint32_t c = 15;
        for (int i = kCodebook - 1; i >= 0; --i)
            if (cb_byte(a, i) == (uint32_t)e) c = i;
        code_of[e] = (uint8_t)c;
    }
}

__global__ __launch_bounds__(kHistThreads) void encode_histogram_kernel(EncodeArgs a) {
    __shared__ uint32_t hist[256];
    for (int i = threadIdx.x; i < 256; i += blockDim.x) hist[i] = 0;
    __syncthreads();
    const int64_t total = a.N * a.K;
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (int64_t)gridDim.x * blockDim.x) {
        const int64_t row = idx / a.K;
        const int64_t col = idx - row * a.K;
        const uint32_t v = a.w[row * a.ld + col];
        atomicAdd(&hist[(v >> 7) & 0xFFu], 1u);
    }
    __syncthreads();
    for (int i = threadIdx.x; i < 256; i += blockDim.x)
        if (hist[i]) atomicAdd(reinterpret_cast<unsigned long long*>(&a.histogram[i]), (unsigned long long)hist[i]);
}

// the lane's 16 weights of chunk j (zero outside the matrix = padding)
__device__ __forceinline__ void load_weights16(const EncodeArgs& a, int64_t row, int64_t col, uint32_t v[8]) {
    const uint16_t* p = a.w + row * a.ld + col;
    if (a.w_vec_ok && row < a.N && col + 16 <= a.K) {
        uint4 u0 = reinterpret_cast<const uint4*>(p)[0];
        uint4 u1 = reinterpret_cast<const uint4*>(p)[1];
        v[0] = u0.x; v[1] = u0.y; v[2] = u0.z; v[3] = u0.w;
        v[4] = u1.x; v[5] = u1.y; v[6] = u1.z; v[7] = u1.w;
    } else {
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            uint32_t lo = (row < a.N && col + 2 * q < a.K) ? (uint32_t)p[2 * q] : 0u;
            uint32_t hi = (row < a.N && col + 2 * q + 1 < a.K) ? (uint32_t)p[2 * q + 1] : 0u;
            v[q] = lo | (hi << 16);
        }
    }
}

// codes of the chunk (padding -> 0) and the escape mask (bit i = weight i)
__device__ __forceinline__ void chunk_codes(const EncodeArgs& a, const uint8_t* code_of, int64_t row, int64_t col,
                                            const uint32_t v[8], uint32_t codes[16], uint32_t& escmask) {
    escmask = 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const uint32_t bits = (v[i >> 1] >> (16 * (i & 1))) & 0xFFFFu;
        const bool valid = row < a.N && col + i < a.K;
        const uint32_t c = valid ? (uint32_t)code_of[(bits >> 7) & 0xFFu] : 0u;
        codes[i] = c;
        if (c == 15u) escmask |= 1u << i;
    }
}

__global__ __launch_bounds__(kEncWaves * kWave) void encode_count_kernel(EncodeArgs a) {
    __shared__ uint8_t code_of[256];
    const int tid = threadIdx.x;
    const uint32_t lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    build_code_lut(code_of, a, tid, blockDim.x);
    __syncthreads();
    const int64_t tile = (int64_t)blockIdx.x * kEncWaves + w;
    if (tile >= a.T) return;
    const int tr = (int)(tile / a.TC);
    const int kt = (int)(tile - (int64_t)tr * a.TC);
    const int64_t col = (int64_t)kt * kTileCols + 16 * (lane & 15u);
    uint32_t count = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int64_t row = (int64_t)tr * kTileRows + 4 * j + (lane >> 4);
        uint32_t v[8], codes[16], m;
        load_weights16(a, row, col, v);
        chunk_codes(a, code_of, row, col, v, codes, m);
        count += __popc(m);
    }
    const uint32_t total = __builtin_amdgcn_readlane(wave_incl_scan(count), kWave - 1);
    if (lane == 0) a.tile_escapes[tile] = (int32_t)total;
}

constexpr int kScanThreads = 1024;

__global__ __launch_bounds__(kScanThreads) void encode_scan_kernel(EncodeArgs a) {
    __shared__ int64_t tmp[kScanThreads];
    const int tid = threadIdx.x;
    int64_t chunk = (a.T + kScanThreads - 1) / kScanThreads;
    chunk = (chunk + 7) & ~int64_t(7);
    const int64_t t0 = (int64_t)tid * chunk;
    const int64_t t1 = t0 + chunk < a.T ? t0 + chunk : a.T;
    int64_t count = 0;
    for (int64_t t = t0; t < t1; ++t) count += a.tile_escapes[t] > kEscBudget ? 1 : 0;
    tmp[tid] = count;
    __syncthreads();
    for (int d = 1; d < kScanThreads; d <<= 1) {
        int64_t u = tid >= d ? tmp[tid - d] : 0;
        __syncthreads();
        tmp[tid] += u;
        __syncthreads();
    }
    int64_t base = tmp[tid] - count;
    for (int64_t t = t0; t < t1; t += 8) {
        uint32_t byte = 0;
        for (int i = 0; i < 8 && t + i < t1; ++i) {
            const bool fb = a.tile_escapes[t + i] > kEscBudget;
            a.fb_rank[t + i] = (int32_t)base;
            base += fb ? 1 : 0;
            byte |= (fb ? 1u : 0u) << (7 - i);
        }
        a.bitmap[t >> 3] = (uint8_t)byte;
    }
    if (tid == kScanThreads - 1) a.totals[0] = tmp[kScanThreads - 1];
}

__global__ __launch_bounds__(kEncWaves * kWave) void encode_write_kernel(EncodeArgs a) {
    __shared__ uint8_t code_of[256];
    __shared__ uint8_t esc_buf[kEncWaves][kEscBudget];
    const int tid = threadIdx.x;
    const uint32_t lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    build_code_lut(code_of, a, tid, blockDim.x);
    __syncthreads();
    const int64_t tile = (int64_t)blockIdx.x * kEncWaves + w;
    if (tile >= a.T) return;
    const int tr = (int)(tile / a.TC);
    const int kt = (int)(tile - (int64_t)tr * a.TC);
    const int64_t col = (int64_t)kt * kTileCols + 16 * (lane & 15u);

    uint32_t v[4][8];
    uint32_t escm[4];
    uint32_t cnt[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int64_t row = (int64_t)tr * kTileRows + 4 * j + (lane >> 4);
        uint32_t codes[16];
        load_weights16(a, row, col, v[j]);
        chunk_codes(a, code_of, row, col, v[j], codes, escm[j]);
        cnt[j] = __popc(escm[j]);
        // sm bytes: ((b >> 8) & 0x80) | (b & 0x7F) for each weight
        uint32_t smw[4];
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            uint32_t word = 0;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int i = 4 * d + k;
                const uint32_t bits = (v[j][i >> 1] >> (16 * (i & 1))) & 0xFFFFu;
                word |= (((bits >> 8) & 0x80u) | (bits & 0x7Fu)) << (8 * k);
            }
            smw[d] = word;
        }
        uint32_t ecw[2] = {0u, 0u};
#pragma unroll
        for (int q = 0; q < 8; ++q) ecw[q >> 2] |= (codes[2 * q] | (codes[2 * q + 1] << 4)) << (8 * (q & 3));
        *reinterpret_cast<uint4*>(a.sm + tile * kTile + 1024 * j + 16 * lane) = make_uint4(smw[0], smw[1], smw[2], smw[3]);
        *reinterpret_cast<uint2*>(a.ec + tile * (kTile / 2) + 512 * j + 8 * lane) = make_uint2(ecw[0], ecw[1]);
    }

    // escape ranks: chunk j, then lane, then position (tile-local row-major)
    const uint32_t s01 = wave_incl_scan(cnt[0] | (cnt[1] << 16));
    const uint32_t s23 = wave_incl_scan(cnt[2] | (cnt[3] << 16));
    const uint32_t t01 = __builtin_amdgcn_readlane(s01, kWave - 1);
    const uint32_t t23 = __builtin_amdgcn_readlane(s23, kWave - 1);
    const uint32_t tot[4] = {t01 & 0xFFFFu, t01 >> 16, t23 & 0xFFFFu, t23 >> 16};
    const uint32_t incl[4] = {s01 & 0xFFFFu, s01 >> 16, s23 & 0xFFFFu, s23 >> 16};
    const uint32_t total = tot[0] + tot[1] + tot[2] + tot[3];
    uint8_t* esc_out = a.esc + tile * kEscBudget;

    if (total <= (uint32_t)kEscBudget) {
        uint32_t run = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            uint32_t r = run + incl[j] - cnt[j];
            uint32_t m = escm[j];
            while (m) {
                const int i = __builtin_ctz(m);
                m &= m - 1u;
                const uint32_t bits = (v[j][i >> 1] >> (16 * (i & 1))) & 0xFFFFu;
                esc_buf[w][r] = (uint8_t)((bits >> 7) & 0xFFu);
                ++r;
            }
            run += tot[j];
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        if (lane < (uint32_t)kEscBudget) esc_out[lane] = lane < total ? esc_buf[w][lane] : (uint8_t)0;
    } else {
        if (lane < (uint32_t)kEscBudget) esc_out[lane] = 0;
        int16_t* raw = a.raw + (int64_t)a.fb_rank[tile] * kTile;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            uint4* p = reinterpret_cast<uint4*>(raw + 1024 * j + 16 * lane);
            p[0] = make_uint4(v[j][0], v[j][1], v[j][2], v[j][3]);
            p[1] = make_uint4(v[j][4], v[j][5], v[j][6], v[j][7]);
        }
    }
}

hipError_t launch_encode_histogram(const EncodeArgs& a, hipStream_t stream) {
    int64_t total = a.N * a.K;
    int64_t blocks = (total + kHistThreads * 16 - 1) / (kHistThreads * 16);
    if (blocks < 1) blocks = 1;
    if (blocks > 4096) blocks = 4096;
    hipLaunchKernelGGL(encode_histogram_kernel, dim3((uint32_t)blocks), dim3(kHistThreads), 0, stream, a);
    return hipGetLastError();
}

hipError_t launch_encode_count(const EncodeArgs& a, hipStream_t stream) {
    const int64_t blocks = (a.T + kEncWaves - 1) / kEncWaves;
    hipLaunchKernelGGL(encode_count_kernel, dim3((uint32_t)blocks), dim3(kEncWaves * kWave), 0, stream, a);
    return hipGetLastError();
}

hipError_t launch_encode_scan(const EncodeArgs& a, hipStream_t stream) {
    hipLaunchKernelGGL(encode_scan_kernel, dim3(1), dim3(kScanThreads), 0, stream, a);
    return hipGetLastError();
}

hipError_t launch_encode_write(const EncodeArgs& a, hipStream_t stream) {
    const int64_t blocks = (a.T + kEncWaves - 1) / kEncWaves;
    hipLaunchKernelGGL(encode_write_kernel, dim3((uint32_t)blocks), dim3(kEncWaves * kWave), 0, stream, a);
    return hipGetLastError();
}

}  // namespace se12
