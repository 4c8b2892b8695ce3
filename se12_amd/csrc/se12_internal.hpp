// Kernel argument blocks and launch entry points shared between the kernel
// translation units and the C ABI (se12_abi.hip). Host and device code.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace se12 {

struct GemvArgs {
    const uint8_t* sm;
    const uint8_t* ec;
    const uint8_t* esc;
    const uint8_t* codebook;
    const int32_t* fb_rank;   // per-tile rank among fallback tiles, -1 if not one
    const int16_t* fb_raw;
    const uint16_t* wraw;     // raw twin: row-major [N, K] BF16 bits
    const void* x;            // [B, K] BF16 or FP32
    float* y;                 // [B, N]
    float* partial;           // [S, B, Np] split-K partial sums
    int32_t* counters;        // [TR] arrival counters (zero between launches)
    int64_t N, K, Np;
    int32_t TR, TC;
    int32_t S;                // K splits per tile row
    int32_t xstride;          // LDS elements per batch row of x
    int32_t x_vec_ok;         // x rows allow 16-byte loads
    int32_t w_vec_ok;         // raw rows allow 16-byte loads
    int32_t mask_tail;        // K % 256 != 0 and codebook[0] == 255
};

struct DecodeArgs {
    const uint8_t* sm;
    const uint8_t* ec;
    const uint8_t* esc;
    const uint8_t* codebook;
    const uint8_t* bitmap;
    const int32_t* fb_rank;
    const int16_t* fb_raw;
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
// waves per block the kernel is compiled for: 16 (1024 threads, <= 128 VGPRs)
// for batch 1 with BF16 x, 4 where more accumulators or FP32 x need registers
constexpr int gemv_max_waves(int batch, bool xf32) { return (batch == 1 && !xf32) ? 16 : 4; }
constexpr int kLutBytes = 1024;

// bytes of dynamic LDS a GEMV launch needs
inline size_t gemv_lds_bytes(int waves, int batch, int xstride, bool xf32) {
    return (size_t)kLutBytes + (size_t)waves * batch * 16 * sizeof(float) +
           (size_t)batch * xstride * (xf32 ? 4 : 2);
}

hipError_t launch_gemv(const GemvArgs& a, int batch, bool xf32, bool raw, int threads, int blocks, size_t lds,
                       hipStream_t stream);
hipError_t launch_decode(const DecodeArgs& a, bool rows, hipStream_t stream);
hipError_t launch_fallback_rank_from_bitmap(const uint8_t* bitmap, int64_t T, int32_t* rank, int64_t* total,
                                            hipStream_t stream);
hipError_t launch_encode_histogram(const EncodeArgs& a, hipStream_t stream);
hipError_t launch_encode_count(const EncodeArgs& a, hipStream_t stream);
hipError_t launch_encode_scan(const EncodeArgs& a, hipStream_t stream);
hipError_t launch_encode_write(const EncodeArgs& a, hipStream_t stream);

}  // namespace se12
