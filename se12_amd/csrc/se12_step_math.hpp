// Device helpers shared by the decode-step kernels (se12_step.hip) and the
// step work fused into the tail of the GEMV kernels (se12_gemv.hip): BF16
// rounding as the framework's BF16 ops round, the tanh GELU, wave and block
// sums. One definition, so that a fused and a separate launch of the same
// step compute the same values.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace se12step {

__device__ __forceinline__ float bf16_to_f(uint32_t b) { return __uint_as_float(b << 16); }

// float -> BF16 bits, round to nearest even; a NaN keeps its top 16 bits
// with the quiet bit set. gfx950's conversion instruction (v_cvt_pk_bf16_f32)
// gives exactly the bits of the integer form (u + 0x7FFF + lsb) >> 16 (NaN:
// (u >> 16) | 0x40) for every one of the 2^32 inputs, checked on MI355X, in
// one instruction per pair instead of six per value.
__device__ __forceinline__ uint16_t f_to_bf16(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }

// two values at once: a in the low half, b in the high half
__device__ __forceinline__ uint32_t f_to_bf16x2(float a, float b) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    const bf16x2_t v = {(__bf16)a, (__bf16)b};
    return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ float round_bf16(float f) { return bf16_to_f(f_to_bf16(f)); }

// BF16 GELU, tanh form, of a BF16 value: 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3)))
// in FP32, rounded to BF16
__device__ __forceinline__ float gelu_tanh_bf16(float x) {
    const float inner = 0.7978845608028654f * (x + 0.044715f * (x * x * x));
    return round_bf16(0.5f * x * (1.0f + tanhf(inner)));
}

// the decoder's MLP gate: bf16(gelu_tanh(g) * u) for BF16 g and u
__device__ __forceinline__ uint16_t gelu_mul_bf16(float g, float u) { return f_to_bf16(gelu_tanh_bf16(g) * u); }

// Gemma's RMSNorm with a BF16 weight w, in FP32: x * inv * (1 + w), where
// inv = rms_inv(sum of x^2 over the row, row length, eps)
__device__ __forceinline__ float rms_inv(float ss, int n, float eps) { return rsqrtf(ss / (float)n + eps); }
__device__ __forceinline__ float rms_scale(float x, float inv, float w) { return (x * inv) * (1.0f + w); }

// Wave reductions without LDS: DPP within each 16-lane row (every lane of
// the row ends with the same value, fp add being commutative), then the four
// row results read as scalars and combined in row order. (A shuffle-based
// reduction goes through the LDS crossbar: six dependent round trips.)
template <typename Op>
__device__ __forceinline__ float row16_reduce(float v, Op op) {
    v = op(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, true)));   // quad_perm 1,0,3,2
    v = op(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, true)));   // quad_perm 2,3,0,1
    v = op(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x141, 0xF, 0xF, true)));  // row_half_mirror
    v = op(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x140, 0xF, 0xF, true)));  // row_mirror
    return v;
}

template <typename Op>
__device__ __forceinline__ float wave_reduce(float v, Op op) {
    v = row16_reduce(v, op);
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return op(op(r0, r1), op(r2, r3));
}

struct AddOp {
    __device__ float operator()(float a, float b) const { return a + b; }
};
struct MaxOp {
    __device__ float operator()(float a, float b) const { return fmaxf(a, b); }
};

__device__ __forceinline__ float wave_sum(float v) { return wave_reduce(v, AddOp()); }
__device__ __forceinline__ float wave_max(float v) { return wave_reduce(v, MaxOp()); }

// block-wide sum (waves in order); `sh` holds >= 16 floats; every thread
// gets the result
__device__ __forceinline__ float block_sum(float v, float* sh) {
    v = wave_sum(v);
    const int waves = blockDim.x >> 6;
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = v;
    __syncthreads();
    float r = sh[0];
    for (int i = 1; i < waves; ++i) r += sh[i];
    __syncthreads();  // sh is free again
    return r;
}

}  // namespace se12step
