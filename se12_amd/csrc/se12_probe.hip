// Device measurement: a streaming read of a buffer, the read-only traffic a
// weight pass makes, for the roofline's bandwidth. Each thread folds 16-byte
// loads with XOR, 8 in flight per iteration over a grid-stride loop; the
// result is written only when it equals a constant no buffer of ones or
// zeros produces, so the stores practically never happen but the loads
// cannot be removed.
#include <hip/hip_runtime.h>

#include "se12_internal.hpp"

namespace {

// 8 loads in flight per thread, nontemporal (each line is read once), 2
// blocks of 512 threads per CU: the fastest of the grid-stride forms
// measured on MI355X over 1 GiB buffers (6.09 TB/s, against 5.28-5.80 with
// plain loads and 5.5-6.0 with other unrolls and block counts).
constexpr int kProbeUnroll = 8;
constexpr int kProbeThreads = 512;
constexpr int kProbeBlocksPerCu = 2;

__global__ __launch_bounds__(kProbeThreads) void read_probe_kernel(const uint4* __restrict__ p, int64_t n16,
                                                                   uint32_t* __restrict__ out) {
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    const u32x4* q = reinterpret_cast<const u32x4*>(p);
    uint32_t acc = 0;
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (; i + (kProbeUnroll - 1) * stride < n16; i += kProbeUnroll * stride) {
        u32x4 v[kProbeUnroll];
#pragma unroll
        for (int u = 0; u < kProbeUnroll; ++u) v[u] = __builtin_nontemporal_load(q + i + u * stride);
#pragma unroll
        for (int u = 0; u < kProbeUnroll; ++u) acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
    }
    for (; i < n16; i += stride) {
        const uint4 v = p[i];
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    if (acc == 0x9E3779B9u) out[blockIdx.x] = acc;
}

}  // namespace

namespace se12 {

int64_t read_probe_blocks(int32_t compute_units) { return (int64_t)(compute_units > 0 ? compute_units : 1) * kProbeBlocksPerCu; }

hipError_t launch_read_probe(const void* buf, int64_t n16, uint32_t* out, int64_t blocks, hipStream_t stream) {
    hipLaunchKernelGGL(read_probe_kernel, dim3((uint32_t)blocks), dim3(kProbeThreads), 0, stream,
                       static_cast<const uint4*>(buf), n16, out);
    return hipGetLastError();
}

}  // namespace se12
