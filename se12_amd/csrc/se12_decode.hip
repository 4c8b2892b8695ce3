// Decode-only kernels: SE12 streams -> row-major BF16 bits, bit-exact with the
// reference decoder (lws/domain/se12/codec.py:144-186). A wave decodes a
// 16x256 tile with the same per-lane routine as the fused GEMV and writes its
// rows straight to the cropped [rows, cols] output (the whole-matrix decode
// streams several tiles per wave; the row decode takes one (row, K tile) per
// wave), replacing the reference's
// one-thread-per-tile kernel plus device untile/crop
// (lws/adapters/cuda/kernels/se12_decode.cu:12-43,
// lws/adapters/cuda/se12_decoder.py:147-185).
//
// Also here: the bind-time per-tile sidecar word. For a fallback tile it holds
// the tile's rank among all fallback tiles (cumsum(bitmap bits) - 1, as in
// lws/adapters/cuda/gemv.py:47-53, computed by a single-block scan); for any
// other tile, which of its four 4-row chunks hold escape codes (one wave per
// tile reads the tile's `ec` bytes). The kernels read it instead of the bitmap.
#include "se12_device.hpp"
#include "se12_internal.hpp"

namespace se12 {

constexpr int kDecodeWaves = 4;

__device__ __forceinline__ void store16(uint16_t* out_row, int64_t col, int64_t K, bool vec_ok, const uint32_t w[8]) {
    if (vec_ok && col + 16 <= K) {
        reinterpret_cast<uint4*>(out_row + col)[0] = make_uint4(w[0], w[1], w[2], w[3]);
        reinterpret_cast<uint4*>(out_row + col)[1] = make_uint4(w[4], w[5], w[6], w[7]);
    } else {
#pragma unroll
        for (int i = 0; i < 16; ++i)
            if (col + i < K) out_row[col + i] = (uint16_t)(w[i >> 1] >> (16 * (i & 1)));
    }
}

// Decodes a loaded tile for this lane; calls sink(j, w) for each chunk j.
template <typename Sink>
__device__ __forceinline__ void decode_loaded(const DecodeArgs& a, const uint32_t* lut, const TileSide& side,
                                              const TileLoads& t, uint32_t lane, Sink&& sink) {
    const uint32_t info = side_info(side, 0);
    if (info_is_fallback(info)) {
        const int16_t* raw = raw_tile_ptr(info, a.fb_raw, a.ovf_raw);
        uint32_t w[4][8];
#pragma unroll
        for (int j = 0; j < 4; ++j) load_raw_chunk(raw, j, lane, w[j]);
        wait_vector_loads();  // rare path: keeps the common path's waits exact
#pragma unroll
        for (int j = 0; j < 4; ++j) sink(j, w[j]);
    } else {
        uint32_t pat[4][8];
        lookup_tile(lut, t, pat);
        patch_tile_escapes(pat, info, side, 0, lane);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            uint32_t w[8];
            merge_chunk(pat[j], t.sm[j], w);
            sink(j, w);
        }
    }
}

// Loads and decodes tile `tile` for this lane; calls sink(j, w) for each chunk j.
template <typename Sink>
__device__ __forceinline__ void decode_tile(const DecodeArgs& a, const uint32_t* lut, int64_t tile, uint32_t lane,
                                            Sink&& sink) {
    TileSide side;
    TileLoads t;
    load_side(side, a.side, tile, lane);
    load_tile(t, a.sm, a.ec, tile, lane);
    decode_loaded(a, lut, side, t, lane, sink);
}

// 8 decoded weights (4 BF16 pairs) to out_row[col .. col + 8) clipped at K:
// one 16-byte nontemporal store when the output allows it (streamed: the
// decoded matrix is written once and read later by another kernel).
__device__ __forceinline__ void store8(uint16_t* out_row, int64_t col, int64_t K, bool vec_ok, const uint32_t w[4]) {
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    if (vec_ok && col + 8 <= K) {
        const u32x4 v = {w[0], w[1], w[2], w[3]};
        __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(out_row + col));
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i)
            if (col + i < K) out_row[col + i] = (uint16_t)(w[i >> 1] >> (16 * (i & 1)));
    }
}

// Whole-matrix decode: nw waves stream the tiles, wave g taking tiles g,
// g + nw, ... (the waves read a moving window of the tile-major streams),
// each with the next tile's loads in flight while it decodes and stores the
// current one. The last tile loads nothing after it (a wave cannot end
// before its loads land), and every load inside the loop is issued on every
// path, so the compiler's wait counts stay exact.
//
// Lane layout (the half layout): part p = 0..7 of a tile covers tile rows
// 2p and 2p + 1; lane l takes row 2p + l / 32, columns 8 (l % 32) .. + 7
// (8 bytes of sm, 4 of ec), so each part's store instruction writes two
// whole 512-byte row segments, 16 contiguous bytes per lane. (The fused
// kernels' chunk layout gives each lane 16 columns, whose two 16-byte stores
// each write alternate halves of 32-byte pieces: 2304x9216 took 19.0 us
// with it against 15.7 here, the stores nontemporal in both; 14336x3584
// 39.0 against 33.5.)
__global__ __launch_bounds__(kDecodeWaves * kWave) void decode_stream_kernel(DecodeArgs a, int64_t nw) {
    SE12_DECLARE_LUT(lut);
    const int tid = threadIdx.x;
    const uint32_t lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    // tile indices in 32 bits (the library refuses matrices of 2^31 tiles or
    // more), so the per-tile division is a 32-bit one
    const uint32_t T = (uint32_t)a.T, NW = (uint32_t)nw, TC = (uint32_t)a.TC;
    const uint32_t g = blockIdx.x * kDecodeWaves + (uint32_t)w;
    const uint32_t n = g < NW && g < T ? (T - 1u - g) / NW + 1u : 0u;  // tiles of this wave
    struct Slot {
        TileSide side;
        HalfTileLoads t;
    };
    auto load = [&](Slot& sl, uint32_t i) {
        const uint32_t tile = min(g + i * NW, T - 1u);
        load_side(sl.side, a.side, tile, lane);
        load_tile_half(sl.t, a.sm, a.ec, tile, lane);
    };
    const bool vec_ok = a.out_vec_ok != 0;
    auto emit = [&](const Slot& sl, uint32_t i) {
        const uint32_t tile = g + i * NW;
        const int tr = (int)(tile / TC);
        const int kt = (int)(tile - (uint32_t)tr * TC);
        const int64_t col = (int64_t)kt * kTileCols + 8 * (lane & 31u);
        const int64_t row0 = (int64_t)tr * kTileRows + (lane >> 5);
        const uint32_t info = side_info(sl.side, 0);
        // wave-uniform: a tile inside the matrix whose rows take whole
        // 16-byte stores needs no per-lane guard
        const bool full = vec_ok && (int64_t)(tr + 1) * kTileRows <= a.N && (int64_t)(kt + 1) * kTileCols <= a.K;
        uint16_t* const out0 = a.out + row0 * a.K + col;
        auto put = [&](int p, const uint32_t wv[4]) {
            if (full) {
                typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
                const u32x4 v = {wv[0], wv[1], wv[2], wv[3]};
                __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(out0 + 2 * p * a.K));
            } else if (row0 + 2 * p < a.N) {
                store8(a.out + (row0 + 2 * p) * a.K, col, a.K, vec_ok, wv);
            }
        };
        if (info_is_fallback(info)) {
            // a tile read as raw BF16 (tile-local row-major, like sm)
            const int16_t* raw = raw_tile_ptr(info, a.fb_raw, a.ovf_raw) + 8 * lane;
            uint4 r[8];
#pragma unroll
            for (int p = 0; p < 8; ++p) r[p] = stream_load(reinterpret_cast<const uint4*>(raw + 512 * p));
            wait_vector_loads();  // rare path: keeps the common path's waits exact
#pragma unroll
            for (int p = 0; p < 8; ++p) {
                const uint32_t wv[4] = {r[p].x, r[p].y, r[p].z, r[p].w};
                put(p, wv);
            }
        } else {
            uint32_t pat[4][8];
            lookup_tile_half(lut, sl.t, pat);
            patch_tile_escapes<kHalfLayout>(pat, info, sl.side, 0, lane);
#pragma unroll
            for (int p = 0; p < 8; ++p) {
                uint32_t wv[4];
                merge_part_half(pat, sl.t, p, wv);
                put(p, wv);
            }
        }
    };
    // the pair table, then the first tile (a wave past the grid's waves
    // re-loads tile g's clamp, so that the table's wait count is exact)
    const uint4 lutv = reinterpret_cast<const uint4*>(a.lut)[lane];
    Slot s0, s1;
    load(s0, 0);
    store_block_lut(lut, lutv, lane);
    lds_barrier();
    if (n == 0) return;
    uint32_t i = 0;
    while (true) {
        if (i + 1 >= n) {
            emit(s0, i);
            break;
        }
        load(s1, i + 1);
        emit(s0, i);
        if (++i + 1 >= n) {
            emit(s1, i);
            break;
        }
        load(s0, i + 1);
        emit(s1, i);
        ++i;
    }
}

template <bool ROWS>
__global__ __launch_bounds__(kDecodeWaves * kWave) void decode_kernel(DecodeArgs a) {
    SE12_DECLARE_LUT(lut);
    const int tid = threadIdx.x;
    const uint32_t lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    store_block_lut(lut, reinterpret_cast<const uint4*>(a.lut)[lane], lane);
    lds_barrier();

    const int64_t item = (int64_t)blockIdx.x * kDecodeWaves + w;
    if (item >= a.items) return;
    const bool vec_ok = a.out_vec_ok != 0;
    if constexpr (!ROWS) {
        const int64_t tile = item;
        const int tr = (int)(tile / a.TC);
        const int kt = (int)(tile - (int64_t)tr * a.TC);
        const int64_t col = (int64_t)kt * kTileCols + 16 * (lane & 15u);
        decode_tile(a, lut, tile, lane, [&](int j, const uint32_t* wv) {
            const int64_t row = (int64_t)tr * kTileRows + 4 * j + (lane >> 4);
            if (row < a.N) store16(a.out + row * a.K, col, a.K, vec_ok, wv);
        });
    } else {
        const int64_t ri = item / a.TC;
        const int kt = (int)(item - ri * a.TC);
        const int64_t row = a.rows[ri];
        const int64_t col = (int64_t)kt * kTileCols + 16 * (lane & 15u);
        uint16_t* out_row = a.out + ri * a.K;
        if (row < 0 || row >= a.N) {
            const uint32_t zero[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            if ((lane >> 4) == 0) store16(out_row, col, a.K, vec_ok, zero);
            return;
        }
        const int lr = (int)(row & (kTileRows - 1));
        const int64_t tile = (row / kTileRows) * a.TC + kt;
        decode_tile(a, lut, tile, lane, [&](int j, const uint32_t* wv) {
            if (4 * j + (int)(lane >> 4) == lr) store16(out_row, col, a.K, vec_ok, wv);
        });
    }
}

// waves of the whole-matrix decode per CU (MI355X, cold HBM, half layout:
// 2304x9216 15.65 us with 4, 16.6 with 6, 15.6 with 8, 15.55 with 12;
// 14336x3584 33.5 / 36.5 / 33.6 / 33.9)
constexpr int kDecodeStreamWavesPerCu = 4;

hipError_t launch_decode(const DecodeArgs& a, bool rows, hipStream_t stream, int cu_count) {
    if (a.items <= 0) return hipSuccess;
    if (rows) {
        const int64_t blocks = (a.items + kDecodeWaves - 1) / kDecodeWaves;
        hipLaunchKernelGGL(decode_kernel<true>, dim3((uint32_t)blocks), dim3(kDecodeWaves * kWave), 0, stream, a);
    } else {
        const int64_t nw = std::min<int64_t>(a.T, (int64_t)std::max(1, cu_count) * kDecodeStreamWavesPerCu);
        const int64_t blocks = (nw + kDecodeWaves - 1) / kDecodeWaves;
        hipLaunchKernelGGL(decode_stream_kernel, dim3((uint32_t)blocks), dim3(kDecodeWaves * kWave), 0, stream, a, nw);
    }
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// bind-time sidecar words
// ---------------------------------------------------------------------------

constexpr int kScanThreads = 1024;

// exclusive scan of one value per thread over the block (1024 threads)
__device__ __forceinline__ int64_t block_exclusive_scan(int64_t v, int64_t* tmp, int64_t* total) {
    const int tid = threadIdx.x;
    tmp[tid] = v;
    __syncthreads();
    for (int d = 1; d < kScanThreads; d <<= 1) {
        int64_t u = tid >= d ? tmp[tid - d] : 0;
        __syncthreads();
        tmp[tid] += u;
        __syncthreads();
    }
    const int64_t incl = tmp[tid];
    *total = tmp[kScanThreads - 1];
    __syncthreads();
    return incl - v;
}

// fallback tiles: kInfoFallback | rank; other tiles: 0 (escape bits come next)
__global__ __launch_bounds__(kScanThreads) void fallback_info_kernel(const uint8_t* bitmap, int64_t T, uint32_t* info,
                                                                     int64_t* total_out) {
    __shared__ int64_t tmp[kScanThreads];
    const int tid = threadIdx.x;
    int64_t chunk = (T + kScanThreads - 1) / kScanThreads;
    chunk = (chunk + 7) & ~int64_t(7);
    const int64_t t0 = (int64_t)tid * chunk;
    const int64_t t1 = t0 + chunk < T ? t0 + chunk : T;
    int64_t count = 0;
    for (int64_t t = t0; t < t1; ++t) count += (bitmap[t >> 3] >> (7 - (t & 7))) & 1;
    int64_t total;
    int64_t base = block_exclusive_scan(count, tmp, &total);
    for (int64_t t = t0; t < t1; ++t) {
        const int bit = (bitmap[t >> 3] >> (7 - (t & 7))) & 1;
        info[t] = bit ? (kInfoFallback | (uint32_t)base) : 0u;
        base += bit;
    }
    if (tid == 0) *total_out = total;
}

// escape chunk bits, escape count and listed escape positions of every
// non-fallback tile: one wave per tile. Escapes are ranked in row-major
// order (chunk, then lane, then weight within the lane), the order in which
// they take the tile's esc slots.
constexpr int kInfoWaves = 4;

__global__ __launch_bounds__(kInfoWaves * kWave) void escape_info_kernel(const uint8_t* ec, int64_t T, uint32_t* info,
                                                                          uint4* escpos) {
    const uint32_t lane = threadIdx.x & 63u;
    const int64_t tile = (int64_t)blockIdx.x * kInfoWaves + (threadIdx.x >> 6);
    if (tile >= T) return;
    const uint8_t* ect = ec + tile * (kTile / 2) + 8u * lane;
    uint16_t* pos = reinterpret_cast<uint16_t*>(escpos + tile);
    uint32_t mask = 0, run = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint2 e = *reinterpret_cast<const uint2*>(ect + 512 * j);
        uint32_t t0 = escape_nibbles(e.x), t1 = escape_nibbles(e.y);
        const uint32_t cnt = __popc(t0) + __popc(t1);
        const uint32_t incl = wave_incl_scan(cnt);
        const uint32_t total = __builtin_amdgcn_readlane(incl, kWave - 1);
        if (total) mask |= 1u << j;
        uint32_t r = run + incl - cnt;
        const uint32_t base = (4u * j + (lane >> 4)) * kTileCols + 16u * (lane & 15u);
        while (t0 | t1) {
            uint32_t p;
            if (t0) {
                p = (uint32_t)__builtin_ctz(t0) >> 2;
                t0 &= t0 - 1u;
            } else {
                p = 8u + ((uint32_t)__builtin_ctz(t1) >> 2);
                t1 &= t1 - 1u;
            }
            if (r < kListedEscapes) pos[r] = (uint16_t)(base + p);
            ++r;
        }
        run += total;
    }
    if (lane == 0 && !info_is_fallback(info[tile]))
        info[tile] = mask | ((run < kInfoCountMax ? run : kInfoCountMax) << kInfoCountShift);
}

// Tiles with more than kListedEscapes escapes become raw tiles: rank them
// (kInfoFallback | kInfoOverflow | rank) and count them.
__global__ __launch_bounds__(kScanThreads) void overflow_info_kernel(int64_t T, uint32_t* info, int64_t* total_out) {
    __shared__ int64_t tmp[kScanThreads];
    const int tid = threadIdx.x;
    const int64_t chunk = (T + kScanThreads - 1) / kScanThreads;
    const int64_t t0 = (int64_t)tid * chunk;
    const int64_t t1 = t0 + chunk < T ? t0 + chunk : T;
    auto over = [&](int64_t t) {
        const uint32_t v = info[t];
        return !info_is_fallback(v) && info_escapes(v) > kListedEscapes;
    };
    int64_t count = 0;
    for (int64_t t = t0; t < t1; ++t) count += over(t) ? 1 : 0;
    int64_t total;
    int64_t base = block_exclusive_scan(count, tmp, &total);
    for (int64_t t = t0; t < t1; ++t)
        if (over(t)) info[t] = kInfoFallback | kInfoOverflow | (uint32_t)base++;
    if (tid == 0) *total_out = total;
}

// Decodes every overflow tile into raw[rank] (tile-local order, the layout of
// the format's fallback tiles), ranking its escapes per chunk (lanes, then
// weights within a lane): one wave per tile.
__global__ __launch_bounds__(kInfoWaves * kWave) void overflow_decode_kernel(DecodeArgs a, int16_t* raw) {
    SE12_DECLARE_LUT(lut);
    const uint32_t lane = threadIdx.x & 63u;
    store_block_lut(lut, reinterpret_cast<const uint4*>(a.lut)[lane], lane);
    lds_barrier();
    const int64_t tile = (int64_t)blockIdx.x * kInfoWaves + (threadIdx.x >> 6);
    if (tile >= a.T) return;
    const uint32_t info = a.info[tile];
    if (!info_is_overflow(info)) return;
    TileLoads t;
    load_tile(t, a.sm, a.ec, tile, lane);
    const uint4 esc = *reinterpret_cast<const uint4*>(a.esc + tile * kEscBudget);
    uint32_t pat[4][8];
    lookup_tile(lut, t, pat);
    resolve_tile_escapes(pat, t, 0xFu, esc);
    int16_t* out = raw + (int64_t)info_rank(info) * kTile;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        uint32_t w[8];
        merge_chunk(pat[j], t.sm[j], w);
        uint4* p = reinterpret_cast<uint4*>(out + 1024 * j + 16 * lane);
        p[0] = make_uint4(w[0], w[1], w[2], w[3]);
        p[1] = make_uint4(w[4], w[5], w[6], w[7]);
    }
}

// The side record of every tile (one thread per record word).
__global__ void side_record_kernel(const uint32_t* info, const uint8_t* esc, const uint4* escpos, int64_t T,
                                   uint32_t* side) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= T * kSideWords) return;
    const int64_t t = i / kSideWords;
    const int k = (int)(i % kSideWords);
    uint32_t v = 0;
    if (k == 0)
        v = info[t];
    else if (k <= 4)
        v = reinterpret_cast<const uint32_t*>(esc + t * kEscBudget)[k - 1];
    else if (k <= 8)
        v = reinterpret_cast<const uint32_t*>(escpos + t)[k - 5];
    side[i] = v;
}

hipError_t launch_side_records(const uint32_t* info, const uint8_t* esc, const uint4* escpos, int64_t T, uint32_t* side,
                               hipStream_t stream) {
    if (T == 0) return hipSuccess;
    const int64_t n = T * kSideWords;
    hipLaunchKernelGGL(side_record_kernel, dim3((uint32_t)((n + 255) / 256)), dim3(256), 0, stream, info, esc, escpos, T,
                       side);
    return hipGetLastError();
}

hipError_t launch_overflow_decode(const DecodeArgs& a, int16_t* raw, hipStream_t stream) {
    const int64_t blocks = (a.T + kInfoWaves - 1) / kInfoWaves;
    hipLaunchKernelGGL(overflow_decode_kernel, dim3((uint32_t)blocks), dim3(kInfoWaves * kWave), 0, stream, a, raw);
    return hipGetLastError();
}

hipError_t launch_tile_info(const uint8_t* bitmap, const uint8_t* ec, int64_t T, uint32_t* info, uint4* escpos,
                            int64_t* total, hipStream_t stream) {
    hipLaunchKernelGGL(fallback_info_kernel, dim3(1), dim3(kScanThreads), 0, stream, bitmap, T, info, total);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || T == 0) return e;
    const int64_t blocks = (T + kInfoWaves - 1) / kInfoWaves;
    hipLaunchKernelGGL(escape_info_kernel, dim3((uint32_t)blocks), dim3(kInfoWaves * kWave), 0, stream, ec, T, info,
                       escpos);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(overflow_info_kernel, dim3(1), dim3(kScanThreads), 0, stream, T, info, total + 1);
    return hipGetLastError();
}

}  // namespace se12
