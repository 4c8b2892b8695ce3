// Device helpers shared by every SE12 kernel for gfx950 (CDNA4, wave64).
//
// Lane mapping used everywhere: a wave owns one 16x256 tile at a time. Lane l
// handles four 16-weight chunks j = 0..3 at tile offset o = 1024*j + 16*l,
// i.e. tile row 4*j + (l >> 4), tile columns 16*(l & 15) .. +15. So each of
// the wave's four `sm` loads (dwordx4 per lane) and four `ec` loads (dwordx2
// per lane) reads 1 KiB / 512 B of contiguous HBM, and the 16 lanes that share
// a tile row hold adjacent columns (reduced with DPP row ops).
//
// Decode of one chunk (16 weights, 8 BF16 pairs):
//   pattern pair  = lut[ec byte]  (LDS, 256 dwords: both nibbles' exponent
//                                  << 7 in each 16-bit half; bit 0 marks an
//                                  escape code 15 in either nibble)
//   sign/mantissa = v_perm of the sm dword duplicating each byte into both
//                   halves of a 16-bit lane: (s<<8)|s keeps the sign at bit
//                   15 and the mantissa at bits 6..0
//   BF16 pair     = v_bfi(0x7F807F80, pattern, sm-dup)
// which rebuilds ((sm & 0x80) << 8) | (exp << 7) | (sm & 0x7F), the join of
// lws/domain/weights.py:109-119, for two weights at once.
//
// Escapes: a code-15 weight takes the next unused slot of its tile's 16 `esc`
// bytes, in tile-local row-major order (lws/domain/se12/codec.py:131,379-391).
// Chunks are visited in that order (j, then lane, then position), so the rank
// of an escape is `run` (escapes of earlier chunks) + the escapes of lower
// lanes in this chunk (a wave scan) + the earlier escapes of this lane. The
// scan and patch only run when some lane of the wave saw an escape in the
// chunk (a wave-uniform branch); the rank is clamped to 15 like the reference
// decoder's clip (codec.py:385).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace se12 {

constexpr int kTileRows = 16;
constexpr int kTileCols = 256;
constexpr int kTile = 4096;
constexpr int kEscBudget = 16;
constexpr int kCodebook = 15;
constexpr int kEscCode = 15;
constexpr int kWave = 64;

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) {
    return __builtin_amdgcn_perm(hi, lo, sel);
}

// bytes 0,1 of w -> [b1 b1 b0 b0]; bytes 2,3 -> [b3 b3 b2 b2]
__device__ __forceinline__ uint32_t dup_lo(uint32_t w) { return perm(w, w, 0x01010000u); }
__device__ __forceinline__ uint32_t dup_hi(uint32_t w) { return perm(w, w, 0x03030202u); }

constexpr uint32_t kExpMask2 = 0x7F807F80u;  // exponent bits of two BF16 values

__device__ __forceinline__ uint32_t merge_pair(uint32_t pattern, uint32_t smdup) {
    return (pattern & kExpMask2) | (smdup & ~kExpMask2);
}

// bit 4*i set iff nibble i of d is 0xF (an escape code)
__device__ __forceinline__ uint32_t escape_nibbles(uint32_t d) {
    return d & (d >> 1) & (d >> 2) & (d >> 3) & 0x11111111u;
}

__device__ __forceinline__ uint32_t lane_id() { return __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u)); }

__device__ __forceinline__ bool wave_any(bool p) { return __builtin_amdgcn_ballot_w64(p) != 0; }

// inclusive prefix sum over the 64 lanes (slow paths only)
__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t v, uint32_t lane) {
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
        uint32_t u = __shfl_up(v, d, kWave);
        if (lane >= (uint32_t)d) v += u;
    }
    return v;
}

// LDS barrier that does not wait for outstanding global loads (a plain
// __syncthreads would also drain vmcnt and kill the prefetch).
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Fills the 256-entry pair table from the 15-byte codebook (all threads of
// the block take part; the caller synchronizes).
__device__ __forceinline__ void build_pair_lut(uint32_t* lut, const uint8_t* codebook, int tid, int nthreads) {
    for (int b = tid; b < 256; b += nthreads) {
        uint32_t c0 = b & 15u, c1 = (uint32_t)b >> 4;
        uint32_t p0 = c0 < 15u ? ((uint32_t)codebook[c0] << 7) : 0u;
        uint32_t p1 = c1 < 15u ? ((uint32_t)codebook[c1] << 7) : 0u;
        lut[b] = p0 | (p1 << 16) | ((c0 == 15u || c1 == 15u) ? 1u : 0u);
    }
}

// escape slot r (0..15) of a tile whose 16 esc bytes are in e
__device__ __forceinline__ uint32_t esc_byte(uint4 e, uint32_t r) {
    uint32_t d = r < 8u ? (r < 4u ? e.x : e.y) : (r < 12u ? e.z : e.w);
    return (d >> ((r & 3u) * 8u)) & 0xFFu;
}

// write exponent e into the pattern of weight p (0..15) of the chunk; every
// element is rewritten through a mask so the array stays in registers
__device__ __forceinline__ void patch_exponent(uint32_t pat[8], uint32_t p, uint32_t e) {
    const uint32_t q = p >> 1;
    const bool hi = (p & 1u) != 0u;
    const uint32_t m = hi ? 0x7F800000u : 0x00007F80u;
    const uint32_t v = hi ? (e << 23) : (e << 7);
#pragma unroll
    for (uint32_t i = 0; i < 8; ++i) {
        const uint32_t sel = 0u - (uint32_t)(i == q);
        pat[i] = (pat[i] & ~(m & sel)) | (v & sel);
    }
}

__device__ __forceinline__ void resolve_escapes(uint32_t pat[8], uint2 ec, uint4 esc, uint32_t& run, uint32_t lane) {
    uint32_t t0 = escape_nibbles(ec.x), t1 = escape_nibbles(ec.y);
    const uint32_t cnt = __popc(t0) + __popc(t1);
    const uint32_t incl = wave_incl_scan(cnt, lane);
    const uint32_t total = __builtin_amdgcn_readlane(incl, kWave - 1);
    uint32_t r = run + incl - cnt;
    while (t0) {
        const uint32_t p = (uint32_t)__builtin_ctz(t0) >> 2;
        t0 &= t0 - 1u;
        patch_exponent(pat, p, esc_byte(esc, r < 15u ? r : 15u));
        ++r;
    }
    while (t1) {
        const uint32_t p = 8u + ((uint32_t)__builtin_ctz(t1) >> 2);
        t1 &= t1 - 1u;
        patch_exponent(pat, p, esc_byte(esc, r < 15u ? r : 15u));
        ++r;
    }
    run += total;
}

// Decodes one chunk (16 weights) into 8 BF16 pairs (low half = even column).
__device__ __forceinline__ void decode_chunk(const uint32_t* lut, uint4 sm, uint2 ec, uint4 esc, uint32_t& run,
                                             uint32_t lane, uint32_t w[8]) {
    uint32_t pat[8];
    pat[0] = lut[ec.x & 0xFFu];
    pat[1] = lut[(ec.x >> 8) & 0xFFu];
    pat[2] = lut[(ec.x >> 16) & 0xFFu];
    pat[3] = lut[ec.x >> 24];
    pat[4] = lut[ec.y & 0xFFu];
    pat[5] = lut[(ec.y >> 8) & 0xFFu];
    pat[6] = lut[(ec.y >> 16) & 0xFFu];
    pat[7] = lut[ec.y >> 24];
    const uint32_t mark = (pat[0] | pat[1] | pat[2] | pat[3] | pat[4] | pat[5] | pat[6] | pat[7]) & 1u;
    if (wave_any(mark != 0u)) resolve_escapes(pat, ec, esc, run, lane);
    w[0] = merge_pair(pat[0], dup_lo(sm.x));
    w[1] = merge_pair(pat[1], dup_hi(sm.x));
    w[2] = merge_pair(pat[2], dup_lo(sm.y));
    w[3] = merge_pair(pat[3], dup_hi(sm.y));
    w[4] = merge_pair(pat[4], dup_lo(sm.z));
    w[5] = merge_pair(pat[5], dup_hi(sm.z));
    w[6] = merge_pair(pat[6], dup_lo(sm.w));
    w[7] = merge_pair(pat[7], dup_hi(sm.w));
}

// One tile's loads for one lane. The per-tile escape slots and fallback rank
// are wave-uniform but loaded like the rest (vector loads of one address):
// scalar loads here would be waited for as soon as the prefetch is issued.
struct TileLoads {
    uint4 sm[4];
    uint2 ec[4];
    uint4 esc;
    int32_t fallback_rank;  // rank among fallback tiles, or -1
};

// the bind-time sidecar: rank of the tile among fallback tiles, -1 if the tile
// is not a fallback tile
__device__ __forceinline__ void load_tile(TileLoads& t, const uint8_t* sm, const uint8_t* ec, const uint8_t* esc,
                                          const int32_t* fb_rank, int64_t tile, uint32_t lane) {
    const uint8_t* smt = sm + tile * kTile + 16u * lane;
    const uint8_t* ect = ec + tile * (kTile / 2) + 8u * lane;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        t.sm[j] = *reinterpret_cast<const uint4*>(smt + 1024 * j);
        t.ec[j] = *reinterpret_cast<const uint2*>(ect + 512 * j);
    }
    t.esc = *reinterpret_cast<const uint4*>(esc + tile * kEscBudget);
    t.fallback_rank = fb_rank[tile];
}

// the (uniform) fallback rank of a loaded tile, in a scalar register
__device__ __forceinline__ int32_t uniform_rank(const TileLoads& t) {
    return __builtin_amdgcn_readfirstlane(t.fallback_rank);
}

// Raw BF16 pairs of chunk j of a fallback tile (tile-local order, like sm).
__device__ __forceinline__ void load_raw_chunk(const int16_t* tile_raw, int j, uint32_t lane, uint32_t w[8]) {
    const uint4* p = reinterpret_cast<const uint4*>(tile_raw + 1024 * j + 16 * lane);
    uint4 a = p[0], b = p[1];
    w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
    w[4] = b.x; w[5] = b.y; w[6] = b.z; w[7] = b.w;
}

// Sum over the 16 lanes of a DPP row; every lane of the row gets the sum.
__device__ __forceinline__ float row16_sum(float v) {
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, true));   // quad_perm 1,0,3,2
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, true));   // quad_perm 2,3,0,1
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x141, 0xF, 0xF, true));  // row_half_mirror
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x140, 0xF, 0xF, true));  // row_mirror
    return v;
}

__device__ __forceinline__ float dot2_bf16(uint32_t w, uint32_t x, float acc) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w), __builtin_bit_cast(bf16x2_t, x), acc, false);
}

}  // namespace se12
