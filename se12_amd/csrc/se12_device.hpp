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
//   pattern pair  = lut[ec byte]  (LDS, 256 dwords built once per matrix at
//                                  bind time: both nibbles' exponent << 7 in
//                                  each 16-bit half)
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
// scan and patch only run for chunks that the tile's bind-time sidecar word
// marks as holding escapes (a wave-uniform branch); the rank is clamped to 15
// like the reference decoder's clip (codec.py:385).
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

// A load of tile-stream bytes that one launch reads exactly once, where each
// load instruction reads whole 128-byte lines that no other instruction
// reads: nontemporal, so the caches keep x, the pair table and the partial
// sums instead of bytes that are never read again. On MI355X, batch-1
// launches measured, against plain loads (same box, interleaved): 2304x9216
// 8.49 -> 8.28 us, 2 x 9216x2304 grouped 14.13 -> 13.41, 14336x3584 16.69
// -> 15.56, 4608x36864 50.5 -> 45.2 us. Where an instruction reads half of
// each line and the next one the other half (the x-slab kernel's row layout,
// the raw twin's 32 bytes per lane as two loads, side records of 64 bytes)
// the hint makes the second read fetch the line again: the x-slab kernel at
// 14336x3584, batch 32, took 31.3 us with it against 26.5 without, the raw
// twin at 2304x9216 16.2 against 11.2; those loads stay plain.
template <typename T>
__device__ __forceinline__ T stream_load(const T* p) {
    if constexpr (sizeof(T) == 16) {
        typedef uint32_t v4 __attribute__((ext_vector_type(4)));
        const v4 v = __builtin_nontemporal_load(reinterpret_cast<const v4*>(p));
        return __builtin_bit_cast(T, v);
    } else if constexpr (sizeof(T) == 8) {
        typedef uint32_t v2 __attribute__((ext_vector_type(2)));
        const v2 v = __builtin_nontemporal_load(reinterpret_cast<const v2*>(p));
        return __builtin_bit_cast(T, v);
    } else {
        static_assert(sizeof(T) == 4, "stream_load: 4, 8 or 16 bytes");
        return __builtin_bit_cast(T, __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(p)));
    }
}

// inclusive prefix sum over the 64 lanes with DPP: shifts of 1, 2, 4, 8
// within each 16-lane row, then the row totals carried across rows by the
// row broadcasts of lanes 15 and 31
__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t v) {
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x111, 0xF, 0xF, false);  // row_shr:1
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x112, 0xF, 0xF, false);  // row_shr:2
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x114, 0xF, 0xF, false);  // row_shr:4
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x118, 0xF, 0xF, false);  // row_shr:8
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x142, 0xA, 0xF, false);  // row_bcast:15 -> rows 1, 3
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x143, 0xC, 0xF, false);  // row_bcast:31 -> rows 2, 3
    return v;
}

// LDS barrier that does not wait for outstanding global loads (a plain
// __syncthreads would also drain vmcnt and kill the prefetch).
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Entry b of the pair table: the exponents of codes (b & 15) and (b >> 4),
// each << 7, in the low and high 16-bit halves; escape code 15 contributes 0
// (its exponent is patched in from the tile's esc slots).
__host__ __device__ inline uint32_t pair_lut_entry(const uint8_t* codebook, uint32_t b) {
    const uint32_t c0 = b & 15u, c1 = b >> 4;
    const uint32_t p0 = c0 < 15u ? ((uint32_t)codebook[c0] << 7) : 0u;
    const uint32_t p1 = c1 < 15u ? ((uint32_t)codebook[c1] << 7) : 0u;
    return p0 | (p1 << 16);
}

// The block's pair table: a static LDS array, so it sits at LDS address 0
// and a lookup's address is one byte-select shift (SDWA) of the ec word.
// Every wave loads the bind-time table (1 KiB, 16 bytes per lane) as its
// first load and stores it whole (the same values, with relaxed atomic
// stores, so the waves' overlapping stores are well defined); an
// unconditional store keeps the load from being sunk behind the tile loads.
// The caller runs lds_barrier() before the first lookup.
#define SE12_DECLARE_LUT(name) __shared__ __attribute__((aligned(16))) uint32_t name[256]

__device__ __forceinline__ void store_block_lut(uint32_t* lut, uint4 v, uint32_t lane) {
    __hip_atomic_store(&lut[4 * lane + 0], v.x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    __hip_atomic_store(&lut[4 * lane + 1], v.y, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    __hip_atomic_store(&lut[4 * lane + 2], v.z, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    __hip_atomic_store(&lut[4 * lane + 3], v.w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// escape slot r (0..15) of a tile whose 16 esc bytes are in e
__device__ __forceinline__ uint32_t esc_byte(uint4 e, uint32_t r) {
    uint32_t d = r < 8u ? (r < 4u ? e.x : e.y) : (r < 12u ? e.z : e.w);
    return (d >> ((r & 3u) * 8u)) & 0xFFu;
}

// write exponent e into the pattern of weight p (0..15) of the chunk. The
// pair table gives the escape code no exponent, so the field is 0 and an OR
// suffices; the word is chosen by a one-hot mask (two instructions per word)
// so the array stays in registers.
__device__ __forceinline__ void patch_exponent(uint32_t pat[8], uint32_t p, uint32_t e) {
    const uint32_t v = e << ((p & 1u) ? 23u : 7u);
    const uint32_t onehot = 1u << (p >> 1);
#pragma unroll
    for (uint32_t i = 0; i < 8; ++i) pat[i] |= v & (uint32_t)((int32_t)(onehot << (31u - i)) >> 31);
}

__device__ __forceinline__ void resolve_escapes(uint32_t pat[8], uint2 ec, uint4 esc, uint32_t& run) {
    uint32_t t0 = escape_nibbles(ec.x), t1 = escape_nibbles(ec.y);
    const uint32_t cnt = __popc(t0) + __popc(t1);
    // escapes of lower lanes: a mask count when no lane holds more than one
    // escape in the chunk (the common case), else a wave prefix sum
    uint32_t below, total;
    if (__builtin_amdgcn_ballot_w64(cnt > 1u) == 0) {
        const uint64_t has = __builtin_amdgcn_ballot_w64(cnt != 0u);
        below = __builtin_amdgcn_mbcnt_hi((uint32_t)(has >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)has, 0u));
        total = (uint32_t)__builtin_popcountll(has);
    } else {
        const uint32_t incl = wave_incl_scan(cnt);
        below = incl - cnt;
        total = __builtin_amdgcn_readlane(incl, kWave - 1);
    }
    // the lane's escapes in weight order, both halves in one loop (one
    // iteration when no lane holds two)
    uint32_t r = run + below;
    while (t0 | t1) {
        uint32_t p;
        if (t0) {
            p = (uint32_t)__builtin_ctz(t0) >> 2;
            t0 &= t0 - 1u;
        } else {
            p = 8u + ((uint32_t)__builtin_ctz(t1) >> 2);
            t1 &= t1 - 1u;
        }
        patch_exponent(pat, p, esc_byte(esc, r < 15u ? r : 15u));
        ++r;
    }
    run += total;
}

// The 8 pattern pairs of one chunk (one LDS lookup per ec byte).
__device__ __forceinline__ void lookup_chunk(const uint32_t* lut, uint2 ec, uint32_t pat[8]) {
    pat[0] = lut[ec.x & 0xFFu];
    pat[1] = lut[(ec.x >> 8) & 0xFFu];
    pat[2] = lut[(ec.x >> 16) & 0xFFu];
    pat[3] = lut[ec.x >> 24];
    pat[4] = lut[ec.y & 0xFFu];
    pat[5] = lut[(ec.y >> 8) & 0xFFu];
    pat[6] = lut[(ec.y >> 16) & 0xFFu];
    pat[7] = lut[ec.y >> 24];
}

// Rebuilds the 8 BF16 pairs of a chunk from its patterns and sm bytes.
__device__ __forceinline__ void merge_chunk(const uint32_t pat[8], uint4 sm, uint32_t w[8]) {
    w[0] = merge_pair(pat[0], dup_lo(sm.x));
    w[1] = merge_pair(pat[1], dup_hi(sm.x));
    w[2] = merge_pair(pat[2], dup_lo(sm.y));
    w[3] = merge_pair(pat[3], dup_hi(sm.y));
    w[4] = merge_pair(pat[4], dup_lo(sm.z));
    w[5] = merge_pair(pat[5], dup_hi(sm.z));
    w[6] = merge_pair(pat[6], dup_lo(sm.w));
    w[7] = merge_pair(pat[7], dup_hi(sm.w));
}

// Per-tile word built at bind time (one per tile):
//   bit 31 set   -> a tile read as raw BF16: bits 0..29 = its rank among the
//                   format's fallback tiles, or, with bit 30 set, among the
//                   tiles holding more than kListedEscapes escapes, which
//                   bind decodes once into a raw buffer of its own
//   bit 31 clear -> bit j (j = 0..3) set iff chunk j (tile rows 4j..4j+3)
//                   holds at least one escape code; bits 8..12 = the tile's
//                   escape count (at most kListedEscapes on this path)
// and, per tile, the positions (row * 256 + column, row-major order: the
// order escapes take their esc slots) of its kListedEscapes first escapes,
// 16 bits each in one 16-byte word.
constexpr uint32_t kInfoFallback = 0x80000000u;
constexpr uint32_t kInfoOverflow = 0x40000000u;
constexpr uint32_t kInfoCountShift = 8;
constexpr uint32_t kInfoCountMax = 31;
constexpr uint32_t kListedEscapes = 8;

__device__ __forceinline__ bool info_is_fallback(uint32_t info) { return (info & kInfoFallback) != 0u; }
__device__ __forceinline__ bool info_is_overflow(uint32_t info) { return (info & kInfoOverflow) != 0u; }
__device__ __forceinline__ uint32_t info_rank(uint32_t info) { return info & ~(kInfoFallback | kInfoOverflow); }
__device__ __forceinline__ uint32_t info_escapes(uint32_t info) { return (info >> kInfoCountShift) & kInfoCountMax; }

// One tile's `sm` and `ec` loads for one lane.
struct TileLoads {
    uint4 sm[4];
    uint2 ec[4];
};

__device__ __forceinline__ void load_tile(TileLoads& t, const uint8_t* sm, const uint8_t* ec, int64_t tile,
                                          uint32_t lane) {
    const uint8_t* smt = sm + tile * kTile + 16u * lane;
    const uint8_t* ect = ec + tile * (kTile / 2) + 8u * lane;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        t.sm[j] = stream_load(reinterpret_cast<const uint4*>(smt + 1024 * j));
        t.ec[j] = stream_load(reinterpret_cast<const uint2*>(ect + 512 * j));
    }
}

// The per-tile side record built at bind time: 16 dwords (64 bytes) per
// tile, word 0 the sidecar word, words 1..4 the tile's 16 esc slots, words
// 5..8 the listed escape positions, 9..15 zero. A wave reads records with one
// dword load, lanes 16 s .. 16 s + 15 holding the record of its tile slot s
// (up to 4 tiles per load): 256 bytes reach the registers instead of the
// 64 x 36 a per-lane copy of each field would move. The per-lane addresses
// differ, so this stays a vector load (a scalar load would share its wait
// counter with the LDS lookups). Read back with readlane.
constexpr int kSideWords = 16;

struct TileSide {
    uint32_t rec;
};

// `tile` is the tile of this lane's slot (lane / 16).
__device__ __forceinline__ void load_side(TileSide& s, const uint32_t* side, int64_t tile, uint32_t lane) {
    s.rec = side[tile * kSideWords + (lane & 15u)];
}

__device__ __forceinline__ uint32_t side_word(const TileSide& s, int g, int k) {
    return (uint32_t)__builtin_amdgcn_readlane((int)s.rec, 16 * g + k);
}

__device__ __forceinline__ uint32_t side_info(const TileSide& s, int g) { return side_word(s, g, 0); }

__device__ __forceinline__ uint4 side_esc(const TileSide& s, int g) {
    return make_uint4(side_word(s, g, 1), side_word(s, g, 2), side_word(s, g, 3), side_word(s, g, 4));
}

__device__ __forceinline__ uint4 side_pos(const TileSide& s, int g) {
    return make_uint4(side_word(s, g, 5), side_word(s, g, 6), side_word(s, g, 7), side_word(s, g, 8));
}

// All 32 pattern lookups of a tile (issued back to back).
__device__ __forceinline__ void lookup_tile(const uint32_t* lut, const TileLoads& t, uint32_t pat[4][8]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) lookup_chunk(lut, t.ec[j], pat[j]);
}

// Patches the escape exponents into the chunks that the tile's sidecar word
// (wave-uniform) marks as holding escapes; escape-free chunks cost nothing.
__device__ __forceinline__ void resolve_tile_escapes(uint32_t pat[4][8], const TileLoads& t, uint32_t info, uint4 esc) {
    uint32_t run = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        if (info & (1u << j)) resolve_escapes(pat[j], t.ec[j], esc, run);
    }
}

// pat[word / 8][word % 8] |= v for a wave-uniform word: the 32 words as
// one vector value, so the uniform index becomes a register-indexed move
// (on an array the computed index would move it to scratch memory).
typedef uint32_t PatternVector __attribute__((ext_vector_type(32)));

__device__ __forceinline__ void or_pattern_word(uint32_t pat[4][8], uint32_t word, uint32_t v) {
    PatternVector t;
#pragma unroll
    for (int i = 0; i < 32; ++i) t[i] = pat[i >> 3][i & 7];
    t[word & 31u] |= v;
#pragma unroll
    for (int i = 0; i < 32; ++i) pat[i >> 3][i & 7] = t[i];
}

// Patches the n (1..kListedEscapes) listed escapes of a tile: escape k sits
// at pos_k = row * 256 + col and takes esc slot k. Everything but the final
// OR is wave-uniform (scalar), so an escape costs a few instructions.
// Three lane layouts of a tile's 16 x 256 weights, 16 consecutive columns
// of one row (a column block, col / 16) per lane in each of 4 parts
// (pat[part][word], word = pair of columns):
//   chunk layout (dot2, decode): part j = rows 4j..4j+3, lane 16 (row % 4) +
//     block;
//   row layout (se12_gemm.hip): part p = columns 64p..64p+63, lane row + 16
//     (block % 4);
//   block layout (se12_gemm_rx.hip): part = block % 4, lane row + 16 (block
//     / 4).
// and one of 8 columns per lane in each of 8 parts:
//   half layout (the decode-only kernel): part p = rows 2p, 2p+1, lane 32
//     (row % 2) + col / 8, word (col % 8) / 2 of the part's 4, stored as
//     pattern word 4p + word (pat[p / 2][4 (p % 2) + word]).
enum TileLayout { kChunkLayout, kRowLayout, kBlockLayout, kHalfLayout };

template <int LAYOUT>
__device__ __forceinline__ void patch_listed_escapes(uint32_t pat[4][8], uint4 pos, uint4 esc, uint32_t n,
                                                     uint32_t lane) {
    for (uint32_t k = 0; k < n; ++k) {
        const uint32_t w = k < 4u ? (k < 2u ? pos.x : pos.y) : (k < 6u ? pos.z : pos.w);
        const uint32_t p = (k & 1u) ? (w >> 16) : (w & 0xFFFFu);
        const uint32_t row = (p >> 8) & 15u, col = p & 255u, block = col >> 4;
        const uint32_t owner = LAYOUT == kChunkLayout ? (((row & 3u) << 4) | block)
                               : LAYOUT == kRowLayout ? (row | ((block & 3u) << 4))
                               : LAYOUT == kHalfLayout ? (((row & 1u) << 5) | (col >> 3))
                                                       : (row | ((block >> 2) << 4));
        const uint32_t part = LAYOUT == kChunkLayout ? (row >> 2) : LAYOUT == kRowLayout ? (block >> 2) : (block & 3u);
        const uint32_t word = LAYOUT == kHalfLayout ? (((row >> 1) << 2) | ((col & 7u) >> 1))
                                                    : ((part << 3) | ((col & 15u) >> 1));
        const uint32_t v = esc_byte(esc, k) << ((col & 1u) ? 23u : 7u);
        or_pattern_word(pat, word, lane == owner ? v : 0u);
    }
}

// The escapes of a tile read through the pair table (at most
// kListedEscapes: bind turns tiles with more into raw tiles).
template <int LAYOUT = kChunkLayout>
__device__ __forceinline__ void patch_tile_escapes(uint32_t pat[4][8], uint32_t info, const TileSide& side, int g,
                                                   uint32_t lane) {
    const uint32_t n = info_escapes(info);
    if (n != 0u) patch_listed_escapes<LAYOUT>(pat, side_pos(side, g), side_esc(side, g), n, lane);
}

// The raw BF16 of a tile that bind marked raw: the format's fallback tiles,
// or the tiles bind decoded because they hold too many escapes.
__device__ __forceinline__ const int16_t* raw_tile_ptr(uint32_t info, const int16_t* fb_raw, const int16_t* ovf_raw) {
    return (info_is_overflow(info) ? ovf_raw : fb_raw) + (int64_t)info_rank(info) * kTile;
}

// Waits for every vector memory load in flight (vmcnt(0)) through the
// compiler's intrinsic, which its wait counting sees (inline asm it does not).
// A branch whose loads fill registers that the other branch computes (a raw
// tile beside a decoded one) ends with it: the join would otherwise inherit
// the pending load and wait there, on the common path too, for every load in
// flight, prefetched tiles included.
// wait_vector_loads_to<N>() leaves the last N in flight (vmcnt(N)).
template <int N>
__device__ __forceinline__ void wait_vector_loads_to() {
    static_assert(N >= 0 && N < 64, "vmcnt holds 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}
__device__ __forceinline__ void wait_vector_loads() { wait_vector_loads_to<0>(); }

// LDS byte address of a pointer into LDS (the low half of its generic address)
__device__ __forceinline__ uint32_t lds_address(const void* p) {
    return __builtin_amdgcn_readfirstlane((uint32_t)reinterpret_cast<uintptr_t>(p));
}

// One 16-byte global load per lane straight into LDS: lane l's bytes land at
// LDS byte address lds + 16 l (lds wave-uniform). Inline asm, which the
// compiler's wait counting does not see: the caller waits for it itself
// (s_waitcnt vmcnt) before reading the LDS it fills. The compiler's own
// waits stay correct as long as loads it tracks are only waited for by
// count (loads complete in order, so an unseen load only makes a count
// wait for more).
__device__ __forceinline__ void lds_load16(const void* src, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(lds) : "memory", "m0");
}

// Raw BF16 pairs of chunk j of a fallback tile (tile-local order, like sm).
__device__ __forceinline__ void load_raw_chunk(const int16_t* tile_raw, int j, uint32_t lane, uint32_t w[8]) {
    const uint4* p = reinterpret_cast<const uint4*>(tile_raw + 1024 * j + 16 * lane);
    uint4 a = p[0], b = p[1];
    w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
    w[4] = b.x; w[5] = b.y; w[6] = b.z; w[7] = b.w;
}

// A wave-uniform global pointer in scalar registers: loads from it plus a
// 32-bit per-lane offset need one VGPR for the address instead of two. The
// result is typed as global memory: a pointer rebuilt from integers would
// otherwise be a flat one, whose loads also count as LDS operations (a wait
// for the pair-table lookups would then wait for the tile loads in flight).
template <typename T>
using global_ptr = const __attribute__((address_space(1))) T*;

template <typename T>
__device__ __forceinline__ global_ptr<T> wave_uniform(const T* p) {
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(v >> 32));
    return reinterpret_cast<global_ptr<T>>(((uint64_t)hi << 32) | lo);
}

__device__ __forceinline__ void load_tile_block_order(TileLoads& t, TileSide& side, const uint8_t* sm, const uint8_t* ec,
                                               const uint32_t* sd, int64_t tile, uint32_t lane) {
    const uint32_t off = (lane & 3u) * kTileCols + 16u * (lane >> 2);
    const global_ptr<uint8_t> smt = wave_uniform(sm + tile * kTile);
    const global_ptr<uint8_t> ect = wave_uniform(ec + tile * (kTile / 2));
    const global_ptr<uint32_t> sdt = wave_uniform(sd + tile * kSideWords);
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    side.rec = sdt[lane & 15u];
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        const u32x4 s4 = __builtin_nontemporal_load(reinterpret_cast<global_ptr<u32x4>>(smt + off + 1024 * p));
        const u32x2 e2 = __builtin_nontemporal_load(reinterpret_cast<global_ptr<u32x2>>(ect + off / 2 + 512 * p));
        t.sm[p] = make_uint4(s4[0], s4[1], s4[2], s4[3]);
        t.ec[p] = make_uint2(e2[0], e2[1]);
    }
}

// Exchanges part bit B with lane bit B + 2 between parts x (bit clear) and
// y (bit set): lanes with the lane bit set take y from the lane 2^(B+2)
// below, and the others x from the lane 2^(B+2) above. One DPP row shift
// each, written only to the lanes that take it: a DPP bank is 4 lanes of a
// 16-lane row, so lane bits 2 and 3 select banks.
template <int B>
__device__ __forceinline__ void swap_part_lane(uint32_t& x, uint32_t& y) {
    constexpr int n = 4 << B;
    constexpr int hi_banks = B == 1 ? 0xC : 0xA;
    const uint32_t nx = (uint32_t)__builtin_amdgcn_update_dpp((int)x, (int)y, 0x110 + n, 0xF, hi_banks, false);
    y = (uint32_t)__builtin_amdgcn_update_dpp((int)y, (int)x, 0x100 + n, 0xF, hi_banks ^ 0xF, false);
    x = nx;
}

// the swaps of W word pairs; the scheduler may not gather the copies of all
// of them up front (each swap keeps one old word until its second move)
template <int B, int W>
__device__ __forceinline__ void swap_part_lane_words(uint32_t (&x)[W], uint32_t (&y)[W]) {
#pragma unroll
    for (int i = 0; i < W; ++i) swap_part_lane<B>(x[i], y[i]);
    __builtin_amdgcn_sched_barrier(0);
}

// Chunk-order loads -> block layout: after the loads lane l holds (row 4p +
// l % 4, block l / 4) in part p, i.e. row bits 3..2 in the part and row bits
// 1..0 in lane bits 1..0; exchanging part bit 1 with lane bit 3 and part bit
// 0 with lane bit 2 leaves lane l with row l % 16 and block 4 (l / 16) + p.
__device__ __forceinline__ void chunks_to_blocks(TileLoads& t) {
    uint32_t s[4][4], e[4][2];
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        s[p][0] = t.sm[p].x; s[p][1] = t.sm[p].y; s[p][2] = t.sm[p].z; s[p][3] = t.sm[p].w;
        e[p][0] = t.ec[p].x; e[p][1] = t.ec[p].y;
    }
    swap_part_lane_words<1>(s[0], s[2]);
    swap_part_lane_words<1>(s[1], s[3]);
    swap_part_lane_words<1>(e[0], e[2]);
    swap_part_lane_words<1>(e[1], e[3]);
    swap_part_lane_words<0>(s[0], s[1]);
    swap_part_lane_words<0>(s[2], s[3]);
    swap_part_lane_words<0>(e[0], e[1]);
    swap_part_lane_words<0>(e[2], e[3]);
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        t.sm[p] = make_uint4(s[p][0], s[p][1], s[p][2], s[p][3]);
        t.ec[p] = make_uint2(e[p][0], e[p][1]);
    }
}

// Split-K partial sums that other blocks read (any XCD): device-scope
// relaxed atomics, which bypass the XCD's own L2. Four consecutive floats
// (16-byte aligned) go as two 64-bit accesses: each access is a separate
// transaction past L2, so fewer, wider ones cost less (2304x9216 B = 32, 4
// splits: 20.6 us with four 32-bit stores and loads against 19.4). The
// reader issues every split's loads before the first add (a loop that added
// as it loaded would wait one round trip per split: 3584x14336 B = 24, 5
// splits, 29.1 against 27.3 us); it adds them in ascending split order.
__device__ __forceinline__ void store_partial4(float* p, const float v[4]) {
    uint64_t* q = reinterpret_cast<uint64_t*>(p);
    __hip_atomic_store(q, ((uint64_t)__float_as_uint(v[1]) << 32) | __float_as_uint(v[0]), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(q + 1, ((uint64_t)__float_as_uint(v[3]) << 32) | __float_as_uint(v[2]), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}

// Split-K sums without an arrival counter: the S partial sums of one output
// meet in a fixed binary tree (level 0 pairs splits 2i and 2i + 1, each level
// pairs the sums of the one below, an odd last one moves up unpaired). A
// pair meets in one 64-bit slot through one device-scope exchange: the first
// of the two to arrive leaves (1 << 32) | its bits there and is done; the
// second gets them back, adds them (a + b == b + a exactly, so the order of
// arrival changes no bit of the result), clears the slot and carries the sum
// up. A thread pays one round trip per level it climbs, where a counter
// costs three (partial store and its wait, counter, reload). Slots are zero
// between launches: every slot a launch fills, the same launch clears.
// `slot0` = this output's slot of node 0, `stride` = elements between nodes.
// Returns true for the one split that ends with the total in v.
__device__ __forceinline__ bool pair_tree_sum(uint64_t* slot0, int64_t stride, int s, int S, float& v) {
    int c = s, n = S;
    int64_t node = 0;  // the level's first node
    while (n > 1) {
        if ((c ^ 1) < n) {
            uint64_t* p = slot0 + (node + (c >> 1)) * stride;
            const uint64_t old = __hip_atomic_exchange(p, (uint64_t(1) << 32) | __float_as_uint(v), __ATOMIC_RELAXED,
                                                       __HIP_MEMORY_SCOPE_AGENT);
            if (old == 0u) return false;
            const float o = __uint_as_float((uint32_t)old);
            v = (c & 1) ? o + v : v + o;
            __hip_atomic_store(p, uint64_t(0), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        node += n >> 1;
        c >>= 1;
        n = (n + 1) >> 1;
    }
    return true;
}

__device__ __forceinline__ uint64_t load_partial2(const float* p) {
    return __hip_atomic_load(reinterpret_cast<const uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float partial_lo(uint64_t v) { return __uint_as_float((uint32_t)v); }
__device__ __forceinline__ float partial_hi(uint64_t v) { return __uint_as_float((uint32_t)(v >> 32)); }

// Raw BF16 rows in the block layout (the raw twin): lane l, part p = row
// l % 16, columns 16 (4 (l / 16) + p) .. + 15, as two 16-byte loads.
__device__ __forceinline__ void load_raw_blocks(uint4 r[4][2], const uint16_t* wraw, int64_t K, int tr, int kt,
                                                uint32_t lane) {
    const uint16_t* p = wraw + ((int64_t)tr * kTileRows + (lane & 15u)) * K + (int64_t)kt * kTileCols + 64 * (lane >> 4);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        r[j][0] = reinterpret_cast<const uint4*>(p + 16 * j)[0];
        r[j][1] = reinterpret_cast<const uint4*>(p + 16 * j)[1];
    }
}

// Part p of a raw tile (fallback or bind-decoded; tile-local row-major) in
// the block layout.
__device__ __forceinline__ void raw_block_part(const int16_t* tile_raw, int p, uint32_t lane, uint32_t w[8]) {
    const uint4* q = reinterpret_cast<const uint4*>(tile_raw + (lane & 15u) * kTileCols + 64 * (lane >> 4) + 16 * p);
    const uint4 a = q[0], b = q[1];
    w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
    w[4] = b.x; w[5] = b.y; w[6] = b.z; w[7] = b.w;
}

// The block layout's first column of part p for a lane: 16 (4 (l / 16) + p).
__device__ __forceinline__ int block_layout_col(int p, uint32_t lane) { return 16 * (4 * (int)(lane >> 4) + p); }

// Sum over the 16 lanes of a DPP row; every lane of the row gets the sum.
__device__ __forceinline__ float row16_sum(float v) {
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, true));   // quad_perm 1,0,3,2
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, true));   // quad_perm 2,3,0,1
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x141, 0xF, 0xF, true));  // row_half_mirror
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x140, 0xF, 0xF, true));  // row_mirror
    return v;
}

// The half layout's loads of one tile for one lane: part p reads 8 bytes of
// `sm` and 4 of `ec` (512 / 256 contiguous bytes per wave instruction).
struct HalfTileLoads {
    uint2 sm[8];
    uint32_t ec[8];
};

__device__ __forceinline__ void load_tile_half(HalfTileLoads& t, const uint8_t* sm, const uint8_t* ec, int64_t tile,
                                               uint32_t lane) {
    const uint8_t* smt = sm + tile * kTile + 8u * lane;
    const uint8_t* ect = ec + tile * (kTile / 2) + 4u * lane;
#pragma unroll
    for (int p = 0; p < 8; ++p) {
        t.sm[p] = stream_load(reinterpret_cast<const uint2*>(smt + 512 * p));
        t.ec[p] = stream_load(reinterpret_cast<const uint32_t*>(ect + 256 * p));
    }
}

// The 32 pattern lookups of a tile in the half layout (pattern word 4 p + k
// in pat[p / 2][4 (p % 2) + k]).
__device__ __forceinline__ void lookup_tile_half(const uint32_t* lut, const HalfTileLoads& t, uint32_t pat[4][8]) {
#pragma unroll
    for (int p = 0; p < 8; ++p) {
        const uint32_t e = t.ec[p];
        uint32_t* q = &pat[p >> 1][4 * (p & 1)];
        q[0] = lut[e & 0xFFu];
        q[1] = lut[(e >> 8) & 0xFFu];
        q[2] = lut[(e >> 16) & 0xFFu];
        q[3] = lut[e >> 24];
    }
}

// The 4 BF16 pairs of part p of a tile in the half layout.
__device__ __forceinline__ void merge_part_half(const uint32_t pat[4][8], const HalfTileLoads& t, int p, uint32_t w[4]) {
    const uint32_t* q = &pat[p >> 1][4 * (p & 1)];
    w[0] = merge_pair(q[0], dup_lo(t.sm[p].x));
    w[1] = merge_pair(q[1], dup_hi(t.sm[p].x));
    w[2] = merge_pair(q[2], dup_lo(t.sm[p].y));
    w[3] = merge_pair(q[3], dup_hi(t.sm[p].y));
}

__device__ __forceinline__ float dot2_bf16(uint32_t w, uint32_t x, float acc) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w), __builtin_bit_cast(bf16x2_t, x), acc, false);
}

}  // namespace se12
