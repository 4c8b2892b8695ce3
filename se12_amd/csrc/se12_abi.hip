// C ABI of libse12_gfx950.so: handle management, argument validation, the
// default launch heuristic and the encoder orchestration. Kernels live in
// se12_gemv.hip, se12_decode.hip and se12_encode.hip.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "se12_gfx950.h"
#include "se12_step.h"
#include "se12_device.hpp"
#include "se12_internal.hpp"

using namespace se12;

static_assert(kMaxGroup == SE12_MAX_GROUP, "group size of the C ABI and the kernels");

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

#define SE12_HIP(call)                                                                        \
    do {                                                                                      \
        hipError_t e_ = (call);                                                               \
        if (e_ != hipSuccess) return fail(SE12_E_HIP, "%s: %s", #call, hipGetErrorString(e_)); \
    } while (0)

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
bool aligned8(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 7u) == 0; }

int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Restores the caller's current device on scope exit.
struct DeviceScope {
    int prev = -1;
    bool changed = false;
    hipError_t enter(int dev) {
        hipError_t e = hipGetDevice(&prev);
        if (e != hipSuccess) return e;
        if (prev != dev) {
            changed = true;
            return hipSetDevice(dev);
        }
        return hipSuccess;
    }
    ~DeviceScope() {
        if (changed) (void)hipSetDevice(prev);
    }
};

constexpr int32_t kMaxSplits = 64;
constexpr int32_t kStepNormMaxRows = 8192;  // se12_step_rmsnorm's hidden limit
constexpr size_t kSideBytes = 64;  // one side record per tile (16 dwords)

}  // namespace

struct se12_handle {
    int32_t format;
    int32_t device;
    int64_t N, K, Np, T;
    int32_t TR, TC;
    se12_streams s;
    const uint16_t* wraw;
    uint32_t* info;      // [T] per-tile sidecar word (bind time only)
    uint4* escpos;       // [T] listed escape positions (bind time only)
    uint32_t* side;      // [T, 16] per-tile side records read by the kernels
    int16_t* ovf_raw;    // tiles with more than the listed escapes, decoded at bind
    int64_t n_overflow;
    uint32_t* lut;       // [256] pair table
    int64_t n_fallback;
    float* partial;
    int64_t partial_elems;
    int32_t* counters;
    uint64_t* pairs;     // [s_cap - 1, 4, Np] dot2 split-K pair slots (zero between launches)
    int64_t pair_elems;
    int32_t max_batch;
    int32_t s_cap;
    int32_t cu_count;
    int64_t lds_per_block;
};

extern "C" {

const char* se12_last_error(void) { return g_last_error.c_str(); }

const char* se12_version(void) {
    return "se12_gfx950 1 (gfx950, wave64, dot2-bf16 fused decode+GEMV, " __VERSION__ ")";
}

int se12_device_info_get(int32_t device, se12_device_info* out) {
    if (!out) return fail(SE12_E_INVALID, "se12_device_info_get: out is NULL");
    hipDeviceProp_t p;
    SE12_HIP(hipGetDeviceProperties(&p, device));
    std::memset(out, 0, sizeof *out);
    std::snprintf(out->name, sizeof out->name, "%s", p.name);
    std::snprintf(out->arch, sizeof out->arch, "%s", p.gcnArchName);
    out->compute_units = p.multiProcessorCount;
    out->wavefront_size = p.warpSize;
    out->l2_bytes = p.l2CacheSize;
    out->lds_bytes_per_cu = (int64_t)p.maxSharedMemoryPerMultiProcessor;
    out->lds_bytes_per_block = (int64_t)p.sharedMemPerBlock;
    out->total_memory_bytes = (int64_t)p.totalGlobalMem;
    out->clock_khz = p.clockRate;
    out->memory_clock_khz = p.memoryClockRate;
    out->memory_bus_width_bits = p.memoryBusWidth;
    out->max_threads_per_block = p.maxThreadsPerBlock;
    out->pci_domain_id = p.pciDomainID;
    out->pci_bus_id = p.pciBusID;
    out->pci_device_id = p.pciDeviceID;
    out->ecc_enabled = p.ECCEnabled;
    out->kernel_timeout = p.kernelExecTimeoutEnabled;
    int v = 0;
    SE12_HIP(hipRuntimeGetVersion(&v));
    out->runtime_version = v;
    v = 0;
    SE12_HIP(hipDriverGetVersion(&v));
    out->driver_version = v;
    return SE12_OK;
}

static int bind_common(se12_handle* h, int64_t rows, int64_t cols, int32_t max_batch) {
    h->N = rows;
    h->K = cols;
    h->TR = (int32_t)ceil_div(rows, SE12_TILE_ROWS);
    h->TC = (int32_t)ceil_div(cols, SE12_TILE_COLS);
    h->Np = (int64_t)h->TR * SE12_TILE_ROWS;
    h->T = (int64_t)h->TR * h->TC;
    h->max_batch = max_batch;
    h->s_cap = std::min<int32_t>(h->TC, kMaxSplits);
    SE12_HIP(hipGetDevice(&h->device));
    hipDeviceProp_t p;
    SE12_HIP(hipGetDeviceProperties(&p, h->device));
    h->cu_count = p.multiProcessorCount;
    h->lds_per_block = (int64_t)p.sharedMemPerBlock;
    // split-K workspace: S x (rows per launch) x Np floats, for the dot2
    // path (up to 4 rows per launch, any split count) and the MFMA path (all
    // rows in one launch, at most kGemmMaxSplits splits)
    if (h->s_cap > 1) {
        int64_t pe = (int64_t)h->s_cap * std::min<int32_t>(max_batch, kGemvMaxBatchPerLaunch);
        if (max_batch >= kGemmMinBatch) pe = std::max<int64_t>(pe, (int64_t)std::min(h->s_cap, kGemmMaxSplits) * max_batch);
        h->partial_elems = pe * h->Np;
        SE12_HIP(hipMalloc(&h->partial, (size_t)h->partial_elems * sizeof(float)));
        // the dot2 kernel's pair slots: S - 1 per output, zero between launches
        h->pair_elems = (int64_t)(h->s_cap - 1) * std::min<int32_t>(max_batch, kGemvMaxBatchPerLaunch) * h->Np;
        SE12_HIP(hipMalloc(&h->pairs, (size_t)h->pair_elems * sizeof(uint64_t)));
        SE12_HIP(hipMemset(h->pairs, 0, (size_t)h->pair_elems * sizeof(uint64_t)));
    }
    // arrival counters: split-K per tile row and the fused step tails'
    const size_t counter_bytes = (size_t)gemv_counter_count(h->TR) * sizeof(int32_t);
    SE12_HIP(hipMalloc(&h->counters, counter_bytes));
    SE12_HIP(hipMemset(h->counters, 0, counter_bytes));
    return SE12_OK;
}

static void free_handle(se12_handle* h) {
    if (!h) return;
    if (h->info) (void)hipFree(h->info);
    if (h->escpos) (void)hipFree(h->escpos);
    if (h->side) (void)hipFree(h->side);
    if (h->ovf_raw) (void)hipFree(h->ovf_raw);
    if (h->lut) (void)hipFree(h->lut);
    if (h->partial) (void)hipFree(h->partial);
    if (h->counters) (void)hipFree(h->counters);
    if (h->pairs) (void)hipFree(h->pairs);
    delete h;
}

static int check_shape(int64_t rows, int64_t cols, int32_t max_batch) {
    if (rows <= 0 || cols <= 0) return fail(SE12_E_INVALID, "shape must be positive, got [%lld, %lld]", (long long)rows, (long long)cols);
    // tile rows index the grid's x dimension; K-tile bounds are computed in
    // 32 bits as split * tile_cols; the decode kernel indexes tiles in 32 bits
    if (ceil_div(rows, SE12_TILE_ROWS) > INT32_MAX / 2 || ceil_div(cols, SE12_TILE_COLS) > (1 << 25) ||
        ceil_div(rows, SE12_TILE_ROWS) * ceil_div(cols, SE12_TILE_COLS) > INT32_MAX)
        return fail(SE12_E_INVALID, "shape [%lld, %lld] too large", (long long)rows, (long long)cols);
    if (max_batch < 1 || max_batch > SE12_MAX_BATCH)
        return fail(SE12_E_INVALID, "max_batch must be in [1, %d], got %d", SE12_MAX_BATCH, max_batch);
    return SE12_OK;
}

static DecodeArgs decode_args(const se12_handle* h, uint16_t* out);

int se12_bind(const se12_streams* s, int64_t rows, int64_t cols, int32_t max_batch, void* stream,
              se12_handle** out) {
    if (!s || !out) return fail(SE12_E_INVALID, "se12_bind: NULL argument");
    *out = nullptr;
    if (int rc = check_shape(rows, cols, max_batch)) return rc;
    if (!s->sm_dev || !s->ec_dev || !s->esc_dev || !s->codebook_dev || !s->fallback_bitmap_dev)
        return fail(SE12_E_INVALID, "se12_bind: a required stream pointer is NULL");
    if (!aligned16(s->sm_dev) || !aligned16(s->ec_dev) || !aligned16(s->esc_dev) ||
        (s->fallback_raw_dev && !aligned16(s->fallback_raw_dev)))
        return fail(SE12_E_INVALID, "se12_bind: sm/ec/esc/fallback_raw must be 16-byte aligned");
    if (s->fallback_raw_elems < 0 || s->fallback_raw_elems % SE12_TILE_SIZE != 0)
        return fail(SE12_E_INVALID, "se12_bind: fallback_raw has %lld elements, not a whole number of tiles",
                    (long long)s->fallback_raw_elems);
    if (s->fallback_raw_elems > 0 && !s->fallback_raw_dev)
        return fail(SE12_E_INVALID, "se12_bind: fallback_raw is NULL but has elements");
    se12_handle* h = new se12_handle();
    std::memset(h, 0, sizeof *h);
    h->format = SE12_FORMAT_SE12;
    h->s = *s;
    if (int rc = bind_common(h, rows, cols, max_batch)) {
        free_handle(h);
        return rc;
    }
    hipStream_t st = static_cast<hipStream_t>(stream);
    int64_t* total_dev = nullptr;
    int64_t totals[2] = {0, 0};  // fallback tiles, tiles with more than the listed escapes
    uint8_t cb[SE12_CODEBOOK_SIZE] = {0};
    uint32_t lut[256];
    hipError_t e = hipMalloc(&h->info, (size_t)h->T * sizeof(uint32_t));
    if (e == hipSuccess) e = hipMalloc(&h->escpos, (size_t)h->T * sizeof(uint4));
    if (e == hipSuccess) e = hipMemsetAsync(h->escpos, 0, (size_t)h->T * sizeof(uint4), st);
    if (e == hipSuccess) e = hipMalloc(&h->side, (size_t)h->T * kSideBytes);
    if (e == hipSuccess) e = hipMalloc(&h->lut, sizeof lut);
    if (e == hipSuccess) e = hipMalloc(&total_dev, sizeof totals);
    if (e == hipSuccess) e = hipMemsetAsync(total_dev, 0, sizeof totals, st);
    if (e == hipSuccess) e = launch_tile_info(s->fallback_bitmap_dev, s->ec_dev, h->T, h->info, h->escpos, total_dev, st);
    if (e == hipSuccess) e = launch_side_records(h->info, s->esc_dev, h->escpos, h->T, h->side, st);
    if (e == hipSuccess) e = hipMemcpyAsync(totals, total_dev, sizeof totals, hipMemcpyDeviceToHost, st);
    if (e == hipSuccess) e = hipMemcpyAsync(cb, s->codebook_dev, sizeof cb, hipMemcpyDeviceToHost, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (e == hipSuccess) {
        for (uint32_t b = 0; b < 256; ++b) lut[b] = pair_lut_entry(cb, b);
        e = hipMemcpyAsync(h->lut, lut, sizeof lut, hipMemcpyHostToDevice, st);
    }
    // tiles with more escapes than the sidecar lists are decoded once here and
    // read as raw tiles by every kernel
    if (e == hipSuccess && totals[1] > 0) {
        e = hipMalloc(&h->ovf_raw, (size_t)totals[1] * SE12_TILE_SIZE * sizeof(int16_t));
        if (e == hipSuccess) e = launch_overflow_decode(decode_args(h, nullptr), h->ovf_raw, st);
    }
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (total_dev) (void)hipFree(total_dev);
    // the side records hold everything the kernels read
    if (e == hipSuccess) {
        (void)hipFree(h->info);
        (void)hipFree(h->escpos);
        h->info = nullptr;
        h->escpos = nullptr;
    }
    if (e != hipSuccess) {
        free_handle(h);
        return fail(SE12_E_HIP, "se12_bind: %s", hipGetErrorString(e));
    }
    if (totals[0] * SE12_TILE_SIZE != s->fallback_raw_elems) {
        free_handle(h);
        return fail(SE12_E_INVALID, "se12_bind: bitmap marks %lld fallback tiles but fallback_raw holds %lld elements",
                    (long long)totals[0], (long long)s->fallback_raw_elems);
    }
    h->n_fallback = totals[0];
    h->n_overflow = totals[1];
    *out = h;
    return SE12_OK;
}

int se12_bind_raw_bf16(const uint16_t* w, int64_t rows, int64_t cols, int32_t max_batch, void* stream,
                       se12_handle** out) {
    (void)stream;
    if (!w || !out) return fail(SE12_E_INVALID, "se12_bind_raw_bf16: NULL argument");
    *out = nullptr;
    if (int rc = check_shape(rows, cols, max_batch)) return rc;
    se12_handle* h = new se12_handle();
    std::memset(h, 0, sizeof *h);
    h->format = SE12_FORMAT_RAW_BF16;
    h->wraw = w;
    if (int rc = bind_common(h, rows, cols, max_batch)) {
        free_handle(h);
        return rc;
    }
    *out = h;
    return SE12_OK;
}

int se12_release(se12_handle* h) {
    if (!h) return SE12_OK;
    DeviceScope ds;
    if (ds.enter(h->device) == hipSuccess) (void)hipDeviceSynchronize();
    free_handle(h);
    return SE12_OK;
}

int se12_handle_bind_stats(const se12_handle* h, int64_t* raw_tiles, int64_t* sidecar_bytes) {
    if (!h) return fail(SE12_E_INVALID, "se12_handle_bind_stats: NULL handle");
    const bool se12 = h->side != nullptr;   // a raw-twin handle derives nothing
    if (raw_tiles) *raw_tiles = se12 ? h->n_overflow : 0;
    if (sidecar_bytes)
        *sidecar_bytes = se12 ? h->T * (int64_t)(se12::kSideWords * sizeof(uint32_t)) + (int64_t)kLutBytes +
                                    h->n_overflow * SE12_TILE_SIZE * (int64_t)sizeof(int16_t)
                              : 0;
    return SE12_OK;
}

int se12_handle_shape(const se12_handle* h, int64_t* rows, int64_t* cols, int64_t* tiles, int64_t* fallback_tiles,
                      int32_t* format) {
    if (!h) return fail(SE12_E_INVALID, "se12_handle_shape: NULL handle");
    if (rows) *rows = h->N;
    if (cols) *cols = h->K;
    if (tiles) *tiles = h->T;
    if (fallback_tiles) *fallback_tiles = h->n_fallback;
    if (format) *format = h->format;
    return SE12_OK;
}

// Largest block (threads) a launch at batch `bl` may use: the lightest
// kernel variant (one tile per round, no prefetch) of the fused kernel and of
// its raw twin must fit its VGPR budget.
// BF16 activations with kGemmMinBatch or more rows take the MFMA kernel (one
// launch, one pass over the weights); FP32 activations and smaller batches
// the dot2 kernel, 4 rows per launch.
static bool uses_mfma(int32_t batch, bool xf32) { return !xf32 && batch >= kGemmMinBatch; }
static bool rx_fits(se12_handle* const* hs, int32_t count, int32_t batch);
static void rx_default_launch(se12_handle* const* hs, int32_t count, int32_t batch, int32_t* waves_out,
                              int32_t* blocks_out);

static int max_threads_for(int32_t bl, bool xf32, bool generic) {
    return std::min(gemv_max_threads(bl, xf32, false, 1, 0, generic), gemv_max_threads(bl, xf32, true, 1, 0, generic));
}

// The default launch, re-derived for MI355X (256 CUs in 8 XCDs, wave64) from
// sweeps of every (waves, splits) pair on cold data at the Gemma-2 2B/9B/27B
// shapes, the grouped q/k/v and gate/up shapes and the LM heads. A batch-1
// GEMV is one pass over the streams. What pays: enough tiles in flight per
// CU to cover HBM latency but not so many that every wave's data lands at
// the end of the pass (the decode would then all run after the last byte
// arrives). K splits meet in the pair tree (one exchange round trip per
// level at the end of a block), which pays where a launch has too few tile
// rows to spread 2-4 batch rows' decode over the CUs. By tiles per CU
// (T / CUs), for rows of at most 32 tiles:
//  - fewer tile rows than CUs, or at most 10 tiles per CU: one wave per K
//    tile (rows longer than 16 tiles: 8 waves streaming with prefetch);
//  - up to 32 tiles per CU: 3 waves; up to 64: about 2 tiles per wave;
//    more (very tall matrices such as an LM head): 6 waves;
// rows longer than 32 tiles on many tile rows: 8 waves and splits of ~36
// tiles; very long rows on very few tile rows are split so that every CU
// gets a block. At batch 1, 3 to 8 tile rows per CU on rows of up to 18
// tiles take one wave per block (a block per tile row, streaming its row
// with prefetch), except under a fused norm head (`head`), whose x rebuild
// wants the block's threads, and in the edge-handling variants, which do
// not prefetch.
static void default_launch(int64_t tr, int64_t tc, int32_t cu_count, int32_t s_cap, int32_t batch, bool xf32,
                           bool generic, bool head, int32_t* waves_out, int32_t* splits_out) {
    const int32_t bl = std::min<int32_t>(batch, kGemvMaxBatchPerLaunch);
    const int64_t mw = max_threads_for(bl, xf32, generic) / 64;
    const int64_t cus = std::max<int32_t>(1, cu_count);
    const int64_t tiles = tr * tc;
    int64_t waves, splits = 1;
    if (!head && !generic && bl == 1 && tr >= 3 * cus && tr <= 8 * cus && tc <= 18) {
        // 2B gate/up grouped (1152 x 9 tiles) 12.45 us against 13.06 with 5
        // waves, 9B gate/up grouped (1792 x 14) 25.7 against 27.4 with 8, 9B
        // gate (896 x 14) 14.55 against 14.7 with 2; 27B gate (2304 x 18, 9
        // rows per CU) keeps 8 (41.1 against 41.7), the LM heads 6 (256000 x
        // 2304: 132.9 either way; 256000x3584: 195-200 against 210)
        waves = 1;
    } else if (tr < cus) {
        // one wave per K tile up to 9 (Gemma-2 2B), else 8 (2048x3584: 5.4 us
        // against 14 waves' slower launch; 3584x4096: 6.3 against 7.4 with
        // 16), 4 at 4 rows per launch (3584x4096 7.7-8.0 against 8.1,
        // 3584x14336 16.7 against 17.0 with 8). Rows of 17-48 K tiles on at
        // most two thirds of the CUs' worth of tile rows take 3 splits of 4
        // waves at 2-4 rows per launch (2304x9216 B = 2 / 3 / 4: 8.8 / 9.6 /
        // 10.3 us against 9.2 / 10.35 / 11.1 unsplit; B = 1 8.3 either way).
        // (Rows of 9 K tiles on a quarter of the CUs' tile rows, Gemma-2 2B
        // k/v alone, measured 4.13 us against 4.47 with 3 splits of 3 waves
        // in a rotation of 300 back-to-back launches, but 4.65 against 4.50
        // in 26 launches after an eviction, so they stay unsplit.)
        waves = tc <= 9 ? tc : (bl >= 4 ? 4 : 8);
        if (tc > 64 && tr * 2 <= cus) splits = std::min<int64_t>(ceil_div(cus, tr), ceil_div(tc, 16));
        if (bl >= 2 && tc > 16 && tc <= 48 && tr * 3 <= cus * 2) {
            waves = 4;
            splits = 3;
        }
    } else if (tc > 32) {
        // long rows on many tile rows (4608x36864): one wave per block and
        // splits of ~24 K tiles (B = 1, heavy-tailed weights: 42.4 us
        // against 43.4 with 4 splits of ~36 and 42.6 with 4 waves x 6;
        // Gaussian weights 42.1-42.5 either way; B = 2 / 3 / 4: 43.0 / 44.0
        // / 46.9 against 43.5 / 45.1 / 47.7 with 3 splits)
        waves = 1;
        splits = std::max<int64_t>(1, (tc + 18) / 36) * 3 / 2;
    } else if (tiles <= 10 * cus) {
        // one wave per K tile; at 4 rows per launch 3 splits of 3 waves for
        // rows of 9 K tiles (2B q/k/v grouped, 256 x 9 tiles: 7.5 us against
        // 7.75 with 8 waves; at 1-3 rows 9 waves stay best)
        waves = std::min<int64_t>(16, tc);
        if (bl >= 4 && tc == 9) {
            waves = 3;
            splits = 3;
        }
    } else if (tiles <= 32 * cus) {
        // 3 waves for 9 K tiles (9216x2304), 3 splits of them at 2-4 rows
        // per launch (B = 2 / 3 / 4: 8.6 / 9.2 / 9.8 us against 8.8 / 9.6 /
        // 10.4 unsplit); longer rows 8 waves at 1..2 rows per launch when
        // the tile rows fill the CUs evenly (4096x3584: 6.3 us against 7.2
        // with 3; 4096x4608: 7.3 against 8.3; 9B q/k/v grouped, 512 tile
        // rows: 9.6 against 10.0 with 2), 4 where some CUs take two blocks
        // and others one (4608x4096: 8.6 against 9.0 with 8) and at 3..4
        // rows (7.95 / 9.0 against 8.2 / 9.2)
        if (tc == 9 && bl >= 2) {
            waves = 3;
            splits = 3;
        } else {
            waves = tc <= 9 ? (bl >= 4 ? 2 : 3) : (bl >= 3 || (tr > cus && tr % cus != 0) ? 4 : 8);
        }
        waves = std::min<int64_t>(waves, tc);
    } else if (tiles <= 64 * cus) {
        // 3..4 rows per launch: 1 wave (14336x3584, B = 3 / 4: 15.5 / 16.4
        // us against 16.0 / 17.1 with 2), 2B gate/up grouped at 4 rows 3
        // (15.1 against 15.6); 2 rows: 1 wave where the tile rows give each
        // CU 3+ blocks (14336x3584 14.9 against 15.4 with 2; 2B gate/up
        // grouped 13.2 against 13.8 with 3), else 2 (27B q/k/v grouped, 512
        // tile rows: 13.6 against 16.5 with 1); one row on fewer than 3 tile
        // rows per CU: two tiles per wave for an odd count, 8 waves for an
        // even one (27B q/k/v grouped: 11.4 against 12.0 with 2)
        if (bl >= 3)
            waves = bl >= 4 && tc == 9 ? 3 : 1;
        else if (bl == 2)
            waves = tr >= 3 * cus ? 1 : 2;
        else
            waves = tc % 2 == 1 ? (tc + 1) / 2 : (tr >= 3 * cus ? 2 : 8);
        waves = std::max<int64_t>(1, std::min<int64_t>(tc, waves));
    } else {
        // many tiles per CU: short rows (256000x2304) take 4 waves at B = 1
        // (heavy-tailed weights 133.5 us against 139.4 with 6, Gaussian 130.9
        // against 132.9) and 2 (129.9 against 132.4 with 3), 3 at B = 3..4
        // (B = 4: 154 against 209 with 6); rows over 12 K tiles 8 waves
        // (36864x4608 B = 1: 41.1 us against 41.5 with 6; 256000x3584: 200
        // against 210 with 1), 4 at B = 2 (256000x3584: 198.5 against 202
        // with 8), at B = 3..4 on 256+ tiles per CU 2 (256000x3584 B = 4:
        // 231 against 258 with 8)
        if (bl == 2 || (bl == 1 && tc <= 12))
            waves = 4;
        else if (tc <= 12)
            waves = 3;
        else
            waves = bl >= 3 && tiles >= 256 * cus ? 2 : 8;
        waves = std::min<int64_t>(waves, tc);
    }
    waves = std::max<int64_t>(1, std::min(waves, mw));
    *waves_out = (int32_t)waves;
    *splits_out = (int32_t)std::max<int64_t>(1, std::min<int64_t>(splits, s_cap));
}

// Row blocks of the MFMA grid: ceil(tile rows / rows per block) per matrix.
static int64_t gemm_row_blocks(se12_handle* const* hs, int32_t count, int32_t rows) {
    int64_t rb = 0;
    for (int32_t i = 0; i < count; ++i) rb += ceil_div(hs[i]->TR, rows);
    return rb;
}

// Default launch of the x-slab MFMA kernel: rows per block fixed by the
// batch (R = the fewest waves whose threads load an x slab, batch / 8
// rounded up, 4 in place of 3); then m waves of K parallelism per tile row, m = 1 on
// matrices of 2 or more tile rows per CU, else about 3.4 waves per CU in
// all (864 on 256 CUs) and at least one per 24 K tiles; split between K
// groups (up to 6 with one row per block, 2 with more, 2+ K tiles per wave)
// and K splits (3+ K tiles per wave, at most 16) so that the blocks spread
// most evenly over the CUs (the fewest blocks on the busiest CU relative to
// the mean), then closest to m, then more K groups. Sweeps on MI355X:
// 4608x36864 B = 8/16/32 (1, 6) 64.2 / (4, 3) 70.9 / (8, 3) 74.9 us against
// 88.0 / 95.3 / 99.5 for the previous rule (K groups first), 3584x14336
// B = 32 (4, 4) 34.4 against 46.2, 4096x3584 B = 32 (4, 3) 19.7 against
// 21.8, 4608x4096 B = 8 (1, 3) 14.8 against 16.2, 9216x2304 B = 8 (1, 1)
// 13.2 against 14.1; 2304x9216 B = 8 (2, 3) 17.1 against 16.8.
static void gemm_default_launch(se12_handle* const* hs, int32_t count, int32_t batch, bool generic, int32_t* waves_out,
                                int32_t* splits_out) {
    const se12_handle* h0 = hs[0];
    int64_t tr = 0;
    for (int32_t i = 0; i < count; ++i) tr += hs[i]->TR;
    const int64_t cus = std::max<int32_t>(1, h0->cu_count);
    const int64_t rows = gemm_min_waves(batch);
    const int64_t row_blocks = gemm_row_blocks(hs, count, (int32_t)rows);
    const int64_t target = 27 * cus / 8;
    const int64_t m =
        tr >= 2 * cus ? 1 : std::max<int64_t>({1, (2 * target + tr) / (2 * tr), ceil_div(h0->TC, 24)});
    const int64_t max_waves = (generic ? kGemmMaxThreadsGeneric : kGemmMaxThreads) / 64;
    const int64_t kg_max = std::max<int64_t>(1, std::min<int64_t>({max_waves / rows, rows == 1 ? 6 : 2, h0->TC / 2}));
    int64_t best_kg = 1, best_s = 1, best_dev = 0;
    double best_imb = 0.0;
    for (int64_t kg = 1; kg <= kg_max; ++kg) {
        const int64_t cap = std::max<int64_t>(1, std::min<int64_t>({(int64_t)kGemmMaxSplits, (int64_t)h0->s_cap,
                                                                   h0->TC / (3 * kg)}));
        const int64_t s = std::max<int64_t>(1, std::min<int64_t>(cap, (2 * m + kg) / (2 * kg)));
        const int64_t blocks = row_blocks * s;
        const double imb = (double)ceil_div(blocks, cus) * (double)cus / (double)blocks;
        const int64_t dev = std::abs(kg * s - m);
        if (kg == 1 || imb < best_imb - 1e-9 || (imb < best_imb + 1e-9 && dev <= best_dev)) {
            best_kg = kg;
            best_s = s;
            best_imb = imb;
            best_dev = dev;
        }
    }
    // one tile row per block on few rows of 32-48 K tiles (2304x9216 and
    // 2048x9216 at 5..8 batch rows): one-wave blocks and splits of ~6 K
    // tiles, no K groups (2304x9216 B = 5 / 6 / 8: 13.6 / 13.7 / 13.8 us
    // against 15.2 / 15.2 / 15.3 with 2 K groups x 3 splits; 2048x9216 B = 8
    // 13.4 against 13.8 with 4 x 2); longer rows keep the rule above
    // (3584x14336 B = 8: 25.0 us with 4 K groups against 30.5 with 10 splits)
    if (rows == 1 && m > 1 && h0->TC >= 32 && h0->TC <= 48) {
        best_kg = 1;
        best_s = std::max<int64_t>(1, std::min<int64_t>({(int64_t)kGemmMaxSplits, (int64_t)h0->s_cap,
                                                         ceil_div(h0->TC, 6)}));
    }
    *waves_out = (int32_t)(rows * best_kg);
    *splits_out = (int32_t)best_s;
}

int se12_read_probe(const void* buf_dev, int64_t bytes, uint32_t* out_dev, int64_t out_elems, void* stream) {
    if (!buf_dev || !out_dev) return fail(SE12_E_INVALID, "se12_read_probe: NULL argument");
    if (bytes < 16 || !aligned16(buf_dev))
        return fail(SE12_E_INVALID, "se12_read_probe: needs a 16-byte aligned buffer of at least 16 bytes");
    int dev = 0, cus = 0;
    SE12_HIP(hipGetDevice(&dev));
    SE12_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    const int64_t blocks = read_probe_blocks(cus);
    if (out_elems < blocks)
        return fail(SE12_E_CAPACITY, "se12_read_probe: out holds %lld words, the grid needs %lld", (long long)out_elems,
                    (long long)blocks);
    SE12_HIP(launch_read_probe(buf_dev, bytes / 16, out_dev, blocks, static_cast<hipStream_t>(stream)));
    return SE12_OK;
}

int se12_set_compute_units(se12_handle* h, int32_t compute_units) {
    if (!h) return fail(SE12_E_INVALID, "se12_set_compute_units: NULL handle");
    if (compute_units < 1 || compute_units > (1 << 16))
        return fail(SE12_E_INVALID, "se12_set_compute_units: %d compute units", compute_units);
    h->cu_count = compute_units;
    return SE12_OK;
}

int se12_default_launch(const se12_handle* h, int32_t batch, se12_launch* out) {
    if (!h || !out) return fail(SE12_E_INVALID, "se12_default_launch: NULL argument");
    if (batch < 1 || batch > SE12_MAX_BATCH) return fail(SE12_E_INVALID, "batch must be in [1, %d]", SE12_MAX_BATCH);
    int32_t waves, splits;
    const bool generic = h->K % SE12_TILE_COLS != 0 ||
                         (h->format == SE12_FORMAT_RAW_BF16 && h->N % SE12_TILE_ROWS != 0);
    se12_handle* hs[1] = {const_cast<se12_handle*>(h)};
    if (uses_mfma(batch, false) && !generic && rx_fits(hs, 1, batch)) {
        int32_t blocks;
        rx_default_launch(hs, 1, batch, &waves, &blocks);
        out->threads_per_block = waves * 64;
        out->blocks = blocks;
        return SE12_OK;
    }
    if (uses_mfma(batch, false)) {
        gemm_default_launch(hs, 1, batch, generic, &waves, &splits);
        out->threads_per_block = waves * 64;
        out->blocks = (int32_t)(gemm_row_blocks(hs, 1, gemm_min_waves(batch)) * splits);
        return SE12_OK;
    }
    default_launch(h->TR, h->TC, h->cu_count, h->s_cap, batch, false, generic, false, &waves, &splits);
    out->threads_per_block = waves * 64;
    out->blocks = h->TR * splits;
    return SE12_OK;
}

// Picks the kernel variant for a launch shape: a wave that owns 4 or more
// tiles streams them with the next tile's loads in flight (PF) when the
// block's register budget allows; otherwise it takes one tile per round.
static GemvPlan plan_gemv(int64_t tr, int64_t tc, bool raw, int32_t bl, bool xf32, bool generic, int32_t waves,
                          int32_t splits) {
    GemvPlan p{};
    p.batch = bl;
    p.xf32 = xf32;
    p.raw = raw;
    p.generic = generic;
    p.waves = waves;
    p.blocks = (int32_t)(tr * splits);
    p.lds = gemv_lds_bytes(waves, bl);
    p.g = 1;
    const int64_t per_wave = ceil_div(ceil_div(tc, splits), waves);
    p.pf = (!generic && per_wave >= 4 && waves * 64 <= gemv_max_threads(bl, xf32, p.raw, 1, 1, false)) ? 1 : 0;
    return p;
}

static GemvPlan plan_gemm(int64_t row_blocks, bool raw, int32_t batch, bool generic, int32_t waves, int32_t splits,
                          int32_t tile_cols, int64_t lds_per_block) {
    GemvPlan p{};
    p.batch = batch;
    p.raw = raw;
    p.generic = generic;
    p.waves = waves;
    p.blocks = (int32_t)(row_blocks * splits);
    // steps of a wave: its K group's share of the split's K tiles
    const int32_t kgroups = std::max(1, waves / gemm_min_waves(batch));
    const int64_t steps = ceil_div(ceil_div(tile_cols, splits), kgroups);
    p.slab_ring = !generic && steps >= kGemmSlabRingMinSteps &&
                          (int64_t)(gemm_lds_bytes(waves, batch, kGemmSlabRing) + kLutBytes) <= lds_per_block
                      ? kGemmSlabRing
                      : 0;
    p.lds = gemm_lds_bytes(waves, batch, p.slab_ring);
    p.g = 1;
    p.pf = 1;
    return p;
}

// The launches of one product over `count` handles that share x (a single
// matrix for se12_gemv, up to kMaxGroup for se12_gemv_grouped): one MFMA
// launch for all rows, or one dot2 launch per 4 rows.
// The resident-x batched kernel serves every FAST MFMA launch (BF16 x with
// kGemmMinBatch or more rows) whose x fits a block's LDS beside the pair
// table, on matrices of whole tile rows (both formats alike, so that a fused
// kernel and its raw twin always run the same kernel and stay bit-identical).
// Since its waits and launch were refitted it beats the x-slab kernel at 5-8
// rows too (default launches, cold: 9216x4096 B = 5 18.5 against 21.0 us,
// 2304x2304 8.5 against 10.2, 3584x14336 22.6 against 24.3, 14336x3584 B = 8
// 20.3 against 20.4), except on few tile rows of long rows (below). With
// 17..32 rows whose x does not fit but 16 rows do
// (K = 3584..4608), on matrices of at most one tile row per CU, LDS holds the
// first 16 rows and batch group 1's operands come from global memory
// (4096x3584 B = 24 / 32: 13.6 / 14.7 us against the x-slab kernel's 18.8 /
// 19.5; 3584x4096 B = 20 / 32: 13.6 / 15.9 against 19.1 / 20.2; on taller
// matrices it lost at 32 rows: 14336x3584 33.5 against 27.3, 36864x4608 85.2
// against 80.5). Otherwise the launch is split along K: split s of S takes
// K tiles [s TC / S, (s + 1) TC / S) of every row and holds only their
// columns of x, with the fewest splits (at most kGemmMaxSplits) whose share
// fits; the splits' partial sums meet per row through device memory.
// `staged` = the rows of x the kernel keeps in LDS, `splits` = K splits;
// staged 0 where the x-slab kernel serves the launch.
struct RxLayout {
    int32_t staged, splits;
};

static RxLayout rx_layout(se12_handle* const* hs, int32_t count, int32_t batch) {
    int64_t rows = 0;
    for (int32_t i = 0; i < count; ++i) {
        if (hs[i]->N % SE12_TILE_ROWS != 0) return {0, 0};
        rows += hs[i]->TR;
    }
    const int64_t lds = hs[0]->lds_per_block;
    const int64_t cus = std::max<int32_t>(1, hs[0]->cu_count);
    if ((int64_t)(rx_lds_bytes(hs[0]->K, batch) + kLutBytes) <= lds) {
        // rows of 32+ K tiles on at most 5/8 of the CUs' worth of tile rows:
        // one resident-x block per tile row leaves CUs idle where the x-slab
        // kernel's K splits reach them all (2304x9216 B = 5 / 6 / 7 / 8: 15.0
        // / 14.9 / 15.0 / 15.1 us against 15.2 / 15.6 / 15.9 / 16.2; 2048x9216
        // B = 8: 13.9 against 16.4; with more rows or shorter ones the
        // resident-x kernel stays ahead: 3584x14336 B = 5 21.5 against 23.6,
        // 2304x6144 B = 8 11.9 against 12.4)
        if (rows * 8 <= cus * 5 && hs[0]->TC >= 32) return {0, 0};
        return {batch, 1};
    }
    if (batch > 16 && (int64_t)(rx_lds_bytes(hs[0]->K, 16) + kLutBytes) <= lds &&
        rows <= cus)
        return {16, 1};
    const int32_t tc = hs[0]->TC;
    int32_t sp = 2;
    while (sp <= std::min<int32_t>(kRxMaxSplits, tc) &&
           (int64_t)(rx_lds_bytes(ceil_div(tc, sp) * SE12_TILE_COLS, batch) + kLutBytes) > lds)
        ++sp;
    if (sp > std::min<int32_t>(kRxMaxSplits, tc)) return {0, 0};
    // what measured faster than the x-slab kernel: single matrices; two
    // splits at one batch group only on 8192+ tiles (3584x14336 B = 6 / 8 /
    // 11: 23.9 / 23.8 / 24.6 us against 24.5 / 24.3 / 26.1; 4096x14336 24.5-
    // 25.5 / 24.4-24.7 / 24.8-25.0 against 28.5 / 27.8-27.9 / 25.9-26.1;
    // 4608x9216 B = 9 / 12 / 16 22.1-22.7 / 22.5-22.6 / 22.9-23.1 against
    // 24.0-24.1 / 24.0 / 23.8; but 2304x9216 B = 9..16 17.6-18.3 against
    // 15.0-15.3), at two batch groups on every size (14336x3584
    // B = 24 / 32: 24.4 / 25.0-26.0 against 25.4-26.1 / 25.5-26.3; 8192x4096
    // 18.9-19.2 / 19.3-19.8 against 25.4-25.9; 6144x4096 17.3 / 17.8 against
    // 19.8 / 20.0; 4608x4096 16.0 / 16.7 against 17.2 / 17.5), the x-slab
    // launch leaving CUs idle there (4 tile rows per block)
    if (count > 1 || (sp == 2 && batch <= 16 && rows * tc < 8192)) return {0, 0};
    return {batch, sp};
}

static bool rx_fits(se12_handle* const* hs, int32_t count, int32_t batch) {
    return rx_layout(hs, count, batch).staged > 0;
}

static int64_t rx_max_blocks(se12_handle* const* hs, int32_t count) {
    int64_t tr = 1;
    for (int32_t i = 0; i < count; ++i) tr = std::max<int64_t>(tr, hs[i]->TR);
    return tr;
}

// Default launch of the resident-x kernel: one block per CU (fewer where a
// matrix has fewer tile rows than its share of the CUs) of 12 waves (3 per
// SIMD, the kernel's register limit) up to 2 tile rows per CU, 8 waves up to
// 3 and, up to 16 batch rows, 12 up to 4 (one K group: the idle waves speed
// the copy of x; 14336x3584 B = 16 20.7 us against 21.4 with 6) and 6 waves
// up to 16, which with the K groups (rx_kgroups) keeps about 4 waves per CU
// on rows, each on more tiles
// (14336x3584, 3.5 rows per CU, B = 9 / 16: 20.0 / 21.5 us with 6 waves
// against 21.6 / 22.5 with 12, B = 20 23.9 against 23.5; 9216x2304, 2.25 rows
// per CU, B = 9 / 16 / 20: 13.3 / 13.9 / 14.7 with 8 against 14.1 / 14.5 /
// 15.2; at 1 to 1.5 rows per CU 12 waves stay best); on
// matrices of 16 or more tile rows per CU, 8 waves, with two blocks per CU
// from 32 tile rows per CU where two fit (256000x2304: 172 us against 191 at
// 8 rows, 184 against 186 at 16, 203 against 201 at 32). A launch with K splits counts each row once per split
// and takes at most one block per CU (each block holds most of the LDS: 258
// blocks on 256 CUs ran a second generation, 39 us against 26 at 3584x14336
// B = 16), with the waves by rows per block as above.
static void rx_default_launch(se12_handle* const* hs, int32_t count, int32_t batch, int32_t* waves_out,
                              int32_t* blocks_out) {
    const int64_t cus = std::max<int32_t>(1, hs[0]->cu_count);
    const RxLayout lay = rx_layout(hs, count, batch);
    const int32_t sp = std::max<int32_t>(1, lay.splits);
    // with K splits each split's blocks cover every row: rows per block as
    // if the matrix had `splits` times its rows
    int64_t rows = 0;
    for (int32_t i = 0; i < count; ++i) rows += hs[i]->TR * sp;
    const bool tall = rows >= 16 * cus;
    // two blocks per CU only on very tall launches whose x leaves room for
    // them (256000x2304 B = 8: 172 against 191 us; 27B gate/up grouped, 18
    // tile rows per CU, B = 8 / 16: 96.6 / 99.3 us with one block per CU
    // against 103.2 / 113.0 with two)
    const bool two_per_cu = rows >= 32 * cus && lay.staged == batch &&
                            2 * (int64_t)(rx_lds_bytes(hs[0]->K, batch) + kLutBytes) <= hs[0]->lds_per_block;
    // a split launch takes at most one block per CU (each holds most of
    // the LDS: a second block per CU would run after the first)
    const int64_t per_matrix = std::max<int64_t>(
        1, std::min<int64_t>(rx_max_blocks(hs, count),
                             sp > 1 ? cus / ((int64_t)count * sp) : ceil_div((two_per_cu ? 2 : 1) * cus, count)));
    int32_t waves = tall                              ? 8
                    : rows > 4 * cus && batch <= 16   ? 6
                    : rows > 3 * cus && batch <= 16   ? kRxMaxThreads / 64
                    : rows > 2 * cus                  ? 8
                                                      : kRxMaxThreads / 64;
    // a grouped launch gives each matrix only its share of the blocks: at
    // most one tile row per row slot where the rows allow it (9B gate/up, 2
    // x 14336x3584, 128 blocks each, B = 8 / 16: 33.0 / 34.3 us with 8 waves
    // against 40.9 / 41.1 with 6; a single matrix stays at 6: 36864x4608 B =
    // 8 / 16 53.0 / 56.1 against 57.1 / 59.2 with 8)
    if (!tall && sp == 1 && count > 1)
        while (waves < 8 && per_matrix * waves < rx_max_blocks(hs, count)) waves = waves < 6 ? 6 : 8;
    if (lay.staged < batch) waves = std::min(waves, kRxMaxThreadsXG / 64);
    int64_t blocks = per_matrix;
    // a grouped launch of 2-3 tile rows per CU whose x leaves room for two
    // blocks per CU: 4 waves and two blocks per CU (9B q/k/v, 512 tile rows,
    // B = 5 / 8: 16.3 / 17.0 us against 17.2 / 17.7 with 12 waves x one
    // block; 27B q/k/v 19.4 / 20.0 against 20.3 / 21.0)
    if (count > 1 && sp == 1 && lay.staged == batch && rows >= 2 * cus && rows <= 3 * cus &&
        2 * (int64_t)(rx_lds_bytes(hs[0]->K, batch) + kLutBytes) <= hs[0]->lds_per_block) {
        waves = 4;
        blocks = std::min<int64_t>(rx_max_blocks(hs, count), ceil_div(2 * cus, count));
    }
    *waves_out = waves;
    *blocks_out = (int32_t)(blocks * sp * count);
}

static GemvPlan plan_rx(bool raw, int32_t batch, int32_t staged, int32_t splits, int32_t waves, int32_t blocks,
                        int64_t k, size_t lds) {
    GemvPlan p{};
    p.ksplits = splits;
    p.batch = batch;
    p.raw = raw;
    p.waves = waves;
    p.blocks = blocks;
    p.lds = std::max(lds, rx_lds_bytes(k, staged));
    p.g = 1;
    p.pf = 1;
    p.xg = staged < batch ? 1 : 0;
    return p;
}

// Device memory the kernels of one product use beyond inputs and outputs:
// split-K partial sums and arrival counters (zero between launches: the last
// block to arrive resets its counter). By default each handle's own,
// allocated at bind; se12_gemv_noalloc passes the library's static scratch.
struct Workspace {
    float* partial;
    int64_t partial_elems;
    int32_t* counters;
    int64_t counter_elems;
    uint64_t* pairs;
    int64_t pair_elems;
};

static int gemv_group(const char* fn, se12_handle* const* hs, int32_t count, const void* x, int32_t x_dtype,
                      int32_t batch, float* const* ys, const se12_launch* launch, void* stream,
                      const GemvEpilogue* epi = nullptr, const GemvPrologue* pro = nullptr,
                      const Workspace* ws = nullptr) {
    if (count < 1 || count > kMaxGroup) return fail(SE12_E_INVALID, "%s: %d matrices, expected 1..%d", fn, count, kMaxGroup);
    if (!x) return fail(SE12_E_INVALID, "%s: NULL x", fn);
    if (x_dtype != SE12_X_BF16 && x_dtype != SE12_X_F32) return fail(SE12_E_INVALID, "%s: unknown x_dtype %d", fn, x_dtype);
    int64_t tr_total = 0;
    for (int32_t i = 0; i < count; ++i) {
        const se12_handle* h = hs[i];
        if (!h) return fail(SE12_E_INVALID, "%s: NULL handle %d", fn, i);
        if (!ys[i]) return fail(SE12_E_INVALID, "%s: NULL y %d", fn, i);
        if (batch < 1 || batch > h->max_batch)
            return fail(SE12_E_INVALID, "%s: batch %d outside [1, %d] (the handle's max_batch)", fn, batch, h->max_batch);
        if (h->K != hs[0]->K || h->format != hs[0]->format || h->device != hs[0]->device)
            return fail(SE12_E_INVALID, "%s: grouped matrices need one K, one format and one device", fn);
        tr_total += h->TR;
    }
    const se12_handle* h0 = hs[0];
    const bool xf32 = x_dtype == SE12_X_F32;
    const bool raw = h0->format == SE12_FORMAT_RAW_BF16;
    const size_t esize = xf32 ? 4 : 2;
    // FAST kernels need whole K tiles and 16-byte aligned BF16 rows of x (and,
    // for the raw twin, whole tile rows of an aligned W); the rest run GENERIC
    bool generic = xf32 || h0->K % SE12_TILE_COLS != 0 || !aligned16(x);
    for (int32_t i = 0; i < count; ++i)
        generic = generic || (raw && (hs[i]->N % SE12_TILE_ROWS != 0 || !aligned16(hs[i]->wraw)));
    const bool mfma = uses_mfma(batch, xf32);
    const RxLayout rx_lay = mfma && !generic ? rx_layout(hs, count, batch) : RxLayout{0, 0};
    const int32_t rx_rows = rx_lay.staged;  // x rows in LDS
    const int32_t rx_splits = std::max<int32_t>(1, rx_lay.splits);
    const int64_t rx_k = ceil_div(h0->TC, rx_splits) * SE12_TILE_COLS;  // x columns a block holds
    const bool rx = rx_rows > 0;
    const int rx_max_threads = rx_rows < batch ? kRxMaxThreadsXG : kRxMaxThreads;
    const int32_t step = mfma ? batch : kGemvMaxBatchPerLaunch;
    const int32_t b_first = std::min<int32_t>(batch, step);
    int32_t waves, splits;
    int32_t rx_blocks = 0;
    int64_t grid_rows = tr_total;  // grid rows per split: tile rows, or row blocks (MFMA)
    if (rx) {
        if (launch) {
            if (launch->threads_per_block < 64 || launch->threads_per_block > rx_max_threads ||
                launch->threads_per_block % 64 != 0)
                return fail(SE12_E_INVALID, "%s: threads_per_block %d must be a multiple of 64 in [64, %d] at batch %d",
                            fn, launch->threads_per_block, rx_max_threads, batch);
            if (launch->blocks <= 0 || launch->blocks % (count * rx_splits) != 0 ||
                launch->blocks / (count * rx_splits) > rx_max_blocks(hs, count))
                return fail(SE12_E_INVALID, "%s: blocks %d must be %d x 1..%lld (matrices x K splits x blocks per "
                            "matrix and split, at most its tile rows)", fn, launch->blocks, count * rx_splits,
                            (long long)rx_max_blocks(hs, count));
            waves = launch->threads_per_block / 64;
            rx_blocks = launch->blocks;
        } else {
            rx_default_launch(hs, count, batch, &waves, &rx_blocks);
        }
        splits = rx_splits;
        grid_rows = rx_blocks / rx_splits;
    } else if (launch) {
        const int max_threads = mfma ? (generic ? kGemmMaxThreadsGeneric : kGemmMaxThreads)
                                     : max_threads_for(b_first, xf32, generic);
        const int min_threads = mfma ? 64 * gemm_min_waves(batch) : 64;
        if (launch->threads_per_block < min_threads || launch->threads_per_block > max_threads ||
            launch->threads_per_block % 64 != 0)
            return fail(SE12_E_INVALID, "%s: threads_per_block %d must be a multiple of 64 in [%d, %d] at batch %d", fn,
                        launch->threads_per_block, min_threads, max_threads, batch);
        waves = launch->threads_per_block / 64;
        if (mfma && waves % gemm_min_waves(batch) != 0)
            return fail(SE12_E_INVALID, "%s: %d waves per block at batch %d: the MFMA kernel takes %d tile rows per block "
                        "times K groups", fn, waves, batch, gemm_min_waves(batch));
        if (mfma) grid_rows = gemm_row_blocks(hs, count, gemm_min_waves(batch));
        if (launch->blocks <= 0 || launch->blocks % grid_rows != 0)
            return fail(SE12_E_INVALID, "%s: blocks %d must be a positive multiple of the %lld %s", fn, launch->blocks,
                        (long long)grid_rows, mfma ? "row blocks (tile rows / waves, rounded up, per matrix)" : "tile rows");
        splits = (int32_t)(launch->blocks / grid_rows);
        const int32_t cap = mfma ? std::min(h0->s_cap, kGemmMaxSplits) : h0->s_cap;
        if (splits > cap)
            return fail(SE12_E_CAPACITY, "%s: %d K splits exceed the limit %d at batch %d", fn, splits, cap, batch);
    } else {
        if (mfma) {
            gemm_default_launch(hs, count, batch, generic, &waves, &splits);
            grid_rows = gemm_row_blocks(hs, count, gemm_min_waves(batch));
        } else {
            default_launch(tr_total, h0->TC, h0->cu_count, h0->s_cap, batch, xf32, generic, pro != nullptr, &waves,
                           &splits);
            // a launch with the norm in its head: one or two waves fewer where
            // that splits the K tiles evenly (Gemma-2-2B gate/up, 9 K tiles: 3
            // waves instead of 4 measured 15 us less per decoded token)
            if (pro && !generic && splits == 1 && waves > 2 && h0->TC % waves != 0) {
                int32_t even = waves - 1;
                while (even > 2 && h0->TC % even != 0) --even;
                if (h0->TC % even == 0 && even >= waves - 2) waves = even;
            }
        }
    }
    if (grid_rows * splits > INT32_MAX) return fail(SE12_E_INVALID, "%s: grid too large", fn);
    DeviceScope ds;
    SE12_HIP(ds.enter(h0->device));
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (ws) {
        if (count != 1 || epi || pro) return fail(SE12_E_INVALID, "%s: a workspace serves one plain product", fn);
        if (gemv_counter_count(h0->TR) > ws->counter_elems)
            return fail(SE12_E_CAPACITY, "%s: %d tile rows need %lld arrival counters, the scratch holds %lld", fn,
                        h0->TR, (long long)gemv_counter_count(h0->TR), (long long)ws->counter_elems);
        if (mfma && splits > 1 && (int64_t)splits * b_first * h0->Np > ws->partial_elems)
            return fail(SE12_E_CAPACITY, "%s: %d K splits x %d batch rows x %lld rows need %lld partial sums, the "
                        "scratch holds %lld", fn, splits, b_first, (long long)h0->Np,
                        (long long)splits * b_first * h0->Np, (long long)ws->partial_elems);
        if (!mfma && splits > 1 && (int64_t)(splits - 1) * b_first * h0->Np > ws->pair_elems)
            return fail(SE12_E_CAPACITY, "%s: %d K splits x %d batch rows x %lld rows need %lld pair slots, the "
                        "scratch holds %lld", fn, splits, b_first, (long long)h0->Np,
                        (long long)(splits - 1) * b_first * h0->Np, (long long)ws->pair_elems);
    } else if (splits > 1) {
        for (int32_t i = 0; i < count; ++i)
            if ((int64_t)splits * b_first * hs[i]->Np > hs[i]->partial_elems ||
                (!mfma && (int64_t)(splits - 1) * b_first * hs[i]->Np > hs[i]->pair_elems))
                return fail(SE12_E_CAPACITY, "%s: %d K splits at batch %d exceed handle %d's split-K workspace", fn,
                            splits, batch, i);
    }
    // the x prologue runs in the dot2 kernel when its rows fit the block's
    // LDS; the caller has checked the rest
    const bool fuse_pro = pro && !mfma && !generic &&
                          (int64_t)(gemv_xn_lds_bytes(h0->K, b_first, waves) + kLutBytes) <= h0->lds_per_block;
    if (pro && !fuse_pro) {
        // the norm as its own kernel into h_out, then the product of h_out
        hipStream_t st0 = static_cast<hipStream_t>(stream);
        if (pro->res_out != pro->res_in)
            SE12_HIP(hipMemcpyAsync(pro->res_out, pro->res_in, (size_t)batch * h0->K * 2, hipMemcpyDeviceToDevice, st0));
        const int rc = se12_step_rmsnorm(pro->y_prev, SE12_STEP_F32, h0->K, pro->w1, pro->res_out, pro->w2, pro->h_out,
                                         batch, (int32_t)h0->K, pro->eps, 0.0f, 1, st0);
        if (rc != SE12_STEP_OK) return fail(SE12_E_HIP, "%s norm: %s", fn, se12_step_last_error());
        return gemv_group(fn, hs, count, pro->h_out, SE12_X_BF16, batch, ys, launch, stream, epi, nullptr);
    }
    // the step tail runs in the dot2 kernel when its row fits the block's LDS
    const bool fuse_epi =
        epi && !mfma &&
        (epi->kind != kEpiRmsNorm ||
         ((int64_t)(gemv_norm_lds_bytes(h0->N) + kLutBytes) <= h0->lds_per_block && h0->N % 4 == 0 &&
          aligned8(ys[0]) && aligned8(epi->w1) && aligned8(epi->w2) && aligned8(epi->residual) && aligned8(epi->out)));
    for (int32_t b0 = 0; b0 < batch; b0 += step) {
        const int32_t bl = std::min<int32_t>(step, batch - b0);
        GemvGroupArgs g{};
        g.count = count;
        g.rows_per_block = mfma ? gemm_min_waves(bl) : 1;
        int32_t start = 0;
        size_t rx_lds = 0;
        for (int32_t i = 0; i < count; ++i) {
            const se12_handle* h = hs[i];
            GemvArgs& a = g.m[i];
            a.sm = h->s.sm_dev;
            a.ec = h->s.ec_dev;
            a.lut = h->lut;
            a.side = h->side;
            a.fb_raw = h->s.fallback_raw_dev;
            a.ovf_raw = h->ovf_raw;
            a.wraw = h->wraw;
            a.x = static_cast<const char*>(x) + (size_t)b0 * h->K * esize;
            a.y = ys[i] + (size_t)b0 * h->N;
            a.partial = ws ? ws->partial : h->partial;
            a.counters = ws ? ws->counters : h->counters;
            a.pairs = ws ? ws->pairs : h->pairs;
            a.N = h->N;
            a.K = h->K;
            a.Np = h->Np;
            a.TR = h->TR;
            a.TC = h->TC;
            a.S = rx ? rx_kgroups(h->TR, h->TC / rx_splits, waves, rx_blocks / (count * rx_splits)) : splits;
            rx_lds = std::max(rx_lds, rx ? rx_lds_total(rx_k, rx_rows, bl, waves, a.S) : 0);
            g.tr_start[i] = start;
            start += mfma ? (int32_t)ceil_div(h->TR, gemm_min_waves(bl)) : h->TR;
        }
        for (int32_t i = count; i <= kMaxGroup; ++i) g.tr_start[i] = start;
        const bool gen = generic || !aligned16(g.m[0].x);
        GemvPlan p = rx     ? plan_rx(raw, bl, rx_rows, rx_splits, waves, rx_blocks, rx_k, rx_lds)
                     : mfma ? plan_gemm(grid_rows, raw, bl, gen, waves, splits, h0->TC, h0->lds_per_block)
                            : plan_gemv(tr_total, h0->TC, raw, bl, xf32, gen, waves, splits);
        if (fuse_pro) {
            g.pro = *pro;
            g.pro.y_prev += (size_t)b0 * h0->K;
            if (g.pro.y_prev_ss) g.pro.y_prev_ss += (size_t)b0 * ceil_div(h0->K, SE12_TILE_ROWS);
            g.pro.res_in += (size_t)b0 * h0->K;
            g.pro.res_out += (size_t)b0 * h0->K;
            g.pro.h_out += (size_t)b0 * h0->K;
            p.xn = true;
            p.lds = gemv_xn_lds_bytes(h0->K, bl, waves);
        }
        if (fuse_epi) {
            g.epi = *epi;
            if (g.epi.out) g.epi.out += (size_t)b0 * h0->N;
            if (g.epi.residual) g.epi.residual += (size_t)b0 * h0->N;
            if (g.epi.row_ss) g.epi.row_ss += (size_t)b0 * h0->TR;
            if (epi->kind == kEpiRmsNorm) p.lds = std::max(p.lds, gemv_norm_lds_bytes(h0->N));
        }
        if ((int64_t)(p.lds + kLutBytes) > h0->lds_per_block)
            return fail(SE12_E_CAPACITY, "%s: launch needs %zu bytes of LDS, the device allows %lld", fn, p.lds,
                        (long long)h0->lds_per_block);
        hipError_t e = rx ? launch_gemm_rx(g, bl, p, st) : mfma ? launch_gemm(g, bl, p, st) : launch_gemv(g, p, st);
        if (e != hipSuccess) return fail(SE12_E_HIP, "%s launch: %s", fn, hipGetErrorString(e));
    }
    if (epi && !fuse_epi) {
        // the step runs as its own kernel after the product
        if (epi->row_ss) {
            const hipError_t e = launch_row_sumsq(ys[0], h0->N, h0->TR, batch, epi->row_ss, st);
            if (e != hipSuccess) return fail(SE12_E_HIP, "%s row sums: %s", fn, hipGetErrorString(e));
        }
        if (epi->kind != kEpiNone) {
            const int rc = epi->kind == kEpiGeluMul
                               ? se12_step_gelu_mul(ys[0], ys[1], SE12_STEP_F32, h0->N, epi->out, batch, (int32_t)h0->N, st)
                               : se12_step_rmsnorm(ys[0], SE12_STEP_F32, h0->N, epi->w1, epi->residual, epi->w2,
                                                   epi->out, batch, (int32_t)h0->N, epi->eps, 0.0f, 1, st);
            if (rc != SE12_STEP_OK) return fail(SE12_E_HIP, "%s step: %s", fn, se12_step_last_error());
        }
    }
    return SE12_OK;
}

int se12_gemv(se12_handle* h, const void* x, int32_t x_dtype, int32_t batch, float* y, const se12_launch* launch,
              void* stream) {
    if (!h) return fail(SE12_E_INVALID, "se12_gemv: NULL handle");
    if (!x || !y) return fail(SE12_E_INVALID, "se12_gemv: NULL x or y");
    se12_handle* hs[1] = {h};
    float* ys[1] = {y};
    return gemv_group("se12_gemv", hs, 1, x, x_dtype, batch, ys, launch, stream);
}

}  // extern "C"

// The zero-allocation product's scratch: one array per device (each GPU the
// library runs on holds its own copy until the process ends), arrival
// counters first, then the dot2 kernel's split-K pair slots, then split-K
// partial sums; the counters and slots start at zero and every launch leaves
// them so. In host code `scratch`
// names a host-side stand-in, not device memory: only the address
// hipGetSymbolAddress returns for the current device may reach a kernel or
// any HIP call.
constexpr size_t kScratchBytes = size_t(8) << 20;
constexpr size_t kScratchCounterBytes = size_t(256) << 10;
constexpr size_t kScratchPairBytes = size_t(2) << 20;
constexpr size_t kScratchZeroBytes = kScratchCounterBytes + kScratchPairBytes;  // cleared at set-up
static_assert(kScratchCounterBytes % 256 == 0 && kScratchPairBytes % 256 == 0 && kScratchZeroBytes < kScratchBytes,
              "scratch layout");
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

namespace {

constexpr int kScratchMaxDevices = 64;
std::mutex g_scratch_mutex;
uint8_t* g_scratch_ptr[kScratchMaxDevices] = {};

__global__ void scratch_clear_kernel(uint32_t* p, int64_t words) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < words; i += (int64_t)gridDim.x * blockDim.x)
        p[i] = 0u;
}

// The device address of `scratch` on `device` (current), set up on the
// first call there: hipGetSymbolAddress, then the counters and pair slots
// cleared by a kernel on `stream` (a fill kernel, so that a caller capturing
// the call records no memset node).
int scratch_for_device(int device, hipStream_t stream, uint8_t** out) {
    if (device < 0 || device >= kScratchMaxDevices)
        return fail(SE12_E_DEVICE, "se12_gemv_noalloc: device %d beyond the %d the scratch table serves", device,
                    kScratchMaxDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (!g_scratch_ptr[device]) {
        void* p = nullptr;
        SE12_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        if (!p) return fail(SE12_E_HIP, "se12_gemv_noalloc: hipGetSymbolAddress gave NULL");
        hipLaunchKernelGGL(scratch_clear_kernel, dim3(64), dim3(256), 0, stream, static_cast<uint32_t*>(p),
                           (int64_t)(kScratchZeroBytes / sizeof(uint32_t)));
        SE12_HIP(hipGetLastError());
        g_scratch_ptr[device] = static_cast<uint8_t*>(p);
    }
    *out = g_scratch_ptr[device];
    return SE12_OK;
}

}  // namespace

extern "C" {

int se12_gemv_noalloc(se12_handle* h, const void* x, int32_t x_dtype, int32_t batch, float* y,
                      const se12_launch* launch, void* stream) {
    if (!h) return fail(SE12_E_INVALID, "se12_gemv_noalloc: NULL handle");
    if (!x || !y) return fail(SE12_E_INVALID, "se12_gemv_noalloc: NULL x or y");
    uint8_t* base = nullptr;
    {
        DeviceScope ds;
        SE12_HIP(ds.enter(h->device));
        if (int rc = scratch_for_device(h->device, static_cast<hipStream_t>(stream), &base)) return rc;
    }
    Workspace ws{reinterpret_cast<float*>(base + kScratchZeroBytes),
                 (int64_t)((kScratchBytes - kScratchZeroBytes) / sizeof(float)),
                 reinterpret_cast<int32_t*>(base),
                 (int64_t)(kScratchCounterBytes / sizeof(int32_t)),
                 reinterpret_cast<uint64_t*>(base + kScratchCounterBytes),
                 (int64_t)(kScratchPairBytes / sizeof(uint64_t))};
    se12_handle* hs[1] = {h};
    float* ys[1] = {y};
    return gemv_group("se12_gemv_noalloc", hs, 1, x, x_dtype, batch, ys, launch, stream, nullptr, nullptr, &ws);
}

int se12_gemv_grouped(se12_handle* const* handles, int32_t count, const void* x, int32_t x_dtype, int32_t batch,
                      float* const* y, const se12_launch* launch, void* stream) {
    if (!handles || !y) return fail(SE12_E_INVALID, "se12_gemv_grouped: NULL handles or y");
    return gemv_group("se12_gemv_grouped", handles, count, x, x_dtype, batch, y, launch, stream);
}

int se12_gemv_gelu_mul(se12_handle* const* gate_up, const void* x, int32_t x_dtype, int32_t batch, float* const* y,
                       uint16_t* out, const se12_launch* launch, void* stream) {
    if (!gate_up || !y || !out) return fail(SE12_E_INVALID, "se12_gemv_gelu_mul: NULL handles, y or out");
    if (!gate_up[0] || !gate_up[1]) return fail(SE12_E_INVALID, "se12_gemv_gelu_mul: NULL handle");
    if (gate_up[0]->N != gate_up[1]->N)
        return fail(SE12_E_INVALID, "se12_gemv_gelu_mul: gate and up have %lld and %lld rows",
                    (long long)gate_up[0]->N, (long long)gate_up[1]->N);
    if (gate_up[0]->N > INT32_MAX) return fail(SE12_E_INVALID, "se12_gemv_gelu_mul: too many rows");
    GemvEpilogue e{};
    e.kind = kEpiGeluMul;
    e.out = out;
    return gemv_group("se12_gemv_gelu_mul", gate_up, 2, x, x_dtype, batch, y, launch, stream, &e);
}

int se12_gemv_rowss(se12_handle* h, const void* x, int32_t x_dtype, int32_t batch, float* y, float* row_ss,
                    const se12_launch* launch, void* stream) {
    if (!h || !y || !row_ss) return fail(SE12_E_INVALID, "se12_gemv_rowss: NULL handle, y or row_ss");
    GemvEpilogue e{};
    e.kind = kEpiNone;
    e.row_ss = row_ss;
    se12_handle* hs[1] = {h};
    float* ys[1] = {y};
    return gemv_group("se12_gemv_rowss", hs, 1, x, x_dtype, batch, ys, launch, stream, &e);
}

int se12_gemv_rmsnorm(se12_handle* h, const void* x, int32_t x_dtype, int32_t batch, float* y, const uint16_t* w1,
                      const uint16_t* w2, uint16_t* residual, uint16_t* out, float eps, const se12_launch* launch,
                      void* stream) {
    if (!h || !y || !w1 || !w2 || !residual || !out)
        return fail(SE12_E_INVALID, "se12_gemv_rmsnorm: NULL handle, y, weights, residual or out");
    if (h->N > kStepNormMaxRows)
        return fail(SE12_E_INVALID, "se12_gemv_rmsnorm: %lld rows, the norm takes at most %d", (long long)h->N,
                    kStepNormMaxRows);
    GemvEpilogue e{};
    e.kind = kEpiRmsNorm;
    e.eps = eps;
    e.w1 = w1;
    e.w2 = w2;
    e.residual = residual;
    e.out = out;
    se12_handle* hs[1] = {h};
    float* ys[1] = {y};
    return gemv_group("se12_gemv_rmsnorm", hs, 1, x, x_dtype, batch, ys, launch, stream, &e);
}

int se12_gemv_prenorm(se12_handle* const* handles, int32_t count, const float* y_prev, const float* y_prev_ss,
                      int32_t batch, const uint16_t* w1, const uint16_t* w2, const uint16_t* residual_in,
                      uint16_t* residual_out, uint16_t* h_out, float eps, float* const* y, uint16_t* gelu_out,
                      const se12_launch* launch, void* stream) {
    const char* fn = "se12_gemv_prenorm";
    if (!handles || !y || !y_prev || !w1 || !w2 || !residual_in || !residual_out || !h_out)
        return fail(SE12_E_INVALID, "%s: NULL handles, y, y_prev, weights, residuals or h_out", fn);
    if (count < 1 || count > kMaxGroup) return fail(SE12_E_INVALID, "%s: %d matrices, expected 1..%d", fn, count, kMaxGroup);
    if (!handles[0]) return fail(SE12_E_INVALID, "%s: NULL handle 0", fn);
    const int64_t K = handles[0]->K;
    if (K > kStepNormMaxRows) return fail(SE12_E_INVALID, "%s: %lld columns, the norm takes at most %d", fn, (long long)K,
                                          kStepNormMaxRows);
    if (batch < 1) return fail(SE12_E_INVALID, "%s: batch %d", fn, batch);
    const size_t row_bytes = (size_t)batch * K * 2;
    const char* ri = reinterpret_cast<const char*>(residual_in);
    const char* ro = reinterpret_cast<const char*>(residual_out);
    if (ri != ro && ri < ro + row_bytes && ro < ri + row_bytes)
        return fail(SE12_E_INVALID, "%s: residual_in and residual_out overlap without being the same tensor", fn);
    GemvPrologue pr{};
    pr.y_prev = y_prev;
    pr.y_prev_ss = y_prev_ss;
    pr.w1 = w1;
    pr.w2 = w2;
    pr.res_in = residual_in;
    pr.res_out = residual_out;
    pr.h_out = h_out;
    pr.eps = eps;
    // the in-kernel prologue reads residual_in while block (0, 0) writes
    // residual_out, and takes 16-byte rows of y_prev: otherwise the norm runs
    // as its own kernel
    const bool ok = ri != ro && K % 4 == 0 && aligned16(y_prev) && aligned8(w1) && aligned8(w2) && aligned8(residual_in) &&
                    aligned8(residual_out) && aligned8(h_out);
    GemvEpilogue e{};
    if (gelu_out) {
        if (count != 2 || !handles[1] || handles[0]->N != handles[1]->N)
            return fail(SE12_E_INVALID, "%s: the MLP gate takes two matrices of one row count", fn);
        e.kind = kEpiGeluMul;
        e.out = gelu_out;
    }
    if (!ok) {
        // same results through the separate kernels (in-place residual update)
        hipStream_t st = static_cast<hipStream_t>(stream);
        if (ri != ro) SE12_HIP(hipMemcpyAsync(residual_out, residual_in, row_bytes, hipMemcpyDeviceToDevice, st));
        const int rc = se12_step_rmsnorm(y_prev, SE12_STEP_F32, K, w1, residual_out, w2, h_out, batch, (int32_t)K, eps,
                                         0.0f, 1, st);
        if (rc != SE12_STEP_OK) return fail(SE12_E_HIP, "%s norm: %s", fn, se12_step_last_error());
        return gemv_group(fn, handles, count, h_out, SE12_X_BF16, batch, y, launch, stream, gelu_out ? &e : nullptr);
    }
    return gemv_group(fn, handles, count, h_out, SE12_X_BF16, batch, y, launch, stream, gelu_out ? &e : nullptr, &pr);
}

static DecodeArgs decode_args(const se12_handle* h, uint16_t* out) {
    DecodeArgs a{};
    a.sm = h->s.sm_dev;
    a.ec = h->s.ec_dev;
    a.esc = h->s.esc_dev;
    a.codebook = h->s.codebook_dev;
    a.bitmap = h->s.fallback_bitmap_dev;
    a.lut = h->lut;
    a.info = h->info;
    a.escpos = h->escpos;
    a.side = h->side;
    a.fb_raw = h->s.fallback_raw_dev;
    a.ovf_raw = h->ovf_raw;
    a.out = out;
    a.N = h->N;
    a.K = h->K;
    a.T = h->T;
    a.TR = h->TR;
    a.TC = h->TC;
    a.out_vec_ok = (aligned16(out) && h->K % 8 == 0) ? 1 : 0;
    return a;
}

int se12_decode(se12_handle* h, uint16_t* out, void* stream) {
    if (!h || !out) return fail(SE12_E_INVALID, "se12_decode: NULL argument");
    if (h->format != SE12_FORMAT_SE12) return fail(SE12_E_INVALID, "se12_decode: handle is not SE12");
    DeviceScope ds;
    SE12_HIP(ds.enter(h->device));
    DecodeArgs a = decode_args(h, out);
    a.items = h->T;
    hipError_t e = launch_decode(a, false, static_cast<hipStream_t>(stream), h->cu_count);
    if (e != hipSuccess) return fail(SE12_E_HIP, "se12_decode launch: %s", hipGetErrorString(e));
    return SE12_OK;
}

int se12_decode_rows(se12_handle* h, const int64_t* rows, int64_t nrows, uint16_t* out, void* stream) {
    if (!h) return fail(SE12_E_INVALID, "se12_decode_rows: NULL handle");
    if (h->format != SE12_FORMAT_SE12) return fail(SE12_E_INVALID, "se12_decode_rows: handle is not SE12");
    if (nrows < 0) return fail(SE12_E_INVALID, "se12_decode_rows: negative row count");
    if (nrows == 0) return SE12_OK;
    if (!rows || !out) return fail(SE12_E_INVALID, "se12_decode_rows: NULL rows or out");
    DeviceScope ds;
    SE12_HIP(ds.enter(h->device));
    DecodeArgs a = decode_args(h, out);
    a.rows = rows;
    a.nrows = nrows;
    a.items = nrows * h->TC;
    hipError_t e = launch_decode(a, true, static_cast<hipStream_t>(stream), h->cu_count);
    if (e != hipSuccess) return fail(SE12_E_HIP, "se12_decode_rows launch: %s", hipGetErrorString(e));
    return SE12_OK;
}

int se12_codebook_from_histogram(const uint64_t counts[256], uint8_t codebook_out[15]) {
    if (!counts || !codebook_out) return fail(SE12_E_INVALID, "se12_codebook_from_histogram: NULL argument");
    int order[256];
    for (int i = 0; i < 256; ++i) order[i] = i;
    std::stable_sort(order, order + 256, [&](int a, int b) {
        if (counts[a] != counts[b]) return counts[a] > counts[b];
        return a > b;
    });
    for (int i = 0; i < SE12_CODEBOOK_SIZE; ++i) codebook_out[i] = (uint8_t)order[i];
    return SE12_OK;
}

static int encode_args(EncodeArgs& a, const uint16_t* w, int64_t rows, int64_t cols, int64_t ld) {
    if (!w) return fail(SE12_E_INVALID, "encode: NULL weights");
    if (rows <= 0 || cols <= 0 || ld < cols) return fail(SE12_E_INVALID, "encode: bad shape [%lld, %lld] ld %lld",
                                                         (long long)rows, (long long)cols, (long long)ld);
    a = EncodeArgs{};
    a.w = w;
    a.N = rows;
    a.K = cols;
    a.ld = ld;
    a.TR = (int32_t)ceil_div(rows, SE12_TILE_ROWS);
    a.TC = (int32_t)ceil_div(cols, SE12_TILE_COLS);
    a.T = (int64_t)a.TR * a.TC;
    a.w_vec_ok = (aligned16(w) && ld % 8 == 0) ? 1 : 0;
    return SE12_OK;
}

static void pack_codebook(EncodeArgs& a, const uint8_t cb[15]) {
    uint8_t b[16] = {0};
    std::memcpy(b, cb, 15);
    std::memcpy(a.codebook, b, 16);
}

int se12_encode_prepare(const uint16_t* w, int64_t rows, int64_t cols, int64_t ld, uint8_t codebook_out[15],
                        int64_t* fallback_tiles_out, void* stream) {
    if (!codebook_out || !fallback_tiles_out) return fail(SE12_E_INVALID, "se12_encode_prepare: NULL output");
    EncodeArgs a;
    if (int rc = encode_args(a, w, rows, cols, ld)) return rc;
    hipStream_t st = static_cast<hipStream_t>(stream);
    uint64_t* hist = nullptr;
    int32_t* counts = nullptr;
    SE12_HIP(hipMalloc(&hist, 256 * sizeof(uint64_t)));
    hipError_t e = hipMalloc(&counts, (size_t)a.T * sizeof(int32_t));
    uint64_t hh[256];
    std::vector<int32_t> ch((size_t)a.T);
    if (e == hipSuccess) e = hipMemsetAsync(hist, 0, 256 * sizeof(uint64_t), st);
    a.histogram = hist;
    a.tile_escapes = counts;
    if (e == hipSuccess) e = launch_encode_histogram(a, st);
    if (e == hipSuccess) e = hipMemcpyAsync(hh, hist, sizeof hh, hipMemcpyDeviceToHost, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (e == hipSuccess) {
        se12_codebook_from_histogram(hh, codebook_out);
        pack_codebook(a, codebook_out);
        e = launch_encode_count(a, st);
    }
    if (e == hipSuccess) e = hipMemcpyAsync(ch.data(), counts, (size_t)a.T * sizeof(int32_t), hipMemcpyDeviceToHost, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    (void)hipFree(hist);
    if (counts) (void)hipFree(counts);
    if (e != hipSuccess) return fail(SE12_E_HIP, "se12_encode_prepare: %s", hipGetErrorString(e));
    int64_t nfb = 0;
    for (int32_t c : ch) nfb += c > SE12_ESCAPE_BUDGET ? 1 : 0;
    *fallback_tiles_out = nfb;
    return SE12_OK;
}

int se12_encode(const uint16_t* w, int64_t rows, int64_t cols, int64_t ld, const uint8_t codebook[15],
                const se12_streams_out* out, int64_t* fallback_tiles_out, void* stream) {
    if (!codebook || !out) return fail(SE12_E_INVALID, "se12_encode: NULL argument");
    EncodeArgs a;
    if (int rc = encode_args(a, w, rows, cols, ld)) return rc;
    if (!out->sm_dev || !out->ec_dev || !out->esc_dev || !out->fallback_bitmap_dev)
        return fail(SE12_E_INVALID, "se12_encode: a required output stream is NULL");
    if (!aligned16(out->sm_dev) || !aligned16(out->ec_dev) ||
        (out->fallback_raw_dev && !aligned16(out->fallback_raw_dev)))
        return fail(SE12_E_INVALID, "se12_encode: sm/ec/fallback_raw outputs must be 16-byte aligned");
    if (out->fallback_raw_tiles < 0) return fail(SE12_E_INVALID, "se12_encode: negative fallback capacity");
    if (out->fallback_raw_tiles > 0 && !out->fallback_raw_dev)
        return fail(SE12_E_INVALID, "se12_encode: fallback_raw is NULL but has capacity");
    pack_codebook(a, codebook);
    a.sm = out->sm_dev;
    a.ec = out->ec_dev;
    a.esc = out->esc_dev;
    a.bitmap = out->fallback_bitmap_dev;
    a.raw = out->fallback_raw_dev;
    hipStream_t st = static_cast<hipStream_t>(stream);
    int32_t* counts = nullptr;
    int32_t* rank = nullptr;
    int64_t* totals = nullptr;
    int64_t total = 0;
    hipError_t e = hipMalloc(&counts, (size_t)a.T * sizeof(int32_t));
    if (e == hipSuccess) e = hipMalloc(&rank, (size_t)a.T * sizeof(int32_t));
    if (e == hipSuccess) e = hipMalloc(&totals, sizeof(int64_t));
    a.tile_escapes = counts;
    a.fb_rank = rank;
    a.totals = totals;
    if (e == hipSuccess) e = launch_encode_count(a, st);
    if (e == hipSuccess) e = launch_encode_scan(a, st);
    if (e == hipSuccess) e = hipMemcpyAsync(&total, totals, sizeof total, hipMemcpyDeviceToHost, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    int rc = SE12_OK;
    if (e != hipSuccess) {
        rc = fail(SE12_E_HIP, "se12_encode: %s", hipGetErrorString(e));
    } else if (total > out->fallback_raw_tiles) {
        rc = fail(SE12_E_CAPACITY, "se12_encode: %lld fallback tiles, fallback_raw holds %lld", (long long)total,
                  (long long)out->fallback_raw_tiles);
    } else {
        e = launch_encode_write(a, st);
        if (e == hipSuccess) e = hipStreamSynchronize(st);
        if (e != hipSuccess) rc = fail(SE12_E_HIP, "se12_encode write: %s", hipGetErrorString(e));
    }
    if (fallback_tiles_out) *fallback_tiles_out = total;
    if (counts) (void)hipFree(counts);
    if (rank) (void)hipFree(rank);
    if (totals) (void)hipFree(totals);
    return rc;
}

}  // extern "C"
