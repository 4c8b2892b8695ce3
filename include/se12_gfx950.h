/*
 * se12_gfx950.h - C ABI of the MI355X (gfx950) SE12 decode + GEMV library.
 *
 * SE12 stores a BF16 matrix [rows, cols] as 16x256 tiles (tile-major,
 * tile t = tile_row * tile_cols + tile_col, in-tile index = local_row*256 +
 * local_col), each tile as 4096 sign|mantissa bytes (`sm`), 2048 bytes of
 * 4-bit exponent codes (`ec`, even index in the low nibble), 16 escape slots
 * (`esc`), plus one bitmap bit per tile (MSB first) marking tiles kept raw in
 * `fallback_raw`, and a 15-entry exponent codebook. The layout is the one the
 * reference encoder writes (lws/domain/se12/codec.py:111-141) and its packer
 * stores (lws/adapters/safetensors/packed_store.py:70-107).
 *
 * Conventions: every pointer named *_dev is device memory owned by the caller
 * (e.g. a torch tensor); streams are hipStream_t passed as void*; every entry
 * point returns 0 on success or a negative SE12_E* code, and se12_last_error()
 * gives the message of the calling thread's last failure. No entry point that
 * launches work synchronizes the stream unless its comment says so.
 */
#ifndef SE12_GFX950_H
#define SE12_GFX950_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SE12_TILE_ROWS 16
#define SE12_TILE_COLS 256
#define SE12_TILE_SIZE 4096
#define SE12_ESCAPE_BUDGET 16
#define SE12_CODEBOOK_SIZE 15
#define SE12_ESCAPE_CODE 15
#define SE12_MAX_BATCH 32
#define SE12_MAX_GROUP 4

/* status codes */
#define SE12_OK 0
#define SE12_E_INVALID (-1)   /* bad argument (null pointer, shape, size) */
#define SE12_E_HIP (-2)       /* a HIP runtime call failed */
#define SE12_E_CAPACITY (-3)  /* an output or workspace is too small */
#define SE12_E_DEVICE (-4)    /* wrong or unsupported device */

/* activation element types */
#define SE12_X_BF16 0
#define SE12_X_F32 1

/* weight formats a handle can be bound to */
#define SE12_FORMAT_SE12 0
#define SE12_FORMAT_RAW_BF16 1

/* The five SE12 streams and the codebook, as device pointers. */
typedef struct se12_streams {
    const uint8_t* sm_dev;              /* [tiles * 4096] */
    const uint8_t* ec_dev;              /* [tiles * 2048] */
    const uint8_t* esc_dev;             /* [tiles * 16] */
    const uint8_t* codebook_dev;        /* [15] */
    const uint8_t* fallback_bitmap_dev; /* [ceil(tiles / 8)] */
    const int16_t* fallback_raw_dev;    /* [fallback_tiles * 4096], may be NULL when empty */
    int64_t fallback_raw_elems;         /* element count of fallback_raw (checked at bind) */
} se12_streams;

/* Writable streams for the encoder. */
typedef struct se12_streams_out {
    uint8_t* sm_dev;
    uint8_t* ec_dev;
    uint8_t* esc_dev;
    uint8_t* fallback_bitmap_dev;
    int16_t* fallback_raw_dev;          /* capacity: fallback_raw_tiles tiles */
    int64_t fallback_raw_tiles;
} se12_streams_out;

/* Launch shape of the GEMV: `threads_per_block` = 64 * waves per workgroup.
 * Its `blocks` depend on the kernel the batch runs:
 *  - dot2 kernel (batch 1..4 per launch, FP32 x): 1..16 waves, `blocks` =
 *    tile_rows * k_splits, k_splits cutting the K tiles into contiguous
 *    ranges;
 *  - x-slab MFMA kernel (BF16 x, 5..32 rows): a multiple of ceil(batch / 8)
 *    waves (4 for 3) up to 8, `blocks` = ceil(tile_rows / (those rows)) *
 *    k_splits (k_splits <= 16);
 *  - resident-x MFMA kernel (BF16 x, 5..32 rows, x or a K split's share of
 *    it held in LDS): 1..12 waves (8 where batch group 1's x comes from
 *    global memory), `blocks` = matrices * k_splits * blocks per matrix and
 *    split (1..tile_rows), the k_splits fixed by the shape.
 * Mirrors the reference LaunchConfiguration (lws/domain/launch/heuristic.py:
 * 40-43) re-derived for wave64. */
typedef struct se12_launch {
    int32_t threads_per_block;
    int32_t blocks;
} se12_launch;

typedef struct se12_device_info {
    char name[256];
    char arch[64];              /* e.g. "gfx950:sramecc+:xnack-" */
    int32_t compute_units;
    int32_t wavefront_size;
    int64_t l2_bytes;
    int64_t lds_bytes_per_cu;
    int64_t lds_bytes_per_block;
    int64_t total_memory_bytes;
    int32_t clock_khz;
    int32_t memory_clock_khz;
    int32_t memory_bus_width_bits;
    int32_t max_threads_per_block;
    int32_t pci_domain_id;
    int32_t pci_bus_id;
    int32_t pci_device_id;
    int32_t ecc_enabled;         /* hipDeviceProp_t.ECCEnabled */
    int32_t kernel_timeout;      /* hipDeviceProp_t.kernelExecTimeoutEnabled (a display watchdog) */
    int32_t runtime_version;     /* hipRuntimeGetVersion */
    int32_t driver_version;      /* hipDriverGetVersion */
} se12_device_info;

typedef struct se12_handle se12_handle;

/* Thread-local message of the last failed call ("" if none). */
const char* se12_last_error(void);

/* Library build string (arch, compiler). Host only, never touches the GPU. */
const char* se12_version(void);

/* Device facts from hipDeviceProp_t. Replaces CudaGpuProbe.properties
 * (lws/adapters/cuda/gpu_probe.py:59-80). */
int se12_device_info_get(int32_t device, se12_device_info* out);

/* Binds a weight matrix already resident on the current device: validates the
 * streams' sizes, builds the per-tile fallback-rank sidecar (the reference's
 * host-side fallback_offsets, lws/adapters/cuda/gemv.py:47-53) on the GPU and
 * allocates the split-K workspace for batches up to `max_batch`.
 * Synchronizes `stream`. Replaces Se12MatVecKernel.__init__ and
 * _upload_se12_streams (lws/adapters/cuda/gemv.py:183-194,229-264); the
 * caller keeps ownership of the streams, which must outlive the handle. */
int se12_bind(const se12_streams* streams, int64_t rows, int64_t cols, int32_t max_batch,
              void* stream, se12_handle** out);

/* Binds a row-major BF16 matrix [rows, cols] for the same-skeleton raw twin.
 * Replaces RawBf16MatVecKernel.__init__ (lws/adapters/cuda/gemv.py:146-155). */
int se12_bind_raw_bf16(const uint16_t* w_dev, int64_t rows, int64_t cols, int32_t max_batch,
                       void* stream, se12_handle** out);

/* Frees the handle's sidecar and workspace (synchronizes its device). */
int se12_release(se12_handle* h);

/* Shape facts of a bound handle (host only). */
int se12_handle_shape(const se12_handle* h, int64_t* rows, int64_t* cols, int64_t* tiles,
                      int64_t* fallback_tiles, int32_t* format);

/* What se12_bind derived for an SE12 handle (host only): `raw_tiles` = the
 * tiles bind decoded once into a raw BF16 buffer of the handle because they
 * hold more escapes than the per-tile side record lists (the kernels read
 * those 8,192 bytes per tile besides the tile's streams); `sidecar_bytes` =
 * the device bytes of the derived data (side records, pair table, that raw
 * buffer). No counterpart in the reference, whose host precompute is
 * fallback_offsets / row_escape_offset (lws/adapters/cuda/gemv.py:47-77). */
int se12_handle_bind_stats(const se12_handle* h, int64_t* raw_tiles, int64_t* sidecar_bytes);

/* The default launch for `batch` (the heuristic of
 * lws/domain/launch/heuristic.py:46-87 re-derived for 256 CUs of wave64). */
int se12_default_launch(const se12_handle* h, int32_t batch, se12_launch* out);

/* Reads `bytes` (16-byte aligned, whole 16-byte words counted) of device
 * memory as a streaming read, the traffic of one pass over a weight matrix,
 * for bandwidth measurement; the kernel writes to out (>= 8 words per compute
 * unit) only in the rare case its XOR of the data equals a fixed constant.
 * No reference counterpart: the reference measures a device copy only
 * (lws/adapters/cuda/benchmark_timer.py:50-66); the roofline here also wants
 * the read-only rate. Same stream rules as se12_gemv. */
int se12_read_probe(const void* buf_dev, int64_t bytes, uint32_t* out_dev, int64_t out_elems, void* stream);

/* Sets the compute-unit count the handle's default launches are derived for
 * (bind takes hipDeviceProp_t.multiProcessorCount). Host only. Replaces the
 * `sm_count` argument that Se12MatVecKernel / RawBf16MatVecKernel take at
 * construction and hand to the default launch heuristic
 * (lws/adapters/cuda/gemv.py:146,183,199). */
int se12_set_compute_units(se12_handle* h, int32_t compute_units);

/* y[b, n] = sum_k W[n, k] * x[b, k] for b < batch (1..32), FP32 accumulate.
 * x: [batch, cols] row-major, BF16 or FP32 (`x_dtype`); y: FP32 [batch, rows].
 * `launch` NULL selects the default. No allocation and no synchronization,
 * so it can be captured in a HIP graph. Calls on one handle must be ordered
 * on one stream (they share the handle's split-K workspace).
 * Replaces the lws_gemv_se12 / lws_gemv_raw_bf16 launches of
 * MatVecKernel.multiply (lws/adapters/cuda/gemv.py:157-172,196-226;
 * kernels: lws/adapters/cuda/kernels/gemv_se12.cu:50-64,
 * gemv_raw_bf16.cu:18-25). */
int se12_gemv(se12_handle* h, const void* x_dev, int32_t x_dtype, int32_t batch, float* y_dev,
              const se12_launch* launch, void* stream);

/* se12_gemv for callers that cannot allocate (code under HIP graph capture,
 * tight serving loops, harnesses that forbid allocation): the same product,
 * launch shapes and results as se12_gemv on the same handle, but its kernels
 * keep their split-K partial sums, pair slots and arrival counters in the
 * library's own static device scratch (8 MiB per GPU, held until the process
 * ends: 65,536 arrival counters, i.e. up to 32,767 tile rows; 262,144 pair
 * slots, i.e. (K splits - 1) x min(batch, 4) x padded rows on the dot2 path;
 * and 1,507,328 partial sums, i.e. K splits x the whole batch x padded rows
 * on the MFMA path) instead of the handle's workspace. A shape or launch
 * beyond those limits fails with SE12_E_CAPACITY before any launch.
 * The call allocates nothing and calls no allocating routine; its first call
 * on a device looks up the scratch and clears its counters and pair slots
 * with a kernel on `stream` (make that first call outside a capture). Every
 * call on one GPU shares that GPU's scratch, whose counters and slots return
 * to zero after each launch: calls that overlap on one GPU (other streams,
 * other threads) race and must be ordered by the caller. No counterpart in
 * the reference. */
int se12_gemv_noalloc(se12_handle* h, const void* x_dev, int32_t x_dtype, int32_t batch, float* y_dev,
                      const se12_launch* launch, void* stream);

/* One launch computing y[i] = W_i x for `count` (1..4) handles of one format
 * bound to matrices with the same number of columns and device (e.g. the q,
 * k and v projections, or gate and up, which read the same x). Each y[i] is
 * FP32 [batch, rows_i]. `launch` counts the handles' tile rows together:
 * blocks = (sum of tile rows) x K splits; NULL selects the default for the
 * combined shape. Results equal those of separate se12_gemv calls under the
 * same waves per block and K splits. Same stream, allocation and ordering
 * rules as se12_gemv; calls on any of the handles must be ordered. No
 * reference counterpart: it serves a runtime that fuses the projections
 * that share an input (lws/adapters/cuda/gemv.py:196-226 runs one GEMV per
 * matrix). */
int se12_gemv_grouped(se12_handle* const* handles, int32_t count, const void* x_dev, int32_t x_dtype,
                      int32_t batch, float* const* y_dev, const se12_launch* launch, void* stream);

/* Products with a decoder step fused into their tail (no reference
 * counterpart: the reference leaves everything but the linear layers to the
 * framework; these let a decode step skip the separate launches of
 * se12_step_gelu_mul and se12_step_rmsnorm, with the same arithmetic).
 *
 * se12_gemv_gelu_mul: the grouped product of two handles with the same rows
 * (gate, up), y[0] and y[1] FP32 [batch, rows] as se12_gemv_grouped, then
 * out[b, n] = bf16(gelu_tanh(bf16(y[0][b, n])) * bf16(y[1][b, n])), BF16
 * [batch, rows].
 *
 * se12_gemv_rmsnorm: y = W x as se12_gemv, then for each batch row
 * residual = bf16(residual + norm(bf16(y)) * (1 + w1)),
 * out = norm(residual) * (1 + w2), norm(t) = t * rsqrt(mean(t^2) + eps) in
 * FP32; residual and out BF16 [batch, rows], w1 and w2 BF16 [rows],
 * rows <= 8192.
 *
 * Where the product runs the dot2 kernel (batch rows per launch <= 4, or FP32
 * x) and, for the norm, rows % 4 == 0, y, w1, w2, residual and out are
 * 8-byte aligned and the row fits a block's LDS (10 bytes per row of W;
 * gfx950 blocks take up to 160 KiB), the block completing the inputs of the
 * step runs it;
 * otherwise (MFMA launches for BF16 x with batch >= 5, longer rows) the
 * separate step kernel follows the product. Same stream, allocation and
 * ordering rules as se12_gemv. */
int se12_gemv_gelu_mul(se12_handle* const* gate_up, const void* x_dev, int32_t x_dtype, int32_t batch,
                       float* const* y_dev, uint16_t* out_dev, const se12_launch* launch, void* stream);
int se12_gemv_rmsnorm(se12_handle* h, const void* x_dev, int32_t x_dtype, int32_t batch, float* y_dev,
                      const uint16_t* w1_dev, const uint16_t* w2_dev, uint16_t* residual_dev, uint16_t* out_dev,
                      float eps, const se12_launch* launch, void* stream);

/* se12_gemv with the sums of squares of the output's tile rows (no reference
 * counterpart; for the decoder's norms): y as se12_gemv, and
 * row_ss[b, t] = sum over the 16 rows n of tile row t of bf16(y[b, n])^2
 * (FP32 [batch, tile rows]), written by the blocks completing each tile row
 * (dot2 launches) or by a small kernel after the product (MFMA launches).
 * Same stream, allocation and ordering rules as se12_gemv. */
int se12_gemv_rowss(se12_handle* h, const void* x_dev, int32_t x_dtype, int32_t batch, float* y_dev,
                    float* row_ss_dev, const se12_launch* launch, void* stream);

/* The product of the decoder's next normalised input, with the norm in the
 * product's head (no reference counterpart; same motivation as above): for
 * each batch row, from the previous product's FP32 output y_prev [batch,
 * cols],
 *   r = bf16(residual_in + norm(bf16(y_prev)) * (1 + w1)),
 *   h = norm(r) * (1 + w2)   (norm as in se12_gemv_rmsnorm),
 * residual_out = r and h_out = h (BF16 [batch, cols]), then y[i] = W_i h for
 * the `count` handles (as se12_gemv_grouped). gelu_out non-NULL (two handles
 * with one row count): the MLP gate of se12_gemv_gelu_mul as well.
 * residual_in and residual_out are either the same tensor or disjoint.
 * Where the product runs the dot2 kernel with BF16 x (batch <= 4), whole K
 * tiles, distinct residuals, 16-byte aligned y_prev and 8-byte aligned
 * weights, residuals and h_out, and a block's LDS holds about cols x (8 x
 * batch + 4) bytes (staged y_prev, residual, weights and x) beside the
 * product's own, every block of the product rebuilds h in LDS (sums of squares
 * over its threads) and block (0, 0) writes residual_out and h_out;
 * otherwise the norm runs as its own kernel (se12_step_rmsnorm mode 1)
 * before the product. y_prev_ss: NULL, or the tile-row sums of squares of
 * y_prev that se12_gemv_rowss wrote with it (FP32 [batch, ceil(cols / 16)]);
 * the fused head then takes the first norm's mean from them instead of a
 * pass over y_prev. Same stream, allocation and ordering rules as
 * se12_gemv. */
int se12_gemv_prenorm(se12_handle* const* handles, int32_t count, const float* y_prev_dev, const float* y_prev_ss_dev,
                      int32_t batch,
                      const uint16_t* w1_dev, const uint16_t* w2_dev, const uint16_t* residual_in_dev,
                      uint16_t* residual_out_dev, uint16_t* h_out_dev, float eps, float* const* y_dev,
                      uint16_t* gelu_out_dev, const se12_launch* launch, void* stream);

/* Decodes the whole matrix to row-major BF16 bits [rows, cols] (cropped).
 * Replaces the lws_se12_decode launch plus the device untile/crop of
 * CudaSe12WeightDecoder (lws/adapters/cuda/se12_decoder.py:58-76,147-185;
 * kernel lws/adapters/cuda/kernels/se12_decode.cu:12-22). */
int se12_decode(se12_handle* h, uint16_t* out_dev, void* stream);

/* Decodes `nrows` rows given by device int64 indices, in that order, to
 * [nrows, cols] BF16 bits; only the tiles covering those rows are read. An
 * index outside [0, rows) yields a row of zeros. Replaces
 * WeightDecoder.decode_rows (lws/application/ports/gpu/weight_decoder.py:30-33,
 * lws/adapters/cuda/se12_decoder.py:64-70). */
int se12_decode_rows(se12_handle* h, const int64_t* rows_dev, int64_t nrows, uint16_t* out_dev,
                     void* stream);

/* Host-only: the 15-entry codebook from a 256-bin exponent histogram of the
 * real weights: descending count, equal counts to the larger exponent value,
 * zero-count values last (lws/domain/se12/codebook.py:41-59). */
int se12_codebook_from_histogram(const uint64_t counts[256], uint8_t codebook_out[15]);

/* Encoder pass 1 on the GPU: exponent histogram of w [rows, cols] (row-major
 * BF16 bits, row stride `ld` elements), codebook, and the number of tiles that
 * exceed the escape budget. Synchronizes `stream`. Together with se12_encode
 * this replaces encode_tensor (lws/domain/se12/codec.py:111-141) for the
 * packer (lws/application/codec/pack_model.py:113-120). */
int se12_encode_prepare(const uint16_t* w_dev, int64_t rows, int64_t cols, int64_t ld,
                        uint8_t codebook_out[15], int64_t* fallback_tiles_out, void* stream);

/* Encoder pass 2: writes every stream for `codebook` (from pass 1). Fails with
 * SE12_E_CAPACITY when out->fallback_raw_tiles is smaller than needed.
 * Synchronizes `stream`. */
int se12_encode(const uint16_t* w_dev, int64_t rows, int64_t cols, int64_t ld,
                const uint8_t codebook[15], const se12_streams_out* out, int64_t* fallback_tiles_out,
                void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SE12_GFX950_H */
