/* Decode-step kernels for a Gemma-2 style decoder, in libse12_gfx950.so.
 *
 * No counterpart in the reference: its runtime leaves everything but the
 * linear layers to the framework (.spec/features/model-integration/spec.md,
 * "Out of scope: changes to attention, KV cache or sampling"). These exist so
 * that an end-to-end decode step is a few launches around the fused SE12
 * products (se12_amd/gemma2.py), with the framework's BF16 rounding sequence.
 *
 * All pointers are device memory; every call is asynchronous on `stream`
 * (a hipStream_t), allocates nothing and is graph-capturable. Returns
 * SE12_STEP_OK or a negative code; se12_step_last_error() gives the message.
 */
#ifndef SE12_STEP_H
#define SE12_STEP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SE12_STEP_OK 0
#define SE12_STEP_E_INVALID (-1)
#define SE12_STEP_E_HIP (-2)

/* element type of an input tensor (outputs are always BF16) */
#define SE12_STEP_BF16 0
#define SE12_STEP_F32 1

const char* se12_step_last_error(void);

/* mode 0: out = norm(x) * (1 + w1), x = in (rounded to BF16, times in_scale
 *         when in_scale != 0, e.g. sqrt(hidden) for Gemma's embedding); when
 *         residual is not NULL it receives x.
 * mode 1: residual = bf16(residual + norm(bf16(in)) * (1 + w1));
 *         out = norm(residual) * (1 + w2).
 * norm(x) = x * rsqrt(mean(x^2) + eps) in FP32. in: [rows, in_stride];
 * residual, out: [rows, hidden] BF16; w1, w2: [hidden] BF16; hidden <= 8192. */
int se12_step_rmsnorm(const void* in, int32_t in_dtype, int64_t in_stride, const uint16_t* w1, uint16_t* residual,
                      const uint16_t* w2, uint16_t* out, int32_t rows, int32_t hidden, float eps, float in_scale,
                      int32_t mode, void* stream);

/* One decode step of grouped-query attention at position *pos for every
 * sequence: q [batch, q_stride] (heads x head_dim used), k and v
 * [batch, kv_stride]; rotary embedding with inv_freq[head_dim / 2]; the
 * rotated key and the value are written to k_cache_t [batch, kv_heads,
 * head_dim, max_len] and v_cache [batch, kv_heads, max_len, head_dim] at
 * *pos; scores = (q . k) * scaling, soft-capped tanh(s / softcap) * softcap
 * when softcap > 0, over positions max(0, *pos - window + 1) .. *pos
 * (window 0 = all); softmax in FP32, probabilities rounded to BF16; out
 * [batch, heads * head_dim] BF16. head_dim a multiple of 8 up to 256;
 * max_len a multiple of 8; heads / kv_heads in {1, 2, 4, 8}; both caches
 * 16-byte aligned. A *pos outside [0, max_len) writes zeros to out and
 * nothing to the caches.
 *
 * Two launches over (sequence, KV head, 64-position chunk). `workspace`
 * (device, 256-byte aligned, se12_step_attention_workspace() bytes for the
 * shape) holds scores, chunk statistics, partial sums and arrival counters:
 * zero-fill it once before its first use; each call leaves the counters at
 * zero again. Calls sharing a workspace must not run concurrently. */
int64_t se12_step_attention_workspace(int32_t batch, int32_t heads, int32_t kv_heads, int32_t head_dim,
                                      int32_t max_len);

int se12_step_attention(const void* q, const void* k, const void* v, int32_t dtype, int64_t q_stride, int64_t kv_stride,
                        uint16_t* k_cache_t, uint16_t* v_cache, const float* inv_freq, const int64_t* pos, uint16_t* out,
                        int32_t batch, int32_t heads, int32_t kv_heads, int32_t head_dim, int32_t max_len, float scaling,
                        float softcap, int32_t window, void* workspace, int64_t workspace_bytes, void* stream);

/* out[r, c] = bf16(gelu_tanh(bf16(gate[r, c])) * bf16(up[r, c])); gate and up
 * [rows, stride], out [rows, cols]. */
int se12_step_gelu_mul(const void* gate, const void* up, int32_t dtype, int64_t stride, uint16_t* out, int32_t rows,
                       int32_t cols, void* stream);

/* Per row: z = bf16(logits) soft-capped (softcap > 0), stored to logits_out
 * [rows, vocab] when not NULL; the first index of the maximum goes to ids[row]
 * and to tokens[row * token_stride + *step] (skipped when *step is outside
 * [0, token_stride)). rows <= 65535.
 *
 * Blocks over slices of 2,048 logits per row; `workspace` (device, 256-byte
 * aligned, se12_step_logits_workspace() bytes) holds their partial results
 * and arrival counters: zero-fill it once before its first use; each call
 * leaves the counters at zero again. Calls sharing a workspace must not run
 * concurrently. */
int64_t se12_step_logits_workspace(int32_t rows, int32_t vocab);

int se12_step_logits_argmax(const void* logits, int32_t dtype, int64_t stride, int32_t rows, int32_t vocab, float softcap,
                            uint16_t* logits_out, int64_t* ids, int64_t* tokens, int64_t token_stride,
                            const int64_t* step, void* workspace, int64_t workspace_bytes, void* stream);

/* *pos += 1, *step += 1 (device counters of a captured decode loop). */
int se12_step_advance(int64_t* pos, int64_t* step, void* stream);

/* se12_step_logits_argmax followed by se12_step_advance, in one launch: once
 * every row's pick is stored (the rows read *step first), the last row's
 * final block sets *pos += 1 and *step += 1. Same workspace. Saves the
 * decode loop the advance launch; no counterpart in the reference, whose
 * sampling is the framework's. */
int se12_step_logits_argmax_advance(const void* logits, int32_t dtype, int64_t stride, int32_t rows, int32_t vocab,
                                    float softcap, uint16_t* logits_out, int64_t* ids, int64_t* tokens,
                                    int64_t token_stride, int64_t* step, int64_t* pos, void* workspace,
                                    int64_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SE12_STEP_H */
