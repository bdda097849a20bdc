/*
 * ivonar_ternary.h - C ABI of the MI355X (gfx950) ternary linear layer.
 *
 * Drop-in replacement for the CUDA kernels the reference decoder launches
 * for its ternary linear ops.  Each entry point has the name and argument
 * order of the reference kernel it replaces (reference paths relative to
 * src/ivonar_inference/), with the launch stream first.  It computes its own
 * grid; the `lanes` argument and the `next`/`next_bytes` L2-prefetch slots
 * are accepted for ABI compatibility and ignored (MI355X has no persisting-L2
 * window; its Infinity Cache needs no hint).
 *
 * Conventions
 *   - Every function returns hipSuccess or a HIP error code; nothing is
 *     synchronised, allocated or read back, so the calls may be recorded
 *     into a HIP graph once ivonar_init() has run for the device.
 *   - All pointers are device pointers on the stream's device.
 *   - packed: uint8 [rows, row_bytes], row_bytes a multiple of 16 and at
 *     least 16*ceil(n/64); byte b holds inputs 4b..4b+3, input 4b+k in bits
 *     2k..2k+1 as code = w + 1 (w in {-1,0,+1}).  16-byte aligned.
 *   - scales: fp16 bit patterns [rows, groups], groups >= ceil(n/128), one
 *     scale per 128 inputs.  bias: fp32 [rows] or NULL.
 *   - q8/xsum/scale buffers hold quantized activations in this library's
 *     private layout; capacity per token row: ceil(n/64)*64 int8,
 *     ceil(n/64) int32 and one fp32 (the reference's q8/q8sum/q8scale sizes).
 *   - fp32 results follow this library's summation order, which the CPU
 *     oracle restates exactly; per-128-group int32 partials are exact.
 */
#ifndef IVONAR_TERNARY_H
#define IVONAR_TERNARY_H

#include <hip/hip_runtime_api.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define IVONAR_ABI_VERSION 1

/* ---------------------------------------------------------------- set-up */

/* Allocates the device's scratch: the activation row a GEMV quantizes in a
 * launch of its own (rows longer than 4096 inputs that the GEMV does not
 * quantize itself: NORM and ATTN rows, unaligned PLAIN rows, rows above
 * 32768 inputs), the 16 MB of fp32 wave chains of a K-sliced token GEMM
 * (1..16 tokens whose q8 rows exceed LDS) with its per-group arrival counts,
 * and the argmax's block count.
 * Besides it, every stream that makes such a call outside graph capture
 * gets a scratch of its own (about 17 MB, kept until the process ends) on
 * its first call, so eager calls on different streams never share one; a
 * call under capture uses its stream's scratch if it has one, else the
 * device's.  The null stream and hipStreamPerThread each use one scratch,
 * whatever thread calls.  Call once per device outside graph capture;
 * replaces the reference's compile_module set-up step
 * (kernels/runtime.py:301-324).  Calls with the device current.  Calling it
 * again clears the arrival counts (argmax, K-sliced token GEMV) of every
 * scratch of the device, with no call of the device in flight. */
hipError_t ivonar_init(int device);

/* Process-wide values the reference passes as -D defines to NVRTC
 * (kernel_decoder.py:215, ternary.cu:1-46): "HEAD_DIM" (ATTN prologue head
 * width, default 64), "TILE" (token rows of quantize_tile_*, default 32),
 * "MAX_CHUNKS" (caller q8 capacity, default 70), "MAX_TOPK" (largest top-k
 * of sample_token, 1..1024, default 256).  Unknown names and out-of-range
 * values return hipErrorInvalidValue. */
hipError_t ivonar_define(const char* name, int value);

const char* ivonar_error_string(hipError_t status);
int ivonar_abi_version(void);

/* Lane layout of the decode GEMV for a K-wide row: lanes per row and rows
 * per lane; the lane count fixes its fp32 summation order.  Host only. */
void ivonar_gemv_plan(int rows, int n, int* lanes, int* rows_per_lane);

/* K-splits S of the token GEMM (gemm_tile_*) for m tokens: its fp32 order is S
 * contiguous ranges of the 128-input groups, each summed in ascending order,
 * then the S partial sums added in order (S = 1: one chain).  S = 0: one
 * token, or two tokens of 4097..32768 inputs, which gemm_tile_* hands to the
 * decode GEMV on each pre-quantized row (gemv_prequant_store's kernel), so
 * each token's order is ivonar_gemv_plan's lane layout.  Uses the current
 * device's LDS size. */
int ivonar_gemm_plan(int m, int rows, int n);

/* ------------------------------------------------------------ decode GEMV
 * GEMV_ARGS of ternary.cu:293-298.  y[r] = s_x * sum_g P[r,g]*scale[r,g]
 * (+ bias[r]).  Prologue: PLAIN quantizes `input`, NORM applies RMSNorm
 * (eps, clip +-8, weight `aux`) first, ATTN merges split-softmax partials
 * [heads, splits, HEAD_DIM+2] first; prequant reads q8_in/xsum_in/scale_in.
 * Epilogue: store, residual (output[r] += y), silu pair (interleaved
 * gate/up rows; output[r/2] = silu(y[r]) * y[r+1], rows even).
 * A 16-byte aligned PLAIN row of 4097..32768 inputs is quantized by every
 * block of the GEMV launch itself, into its own shared memory (no scratch,
 * no waiting between blocks); other rows longer than 4096 inputs are
 * quantized into the stream's scratch (see ivonar_init) by a separate
 * quantizer launch and then read by the GEMV.  Calls in one stream order are
 * safe, and so are eager calls on different streams; graphs whose captured
 * calls share a scratch (captured on one stream, or on streams that had
 * none) give undefined outputs for those calls when replayed at once. */
#define IVONAR_GEMV_ARGS                                                                                    \
  const float *input, const float *aux, const int8_t *q8_in, const int32_t *xsum_in, const float *scale_in, \
      const uint8_t *packed, const uint16_t *scales, const float *bias, float *output, int rows, int n,      \
      int row_bytes, int groups, int lanes, int splits, float eps, const uint8_t *next, int next_bytes

/* ternary.cu:356-358 */
hipError_t gemv_plain_store(hipStream_t stream, IVONAR_GEMV_ARGS);
/* ternary.cu:359-361 */
hipError_t gemv_plain_residual(hipStream_t stream, IVONAR_GEMV_ARGS);
/* ternary.cu:365-367 */
hipError_t gemv_norm_store(hipStream_t stream, IVONAR_GEMV_ARGS);
/* ternary.cu:368-370 */
hipError_t gemv_norm_silu_pair(hipStream_t stream, IVONAR_GEMV_ARGS);
/* ternary.cu:371-373 */
hipError_t gemv_attn_residual(hipStream_t stream, IVONAR_GEMV_ARGS);
/* ternary.cu:374-376 (LM head: reads q8_in/xsum_in/scale_in) */
hipError_t gemv_prequant_store(hipStream_t stream, IVONAR_GEMV_ARGS);
/* ternary.cu:377-388: the _wide variants (K > 1024) share the kernels above. */
hipError_t gemv_plain_store_wide(hipStream_t stream, IVONAR_GEMV_ARGS);
hipError_t gemv_plain_residual_wide(hipStream_t stream, IVONAR_GEMV_ARGS);
hipError_t gemv_norm_store_wide(hipStream_t stream, IVONAR_GEMV_ARGS);
hipError_t gemv_norm_silu_pair_wide(hipStream_t stream, IVONAR_GEMV_ARGS);
hipError_t gemv_attn_residual_wide(hipStream_t stream, IVONAR_GEMV_ARGS);

/* No reference counterpart; for callers that cannot allocate device memory
 * (code under graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  gemv_plain_store with the same arguments and results, except
 * that a row longer than 4096 inputs that the GEMV launch does not quantize
 * itself (an input not 16-byte aligned) is quantized into a fixed
 * 35,072-byte array of the library's device code (one per device, set up on
 * the first call on each device) instead of the scratch gemv_plain_store
 * allocates: nothing is allocated or freed, by this call or the library.  n above
 * 32768 returns hipErrorInvalidValue.  Every call on a device shares that
 * array, so calls that overlap on one device race (their outputs are
 * undefined); calls in one stream order are safe.  Nothing in the array
 * needs to start at zero: each call writes all of it that it reads. */
hipError_t ivonar_gemv_plain_store_noalloc(hipStream_t stream, IVONAR_GEMV_ARGS);

/* Test export (no reference counterpart; requested by the decode-path parity
 * checks): the exact int32 partials P[r, g] of the GEMV's integer core, from
 * pre-quantized activations, into partials int32 [rows, groups]. */
hipError_t gemv_group_partials(hipStream_t stream, const int8_t* q8_in, const int32_t* xsum_in,
                               const uint8_t* packed, int rows, int n, int row_bytes, int groups,
                               int32_t* partials);

/* -------------------------------------------------------------- quantizer */

/* QUANT_ARGS of ternary.cu:390-392 (quantize_norm :404-409): one token row. */
hipError_t quantize_norm(hipStream_t stream, const float* input, const float* aux, int n, float eps, int splits,
                         int8_t* q8_out, int32_t* xsum_out, float* scale_out);
hipError_t quantize_norm_wide(hipStream_t stream, const float* input, const float* aux, int n, float eps,
                              int splits, int8_t* q8_out, int32_t* xsum_out, float* scale_out);

/* QUANT_TILE_ARGS of ternary.cu:632-634 (quantize_tile_* :652-669): TILE
 * token rows, row t read from input + t*in_stride; q8 row stride
 * ceil(n/64)*64, xsum row stride ceil(n/64). */
#define IVONAR_QUANT_TILE_ARGS                                                                           \
  const float *input, int in_stride, const float *aux, int n, float eps, int splits, int8_t *q8_out, \
      int32_t *xsum_out, float *scale_out
hipError_t quantize_tile_plain(hipStream_t stream, IVONAR_QUANT_TILE_ARGS);
hipError_t quantize_tile_plain_wide(hipStream_t stream, IVONAR_QUANT_TILE_ARGS);
hipError_t quantize_tile_norm(hipStream_t stream, IVONAR_QUANT_TILE_ARGS);
hipError_t quantize_tile_norm_wide(hipStream_t stream, IVONAR_QUANT_TILE_ARGS);
hipError_t quantize_tile_attn(hipStream_t stream, IVONAR_QUANT_TILE_ARGS);
hipError_t quantize_tile_attn_wide(hipStream_t stream, IVONAR_QUANT_TILE_ARGS);

/* Same quantizer for an explicit row count m and mode (0 PLAIN, 1 NORM,
 * 2 ATTN); the reference launches its tile quantizers with grid = m
 * (kernel_decoder.py:370-386). */
hipError_t ivonar_quantize_rows(hipStream_t stream, int mode, const float* input, int in_stride, const float* aux,
                                int n, float eps, int splits, int m, int8_t* q8_out, int32_t* xsum_out,
                                float* scale_out);

/* ---------------------------------------------------------- token GEMM
 * GEMM_ARGS of ternary.cu:671-674 (gemm_tile_* :767-784): m token rows of
 * pre-quantized activations against `rows` weight rows on int8 MFMA; output
 * row t at output + t*out_stride.  For 1..16 tokens with n a multiple of 256
 * whose q8 rows exceed LDS, the call is two launches through the stream's
 * scratch (see ivonar_init), with the same concurrency rule as the GEMV's. */
#define IVONAR_GEMM_ARGS                                                                                      \
  const int8_t *q8_in, const int32_t *xsum_in, const float *scale_in, const uint8_t *packed,              \
      const uint16_t *scales, const float *bias, float *output, int rows, int n, int row_bytes, int groups, \
      int lanes, int out_stride, int m
hipError_t gemm_tile_store(hipStream_t stream, IVONAR_GEMM_ARGS);
hipError_t gemm_tile_residual(hipStream_t stream, IVONAR_GEMM_ARGS);
hipError_t gemm_tile_silu_pair(hipStream_t stream, IVONAR_GEMM_ARGS);
hipError_t gemm_tile_store_wide(hipStream_t stream, IVONAR_GEMM_ARGS);
hipError_t gemm_tile_residual_wide(hipStream_t stream, IVONAR_GEMM_ARGS);
hipError_t gemm_tile_silu_pair_wide(hipStream_t stream, IVONAR_GEMM_ARGS);

/* ------------------------------------------------------------- embedding */

/* ternary.cu:411-419: output[i] = (code[token, i] - 1) * scale[token, i/128]. */
hipError_t embed_token(hipStream_t stream, const int64_t* token, const uint8_t* packed, const uint16_t* scales,
                       float* output, int n, int row_bytes, int groups);
/* ternary.cu:613-622: m token rows into output [m, n]. */
hipError_t embed_tile(hipStream_t stream, const int64_t* tokens, const uint8_t* packed, const uint16_t* scales,
                      float* output, int n, int row_bytes, int groups, int m);
/* ternary.cu:624-630: output = tile[max(*valid - 1, 0)]. */
hipError_t gather_token(hipStream_t stream, const float* tile, float* output, int n, const int64_t* valid);

/* Greedy token: first index of the maximum of values[0..n) (no reference
 * counterpart as a kernel; the reference's greedy sampler is top_k = 1 of
 * sample_token, ternary.cu:1099-1337). */
hipError_t ivonar_argmax(hipStream_t stream, const float* values, int n, int64_t* out);

/* --------------------------------------------------------------- sampler
 * The reference's on-device sampler (ternary.cu:1083-1092 and :1098-1337,
 * launched by kernel_decoder.py:619-634), argument order kept.  Rule:
 * score = logits[i] * (1 / *temperature), multiplied by *inverse_penalty
 * (score > 0) or *penalty (score <= 0) where seen[i]; the k = clamp(*top_k,
 * 1, min(MAX_TOPK, vocab)) largest scores (ties at the cut: lowest index);
 * softmax over them; inverse-CDF draw with *uniform in [0, 1) over the picks
 * in ascending index order.  token[0] and history[0] (if not NULL) receive
 * the draw and seen[token] is set to 1.  vocab <= 262144.  bounds holds
 * ceil(vocab / 64) floats (the largest score of each 64-entry group) and is
 * written by logit_bounds, read by sample_token; the two run back to back on
 * one stream with the same logits, seen and rule. */
hipError_t logit_bounds(hipStream_t stream, const float* logits, const float* temperature, const float* penalty,
                        const float* inverse_penalty, const uint8_t* seen, float* bounds, int vocab);
hipError_t sample_token(hipStream_t stream, const float* logits, const float* bounds, const float* temperature,
                        const float* penalty, const float* inverse_penalty, uint8_t* seen, const int64_t* top_k,
                        const float* uniform, int64_t* token, int64_t* history, int vocab);

/* ------------------------------------------------------ checkpoint checks
 * The packed-buffer tests of the reference loader (loader.py:94-112), on the
 * device: ORs into flags[0] bit 0 when a byte of packed[0..packed_bytes)
 * holds the reserved code 3, bit 1 when a scale of scales[0..scale_count) is
 * not finite, bit 2 when one is not positive.  The caller zeroes flags first
 * and reads it after the stream completes.  Both buffers 16-byte aligned. */
hipError_t ivonar_validate_ternary(hipStream_t stream, const uint8_t* packed, long long packed_bytes,
                                   const uint16_t* scales, long long scale_count, unsigned* flags);

/* Measurement export (no reference counterpart): reads `bytes` (a multiple of
 * 16, 16-byte aligned) of `data` with 16-byte loads at full occupancy and
 * writes nothing in practice; `sink` must hold ivonar_stream_read_sink_words()
 * uint32.  Its bandwidth is the streaming-read ceiling the GEMV is compared
 * with. */
int ivonar_stream_read_sink_words(void);
hipError_t ivonar_stream_read(hipStream_t stream, const void* data, long long bytes, unsigned* sink);

/* Test export (no reference counterpart): the largest number of row-tile
 * groups whose K-sliced token GEMV is finished inside its own launch (by the
 * last slice of each group); larger calls add the slices' chains in a second
 * kernel.  Default and maximum 992; 0 makes every K-sliced call take the
 * second kernel.  Process-wide; returns the previous value, or -1 (and
 * changes nothing) for a value outside 0..992. */
int ivonar_token_finish_limit(int groups);

#ifdef __cplusplus
}
#endif

#endif /* IVONAR_TERNARY_H */
