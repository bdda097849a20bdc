// Host-side launchers shared by the C-ABI entry points (capi.cpp).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>

namespace ivo {

// Process-wide values the reference passes as compile-time defines
// (kernel_decoder.py:215): HEAD_DIM for the ATTN prologue, TILE for the
// token count of the quantize_tile_* entry points, MAX_CHUNKS (capacity of
// the caller's q8 buffers, used only for argument checks) and MAX_TOPK
// (largest top-k of the sampler, ternary.cu:8).  Atomic, so that
// ivonar_define on one thread and a launch on another never race (a launch
// reads each value once).
constexpr int kMaxTopK = 1024;
constexpr int kMaxSampleVocab = 1 << 18;
struct Defines {
  std::atomic<int> head_dim{64};
  std::atomic<int> tile{32};
  std::atomic<int> max_chunks{70};
  std::atomic<int> max_topk{256};
  // Tile groups of a K-sliced token GEMV finished in-launch (at most the
  // scratch's counters; ivonar_token_finish_limit).
  std::atomic<int> token_finish_groups{992};
};
Defines& defines();

// Per-device activation scratch for the two-pass GEMV (quantize, then GEMV).
struct Scratch {
  int8_t* q8 = nullptr;
  int32_t* xsum = nullptr;
  float* scale = nullptr;
  int capacity_chunks = 0;
  float* token_partials = nullptr;  // fp32 wave partials of the K-sliced token GEMV
  // Counters that start and end every launch at zero (kSyncBytes): the
  // argmax's block count and the sliced token GEMV's tile-group arrivals.
  unsigned* sync = nullptr;
};
constexpr int kSyncBytes = 4096;
// The argmax's block count, in the last 128-byte line of the sync region.
constexpr int kArgmaxCountWord = kSyncBytes / 4 - 32;
// Arrival counters of the K-sliced token GEMV's tile groups: the sync
// region's words 0 .. kTokenFinishCounters - 1.
constexpr int kTokenFinishCounters = kArgmaxCountWord;
static_assert(kTokenFinishCounters == 992, "the default of Defines::token_finish_groups");
// Capacity of Scratch::token_partials (floats; 16 MB per device).
constexpr long long kTokenPartialFloats = 4LL << 20;
hipError_t scratch_for_stream(hipStream_t stream, Scratch** out);
hipError_t init_device(int device);

struct QuantArgs {
  int mode;
  const float* input;
  int in_stride;
  const float* aux;
  int n;
  float eps;
  int splits;
  int head_dim;
  int m;
  int8_t* q8;
  int32_t* xsum;
  float* scale;
  // Write each quad in the nibble-split form the 4-bit GEMV reads (split_quad_word)
  // instead of q8 bytes; the chunk sums and the scale are the same.
  bool split = false;
};
hipError_t launch_quantize(hipStream_t stream, const QuantArgs& a);

struct GemvArgs {
  int mode;    // kPlain / kNorm / kAttn (ignored when q8_in is set)
  int epi;     // kStore / kResidual / kSiluPair / kPartials
  const float* input;
  const float* aux;
  const int8_t* q8_in;  // pre-quantized activations (q8 layout) or null
  const int32_t* xsum_in;
  const float* scale_in;
  const uint8_t* packed;
  const uint16_t* scales;
  const float* bias;
  float* output;
  int32_t* partials;  // kPartials only: int32 [rows, groups]
  // Where a row longer than the fused limit is quantized to when q8_in is
  // null: this buffer if set (capacity work_chunks chunks), else the device
  // scratch allocated by the library.
  Scratch* work;
  int rows;
  int n;
  int row_bytes;
  int groups;
  int splits;
  float eps;
  int head_dim;
};
hipError_t launch_gemv(hipStream_t stream, const GemvArgs& a);
// Two tokens of pre-quantized rows through the long-row GEMV (4097..32768
// inputs): each token's outputs are bit-identical to the one-token GEMV's on
// its row.  (Three tokens this way ran slower than the token GEMV.)
constexpr int kGemvTokensMax = 2;
bool gemv_tokens_apply(int m, int n);
hipError_t launch_gemv_tokens(hipStream_t stream, const GemvArgs& a, int m, int out_stride);

// Lane layout the decode GEMV uses for a K-wide row (also defines its fp32
// summation order): lanes per row (power of two in [2, 64]) and rows per lane.
void gemv_plan(int rows, int n, int* lanes, int* rows_per_lane);
int gemv_fused_limit();
// Whether the decode GEMV takes a pre-quantized K = n row (its LDS bound).
bool gemv_prequant_applies(int n);

struct GemmArgs {
  int epi;  // kStore / kResidual / kSiluPair
  const int8_t* q8_in;
  const int32_t* xsum_in;
  const float* scale_in;
  const uint8_t* packed;
  const uint16_t* scales;
  const float* bias;
  float* output;
  int rows;
  int n;
  int row_bytes;
  int groups;
  int out_stride;
  int m;
};
hipError_t launch_gemm(hipStream_t stream, const GemmArgs& a);
// Long-prompt token GEMM (64- or 128-token wave tiles, LDS DMA staging); same
// fp32 order as the tiled GEMM.
int gemm_wide_tokens(int m, int rows, int n);  // token tile (128, 64 or 32), 0 = does not apply
hipError_t launch_gemm_wide(hipStream_t stream, const GemmArgs& a);
// Long-prompt token GEMM split four ways along K (few output rows); its fp32
// order is four contiguous group ranges added in order.
bool gemm_split_applies(int m, int rows, int n);
int split_waves(int m, int rows, int n);  // K-splits of the split-K kernel (4 or 8)
hipError_t launch_gemm_split(hipStream_t stream, const GemmArgs& a);

// K-splits of the GEMM for m tokens (its fp32 order: S contiguous group ranges,
// each an fmaf chain, added in order); 1 = one chain over all groups; 0 = one
// token, run by the decode GEMV (its order is the GEMV's lane layout).
int gemm_splits(int m, int rows, int n);
int max_lds_per_block();
// Skinny token GEMM (m <= 32, and up to kSlicedTokens in 32-token slices):
// K-splits (its fp32 order), 16-row tiles per wave and, for the kernel that
// stages the token tile in LDS, the register slots for groups per wave (0: the
// token operand is read from the caches); splits == 0 means it does not apply.
constexpr int kSlicedTokens = 512;
struct SkinnyPlan {
  int splits;
  int row_tiles;
  int lds_groups;
};
SkinnyPlan skinny_plan(int m, int rows, int n, size_t max_lds);
hipError_t launch_skinny(hipStream_t stream, const GemmArgs& a, SkinnyPlan plan);
// Token GEMV (1..16 tokens, K a multiple of 256, the tokens' q8 rows resident
// in LDS): K-split into `parts` contiguous ranges of `part_spans` 256-input
// spans (its fp32 order, as the GEMM's splits); parts == 0 means it does not
// apply.
struct TokenPlan {
  int parts;  // waves per row tile within one K slice
  int part_spans;
  int tiles_per_block;
  int fill;
  size_t lds;
  int slices;  // K slices (blocks along grid y); above 1 the wave partials go through the scratch
};
TokenPlan token_gemv_plan(int m, int rows, int n, int cus, size_t max_lds);
hipError_t launch_token_gemv(hipStream_t stream, const GemmArgs& a, const TokenPlan& plan);
// Compute units of the current device.
int device_cus();

hipError_t launch_embed(hipStream_t stream, const int64_t* tokens, int m, const uint8_t* packed,
                        const uint16_t* scales, float* output, int n, int row_bytes, int groups);
hipError_t launch_gather(hipStream_t stream, const float* tile, float* output, int n, const int64_t* valid);
hipError_t launch_argmax(hipStream_t stream, const float* values, int n, int64_t* out);
hipError_t launch_logit_bounds(hipStream_t stream, const float* logits, const float* temperature,
                               const float* penalty, const float* inverse_penalty, const uint8_t* seen,
                               float* bounds, int vocab);
hipError_t launch_sample_token(hipStream_t stream, const float* logits, const float* bounds, const float* temperature,
                               const float* penalty, const float* inverse_penalty, uint8_t* seen,
                               const int64_t* top_k, const float* uniform, int64_t* token, int64_t* history,
                               int vocab);
// Reserved codes in a packed operand (flag 1), non-finite (2) or non-positive
// (4) fp16 scales, ORed into flags[0]; packed and scales 16-byte aligned.
hipError_t launch_validate(hipStream_t stream, const uint8_t* packed, long long packed_bytes, const uint16_t* scales,
                           long long scale_count, unsigned* flags);
// Streaming-read reference (measurement): reads bytes/16 16-byte words of data;
// sink holds stream_read_sink_words() uint32 and is written only in theory.
int stream_read_sink_words();
hipError_t launch_stream_read(hipStream_t stream, const void* data, long long bytes, unsigned* sink);

inline int ceil_div(int a, int b) { return (a + b - 1) / b; }

}  // namespace ivo
