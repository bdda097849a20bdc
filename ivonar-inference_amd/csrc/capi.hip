// C-ABI entry points (declared in include/ivonar_ternary.h): argument checks,
// process defines, the per-device and per-stream scratch, and dispatch to the launchers.
#include <stdint.h>
#include <string.h>

#include <map>
#include <mutex>
#include <utility>

#include "ivonar_ternary.h"
#include "internal.hpp"
#include "ternary_device.hpp"

namespace ivo {

Defines& defines() {
  static Defines values;
  return values;
}

namespace {

constexpr int kMaxDevices = 64;
constexpr int kScratchChunks = 16384;  // rows up to 1,048,576 inputs
// Scratch per (device, stream): the device's own (set up by ivonar_init, used
// by the null stream and by calls under graph capture on a stream that has
// none yet), and one per stream that calls outside capture, so that eager
// calls on different streams never share one.  Entries are kept until the
// process ends (a stream handle that HIP hands out again after its stream
// was destroyed finds the same scratch, which its predecessor no longer uses).
std::mutex g_scratch_lock;
Scratch g_scratch[kMaxDevices];
std::map<std::pair<int, uintptr_t>, Scratch> g_stream_scratch;  // node-based: entries never move

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

hipError_t allocate_scratch(Scratch& s) {
  if (s.q8 != nullptr) return hipSuccess;
  void* q8 = nullptr;
  void* xsum = nullptr;
  void* scale = nullptr;
  void* partials = nullptr;
  void* sync = nullptr;
  hipError_t status = hipMalloc(&q8, (size_t)kScratchChunks * kChunk);
  if (status == hipSuccess) status = hipMalloc(&xsum, (size_t)kScratchChunks * sizeof(int32_t));
  if (status == hipSuccess) status = hipMalloc(&scale, 256);
  if (status == hipSuccess) status = hipMalloc(&partials, (size_t)kTokenPartialFloats * sizeof(float));
  if (status == hipSuccess) status = hipMalloc(&sync, kSyncBytes);
  if (status == hipSuccess) status = hipMemset(sync, 0, kSyncBytes);  // the argmax's block count starts at zero
  if (status != hipSuccess) {
    if (q8) (void)hipFree(q8);
    if (xsum) (void)hipFree(xsum);
    if (scale) (void)hipFree(scale);
    if (partials) (void)hipFree(partials);
    if (sync) (void)hipFree(sync);
    return status;
  }
  s.q8 = static_cast<int8_t*>(q8);
  s.xsum = static_cast<int32_t*>(xsum);
  s.scale = static_cast<float*>(scale);
  s.sync = static_cast<unsigned*>(sync);
  s.token_partials = static_cast<float*>(partials);
  s.capacity_chunks = kScratchChunks;
  return hipSuccess;
}

// Checks shared by the GEMV and GEMM entry points.
hipError_t check_matrix(const uint8_t* packed, const uint16_t* scales, int rows, int n, int row_bytes, int groups) {
  if (rows < 0 || n <= 0 || packed == nullptr || scales == nullptr) return hipErrorInvalidValue;
  const int chunks = ceil_div(n, kChunk);
  if (row_bytes < chunks * 16 || (row_bytes & 15) != 0 || !aligned16(packed)) return hipErrorInvalidValue;
  if (groups < ceil_div(n, kGroup)) return hipErrorInvalidValue;
  return hipSuccess;
}

hipError_t gemv_entry(hipStream_t stream, int mode, int epi, bool prequant, const float* input, const float* aux,
                      const int8_t* q8_in, const int32_t* xsum_in, const float* scale_in, const uint8_t* packed,
                      const uint16_t* scales, const float* bias, float* output, int rows, int n, int row_bytes,
                      int groups, int splits, float eps, Scratch* work = nullptr) {
  hipError_t status = check_matrix(packed, scales, rows, n, row_bytes, groups);
  if (status != hipSuccess) return status;
  if (output == nullptr) return hipErrorInvalidValue;
  if (epi == kSiluPair && (rows & 1) != 0) return hipErrorInvalidValue;
  const int head_dim = defines().head_dim;  // read once: checked and used with the same value
  if (prequant) {
    if (q8_in == nullptr || xsum_in == nullptr || scale_in == nullptr || !aligned16(q8_in))
      return hipErrorInvalidValue;
  } else {
    if (input == nullptr) return hipErrorInvalidValue;
    if (mode == kNorm && aux == nullptr) return hipErrorInvalidValue;
    if (mode == kAttn && (splits <= 0 || n % head_dim != 0)) return hipErrorInvalidValue;
  }
  GemvArgs a{};
  a.mode = mode;
  a.epi = epi;
  a.input = input;
  a.aux = aux;
  a.q8_in = prequant ? q8_in : nullptr;
  a.xsum_in = prequant ? xsum_in : nullptr;
  a.scale_in = prequant ? scale_in : nullptr;
  a.packed = packed;
  a.scales = scales;
  a.bias = bias;
  a.output = output;
  a.partials = nullptr;
  a.work = work;
  a.rows = rows;
  a.n = n;
  a.row_bytes = row_bytes;
  a.groups = groups;
  a.splits = splits > 0 ? splits : 1;
  a.eps = eps;
  a.head_dim = head_dim;
  return launch_gemv(stream, a);
}

// ------------------------------------------------ no-allocation GEMV scratch
// Rows longer than the fused limit that the long-row GEMV does not quantize
// itself (unaligned inputs) are quantized before the GEMV; the no-allocation
// entry point quantizes them into this array (q8, chunk sums, token scale)
// instead of the scratch the library allocates, in a launch of its own
// (nothing in the array must start at zero).  Each device holds its own copy
// at its own address, looked up once per device with hipGetSymbolAddress;
// host code uses only that address.
constexpr int kStaticChunks = 512;  // rows up to 32768 inputs
constexpr size_t kStaticQ8Bytes = (size_t)kStaticChunks * kChunk;
constexpr size_t kStaticScaleOffset = kStaticQ8Bytes + (size_t)kStaticChunks * sizeof(int32_t);
constexpr size_t kStaticBytes = kStaticScaleOffset + 256;
static __device__ __align__(256) unsigned char scratch[kStaticBytes];
std::mutex g_static_lock;
Scratch g_static[kMaxDevices];

hipError_t static_scratch(Scratch** out) {
  int device = 0;
  hipError_t status = hipGetDevice(&device);
  if (status != hipSuccess) return status;
  if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> guard(g_static_lock);
  Scratch& s = g_static[device];
  if (s.q8 == nullptr) {
    void* base = nullptr;
    status = hipGetSymbolAddress(&base, HIP_SYMBOL(scratch));
    if (status != hipSuccess) return status;
    unsigned char* bytes = static_cast<unsigned char*>(base);
    s.xsum = reinterpret_cast<int32_t*>(bytes + kStaticQ8Bytes);
    s.scale = reinterpret_cast<float*>(bytes + kStaticScaleOffset);
    s.sync = nullptr;  // no counters: the GEMV uses none, and the argmax takes its own scratch
    s.capacity_chunks = kStaticChunks;
    s.q8 = reinterpret_cast<int8_t*>(bytes);
  }
  *out = &s;
  return hipSuccess;
}

hipError_t quant_entry(hipStream_t stream, int mode, const float* input, int in_stride, const float* aux, int n,
                       float eps, int splits, int m, int8_t* q8_out, int32_t* xsum_out, float* scale_out) {
  if (n <= 0 || m < 0 || input == nullptr || q8_out == nullptr || xsum_out == nullptr || scale_out == nullptr)
    return hipErrorInvalidValue;
  if (!aligned16(q8_out) || ((uintptr_t)xsum_out & 3u) != 0) return hipErrorInvalidValue;
  if (mode == kNorm && aux == nullptr) return hipErrorInvalidValue;
  const int head_dim = defines().head_dim;  // read once: checked and used with the same value
  if (mode == kAttn && (splits <= 0 || n % head_dim != 0)) return hipErrorInvalidValue;
  if (mode < kPlain || mode > kAttn) return hipErrorInvalidValue;
  if (m > 1 && in_stride < (mode == kAttn ? 1 : n)) return hipErrorInvalidValue;
  QuantArgs q{mode, input, in_stride, aux, n, eps, splits > 0 ? splits : 1, head_dim, m,
              q8_out, xsum_out, scale_out};
  return launch_quantize(stream, q);
}

hipError_t gemm_entry(hipStream_t stream, int epi, const int8_t* q8_in, const int32_t* xsum_in,
                      const float* scale_in, const uint8_t* packed, const uint16_t* scales, const float* bias,
                      float* output, int rows, int n, int row_bytes, int groups, int out_stride, int m) {
  hipError_t status = check_matrix(packed, scales, rows, n, row_bytes, groups);
  if (status != hipSuccess) return status;
  if (m < 0 || q8_in == nullptr || xsum_in == nullptr || scale_in == nullptr || output == nullptr)
    return hipErrorInvalidValue;
  if (!aligned16(q8_in)) return hipErrorInvalidValue;
  if (epi == kSiluPair && (rows & 1) != 0) return hipErrorInvalidValue;
  const int width = epi == kSiluPair ? rows / 2 : rows;
  if (m > 1 && out_stride < width) return hipErrorInvalidValue;
  GemmArgs a{epi, q8_in, xsum_in, scale_in, packed, scales, bias, output, rows, n, row_bytes, groups, out_stride, m};
  return launch_gemm(stream, a);
}

}  // namespace

hipError_t init_device(int device) {
  if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> guard(g_scratch_lock);
  int current = 0;
  hipError_t status = hipGetDevice(&current);
  if (status != hipSuccess) return status;
  if (current != device) {
    status = hipSetDevice(device);
    if (status != hipSuccess) return status;
  }
  status = allocate_scratch(g_scratch[device]);
  // The argmax's block count is zero between launches; clearing it here
  // recovers a scratch that overlapping graph replays left set.
  if (status == hipSuccess) status = hipMemset(g_scratch[device].sync, 0, kSyncBytes);
  for (auto it = g_stream_scratch.lower_bound({device, 0}); status == hipSuccess && it != g_stream_scratch.end() &&
                                                             it->first.first == device;
       ++it)
    status = hipMemset(it->second.sync, 0, kSyncBytes);
  if (current != device) (void)hipSetDevice(current);
  return status;
}

hipError_t scratch_for_stream(hipStream_t stream, Scratch** out) {
  int device = 0;
  hipError_t status = hipGetDevice(&device);
  if (status != hipSuccess) return status;
  if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
  hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
  status = hipStreamIsCapturing(stream, &capture);
  if (status != hipSuccess) return status;
  const bool capturing = capture != hipStreamCaptureStatusNone;
  std::lock_guard<std::mutex> guard(g_scratch_lock);
  if (stream != nullptr) {
    const std::pair<int, uintptr_t> key{device, reinterpret_cast<uintptr_t>(stream)};
    auto found = g_stream_scratch.find(key);
    if (found != g_stream_scratch.end()) {
      *out = &found->second;
      return hipSuccess;
    }
    if (!capturing) {
      Scratch fresh;
      status = allocate_scratch(fresh);
      if (status != hipSuccess) return status;
      *out = &g_stream_scratch.emplace(key, fresh).first->second;
      return hipSuccess;
    }
  }
  if (g_scratch[device].q8 == nullptr) {
    if (capturing) return hipErrorStreamCaptureUnsupported;
    status = allocate_scratch(g_scratch[device]);
    if (status != hipSuccess) return status;
  }
  *out = &g_scratch[device];
  return hipSuccess;
}

}  // namespace ivo

using namespace ivo;

extern "C" {

hipError_t ivonar_init(int device) { return init_device(device); }

hipError_t ivonar_define(const char* name, int value) {
  if (name == nullptr || value <= 0) return hipErrorInvalidValue;
  if (strcmp(name, "HEAD_DIM") == 0) defines().head_dim = value;
  else if (strcmp(name, "TILE") == 0) defines().tile = value;
  else if (strcmp(name, "MAX_CHUNKS") == 0) defines().max_chunks = value;
  else if (strcmp(name, "MAX_TOPK") == 0 && value <= kMaxTopK) defines().max_topk = value;
  else return hipErrorInvalidValue;
  return hipSuccess;
}

const char* ivonar_error_string(hipError_t status) { return hipGetErrorString(status); }

int ivonar_abi_version(void) { return IVONAR_ABI_VERSION; }

void ivonar_gemv_plan(int rows, int n, int* lanes, int* rows_per_lane) { gemv_plan(rows, n, lanes, rows_per_lane); }

int ivonar_gemm_plan(int m, int rows, int n) { return gemm_splits(m, rows, n); }

int ivonar_token_finish_limit(int groups) {
  if (groups < 0 || groups > kTokenFinishCounters) return -1;
  return defines().token_finish_groups.exchange(groups);
}

#define GEMV_PASS_ENTRY(MODE, EPI, PREQUANT)                                                                      \
  gemv_entry(stream, MODE, EPI, PREQUANT, input, aux, q8_in, xsum_in, scale_in, packed, scales, bias, output, rows, \
             n, row_bytes, groups, splits, eps)
#define GEMV_UNUSED \
  (void)lanes;      \
  (void)next;       \
  (void)next_bytes

hipError_t gemv_plain_store(hipStream_t stream, IVONAR_GEMV_ARGS) {
  GEMV_UNUSED;
  return GEMV_PASS_ENTRY(kPlain, kStore, false);
}
hipError_t ivonar_gemv_plain_store_noalloc(hipStream_t stream, IVONAR_GEMV_ARGS) {
  GEMV_UNUSED;
  if (n > kStaticChunks * kChunk) return hipErrorInvalidValue;  // beyond the static scratch
  Scratch* work = nullptr;
  if (n > gemv_fused_limit()) {
    hipError_t status = static_scratch(&work);
    if (status != hipSuccess) return status;
  }
  return gemv_entry(stream, kPlain, kStore, false, input, aux, q8_in, xsum_in, scale_in, packed, scales, bias, output,
                    rows, n, row_bytes, groups, splits, eps, work);
}
hipError_t gemv_plain_residual(hipStream_t stream, IVONAR_GEMV_ARGS) {
  GEMV_UNUSED;
  return GEMV_PASS_ENTRY(kPlain, kResidual, false);
}
hipError_t gemv_norm_store(hipStream_t stream, IVONAR_GEMV_ARGS) {
  GEMV_UNUSED;
  return GEMV_PASS_ENTRY(kNorm, kStore, false);
}
hipError_t gemv_norm_silu_pair(hipStream_t stream, IVONAR_GEMV_ARGS) {
  GEMV_UNUSED;
  return GEMV_PASS_ENTRY(kNorm, kSiluPair, false);
}
hipError_t gemv_attn_residual(hipStream_t stream, IVONAR_GEMV_ARGS) {
  GEMV_UNUSED;
  return GEMV_PASS_ENTRY(kAttn, kResidual, false);
}
hipError_t gemv_prequant_store(hipStream_t stream, IVONAR_GEMV_ARGS) {
  GEMV_UNUSED;
  return GEMV_PASS_ENTRY(kPlain, kStore, true);
}
hipError_t gemv_plain_store_wide(hipStream_t stream, IVONAR_GEMV_ARGS) {
  GEMV_UNUSED;
  return GEMV_PASS_ENTRY(kPlain, kStore, false);
}
hipError_t gemv_plain_residual_wide(hipStream_t stream, IVONAR_GEMV_ARGS) {
  GEMV_UNUSED;
  return GEMV_PASS_ENTRY(kPlain, kResidual, false);
}
hipError_t gemv_norm_store_wide(hipStream_t stream, IVONAR_GEMV_ARGS) {
  GEMV_UNUSED;
  return GEMV_PASS_ENTRY(kNorm, kStore, false);
}
hipError_t gemv_norm_silu_pair_wide(hipStream_t stream, IVONAR_GEMV_ARGS) {
  GEMV_UNUSED;
  return GEMV_PASS_ENTRY(kNorm, kSiluPair, false);
}
hipError_t gemv_attn_residual_wide(hipStream_t stream, IVONAR_GEMV_ARGS) {
  GEMV_UNUSED;
  return GEMV_PASS_ENTRY(kAttn, kResidual, false);
}

hipError_t gemv_group_partials(hipStream_t stream, const int8_t* q8_in, const int32_t* xsum_in,
                               const uint8_t* packed, int rows, int n, int row_bytes, int groups,
                               int32_t* partials) {
  static const uint16_t kNoScales = 0;
  hipError_t status = check_matrix(packed, &kNoScales, rows, n, row_bytes, groups);
  if (status != hipSuccess) return status;
  if (q8_in == nullptr || xsum_in == nullptr || partials == nullptr || !aligned16(q8_in))
    return hipErrorInvalidValue;
  GemvArgs a{};
  a.mode = kPlain;
  a.epi = kPartials;
  a.q8_in = q8_in;
  a.xsum_in = xsum_in;
  a.scale_in = nullptr;
  a.packed = packed;
  a.scales = nullptr;
  a.partials = partials;
  a.rows = rows;
  a.n = n;
  a.row_bytes = row_bytes;
  a.groups = groups;
  a.splits = 1;
  a.head_dim = defines().head_dim;
  return launch_gemv(stream, a);
}

hipError_t quantize_norm(hipStream_t stream, const float* input, const float* aux, int n, float eps, int splits,
                         int8_t* q8_out, int32_t* xsum_out, float* scale_out) {
  return quant_entry(stream, kNorm, input, n, aux, n, eps, splits, 1, q8_out, xsum_out, scale_out);
}
hipError_t quantize_norm_wide(hipStream_t stream, const float* input, const float* aux, int n, float eps,
                              int splits, int8_t* q8_out, int32_t* xsum_out, float* scale_out) {
  return quant_entry(stream, kNorm, input, n, aux, n, eps, splits, 1, q8_out, xsum_out, scale_out);
}

#define QUANT_TILE_PASS(MODE) \
  quant_entry(stream, MODE, input, in_stride, aux, n, eps, splits, defines().tile, q8_out, xsum_out, scale_out)

hipError_t quantize_tile_plain(hipStream_t stream, IVONAR_QUANT_TILE_ARGS) { return QUANT_TILE_PASS(kPlain); }
hipError_t quantize_tile_plain_wide(hipStream_t stream, IVONAR_QUANT_TILE_ARGS) { return QUANT_TILE_PASS(kPlain); }
hipError_t quantize_tile_norm(hipStream_t stream, IVONAR_QUANT_TILE_ARGS) { return QUANT_TILE_PASS(kNorm); }
hipError_t quantize_tile_norm_wide(hipStream_t stream, IVONAR_QUANT_TILE_ARGS) { return QUANT_TILE_PASS(kNorm); }
hipError_t quantize_tile_attn(hipStream_t stream, IVONAR_QUANT_TILE_ARGS) { return QUANT_TILE_PASS(kAttn); }
hipError_t quantize_tile_attn_wide(hipStream_t stream, IVONAR_QUANT_TILE_ARGS) { return QUANT_TILE_PASS(kAttn); }

hipError_t ivonar_quantize_rows(hipStream_t stream, int mode, const float* input, int in_stride, const float* aux,
                                int n, float eps, int splits, int m, int8_t* q8_out, int32_t* xsum_out,
                                float* scale_out) {
  return quant_entry(stream, mode, input, in_stride, aux, n, eps, splits, m, q8_out, xsum_out, scale_out);
}

#define GEMM_PASS_ENTRY(EPI)                                                                                      \
  gemm_entry(stream, EPI, q8_in, xsum_in, scale_in, packed, scales, bias, output, rows, n, row_bytes, groups, \
             out_stride, m)

hipError_t gemm_tile_store(hipStream_t stream, IVONAR_GEMM_ARGS) {
  (void)lanes;
  return GEMM_PASS_ENTRY(kStore);
}
hipError_t gemm_tile_residual(hipStream_t stream, IVONAR_GEMM_ARGS) {
  (void)lanes;
  return GEMM_PASS_ENTRY(kResidual);
}
hipError_t gemm_tile_silu_pair(hipStream_t stream, IVONAR_GEMM_ARGS) {
  (void)lanes;
  return GEMM_PASS_ENTRY(kSiluPair);
}
hipError_t gemm_tile_store_wide(hipStream_t stream, IVONAR_GEMM_ARGS) {
  (void)lanes;
  return GEMM_PASS_ENTRY(kStore);
}
hipError_t gemm_tile_residual_wide(hipStream_t stream, IVONAR_GEMM_ARGS) {
  (void)lanes;
  return GEMM_PASS_ENTRY(kResidual);
}
hipError_t gemm_tile_silu_pair_wide(hipStream_t stream, IVONAR_GEMM_ARGS) {
  (void)lanes;
  return GEMM_PASS_ENTRY(kSiluPair);
}

hipError_t embed_token(hipStream_t stream, const int64_t* token, const uint8_t* packed, const uint16_t* scales,
                       float* output, int n, int row_bytes, int groups) {
  if (token == nullptr || packed == nullptr || scales == nullptr || output == nullptr || n <= 0 ||
      row_bytes < ceil_div(n, 4) || groups < ceil_div(n, kGroup))
    return hipErrorInvalidValue;
  return launch_embed(stream, token, 1, packed, scales, output, n, row_bytes, groups);
}

hipError_t embed_tile(hipStream_t stream, const int64_t* tokens, const uint8_t* packed, const uint16_t* scales,
                      float* output, int n, int row_bytes, int groups, int m) {
  if (tokens == nullptr || packed == nullptr || scales == nullptr || output == nullptr || n <= 0 || m < 0 ||
      row_bytes < ceil_div(n, 4) || groups < ceil_div(n, kGroup))
    return hipErrorInvalidValue;
  return launch_embed(stream, tokens, m, packed, scales, output, n, row_bytes, groups);
}

hipError_t gather_token(hipStream_t stream, const float* tile, float* output, int n, const int64_t* valid) {
  if (tile == nullptr || output == nullptr || valid == nullptr || n <= 0) return hipErrorInvalidValue;
  return launch_gather(stream, tile, output, n, valid);
}

hipError_t ivonar_argmax(hipStream_t stream, const float* values, int n, int64_t* out) {
  if (values == nullptr || out == nullptr || n <= 0) return hipErrorInvalidValue;
  return launch_argmax(stream, values, n, out);
}

hipError_t logit_bounds(hipStream_t stream, const float* logits, const float* temperature, const float* penalty,
                        const float* inverse_penalty, const uint8_t* seen, float* bounds, int vocab) {
  if (logits == nullptr || temperature == nullptr || penalty == nullptr || inverse_penalty == nullptr ||
      seen == nullptr || bounds == nullptr)
    return hipErrorInvalidValue;
  return launch_logit_bounds(stream, logits, temperature, penalty, inverse_penalty, seen, bounds, vocab);
}

hipError_t sample_token(hipStream_t stream, const float* logits, const float* bounds, const float* temperature,
                        const float* penalty, const float* inverse_penalty, uint8_t* seen, const int64_t* top_k,
                        const float* uniform, int64_t* token, int64_t* history, int vocab) {
  if (logits == nullptr || bounds == nullptr || temperature == nullptr || penalty == nullptr ||
      inverse_penalty == nullptr || seen == nullptr || top_k == nullptr || uniform == nullptr || token == nullptr)
    return hipErrorInvalidValue;
  return launch_sample_token(stream, logits, bounds, temperature, penalty, inverse_penalty, seen, top_k, uniform, token,
                             history, vocab);
}

hipError_t ivonar_validate_ternary(hipStream_t stream, const uint8_t* packed, long long packed_bytes,
                                   const uint16_t* scales, long long scale_count, unsigned* flags) {
  if (flags == nullptr || packed_bytes < 0 || scale_count < 0) return hipErrorInvalidValue;
  if ((packed_bytes > 0 && (packed == nullptr || !aligned16(packed))) ||
      (scale_count > 0 && (scales == nullptr || !aligned16(scales))))
    return hipErrorInvalidValue;
  if (packed_bytes == 0 && scale_count == 0) return hipSuccess;
  return launch_validate(stream, packed, packed_bytes, scales, scale_count, flags);
}

int ivonar_stream_read_sink_words(void) { return stream_read_sink_words(); }

hipError_t ivonar_stream_read(hipStream_t stream, const void* data, long long bytes, unsigned* sink) {
  if (data == nullptr || sink == nullptr || bytes < 0 || (bytes & 15) != 0 || !aligned16(data))
    return hipErrorInvalidValue;
  return launch_stream_read(stream, data, bytes, sink);
}

}  // extern "C"
