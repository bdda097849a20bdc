// Per-token int8 activation quantizer (reference semantics:
// kernels/ternary.cu:148-197, quantization.py:35-38).
//
// One block of 256 threads quantizes a slice of 16 chunks (1024 inputs) of
// one token row; grid = (ceil(C/16), m).  Every block first reduces the whole
// row (sum of squares in the reference tree for NORM, then amax), which is
// cheap next to the division per input, so long rows spread over many CUs
// instead of serialising on one.  Thread d of a slice writes q8 word d of it
// and 16 neighbouring lanes reduce one chunk's xsum exactly.
#include "internal.hpp"
#include "ternary_device.hpp"

namespace ivo {
namespace {

constexpr int kSliceChunks = kThreads / 16;  // 16 chunks, one q8 word per thread

template <int MODE>
__global__ __launch_bounds__(kThreads) void quantize_rows_kernel(QuantArgs a) {
  __shared__ float slots[64];
  const int t = blockIdx.y;
  const int chunks = (a.n + kChunk - 1) / kChunk;
  const RowSource src{a.input + (size_t)t * a.in_stride, a.aux, a.n, a.eps, a.splits, a.head_dim};
  float inv_rms;
  const float scale = row_scale<MODE>(src, inv_rms, slots);
  const int word = threadIdx.x;
  const int u = blockIdx.x * kSliceChunks + (word >> 4);
  int value = 0;
  if (u < chunks) value = quantize_word<MODE>(src, u, (word >> 2) & 3, word & 3, inv_rms, scale);
  const int total = chunk_lane_sum(word_sum(value));
  if (u < chunks) {
    int32_t* q8 = reinterpret_cast<int32_t*>(a.q8 + (size_t)t * chunks * kChunk);
    q8[u * 16 + (word & 15)] = value;
    if ((word & 15) == 0) a.xsum[(size_t)t * chunks + u] = total;
  }
  if (blockIdx.x == 0 && threadIdx.x == 0) a.scale[t] = scale;
}

}  // namespace

hipError_t launch_quantize(hipStream_t stream, const QuantArgs& a) {
  if (a.m <= 0) return hipSuccess;
  const int chunks = ceil_div(a.n, kChunk);
  const dim3 grid(ceil_div(chunks, kSliceChunks), a.m);
  switch (a.mode) {
    case kPlain: hipLaunchKernelGGL(quantize_rows_kernel<kPlain>, grid, dim3(kThreads), 0, stream, a); break;
    case kNorm: hipLaunchKernelGGL(quantize_rows_kernel<kNorm>, grid, dim3(kThreads), 0, stream, a); break;
    case kAttn: hipLaunchKernelGGL(quantize_rows_kernel<kAttn>, grid, dim3(kThreads), 0, stream, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace ivo
