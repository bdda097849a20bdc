// Per-token int8 activation quantizer (reference semantics:
// kernels/ternary.cu:148-197, quantization.py:35-38).
//
// PLAIN rows that are 16-byte aligned take quantize_plain_kernel: a block of
// T threads (256, or 1024 for rows longer than 16 chunks) quantizes T/16
// chunks of one token row, one q8 word per thread (quantize_plain_slice, which
// the long-row GEMV launches also run in their first blocks).  Every thread
// issues all of its loads in one round - its four inputs and its share of the
// row's amax as float4 - so the kernel costs one memory round trip, a block
// max and the divisions.  Other rows (NORM, ATTN, unaligned) take
// quantize_rows_kernel: one block of 256 threads per slice of 16 chunks that
// first reduces the whole row (sum of squares in the reference tree for NORM,
// then amax) and then quantizes its slice.  Thread d of a slice writes q8
// word d of it and 16 neighbouring lanes reduce one chunk's xsum exactly.
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
  // Rows of up to 1024 inputs (the decoder's model width) load 4 inputs per
  // thread and pass, not 16 mostly clamped ones (one block-uniform branch).
  const float scale = a.n <= 4 * kThreads ? row_scale<MODE, 4>(src, inv_rms, slots) : row_scale<MODE>(src, inv_rms, slots);
  const int word = threadIdx.x;
  const int u = blockIdx.x * kSliceChunks + (word >> 4);
  int value = 0;
  if (u < chunks) value = quantize_word<MODE>(src, u, (word >> 2) & 3, word & 3, inv_rms, scale);
  const int total = chunk_lane_sum(word_sum(value));
  const unsigned partner = (unsigned)__builtin_amdgcn_mov_dpp(value, 0x4E, 0xF, 0xF, false);  // lane ^ 2
  if (u < chunks) {
    int32_t* q8 = reinterpret_cast<int32_t*>(a.q8 + (size_t)t * chunks * kChunk);
    q8[u * 16 + (word & 15)] = a.split ? (int)split_quad_word((unsigned)value, partner, word & 3) : value;
    if ((word & 15) == 0) a.xsum[(size_t)t * chunks + u] = total;
  }
  if (blockIdx.x == 0 && threadIdx.x == 0) a.scale[t] = scale;
}

// NORM rows of up to kSliceChunks chunks (1024 inputs, the decoder's model
// width), one block per token: the row and its NORM weights are read once
// into registers (quantize_row_to_lds: the same sum of squares in the same
// order, the same fp32 operations per input as quantize_word), the q8 bytes
// are exchanged through LDS, and thread w writes q8 word w and the chunk
// sums as quantize_rows_kernel does.  One global round trip instead of three
// (the row for the sum of squares, then row and weights for the absmax, then
// again per q8 word).
__global__ __launch_bounds__(kThreads) void quantize_norm_short_kernel(QuantArgs a) {
  __shared__ float slots[64];
  __shared__ __align__(16) unsigned char lds_q[kSliceChunks * kChunk];
  const int t = blockIdx.y;
  const int chunks = (a.n + kChunk - 1) / kChunk;
  const RowSource src{a.input + (size_t)t * a.in_stride, a.aux, a.n, a.eps, a.splits, a.head_dim};
  const float scale = quantize_row_to_lds<kNorm, kSliceChunks * kChunk / kThreads>(src, chunks, lds_q, slots);
  __syncthreads();
  const int word = threadIdx.x;
  const int u = word >> 4, w = (word >> 2) & 3, k = word & 3;
  const int value = u < chunks ? reinterpret_cast<const int*>(lds_q)[(w * chunks + u) * 4 + k] : 0;
  const int total = chunk_lane_sum(word_sum(value));
  const unsigned partner = (unsigned)__builtin_amdgcn_mov_dpp(value, 0x4E, 0xF, 0xF, false);  // lane ^ 2
  if (u < chunks) {
    int32_t* q8 = reinterpret_cast<int32_t*>(a.q8 + (size_t)t * chunks * kChunk);
    q8[u * 16 + (word & 15)] = a.split ? (int)split_quad_word((unsigned)value, partner, word & 3) : value;
    if ((word & 15) == 0) a.xsum[(size_t)t * chunks + u] = total;
  }
  if (threadIdx.x == 0) a.scale[t] = scale;
}

template <int T>
__global__ __launch_bounds__(T) void quantize_plain_kernel(QuantArgs a) {
  __shared__ float slots[T / 64];
  const int t = blockIdx.y;
  const int chunks = (a.n + kChunk - 1) / kChunk;
  quantize_plain_slice<T>(a.input + (size_t)t * a.in_stride, a.n, blockIdx.x, a.split,
                          a.q8 + (size_t)t * chunks * kChunk, a.xsum + (size_t)t * chunks, a.scale + t, slots);
}

}  // namespace

hipError_t launch_quantize(hipStream_t stream, const QuantArgs& a) {
  if (a.m <= 0) return hipSuccess;
  const int chunks = ceil_div(a.n, kChunk);
  const bool aligned = (a.n & 3) == 0 && (a.in_stride & 3) == 0 && (reinterpret_cast<uintptr_t>(a.input) & 15) == 0;
  if (a.mode == kPlain && aligned && a.n > 0) {
    if (chunks <= kSliceChunks) {
      hipLaunchKernelGGL(quantize_plain_kernel<kThreads>, dim3(1, a.m), dim3(kThreads), 0, stream, a);
    } else {
      hipLaunchKernelGGL(quantize_plain_kernel<1024>, dim3(ceil_div(chunks, 64), a.m), dim3(1024), 0, stream, a);
    }
    return hipGetLastError();
  }
  if (a.mode == kNorm && a.n > 0 && chunks <= kSliceChunks) {
    hipLaunchKernelGGL(quantize_norm_short_kernel, dim3(1, a.m), dim3(kThreads), 0, stream, a);
    return hipGetLastError();
  }
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
