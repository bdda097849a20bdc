// Ternary row decode for the tied embedding (reference: kernels/ternary.cu
// embed_token :411-419, embed_tile :613-622, gather_token :624-630) and the
// greedy argmax used by the decode driver.
#include "internal.hpp"
#include "ternary_device.hpp"

namespace ivo {
namespace {

// out[t, i] = (code[tokens[t], i] - 1) * scale[tokens[t], i / 128]; exact.
__global__ __launch_bounds__(kThreads) void embed_kernel(const int64_t* __restrict__ tokens,
                                                         const uint8_t* __restrict__ packed,
                                                         const uint16_t* __restrict__ scales,
                                                         float* __restrict__ output, int n, int row_bytes,
                                                         int groups) {
  const int t = blockIdx.y;
  const int i = blockIdx.x * kThreads + threadIdx.x;
  if (i >= n) return;
  const size_t row = (size_t)tokens[t];
  const int code = (packed[row * row_bytes + (i >> 2)] >> ((i & 3) * 2)) & 3;
  output[(size_t)t * n + i] = (float)(code - 1) * h2f(scales[row * groups + (i >> 7)]);
}

__global__ __launch_bounds__(kThreads) void gather_kernel(const float* __restrict__ tile, float* __restrict__ output,
                                                          int n, const int64_t* __restrict__ valid) {
  const int i = blockIdx.x * kThreads + threadIdx.x;
  if (i >= n) return;
  const long long last = *valid - 1;
  const size_t t = last > 0 ? (size_t)last : 0;
  output[i] = tile[t * n + i];
}

constexpr int kArgmaxThreads = 1024;

// First index of the maximum over n values (one block).
__global__ __launch_bounds__(kArgmaxThreads) void argmax_kernel(const float* __restrict__ values, int n,
                                                                 int64_t* __restrict__ out) {
  __shared__ float best_value[kArgmaxThreads / 64];
  __shared__ int best_index[kArgmaxThreads / 64];
  // (value, index) pairs are compared by value, then by smaller index, so
  // the result does not depend on the order the elements are visited in.
  // Loads go out in batches (a 16-byte vector per element group when the
  // row allows it), clamped to the row and masked after.
  float value = -__builtin_inff();
  int index = n;
  auto consider = [&](float v, int i) {
    if (v > value || (v == value && i < index)) {
      value = v;
      index = i;
    }
  };
  constexpr int kBatch = 8;
  int scalar_from = 0;
  if ((n & 3) == 0 && (reinterpret_cast<uintptr_t>(values) & 15) == 0) {
    const float4* v4 = reinterpret_cast<const float4*>(values);
    const int n4 = n >> 2;
    for (int base = 0; base < n4; base += kArgmaxThreads * kBatch) {
      float4 b[kBatch];
#pragma unroll
      for (int k = 0; k < kBatch; ++k) b[k] = v4[min(base + k * kArgmaxThreads + (int)threadIdx.x, n4 - 1)];
#pragma unroll
      for (int k = 0; k < kBatch; ++k) {
        const int j = base + k * kArgmaxThreads + threadIdx.x;
        if (j < n4) {
          consider(b[k].x, 4 * j);
          consider(b[k].y, 4 * j + 1);
          consider(b[k].z, 4 * j + 2);
          consider(b[k].w, 4 * j + 3);
        }
      }
    }
    scalar_from = n;
  }
  for (int base = scalar_from; base < n; base += kArgmaxThreads * kBatch) {
    float b[kBatch];
#pragma unroll
    for (int k = 0; k < kBatch; ++k) b[k] = values[min(base + k * kArgmaxThreads + (int)threadIdx.x, n - 1)];
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
      const int i = base + k * kArgmaxThreads + threadIdx.x;
      if (i < n) consider(b[k], i);
    }
  }
  // Wave reduction, complete in lane 0 only (DPP row shifts and permlane
  // swaps; each stage reads a lane that has already folded its share, and
  // the (value, smaller index) order over NaN-free values does not depend on
  // the pairing).
  auto take = [&](float other, int other_index) {
    if (other > value || (other == value && other_index < index)) {
      value = other;
      index = other_index;
    }
  };
  take(row_shl<1>(value), row_shl_int<1>(index));
  take(row_shl<2>(value), row_shl_int<2>(index));
  take(row_shl<4>(value), row_shl_int<4>(index));
  take(row_shl<8>(value), row_shl_int<8>(index));
  take(row_swap16(value), __float_as_int(row_swap16(__int_as_float(index))));
  take(row_swap32(value), __float_as_int(row_swap32(__int_as_float(index))));
  if ((threadIdx.x & 63) == 0) {
    best_value[threadIdx.x >> 6] = value;
    best_index[threadIdx.x >> 6] = index;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float v = best_value[0];
    int k = best_index[0];
    for (int w = 1; w < kArgmaxThreads / 64; ++w) {
      if (best_value[w] > v || (best_value[w] == v && best_index[w] < k)) {
        v = best_value[w];
        k = best_index[w];
      }
    }
    *out = k < n ? k : 0;
  }
}

}  // namespace

hipError_t launch_embed(hipStream_t stream, const int64_t* tokens, int m, const uint8_t* packed,
                        const uint16_t* scales, float* output, int n, int row_bytes, int groups) {
  if (m <= 0 || n <= 0) return hipSuccess;
  hipLaunchKernelGGL(embed_kernel, dim3(ceil_div(n, kThreads), m), dim3(kThreads), 0, stream, tokens, packed, scales,
                     output, n, row_bytes, groups);
  return hipGetLastError();
}

hipError_t launch_gather(hipStream_t stream, const float* tile, float* output, int n, const int64_t* valid) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(gather_kernel, dim3(ceil_div(n, kThreads)), dim3(kThreads), 0, stream, tile, output, n, valid);
  return hipGetLastError();
}

hipError_t launch_argmax(hipStream_t stream, const float* values, int n, int64_t* out) {
  if (n <= 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(argmax_kernel, dim3(1), dim3(kArgmaxThreads), 0, stream, values, n, out);
  return hipGetLastError();
}

}  // namespace ivo
