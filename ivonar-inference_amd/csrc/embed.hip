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

// Greedy argmax: first index of the maximum over n values.  One block of
// 1024 threads reading 128 KB of logits is bound by how many misses one CU
// keeps in flight, so the values are split into tiles of kArgmaxTile
// elements over up to kArgmaxBlocks blocks (grid-stride over tiles).  Every
// block reduces its tiles to one (value, index) pair; with more than one
// block, each stores its pair device-coherently into the stream's scratch,
// waits for the store, and counts itself; the block that makes the count
// complete reduces the pairs and resets the count to zero (so every launch
// starts from zero).  (value, index) pairs are ordered by value, then by the
// smaller index, over NaN-free values, so the result does not depend on how
// the elements are split or in which order pairs are merged.
constexpr int kArgmaxThreads = 256;
constexpr int kArgmaxTile = kArgmaxThreads * 8;  // elements per tile: 8 per thread (two float4)
constexpr int kArgmaxBlocks = 64;

struct Best {
  float value;
  int index;
  __device__ void take(float v, int i) {
    if (v > value || (v == value && i < index)) {
      value = v;
      index = i;
    }
  }
};

// Wave reduction, complete in lane 0 only (DPP row shifts and permlane swaps;
// each stage reads a lane that has already folded its share, and the order
// above does not depend on the pairing).
__device__ __forceinline__ void wave_best(Best& b) {
  b.take(row_shl<1>(b.value), row_shl_int<1>(b.index));
  b.take(row_shl<2>(b.value), row_shl_int<2>(b.index));
  b.take(row_shl<4>(b.value), row_shl_int<4>(b.index));
  b.take(row_shl<8>(b.value), row_shl_int<8>(b.index));
  b.take(row_swap16(b.value), __float_as_int(row_swap16(__int_as_float(b.index))));
  b.take(row_swap32(b.value), __float_as_int(row_swap32(__int_as_float(b.index))));
}

__global__ __launch_bounds__(kArgmaxThreads) void argmax_kernel(const float* __restrict__ values, int n,
                                                                 int64_t* __restrict__ out, float* part_value,
                                                                 int* part_index, unsigned* count) {
  __shared__ float best_value[kArgmaxThreads / 64];
  __shared__ int best_index[kArgmaxThreads / 64];
  __shared__ int last_block;
  Best b{-__builtin_inff(), n};
  const int tiles = (n + kArgmaxTile - 1) / kArgmaxTile;
  const int tid = threadIdx.x;
  // Loads go out two float4 (or eight scalars) per thread and tile, clamped
  // to the row and masked after.
  const bool vec = (n & 3) == 0 && (reinterpret_cast<uintptr_t>(values) & 15) == 0;
  for (int tile = blockIdx.x; tile < tiles; tile += gridDim.x) {
    if (vec) {
      const float4* v4 = reinterpret_cast<const float4*>(values);
      const int n4 = n >> 2;
      const int j0 = tile * (kArgmaxTile / 4) + tid, j1 = j0 + kArgmaxThreads;
      const float4 a = v4[min(j0, n4 - 1)], c = v4[min(j1, n4 - 1)];
      if (j0 < n4) {
        b.take(a.x, 4 * j0);
        b.take(a.y, 4 * j0 + 1);
        b.take(a.z, 4 * j0 + 2);
        b.take(a.w, 4 * j0 + 3);
      }
      if (j1 < n4) {
        b.take(c.x, 4 * j1);
        b.take(c.y, 4 * j1 + 1);
        b.take(c.z, 4 * j1 + 2);
        b.take(c.w, 4 * j1 + 3);
      }
    } else {
      float v[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) v[k] = values[min(tile * kArgmaxTile + k * kArgmaxThreads + tid, n - 1)];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const int i = tile * kArgmaxTile + k * kArgmaxThreads + tid;
        if (i < n) b.take(v[k], i);
      }
    }
  }
  wave_best(b);
  if ((tid & 63) == 0) {
    best_value[tid >> 6] = b.value;
    best_index[tid >> 6] = b.index;
  }
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < kArgmaxThreads / 64; ++w) b.take(best_value[w], best_index[w]);
    int last = 1;
    if (gridDim.x > 1) {
      // The hand-over of store_device (ternary_device.hpp), one thread per block.
      store_device(part_value + blockIdx.x, b.value);
      store_device(part_index + blockIdx.x, b.index);
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the pair is performed device-wide before the count
      last = __hip_atomic_fetch_add(count, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == gridDim.x - 1;
    }
    last_block = last;
    if (gridDim.x == 1) *out = b.index < n ? b.index : 0;
  }
  __syncthreads();
  if (gridDim.x == 1 || !last_block || tid >= 64) return;
  // The last block's first wave: lane l reads the pairs of blocks l and l + 64 (issued after the
  // count returned, device-coherent).
  Best f{-__builtin_inff(), n};
  for (int blk = tid; blk < (int)gridDim.x; blk += 64)
    f.take(load_device(part_value + blk), load_device(part_index + blk));
  wave_best(f);
  if (tid == 0) {
    *out = f.index < n ? f.index : 0;
    __hip_atomic_store(count, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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
  const int tiles = ceil_div(n, kArgmaxTile);
  int blocks = tiles < kArgmaxBlocks ? tiles : kArgmaxBlocks;
  float* part_value = nullptr;
  int* part_index = nullptr;
  unsigned* count = nullptr;
  if (blocks > 1) {
    Scratch* scratch = nullptr;
    const hipError_t status = scratch_for_stream(stream, &scratch);
    if (status != hipSuccess) return status;
    if (scratch->token_partials == nullptr || scratch->sync == nullptr) {
      blocks = 1;  // no scratch for the pairs: one block scans every tile
    } else {
      part_value = scratch->token_partials;
      part_index = reinterpret_cast<int*>(scratch->token_partials + kArgmaxBlocks);
      count = scratch->sync + kArgmaxCountWord;
    }
  }
  hipLaunchKernelGGL(argmax_kernel, dim3(blocks), dim3(kArgmaxThreads), 0, stream, values, n, out, part_value,
                     part_index, count);
  return hipGetLastError();
}

}  // namespace ivo
