// Device check of a packed ternary operand (reference: loader.py:94-112,
// which runs the same tests on the CPU before a checkpoint is built):
//   bit 0  a packed byte holds the reserved code 3 in some field
//          (b & (b >> 1) & 0x55 != 0);
//   bit 1  a group scale is not finite (fp16 exponent all ones);
//   bit 2  a group scale is not positive (sign bit set, or +0).
// One pass over both buffers with 16-byte loads, grid-stride, 1024 blocks of
// 256 threads; each wave folds its findings with ballots and one lane ORs
// them into flags[0] only when something was found, so a clean operand
// issues no atomics.  The caller zeroes flags before the launch.
#include "internal.hpp"
#include "ternary_device.hpp"

namespace ivo {
namespace {

constexpr int kValidateBlocks = 1024;
constexpr int kValidateUnroll = 4;

__device__ __forceinline__ unsigned reserved_code(unsigned w) { return w & (w >> 1) & 0x55555555u; }

// Flags of one fp16 scale, and of two packed in a word.
__device__ __forceinline__ unsigned half_flags(unsigned bits) {
  unsigned flags = 0;
  if ((bits & 0x7c00u) == 0x7c00u) flags |= 2u;
  if ((bits & 0x8000u) != 0u || bits == 0u) flags |= 4u;
  return flags;
}

__device__ __forceinline__ unsigned scale_flags(unsigned w) { return half_flags(w & 0xffffu) | half_flags(w >> 16); }

__global__ __launch_bounds__(kThreads) void validate_kernel(const uint4* __restrict__ packed, long long packed_words,
                                                            const uint8_t* __restrict__ packed_tail, int tail_bytes,
                                                            const uint4* __restrict__ scales, long long scale_words,
                                                            const uint16_t* __restrict__ scale_tail, int tail_scales,
                                                            unsigned* __restrict__ flags) {
  unsigned found = 0;
  const long long stride = (long long)gridDim.x * kThreads;
  const long long first = (long long)blockIdx.x * kThreads + threadIdx.x;
  for (long long base = first; base < packed_words; base += stride * kValidateUnroll) {
    uint4 v[kValidateUnroll];
#pragma unroll
    for (int u = 0; u < kValidateUnroll; ++u) {
      const long long i = base + (long long)u * stride;
      v[u] = packed[i < packed_words ? i : packed_words - 1];
    }
#pragma unroll
    for (int u = 0; u < kValidateUnroll; ++u)
      found |= reserved_code(v[u].x) | reserved_code(v[u].y) | reserved_code(v[u].z) | reserved_code(v[u].w);
  }
  found = found != 0u ? 1u : 0u;
  for (long long i = first; i < scale_words; i += stride) {
    const uint4 v = scales[i];
    found |= scale_flags(v.x) | scale_flags(v.y) | scale_flags(v.z) | scale_flags(v.w);
  }
  if (first < tail_bytes) found |= reserved_code(packed_tail[first]) != 0u ? 1u : 0u;
  if (first < tail_scales) found |= half_flags(scale_tail[first]);
  // Fold over the wave: one lane reports what the wave found.
  unsigned wave = 0;
#pragma unroll
  for (int bit = 0; bit < 3; ++bit)
    if (__ballot((found >> bit) & 1u) != 0ull) wave |= 1u << bit;
  if ((threadIdx.x & 63) == 0 && wave != 0u) atomicOr(flags, wave);
}

}  // namespace

hipError_t launch_validate(hipStream_t stream, const uint8_t* packed, long long packed_bytes, const uint16_t* scales,
                           long long scale_count, unsigned* flags) {
  const long long packed_words = packed_bytes / 16;
  const long long scale_words = scale_count / 8;
  const int tail_bytes = (int)(packed_bytes - packed_words * 16);
  const int tail_scales = (int)(scale_count - scale_words * 8);
  hipLaunchKernelGGL(validate_kernel, dim3(kValidateBlocks), dim3(kThreads), 0, stream,
                     reinterpret_cast<const uint4*>(packed), packed_words, packed + packed_words * 16, tail_bytes,
                     reinterpret_cast<const uint4*>(scales), scale_words, scales + scale_words * 8, tail_scales,
                     flags);
  return hipGetLastError();
}

}  // namespace ivo
