// Streaming-read reference kernel (no counterpart in the reference): reads a
// buffer once with non-temporal 16-byte loads, four per thread in flight,
// grid-stride over 1024 blocks, and folds the words into an XOR that is stored
// only when it equals a fixed constant (so the loads are kept and nothing is
// written in practice).  Its bandwidth over the same rotating buffers the GEMV
// streams is the per-launch read ceiling the GEMV's roofline fraction is
// compared with.  (Measured on MI355X: non-temporal loads read 58.7 MB per
// launch in 10.1 us and 1 GiB in 161 us, plain loads in 10.7 and 180 us;
// other depths, block counts and per-block slices were no faster.)
#include "internal.hpp"
#include "ternary_device.hpp"

namespace ivo {
namespace {

constexpr int kUnroll = 4;
constexpr int kStreamBlocks = 1024;

__global__ __launch_bounds__(kThreads) void stream_read_kernel(const uint4* __restrict__ data, long long words,
                                                               unsigned* __restrict__ sink) {
  unsigned fold = 0;
  const long long tile = (long long)kThreads * kUnroll;
  for (long long base = (long long)blockIdx.x * tile; base < words; base += (long long)gridDim.x * tile) {
    uint4 v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      long long i = base + (long long)u * kThreads + threadIdx.x;
      typedef unsigned v4u __attribute__((ext_vector_type(4)));
      const v4u w = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(data) + (i < words ? i : words - 1));
      v[u] = make_uint4(w[0], w[1], w[2], w[3]);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) fold ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  if (fold == 0x9e3779b9u) sink[blockIdx.x * kThreads + threadIdx.x] = fold;
}

}  // namespace

int stream_read_sink_words() { return kStreamBlocks * kThreads; }

hipError_t launch_stream_read(hipStream_t stream, const void* data, long long bytes, unsigned* sink) {
  const long long words = bytes / 16;
  if (words <= 0) return hipSuccess;
  hipLaunchKernelGGL(stream_read_kernel, dim3(kStreamBlocks), dim3(kThreads), 0, stream,
                     static_cast<const uint4*>(data), words, sink);
  return hipGetLastError();
}

}  // namespace ivo
