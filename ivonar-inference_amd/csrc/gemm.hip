// Token-tile GEMM on CDNA4 int8 MFMA (reference: kernels/ternary.cu:688-784,
// entry points gemm_tile_* with GEMM_ARGS; the reference uses dp4a).
//
// y[t, r] = s_x[t] * sum_g P[t, r, g] * scale[r, g] (+ bias[r]), where
// P[t, r, g] = sum over the 128 inputs of group g of (code - 1) * q is exact.
//
// Each wave owns 16 weight rows and MT 16-token tiles.  Per 128-input group a
// lane (row = lane % 16, k-block = lane / 16) loads 8 packed bytes, i.e.
// words 2kb and 2kb+1 of the group's 32 bytes, and expands each word to 16
// int8 codes in registers ((w >> 2k) & 0x03030303); those are the B operands
// of two v_mfma_i32_16x16x64_i8.  The A operands are the 16-byte q8 quads of
// the same words, which the q8 layout stores in exactly the order the
// expansion produces, so one MFMA pair gives sum(code * q) for 16 tokens x 16
// rows over the group with int32 accumulation.  Subtracting the group's
// activation sum turns codes into ternary values; one fmaf per output folds
// P * scale[r, g] into an fp32 accumulator in ascending group order (the
// order restated by the CPU oracle, orc_gemm_seq).
#include "internal.hpp"
#include "ternary_device.hpp"

namespace ivo {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

__device__ __forceinline__ v4i expand_word(unsigned w) {
  v4i v;
  v.x = (int)(w & kLow2);
  v.y = (int)((w >> 2) & kLow2);
  v.z = (int)((w >> 4) & kLow2);
  v.w = (int)((w >> 6) & kLow2);
  return v;
}

template <int EPI, int MT>
__global__ __launch_bounds__(kThreads) void gemm_kernel(GemmArgs a) {
  const int chunks = (a.n + kChunk - 1) / kChunk;
  const int groups = (a.n + kGroup - 1) / kGroup;
  const int lane = threadIdx.x & 63;
  const int col = lane & 15;   // weight row inside the wave's 16 and token inside an A tile
  const int kb = lane >> 4;    // k-block of the MFMA operands; also the output token quad
  const int row = (blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6)) * 16 + col;
  const int token0 = blockIdx.y * (16 * MT);
  const bool row_live = row < a.rows;
  const uint8_t* wrow = a.packed + (size_t)(row_live ? row : 0) * a.row_bytes;
  const uint16_t* srow = a.scales + (size_t)(row_live ? row : 0) * a.groups;
  const size_t q8_stride = (size_t)chunks * kChunk;

  float acc[MT][4];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[mt][i] = 0.0f;

  for (int g = 0; g < groups; ++g) {
    // Bytes [8kb, 8kb+8) of the group: chunk 2g for kb < 2, chunk 2g+1 otherwise.
    const bool part_live = (2 * g + (kb >> 1)) < chunks;
    uint2 w = make_uint2(0u, 0u);
    if (row_live && part_live) w = *reinterpret_cast<const uint2*>(wrow + (size_t)g * 32 + kb * 8);
    const v4i b0 = expand_word(w.x);
    const v4i b1 = expand_word(w.y);
    const float scale = row_live ? h2f(srow[g]) : 0.0f;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int t_in = token0 + mt * 16 + col;
      v4i a0 = {0, 0, 0, 0}, a1 = {0, 0, 0, 0};
      if (t_in < a.m && part_live) {
        const v4i* q = reinterpret_cast<const v4i*>(a.q8_in + (size_t)t_in * q8_stride + (size_t)g * kGroup +
                                                    (size_t)kb * 32);
        a0 = q[0];
        a1 = q[1];
      }
      v4i d = {0, 0, 0, 0};
      d = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, b0, d, 0, 0, 0);
      d = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, b1, d, 0, 0, 0);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = token0 + mt * 16 + kb * 4 + i;
        int xs = 0;
        if (t < a.m) {
          const int32_t* xrow = a.xsum_in + (size_t)t * chunks;
          xs = xrow[2 * g] + (2 * g + 1 < chunks ? xrow[2 * g + 1] : 0);
        }
        acc[mt][i] = __builtin_fmaf((float)(d[i] - xs), scale, acc[mt][i]);
      }
    }
  }

  const float bias = (a.bias != nullptr && row_live) ? a.bias[row] : 0.0f;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int t = token0 + mt * 16 + kb * 4 + i;
      const bool live = t < a.m && row_live;
      float y = acc[mt][i] * (t < a.m ? a.scale_in[t] : 0.0f);
      if (a.bias != nullptr) y = y + bias;
      float* orow = a.output + (size_t)(t < a.m ? t : 0) * a.out_stride;
      if constexpr (EPI == kSiluPair) {
        const float partner = __shfl_xor(y, 1);
        if (live && (row & 1) == 0 && row + 1 < a.rows) orow[row >> 1] = ivo_silu(y) * partner;
      } else if constexpr (EPI == kResidual) {
        if (live) orow[row] = orow[row] + y;
      } else {
        if (live) orow[row] = y;
      }
    }
  }
}

template <int EPI>
hipError_t launch_epi(hipStream_t stream, const GemmArgs& a) {
  constexpr int MT = 2;
  const dim3 grid(ceil_div(a.rows, 16 * (kThreads / 64)), ceil_div(a.m, 16 * MT));
  hipLaunchKernelGGL((gemm_kernel<EPI, MT>), grid, dim3(kThreads), 0, stream, a);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_gemm(hipStream_t stream, const GemmArgs& a) {
  if (a.rows <= 0 || a.m <= 0) return hipSuccess;
  switch (a.epi) {
    case kStore: return launch_epi<kStore>(stream, a);
    case kResidual: return launch_epi<kResidual>(stream, a);
    case kSiluPair: return launch_epi<kSiluPair>(stream, a);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace ivo
