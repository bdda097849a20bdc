// Skinny token GEMM on int8 MFMA for a few tokens (M <= 32): the decode and
// short-prefill shapes, where a tile of 64+ tokens would idle most of the
// MFMA work and leave most CUs without a block.
//
// A block owns 16 weight rows and S waves; wave s walks the contiguous group
// range [s*GS, min((s+1)*GS, G)), GS = ceil(G/S), so the matrix is streamed by
// (rows/16) * S waves.  Per 128-input group a lane (c = lane % 16 = weight row,
// kb = lane / 16) loads the 8 packed bytes of words 2kb, 2kb+1 of its row and
// expands them to signed int8 codes (one v_perm_b32 table lookup per 4
// codes); these are the B operands of two v_mfma_i32_16x16x64_i8 whose A
// operands are the q8 quads of the same words for 16 tokens, read from LDS.
// The packed weights and scales are prefetched kStage groups ahead into
// registers, double buffered, so each wave keeps 2 * kStage * 512 bytes of
// its stream in flight.
//
// The block copies the tokens' q8 rows to LDS once (row pitch G*128 + 16
// bytes: a missing second chunk of the last group reads zeros, and the 16
// byte skew spreads 16 tokens over distinct banks).
//
// fp32 order (restated by the CPU oracle as orc_gemm_split): each wave folds
// its groups' exact int32 tiles into fp32 with one fmaf per output in
// ascending group order; the S partial sums are then added in wave order
// through LDS, and the token scale and bias applied.
#include "internal.hpp"
#include "ternary_device.hpp"

namespace ivo {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kStage = 8;                     // groups per prefetch stage
constexpr unsigned kSignedLut = 0x000100FFu;  // v_perm table: code 0 -> -1, 1 -> 0, 2 -> +1

__device__ __forceinline__ unsigned signed_codes(unsigned w, int k) {
  return __builtin_amdgcn_perm(0u, kSignedLut, (w >> (2 * k)) & kLow2);
}

struct SkinnyStage {
  uint2 w[kStage];
  uint16_t s[kStage];
};

template <int MT, int S>
struct SkinnyShape {
  static constexpr int kThreadsPerBlock = 64 * S;
  static constexpr int kPartials = S * 16 * 16 * MT;  // floats in the reduction area
};

template <int EPI, int MT, int S>
__global__ __launch_bounds__(64 * S) void skinny_kernel(const int8_t* __restrict__ q8,
                                                        const float* __restrict__ scale_in,
                                                        const uint8_t* __restrict__ packed,
                                                        const uint16_t* __restrict__ scales,
                                                        const float* __restrict__ bias,
                                                        float* __restrict__ output, GemmArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int s = tid >> 6;
  const int col = lane & 15, kb = lane >> 4;
  const int chunks = (a.n + kChunk - 1) / kChunk;
  const int groups = (a.n + kGroup - 1) / kGroup;
  const int pitch = groups * kGroup + 16;
  const int row0 = blockIdx.x * 16;
  const int row = min(row0 + col, a.rows - 1);
  const int per_wave = (groups + S - 1) / S;
  const int g_begin = min(s * per_wave, groups);
  const int g_end = min(g_begin + per_wave, groups);
  const uint8_t* wrow = packed + (size_t)row * a.row_bytes + kb * 8;
  const uint16_t* srow = scales + (size_t)row * a.groups;

  // Weights of group g for this lane; the dead second chunk of the last group loads nothing.
  auto load_stage = [&](SkinnyStage& st, int first) {
#pragma unroll
    for (int j = 0; j < kStage; ++j) {
      const int g = min(first + j, groups - 1);
      const bool live = (2 * g + (kb >> 1)) < chunks;
      st.w[j] = live ? *reinterpret_cast<const uint2*>(wrow + (size_t)g * 32) : make_uint2(0u, 0u);
      st.s[j] = srow[g];
    }
  };

  SkinnyStage bufa, bufb;
  load_stage(bufa, g_begin);

  // Stage the tokens' q8 rows (zero-filling the missing chunk of an odd chunk count).
  const int row_bytes_q8 = chunks * kChunk;
  for (int t = 0; t < a.m; ++t) {
    const int4* src = reinterpret_cast<const int4*>(q8 + (size_t)t * row_bytes_q8);
    int4* dst = reinterpret_cast<int4*>(smem + (size_t)t * pitch);
    for (int e = tid; e < groups * 8; e += 64 * S) dst[e] = e < chunks * 4 ? src[e] : make_int4(0, 0, 0, 0);
  }
  __syncthreads();

  const unsigned char* a_base[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) a_base[mt] = smem + (size_t)min(mt * 16 + col, a.m - 1) * pitch + kb * 32;

  float acc[MT][4];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[mt][i] = 0.0f;

  auto compute_stage = [&](const SkinnyStage& st, int first) {
#pragma unroll
    for (int j = 0; j < kStage; ++j) {
      const int g = first + j;
      const bool live = g < g_end;
      const int gc = min(g, groups - 1);
      v4i b0, b1;
      b0.x = (int)signed_codes(st.w[j].x, 0);
      b0.y = (int)signed_codes(st.w[j].x, 1);
      b0.z = (int)signed_codes(st.w[j].x, 2);
      b0.w = (int)signed_codes(st.w[j].x, 3);
      b1.x = (int)signed_codes(st.w[j].y, 0);
      b1.y = (int)signed_codes(st.w[j].y, 1);
      b1.z = (int)signed_codes(st.w[j].y, 2);
      b1.w = (int)signed_codes(st.w[j].y, 3);
      const float scale = h2f(st.s[j]);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const v4i a0 = *reinterpret_cast<const v4i*>(a_base[mt] + (size_t)gc * kGroup);
        const v4i a1 = *reinterpret_cast<const v4i*>(a_base[mt] + (size_t)gc * kGroup + 16);
        const v4i zero = {0, 0, 0, 0};
        v4i p = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, b0, zero, 0, 0, 0);
        p = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, b1, p, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float partial = live ? (float)p[i] : 0.0f;
          acc[mt][i] = __builtin_fmaf(partial, scale, acc[mt][i]);
        }
      }
    }
  };

  for (int first = g_begin; first < g_end; first += 2 * kStage) {
    load_stage(bufb, first + kStage);
    compute_stage(bufa, first);
    if (first + kStage >= g_end) break;
    load_stage(bufa, first + 2 * kStage);
    compute_stage(bufb, first + kStage);
  }

  // Add the S partial sums in wave order: red[s][mt*16 + 4kb + i][col].
  float* red = reinterpret_cast<float*>(smem + (size_t)a.m * pitch + 15) ;
  red = reinterpret_cast<float*>(((uintptr_t)red) & ~(uintptr_t)15);
  __syncthreads();
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int i = 0; i < 4; ++i) red[((s * MT + mt) * 16 + 4 * kb + i) * 16 + col] = acc[mt][i];
  __syncthreads();
  if (s != 0) return;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float total = acc[mt][i];
      for (int w = 1; w < S; ++w) total = total + red[((w * MT + mt) * 16 + 4 * kb + i) * 16 + col];
      acc[mt][i] = total;
    }

  const int out_row = row0 + col;
  const bool row_live = out_row < a.rows;
  const float b = (bias != nullptr && row_live) ? bias[out_row] : 0.0f;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int t = mt * 16 + 4 * kb + i;
      const bool live = row_live && t < a.m;
      float y = acc[mt][i] * scale_in[min(t, a.m - 1)];
      if (bias != nullptr) y = y + b;
      float* orow = output + (size_t)min(t, a.m - 1) * a.out_stride;
      if constexpr (EPI == kSiluPair) {
        const float partner = __shfl_xor(y, 1);
        if (live && (out_row & 1) == 0 && out_row + 1 < a.rows) orow[out_row >> 1] = ivo_silu(y) * partner;
      } else if constexpr (EPI == kResidual) {
        if (live) orow[out_row] = orow[out_row] + y;
      } else {
        if (live) orow[out_row] = y;
      }
    }
}

size_t skinny_lds(int m, int n, int mt, int splits) {
  const int groups = ceil_div(n, kGroup);
  return (size_t)m * (groups * kGroup + 16) + 16 + (size_t)splits * 16 * 16 * mt * sizeof(float);
}

template <int EPI, int MT, int S>
hipError_t launch_skinny_shape(hipStream_t stream, const GemmArgs& a) {
  const size_t lds = skinny_lds(a.m, a.n, MT, S);
  hipLaunchKernelGGL((skinny_kernel<EPI, MT, S>), dim3(ceil_div(a.rows, 16)), dim3(64 * S), lds, stream, a.q8_in,
                     a.scale_in, a.packed, a.scales, a.bias, a.output, a);
  return hipGetLastError();
}

template <int EPI, int MT>
hipError_t launch_skinny_mt(hipStream_t stream, const GemmArgs& a, int splits) {
  switch (splits) {
    case 1: return launch_skinny_shape<EPI, MT, 1>(stream, a);
    case 2: return launch_skinny_shape<EPI, MT, 2>(stream, a);
    case 4: return launch_skinny_shape<EPI, MT, 4>(stream, a);
    default: return launch_skinny_shape<EPI, MT, 8>(stream, a);
  }
}

template <int EPI>
hipError_t launch_skinny_epi(hipStream_t stream, const GemmArgs& a, int splits) {
  return a.m <= 16 ? launch_skinny_mt<EPI, 1>(stream, a, splits) : launch_skinny_mt<EPI, 2>(stream, a, splits);
}

}  // namespace

int skinny_splits(int m, int rows, int n, size_t max_lds) {
  if (m < 1 || m > 32) return 0;
  const int groups = ceil_div(n, kGroup);
  const int tiles = ceil_div(rows, 16);
  int splits = 1;
  while (splits < 8 && (long long)tiles * splits < 2048 && splits * 2 <= groups) splits *= 2;
  const int mt = m <= 16 ? 1 : 2;
  if (skinny_lds(m, n, mt, splits) > max_lds) return 0;
  return splits;
}

hipError_t launch_skinny(hipStream_t stream, const GemmArgs& a, int splits) {
  switch (a.epi) {
    case kStore: return launch_skinny_epi<kStore>(stream, a, splits);
    case kResidual: return launch_skinny_epi<kResidual>(stream, a, splits);
    case kSiluPair: return launch_skinny_epi<kSiluPair>(stream, a, splits);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace ivo
