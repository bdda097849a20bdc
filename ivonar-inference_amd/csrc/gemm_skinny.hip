// Skinny token GEMM on int8 MFMA for a few tokens (M <= 32): the decode and
// short-prefill shapes, where a tile of 64+ tokens would idle most of the
// MFMA work and leave most CUs without a block.
//
// A block owns 16 weight rows and S waves; wave s walks the contiguous group
// range [s*GS, min((s+1)*GS, G)), GS = ceil(G/S), so the matrix is streamed by
// (rows/16) * S waves.  Per 128-input group a lane (c = lane % 16, kb =
// lane / 16) loads the 8 packed bytes of words 2kb, 2kb+1 of weight row c and
// expands them to signed int8 codes (one v_perm_b32 table lookup per 4
// codes): the B operands of two v_mfma_i32_16x16x64_i8.  The A operands are
// the q8 bytes of the same words for token c of each 16-token tile, read
// straight from global memory (32 contiguous bytes per lane and group), so
// no stage, copy or barrier precedes the first MFMA.  All loads are
// unconditional, with addresses clamped into the operands, and go out
// kStage groups ahead, double buffered; the second chunk of the last group
// of an odd chunk count is masked to zero on the A side (its weight bytes
// may then be anything).
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

constexpr unsigned kSignedLut = 0x000100FFu;  // v_perm table: code 0 -> -1, 1 -> 0, 2 -> +1
constexpr int kMaxSplits = 16;  // 1024-thread blocks; two token tiles stop at 8 (register budget)

__device__ __forceinline__ unsigned signed_codes(unsigned w, int k) {
  return __builtin_amdgcn_perm(0u, kSignedLut, (w >> (2 * k)) & kLow2);
}

template <int MT>
struct SkinnyStage {
  static constexpr int kGroups = MT == 1 ? 4 : 2;  // groups per stage (register budget)
  uint2 w[kGroups];
  uint16_t s[kGroups];
  v4i a[kGroups][MT][2];
};

template <int EPI, int MT, int S>
__global__ __launch_bounds__(64 * S) void skinny_kernel(const int8_t* __restrict__ q8,
                                                        const float* __restrict__ scale_in,
                                                        const uint8_t* __restrict__ packed,
                                                        const uint16_t* __restrict__ scales,
                                                        const float* __restrict__ bias,
                                                        float* __restrict__ output, GemmArgs a) {
  using Stage = SkinnyStage<MT>;
  constexpr int kStage = Stage::kGroups;
  extern __shared__ __align__(16) unsigned char smem[];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int s = tid >> 6;
  const int col = lane & 15, kb = lane >> 4;
  const int chunks = (a.n + kChunk - 1) / kChunk;
  const int groups = (a.n + kGroup - 1) / kGroup;
  // The last group lacks its second chunk (lanes kb >= 2) when the chunk count is odd.
  const int short_group = (chunks & 1) ? groups - 1 : groups;
  const int row0 = blockIdx.x * 16;
  const int row = min(row0 + col, a.rows - 1);
  const int per_wave = (groups + S - 1) / S;
  const int g_begin = min(s * per_wave, groups);
  const int g_end = min(g_begin + per_wave, groups);
  const uint8_t* wrow = packed + (size_t)row * a.row_bytes;
  const uint16_t* srow = scales + (size_t)row * a.groups;
  const size_t q8_stride = (size_t)chunks * kChunk;
  const int8_t* arow[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) arow[mt] = q8 + (size_t)min(mt * 16 + col, a.m - 1) * q8_stride;

  auto load_stage = [&](Stage& st, int first) {
#pragma unroll
    for (int j = 0; j < kStage; ++j) {
      const int g = min(first + j, groups - 1);
      const bool dead = g == short_group && kb >= 2;  // read the group's first chunk instead
      st.w[j] = *reinterpret_cast<const uint2*>(wrow + (size_t)g * 32 + (dead ? 0 : kb * 8));
      st.s[j] = srow[g];
      const size_t offset = (size_t)g * kGroup + (dead ? 0 : kb * 32);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        st.a[j][mt][0] = *reinterpret_cast<const v4i*>(arow[mt] + offset);
        st.a[j][mt][1] = *reinterpret_cast<const v4i*>(arow[mt] + offset + 16);
      }
    }
  };

  float acc[MT][4];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[mt][i] = 0.0f;

  auto compute_stage = [&](const Stage& st, int first) {
#pragma unroll
    for (int j = 0; j < kStage; ++j) {
      const int g = first + j;
      if (g >= g_end) break;  // wave-uniform
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
      const int keep = (g == short_group && kb >= 2) ? 0 : -1;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        v4i a0 = st.a[j][mt][0], a1 = st.a[j][mt][1];
        if (g == short_group) {  // wave-uniform
          a0 &= keep;
          a1 &= keep;
        }
        const v4i zero = {0, 0, 0, 0};
        v4i p = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, b0, zero, 0, 0, 0);
        p = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, b1, p, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[mt][i] = __builtin_fmaf((float)p[i], scale, acc[mt][i]);
      }
    }
  };

  Stage bufa, bufb;
  load_stage(bufa, g_begin);
  for (int first = g_begin; first < g_end; first += 2 * kStage) {
    load_stage(bufb, first + kStage);
    compute_stage(bufa, first);
    if (first + kStage >= g_end) break;
    load_stage(bufa, first + 2 * kStage);
    compute_stage(bufb, first + kStage);
  }

  // Add the S partial sums in wave order: red[s][mt*16 + 4kb + i][col].
  float* red = reinterpret_cast<float*>(smem);
  if constexpr (S > 1) {
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

size_t skinny_lds(int mt, int splits) { return splits > 1 ? (size_t)splits * 16 * 16 * mt * sizeof(float) : 0; }

template <int EPI, int MT, int S>
hipError_t launch_skinny_shape(hipStream_t stream, const GemmArgs& a) {
  const size_t lds = skinny_lds(MT, S);
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
    case 8: return launch_skinny_shape<EPI, MT, 8>(stream, a);
    default:
      if constexpr (MT == 1) return launch_skinny_shape<EPI, MT, kMaxSplits>(stream, a);
      return hipErrorInvalidValue;
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
  const int mt = m <= 16 ? 1 : 2;
  const int max_splits = mt == 1 ? kMaxSplits : 8;
  int splits = 1;
  while (splits < max_splits && (long long)tiles * splits < 2048 && splits * 2 <= groups) splits *= 2;
  if (skinny_lds(mt, splits) > max_lds) return 0;
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
