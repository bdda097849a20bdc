// Token GEMM on CDNA4 int8 MFMA (reference: kernels/ternary.cu:688-784,
// entry points gemm_tile_* with GEMM_ARGS; the reference uses dp4a).
//
// y[t, r] = s_x[t] * sum_g P[t, r, g] * scale[r, g] (+ bias[r]), where
// P[t, r, g] = sum over the 128 inputs of group g of (code - 1) * q is exact.
//
// Block tile: (64*WM) tokens x (64*WN) weight rows, WM*WN waves, each wave a
// 64 x 64 output tile = 4 x 4 MFMA tiles of v_mfma_i32_16x16x64_i8.  The K
// loop walks the 128-input groups.  For each group the block stages, double
// buffered in LDS:
//   * the q8 bytes of its tokens (128 per token, the q8 layout's two chunks);
//   * its weight rows' 32 packed bytes, expanded once per block to signed
//     int8 (code - 1) with one v_perm_b32 table lookup per 4 codes, so the
//     MFMA produces P directly (no activation-sum correction);
//   * the fp16 group scales of its rows.
// LDS rows are padded from 128 to 144 bytes, which spreads the 16 lanes of
// each 16-byte operand read over distinct banks.  The global loads of group
// g+1 are issued before the MFMAs of group g and written to the other buffer
// after them, with one barrier per group.
//
// Operand pairing: MFMA half h of a group takes, in lane (c = lane % 16,
// kb = lane / 16), the 16 bytes of word 2*kb + h of the group (inputs
// 16*(2kb+h) .. +15).  The q8 layout stores a word's quad in exactly the
// order the expansion (w >> 2k) & 0x03030303 produces, so both operands see
// the same input in the same byte slot.  Each group's int32 tile is folded
// into fp32 with one fmaf per output in ascending group order (the order the
// CPU oracle restates as orc_gemm_seq).
#include "internal.hpp"
#include "ternary_device.hpp"

namespace ivo {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kRowPitch = 144;        // bytes per staged LDS row (128 + 16 padding)
constexpr unsigned kSignedLut = 0x000100FFu;  // v_perm table: code 0 -> -1, 1 -> 0, 2 -> +1

__device__ __forceinline__ unsigned signed_codes(unsigned w, int k) {
  return __builtin_amdgcn_perm(0u, kSignedLut, (w >> (2 * k)) & kLow2);
}

template <int WM, int WN>
struct Tile {
  static constexpr int kWaves = WM * WN;
  static constexpr int kThreadsPerBlock = 64 * kWaves;
  static constexpr int kTokens = 64 * WM;
  static constexpr int kRowsPerBlock = 64 * WN;
  static constexpr int kStageBytes = (kTokens + kRowsPerBlock) * kRowPitch + kRowsPerBlock * 4;
};

template <int EPI, int WM, int WN>
__global__ __launch_bounds__(64 * WM * WN) void gemm_kernel(const int8_t* __restrict__ q8,
                                                            const float* __restrict__ scale_in,
                                                            const uint8_t* __restrict__ packed,
                                                            const uint16_t* __restrict__ scales,
                                                            const float* __restrict__ bias,
                                                            float* __restrict__ output, GemmArgs a) {
  using T = Tile<WM, WN>;
  extern __shared__ __align__(16) unsigned char smem[];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int col = lane & 15, kb = lane >> 4;
  const int chunks = (a.n + kChunk - 1) / kChunk;
  const int groups = (a.n + kGroup - 1) / kGroup;
  const size_t q8_stride = (size_t)chunks * kChunk;
  const int token0 = blockIdx.y * T::kTokens;
  const int row0 = blockIdx.x * T::kRowsPerBlock;

  // Staging: A in 64-byte pieces (two per token), B in 16-byte packed pieces
  // (two per weight row, each expanding to 64 bytes), one scale per row.
  // Two register sets hold the next two groups while the MFMAs consume the
  // third from LDS, so a group's loads have two group-steps to arrive.
  constexpr int kThreadsN = T::kThreadsPerBlock;
  constexpr int kPiecesA = (2 * T::kTokens + kThreadsN - 1) / kThreadsN;
  constexpr int kPiecesB = (2 * T::kRowsPerBlock + kThreadsN - 1) / kThreadsN;
  struct Regs {
    uint4 a[kPiecesA][4];
    uint4 b[kPiecesB];
    uint16_t s;
    int g;
  };
  const bool s_thread = tid < T::kRowsPerBlock;
  const uint16_t* s_src = scales + (size_t)min(row0 + tid % T::kRowsPerBlock, a.rows - 1) * a.groups;

  // Loads are unconditional, with the group clamped into the matrix (a
  // predicated load would make the compiler wait for every outstanding load
  // at its first use).  A missing second chunk reads the group's first chunk;
  // its activations are replaced by zeros when staged, which also cancels
  // whatever its weight bytes hold.
  auto fetch = [&](Regs& r, int g_raw) {
    const int g = min(g_raw, groups - 1);
    r.g = g;
    const bool second_live = 2 * g + 1 < chunks;
#pragma unroll
    for (int k = 0; k < kPiecesA; ++k) {
      const int piece = tid + k * kThreadsN;
      const int token = min(token0 + piece % T::kTokens, a.m - 1), half = (piece / T::kTokens) & 1;
      const bool live = half == 0 || second_live;
      const int8_t* src = q8 + (size_t)token * q8_stride + (size_t)g * kGroup + (live ? half * 64 : 0);
#pragma unroll
      for (int i = 0; i < 4; ++i) r.a[k][i] = *reinterpret_cast<const uint4*>(src + i * 16);
    }
#pragma unroll
    for (int k = 0; k < kPiecesB; ++k) {
      const int piece = tid + k * kThreadsN;
      const int row = min(row0 + piece % T::kRowsPerBlock, a.rows - 1), half = (piece / T::kRowsPerBlock) & 1;
      const bool live = half == 0 || second_live;
      r.b[k] = *reinterpret_cast<const uint4*>(packed + (size_t)row * a.row_bytes + (size_t)g * 32 + (live ? half * 16 : 0));
    }
    r.s = s_src[g];  // clamped row: valid for every thread
  };
  auto stage = [&](const Regs& r, int buffer) {
    unsigned char* base = smem + (size_t)buffer * T::kStageBytes;
    const bool second_live = 2 * r.g + 1 < chunks;  // wave-uniform
#pragma unroll
    for (int k = 0; k < kPiecesA; ++k) {
      const int piece = tid + k * kThreadsN;
      if (piece < 2 * T::kTokens) {
        const int half = piece / T::kTokens;
        unsigned char* dst = base + (piece % T::kTokens) * kRowPitch + half * 64;
        if (second_live) {
#pragma unroll
          for (int i = 0; i < 4; ++i) *reinterpret_cast<uint4*>(dst + i * 16) = r.a[k][i];
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            *reinterpret_cast<uint4*>(dst + i * 16) = half == 0 ? r.a[k][i] : make_uint4(0u, 0u, 0u, 0u);
        }
      }
    }
#pragma unroll
    for (int k = 0; k < kPiecesB; ++k) {
      const int piece = tid + k * kThreadsN;
      if (piece < 2 * T::kRowsPerBlock) {
        unsigned char* dst = base + (T::kTokens + piece % T::kRowsPerBlock) * kRowPitch + (piece / T::kRowsPerBlock) * 64;
        const unsigned words[4] = {r.b[k].x, r.b[k].y, r.b[k].z, r.b[k].w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          uint4 e;
          e.x = signed_codes(words[j], 0);
          e.y = signed_codes(words[j], 1);
          e.z = signed_codes(words[j], 2);
          e.w = signed_codes(words[j], 3);
          *reinterpret_cast<uint4*>(dst + j * 16) = e;
        }
      }
    }
    if (s_thread) reinterpret_cast<float*>(base + (T::kTokens + T::kRowsPerBlock) * kRowPitch)[tid] = h2f(r.s);
  };

  float acc[4][4][4];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[mt][nt][i] = 0.0f;

  // One group from LDS.  The weight fragments of both MFMA halves stay in
  // registers; per 16-token row of tiles the two halves accumulate the exact
  // int32 partials, which are folded into fp32 with one fmaf per output and
  // the row's group scale while the next row of tiles runs on the MFMA unit.
  auto compute = [&](int buffer) {
    const unsigned char* base = smem + (size_t)buffer * T::kStageBytes;
    const unsigned char* a_lds = base + (wm * 64 + col) * kRowPitch;
    const unsigned char* b_lds = base + (T::kTokens + wn * 64 + col) * kRowPitch;
    const float* s_lds = reinterpret_cast<const float*>(base + (T::kTokens + T::kRowsPerBlock) * kRowPitch);
    v4i bf[2][4];
    float sc[4];
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      bf[0][nt] = *reinterpret_cast<const v4i*>(b_lds + nt * 16 * kRowPitch + (2 * kb) * 16);
      bf[1][nt] = *reinterpret_cast<const v4i*>(b_lds + nt * 16 * kRowPitch + (2 * kb + 1) * 16);
      sc[nt] = s_lds[wn * 64 + nt * 16 + col];
    }
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      const v4i a0 = *reinterpret_cast<const v4i*>(a_lds + mt * 16 * kRowPitch + (2 * kb) * 16);
      const v4i a1 = *reinterpret_cast<const v4i*>(a_lds + mt * 16 * kRowPitch + (2 * kb + 1) * 16);
      v4i p[4];
      const v4i zero = {0, 0, 0, 0};
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) p[nt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, bf[0][nt], zero, 0, 0, 0);
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) p[nt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, bf[1][nt], p[nt], 0, 0, 0);
#pragma unroll
      for (int nt = 0; nt < 4; ++nt)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[mt][nt][i] = __builtin_fmaf((float)p[nt][i], sc[nt], acc[mt][nt][i]);
    }
  };

  // LDS buffer g & 1 holds group g; register sets r0 / r1 alternate.
  Regs r0, r1;
  fetch(r0, 0);
  fetch(r1, 1);
  stage(r0, 0);
  __syncthreads();
  fetch(r0, 2);
  for (int g = 0; g < groups; g += 2) {
    compute(0);
    if (g + 1 < groups) stage(r1, 1);
    __syncthreads();
    fetch(r1, g + 3);
    if (g + 1 >= groups) break;
    compute(1);
    if (g + 2 < groups) stage(r0, 0);
    __syncthreads();
    fetch(r0, g + 4);
  }

  // Epilogue: lane holds rows row0 + wn*64 + nt*16 + col, tokens token0 + wm*64 + mt*16 + 4*kb + i.
  const bool full = token0 + T::kTokens <= a.m && row0 + T::kRowsPerBlock <= a.rows;
  float sx[4][4];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int i = 0; i < 4; ++i) sx[mt][i] = scale_in[min(token0 + wm * 64 + mt * 16 + 4 * kb + i, a.m - 1)];
#pragma unroll
  for (int nt = 0; nt < 4; ++nt) {
    const int row = row0 + wn * 64 + nt * 16 + col;
    const bool row_live = row < a.rows;
    const float b = (bias != nullptr && row_live) ? bias[row] : 0.0f;
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = token0 + wm * 64 + mt * 16 + 4 * kb + i;
        const bool live = full || (row_live && t < a.m);
        float y = acc[mt][nt][i] * sx[mt][i];
        if (bias != nullptr) y = y + b;
        float* orow = output + (size_t)min(t, a.m - 1) * a.out_stride;
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
}

template <int EPI, int WM, int WN>
hipError_t launch_shape(hipStream_t stream, const GemmArgs& a) {
  using T = Tile<WM, WN>;
  const dim3 grid(ceil_div(a.rows, T::kRowsPerBlock), ceil_div(a.m, T::kTokens));
  const size_t lds = 2 * (size_t)T::kStageBytes;
  hipLaunchKernelGGL((gemm_kernel<EPI, WM, WN>), grid, dim3(T::kThreadsPerBlock), lds, stream, a.q8_in, a.scale_in,
                     a.packed, a.scales, a.bias, a.output, a);
  return hipGetLastError();
}

}  // namespace

int max_lds_per_block() {
  static int cached[64] = {0};
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= 64) return 64 * 1024;
  if (cached[device] == 0) {
    int bytes = 0;
    if (hipDeviceGetAttribute(&bytes, hipDeviceAttributeMaxSharedMemoryPerBlock, device) != hipSuccess || bytes <= 0)
      bytes = 64 * 1024;
    cached[device] = bytes;
  }
  return cached[device];
}

namespace {

template <int WM, int WN>
bool fits() {
  return 2 * Tile<WM, WN>::kStageBytes <= max_lds_per_block();
}

// Block shape: the largest tile that still gives about one block per CU and
// whose double-buffered stage fits the device's LDS per block.
template <int EPI>
hipError_t launch_epi(hipStream_t stream, const GemmArgs& a) {
  const long long tiles_2x2 = (long long)ceil_div(a.rows, 128) * ceil_div(a.m, 128);
  if (a.m > 64 && tiles_2x2 >= 200 && fits<2, 2>()) return launch_shape<EPI, 2, 2>(stream, a);
  if (a.m > 64) return launch_shape<EPI, 2, 1>(stream, a);
  return launch_shape<EPI, 1, 1>(stream, a);
}

}  // namespace

int gemm_splits(int m, int rows, int n) {
  const int splits = skinny_splits(m, rows, n, (size_t)max_lds_per_block());
  return splits > 0 ? splits : 1;
}

hipError_t launch_gemm(hipStream_t stream, const GemmArgs& a) {
  if (a.rows <= 0 || a.m <= 0) return hipSuccess;
  const int splits = skinny_splits(a.m, a.rows, a.n, (size_t)max_lds_per_block());
  if (splits > 0) return launch_skinny(stream, a, splits);
  switch (a.epi) {
    case kStore: return launch_epi<kStore>(stream, a);
    case kResidual: return launch_epi<kResidual>(stream, a);
    case kSiluPair: return launch_epi<kSiluPair>(stream, a);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace ivo
