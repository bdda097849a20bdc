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
//   * its weight rows' 32 packed bytes, which each wave reads as 8 bytes per
//     lane and expands in registers to the codes 0, 1, 2 as int8 (two VALU
//     operations per 4 codes) - a quarter of the LDS traffic of staging the
//     expanded codes;
//   * minus each token's activation sum over the group, which seeds the
//     MFMA accumulator, so sum (code * q) - sum q = P comes out exact with no
//     per-output correction;
//   * the fp16 group scales of its rows.
// LDS rows are padded (q8 rows from 128 to 144 bytes, packed rows from 32 to
// 48), which spreads the lanes of each operand read over distinct banks.
// Each group's global loads are issued two group-steps before they are
// staged, from two register sets, and there is one barrier per group.
//
// Operand pairing: MFMA half h of a group takes, in lane (c = lane % 16,
// kb = lane / 16), the 16 bytes of word 2*kb + h of the group (inputs
// 16*(2kb+h) .. +15).  The q8 layout stores a word's quad in exactly the
// order the expansion (w >> 2k) & 0x03030303 produces, so both operands see
// the same input in the same byte slot.  Each group's int32 tile is folded
// into fp32 with one fmaf per output in ascending group order (the order the
// CPU oracle restates as orc_gemm_seq); the fold of one 16-token row of tiles
// is independent of the next row's MFMAs, so the two overlap.
#include "internal.hpp"
#include "ternary_device.hpp"

namespace ivo {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kRowPitch = 144;  // bytes per staged LDS row (128 + 16 padding)

// Raw buffer resource over `bytes` bytes of an operand (the launcher keeps
// every operand below 2 GiB).  Offsets at or past the size read zeros.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t operand_buffer(const void* base, long long bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

// Codes of field k of four packed bytes, one per byte (0, 1, 2).
__device__ __forceinline__ unsigned field_codes(unsigned w, int k) { return (w >> (2 * k)) & kLow2; }

constexpr int kPackedPitch = 48;  // bytes per staged packed weight row (32 + 16 padding)
constexpr int kOutPitch = 68;     // floats per row of the epilogue's transpose tile

// LDS stage: A rows (q8), packed B rows, fp32 row scales, minus the token
// sums.  Two stages, and afterwards the epilogue's transpose tiles.
template <int WM, int WN>
struct Tile {
  static constexpr int kWaves = WM * WN;
  static constexpr int kThreadsPerBlock = 64 * kWaves;
  static constexpr int kTokens = 64 * WM;
  static constexpr int kRowsPerBlock = 64 * WN;
  static constexpr int kPackedOffset = kTokens * kRowPitch;
  static constexpr int kScaleOffset = kPackedOffset + kRowsPerBlock * kPackedPitch;
  static constexpr int kSumOffset = kScaleOffset + kRowsPerBlock * 4;
  static constexpr int kStageBytes = kSumOffset + kTokens * 4;
  static constexpr int kOutBytes = kWaves * 64 * kOutPitch * 4;
  static constexpr int kLdsBytes = 2 * kStageBytes > kOutBytes ? 2 * kStageBytes : kOutBytes;
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

  // Staging: A in 16-byte pieces, eight per token and group (consecutive
  // threads read consecutive pieces of a token, so each load instruction
  // covers whole 128-byte lines); B in 16-byte packed pieces, two per weight
  // row (each expanding to 64 bytes); one scale per row and the two chunk
  // sums per token.  Two register sets hold the next two groups while the
  // MFMAs consume the third from LDS.
  constexpr int kThreadsN = T::kThreadsPerBlock;
  constexpr int kLoadsA = T::kTokens * 8 / kThreadsN;
  constexpr int kLoadsB = T::kRowsPerBlock * 2 / kThreadsN;
  static_assert(T::kTokens * 8 % kThreadsN == 0 && T::kRowsPerBlock * 2 % kThreadsN == 0, "whole pieces");
  static_assert(T::kTokens <= kThreadsN && T::kRowsPerBlock <= kThreadsN, "one thread per token sum and scale");
  struct Regs {
    uint4 a[kLoadsA];
    uint4 b[kLoadsB];
    uint16_t s;
    int x0, x1;
    int g;
  };
  const bool s_thread = tid < T::kRowsPerBlock;
  const bool x_thread = tid < T::kTokens;

  // Buffer loads: each operand is a buffer resource whose size the hardware
  // checks, returning zeros past it (tokens past m, rows past the matrix),
  // so no address is clamped.  A thread's offsets into the operands are
  // fixed for the whole kernel; the group advances a scalar offset.  A
  // missing second chunk (odd chunk count, last group) is read at an offset
  // past the operand, and its chunk sum is dropped when staged.  Loads are
  // never predicated (a predicated load would make the compiler wait for
  // every outstanding load at its first use).
  constexpr int kPast = 0x7FFFFFF0;
  const __amdgpu_buffer_rsrc_t q8_buf = operand_buffer(q8, (long long)a.m * (long long)q8_stride);
  const __amdgpu_buffer_rsrc_t w_buf = operand_buffer(packed, (long long)a.rows * a.row_bytes);
  const __amdgpu_buffer_rsrc_t s_buf = operand_buffer(scales, (long long)a.rows * a.groups * 2);
  const __amdgpu_buffer_rsrc_t x_buf = operand_buffer(a.xsum_in, (long long)a.m * chunks * 4);
  int a_off[kLoadsA], a_dead[kLoadsA], b_off[kLoadsB], b_dead[kLoadsB];
#pragma unroll
  for (int k = 0; k < kLoadsA; ++k) {
    const int f = k * kThreadsN + tid;
    a_off[k] = (token0 + (f >> 3)) * (int)q8_stride + (f & 7) * 16;
    a_dead[k] = (f & 7) < 4 ? a_off[k] : kPast;
  }
#pragma unroll
  for (int k = 0; k < kLoadsB; ++k) {
    const int f = k * kThreadsN + tid;
    b_off[k] = (row0 + (f >> 1)) * a.row_bytes + (f & 1) * 16;
    b_dead[k] = (f & 1) == 0 ? b_off[k] : kPast;
  }
  const int s_off = (row0 + tid % T::kRowsPerBlock) * a.groups * 2;
  const int x_off = (token0 + tid % T::kTokens) * chunks * 4;

  auto fetch = [&](Regs& r, int g_raw) {
    const int g = min(g_raw, groups - 1);
    r.g = g;
    const bool second_live = 2 * g + 1 < chunks;
#pragma unroll
    for (int k = 0; k < kLoadsA; ++k)
      r.a[k] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(q8_buf, second_live ? a_off[k] : a_dead[k], g * kGroup, 0));
#pragma unroll
    for (int k = 0; k < kLoadsB; ++k)
      r.b[k] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(w_buf, second_live ? b_off[k] : b_dead[k], g * 32, 0));
    r.s = __builtin_amdgcn_raw_buffer_load_b16(s_buf, s_off, g * 2, 0);
    r.x0 = (int)__builtin_amdgcn_raw_buffer_load_b32(x_buf, x_off, g * 8, 0);
    r.x1 = (int)__builtin_amdgcn_raw_buffer_load_b32(x_buf, second_live ? x_off + 4 : kPast, g * 8, 0);
  };
  auto stage = [&](const Regs& r, int buffer) {
    unsigned char* base = smem + (size_t)buffer * T::kStageBytes;
    const bool second_live = 2 * r.g + 1 < chunks;  // wave-uniform
#pragma unroll
    for (int k = 0; k < kLoadsA; ++k) {
      const int f = k * kThreadsN + tid;
      const int piece = f & 7;
      uint4* dst = reinterpret_cast<uint4*>(base + (f >> 3) * kRowPitch + piece * 16);
      *dst = (second_live || piece < 4) ? r.a[k] : make_uint4(0u, 0u, 0u, 0u);
    }
#pragma unroll
    for (int k = 0; k < kLoadsB; ++k) {
      const int f = k * kThreadsN + tid;
      *reinterpret_cast<uint4*>(base + T::kPackedOffset + (f >> 1) * kPackedPitch + (f & 1) * 16) = r.b[k];
    }
    if (s_thread) reinterpret_cast<float*>(base + T::kScaleOffset)[tid] = h2f(r.s);
    if (x_thread) reinterpret_cast<int*>(base + T::kSumOffset)[tid] = -(r.x0 + (second_live ? r.x1 : 0));
  };

  float acc[4][4][4];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[mt][nt][i] = 0.0f;

  // One group from LDS.  The weight fragments of both MFMA halves stay in
  // registers; per 16-token row of tiles the accumulators start at minus the
  // tokens' group sums and the two halves add sum(code * q), giving P; the
  // previous row's P is folded into fp32 (one fmaf per output with the row's
  // group scale) while this row's MFMAs run.
  auto compute = [&](int buffer) {
    const unsigned char* base = smem + (size_t)buffer * T::kStageBytes;
    const unsigned char* a_lds = base + (wm * 64 + col) * kRowPitch;
    const unsigned char* b_lds = base + T::kPackedOffset + (wn * 64 + col) * kPackedPitch + kb * 8;
    const float* s_lds = reinterpret_cast<const float*>(base + T::kScaleOffset);
    const int* x_lds = reinterpret_cast<const int*>(base + T::kSumOffset) + wm * 64 + 4 * kb;
    v4i bf[2][4];
    float sc[4];
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      // Words 2kb and 2kb+1 of the row's group, expanded to one code per byte.
      const uint2 w = *reinterpret_cast<const uint2*>(b_lds + nt * 16 * kPackedPitch);
      bf[0][nt] = v4i{(int)field_codes(w.x, 0), (int)field_codes(w.x, 1), (int)field_codes(w.x, 2),
                      (int)field_codes(w.x, 3)};
      bf[1][nt] = v4i{(int)field_codes(w.y, 0), (int)field_codes(w.y, 1), (int)field_codes(w.y, 2),
                      (int)field_codes(w.y, 3)};
      sc[nt] = s_lds[wn * 64 + nt * 16 + col];
    }
    auto fold = [&](const v4i (&p)[4], int mt) {
#pragma unroll
      for (int nt = 0; nt < 4; ++nt)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[mt][nt][i] = __builtin_fmaf((float)p[nt][i], sc[nt], acc[mt][nt][i]);
    };
    v4i prev[4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      const v4i a0 = *reinterpret_cast<const v4i*>(a_lds + mt * 16 * kRowPitch + (2 * kb) * 16);
      const v4i a1 = *reinterpret_cast<const v4i*>(a_lds + mt * 16 * kRowPitch + (2 * kb + 1) * 16);
      const v4i seed = *reinterpret_cast<const v4i*>(x_lds + mt * 16);
      v4i p[4];
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) p[nt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, bf[0][nt], seed, 0, 0, 0);
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) p[nt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, bf[1][nt], p[nt], 0, 0, 0);
      if (mt > 0) fold(prev, mt - 1);
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) prev[nt] = p[nt];
      if (mt > 0) {
        // Issue order hint: each of this row's MFMAs followed by four VALU
        // instructions of the previous row's fold.
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
        }
      }
    }
    fold(prev, 3);
  };

  // LDS buffer g & 1 holds group g; register sets r0 / r1 alternate.
  Regs r0, r1;
  fetch(r0, 0);
  fetch(r1, 1);
  stage(r0, 0);
  __syncthreads();
  fetch(r0, 2);
  // Staging is unconditional (past the last group it rewrites the idle
  // buffer with the last group's data), so each group step is one straight
  // block the scheduler can interleave.
  for (int g = 0; g < groups; g += 2) {
    compute(0);
    stage(r1, 1);
    __syncthreads();
    fetch(r1, g + 3);
    if (g + 1 >= groups) break;
    compute(1);
    stage(r0, 0);
    __syncthreads();
    fetch(r0, g + 4);
  }

  // Epilogue.  y = acc * s_x[t] (+ bias[r]) in the MFMA layout (lane holds
  // row nt*16 + col of tokens mt*16 + 4*kb + i), transposed through LDS (the
  // stage buffers are free by now) so that each lane then owns four
  // consecutive rows of one token and the stores are 16-byte vectors over
  // whole rows of the output.
  float sx[4][4];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int i = 0; i < 4; ++i) sx[mt][i] = scale_in[min(token0 + wm * 64 + mt * 16 + 4 * kb + i, a.m - 1)];
  constexpr int kPitch = kOutPitch;  // conflict-free column writes
  float* tile = reinterpret_cast<float*>(smem) + wave * 64 * kPitch;
  __syncthreads();
#pragma unroll
  for (int nt = 0; nt < 4; ++nt) {
    const int row = row0 + wn * 64 + nt * 16 + col;
    const float b = (bias != nullptr && row < a.rows) ? bias[row] : 0.0f;
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float y = acc[mt][nt][i] * sx[mt][i];
        if (bias != nullptr) y = y + b;
        tile[(mt * 16 + 4 * kb + i) * kPitch + nt * 16 + col] = y;
      }
  }
  __syncthreads();
  const int r4 = (lane & 15) * 4;
  const int row = row0 + wn * 64 + r4;  // first of the lane's four rows (a multiple of 4)
  const bool rows_whole = row + 3 < a.rows;
  const uintptr_t base_addr = reinterpret_cast<uintptr_t>(output);
  const bool vec4 = (a.out_stride & 3) == 0 && (base_addr & 15) == 0;
  const bool vec2 = (a.out_stride & 1) == 0 && (base_addr & 7) == 0;
#pragma unroll 4
  for (int j = 0; j < 16; ++j) {
    const int tl = j * 4 + (lane >> 4);
    const int t = token0 + wm * 64 + tl;
    if (t >= a.m) continue;
    const float4 v = *reinterpret_cast<const float4*>(tile + tl * kPitch + r4);
    float* orow = output + (size_t)t * a.out_stride;
    if constexpr (EPI == kSiluPair) {
      const float p0 = ivo_silu(v.x) * v.y, p1 = ivo_silu(v.z) * v.w;
      if (rows_whole && vec2) {
        *reinterpret_cast<float2*>(orow + (row >> 1)) = make_float2(p0, p1);
      } else {
        if (row + 1 < a.rows) orow[row >> 1] = p0;
        if (row + 3 < a.rows) orow[(row >> 1) + 1] = p1;
      }
    } else if (rows_whole && vec4) {
      float4* dst = reinterpret_cast<float4*>(orow + row);
      if constexpr (EPI == kResidual) {
        const float4 o = *dst;
        *dst = make_float4(o.x + v.x, o.y + v.y, o.z + v.z, o.w + v.w);
      } else {
        *dst = v;
      }
    } else {
      const float vs[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        if (row + k < a.rows) {
          if constexpr (EPI == kResidual) orow[row + k] = orow[row + k] + vs[k];
          else orow[row + k] = vs[k];
        }
      }
    }
  }
}

template <int EPI, int WM, int WN>
hipError_t launch_shape(hipStream_t stream, const GemmArgs& a) {
  using T = Tile<WM, WN>;
  const dim3 grid(ceil_div(a.rows, T::kRowsPerBlock), ceil_div(a.m, T::kTokens));
  const size_t lds = (size_t)T::kLdsBytes;
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
  return Tile<WM, WN>::kLdsBytes <= max_lds_per_block();
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

// Kernel choice: the decode GEMV for one token, and for two tokens with
// 4097..32768 inputs (the long-row GEMV over both tokens' copies: each
// token's outputs are those of its own GEMV); the token GEMV for up to 16
// tokens (K a multiple of 256; K sliced across blocks where the tokens' q8
// rows do not fit in LDS whole);
// the skinny kernels up to 32 tokens; then the long-prompt
// tilings; then the LDS-staged skinny kernel in 32-token slices up to
// kSlicedTokens; otherwise the tiled kernel.
int gemm_splits(int m, int rows, int n) {
  if (m == 1 && gemv_prequant_applies(n)) return 0;
  if (gemv_tokens_apply(m, n)) return 0;
  const size_t lds = (size_t)max_lds_per_block();
  const TokenPlan tokens = token_gemv_plan(m, rows, n, device_cus(), lds);
  if (tokens.parts > 0) return tokens.parts * tokens.slices;
  if (gemm_wide_tokens(m, rows, n) > 0) return 1;
  if (gemm_split_applies(m, rows, n)) return split_waves(m, rows, n);
  const SkinnyPlan plan = skinny_plan(m, rows, n, lds);
  return plan.splits > 0 ? plan.splits : 1;
}

hipError_t launch_gemm(hipStream_t stream, const GemmArgs& a) {
  if (a.rows <= 0 || a.m <= 0) return hipSuccess;
  const bool tokens_gemv = gemv_tokens_apply(a.m, a.n);
  if ((a.m == 1 && gemv_prequant_applies(a.n)) || tokens_gemv) {
    // One token: the decode GEMV on the pre-quantized row (the q8 row layout
    // is the same); the output stride does not matter for a single row.
    // Two tokens of long rows: the long-row GEMV over each token's copy,
    // outputs out_stride floats apart.
    GemvArgs g{};
    g.mode = kPlain;
    g.epi = a.epi;
    g.q8_in = a.q8_in;
    g.xsum_in = a.xsum_in;
    g.scale_in = a.scale_in;
    g.packed = a.packed;
    g.scales = a.scales;
    g.bias = a.bias;
    g.output = a.output;
    g.rows = a.rows;
    g.n = a.n;
    g.row_bytes = a.row_bytes;
    g.groups = a.groups;
    g.splits = 1;
    g.head_dim = defines().head_dim;
    if (tokens_gemv) return launch_gemv_tokens(stream, g, a.m, a.out_stride);
    return launch_gemv(stream, g);
  }
  const size_t lds = (size_t)max_lds_per_block();
  const TokenPlan tokens = token_gemv_plan(a.m, a.rows, a.n, device_cus(), lds);
  if (tokens.parts > 0) return launch_token_gemv(stream, a, tokens);
  if (a.m <= 32) {
    const SkinnyPlan plan = skinny_plan(a.m, a.rows, a.n, lds);
    if (plan.splits > 0) return launch_skinny(stream, a, plan);
  }
  // Buffer offsets are 32-bit: every operand (with a tile of slack) stays below 2 GiB.
  const long long limit = 0x7FFFFFF0LL;
  if (((long long)a.m + 256) * ceil_div(a.n, kChunk) * kChunk >= limit ||
      ((long long)a.rows + 256) * a.row_bytes >= limit || ((long long)a.rows + 256) * a.groups * 2 >= limit)
    return hipErrorInvalidValue;
  if (gemm_wide_tokens(a.m, a.rows, a.n) > 0) return launch_gemm_wide(stream, a);
  if (gemm_split_applies(a.m, a.rows, a.n)) return launch_gemm_split(stream, a);
  const SkinnyPlan sliced = skinny_plan(a.m, a.rows, a.n, lds);
  if (sliced.splits > 0) return launch_skinny(stream, a, sliced);
  switch (a.epi) {
    case kStore: return launch_epi<kStore>(stream, a);
    case kResidual: return launch_epi<kResidual>(stream, a);
    case kSiluPair: return launch_epi<kSiluPair>(stream, a);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace ivo
