// Token GEMM for long prompts on CDNA4 int8 MFMA (reference: kernels/ternary.cu:
// 688-784, entry points gemm_tile_* with GEMM_ARGS; the reference uses dp4a).
//
// y[t, r] = s_x[t] * sum_g P[t, r, g] * scale[r, g] (+ bias[r]), where
// P[t, r, g] = sum over the 128 inputs of group g of (code - 1) * q is exact.
//
// Why a second tiled kernel: every (token, row, group) needs one int -> fp32
// conversion and one fmaf after its two MFMAs, i.e. four VALU instructions per
// v_mfma_i32_16x16x64_i8.  On gfx950 a VALU instruction between MFMAs costs
// about as much issue time as a quarter of an MFMA, so the MFMA pipe stays
// busy only if (a) nothing else adds VALU work and (b) the conversions of one
// tile run while the next tile's MFMAs execute.  This kernel is built for
// that:
//   * a wave owns 16*MT tokens x 64 rows (MT = 8: 128 tokens), so each
//     expanded weight fragment feeds MT MFMA rows and the expansion costs
//     under one VALU instruction per MFMA;
//   * operands reach LDS by direct buffer-to-LDS loads (no staging registers,
//     no VALU, no LDS write instructions); tokens past m, rows past the
//     matrix and the missing second chunk of an odd chunk count read as zeros
//     through the buffer range check;
//   * the fold of token row mt-1 (int32 -> fp32, one fmaf per output with the
//     row's group scale, ascending groups: the order the CPU oracle restates
//     as orc_gemm_seq) is interleaved with the MFMAs of token row mt, and the
//     last row of a group with the first row of the next group.
//
// LDS stage (three, so that two groups are in flight; one barrier per group):
//   A: 16*MT token rows x 8 pieces of 16 bytes (the group's q8 bytes), piece p
//      of token t at slot t*8 + (p ^ swz(t)), swz(t) = (t & 7) ^ ((t >> 3) & 1),
//      which keeps each 8- or 16-lane phase of the operand reads on distinct
//      banks;
//   B: 64*WN weight rows x 2 pieces of 16 bytes (the group's packed bytes),
//      piece p of row r at slot p * 64*WN + r, so the 8-byte operand reads of
//      a wave cover two contiguous 256-byte runs;
//   the rows' fp32 scales, loaded into registers three groups ahead and
//   written to LDS one step before their group is computed.
// The weight fragments are expanded to signed int8 codes (-1, 0, +1; one
// v_perm_b32 table lookup per four codes), so the MFMA chain of a group starts
// from zero and returns P itself: no per-token group sums are staged or read
// (with the unsigned codes 0..2, the seed -sum(q) of every token row was a
// third of the LDS operand reads; K=4096 -> N=14336 at M=2048: 164 -> 151 us).
// Loading the side values three groups ahead instead of two: 164 -> 158.6 us
// with the seeds, 151.1 -> 149.4 us with the signed codes.
#include "buffer_ops.hpp"
#include "internal.hpp"
#include "ternary_device.hpp"

namespace ivo {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

template <int MT, int WN>
struct WideTile {
  static constexpr int kThreads = 64 * WN;
  static constexpr int kTokens = 16 * MT;
  static constexpr int kRows = 64 * WN;
  static constexpr int kAOffset = 0;
  static constexpr int kBOffset = kTokens * 128;
  static constexpr int kStageBytes = kBOffset + kRows * 32;  // DMA part of one stage
  static constexpr int kLdsBytes = 3 * (kStageBytes + kRows * 4);
  static constexpr int kLoadsA = kTokens * 8 / kThreads;  // 16-byte pieces per thread and group
  static constexpr int kLoadsB = kRows * 2 / kThreads;
  static constexpr int kLoads = kLoadsA + kLoadsB;         // DMA instructions per thread and group
  static_assert(kTokens * 8 % kThreads == 0 && kRows * 2 == 2 * kThreads, "whole DMA rounds");
};

template <int EPI, int MT, int WN>
__global__ __launch_bounds__(64 * WN) void gemm_wide_kernel(const int8_t* __restrict__ q8,
                                                            const float* __restrict__ scale_in,
                                                            const uint8_t* __restrict__ packed,
                                                            const uint16_t* __restrict__ scales,
                                                            const float* __restrict__ bias,
                                                            float* __restrict__ output, GemmArgs a) {
  using T = WideTile<MT, WN>;
  __shared__ __align__(16) unsigned char stages[3][T::kStageBytes];
  __shared__ __align__(16) float row_scales[3][T::kRows];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 15, kb = lane >> 4;
  const int chunks = (a.n + kChunk - 1) / kChunk;
  const int groups = (a.n + kGroup - 1) / kGroup;
  const int q8_stride = chunks * kChunk;
  const int token0 = blockIdx.y * T::kTokens;
  const int row0 = blockIdx.x * T::kRows;
  constexpr int kPast = 0x7FFFFFF0;

  const v4u q8_buf = wide_buffer(q8, (long long)a.m * q8_stride);
  const v4u w_buf = wide_buffer(packed, (long long)a.rows * a.row_bytes);
  const v4u s_buf = wide_buffer(scales, (long long)a.rows * a.groups * 2);

  // Per-thread DMA offsets, fixed for the kernel (the group moves the scalar
  // offset).  A: slot s = j * threads + tid holds token s >> 3, piece
  // (s & 7) ^ swz(token).  Pieces 4..7 are the group's second chunk.
  int a_live[T::kLoadsA], a_dead[T::kLoadsA];
#pragma unroll
  for (int j = 0; j < T::kLoadsA; ++j) {
    const int s = j * T::kThreads + tid;
    const int t = s >> 3;
    const int p = (s & 7) ^ a_swizzle(t);
    a_live[j] = (token0 + t) * q8_stride + p * 16;
    a_dead[j] = p < 4 ? a_live[j] : kPast;
  }
  // B: slot s = j * threads + tid holds row tid, piece j.
  const int b_off = (row0 + tid) * a.row_bytes;
  const int s_off = (row0 + tid) * a.groups * 2;

  auto dma = [&](int g, int stage) {
    const bool second_live = 2 * g + 1 < chunks;
    const unsigned base = __builtin_amdgcn_readfirstlane(lds_address(stages[stage]) + wave * 64 * 16);
#pragma unroll
    for (int j = 0; j < T::kLoadsA; ++j)
      dma16(q8_buf, base + T::kAOffset + j * T::kThreads * 16, second_live ? a_live[j] : a_dead[j], g * kGroup);
#pragma unroll
    for (int j = 0; j < T::kLoadsB; ++j)
      dma16(w_buf, base + T::kBOffset + j * T::kThreads * 16, b_off + j * 16, g * 32);
  };
  // The row scale of a group (thread tid: row tid), loaded into a register
  // three groups ahead and written to LDS as fp32 two steps later.  The
  // wait before the store leaves in flight only what the wave issued after
  // that load: the DMA of the next group (kLoads) and the next scale load (1).
  auto scale_load = [&](int g) { return load_u16(s_buf, s_off, g * 2); };
  auto scale_store = [&](int& r, int stage) {
    asm volatile("s_waitcnt vmcnt(%1)" : "+v"(r) : "n"(T::kLoads + 1) : "memory");
    row_scales[stage][tid] = h2f((uint16_t)r);
  };

  float acc[MT][4][4];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[mt][nt][i] = 0.0f;

  // The previous token row's int32 tiles and scales, folded while the next
  // row's MFMAs run.  Zero before the first group (a fold of zeros leaves
  // acc at +0).
  v4i prev[4];
  float prev_sc[4];
#pragma unroll
  for (int nt = 0; nt < 4; ++nt) {
    prev[nt] = v4i{0, 0, 0, 0};
    prev_sc[nt] = 0.0f;
  }
  auto fold = [&](int mt) {
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[mt][nt][i] = __builtin_fmaf((float)prev[nt][i], prev_sc[nt], acc[mt][nt][i]);
  };

  const int b_read = ((kb >> 1) * T::kRows + wave * 64 + col) * 16 + (kb & 1) * 8;
  const int sc_read = wave * 64 + col;

  // One group step.  Group g+2 streams into the stage group g-1 used while
  // group g is computed: first its DMA, then the scale load of g+3, then the
  // MFMAs of g, then the scale of g+2 (loaded in the previous step) goes to
  // LDS.  The wait before that store also retires the DMA of g+1 (loads
  // complete in order) and leaves the DMA of g+2 and the scale load of g+3
  // in flight; lgkmcnt(0) and the barrier at the top of the next step
  // complete direct_load_sync's sequence for every wave's pieces of g+1.  `pending` holds the scale of g+2 and `fresh`
  // receives that of g+3; the caller alternates the two registers.
  auto step = [&](int g, int cur, int fill, int& pending, int& fresh) {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    dma(min(g + 2, groups - 1), fill);  // past the end: the last group again (never read)
    fresh = scale_load(min(g + 3, groups - 1));

    // The step is written as a fixed issue order (scheduling fences between
    // units): per token row, eight units of one MFMA and two outputs (four
    // VALU instructions) of the previous row's fold; the next row's operand
    // reads go out at the start of a row; in the first row each unit also
    // expands the weight fragment its MFMA takes.
    const unsigned char* base = stages[cur];
    const v4i zero = {0, 0, 0, 0};
    uint2 w[4];
    float sc[4];
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      w[nt] = *reinterpret_cast<const uint2*>(base + T::kBOffset + b_read + nt * 16 * 16);
      sc[nt] = row_scales[cur][sc_read + nt * 16];
    }
    auto operands = [&](int mt, v4i& a0, v4i& a1) {
      const int t = mt * 16 + col;
      const unsigned char* arow = base + T::kAOffset + t * 128;
      a0 = *reinterpret_cast<const v4i*>(arow + (((2 * kb) ^ a_swizzle(t)) * 16));
      a1 = *reinterpret_cast<const v4i*>(arow + (((2 * kb + 1) ^ a_swizzle(t)) * 16));
    };
    v4i a0, a1;
    operands(0, a0, a1);
    v4i bf[2][4];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      v4i na0, na1;
      if (mt + 1 < MT) operands(mt + 1, na0, na1);
      const int fold_row = mt == 0 ? MT - 1 : mt - 1;
      v4i p[4];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int h = u >> 2, nt = u & 3;
        if (mt == 0) {
          const unsigned x = h ? w[nt].y : w[nt].x;
          bf[h][nt] = v4i{(int)signed_codes(x, 0), (int)signed_codes(x, 1), (int)signed_codes(x, 2),
                          (int)signed_codes(x, 3)};
        }
        p[nt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(h ? a1 : a0, bf[h][nt], h ? p[nt] : zero, 0, 0, 0);
        const int ft = u >> 1, fi = (u & 1) * 2;
        acc[fold_row][ft][fi] = __builtin_fmaf((float)prev[ft][fi], prev_sc[ft], acc[fold_row][ft][fi]);
        acc[fold_row][ft][fi + 1] = __builtin_fmaf((float)prev[ft][fi + 1], prev_sc[ft], acc[fold_row][ft][fi + 1]);
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) prev[nt] = p[nt];
      if (mt == 0) {
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) prev_sc[nt] = sc[nt];
      }
      if (mt + 1 < MT) {
        a0 = na0;
        a1 = na1;
      }
    }
    scale_store(pending, fill);
  };

  // Prologue: groups 0 and 1 staged, the scales of 0 and 1 in LDS (the wait
  // of each store leaves the DMA of group 1 and the scale load of group 2 in
  // flight), the scale of group 2 pending.
  int scale_a, scale_b;
  {
    int s0 = scale_load(0);
    dma(0, 0);
    int s1 = scale_load(min(1, groups - 1));
    dma(min(1, groups - 1), 1);
    scale_a = scale_load(min(2, groups - 1));
    scale_store(s0, 0);
    scale_store(s1, 1);
  }
  // Unrolled by two so that the pending and the fresh scale swap registers
  // without a copy: a copy would read a register whose load may not have
  // landed yet.
  int cur = 0;
  int g = 0;
  for (; g + 1 < groups; g += 2) {
    step(g, cur, cur == 0 ? 2 : cur - 1, scale_a, scale_b);  // fill = (g + 2) % 3
    cur = cur == 2 ? 0 : cur + 1;
    step(g + 1, cur, cur == 0 ? 2 : cur - 1, scale_b, scale_a);
    cur = cur == 2 ? 0 : cur + 1;
  }
  if (g < groups) step(g, cur, cur == 0 ? 2 : cur - 1, scale_a, scale_b);
  // No direct-to-LDS load may still be in flight when the block's LDS is
  // handed to the next block, and the last scale loads (never stored) keep
  // their registers until they have landed.
  asm volatile("s_waitcnt vmcnt(0)" : "+v"(scale_a), "+v"(scale_b)::"memory");
  fold(MT - 1);

  // Epilogue.  y = acc * s_x[t] (+ bias[r]) in the MFMA layout (lane holds
  // rows wave*64 + nt*16 + col of tokens mt*16 + 4*kb + i), transposed through
  // LDS one 16-token row of tiles at a time, so that each lane then owns four
  // consecutive rows of one token and every store is a 16-byte vector, 16
  // lanes covering 256 contiguous bytes of an output row, written with the
  // non-temporal hint (the output is streamed once; measured 2-9% faster on
  // the prefill shapes than plain stores).  Each wave uses its
  // own slice of the stages; a wave's LDS operations complete in order,
  // so the slice needs no barrier between its writes and reads.
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  constexpr int kPitch = 68;  // floats per token row of a slice (conflict-free column writes)
  static_assert(4 * 16 * kPitch * 4 <= 3 * T::kStageBytes, "transpose slices fit the stages");
  float* slice = reinterpret_cast<float*>(&stages[0][0]) + wave * 16 * kPitch;
  const bool has_bias = bias != nullptr;
  float bv[4];
#pragma unroll
  for (int nt = 0; nt < 4; ++nt) {
    const int row = row0 + wave * 64 + nt * 16 + col;
    bv[nt] = (has_bias && row < a.rows) ? bias[row] : 0.0f;
  }
  const int r4 = (lane & 15) * 4;
  const int row = row0 + wave * 64 + r4;  // first of the lane's four rows (a multiple of 4)
  const bool rows_whole = row + 3 < a.rows;
  const uintptr_t base_addr = reinterpret_cast<uintptr_t>(output);
  const bool vec4 = (a.out_stride & 3) == 0 && (base_addr & 15) == 0;
  const bool vec2 = (a.out_stride & 1) == 0 && (base_addr & 7) == 0;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    float sx[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) sx[i] = scale_in[min(token0 + mt * 16 + 4 * kb + i, a.m - 1)];
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float y = acc[mt][nt][i] * sx[i];
        if (has_bias) y = y + bv[nt];
        slice[(4 * kb + i) * kPitch + nt * 16 + col] = y;
      }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int tl = j * 4 + (lane >> 4);
      const int t = token0 + mt * 16 + tl;
      const float4 v = *reinterpret_cast<const float4*>(slice + tl * kPitch + r4);
      if (t >= a.m) continue;
      float* orow = output + (size_t)t * a.out_stride;
      if constexpr (EPI == kSiluPair) {
        const float p0 = ivo_silu(v.x) * v.y, p1 = ivo_silu(v.z) * v.w;
        if (rows_whole && vec2) {
          __builtin_nontemporal_store(f2v{p0, p1}, reinterpret_cast<f2v*>(orow + (row >> 1)));
        } else {
          if (row + 1 < a.rows) orow[row >> 1] = p0;
          if (row + 3 < a.rows) orow[(row >> 1) + 1] = p1;
        }
      } else if (rows_whole && vec4) {
        f4v* dst = reinterpret_cast<f4v*>(orow + row);
        if constexpr (EPI == kResidual) {
          const f4v o = *dst;
          __builtin_nontemporal_store(f4v{o.x + v.x, o.y + v.y, o.z + v.z, o.w + v.w}, dst);
        } else {
          __builtin_nontemporal_store(f4v{v.x, v.y, v.z, v.w}, dst);
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
}

template <int EPI, int MT, int WN>
hipError_t launch_wide_shape(hipStream_t stream, const GemmArgs& a) {
  using T = WideTile<MT, WN>;
  const dim3 grid(ceil_div(a.rows, T::kRows), ceil_div(a.m, T::kTokens));
  hipLaunchKernelGGL((gemm_wide_kernel<EPI, MT, WN>), grid, dim3(T::kThreads), 0, stream,
                     a.q8_in, a.scale_in, a.packed, a.scales, a.bias, a.output, a);
  return hipGetLastError();
}

template <int EPI>
hipError_t launch_wide_epi(hipStream_t stream, const GemmArgs& a, int tokens) {
  if (tokens == 32) return launch_wide_shape<EPI, 2, 4>(stream, a);
  if (tokens == 64) return launch_wide_shape<EPI, 4, 4>(stream, a);
  return launch_wide_shape<EPI, 8, 4>(stream, a);
}

// Block -> output tile of the split-K kernel.  Blocks are dispatched to the
// device's 8 XCDs round robin (block b on XCD b % 8), each XCD with its own
// L2; this mapping gives each XCD a run of consecutive tiles in token-major
// order (all row tiles of one token tile, then the next), so the q8 rows and
// weight rows an XCD's blocks read stay in that XCD's L2 (K=4096 -> N=1024 at
// M=2048: 1 MB of q8 and the whole 1 MB matrix per XCD; 23.6 -> 21 us).
constexpr int kXcds = 8;
__device__ __forceinline__ void xcd_tile(int& tile_x, int& tile_y) {
  const int nx = gridDim.x, nb = gridDim.x * gridDim.y;
  const int b = blockIdx.x + nx * blockIdx.y;
  const int q = nb / kXcds, r = nb % kXcds;
  const int xcd = b % kXcds, idx = b / kXcds;
  const int t = xcd < r ? xcd * (q + 1) + idx : r * (q + 1) + (xcd - r) * q + idx;
  tile_x = t % nx;
  tile_y = t / nx;
}

// Split-K variant for long prompts with few output rows (K=4096 -> N=1024 at
// M=2048 has only 64 tiles of 128 x 256): a block of SW waves (4, or 8 with
// 32-token tiles and at least 32 groups) owns one 16*MT-token x 64-row output
// tile and wave w walks the contiguous group range [w*per, (w+1)*per),
// per = ceil(G/SW).  Each wave stages its own
// operands (its own two-stage ring of direct-to-LDS loads) and runs the same
// fixed-order MFMA/fold units as gemm_wide_kernel; the direct-to-LDS loads of
// the next group are spread over the first units (one per MFMA unit), so
// that a load instruction that waits for the memory pipeline to accept it
// stalls the wave while its MFMAs run (issued back to back before the MFMAs,
// they took 0.85 us of a 1.9 us step at M=512).  A stage is read after the
// loading wave's vmcnt wait, lgkmcnt(0) and a workgroup barrier
// (direct_load_sync), so every wave runs `per` steps: a wave with fewer
// groups (or none) loads again and skips the compute in the steps it lacks,
// and reaches every barrier.  The SW partial tiles are then added in wave
// order through LDS - the order the CPU oracle restates as orc_gemm_split(SW):
// each range an fmaf chain, total = ((s0 + s1) + s2) + ... - scaled by s_x and
// biased, and stored as 16-byte vectors.  MT (8, 4 or 2: 128, 64 or 32 token
// rows) is chosen by the launcher so that the grid fills the CUs; it does not
// change the order.  Eight waves halve each wave's dependent steps and put two
// waves on each SIMD; with 32- and 64-token tiles each wave keeps three stages
// (two groups in flight).  K=4096 -> N=1024 at M=512: 11.4 us with four waves
// and two stages, 10.9 with eight waves, 10.5 with three stages; at M=1024
// (64-token tiles, four waves) 14.9 -> 14.0 us.
constexpr int kSplitRows = 64;
constexpr int kSplitPitch = 68;  // floats per token row of a partial tile

template <int MT>
struct SplitTile {
  static constexpr int kTokens = 16 * MT;
  static constexpr int kStage = kTokens * 128 + kSplitRows * 32;  // A then B, one group
  static constexpr int kDmaA = kTokens * 8 / 64;                  // 16-byte pieces per lane and group
  static constexpr int kDma = kDmaA + 2;                          // direct-to-LDS loads per lane and group
  static_assert(kDma <= 8 * MT, "one load per MFMA unit at most");
};

template <int EPI, int MT, int SW, int NS>
__global__ __launch_bounds__(64 * SW) void gemm_split_kernel(const int8_t* __restrict__ q8,
                                                                     const float* __restrict__ scale_in,
                                                                     const uint8_t* __restrict__ packed,
                                                                     const uint16_t* __restrict__ scales,
                                                                     const float* __restrict__ bias,
                                                                     float* __restrict__ output, GemmArgs a) {
  using T = SplitTile<MT>;
  static_assert(NS == 2 || NS == 3, "two or three stages per wave");
  __shared__ __align__(16) unsigned char stages[SW][NS][T::kStage];
  __shared__ __align__(16) float row_scales[SW][NS][kSplitRows];
  static_assert(SW * T::kTokens * kSplitPitch * 4 <= (int)sizeof(stages), "partial tiles fit");
  static_assert(T::kTokens % (4 * SW) == 0, "each wave finishes whole rows of four tokens");
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 15, kb = lane >> 4;
  const int chunks = (a.n + kChunk - 1) / kChunk;
  const int groups = (a.n + kGroup - 1) / kGroup;
  const int q8_stride = chunks * kChunk;
  int tile_x, tile_y;
  xcd_tile(tile_x, tile_y);
  const int token0 = tile_y * T::kTokens;
  const int row0 = tile_x * kSplitRows;
  const int per = (groups + SW - 1) / SW;
  const int g_begin = min(wave * per, groups), g_end = min(g_begin + per, groups);
  constexpr int kPast = 0x7FFFFFF0;

  const v4u q8_buf = wide_buffer(q8, (long long)a.m * q8_stride);
  const v4u w_buf = wide_buffer(packed, (long long)a.rows * a.row_bytes);
  const v4u s_buf = wide_buffer(scales, (long long)a.rows * a.groups * 2);

  // A piece j of a lane: slot j*64 + lane = token 8j + (lane >> 3), piece
  // (lane & 7) ^ swz(token), where swz(8j + (lane >> 3)) = (lane >> 3) ^ (j & 1).
  int a_base[2], a_second[2];
#pragma unroll
  for (int parity = 0; parity < 2; ++parity) {
    const int p = (lane & 7) ^ (lane >> 3) ^ parity;
    a_base[parity] = (token0 + (lane >> 3)) * q8_stride + p * 16;
    a_second[parity] = p >= 4;
  }
  const int a_step = 8 * q8_stride;  // next DMA round: 8 tokens on
  const int b_off = (row0 + lane) * a.row_bytes;
  const int s_off = (row0 + lane) * a.groups * 2;

  // Direct-to-LDS load j (< kDma) of group g into stage `stage`: A pieces
  // first, then the two B pieces.
  auto dma = [&](int g, int stage, int j) {
    const unsigned base = __builtin_amdgcn_readfirstlane(lds_address(stages[wave][stage]));
    if (j < T::kDmaA) {
      const bool second_live = 2 * g + 1 < chunks;
      const int live = a_base[j & 1] + j * a_step;
      dma16(q8_buf, base + j * 64 * 16, second_live || !a_second[j & 1] ? live : kPast, g * kGroup);
    } else {
      const int jb = j - T::kDmaA;
      dma16(w_buf, base + T::kTokens * 128 + jb * 64 * 16, b_off + jb * 16, g * 32);
    }
  };
  // The row scale of a group (lane: row lane of the tile), written to LDS as
  // fp32 once every load of the wave has retired: the scale arrived and the
  // loads of the stage just filled are retired (direct_load_sync then makes
  // that stage readable).
  auto scale_load = [&](int g) { return load_u16(s_buf, s_off, g * 2); };
  auto scale_store = [&](int& r, int stage) {
    asm volatile("s_waitcnt vmcnt(0)" : "+v"(r)::"memory");
    row_scales[wave][stage][lane] = h2f((uint16_t)r);
  };

  float acc[MT][4][4];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[mt][nt][i] = 0.0f;
  v4i prev[4];
  float prev_sc[4];
#pragma unroll
  for (int nt = 0; nt < 4; ++nt) {
    prev[nt] = v4i{0, 0, 0, 0};
    prev_sc[nt] = 0.0f;
  }
  const int b_read = ((kb >> 1) * kSplitRows + col) * 16 + (kb & 1) * 8;

  // The MFMAs and fold of the group in stage `cur`, with the loads of group
  // g_fill into stage `fill` issued one per unit.
  auto compute = [&](int cur, int g_fill, int fill) {
    const unsigned char* base = stages[wave][cur];
    const v4i zero = {0, 0, 0, 0};
    uint2 w[4];
    float sc[4];
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      w[nt] = *reinterpret_cast<const uint2*>(base + T::kTokens * 128 + b_read + nt * 16 * 16);
      sc[nt] = row_scales[wave][cur][col + nt * 16];
    }
    auto operands = [&](int mt, v4i& a0, v4i& a1) {
      const int t = mt * 16 + col;
      const unsigned char* arow = base + t * 128;
      a0 = *reinterpret_cast<const v4i*>(arow + (((2 * kb) ^ a_swizzle(t)) * 16));
      a1 = *reinterpret_cast<const v4i*>(arow + (((2 * kb + 1) ^ a_swizzle(t)) * 16));
    };
    v4i a0, a1;
    operands(0, a0, a1);
    v4i bf[2][4];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      v4i na0, na1;
      if (mt + 1 < MT) operands(mt + 1, na0, na1);
      const int fold_row = mt == 0 ? MT - 1 : mt - 1;
      v4i p[4];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int h = u >> 2, nt = u & 3;
        if (mt == 0) {
          const unsigned x = h ? w[nt].y : w[nt].x;
          bf[h][nt] = v4i{(int)signed_codes(x, 0), (int)signed_codes(x, 1), (int)signed_codes(x, 2),
                          (int)signed_codes(x, 3)};
        }
        p[nt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(h ? a1 : a0, bf[h][nt], h ? p[nt] : zero, 0, 0, 0);
        if (mt * 8 + u < T::kDma) dma(g_fill, fill, mt * 8 + u);
        const int ft = u >> 1, fi = (u & 1) * 2;
        acc[fold_row][ft][fi] = __builtin_fmaf((float)prev[ft][fi], prev_sc[ft], acc[fold_row][ft][fi]);
        acc[fold_row][ft][fi + 1] = __builtin_fmaf((float)prev[ft][fi + 1], prev_sc[ft], acc[fold_row][ft][fi + 1]);
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) prev[nt] = p[nt];
      if (mt == 0) {
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) prev_sc[nt] = sc[nt];
      }
      if (mt + 1 < MT) {
        a0 = na0;
        a1 = na1;
      }
    }
  };

  if constexpr (NS == 2) {
    // One group step: the next group's loads into stage `fill` (inside the
    // MFMAs of stage `cur` when the wave has a group left, `live`; else on
    // their own), then the wait that retires them and the workgroup barrier.
    auto step = [&](int cur, int fill, int g_fill, bool live) {
      int scale = scale_load(g_fill);
      if (live) {
        compute(cur, g_fill, fill);
      } else {
#pragma unroll
        for (int j = 0; j < T::kDma; ++j) dma(g_fill, fill, j);
      }
      scale_store(scale, fill);
      direct_load_sync();
    };

    // Every wave runs `per` steps and passes every barrier; a wave whose range
    // is shorter (or empty) loads its last group (or the matrix's last) again
    // and skips the compute.
    {
      const int g0 = min(g_begin, groups - 1);
      int s0 = scale_load(g0);
#pragma unroll
      for (int j = 0; j < T::kDma; ++j) dma(g0, 0, j);
      scale_store(s0, 0);
      direct_load_sync();
    }
    int cur = 0;
    for (int i = 0; i < per; ++i) {
      const int g = g_begin + i;
      step(cur, cur ^ 1, max(min(g + 1, g_end - 1), 0), g < g_end);
      cur ^= 1;
    }
  } else {
    // Three stages, two groups in flight: step i computes stage i % 3 while
    // the loads of group i + 2 of the wave's range (and its scale) go to stage
    // (i + 2) % 3.  Its end retires the loads of group i + 1, issued one step
    // earlier (those of group i + 2, issued after them, stay in flight:
    // vmcnt(kDma + 1)), writes that group's scale to LDS and passes rule 5's
    // barrier.  The scales of groups i + 1 and i + 2 sit in two registers that
    // swap roles from step to step (the loop is unrolled by two), so no copy
    // ever reads a register whose load is still in flight.
    //
    // A step past the wave's range (a wave with fewer groups, or none) runs
    // the same code on the range's last group again (the matrix's last group
    // for an empty range) with its scale written as 0: every fold of that
    // step is fmaf(P, 0, acc) with P a finite integer, which returns acc
    // unchanged (acc starts at +0 and no fmaf of finite values with positive
    // scales makes it -0), so the sums are those of the range alone.  With no
    // branch between the live and the padding steps, every path issues the
    // same loads before each counter wait.
    auto gload = [&](int i) { return max(min(g_begin + i, g_end - 1), 0); };
    auto retire = [&](int& pending, int stage, bool live) {
      asm volatile("s_waitcnt vmcnt(%1)" : "+v"(pending) : "n"(T::kDma + 1) : "memory");
      row_scales[wave][stage][lane] = live ? h2f((uint16_t)pending) : 0.0f;
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    };
    int sa = scale_load(gload(0));
#pragma unroll
    for (int j = 0; j < T::kDma; ++j) dma(gload(0), 0, j);
    int sb = scale_load(gload(1));
#pragma unroll
    for (int j = 0; j < T::kDma; ++j) dma(gload(1), 1, j);
    retire(sa, 0, g_begin < g_end);
    auto step3 = [&](int i, int& pending, int& fresh) {
      const int cur = i % 3, fill = (i + 2) % 3;
      const int g_fill = gload(i + 2);
      fresh = scale_load(g_fill);
      compute(cur, g_fill, fill);
      retire(pending, (i + 1) % 3, g_begin + i + 1 < g_end);
    };
    int i = 0;
    for (; i + 1 < per; i += 2) {
      step3(i, sb, sa);
      step3(i + 1, sa, sb);
    }
    if (i < per) step3(i, sb, sa);
    // The last scale loads keep their registers until they have landed.
    asm volatile("s_waitcnt vmcnt(0)" : "+v"(sa), "+v"(sb)::"memory");
  }
  // The last row of tiles; a wave without groups folds zeros.
#pragma unroll
  for (int nt = 0; nt < 4; ++nt)
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[MT - 1][nt][i] = __builtin_fmaf((float)prev[nt][i], prev_sc[nt], acc[MT - 1][nt][i]);

  // Partial tiles of the SW waves into LDS (the stages are free once every
  // wave is here), then wave w finishes its kTokens / SW tokens.
  asm volatile("s_waitcnt vmcnt(0)\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  float* tiles = reinterpret_cast<float*>(&stages[0][0][0]);
  float* own = tiles + wave * T::kTokens * kSplitPitch;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
      for (int i = 0; i < 4; ++i) own[(mt * 16 + 4 * kb + i) * kSplitPitch + nt * 16 + col] = acc[mt][nt][i];
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");

  const bool has_bias = bias != nullptr;
  const int r4 = (lane & 15) * 4;
  const int row = row0 + r4;  // first of the lane's four rows (a multiple of 4)
  float bv[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) bv[k] = (has_bias && row + k < a.rows) ? bias[row + k] : 0.0f;
  const bool rows_whole = row + 3 < a.rows;
  const uintptr_t base_addr = reinterpret_cast<uintptr_t>(output);
  const bool vec4 = (a.out_stride & 3) == 0 && (base_addr & 15) == 0;
  const bool vec2 = (a.out_stride & 1) == 0 && (base_addr & 7) == 0;
  constexpr int kOwn = T::kTokens / SW;  // tokens each wave finishes
#pragma unroll
  for (int j = 0; j < kOwn / 4; ++j) {
    const int tl = wave * kOwn + j * 4 + (lane >> 4);
    const int t = token0 + tl;
    f4v total = *reinterpret_cast<const f4v*>(tiles + tl * kSplitPitch + r4);
#pragma unroll
    for (int w = 1; w < SW; ++w)
      total = total + *reinterpret_cast<const f4v*>(tiles + (w * T::kTokens + tl) * kSplitPitch + r4);
    if (t >= a.m) continue;
    const float sx = scale_in[t];
    float y[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      y[k] = total[k] * sx;
      if (has_bias) y[k] = y[k] + bv[k];
    }
    float* orow = output + (size_t)t * a.out_stride;
    if constexpr (EPI == kSiluPair) {
      const float p0 = ivo_silu(y[0]) * y[1], p1 = ivo_silu(y[2]) * y[3];
      if (rows_whole && vec2) {
        __builtin_nontemporal_store(f2v{p0, p1}, reinterpret_cast<f2v*>(orow + (row >> 1)));
      } else {
        if (row + 1 < a.rows) orow[row >> 1] = p0;
        if (row + 3 < a.rows) orow[(row >> 1) + 1] = p1;
      }
    } else if (rows_whole && vec4) {
      f4v* dst = reinterpret_cast<f4v*>(orow + row);
      if constexpr (EPI == kResidual) {
        const f4v o = *dst;
        __builtin_nontemporal_store(f4v{o.x + y[0], o.y + y[1], o.z + y[2], o.w + y[3]}, dst);
      } else {
        __builtin_nontemporal_store(f4v{y[0], y[1], y[2], y[3]}, dst);
      }
    } else {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        if (row + k < a.rows) {
          if constexpr (EPI == kResidual) orow[row + k] = orow[row + k] + y[k];
          else orow[row + k] = y[k];
        }
      }
    }
  }
}

// Token rows per split-K tile: the largest of 128, 64, 32 whose grid keeps
// three quarters of the CUs busy (else 32).  K=4096 -> N=1024 at M=512: 32
// (256 blocks), 11.4 us against 19.1 us with 128 (64 blocks); K=4096 ->
// N=14336 at M=128: 128 (224 blocks), 20.4 us against 24.5 us with 64.
int split_tokens(int m, int rows) {
  const long long row_tiles = ceil_div(rows, kSplitRows);
  const int busy = device_cus() * 3 / 4;
  for (int tokens : {128, 64}) {
    if (row_tiles * ceil_div(m, tokens) >= busy) return tokens;
  }
  return 32;
}

}  // namespace

// Waves (K-splits) per split-K tile: 8 with 32-token tiles when every wave
// still gets 4 groups (the stages of 8 waves fit in LDS only at 32 tokens),
// else 4.  The count is the order's split count, which ivonar_gemm_plan
// reports.
int split_waves(int m, int rows, int n) {
  return split_tokens(m, rows) == 32 && ceil_div(n, kGroup) >= 32 ? 8 : 4;
}

namespace {

// Three stages per wave where they fit in LDS (32 and 64-token tiles: 150 KB
// with eight waves, 126 KB with four), two at 128 tokens.
template <int EPI, int MT, int SW>
hipError_t launch_split_shape(hipStream_t stream, const GemmArgs& a) {
  constexpr int NS = MT <= 4 ? 3 : 2;
  const dim3 grid(ceil_div(a.rows, kSplitRows), ceil_div(a.m, SplitTile<MT>::kTokens));
  hipLaunchKernelGGL((gemm_split_kernel<EPI, MT, SW, NS>), grid, dim3(64 * SW), 0, stream, a.q8_in, a.scale_in,
                     a.packed, a.scales, a.bias, a.output, a);
  return hipGetLastError();
}

template <int EPI>
hipError_t launch_split_epi(hipStream_t stream, const GemmArgs& a) {
  switch (split_tokens(a.m, a.rows)) {
    case 128: return launch_split_shape<EPI, 8, 4>(stream, a);
    case 64: return launch_split_shape<EPI, 4, 4>(stream, a);
    default:
      if (split_waves(a.m, a.rows, a.n) == 8) return launch_split_shape<EPI, 2, 8>(stream, a);
      return launch_split_shape<EPI, 2, 4>(stream, a);
  }
}

}  // namespace

// Token tile of the long-prompt kernel (0: it does not apply; 32 below 2048
// inputs where 64-token tiles leave CUs idle, see the end).  128 tokens x
// 256 rows from 2048 inputs on, where the loop dominates: it pays from about
// 192 blocks (three quarters of the CUs busy; K=4096 -> N=14336 at M=512, 224
// blocks: 60.8 us against 66.7 us for the 64 x 64-wave-tile kernel).  Below
// 2048 inputs the loads before the first MFMA and the output write dominate
// and 64-token tiles (half the registers, two blocks per CU) pay from 96
// blocks: K=1024 -> N=4096 at M=512 13.1 us against 18.8 us with 128-token
// tiles, at M=2048 20.9 against 21.8 us; with 4096 inputs they lose (68.8
// against 61.0 us at M=2048, N=4096).
int gemm_wide_tokens(int m, int rows, int n) {
  if (m < 128) return 0;
  const long long row_blocks = ceil_div(rows, 256);
  if (ceil_div(n, kGroup) >= 16) {
    const bool fits = WideTile<8, 4>::kLdsBytes <= max_lds_per_block();
    if (fits && row_blocks * ceil_div(m, 128) >= 192) return 128;
    // Too few 128-token tiles: 64-token tiles beat the split-K kernel once
    // they give 192 blocks (K=4096 -> N=14336 at M=256: 32.4 against 35.2 us;
    // K=4096 -> N=4096 at M=1024: 35.1 against 37.4 us).
    const bool fits64 = WideTile<4, 4>::kLdsBytes <= max_lds_per_block();
    return fits64 && row_blocks * ceil_div(m, 64) >= 192 ? 64 : 0;
  }
  const bool fits = WideTile<4, 4>::kLdsBytes <= max_lds_per_block();
  if (!fits || row_blocks * ceil_div(m, 64) < 96) return 0;
  // 32-token tiles where 64-token tiles leave CUs idle (K=1024 -> N=4096 at
  // M=512: 256 blocks, 10.0 us against 12.5 us with 128 blocks of 64 tokens;
  // K=1024 -> N=8192 at M=256: 9.6 against 12.3 us), though each expanded
  // weight fragment then feeds two MFMA rows instead of four.
  return row_blocks * ceil_div(m, 64) < 192 && row_blocks * ceil_div(m, 32) >= 192 ? 32 : 64;
}

hipError_t launch_gemm_wide(hipStream_t stream, const GemmArgs& a) {
  const int tokens = gemm_wide_tokens(a.m, a.rows, a.n);
  if (tokens == 0) return hipErrorInvalidValue;
  switch (a.epi) {
    case kStore: return launch_wide_epi<kStore>(stream, a, tokens);
    case kResidual: return launch_wide_epi<kResidual>(stream, a, tokens);
    case kSiluPair: return launch_wide_epi<kSiluPair>(stream, a, tokens);
    default: return hipErrorInvalidValue;
  }
}

// The split-K tiling for prompts of more than 32 tokens that the 128 x 256
// tiling leaves with too few blocks: at least 32 tiles of 128 tokens x 64
// rows and at least 4 groups per wave (a partial token tile reads zeros).
// Measured: K=4096 -> N=1024 at M=2048 25.0 us and K=4096 -> N=14336 at
// M=128 22.0 us, against 45.4 and 42.6 us for the 64 x 64-wave-tile kernel.
bool gemm_split_applies(int m, int rows, int n) {
  const long long tiles = (long long)ceil_div(rows, kSplitRows) * ceil_div(m, 128);
  return m > 32 && gemm_wide_tokens(m, rows, n) == 0 && tiles >= 32 && ceil_div(n, kGroup) >= 16;
}

hipError_t launch_gemm_split(hipStream_t stream, const GemmArgs& a) {
  switch (a.epi) {
    case kStore: return launch_split_epi<kStore>(stream, a);
    case kResidual: return launch_split_epi<kResidual>(stream, a);
    case kSiluPair: return launch_split_epi<kSiluPair>(stream, a);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace ivo
