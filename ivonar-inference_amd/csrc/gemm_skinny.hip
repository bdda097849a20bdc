// Skinny token GEMM on int8 MFMA for a few tokens (M <= 32): the decode and
// short-prefill shapes, where a tile of 64+ tokens would idle most of the
// MFMA work and leave most CUs without a block.
//
// A wave owns R tiles of 16 weight rows (16R rows) and 16*MT tokens; the S
// waves of a block share those rows and walk the contiguous group ranges
// [s*GS, min((s+1)*GS, G)), GS = ceil(G/S).  Per 128-input group a lane
// (c = lane % 16, kb = lane / 16) loads, for each row tile, the 8 packed
// bytes of words 2kb, 2kb+1 of its row c and expands them to signed int8
// codes (one v_perm_b32 table lookup per 4 codes): the B operands of two
// v_mfma_i32_16x16x64_i8.  The A operands are the q8 bytes of the same words
// for token c of each 16-token tile, read straight from global memory (32
// contiguous bytes per lane and group) and used by all R row tiles: the
// token operand is re-read from the caches once per 16R rows, which is what
// bounds this kernel when R = 1 (at 32 tokens the token bytes read per group
// are 8x the weight bytes).  All loads are unconditional, with addresses
// clamped into the operands, and go out one stage of groups ahead, double
// buffered; the second chunk of the last group of an odd chunk count is
// masked to zero on the A side (its weight bytes may then be anything).
//
// fp32 order (restated by the CPU oracle as orc_gemm_split): each wave folds
// its groups' exact int32 tiles into fp32 with one fmaf per output in
// ascending group order; the S partial tiles go through LDS and are added in
// wave order, then the token scale and the bias are applied.  The whole block
// shares that epilogue: thread i finishes outputs i, i + 64S, ... of the tile
// (rows fastest), so the stores are contiguous runs of 16R floats.
#include <type_traits>

#include "buffer_ops.hpp"
#include "internal.hpp"
#include "ternary_device.hpp"

namespace ivo {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

template <int MT, int R>
struct SkinnyStage {
  static constexpr int kGroups = (MT == 1 && R <= 2) ? 4 : 2;  // groups per stage (register budget)
  uint2 w[kGroups][R];
  uint16_t s[kGroups][R];
  v4i a[kGroups][MT][2];
};

// Partial tiles in LDS: [wave][token][row], row pitch 16R + 4 floats (the
// four kb lane groups of a fold land on distinct banks).
template <int MT, int R>
struct SkinnyRed {
  static constexpr int kPitch = 16 * R + 4;
  static constexpr int kWaveFloats = 16 * MT * kPitch;
};

template <int EPI, int MT, int R, int S>
__global__ __launch_bounds__(64 * S) void skinny_kernel(const int8_t* __restrict__ q8,
                                                        const float* __restrict__ scale_in,
                                                        const uint8_t* __restrict__ packed,
                                                        const uint16_t* __restrict__ scales,
                                                        const float* __restrict__ bias,
                                                        float* __restrict__ output, GemmArgs a) {
  using Stage = SkinnyStage<MT, R>;
  using Red = SkinnyRed<MT, R>;
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
  const int row0 = blockIdx.x * 16 * R;
  const int per_wave = (groups + S - 1) / S;
  const int g_begin = min(s * per_wave, groups);
  const int g_end = min(g_begin + per_wave, groups);
  const uint8_t* wrow[R];
  const uint16_t* srow[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int row = min(row0 + r * 16 + col, a.rows - 1);
    wrow[r] = packed + (size_t)row * a.row_bytes;
    srow[r] = scales + (size_t)row * a.groups;
  }
  const size_t q8_stride = (size_t)chunks * kChunk;
  const int8_t* arow[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) arow[mt] = q8 + (size_t)min(mt * 16 + col, a.m - 1) * q8_stride;

  auto load_stage = [&](Stage& st, int first) {
#pragma unroll
    for (int j = 0; j < kStage; ++j) {
      const int g = min(first + j, groups - 1);
      const bool dead = g == short_group && kb >= 2;  // read the group's first chunk instead
      const size_t offset = (size_t)g * kGroup + (dead ? 0 : kb * 32);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        st.a[j][mt][0] = *reinterpret_cast<const v4i*>(arow[mt] + offset);
        st.a[j][mt][1] = *reinterpret_cast<const v4i*>(arow[mt] + offset + 16);
      }
#pragma unroll
      for (int r = 0; r < R; ++r) {
        st.w[j][r] = *reinterpret_cast<const uint2*>(wrow[r] + (size_t)g * 32 + (dead ? 0 : kb * 8));
        st.s[j][r] = srow[r][g];
      }
    }
  };

  float acc[MT][R][4];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[mt][r][i] = 0.0f;

  auto compute_stage = [&](const Stage& st, int first) {
#pragma unroll
    for (int j = 0; j < kStage; ++j) {
      const int g = first + j;
      if (g >= g_end) break;  // wave-uniform
      const int keep = (g == short_group && kb >= 2) ? 0 : -1;
      v4i a0[MT], a1[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        a0[mt] = st.a[j][mt][0];
        a1[mt] = st.a[j][mt][1];
        if (g == short_group) {  // wave-uniform
          a0[mt] &= keep;
          a1[mt] &= keep;
        }
      }
#pragma unroll
      for (int r = 0; r < R; ++r) {
        v4i b0, b1;
        b0.x = (int)signed_codes(st.w[j][r].x, 0);
        b0.y = (int)signed_codes(st.w[j][r].x, 1);
        b0.z = (int)signed_codes(st.w[j][r].x, 2);
        b0.w = (int)signed_codes(st.w[j][r].x, 3);
        b1.x = (int)signed_codes(st.w[j][r].y, 0);
        b1.y = (int)signed_codes(st.w[j][r].y, 1);
        b1.z = (int)signed_codes(st.w[j][r].y, 2);
        b1.w = (int)signed_codes(st.w[j][r].y, 3);
        const float scale = h2f(st.s[j][r]);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const v4i zero = {0, 0, 0, 0};
          v4i p = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0[mt], b0, zero, 0, 0, 0);
          p = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1[mt], b1, p, 0, 0, 0);
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[mt][r][i] = __builtin_fmaf((float)p[i], scale, acc[mt][r][i]);
        }
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

  // Partial tiles to LDS: lane (col, kb) holds token mt*16 + 4kb + i of row r*16 + col.
  float* red = reinterpret_cast<float*>(smem);
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        red[s * Red::kWaveFloats + (mt * 16 + 4 * kb + i) * Red::kPitch + r * 16 + col] = acc[mt][r][i];
  __syncthreads();

  // Epilogue: output o of the tile is token o / 16R, row o % 16R; wave partials added in order.
  constexpr int kOutputs = 16 * MT * 16 * R;
  constexpr int kPerThread = (kOutputs + 64 * S - 1) / (64 * S);
#pragma unroll
  for (int j = 0; j < kPerThread; ++j) {
    const int o = tid + j * 64 * S;
    if (kOutputs % (64 * S) != 0 && o >= kOutputs) break;  // whole waves (16R is a multiple of 16)
    const int t = o / (16 * R), rr = o % (16 * R);
    const int out_row = row0 + rr;
    float total = red[t * Red::kPitch + rr];
#pragma unroll
    for (int w = 1; w < S; ++w) total = total + red[w * Red::kWaveFloats + t * Red::kPitch + rr];
    const bool row_live = out_row < a.rows;
    const bool live = row_live && t < a.m;
    float y = total * scale_in[min(t, a.m - 1)];
    if (bias != nullptr) y = y + bias[min(out_row, a.rows - 1)];
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

// f(integral_constant<int, 0>) ... f(integral_constant<int, N - 1>): an unrolled loop whose index
// can feed an immediate operand.
template <int N, int I = 0, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<N, I + 1>(f);
  }
}

// Token operand staged in LDS (prompts whose token bytes for a wave's groups
// fit: 16*MT tokens x 128 bytes per group).  A block is S waves over the same
// 16R rows (R row tiles per wave), wave s owning the group range
// [s*GS, min((s+1)*GS, G)) (the same fp32 order as above).  Each wave sends to
// its own LDS region the token bytes of its groups (direct buffer-to-LDS
// loads, 16 bytes per lane, XOR-swizzled pieces) and the fp16 scales of the
// block's rows from its first group on, and loads the packed bytes of its
// groups into registers, group by group, so that group j's loads are complete
// once no more than (NG-1-j) groups' loads are outstanding (vector loads,
// direct-to-LDS ones included, retire in issue order on the counter): step j
// waits for that count and then a barrier.  The counter is what the ISA
// documents; the barrier is a measured guard (on MI355X a wave that read its
// own direct-to-LDS bytes right after the counter reached them sometimes read
// the half of the 64 lanes that was still being written, and with the barrier
// it never did).  The token fragments of a group feed all R row tiles.  Prompts
// of more than 32 tokens run as slices of 32 tokens (grid dimension y).  Tokens
// past the slice and the missing second chunk of an odd chunk count read as
// zeros through the buffer range check; rows past the matrix are clamped and
// not stored.
template <int MT, int R, int S, int NG>
struct RowTile {
  static constexpr int kTokens = 16 * MT;
  static constexpr int kGroupBytes = kTokens * kGroup;  // token bytes of one group
  static constexpr int kWaveA = NG * kGroupBytes;
  static constexpr int kWaveScales = 2048;              // 64 lanes x two 16-byte pieces
  static constexpr int kWaveBytes = kWaveA + kWaveScales;
  static constexpr int kLoadsPerGroup = 2 * MT + R;      // DMA pieces + weight loads
  static constexpr int kPitch = 16 * R + 4;             // partial tile row pitch (floats)
  static constexpr int kRedBytes = S * kTokens * kPitch * 4;
  static constexpr int kLdsBytes = S * kWaveBytes > kRedBytes ? S * kWaveBytes : kRedBytes;
  static_assert(2 + NG * kLoadsPerGroup <= 63, "loads in flight fit the vmcnt counter");
  static_assert(16 * R <= 64 && NG <= 8, "one scale piece pair per row, eight groups per wave");
};

template <int EPI, int MT, int R, int S, int NG>
__global__ __launch_bounds__(64 * S) void skinny_row_kernel(const int8_t* __restrict__ q8,
                                                            const float* __restrict__ scale_in,
                                                            const uint8_t* __restrict__ packed,
                                                            const uint16_t* __restrict__ scales,
                                                            const float* __restrict__ bias,
                                                            float* __restrict__ output, GemmArgs a) {
  using T = RowTile<MT, R, S, NG>;
  __shared__ __align__(16) unsigned char smem[T::kLdsBytes];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int s = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 15, kb = lane >> 4;
  const int chunks = (a.n + kChunk - 1) / kChunk;
  const int groups = (a.n + kGroup - 1) / kGroup;
  const int short_group = (chunks & 1) ? groups - 1 : groups;
  const int q8_stride = chunks * kChunk;
  // Token slice blockIdx.y: tokens [16*MT*y, 16*MT*y + m) of the prompt.
  const int token0 = blockIdx.y * T::kTokens;
  const int m = min(a.m - token0, T::kTokens);
  q8 += (size_t)token0 * q8_stride;
  scale_in += token0;
  output += (size_t)token0 * a.out_stride;
  const int per_wave = (groups + S - 1) / S;
  const int g0 = min(s * per_wave, groups);
  const int count = min(per_wave, groups - g0);
  const int row0 = blockIdx.x * 16 * R;
  unsigned char* wave_a = smem + s * T::kWaveBytes;
  unsigned char* wave_scales = wave_a + T::kWaveA;
  const unsigned a_lds = lds_address(wave_a);
  const unsigned s_lds = lds_address(wave_scales);
  constexpr int kPast = 0x7FFFFFF0;
  const v4u q8_buf = wide_buffer(q8, (long long)m * q8_stride);
  const v4u w_buf = wide_buffer(packed, (long long)a.rows * a.row_bytes);
  const v4u s_buf = wide_buffer(scales, (long long)a.rows * a.groups * 2);

  // What the epilogue reads from global memory (token scales, biases, residual
  // bases of this thread's outputs) goes out first: older than every
  // hand-counted load below, so those waits stay exact, and the epilogue is
  // not followed by a load round trip of its own.  Output o of the tile is
  // token o / 16R, row o % 16R.
  constexpr int kOutputs = T::kTokens * 16 * R;  // a multiple of 64: whole waves stay active together
  constexpr int kEpi = (kOutputs + 64 * S - 1) / (64 * S);
  float epi_sx[kEpi], epi_bias[kEpi], epi_base[kEpi];
#pragma unroll
  for (int jo = 0; jo < kEpi; ++jo) {
    const int o = min(tid + jo * 64 * S, kOutputs - 1);
    const int t = min(o / (16 * R), m - 1), row = min(row0 + o % (16 * R), a.rows - 1);
    epi_sx[jo] = scale_in[t];
    // Without a bias the load reads a token scale instead (no branch before the loads below).
    const float b = *(bias != nullptr ? bias + row : scale_in);
    epi_bias[jo] = bias != nullptr ? b : 0.0f;
    epi_base[jo] = EPI == kResidual ? output[(size_t)t * a.out_stride + row] : 0.0f;
  }

  // Scales: lane l < 16R fetches row row0 + l from group g0 on, 32 bytes from the dword below.
  const int scale_byte = ((row0 + lane) * a.groups + g0) * 2;
  const int scale_shift = scale_byte & 3;
  const bool scale_lane = lane < 16 * R && row0 + lane < a.rows;
  dma16(s_buf, s_lds, scale_lane ? scale_byte - scale_shift : kPast, 0);
  dma16(s_buf, s_lds + 1024, scale_lane ? scale_byte - scale_shift + 16 : kPast, 0);

  // Group by group: the token pieces (2MT instructions of 8 tokens), then the R weight loads.
  uint2 wq[NG][R];
#pragma unroll
  for (int j = 0; j < NG; ++j) {
    const int g = min(g0 + j, groups - 1);
#pragma unroll
    for (int q = 0; q < 2 * MT; ++q) {
      const int slot = q * 64 + lane;
      const int t = slot >> 3;
      const int piece = (slot & 7) ^ a_swizzle(t);
      const bool dead = (g == short_group && piece >= 4) || q * 8 >= m;
      dma16(q8_buf, a_lds + j * T::kGroupBytes + q * 1024, dead ? kPast : t * q8_stride + g * kGroup + piece * 16, 0);
    }
    const bool wdead = g == short_group && kb >= 2;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int row = min(row0 + r * 16 + col, a.rows - 1);
      wq[j][r] = load_b64(w_buf, row * a.row_bytes + g * 32 + (wdead ? 0 : kb * 8), 0);
    }
  }

  float acc[MT][R][4];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[mt][r][i] = 0.0f;
  static_for<NG>([&](auto jc) {
    constexpr int j = decltype(jc)::value;
    // The reads of a direct-to-LDS load's bytes follow direct_load_sync's sequence (the counter
    // here leaves the later groups' loads in flight; every wave passes all NG barriers).
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier" ::"n"((NG - 1 - j) * T::kLoadsPerGroup)
                 : "memory");
    if (j >= count) return;  // wave-uniform
#pragma unroll
    for (int r = 0; r < R; ++r) asm volatile("" : "+v"(wq[j][r]));
    const v4i* tile = reinterpret_cast<const v4i*>(wave_a + j * T::kGroupBytes);
    v4i a0[MT], a1[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int t = mt * 16 + col;
      a0[mt] = tile[t * 8 + ((2 * kb) ^ a_swizzle(t))];
      a1[mt] = tile[t * 8 + ((2 * kb + 1) ^ a_swizzle(t))];
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      v4i b0, b1;
      b0.x = (int)signed_codes(wq[j][r].x, 0);
      b0.y = (int)signed_codes(wq[j][r].x, 1);
      b0.z = (int)signed_codes(wq[j][r].x, 2);
      b0.w = (int)signed_codes(wq[j][r].x, 3);
      b1.x = (int)signed_codes(wq[j][r].y, 0);
      b1.y = (int)signed_codes(wq[j][r].y, 1);
      b1.z = (int)signed_codes(wq[j][r].y, 2);
      b1.w = (int)signed_codes(wq[j][r].y, 3);
      // Scale of row r*16 + col, group g0 + j: byte scale_shift + 2j of that row's 32-byte window.
      const int srow = r * 16 + col;
      const int o = __shfl(scale_shift, srow) + 2 * j;
      const float scale = h2f(*reinterpret_cast<const uint16_t*>(wave_scales + (o < 16 ? 0 : 1024 - 16) + srow * 16 + o));
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const v4i zero = {0, 0, 0, 0};
        v4i p = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0[mt], b0, zero, 0, 0, 0);
        p = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1[mt], b1, p, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[mt][r][i] = __builtin_fmaf((float)p[i], scale, acc[mt][r][i]);
      }
    }
  });
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the slots past count

  // Partial tiles [s][token][row] over the token regions (every wave is done with them), then
  // the block's epilogue: output o is token o / 16R, row o % 16R; the S partials added in order.
  __syncthreads();
  float* red = reinterpret_cast<float*>(smem);
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        red[(s * T::kTokens + mt * 16 + 4 * kb + i) * T::kPitch + r * 16 + col] = acc[mt][r][i];
  __syncthreads();
#pragma unroll
  for (int jo = 0; jo < kEpi; ++jo) {
    const int o = tid + jo * 64 * S;
    if (kOutputs % (64 * S) != 0 && o >= kOutputs) break;
    const int t = o / (16 * R), rr = o % (16 * R);
    const int out_row = row0 + rr;
    float total = red[t * T::kPitch + rr];
#pragma unroll
    for (int k = 1; k < S; ++k) total = total + red[(k * T::kTokens + t) * T::kPitch + rr];
    const bool row_live = out_row < a.rows;
    const bool live = row_live && t < m;
    float y = total * epi_sx[jo];
    if (bias != nullptr) y = y + epi_bias[jo];
    float* orow = output + (size_t)min(t, m - 1) * a.out_stride;
    if constexpr (EPI == kSiluPair) {
      const float partner = __shfl_xor(y, 1);
      if (live && (out_row & 1) == 0 && out_row + 1 < a.rows) orow[out_row >> 1] = ivo_silu(y) * partner;
    } else if constexpr (EPI == kResidual) {
      if (live) orow[out_row] = epi_base[jo] + y;
    } else {
      if (live) orow[out_row] = y;
    }
  }
}

template <int EPI, int MT, int R, int S, int NG>
hipError_t launch_skinny_row_shape(hipStream_t stream, const GemmArgs& a) {
  hipLaunchKernelGGL((skinny_row_kernel<EPI, MT, R, S, NG>), dim3(ceil_div(a.rows, 16 * R), ceil_div(a.m, 16 * MT)),
                     dim3(64 * S), 0, stream,
                     a.q8_in, a.scale_in, a.packed, a.scales, a.bias, a.output, a);
  return hipGetLastError();
}

template <int MT, int R>
constexpr size_t skinny_lds(int splits) {
  return (size_t)splits * SkinnyRed<MT, R>::kWaveFloats * sizeof(float);
}

template <int EPI, int MT, int R, int S>
hipError_t launch_skinny_shape(hipStream_t stream, const GemmArgs& a) {
  const size_t lds = skinny_lds<MT, R>(S);
  hipLaunchKernelGGL((skinny_kernel<EPI, MT, R, S>), dim3(ceil_div(a.rows, 16 * R)), dim3(64 * S), lds, stream,
                     a.q8_in, a.scale_in, a.packed, a.scales, a.bias, a.output, a);
  return hipGetLastError();
}

template <int EPI, int MT, int R>
hipError_t launch_skinny_r(hipStream_t stream, const GemmArgs& a, int splits) {
  switch (splits) {
    case 1: return launch_skinny_shape<EPI, MT, R, 1>(stream, a);
    case 2: return launch_skinny_shape<EPI, MT, R, 2>(stream, a);
    case 4: return launch_skinny_shape<EPI, MT, R, 4>(stream, a);
    default: return hipErrorInvalidValue;
  }
}

// Shapes of the LDS-staged kernel that the plan can pick: (S, NG) with R = 1;
// R = 2 (16 tokens) or 4 (32 tokens) with S = 8.
template <int EPI, int MT, int R>
hipError_t launch_skinny_row_r(hipStream_t stream, const GemmArgs& a, int splits, int ng) {
  const int key = splits * 16 + ng;
  if constexpr (R > 1) {
    switch (key) {
      case 8 * 16 + 1: return launch_skinny_row_shape<EPI, MT, R, 8, 1>(stream, a);
      case 8 * 16 + 2: return launch_skinny_row_shape<EPI, MT, R, 8, 2>(stream, a);
      case 8 * 16 + 4: return launch_skinny_row_shape<EPI, MT, R, 8, 4>(stream, a);
      case 8 * 16 + 8:
        if constexpr (MT == 1) return launch_skinny_row_shape<EPI, MT, R, 8, 8>(stream, a);
        return hipErrorInvalidValue;
      default: return hipErrorInvalidValue;
    }
  } else {
    switch (key) {
      case 1 * 16 + 1: return launch_skinny_row_shape<EPI, MT, 1, 1, 1>(stream, a);
      case 2 * 16 + 1: return launch_skinny_row_shape<EPI, MT, 1, 2, 1>(stream, a);
      case 2 * 16 + 2: return launch_skinny_row_shape<EPI, MT, 1, 2, 2>(stream, a);
      case 4 * 16 + 1: return launch_skinny_row_shape<EPI, MT, 1, 4, 1>(stream, a);
      case 4 * 16 + 2: return launch_skinny_row_shape<EPI, MT, 1, 4, 2>(stream, a);
      case 8 * 16 + 1: return launch_skinny_row_shape<EPI, MT, 1, 8, 1>(stream, a);
      case 8 * 16 + 2: return launch_skinny_row_shape<EPI, MT, 1, 8, 2>(stream, a);
      case 8 * 16 + 4: return launch_skinny_row_shape<EPI, MT, 1, 8, 4>(stream, a);
      case 8 * 16 + 8:
        if constexpr (MT == 1) return launch_skinny_row_shape<EPI, MT, 1, 8, 8>(stream, a);
        return hipErrorInvalidValue;  // 272 KB of LDS
      default: return hipErrorInvalidValue;
    }
  }
}

template <int EPI, int MT>
hipError_t launch_skinny_mt(hipStream_t stream, const GemmArgs& a, SkinnyPlan plan) {
  if (plan.lds_groups > 0) {
    if (plan.row_tiles == 1) return launch_skinny_row_r<EPI, MT, 1>(stream, a, plan.splits, plan.lds_groups);
    if (plan.row_tiles == (MT == 1 ? 2 : 4))
      return launch_skinny_row_r<EPI, MT, MT == 1 ? 2 : 4>(stream, a, plan.splits, plan.lds_groups);
    return hipErrorInvalidValue;
  }
  switch (plan.row_tiles) {
    case 1: return launch_skinny_r<EPI, MT, 1>(stream, a, plan.splits);
    case 2: return launch_skinny_r<EPI, MT, 2>(stream, a, plan.splits);
    default: return hipErrorInvalidValue;
  }
}

template <int EPI>
hipError_t launch_skinny_epi(hipStream_t stream, const GemmArgs& a, SkinnyPlan plan) {
  return a.m <= 16 ? launch_skinny_mt<EPI, 1>(stream, a, plan) : launch_skinny_mt<EPI, 2>(stream, a, plan);
}

// LDS of the LDS-staged kernel (per wave: the token bytes of NG groups and two
// 1 KB scale pieces), or of the cache-read kernel's partial tiles.
size_t skinny_lds_bytes(int m, SkinnyPlan plan) {
  const size_t mt = m <= 16 ? 1 : 2;
  if (plan.lds_groups > 0) return (size_t)plan.splits * (plan.lds_groups * 16 * mt * kGroup + 2048);
  return (size_t)plan.splits * 16 * mt * (16 * plan.row_tiles + 4) * sizeof(float);
}

}  // namespace

// Prompts of 33..kSlicedTokens tokens that neither long-prompt tiling takes run
// the LDS-staged kernel in 32-token slices when it fits.
// The LDS-staged kernel whenever a wave's share fits (up to 64 groups, i.e.
// K <= 8192): 8 K-splits from 8 groups on, 4 from 4, 2 from 2; from 768 row
// tiles on, two row tiles per wave for up to 16 tokens and four above (fewer
// blocks, each token fragment read once for more rows), one below.  Otherwise
// the token operand is read from the caches per wave: four K-splits, two row
// tiles per wave for 8192 rows and more (fewer re-reads of the token
// operand), one below (measured at K=28672 -> N=8192, 1 token: 31 us against
// 56 us with four row tiles and two K-splits).
SkinnyPlan skinny_plan(int m, int rows, int n, size_t max_lds) {
  if (m < 1 || m > kSlicedTokens) return {0, 0, 0};
  const int groups = ceil_div(n, kGroup);
  const int tiles = ceil_div(rows, 16);
  const int mt = m <= 16 ? 1 : 2;
  SkinnyPlan plan{groups >= 8 ? 8 : groups >= 4 ? 4 : groups >= 2 ? 2 : 1, 1, 0};
  const int per_wave = ceil_div(groups, plan.splits);
  int ng = 1;
  while (ng < per_wave) ng *= 2;
  plan.lds_groups = ng;
  if (plan.splits == 8 && tiles >= 768 && (mt == 1 || ng <= 4)) plan.row_tiles = mt == 1 ? 2 : 4;
  // Its buffer offsets are 32-bit.
  const long long row_bytes = (ceil_div(n, 4) + 15) / 16 * 16;
  const bool small = (long long)rows * row_bytes < (1LL << 31) && (long long)rows * groups * 2 < (1LL << 31);
  if (ng <= 8 && small && skinny_lds_bytes(m, plan) <= max_lds) return plan;
  if (m > 32) return {0, 0, 0};
  return {groups >= 4 ? 4 : groups >= 2 ? 2 : 1, rows >= 8192 ? 2 : 1, 0};
}

hipError_t launch_skinny(hipStream_t stream, const GemmArgs& a, SkinnyPlan plan) {
  if (plan.splits < 1 || skinny_lds_bytes(a.m, plan) > (size_t)max_lds_per_block()) return hipErrorInvalidValue;
  if (plan.lds_groups > 0 &&
      ((long long)a.rows * a.row_bytes >= (1LL << 31) || (long long)a.rows * a.groups * 2 >= (1LL << 31)))
    return hipErrorInvalidValue;
  switch (a.epi) {
    case kStore: return launch_skinny_epi<kStore>(stream, a, plan);
    case kResidual: return launch_skinny_epi<kResidual>(stream, a, plan);
    case kSiluPair: return launch_skinny_epi<kSiluPair>(stream, a, plan);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace ivo
