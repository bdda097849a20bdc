// Token GEMV: M = 1..16 tokens against one packed matrix, each weight byte
// streamed once for all tokens, on v_mfma_i32_16x16x64_i8 (the gemm_tile_*
// entry points with m <= 16; reference: kernels/ternary.cu:688-765, the
// 32-token tile it replaces for short prompts and decode batches).
//
// Work split.  A wave owns one tile of 16 weight rows and the contiguous span
// range [p*PART, (p+1)*PART) of its row, a span being 64 packed bytes (two
// 128-input groups).  The PARTS waves of a row tile sit in one block, with up
// to 16/PARTS tiles per block.  Per span a lane (c = lane % 16, kb = lane / 16)
// loads the 16 bytes [64s + 16kb, +16) of row c: one wave instruction reads
// 16 rows x 64 contiguous bytes.  Two v_permlane32_swap exchanges give every
// lane 8 bytes of the span's first group (group bytes 0-7, 16-23, 8-15, 24-31
// for kb = 0..3) and 8 of its second, so that one MFMA's 64-input sum never
// mixes groups.  The 2-bit fields of those 8 bytes, shifted to bit 0 and
// masked (codes 0..2 as int8), are the B operands of two chained MFMAs per
// group; the A operands are the q8 bytes of the same inputs for token c (the
// token slots past M read token M-1 and are not stored).  The chain starts
// from minus the group's q sum of the lane's four output tokens, so the int32
// result is the exact group partial sum((code - 1) * q) for tokens 4kb..4kb+3
// of row c.
//
// Activations.  The block copies the whole q8 rows of the M tokens (the
// quantizer's layout, 8-byte pieces gathered into MFMA operand order) and the
// group q sums into LDS once, after its waves have issued their first weight
// loads; all waves then read their operands from LDS.  Weights stream through
// a register ring UW spans deep (kRing); all scales of the wave's range are
// loaded up front.  What the block's epilogue reads from global memory (token
// scales, biases, residual bases) is loaded before the block barrier, so the
// last step is not followed by a load round trip (K=8192 -> N=28672, 8
// rotating copies: M=2 18.0 -> 17.4 us, M=4 19.4-19.9 -> 17.7, M=16 20.9-21.4
// -> 20.0).  (Staging the block's scales in LDS instead, one 16-byte piece
// per thread, saved another 0.3-0.5 us at M=2..4 but pushed M=16 over the
// LDS budget into two K slices, 1.6 us slower; not kept.)
//
// Long rows.  Where the tokens' whole q8 rows do not fit in LDS, K is cut
// into `slices` equal span ranges, one per block row of the grid (grid y):
// a block then copies and reads only its slice's q8 bytes and q sums, and
// its waves write their fp32 chains to the scratch ([slice * parts + part]
// [token][row]) instead of adding them; the last of a tile group's slices to
// arrive adds them (token_finish_kernel, in a launch of its own, where the
// tile groups outnumber the scratch's counters).
//
// fp32 order (the CPU oracle's orc_gemm_split with S = PARTS * slices): each
// wave folds its groups' partials into one fmaf chain per output in ascending
// group order; the S chains of an output are added in wave order (slice
// first, then the part within it), then the token scale, the bias and the
// epilogue follow.
#include <type_traits>

#include "internal.hpp"
#include "ternary_device.hpp"

namespace ivo {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef unsigned v4u __attribute__((ext_vector_type(4)));

constexpr int kMaxTokens = 16;
constexpr int kMaxWaves = 16;
// Spans of weights in flight per wave.  Deeper rings only queue loads the
// CU cannot take yet (the wave then stalls at issue): 1..16 tokens over
// K=8192 -> N=28672 and K=28672 -> N=8192 take 3-6% longer with 8 spans than
// with 4, and 10-20% longer with 16; 2, 3, 5 and 6 are within 2% of 4.
constexpr int kRing = 4;
constexpr int kSeedsPerThread = 4;  // group q sums each thread copies
constexpr int kSpanBytes = 64;
constexpr int kMaxSlices = 16;
constexpr int kSlicePartials = 100;  // EPI of a sliced launch: wave chains to the scratch

struct TokenShape {
  int rows, n, row_bytes, groups, m, parts, tiles_per_block, out_stride;
  int slice_groups;  // groups per K slice (= groups when the grid has one slice)
  // K-sliced launches: the epilogue the last slice of a tile group applies
  // after adding the chains itself (kStore, kResidual, kSiluPair), with one
  // arrival counter per tile group in `counters`; -1: token_finish_kernel
  // adds them in a launch of its own.
  int finish_epi;
  unsigned* counters;
};

// 2-bit field f of each byte of w, as an int8 code 0..2.
template <int F>
__device__ __forceinline__ int field(unsigned w) {
  return (int)((w >> (2 * F)) & kLow2);
}

template <int EPI, int PART, int FILL>
__global__ __launch_bounds__(64 * kMaxWaves) void token_gemv_kernel(const int8_t* __restrict__ q8,
                                                                     const int32_t* __restrict__ xsum,
                                                                     const float* __restrict__ scale_in,
                                                                     const uint8_t* __restrict__ packed,
                                                                     const uint16_t* __restrict__ scales,
                                                                     const float* __restrict__ bias,
                                                                     float* __restrict__ output,
                                                                     float* __restrict__ chains, TokenShape sh) {
  constexpr int UW = PART < kRing ? PART : kRing;
  extern __shared__ __align__(16) unsigned char lds[];
  const int tid = threadIdx.x;
  const int nthr = blockDim.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int c = lane & 15, kb = lane >> 4;
  const int m = sh.m;
  const int tile = blockIdx.x * sh.tiles_per_block + wave / sh.parts;
  const int part = wave % sh.parts;
  const int span0 = part * PART;  // within the slice
  const int chunks = sh.n / kChunk;
  const int sg = sh.slice_groups;
  const int g_first = blockIdx.y * sg;  // the slice's first group
  // LDS: A operands [group][o][kb][m][16 B] of the slice's groups, then their
  // negated q sums [group][4*sq] (tokens 4*sq and up zero), then (one slice
  // only) the wave partials [wave][16 tokens][16 rows], then a 16-byte dump
  // slot for fill pieces past the end.
  const int abytes = sg * 128 * m;
  const int sq = (m + 3) >> 2;
  const int seeds = sg * 4 * sq;
  int* lseed = reinterpret_cast<int*>(lds + abytes);
  float* partial = reinterpret_cast<float*>(lds + abytes + 4 * seeds);
  unsigned char* dump = lds + abytes + 4 * seeds + (EPI == kSlicePartials ? 0 : nthr / 64 * 1024);

  // Token operand first (it is waited for before the weights), then the group
  // q sums, the scales and the first UW spans of weights.  Fill item p is q8
  // quad p of the block's tokens (token p / (8G), 16 contiguous bytes: the four
  // fields of one packed word W of a group); its fields (0, 1) and (2, 3) are
  // the halves W & 1 of the operands o = 0, 1 of lane group kb = 0, 0, 2, 2,
  // 1, 1, 3, 3 (W = 0..7).
  // A token's q8 row is chunks * 64 bytes (K is a multiple of 256 here); the
  // scale rows may be longer (sh.groups >= K / 128) and only set their stride.
  const int quads = abytes / 16;  // m * 8 * sg
  const int row_quads = chunks * 4;
  v4u fill[FILL];
#pragma unroll
  for (int j = 0; j < FILL; ++j) {
    const int p = min(j * nthr + tid, quads - 1);
    const int t = p / (8 * sg), quad = p - t * (8 * sg);
    fill[j] = *reinterpret_cast<const v4u*>(q8 + ((size_t)t * row_quads + 8 * g_first + quad) * 16);
  }
  int seed_value[kSeedsPerThread];
#pragma unroll
  for (int j = 0; j < kSeedsPerThread; ++j) {
    const int p = min(j * nthr + tid, seeds - 1);
    const int g = p / (4 * sq), t = p % (4 * sq);
    const int2 xs = *reinterpret_cast<const int2*>(xsum + (size_t)min(t, m - 1) * chunks + 2 * (g_first + g));
    seed_value[j] = t < m ? -(xs.x + xs.y) : 0;
  }
  const int row = min(tile * 16 + c, sh.rows - 1);
  const uint8_t* wrow = packed + (size_t)row * sh.row_bytes + (size_t)(g_first / 2 + span0) * kSpanBytes + kb * 16;
  const uint16_t* srow = scales + (size_t)row * sh.groups + g_first + span0 * 2;
  unsigned sc[PART];  // the two fp16 group scales of each span
  if ((sh.groups & 1) == 0) {
    // Even scale rows: every span's scale pair sits at a multiple of 4 bytes.
#pragma unroll
    for (int i = 0; i < PART; i += 2) {
      if (i + 1 < PART) {
        const uint2 v = *reinterpret_cast<const uint2*>(srow + 2 * i);
        sc[i] = v.x;
        sc[i + 1] = v.y;
      } else {
        sc[i] = *reinterpret_cast<const unsigned*>(srow + 2 * i);
      }
    }
  } else {
    // Odd scale rows (padded past K / 128 groups): 2-byte aligned, one fp16 per load.
#pragma unroll
    for (int i = 0; i < PART; ++i) sc[i] = (unsigned)srow[2 * i] | ((unsigned)srow[2 * i + 1] << 16);
  }
  v4u w[UW];
#pragma unroll
  for (int i = 0; i < UW; ++i) w[i] = *reinterpret_cast<const v4u*>(wrow + i * kSpanBytes);

#pragma unroll
  for (int j = 0; j < FILL; ++j) {
    const int p = j * nthr + tid;
    const int t = p / (8 * sg), quad = p % (8 * sg);
    const int g = quad >> 3, word = quad & 7;
    const int k = (0x33112200 >> (4 * word)) & 15;  // lane group of packed word `word`
    unsigned char* piece = lds + (((g * 2) * 4 + k) * m + t) * 16 + 8 * (word & 1);
    const bool live = p < quads;
    *reinterpret_cast<uint2*>(live ? piece : dump) = uint2{fill[j][0], fill[j][1]};
    *reinterpret_cast<uint2*>(live ? piece + 64 * m : dump) = uint2{fill[j][2], fill[j][3]};
  }
#pragma unroll
  for (int j = 0; j < kSeedsPerThread; ++j) {
    const int p = j * nthr + tid;
    *(p < seeds ? lseed + p : reinterpret_cast<int*>(dump)) = seed_value[j];
  }
  // What the epilogue reads from global memory (token scales, biases, the
  // residual base), loaded now (after the fill registers are free) so that
  // the block's last step is not followed by a load round trip: output
  // o = tid + j * nthr of the block (at most kEpiOutputs per thread).
  const int tiles = sh.tiles_per_block;
  constexpr int kEpiOutputs = 4;
  float epi_sx[kEpiOutputs], epi_b0[kEpiOutputs], epi_b1[kEpiOutputs], epi_base[kEpiOutputs];
  if constexpr (EPI != kSlicePartials) {
#pragma unroll
    for (int j = 0; j < kEpiOutputs; ++j) {
      const int o = tid + j * nthr;
      if constexpr (EPI == kSiluPair) {
        const int pair = o & 7, t = (o >> 3) & 15, tl = o >> 7;
        const int r0 = (blockIdx.x * tiles + tl) * 16 + 2 * pair;
        epi_sx[j] = scale_in[min(t, m - 1)];
        epi_b0[j] = bias != nullptr ? bias[min(r0, sh.rows - 1)] : 0.0f;
        epi_b1[j] = bias != nullptr ? bias[min(r0 + 1, sh.rows - 1)] : 0.0f;
        epi_base[j] = 0.0f;
      } else {
        const int r = o & 15, t = (o >> 4) & 15, tl = o >> 8;
        const int out_row = (blockIdx.x * tiles + tl) * 16 + r;
        epi_sx[j] = scale_in[min(t, m - 1)];
        epi_b0[j] = bias != nullptr ? bias[min(out_row, sh.rows - 1)] : 0.0f;
        epi_b1[j] = 0.0f;
        const bool owned = o < tiles * 256 && t < m && out_row < sh.rows;
        epi_base[j] = EPI == kResidual && owned ? output[(size_t)t * sh.out_stride + out_row] : 0.0f;
      }
    }
  }

  // Only the LDS stores are waited for: the weight loads stay in flight.
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");

  const unsigned char* abase = lds + (size_t)span0 * 2 * 128 * m + kb * 16 * m + min(c, m - 1) * 16;
  const int* sbase = lseed + span0 * 2 * 4 * sq + min(kb, sq - 1) * 4;
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int i = 0; i < PART; ++i) {
    v4i a[2][2], seed[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
      for (int o = 0; o < 2; ++o)
        a[h][o] = *reinterpret_cast<const v4i*>(abase + (size_t)((2 * i + h) * 2 + o) * 64 * m);
      seed[h] = *reinterpret_cast<const v4i*>(sbase + (2 * i + h) * 4 * sq);
    }
    const v4u wk = w[i % UW];
    if (i + UW < PART) w[i % UW] = *reinterpret_cast<const v4u*>(wrow + (i + UW) * kSpanBytes);
    // Lanes kb = 0, 1 keep their first 8 bytes and take the first 8 of lane
    // kb + 2 for the span's first group; lanes kb = 2, 3 the reverse.
    const auto s0 = __builtin_amdgcn_permlane32_swap(wk[0], wk[2], false, false);
    const auto s1 = __builtin_amdgcn_permlane32_swap(wk[1], wk[3], false, false);
    const unsigned x0[2] = {s0[0], s0[1]}, x1[2] = {s1[0], s1[1]};
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const v4i b0 = {field<0>(x0[h]), field<1>(x0[h]), field<0>(x1[h]), field<1>(x1[h])};
      const v4i b1 = {field<2>(x0[h]), field<3>(x0[h]), field<2>(x1[h]), field<3>(x1[h])};
      v4i d = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[h][0], b0, seed[h], 0, 0, 0);
      d = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[h][1], b1, d, 0, 0, 0);
      const float s = h2f((uint16_t)(h ? sc[i] >> 16 : sc[i] & 0xffffu));
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[v] = __builtin_fmaf((float)d[v], s, acc[v]);
    }
    // One span per step: the accumulators and the memory operations stay in
    // program order, which keeps the ring's registers from piling up.
#pragma unroll
    for (int v = 0; v < 4; ++v) asm volatile("" : "+v"(acc[v]));
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
  }

  if constexpr (EPI == kSlicePartials) {
    // Chain of lane (c, kb) for tokens 4kb + v of row c, to [slice * parts + part][token][row],
    // stored device-coherent (performed past the XCD's L2) for the in-kernel finish.
    const int out_row = tile * 16 + c;
    const int chain = blockIdx.y * sh.parts + part;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int t = 4 * kb + v;
      if (t < m && out_row < sh.rows)
        store_device(chains + ((size_t)chain * m + t) * sh.rows + out_row, acc[v]);
    }
    if (sh.finish_epi < 0) return;
    // In-kernel finish, by the hand-over of store_device (ternary_device.hpp).
    // Every thread's chains are performed device-wide before the block counts
    // itself in; the block whose count is the last of the tile group's slices
    // then reads all of the group's chains (after its count returned,
    // device-coherent) and finishes them as token_finish_kernel does, then
    // clears the counter for the next launch.  No block waits for another.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    int* last_slot = reinterpret_cast<int*>(dump);
    if (tid == 0)
      *last_slot = __hip_atomic_fetch_add(sh.counters + blockIdx.x, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                   gridDim.y - 1;
    __syncthreads();
    if (*last_slot == 0) return;
    const int chain_count = (int)gridDim.y * sh.parts;
    const size_t stride = (size_t)m * sh.rows;
    const int tiles = sh.tiles_per_block;
    // The chains are loaded eight at a time before they are added (in chain
    // order), so a row's loads share one round trip per eight.
    auto total_of = [&](int t, int r) {
      const float* src = chains + (size_t)t * sh.rows + r;
      float total = 0.0f;
      for (int k0 = 0; k0 < chain_count; k0 += 8) {
        float part[8];
#pragma unroll
        for (int j = 0; j < 8; ++j)
          part[j] = k0 + j < chain_count
                        ? load_device(src + (size_t)(k0 + j) * stride)
                        : 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j)
          if (k0 + j < chain_count) total = k0 + j == 0 ? part[0] : total + part[j];
      }
      float y = total * scale_in[t];
      if (bias != nullptr) y = y + bias[r];
      return y;
    };
    if (sh.finish_epi == kSiluPair) {
      for (int o = tid; o < tiles * 8 * m; o += nthr) {
        const int pair = o & 7, rest = o >> 3, tl = rest % tiles, t = rest / tiles;
        const int r0 = (blockIdx.x * tiles + tl) * 16 + 2 * pair;
        if (r0 + 1 < sh.rows) output[(size_t)t * sh.out_stride + (r0 >> 1)] = ivo_silu(total_of(t, r0)) * total_of(t, r0 + 1);
      }
    } else {
      for (int o = tid; o < tiles * 16 * m; o += nthr) {
        const int r = o & 15, rest = o >> 4, tl = rest % tiles, t = rest / tiles;
        const int out_row = (blockIdx.x * tiles + tl) * 16 + r;
        if (out_row >= sh.rows) continue;
        float* dst = output + (size_t)t * sh.out_stride + out_row;
        const float y = total_of(t, out_row);
        if (sh.finish_epi == kResidual) *dst = *dst + y;
        else *dst = y;
      }
    }
    if (tid == 0) __hip_atomic_store(sh.counters + blockIdx.x, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }

  // Partials of lane (c, kb): tokens 4kb + v of row c.
#pragma unroll
  for (int v = 0; v < 4; ++v) partial[(wave * 16 + 4 * kb + v) * 16 + c] = acc[v];
  __syncthreads();

  if constexpr (EPI == kSiluPair) {
    // Output j of a token pairs gate row 2j and up row 2j + 1 of the tile.
#pragma unroll
    for (int j = 0; j < kEpiOutputs; ++j) {
      const int o = tid + j * nthr;
      if (o >= tiles * 16 * 8) break;
      const int pair = o & 7, t = (o >> 3) & 15, tl = o >> 7;
      const int r0 = (blockIdx.x * tiles + tl) * 16 + 2 * pair;
      float y[2];
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const float* src = partial + ((tl * sh.parts) * 16 + t) * 16 + 2 * pair + e;
        float total = src[0];
        for (int p = 1; p < sh.parts; ++p) total = total + src[p * 256];
        y[e] = total * epi_sx[j];
        if (bias != nullptr) y[e] = y[e] + (e ? epi_b1[j] : epi_b0[j]);
      }
      if (t < m && r0 + 1 < sh.rows) output[(size_t)t * sh.out_stride + (r0 >> 1)] = ivo_silu(y[0]) * y[1];
    }
  } else {
#pragma unroll
    for (int j = 0; j < kEpiOutputs; ++j) {
      const int o = tid + j * nthr;
      if (o >= tiles * 256) break;
      const int r = o & 15, t = (o >> 4) & 15, tl = o >> 8;
      const int out_row = (blockIdx.x * tiles + tl) * 16 + r;
      const float* src = partial + ((tl * sh.parts) * 16 + t) * 16 + r;
      float total = src[0];
      for (int p = 1; p < sh.parts; ++p) total = total + src[p * 256];
      float y = total * epi_sx[j];
      if (bias != nullptr) y = y + epi_b0[j];
      if (t < m && out_row < sh.rows) {
        float* dst = output + (size_t)t * sh.out_stride + out_row;
        if constexpr (EPI == kResidual) *dst = epi_base[j] + y;
        else *dst = y;
      }
    }
  }
}

// Finish of a sliced launch: output (token t, row r) = the `chains` fp32
// chains of (t, r) added in chain order, times the token scale, plus the bias,
// then the epilogue (a SiLU pair takes rows 2j and 2j + 1).  One thread per
// output.
template <int EPI>
__global__ __launch_bounds__(256) void token_finish_kernel(const float* __restrict__ partials, int chains,
                                                           const float* __restrict__ scale_in,
                                                           const float* __restrict__ bias, float* __restrict__ output,
                                                           int m, int rows, int out_stride) {
  const int width = EPI == kSiluPair ? rows / 2 : rows;
  const long long o = (long long)blockIdx.x * 256 + threadIdx.x;
  if (o >= (long long)m * width) return;
  const int t = (int)(o / width), j = (int)(o - (long long)t * width);
  const size_t stride = (size_t)m * rows;
  auto finish = [&](int r) {
    const float* src = partials + (size_t)t * rows + r;
    float total = src[0];
    for (int c = 1; c < chains; ++c) total = total + src[c * stride];
    float y = total * scale_in[t];
    if (bias != nullptr) y = y + bias[r];
    return y;
  };
  float* dst = output + (size_t)t * out_stride + j;
  if constexpr (EPI == kSiluPair) {
    const float gate = finish(2 * j);
    *dst = ivo_silu(gate) * finish(2 * j + 1);
  } else if constexpr (EPI == kResidual) {
    *dst = *dst + finish(j);
  } else {
    *dst = finish(j);
  }
}

constexpr int kPartSpans[] = {16, 14, 8, 4, 2, 1};

template <int EPI, int PART>
hipError_t launch_part(hipStream_t stream, const GemmArgs& a, const TokenShape& sh, int fill, dim3 blocks, int threads,
                       size_t lds, float* chains) {
  auto go = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, blocks, dim3(threads), lds, stream, a.q8_in, a.xsum_in, a.scale_in, a.packed,
                       a.scales, a.bias, a.output, chains, sh);
    return hipGetLastError();
  };
  if (fill <= 2) return go(token_gemv_kernel<EPI, PART, 2>);
  if (fill <= 4) return go(token_gemv_kernel<EPI, PART, 4>);
  if (fill <= 8) return go(token_gemv_kernel<EPI, PART, 8>);
  if (fill <= 12) return go(token_gemv_kernel<EPI, PART, 12>);
  // The plan gives 16-span waves at most 12 fill pieces (16 would spill).
  if constexpr (PART == 16) return hipErrorInvalidValue;
  else return go(token_gemv_kernel<EPI, PART, 16>);
}

template <int EPI>
hipError_t launch_epi(hipStream_t stream, const GemmArgs& a, const TokenPlan& plan, float* chains,
                      unsigned* counters = nullptr, int finish_epi = -1) {
  const int groups = a.n / kGroup;
  TokenShape sh{a.rows, a.n, a.row_bytes, a.groups, a.m, plan.parts, plan.tiles_per_block, a.out_stride,
                groups / plan.slices, finish_epi, counters};
  const int threads = 64 * plan.parts * plan.tiles_per_block;
  const dim3 blocks(ceil_div(ceil_div(a.rows, 16), plan.tiles_per_block), plan.slices);
  switch (plan.part_spans) {
    case 16: return launch_part<EPI, 16>(stream, a, sh, plan.fill, blocks, threads, plan.lds, chains);
    case 14: return launch_part<EPI, 14>(stream, a, sh, plan.fill, blocks, threads, plan.lds, chains);
    case 8: return launch_part<EPI, 8>(stream, a, sh, plan.fill, blocks, threads, plan.lds, chains);
    case 4: return launch_part<EPI, 4>(stream, a, sh, plan.fill, blocks, threads, plan.lds, chains);
    case 2: return launch_part<EPI, 2>(stream, a, sh, plan.fill, blocks, threads, plan.lds, chains);
    case 1: return launch_part<EPI, 1>(stream, a, sh, plan.fill, blocks, threads, plan.lds, chains);
    default: return hipErrorInvalidValue;
  }
}

template <int EPI>
hipError_t launch_finish(hipStream_t stream, const GemmArgs& a, int chains, const float* partials) {
  const int width = EPI == kSiluPair ? a.rows / 2 : a.rows;
  const long long outputs = (long long)a.m * width;
  if (outputs == 0) return hipSuccess;
  hipLaunchKernelGGL(token_finish_kernel<EPI>, dim3((unsigned)((outputs + 255) / 256)), dim3(256), 0, stream,
                     partials, chains, a.scale_in, a.bias, a.output, a.m, a.rows, a.out_stride);
  return hipGetLastError();
}

}  // namespace

TokenPlan token_gemv_plan(int m, int rows, int n, int cus, size_t max_lds) {
  TokenPlan plan{0, 0, 0, 0, 0, 1};
  if (m < 1 || m > kMaxTokens || rows < 1 || n < 256 || n % 256 != 0) return plan;
  const int spans = n / 256, tiles = ceil_div(rows, 16);
  const int sq = (m + 3) / 4;
  // The fewest K slices whose q8 bytes fit in LDS (one slice: the whole rows).
  for (int slices = 1; slices <= kMaxSlices; ++slices) {
    if (spans % slices != 0) continue;
    const int slice_spans = spans / slices, slice_groups = 2 * slice_spans;
    // Spans per wave: the longest range that still gives every CU eight
    // waves, else the shortest available; at most 16 waves per row tile.
    int part_spans = 0;
    for (int candidate : kPartSpans) {
      if (slice_spans % candidate != 0 || slice_spans / candidate > kMaxWaves) continue;
      part_spans = candidate;
      if ((long long)tiles * (slice_spans / candidate) * slices >= 8LL * cus) break;
    }
    if (part_spans == 0) continue;
    const int parts = slice_spans / part_spans;
    int tiles_per_block = ceil_div(tiles * slices, cus);
    if (tiles_per_block > kMaxWaves / parts) tiles_per_block = kMaxWaves / parts;
    if (tiles_per_block < 1) tiles_per_block = 1;
    const int threads = 64 * parts * tiles_per_block;
    const size_t abytes = (size_t)slice_groups * 128 * m;
    const size_t seeds = (size_t)slice_groups * 4 * sq;
    const size_t partials = slices == 1 ? (size_t)threads / 64 * 1024 : 0;
    const size_t lds = abytes + 4 * seeds + partials + 16;
    const int fill = (int)((abytes / 16 + threads - 1) / threads);
    // (Sixteen fill pieces per thread on top of a 16-span ring would spill.)
    if (lds > max_lds || fill > (part_spans == 16 ? 12 : 16) || seeds > (size_t)kSeedsPerThread * threads) continue;
    if (slices > 1 && (long long)slices * parts * m * rows > kTokenPartialFloats) return plan;
    plan.parts = parts;
    plan.part_spans = part_spans;
    plan.tiles_per_block = tiles_per_block;
    plan.fill = fill;
    plan.lds = lds;
    plan.slices = slices;
    return plan;
  }
  return plan;
}

hipError_t launch_token_gemv(hipStream_t stream, const GemmArgs& a, const TokenPlan& plan) {
  if (plan.parts == 0) return hipErrorInvalidValue;
  if (plan.slices == 1) {
    switch (a.epi) {
      case kStore: return launch_epi<kStore>(stream, a, plan, nullptr);
      case kResidual: return launch_epi<kResidual>(stream, a, plan, nullptr);
      case kSiluPair: return launch_epi<kSiluPair>(stream, a, plan, nullptr);
      default: return hipErrorInvalidValue;
    }
  }
  if (a.epi != kStore && a.epi != kResidual && a.epi != kSiluPair) return hipErrorInvalidValue;
  Scratch* work = nullptr;
  hipError_t status = scratch_for_stream(stream, &work);
  if (status != hipSuccess) return status;
  // The last slice of each tile group finishes it in the same launch when the
  // group count fits the scratch's counters; otherwise a second kernel does.
  const int tile_groups = ceil_div(ceil_div(a.rows, 16), plan.tiles_per_block);
  if (work->sync != nullptr && tile_groups <= defines().token_finish_groups && tile_groups <= kTokenFinishCounters)
    return launch_epi<kSlicePartials>(stream, a, plan, work->token_partials, work->sync, a.epi);
  status = launch_epi<kSlicePartials>(stream, a, plan, work->token_partials);
  if (status != hipSuccess) return status;
  const int chains = plan.parts * plan.slices;
  switch (a.epi) {
    case kStore: return launch_finish<kStore>(stream, a, chains, work->token_partials);
    case kResidual: return launch_finish<kResidual>(stream, a, chains, work->token_partials);
    default: return launch_finish<kSiluPair>(stream, a, chains, work->token_partials);
  }
}

}  // namespace ivo
