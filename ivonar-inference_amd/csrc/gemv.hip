// Decode GEMV for one token (reference: kernels/ternary.cu:302-388,
// entry points gemv_* with GEMV_ARGS).
//
// Work split.  A row of the packed matrix is covered by `lanes` lanes of a
// wave (a power of two, 2..64, the smallest that spans the row's chunks); a
// wave holds 64/lanes row slots and each lane streams kRows rows, so one
// wave step reads kRows * 64 lanes * 16 bytes with 128-bit loads that are
// contiguous across the lanes of a slot.  Lane `sub` takes chunks
// u = j*lanes + sub (j = 0..NJ-1), so the two chunks of a 128-input group
// land on a lane pair: each lane forms its chunk's exact int32 sum of
// code*q minus the chunk's q sum, and one DPP swap (quad_perm [1,0,3,2])
// adds the pair into the group partial P[r, g].  The pair folds
// P * scale[r, g] into an fp32 fma chain over its groups (g = pair,
// pair + lanes/2, ...); a butterfly over the pairs in xor order (formed with
// DPP row shifts and permlane swaps, pair_tree_sum), the token scale and the
// bias finish the row.  The CPU oracle restates that order bit for bit
// (orc_gemv_pairs).
//
// Memory.  Loads are unconditional: indices past the row or the matrix are
// clamped to valid addresses and the integer result is masked, which keeps
// the loop free of exec-mask branches.  The first weight loads are issued
// before the activation prologue, and when a row needs one step per lane the
// next row's weights are prefetched while the current one is computed
// (double buffering), so each wave keeps 2-4 KB in flight; rows of 2..8
// steps keep all steps of a row pair in flight (gemv_rows_kernel).
//
// Activations.  For rows up to kFusedLimit inputs the block quantizes the
// fp32 input itself into LDS (the fused prologue of gemv_plain_*,
// gemv_norm_*, gemv_attn_*), quad-planar (quad w of chunk u at int4 index
// w*C + u), and each lane then keeps its chunks' quads in registers.  PLAIN
// rows (16-byte aligned) of 4097..32768 inputs are quantized by every block
// of the long-row GEMV itself into its LDS (quantize_row_split), while its
// first weights stream; other long rows are quantized once into the stream's
// scratch by the quantizer, in a launch of its own.  Pre-quantized activations are read by each lane straight from
// global memory when a row needs one step per lane (no LDS: the q8 row is
// small and stays in the caches for every block), else copied to LDS once
// per block (gemv_rows_kernel for 2..8 steps, the rolling layout above).
//
// Integer core.  The fused kernels take 8-bit dot products on q8 quads
// (chunk_code_dot, 9 VALU per packed word).  Pre-quantized activations take
// 4-bit dot products on nibble-split quads (chunk_split_dot, 7 VALU per
// word): the quantizer writes the scratch row split, and a caller's q8 quads
// are split as they are loaded (split_quad, once per quad and lane in
// registers, once per block in the LDS copies).  Both return the same exact
// int32 sums, so the fp32 order and the outputs do not depend on the form.
#include <type_traits>

#include "internal.hpp"
#include "ternary_device.hpp"

namespace ivo {
namespace {

constexpr int kRows = 2;  // rows per lane; even, so a silu pair stays in one lane
constexpr int kFusedLimit = 4096;
static_assert(kFusedLimit <= kThreads * kBatch, "the fused prologue holds a row in registers");
constexpr int kMaxLdsBytes = 64 * 1024;
constexpr int kBlocksPerCu = 4;

struct GemvShape {
  int rows, n, row_bytes, groups, splits, head_dim;
  float eps;
  int lanes, lane_shift, iters;
  int exact;  // every lane's chunks exist (C is a multiple of lanes): no per-chunk masks
  int split;  // the activations are nibble-split quads (the two-pass path's own scratch)
  int out_stride;  // floats between the output rows of consecutive tokens (several tokens only)
};

struct GemvPtrs {
  const float* input;
  const float* aux;
  const int8_t* q8_in;
  const int32_t* xsum_in;
  const float* scale_in;
};

// One pipeline item's loads: weights of NJ steps for kRows rows (w[j][0] of
// the lane's own row row0 + (sub & 1), w[j][1] of its partner's), per step
// the group scale of the lane's own row (row0 + (sub & 1)), and for the
// residual epilogue that row's output value, so the read of the residual base
// travels with the weights instead of adding a round trip after the sums.
template <int NJ>
struct Step {
  uint4 w[NJ][kRows];
  uint16_t s[NJ];
  float base;
};

__device__ __forceinline__ uint4 load16(const uint8_t* __restrict__ p) {
  return *reinterpret_cast<const uint4*>(p);
}

template <int NJ, bool SCALES, int LANES, bool BASE, bool EXACT>
__device__ __forceinline__ void load_step(Step<NJ>& st, const uint8_t* __restrict__ packed,
                                          const uint16_t* __restrict__ scales, const float* __restrict__ base,
                                          const GemvShape& sh, int row0, int j0, int sub, int chunks) {
  const int lanes = LANES ? LANES : sh.lanes;
  const int own_row = min(row0 + (sub & 1), sh.rows - 1);
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    // With EXACT every chunk of an item exists (items hold no dead steps), and
    // leaving out the clamp lets the step offsets fold into the loads.
    const int u = EXACT ? (j0 + j) * lanes + sub : min((j0 + j) * lanes + sub, chunks - 1);
#pragma unroll
    for (int r = 0; r < kRows; ++r) {
      const int row = min(row0 + (r ^ (sub & 1)), sh.rows - 1);
      st.w[j][r] = load16(packed + (size_t)row * sh.row_bytes + (size_t)u * 16);
    }
    st.s[j] = SCALES ? scales[(size_t)own_row * sh.groups + (u >> 1)] : (uint16_t)0;
  }
  st.base = BASE ? base[own_row] : 0.0f;
}

// Lane pair (sub, sub ^ 1) covers the two chunks of a group for rows row0 and
// row0 + 1; each lane keeps the accumulator of its own row (sub & 1).  A lane
// forms both rows' chunk sums (its own row's first), sends the partner's row
// across the pair (one DPP swap) and adds the partner's sum for its own row:
// the exact group partial P[own row, g].
template <int EPI, int NJ, bool QREG, int LANES, bool EXACT, bool XNEG = false, bool SPLIT = false>
__device__ __forceinline__ void compute_step(const Step<NJ>& st, const int4 (&qr)[QREG ? NJ : 1][4],
                                             const int (&xr)[QREG ? NJ : 1], const int4* __restrict__ lds_q,
                                             const int* __restrict__ lds_x, float& acc,
                                             int32_t* __restrict__ partials, const GemvShape& sh, int row0, int j0,
                                             int sub, int chunks) {
  static_assert(kRows == 2, "a lane pair holds two rows");
  const int lanes = LANES ? LANES : sh.lanes;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int u_raw = (j0 + j) * lanes + sub;
    const bool live = EXACT || u_raw < chunks;
    const int g = u_raw >> 1;
    const bool group_live = EXACT || 2 * g < chunks;
    int4 q0, q1, q2, q3;
    int xs;
    if constexpr (QREG) {
      q0 = qr[j][0];
      q1 = qr[j][1];
      q2 = qr[j][2];
      q3 = qr[j][3];
      xs = xr[j];
    } else {
      const int u = EXACT ? u_raw : min(u_raw, chunks - 1);
      q0 = lds_q[u];
      q1 = lds_q[chunks + u];
      q2 = lds_q[2 * chunks + u];
      q3 = lds_q[3 * chunks + u];
      xs = lds_x[u];
    }
    const int seed = XNEG ? xs : -xs;  // XNEG: the LDS copy holds minus the chunk sums
    // The partner's row first: its sum crosses the pair by DPP, and a DPP read
    // of a VGPR needs two wait states after the VALU instruction that wrote it
    // (gfx9 family).  The compiler pads that gap with s_nop where nothing
    // independent fills it; computing the partner's sum first puts the own
    // row's dot products in the gap.  The order saves issue cycles only: the
    // result does not depend on it.
    // SPLIT: the activations are nibble-split quads (4-bit dot products).
    int d1 = SPLIT ? chunk_split_dot(st.w[j][1], q0, q1, q2, q3, seed) : chunk_code_dot(st.w[j][1], q0, q1, q2, q3, seed);
    int d0 = SPLIT ? chunk_split_dot(st.w[j][0], q0, q1, q2, q3, seed) : chunk_code_dot(st.w[j][0], q0, q1, q2, q3, seed);
    if constexpr (!EXACT) {
      d0 = live ? d0 : 0;
      d1 = live ? d1 : 0;
    }
    const int d = d0 + pair_swap(d1);
    if constexpr (EPI == kPartials) {
      const int row = row0 + (sub & 1);
      if (group_live && row < sh.rows) partials[(size_t)row * sh.groups + g] = d >> 4;
    } else {
      const float contribution = EXACT || group_live ? (float)d : 0.0f;
      acc = __builtin_fmaf(contribution, h2f(st.s[j]), acc);
    }
  }
}

// Threads per block: the rolling layout (long rows, q8 copied to LDS) runs
// one 1024-thread block per CU, so each CU copies the q8 row once and the
// copy takes one load round trip; the others run four 256-thread blocks.
template <bool ROLL>
constexpr int block_threads() {
  return ROLL ? 1024 : kThreads;
}

template <int MODE, int EPI, bool FUSED, int NJ, int LANES, bool EXACT, bool ROLL>
__global__ __launch_bounds__(block_threads<ROLL>()) void gemv_kernel(GemvPtrs in, const uint8_t* __restrict__ packed,
                                                        const uint16_t* __restrict__ scales,
                                                        const float* __restrict__ bias, float* __restrict__ output,
                                                        int32_t* __restrict__ partials, GemvShape sh) {
  // One block of steps per row (no rolling over steps) keeps the lane's q8
  // words in registers for the whole kernel; a rolling pipeline reads them
  // from the block's LDS copy at every step.
  constexpr bool QREG = !ROLL;
  static_assert(!(FUSED && ROLL), "the fused prologue keeps q8 in registers");
  // Pre-quantized activations take the 4-bit dot products: quads arrive split
  // (sh.split, the two-pass path's scratch) or are split as they are loaded.
  constexpr bool SPLIT = !FUSED;
  extern __shared__ __align__(16) unsigned char lds_raw[];
  __shared__ float slots[64];
  const int chunks = (sh.n + kChunk - 1) / kChunk;
  int4* lds_q = reinterpret_cast<int4*>(lds_raw);  // quad w of chunk u at w*C + u
  int* lds_x = reinterpret_cast<int*>(lds_raw + (size_t)chunks * kChunk);
  const int4* gq = reinterpret_cast<const int4*>(in.q8_in);  // chunk u, quad w at u*4 + w

  const int lane = threadIdx.x & 63;
  const int lanes = LANES ? LANES : sh.lanes;
  const int lane_shift = LANES ? __builtin_ctz(LANES) : sh.lane_shift;
  const int sub = lane & (lanes - 1);
  const int slot = lane >> lane_shift;
  const int rows_per_iter = (64 >> lane_shift) * kRows;
  constexpr int kBlock = block_threads<ROLL>();
  const int waves = gridDim.x * (kBlock / 64);
  const int first = blockIdx.x * (kBlock / 64) + (threadIdx.x >> 6);
  const int steps = (chunks + lanes - 1) / lanes;

  // Weights of the first row step go out before the activation prologue
  // (for rows the block quantizes from registers, right behind the row).
  // Loads are never predicated (rows past the matrix are clamped inside
  // load_step), so the wait counts before each use stay exact.
  Step<NJ> a, b;
  int it = __builtin_amdgcn_readfirstlane(first);  // wave-uniform: the per-item branches are scalar
  auto first_loads = [&]() {
    load_step<NJ, EPI != kPartials, LANES, EPI == kResidual, EXACT>(a, packed, scales, output, sh,
                                                            it * rows_per_iter + slot * kRows, 0, sub, chunks);
  };
  // PLAIN and NORM rows quantized in the block, and pre-quantized rows held
  // in registers, issue the first weights right behind the row's loads, so
  // the prologue waits for the row only.
  constexpr bool kWeightsAfterRow = (FUSED && MODE != kAttn) || (!FUSED && QREG);
  if constexpr (!kWeightsAfterRow) first_loads();

  float sx;
  int4 qr[QREG ? NJ : 1][4];
  int xr[QREG ? NJ : 1];
  if constexpr (FUSED) {
    // The block quantizes the token into LDS, then each lane takes its
    // chunks' quads.  PLAIN and NORM rows are read once into registers; the
    // lane forms its chunks' sums from the quads it holds.
    const RowSource src{in.input, in.aux, sh.n, sh.eps, sh.splits, sh.head_dim};
    if constexpr (MODE == kAttn) {
      float inv_rms;
      sx = row_scale<MODE>(src, inv_rms, slots);
      for (int d = threadIdx.x; d < chunks * 16; d += kThreads) {
        const int u = d >> 4, w = (d >> 2) & 3, k = d & 3;
        const int value = quantize_word<MODE>(src, u, w, k, inv_rms, sx);
        reinterpret_cast<int*>(lds_q)[(w * chunks + u) * 4 + k] = value;
      }
    } else {
      // Each thread loads only the batches of 256 inputs a row can reach
      // (the clamped loads past the row are not free): rows of fewer than 64
      // lanes have at most 32 chunks (one step per lane), 2048 inputs, and
      // rows of up to 1024 inputs (the decoder's model width) take a
      // four-batch copy of the prologue (one block-uniform branch).
      // A 16-byte aligned PLAIN row is read as float4.
      unsigned char* q = reinterpret_cast<unsigned char*>(lds_q);
      const bool vec = MODE == kPlain && (sh.n & 3) == 0 && (reinterpret_cast<uintptr_t>(in.input) & 15) == 0;
      auto quantize = [&](auto nb_c) {
        constexpr int NB = decltype(nb_c)::value;
        if (vec) return quantize_plain_row4_to_lds<NB>(src, chunks, q, slots, first_loads);
        return quantize_row_to_lds<MODE, NB>(src, chunks, q, slots, first_loads);
      };
      if constexpr (LANES == 64) sx = quantize(std::integral_constant<int, kBatch>{});
      else if (sh.n <= 4 * kThreads) sx = quantize(std::integral_constant<int, 4>{});
      else sx = quantize(std::integral_constant<int, kBatch / 2>{});
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int u = min(j * lanes + sub, chunks - 1);
      int total = 0;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        qr[j][w] = lds_q[w * chunks + u];
        total = word_sum(qr[j][w].x) + word_sum(qr[j][w].y) + word_sum(qr[j][w].z) + word_sum(qr[j][w].w) + total;
      }
      xr[j] = total;
    }
  } else if constexpr (QREG) {
    // Pre-quantized and at most two steps per lane: the lane's quads straight from global memory.
    sx = *in.scale_in;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int u = min(j * lanes + sub, chunks - 1);
#pragma unroll
      for (int w = 0; w < 4; ++w) qr[j][w] = gq[u * 4 + w];
      xr[j] = in.xsum_in[u];
    }
    __builtin_amdgcn_sched_barrier(0);
    first_loads();
    __builtin_amdgcn_sched_barrier(0);
    if (!sh.split) {
#pragma unroll
      for (int j = 0; j < NJ; ++j)
#pragma unroll
        for (int w = 0; w < 4; ++w) qr[j][w] = split_quad(qr[j][w]);
    }
  } else {
    // Rolling over a long row: the block copies the q8 row to LDS.  All of a
    // thread's loads go out before its LDS stores.
    constexpr int kCopyBatch = 8;
    const int words = chunks * 4;
    for (int base = 0; base < words; base += kBlock * kCopyBatch) {
      int4 v[kCopyBatch];
#pragma unroll
      for (int k = 0; k < kCopyBatch; ++k) v[k] = gq[min(base + k * kBlock + (int)threadIdx.x, words - 1)];
#pragma unroll
      for (int k = 0; k < kCopyBatch; ++k) {
        const int e = base + k * kBlock + threadIdx.x;
        if (e < words) lds_q[(e & 3) * chunks + (e >> 2)] = sh.split ? v[k] : split_quad(v[k]);
      }
    }
    for (int u = threadIdx.x; u < chunks; u += kBlock) lds_x[u] = in.xsum_in[u];
    sx = *in.scale_in;
    __syncthreads();
  }

  // Butterfly over the pairs (offsets 2 .. lanes/2 keep each lane's row),
  // then lane sub = r finishes row row0 + r.
  auto finish = [&](float acc, int row0, float base) {
    if constexpr (EPI != kPartials) {
      acc = pair_tree_sum(acc, lanes);
      const int row = row0 + (sub & 1);
      float y = acc * 0.0625f * sx;  // the folded sums carry chunk_code_dot's factor 16
      if (bias != nullptr && row < sh.rows) y = y + bias[row];
      if constexpr (EPI == kSiluPair) {
        const float up = __int_as_float(pair_swap(__float_as_int(y)));
        if (sub == 0 && row + 1 < sh.rows) output[row >> 1] = ivo_silu(y) * up;
      } else if (sub < 2 && row < sh.rows) {
        if constexpr (EPI == kStore) output[row] = y;
        else output[row] = base + y;
      }
    }
  };

  // Rolling pipeline over items (row step, block of NJ steps): the next
  // item's weights are in flight while the current one is computed.
  // With q8 in registers an item is a whole row (NJ == steps, the host's
  // layouts): jb stays 0, and saying so lets the step offsets fold into the
  // loads' immediate offsets.
  // The wave's last item prefetches nothing (no loads go out for rows past the end).
  const int blocks_per_row = QREG ? 1 : (steps + NJ - 1) / NJ;
  int jb = 0;
  float acc = 0.0f;
  auto item = [&](Step<NJ>& current, Step<NJ>& next) -> bool {
    int it_next = it, jb_next = jb + 1;
    if (jb_next == blocks_per_row) {
      jb_next = 0;
      it_next = it + waves;
    }
    const int row0 = it * rows_per_iter + slot * kRows;
    const bool more = it_next < sh.iters;
    if (more) {
      const int j_next = QREG ? 0 : jb_next * NJ;
      load_step<NJ, EPI != kPartials, LANES, EPI == kResidual, EXACT>(next, packed, scales, output, sh,
                                                                     it_next * rows_per_iter + slot * kRows, j_next,
                                                                     sub, chunks);
    }
    compute_step<EPI, NJ, QREG, LANES, EXACT, false, SPLIT>(current, qr, xr, lds_q, lds_x, acc, partials, sh, row0,
                                              QREG ? 0 : jb * NJ, sub, chunks);
    if (jb == blocks_per_row - 1) {
      finish(acc, row0, current.base);
      acc = 0.0f;
    }
    it = it_next;
    jb = jb_next;
    return more;
  };
  if (it < sh.iters) {
    while (item(a, b) && item(b, a)) {
    }
  }
}

typedef int v4i32 __attribute__((ext_vector_type(4)));

// Loads the compiler does not track (see gemv_rows_kernel).
__device__ __forceinline__ v4i32 load_b128(const void* p) {
  v4i32 r;
  asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(r) : "v"(p) : "memory");
  return r;
}
__device__ __forceinline__ int load_b32(const void* p) {
  int r;
  asm volatile("global_load_dword %0, %1, off" : "=v"(r) : "v"(p) : "memory");
  return r;
}
__device__ __forceinline__ int load_u16(const void* p) {
  int r;
  asm volatile("global_load_ushort %0, %1, off" : "=v"(r) : "v"(p) : "memory");
  return r;
}
// The same loads at a constant byte offset (-4096..4095) from p.
template <int OFF>
__device__ __forceinline__ v4i32 load_b128_at(const void* p) {
  static_assert(OFF >= -4096 && OFF < 4096, "13-bit signed instruction offset");
  v4i32 r;
  asm volatile("global_load_dwordx4 %0, %1, off offset:%2" : "=v"(r) : "v"(p), "n"(OFF) : "memory");
  return r;
}
template <int OFF>
__device__ __forceinline__ int load_u16_at(const void* p) {
  static_assert(OFF >= -4096 && OFF < 4096, "13-bit signed instruction offset");
  int r;
  asm volatile("global_load_ushort %0, %1, off offset:%2" : "=v"(r) : "v"(p), "n"(OFF) : "memory");
  return r;
}

typedef float v4f32 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ v4f32 load_f128(const void* p) {
  v4f32 r;
  asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(r) : "v"(p) : "memory");
  return r;
}
// A value u = fma(x, 1/s, 128) at least this far below the next half-integer
// and above the previous one rounds like x/s + 128 (see quantize_row_split).
constexpr float kTieGuard = 0.49997f;

// f(integral_constant<int, 0>) ... f(integral_constant<int, N - 1>): an
// unrolled loop whose index can feed an immediate operand.
template <int N, int I = 0, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<N, I + 1>(f);
  }
}

// In-launch quantization of a PLAIN row (the long-row kernel with QUANT): every
// block quantizes the whole row into its own LDS copy, so no block waits for
// another.  T threads; thread t holds float4 k*T + t of the row (inputs
// 4f .. 4f + 3 of float4 f, k < X) in xv: coalesced loads.  n is a multiple of
// 4; the row is zero past n up to its C = `chunks` chunks of 64.  Writes the
// nibble-split quads (word k of quad w of chunk u at lds_words[(w*C + u)*4 + k],
// the form split_quad gives) and minus the chunk sums (lds_x[u]) and returns
// the token scale.  step(k) runs after the k-th float4 is quantized (the
// caller issues weight loads there).  slots holds T/64 floats.  The LDS
// writes are not yet waited for.
//
// Bit-exact with the quantizer kernels (quantize_plain_slice):
// scale = max(amax/127, 1e-5) and q = (int)rint(x / scale).  The division is
// replaced by u = RN(x * inv + 128) with inv = RN(1/scale), q + 128 = rint(u):
// |x/scale| <= 127 * (1 + 2^-23), so |x*inv - x/scale| <= 127 * 2^-24 and the
// fma's rounding adds at most 2^-17 (half an ulp below 256), |u - (x/scale + 128)|
// < 1.6e-5; the correctly rounded quotient is within 2^-18 of x/scale.  When u
// lies more than 2e-5 from every half-integer, rint(u) - 128 is therefore
// rint(RN(x/scale)).  Closer values (about 6 in 10^5 inputs, exact ties among
// them), NaN and infinities take the division itself.
//
// Layout: the lanes 4g .. 4g + 3 hold the four float4 of one 16-input quad g;
// q8 word k of the quad holds inputs 4b + k at byte b, so lane j (= t & 3)
// forms word j from byte j of each of the four lanes' q bytes: three DPP quad
// permutations bring the other lanes' bytes over and two v_perm_b32 place
// byte j of each at byte i of the word (source lane i).  The split word j then
// takes nibbles of its own word and of the word of lane j ^ 2 (see
// split_quad_word): one rotate and one bitfield insert with per-lane constants.
// The converted bytes are biased (b = q + 128); one XOR with 0x80 per byte
// gives q itself.  The chunk sums are dot products of the q bytes with -1 (the
// LDS copy holds minus the sums) added over the chunk's 16 lanes.
//
// ALL: every float4 of the X per thread lies inside the row's chunks (the
// rows of exact long-row launches), so no store is predicated.
template <int T, int X, bool ALL, typename Step>
__device__ __forceinline__ float quantize_row_split(v4f32 (&xv)[X], int n, int chunks, int* lds_words, int* lds_x,
                                                    float* slots, Step&& step) {
  static_assert(T % 16 == 0, "a row of 16 float4 per chunk starts at a multiple of 16 lanes");
  const int tid = threadIdx.x;
  const int n4 = n >> 2;
  const int j = tid & 3;
  if (n4 < X * T) {  // zeros past the row (uniform: only rows that are not a whole number of blocks)
#pragma unroll
    for (int k = 0; k < X; ++k)
      if (k * T + tid >= n4) xv[k] = v4f32{0.0f, 0.0f, 0.0f, 0.0f};
  }
  float amax = 0.0f;
#pragma unroll
  for (int k = 0; k < X; ++k)
    amax = fmaxf(fmaxf(amax, fmaxf(fabsf(xv[k][0]), fabsf(xv[k][1]))), fmaxf(fabsf(xv[k][2]), fabsf(xv[k][3])));
  amax = wave_max(amax);
  if ((tid & 63) == 0) slots[tid >> 6] = amax;
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");  // the weight loads stay in flight
  amax = slots[0];
#pragma unroll
  for (int w = 1; w < T / 64; ++w) amax = fmaxf(amax, slots[w]);
  const float scale = fmaxf(amax / 127.0f, 1e-5f);
  const float inv = 1.0f / scale;
  // Per-lane constants: v_perm_b32 selectors (byte values 0..3 pick from the
  // second operand, 4..7 from the first, 0x0C gives zero) and the split's
  // rotation and nibble mask.
  unsigned sel_near = 0x0C0C0C0Cu, sel_far = 0x0C0C0C0Cu;
  sel_near = (sel_near & ~(0xFFu << (8 * j))) | ((unsigned)j << (8 * j));                  // own byte j at j
  sel_near = (sel_near & ~(0xFFu << (8 * (j ^ 1)))) | ((unsigned)(4 + j) << (8 * (j ^ 1)));  // lane j^1's at j^1
  sel_far = (sel_far & ~(0xFFu << (8 * (j ^ 2)))) | ((unsigned)j << (8 * (j ^ 2)));          // lane j^2's at j^2
  sel_far = (sel_far & ~(0xFFu << (8 * (j ^ 3)))) | ((unsigned)(4 + j) << (8 * (j ^ 3)));    // lane j^3's at j^3
  const unsigned rot = j < 2 ? 4u : 28u;
  const unsigned nibbles = j < 2 ? 0x0F0F0F0Fu : 0xF0F0F0F0u;
  // float4 f = k*T + tid is quad g = f >> 2 (chunk g >> 2, quad g & 3) and
  // chunk f >> 4: both advance by a constant per k.
  int* word_dst = lds_words + ((((tid >> 2) & 3) * chunks + (tid >> 4)) << 2) + j;
  int* sum_dst = lds_x + (tid >> 4);
  static_for<X>([&](auto kc) {
    constexpr int k = decltype(kc)::value;
    const int f = k * T + tid;
    float v[4];
    bool near = false;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float u = __builtin_fmaf(xv[k][e], inv, 128.0f);
      const float r = __builtin_rintf(u);
      near = near || !(fabsf(u - r) < kTieGuard);
      v[e] = r;
    }
    if (near) {
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = (float)((int)__builtin_rintf(xv[k][e] / scale) + 128);
    }
    unsigned biased = __builtin_amdgcn_cvt_pk_u8_f32(v[0], 0, 0u);
    biased = __builtin_amdgcn_cvt_pk_u8_f32(v[1], 1, biased);
    biased = __builtin_amdgcn_cvt_pk_u8_f32(v[2], 2, biased);
    biased = __builtin_amdgcn_cvt_pk_u8_f32(v[3], 3, biased);
    const unsigned q4 = biased ^ 0x80808080u;  // the four q bytes
    const unsigned p1 = (unsigned)__builtin_amdgcn_mov_dpp((int)q4, 0xB1, 0xF, 0xF, false);  // lane ^ 1
    const unsigned p2 = (unsigned)__builtin_amdgcn_mov_dpp((int)q4, 0x4E, 0xF, 0xF, false);  // lane ^ 2
    const unsigned p3 = (unsigned)__builtin_amdgcn_mov_dpp((int)q4, 0x1B, 0xF, 0xF, false);  // lane ^ 3
    const unsigned word = __builtin_amdgcn_perm(p1, q4, sel_near) | __builtin_amdgcn_perm(p3, p2, sel_far);
    const unsigned partner = (unsigned)__builtin_amdgcn_mov_dpp((int)word, 0x4E, 0xF, 0xF, false);  // lane ^ 2
    const unsigned turned = __builtin_amdgcn_alignbit(word, word, rot);
    const unsigned split = (turned & nibbles) | (partner & ~nibbles);
    // Minus the chunk sums: the 16 float4 of chunk f / 16 sit in one 16-lane row.
    const int neg_sum = chunk_lane_sum(sdot4(q4, -1, 0));
    if (ALL || f < chunks * 16) {
      word_dst[k * (T / 4)] = (int)split;
      if ((tid & 15) == 0) sum_dst[k * (T / 16)] = neg_sum;
    }
    step(kc);
  });
  return scale;
}

// Byte offset of gemv_rows_kernel's 16-byte dump slot: past the q8 row and
// its chunk sums, 16-byte aligned.
__host__ __device__ constexpr int rows_dump_offset(int chunks) { return (chunks * (kChunk + 4) + 15) & ~15; }
constexpr int kRowsQuantLds = 64;  // QUANT, after the dump slot: the 8 waves' row maxima
constexpr int kRowsBlocksPerCu2 = 2;  // blocks per CU with two steps per row (one above)

// One step of a row pair in flight: the 16 weight bytes of the lane's chunk in
// its own row (w0) and in its partner's row (w1), and the group scale of the
// lane's own row.
struct RowStep {
  v4i32 w0, w1;
  int s;
};

// Rows of 2..8 steps (4097 <= K <= 32768 inputs, two blocks per CU at two
// steps, one above), 64 lanes per row, activation row in LDS (nibble-split).  Every lane keeps all STEPS steps of its row pair in
// flight (3*STEPS loads: 14 KB per wave at K=28672, 8 waves and 112 KB per
// CU) instead of the rolling pipeline's one or two, and refills a step with
// the same step of the wave's next row pair as soon as it is computed.
//
// All loads of the kernel are issued as inline assembly in a fixed order, so
// the number issued after any step's loads is a constant and the kernel
// waits for exactly that step.  A row pair's bias and residual base are
// loaded at the top of its own iteration, after its steps' weights, and
// consumed at its end: vmcnt(3*(STEPS-1) + 2) before every step (younger:
// the pair's later steps, its two side loads, the refills issued so far),
// vmcnt(3*STEPS) before the epilogue (younger: the STEPS refills).  A
// wave's last row pair issues no refills (its waits count only the pair's
// later steps and side loads), so no loads go out for rows past the end.  No value
// an asm load writes is carried across the loop's back edge except the
// step registers, which are rewritten in place (the compiler has no copy to
// make of them); a value carried across the edge can be copied by the
// compiler ahead of the wait that covers it.  Vector memory loads return in
// order, so a count that leaves only younger loads outstanding proves the
// step complete; stores only make the waits longer.  (Compiled loads would
// get compiler-placed waits, which at this depth drain every load in flight
// at loop joins.)  The activation row's loads (the q8 copy, or with QUANT the
// fp32 row the block quantizes itself) go out first, with the first step of
// weights behind them; the other steps of the first row pair go out between
// the pieces of the copy or of the quantization (see the prologue).  The
// build disassembles these kernels and checks every VGPR access against the
// loads in flight (asmcheck.py).  Lane layout and fp32 order are those of
// gemv_kernel (orc_gemv_pairs).
//
// MT = 2 (two pre-quantized tokens, the gemm_tile_* entry points' m = 2 on
// long rows): the block copies both tokens' rows into LDS and every step's
// weights feed one fmaf chain per token, each in the one-token kernel's order,
// so a token's outputs are those of its own GEMV.  Each step ends with the
// tokens' sums tied in registers before its refill loads go out; left free,
// the compiler finished the second token's products after the refill and kept
// copies of the step's weights (35 instead of 10 VGPRs per step, spills from
// six steps on, and register copies of refilled steps ahead of their waits).
template <int EPI, int STEPS, bool EXACT, bool QUANT, int MT = 1>
__global__ __launch_bounds__(512) void gemv_rows_kernel(GemvPtrs in, const uint8_t* __restrict__ packed,
                                                        const uint16_t* __restrict__ scales,
                                                        const float* __restrict__ bias, float* __restrict__ output,
                                                        int32_t* __restrict__ partials, GemvShape sh) {
  constexpr int kBlock = 512;  // one block of 8 waves per CU: up to 256 VGPRs for the steps in flight
  // int4 words of a q8 row per thread: a row of STEPS * 4096 inputs is STEPS * 256 of them (no
  // clamped duplicate loads: each load instruction costs the CU's memory pipeline).
  constexpr int kCopy = (STEPS * 256 + kBlock - 1) / kBlock;
  // Loads of a row pair besides its steps: the bias, and one residual base per
  // token where the epilogue adds to the output.
  constexpr bool kBase = EPI == kResidual;
  constexpr int kSide = 1 + (kBase ? MT : 0);
  static_assert(MT == 1 || (!QUANT && EPI != kPartials), "several tokens: pre-quantized rows and an output epilogue");
  extern __shared__ __align__(16) unsigned char lds_raw[];
  const int chunks = (sh.n + kChunk - 1) / kChunk;
  // Token t's copy: quad w of chunk u at lds_q(t)[w*C + u], then minus its chunk sums.
  const int token_bytes = rows_dump_offset(chunks);
  auto lds_q_of = [&](int t) { return reinterpret_cast<int4*>(lds_raw + t * token_bytes); };
  auto lds_x_of = [&](int t) { return reinterpret_cast<int*>(lds_raw + t * token_bytes + (size_t)chunks * kChunk); };
  int4* lds_q = lds_q_of(0);
  int* lds_x = lds_x_of(0);
  unsigned char* lds_dump = lds_raw + MT * token_bytes;
  const int4* gq = reinterpret_cast<const int4*>(in.q8_in);
  const int tid = threadIdx.x;
  const int sub = tid & 63;  // 64 lanes per row: lane = sub, one row slot per wave
  const int waves = gridDim.x * (kBlock / 64);
  const int words = chunks * 4;
  constexpr bool kScales = EPI != kPartials;  // the partials export passes no scales
  static_assert(!(QUANT && EPI == kPartials), "the partials export reads a pre-quantized row");
  float sx[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) sx[t] = 1.0f;
  if constexpr (!QUANT) {
#pragma unroll
    for (int t = 0; t < MT; ++t) sx[t] = kScales ? in.scale_in[t] : 1.0f;
  }

  // Loads that a layout does not need still go out, from the first bytes of
  // the packed matrix (the one operand every entry point passes), so that the
  // count of loads per step stays fixed.
  //
  // With EXACT (K a multiple of 4096) no chunk is clamped, so a row pair's
  // loads sit at fixed offsets from three bases: step s reads 1024*s bytes
  // past the lane's first weight bytes and 64*s bytes past its first scale.
  // The weight bases point 4096 bytes in, so the offsets of all 8 steps fit
  // the instruction's signed 13-bit field.
  constexpr int kMid = 4096;
  static_assert(STEPS <= 8, "step offsets -4096 .. 3072");
  struct PairBase {
    const uint8_t* w0;
    const uint8_t* w1;
    const void* s;
  };
  auto pair_base = [&](int row_pair) {
    PairBase b;
    const int r0 = min(row_pair * kRows, sh.rows - 1), r1 = min(row_pair * kRows + 1, sh.rows - 1);
    const int own = (sub & 1) ? r1 : r0;
    b.w0 = packed + (size_t)own * sh.row_bytes + sub * 16 + kMid;
    b.w1 = packed + (size_t)((sub & 1) ? r0 : r1) * sh.row_bytes + sub * 16 + kMid;
    b.s = kScales ? static_cast<const void*>(scales + (size_t)own * sh.groups + (sub >> 1))
                  : static_cast<const void*>(packed);
    return b;
  };
  auto issue_step = [&](RowStep& st, const PairBase& pb, int row_pair, auto step_c) {
    constexpr int step = decltype(step_c)::value;
    if constexpr (EXACT) {
      st.w0 = load_b128_at<step * 1024 - kMid>(pb.w0);
      st.w1 = load_b128_at<step * 1024 - kMid>(pb.w1);
      st.s = load_u16_at<step * 64>(pb.s);
    } else {
      const int u = min(step * 64 + sub, chunks - 1);
      const int r0 = min(row_pair * kRows, sh.rows - 1), r1 = min(row_pair * kRows + 1, sh.rows - 1);
      const int own = (sub & 1) ? r1 : r0;
      const uint8_t* p0 = packed + (size_t)own * sh.row_bytes + (size_t)u * 16;
      const uint8_t* p1 = packed + (size_t)((sub & 1) ? r0 : r1) * sh.row_bytes + (size_t)u * 16;
      const void* ps = kScales ? static_cast<const void*>(scales + (size_t)own * sh.groups + (u >> 1))
                               : static_cast<const void*>(packed);
      st.w0 = load_b128(p0);
      st.w1 = load_b128(p1);
      st.s = load_u16(ps);
    }
  };
  // Bias and residual bases (token t at output + t * out_stride) of the lane's own row.
  auto issue_side = [&](int row_pair, int& b, int (&base)[MT]) {
    const int own = min(row_pair * kRows + (sub & 1), sh.rows - 1);
    b = load_b32(bias != nullptr ? static_cast<const void*>(bias + own) : static_cast<const void*>(packed));
    if constexpr (kBase) {
#pragma unroll
      for (int t = 0; t < MT; ++t) base[t] = load_b32(output + (size_t)t * sh.out_stride + own);
    } else {
#pragma unroll
      for (int t = 0; t < MT; ++t) base[t] = 0;
    }
  };
  // The wait that covers the side loads, repeated per register group so that
  // every register it covers is tied to a wait instruction (repeating a wait
  // whose count is already reached costs one instruction).
  auto side_wait = [&](int& b, int (&base)[MT], auto count_c) {
    constexpr int count = decltype(count_c)::value;
    asm volatile("s_waitcnt vmcnt(%1)" : "+v"(b) : "n"(count) : "memory");
    if constexpr (kBase) {
#pragma unroll
      for (int t = 0; t < MT; ++t) asm volatile("s_waitcnt vmcnt(%1)" : "+v"(base[t]) : "n"(count) : "memory");
    }
  };

  RowStep st[STEPS];
  int it;
  PairBase pb;
  // The activation row goes out first, with one step of weights behind it;
  // the other steps are issued one by one between the pieces of the copy or
  // of the quantization.  (Memory serves the row's loads among the weight
  // bytes in flight, not ahead of them: with a row pair's 14 KB per wave
  // already requested, 28 KB of q8 take about 3 us to arrive instead of
  // 0.5 us.  And a wave that issues many loads at once stalls until the
  // CU's memory pipeline accepts them, so work placed after a burst of loads
  // waits for it.)
  it = __builtin_amdgcn_readfirstlane(blockIdx.x * (kBlock / 64) + (tid >> 6));  // wave-uniform
  pb = pair_base(it);
  if constexpr (!QUANT) {
    // Token t's q8 row: chunks * 64 bytes at q8_in + t * chunks * 64, its
    // chunk sums at xsum_in + t * chunks.
    v4i32 qv[MT][kCopy];
    int xv[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) {
#pragma unroll
      for (int k = 0; k < kCopy; ++k) qv[t][k] = load_b128(gq + (size_t)t * words + min(k * kBlock + tid, words - 1));
      xv[t] = load_b32(in.xsum_in + (size_t)t * chunks + min(tid, chunks - 1));
    }
    issue_step(st[0], pb, it, std::integral_constant<int, 0>{});
    // The copy's loads are older than step 0's three.
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      asm volatile("s_waitcnt vmcnt(3)" : "+v"(xv[t]) : : "memory");
#pragma unroll
      for (int k = 0; k < kCopy; ++k) asm volatile("s_waitcnt vmcnt(3)" : "+v"(qv[t][k]) : : "memory");
    }
    int4* dump = reinterpret_cast<int4*>(lds_dump);
    static_for<kCopy>([&](auto kc) {
      constexpr int k = decltype(kc)::value;
      const int e = k * kBlock + tid;
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        // Caller q8 quads are split here, once per block (the scratch's arrive split).
        const int4 quad = __builtin_bit_cast(int4, qv[t][k]);
        const int4 stored = sh.split ? quad : split_quad(quad);
        *(e < words ? lds_q_of(t) + (e & 3) * chunks + (e >> 2) : dump) = stored;
      }
      if constexpr (k + 1 < STEPS) issue_step(st[k + 1], pb, it, std::integral_constant<int, k + 1>{});
    });
#pragma unroll
    for (int t = 0; t < MT; ++t)  // minus the chunk sums
      *(tid < chunks ? lds_x_of(t) + tid : reinterpret_cast<int*>(dump)) = -xv[t];
    static_for<STEPS>([&](auto sc) {
      if constexpr (decltype(sc)::value > kCopy) issue_step(st[sc], pb, it, sc);
    });
  } else {
    // The block quantizes the PLAIN row itself (quantize_row_split), issuing
    // one step of weights after every second float4 of the row.
    constexpr int kX = 2 * STEPS;  // float4 per thread: rows of STEPS * 4096 inputs
    constexpr int kMid = STEPS <= 2 ? STEPS - 1 : 0;
    v4f32 xv[kX];
    const v4f32* x4 = reinterpret_cast<const v4f32*>(in.input);
    const int n4 = sh.n >> 2;
#pragma unroll
    for (int k = 0; k < kX; ++k) xv[k] = load_f128(x4 + min(k * kBlock + tid, n4 - 1));
    issue_step(st[0], pb, it, std::integral_constant<int, 0>{});
    // The row's loads are older than step 0's three.
#pragma unroll
    for (int k = 0; k < kX; ++k) asm volatile("s_waitcnt vmcnt(3)" : "+v"(xv[k]) : : "memory");
    // Rows of two steps: step 1 goes out as soon as the row is in.  Longer
    // rows: steps 1.. go out one after every second float4 of the
    // quantization (all at once, they stall the wave until the memory
    // pipeline takes them and hold up the quantization: 16.5 us against
    // 16.8-18.1 us per K=28672 -> N=8192 call with 1, 2, 3 or 5 of them up
    // front).
    static_for<kMid + 1>([&](auto sc) {
      if constexpr (decltype(sc)::value > 0) issue_step(st[sc], pb, it, sc);
    });
    float* slots = reinterpret_cast<float*>(lds_dump + 16);
    sx[0] = quantize_row_split<kBlock, kX, EXACT>(xv, sh.n, chunks, reinterpret_cast<int*>(lds_q), lds_x, slots,
                                                   [&](auto kc) {
      constexpr int k = decltype(kc)::value;
      if constexpr (k % 2 == 0 && k / 2 + kMid + 1 < STEPS)
        issue_step(st[k / 2 + kMid + 1], pb, it, std::integral_constant<int, k / 2 + kMid + 1>{});
    });
  }
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");

  const int4 qr_unused[1][4] = {};
  const int xr_unused[1] = {0};
  // The same weights against each token's copy, one fmaf chain per token.
  auto compute = [&](const RowStep& step, float (&acc)[MT], int row0, auto step_c) {
    Step<1> view;
    view.w[0][0] = __builtin_bit_cast(uint4, step.w0);
    view.w[0][1] = __builtin_bit_cast(uint4, step.w1);
    view.s[0] = (uint16_t)step.s;
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      // The token's copy is addressed through an opaque offset: its quads are
      // the same at every row pair, and left visible the compiler keeps them
      // in registers across the loop (16 VGPRs per step and token).
      int toff = t * token_bytes;
      if constexpr (MT > 1) asm volatile("" : "+v"(toff));
      const int4* q = reinterpret_cast<const int4*>(lds_raw + toff);
      const int* x = reinterpret_cast<const int*>(lds_raw + toff + chunks * kChunk);
      compute_step<EPI, 1, false, 64, EXACT, true, true>(view, qr_unused, xr_unused, q, x, acc[t], partials, sh, row0,
                                                       decltype(step_c)::value, sub, chunks);
    }
    if constexpr (MT > 1) {
      // Every token's sum of this step is complete before the step's
      // registers are refilled (otherwise the compiler may finish the later
      // tokens after the refill loads and keep copies of the step's weights).
#pragma unroll
      for (int t = 0; t < MT; ++t) asm volatile("" : "+v"(acc[t]));
    }
  };
  auto epilogue = [&](float (&acc)[MT], int row0, int b_side, const int (&base_side)[MT]) {
    if constexpr (EPI != kPartials) {
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        const float total = pair_tree_sum(acc[t], 64);
        const int row = row0 + (sub & 1);
        float y = total * 0.0625f * sx[t];  // the folded sums carry chunk_code_dot's factor 16
        if (bias != nullptr) y = y + __int_as_float(b_side);
        float* out = output + (size_t)t * sh.out_stride;
        if constexpr (EPI == kSiluPair) {
          const float up = __int_as_float(pair_swap(__float_as_int(y)));
          if (sub == 0 && row + 1 < sh.rows) out[row >> 1] = ivo_silu(y) * up;
        } else if (sub < 2 && row < sh.rows) {
          if constexpr (EPI == kStore) out[row] = y;
          else out[row] = __int_as_float(base_side[t]) + y;
        }
      }
    }
  };
  if (it < sh.iters) {
    // Steady state: each computed step is refilled with the same step of the wave's next row pair.
    while (it + waves < sh.iters) {
      const int row0 = it * kRows;
      const int it_next = it + waves;
      // This row pair's bias and residual bases, younger than its steps' weights.
      int b_side, base_side[MT];
      issue_side(it, b_side, base_side);
      pb = pair_base(it_next);
      float acc[MT];
#pragma unroll
      for (int t = 0; t < MT; ++t) acc[t] = 0.0f;
      static_for<STEPS>([&](auto s) {
        asm volatile("s_waitcnt vmcnt(%3)"
                     : "+v"(st[s].w0), "+v"(st[s].w1), "+v"(st[s].s)
                     : "n"(3 * (STEPS - 1) + kSide)
                     : "memory");
        compute(st[s], acc, row0, s);
        issue_step(st[s], pb, it_next, s);
        __builtin_amdgcn_sched_barrier(0);
      });
      // Younger than the side loads: the STEPS refills of the next row pair.
      side_wait(b_side, base_side, std::integral_constant<int, 3 * STEPS>{});
      epilogue(acc, row0, b_side, base_side);
      it = it_next;
    }
    // The wave's last row pair: no refills, so fewer loads are younger than each step.
    const int row0 = it * kRows;
    int b_side, base_side[MT];
    issue_side(it, b_side, base_side);
    float acc[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[t] = 0.0f;
    static_for<STEPS>([&](auto s) {
      asm volatile("s_waitcnt vmcnt(%3)"
                   : "+v"(st[s].w0), "+v"(st[s].w1), "+v"(st[s].s)
                   : "n"(3 * (STEPS - 1 - decltype(s)::value) + kSide)
                   : "memory");
      compute(st[s], acc, row0, s);
      __builtin_amdgcn_sched_barrier(0);
    });
    side_wait(b_side, base_side, std::integral_constant<int, 0>{});
    epilogue(acc, row0, b_side, base_side);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // a wave with no row pair still has its first loads out
}

template <int MODE, int EPI, bool FUSED, int NJ, int LANES, bool EXACT, bool ROLL>
void launch_one(hipStream_t stream, const GemvPtrs& p, const GemvArgs& a, const GemvShape& sh, int blocks,
                size_t lds) {
  hipLaunchKernelGGL((gemv_kernel<MODE, EPI, FUSED, NJ, LANES, EXACT, ROLL>), dim3(blocks),
                     dim3(block_threads<ROLL>()), lds,
                     stream, p, a.packed, a.scales, a.bias, a.output, a.partials, sh);
}

// Compiled layouts: 64 lanes per row (rows of more than 32 chunks) with or
// without dead lanes, and any narrower power of two (one step) likewise.
// Returns false when the plan asks for a layout that is not compiled.
template <int MODE, int EPI, bool FUSED, int NJ, bool ROLL>
bool launch_layout(hipStream_t stream, const GemvPtrs& p, const GemvArgs& a, const GemvShape& sh, int blocks,
                   size_t lds) {
  if (sh.lanes == 64) {
    if (sh.exact) launch_one<MODE, EPI, FUSED, NJ, 64, true, ROLL>(stream, p, a, sh, blocks, lds);
    else launch_one<MODE, EPI, FUSED, NJ, 64, false, ROLL>(stream, p, a, sh, blocks, lds);
    return true;
  } else if constexpr (NJ == 1 && !ROLL) {
    if (sh.exact) launch_one<MODE, EPI, FUSED, 1, 0, true, false>(stream, p, a, sh, blocks, lds);
    else launch_one<MODE, EPI, FUSED, 1, 0, false, false>(stream, p, a, sh, blocks, lds);
    return true;
  }
  return false;
}

template <int EPI, int STEPS, bool QUANT>
void launch_rows_as(hipStream_t stream, const GemvPtrs& p, const GemvArgs& a, const GemvShape& sh, int blocks,
                    size_t lds) {
  if (sh.exact)
    hipLaunchKernelGGL((gemv_rows_kernel<EPI, STEPS, true, QUANT>), dim3(blocks), dim3(512), lds, stream, p, a.packed,
                       a.scales, a.bias, a.output, a.partials, sh);
  else
    hipLaunchKernelGGL((gemv_rows_kernel<EPI, STEPS, false, QUANT>), dim3(blocks), dim3(512), lds, stream, p,
                       a.packed, a.scales, a.bias, a.output, a.partials, sh);
}

template <int EPI, int STEPS>
void launch_rows(hipStream_t stream, const GemvPtrs& p, const GemvArgs& a, const GemvShape& sh, int /*blocks*/,
                 size_t /*lds*/, bool quant) {
  const int cus = device_cus();
  // Two steps per row leave room for two blocks per CU (more bytes in flight).
  const int cap = (STEPS == 2 ? kRowsBlocksPerCu2 : 1) * cus;
  const int blocks = ceil_div(sh.iters, 8) < cap ? ceil_div(sh.iters, 8) : cap;
  const size_t lds = (size_t)rows_dump_offset((sh.n + kChunk - 1) / kChunk) + 16;
  if constexpr (EPI != kPartials) {
    if (quant) {
      launch_rows_as<EPI, STEPS, true>(stream, p, a, sh, blocks, lds + kRowsQuantLds);
      return;
    }
  }
  launch_rows_as<EPI, STEPS, false>(stream, p, a, sh, blocks, lds);
}

// Several tokens through the long-row kernel (pre-quantized rows): the same
// grid, MT copies of the activations in LDS.
template <int EPI, int STEPS, int MT>
void launch_rows_tokens(hipStream_t stream, const GemvPtrs& p, const GemvArgs& a, const GemvShape& sh) {
  const int cus = device_cus();
  const int cap = (STEPS == 2 ? kRowsBlocksPerCu2 : 1) * cus;
  const int blocks = ceil_div(sh.iters, 8) < cap ? ceil_div(sh.iters, 8) : cap;
  const size_t lds = (size_t)MT * rows_dump_offset((sh.n + kChunk - 1) / kChunk) + 16;
  if (sh.exact)
    hipLaunchKernelGGL((gemv_rows_kernel<EPI, STEPS, true, false, MT>), dim3(blocks), dim3(512), lds, stream, p,
                       a.packed, a.scales, a.bias, a.output, a.partials, sh);
  else
    hipLaunchKernelGGL((gemv_rows_kernel<EPI, STEPS, false, false, MT>), dim3(blocks), dim3(512), lds, stream, p,
                       a.packed, a.scales, a.bias, a.output, a.partials, sh);
}

template <int EPI, int MT>
void launch_tokens_steps(hipStream_t stream, const GemvPtrs& p, const GemvArgs& a, const GemvShape& sh, int steps) {
  switch (steps) {
    case 2: launch_rows_tokens<EPI, 2, MT>(stream, p, a, sh); break;
    case 3: launch_rows_tokens<EPI, 3, MT>(stream, p, a, sh); break;
    case 4: launch_rows_tokens<EPI, 4, MT>(stream, p, a, sh); break;
    case 5: launch_rows_tokens<EPI, 5, MT>(stream, p, a, sh); break;
    case 6: launch_rows_tokens<EPI, 6, MT>(stream, p, a, sh); break;
    case 7: launch_rows_tokens<EPI, 7, MT>(stream, p, a, sh); break;
    default: launch_rows_tokens<EPI, 8, MT>(stream, p, a, sh); break;
  }
}

// Steps per pipeline item of the rolling layout (rows of more than 8 steps):
// the largest of 4, 2, 1 that divides the row's steps (no dead steps).
int steps_per_item(int steps) {
  if (steps % 4 == 0) return 4;
  if (steps % 2 == 0) return 2;
  return 1;
}

template <int MODE, int EPI, bool FUSED>
hipError_t launch_nj(hipStream_t stream, const GemvPtrs& p, const GemvArgs& a, const GemvShape& sh, int blocks,
                     size_t lds, int steps, bool quant = false) {
  bool launched = false;
  if (steps <= 1) {  // one step per row: q8 in registers
    launched = launch_layout<MODE, EPI, FUSED, 1, false>(stream, p, a, sh, blocks, lds);
  } else if constexpr (!FUSED) {
    // Rows of more than one step have 64 lanes (lanes < 64 span a row in one step).
    if (sh.lanes == 64 && steps <= 8) {
      switch (steps) {
        case 2: launch_rows<EPI, 2>(stream, p, a, sh, blocks, lds, quant); break;
        case 3: launch_rows<EPI, 3>(stream, p, a, sh, blocks, lds, quant); break;
        case 4: launch_rows<EPI, 4>(stream, p, a, sh, blocks, lds, quant); break;
        case 5: launch_rows<EPI, 5>(stream, p, a, sh, blocks, lds, quant); break;
        case 6: launch_rows<EPI, 6>(stream, p, a, sh, blocks, lds, quant); break;
        case 7: launch_rows<EPI, 7>(stream, p, a, sh, blocks, lds, quant); break;
        default: launch_rows<EPI, 8>(stream, p, a, sh, blocks, lds, quant); break;
      }
      return hipGetLastError();
    }
    const int nj = steps_per_item(steps);
    if (nj == 4) launched = launch_layout<MODE, EPI, FUSED, 4, true>(stream, p, a, sh, blocks, lds);
    else if (nj == 2) launched = launch_layout<MODE, EPI, FUSED, 2, true>(stream, p, a, sh, blocks, lds);
    else launched = launch_layout<MODE, EPI, FUSED, 1, true>(stream, p, a, sh, blocks, lds);
  }
  if (!launched) return hipErrorInvalidValue;
  return hipGetLastError();
}

template <int MODE>
hipError_t launch_fused(hipStream_t stream, const GemvPtrs& p, const GemvArgs& a, const GemvShape& sh, int blocks,
                        size_t lds) {
  switch (a.epi) {
    case kStore: return launch_nj<MODE, kStore, true>(stream, p, a, sh, blocks, lds, 1);
    case kResidual: return launch_nj<MODE, kResidual, true>(stream, p, a, sh, blocks, lds, 1);
    case kSiluPair: return launch_nj<MODE, kSiluPair, true>(stream, p, a, sh, blocks, lds, 1);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

int device_cus() {
  static int cached[64] = {0};
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= 64) return 256;
  if (cached[device] == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess || cus <= 0)
      cus = 256;
    cached[device] = cus;
  }
  return cached[device];
}

int gemv_fused_limit() { return kFusedLimit; }

bool gemv_prequant_applies(int n) { return n > 0 && (size_t)ceil_div(n, kChunk) * (kChunk + 4) <= (size_t)kMaxLdsBytes; }

void gemv_plan(int rows, int n, int* lanes, int* rows_per_lane) {
  (void)rows;
  const int chunks = ceil_div(n, kChunk);
  int l = 2;
  while (l < 64 && l < chunks) l <<= 1;
  *lanes = l;
  *rows_per_lane = kRows;
}

hipError_t launch_gemv(hipStream_t stream, const GemvArgs& in) {
  if (in.rows <= 0) return hipSuccess;
  GemvArgs a = in;
  const int chunks = ceil_div(a.n, kChunk);
  const bool fused = a.q8_in == nullptr && a.n <= kFusedLimit;
  const size_t lds = (size_t)chunks * (kChunk + 4);  // unused by the non-rolling pre-quantized layouts
  if (lds > (size_t)kMaxLdsBytes) return hipErrorInvalidValue;
  int lanes, rows_per_lane;
  gemv_plan(a.rows, a.n, &lanes, &rows_per_lane);
  GemvShape sh;
  sh.rows = a.rows;
  sh.n = a.n;
  sh.row_bytes = a.row_bytes;
  sh.groups = a.groups;
  sh.splits = a.splits;
  sh.head_dim = a.head_dim;
  sh.eps = a.eps;
  sh.lanes = lanes;
  sh.lane_shift = __builtin_ctz((unsigned)lanes);
  sh.iters = ceil_div(a.rows, (64 / lanes) * rows_per_lane);
  const int steps = ceil_div(chunks, lanes);
  // Dead lanes exist when the last step is partial (items never hold dead steps).
  sh.exact = chunks % lanes == 0;
  sh.split = 0;
  sh.out_stride = 0;
  const int cus = device_cus();
  const bool roll = !fused && steps > 8;  // the rolling layout (2..8 steps: the long-row kernel sizes its own grid)
  int blocks = ceil_div(sh.iters, (roll ? block_threads<true>() : kThreads) / 64);
  const int cap = (fused ? 2 : roll ? 1 : kBlocksPerCu) * cus;
  if (blocks > cap) blocks = cap;

  if (fused) {
    if (a.epi == kPartials) return hipErrorInvalidValue;
    const GemvPtrs p{a.input, a.aux, nullptr, nullptr, nullptr};
    switch (a.mode) {
      case kPlain: return launch_fused<kPlain>(stream, p, a, sh, blocks, lds);
      case kNorm: return launch_fused<kNorm>(stream, p, a, sh, blocks, lds);
      case kAttn: return launch_fused<kAttn>(stream, p, a, sh, blocks, lds);
      default: return hipErrorInvalidValue;
    }
  }
  // A 16-byte aligned PLAIN row of 2..8 steps is quantized by every block of
  // the long-row kernel itself; other rows by the quantizer, into the
  // stream's scratch, in a launch of its own.
  const bool aligned = (a.n & 3) == 0 && (reinterpret_cast<uintptr_t>(a.input) & 15) == 0;
  const bool quant = a.q8_in == nullptr && a.mode == kPlain && aligned && lanes == 64 && steps >= 2 && steps <= 8;
  if (a.q8_in == nullptr && !quant) {
    Scratch* scratch = a.work;
    if (scratch == nullptr) {
      hipError_t status = scratch_for_stream(stream, &scratch);
      if (status != hipSuccess) return status;
    }
    if (chunks > scratch->capacity_chunks) return hipErrorInvalidValue;
    // The scratch row is the GEMV's alone: it is written nibble-split for the 4-bit dots.
    sh.split = 1;
    QuantArgs q{a.mode, a.input, a.n, a.aux, a.n, a.eps, a.splits, a.head_dim, 1, scratch->q8, scratch->xsum,
                scratch->scale, true};
    const hipError_t status = launch_quantize(stream, q);
    if (status != hipSuccess) return status;
    a.q8_in = scratch->q8;
    a.xsum_in = scratch->xsum;
    a.scale_in = scratch->scale;
  }
  const GemvPtrs p = quant ? GemvPtrs{a.input, nullptr, nullptr, nullptr, nullptr}
                           : GemvPtrs{nullptr, nullptr, a.q8_in, a.xsum_in, a.scale_in};
  switch (a.epi) {
    case kStore: return launch_nj<kPlain, kStore, false>(stream, p, a, sh, blocks, lds, steps, quant);
    case kResidual: return launch_nj<kPlain, kResidual, false>(stream, p, a, sh, blocks, lds, steps, quant);
    case kSiluPair: return launch_nj<kPlain, kSiluPair, false>(stream, p, a, sh, blocks, lds, steps, quant);
    case kPartials: return launch_nj<kPlain, kPartials, false>(stream, p, a, sh, blocks, lds, steps, quant);
    default: return hipErrorInvalidValue;
  }
}

bool gemv_tokens_apply(int m, int n) {
  if (m < 2 || m > kGemvTokensMax || n <= 64 * kChunk) return false;
  const int chunks = ceil_div(n, kChunk);
  return ceil_div(chunks, 64) <= 8 && (size_t)m * rows_dump_offset(chunks) + 16 <= (size_t)max_lds_per_block();
}

hipError_t launch_gemv_tokens(hipStream_t stream, const GemvArgs& a, int m, int out_stride) {
  if (a.rows <= 0) return hipSuccess;
  if (!gemv_tokens_apply(m, a.n) || a.q8_in == nullptr || a.xsum_in == nullptr || a.scale_in == nullptr)
    return hipErrorInvalidValue;
  const int chunks = ceil_div(a.n, kChunk);
  int lanes, rows_per_lane;
  gemv_plan(a.rows, a.n, &lanes, &rows_per_lane);
  GemvShape sh{};
  sh.rows = a.rows;
  sh.n = a.n;
  sh.row_bytes = a.row_bytes;
  sh.groups = a.groups;
  sh.splits = 1;
  sh.head_dim = a.head_dim;
  sh.lanes = lanes;
  sh.lane_shift = __builtin_ctz((unsigned)lanes);
  sh.iters = ceil_div(a.rows, (64 / lanes) * rows_per_lane);
  sh.exact = chunks % lanes == 0;
  sh.split = 0;
  sh.out_stride = out_stride;
  const int steps = ceil_div(chunks, lanes);
  const GemvPtrs p{nullptr, nullptr, a.q8_in, a.xsum_in, a.scale_in};
  auto go = [&](auto epi_c) -> hipError_t {
    constexpr int EPI = decltype(epi_c)::value;
    static_assert(kGemvTokensMax == 2, "one token count compiled");
    launch_tokens_steps<EPI, 2>(stream, p, a, sh, steps);
    return hipGetLastError();
  };
  switch (a.epi) {
    case kStore: return go(std::integral_constant<int, kStore>{});
    case kResidual: return go(std::integral_constant<int, kResidual>{});
    case kSiluPair: return go(std::integral_constant<int, kSiluPair>{});
    default: return hipErrorInvalidValue;
  }
}

}  // namespace ivo
