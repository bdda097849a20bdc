// Device-side building blocks shared by the ternary kernels (gfx950, wave64).
//
// Packed weights (reference format, quantization.py:10-18): row r of a
// matrix holds ceil(K/4) bytes padded to a multiple of 16 (row_bytes); byte b
// carries inputs 4b..4b+3, input 4b+k in bits 2k..2k+1 as code = w + 1 with
// w in {-1, 0, +1}.  One fp16 scale per 128 inputs, scales[r * groups + g].
//
// Activation scratch ("q8 layout", private to this library): token row t
// holds C = ceil(K/64) chunks of 64 int8 (t * C * 64), zero padded past K.
// Inside chunk u, the 16-byte quad w covers inputs 64u+16w .. 64u+16w+15 and
// its 32-bit word k holds inputs {16w+k, 16w+4+k, 16w+8+k, 16w+12+k}, so
// (packed_word >> 2k) & 0x03030303 lines up byte for byte with word k.
// xsum[t * C + u] is the int32 sum of chunk u; scale[t] the fp32 token scale.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ivo {

constexpr int kThreads = 256;  // every kernel here runs 256-thread blocks (4 waves)
constexpr int kChunk = 64;
constexpr int kGroup = 128;
constexpr unsigned kLow2 = 0x03030303u;

enum Mode : int { kPlain = 0, kNorm = 1, kAttn = 2 };
enum Epi : int { kStore = 0, kResidual = 1, kSiluPair = 2, kPartials = 3 };

constexpr unsigned kSignedLut = 0x000100FFu;  // v_perm table: code 0 -> -1, 1 -> 0, 2 -> +1

// Code field k (inputs 4b + k of bytes b = 0..3) of a packed word as four
// signed int8 weights (-1, 0, +1): one v_perm_b32 table lookup per four codes.
__device__ __forceinline__ unsigned signed_codes(unsigned w, int k) {
  return __builtin_amdgcn_perm(0u, kSignedLut, (w >> (2 * k)) & kLow2);
}

__device__ __forceinline__ float h2f(uint16_t bits) {
  _Float16 h;
  __builtin_memcpy(&h, &bits, 2);
  return (float)h;
}

// exp(x): Cody-Waite reduction x = n*ln2 + r, degree-7 Taylor polynomial of
// e^r in Horner form, scaling by 2^n in two exact steps.  Every operation is
// an explicit IEEE fp32 op, so the CPU oracle reproduces it bit for bit.
__device__ __forceinline__ float ivo_expf(float x) {
  if (x != x) return x;
  if (x > 88.72283935546875f) return __builtin_inff();
  if (x < -103.97208404541015625f) return 0.0f;
  const float n = __builtin_rintf(x * 1.44269502162933349609375f);
  float r = __builtin_fmaf(n, -0.693145751953125f, x);
  r = __builtin_fmaf(n, -1.428606765330187045e-06f, r);
  float p = 1.9841270113829523e-04f;
  p = __builtin_fmaf(p, r, 1.3888889225199819e-03f);
  p = __builtin_fmaf(p, r, 8.3333337679505348e-03f);
  p = __builtin_fmaf(p, r, 4.1666667908430099e-02f);
  p = __builtin_fmaf(p, r, 1.6666667163372040e-01f);
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  const int ni = (int)n;
  const int n1 = ni / 2, n2 = ni - n1;
  const float s1 = __int_as_float((n1 + 127) << 23);
  const float s2 = __int_as_float((n2 + 127) << 23);
  return (p * s1) * s2;
}

__device__ __forceinline__ float ivo_silu(float x) { return x / (1.0f + ivo_expf(-x)); }

__device__ __forceinline__ int sdot4(unsigned a, int b, int c) {
  return __builtin_amdgcn_sdot4((int)a, b, c, false);
}

// Sum over one 64-input chunk of code * q, times 16 (chunk_code_dot): 16
// packed words against 16 q8 words.
// Each packed word w holds 16 codes as four byte-wise 2-bit fields; instead of
// shifting every field down (7 ops), the fields are isolated in place with
// masks (w & 0x03, w & 0x0c, w & 0x30 per byte, and (w >> 2) & 0x30 for the
// top field: 5 ops), so the dot products see code, 4*code and 16*code.  Three
// accumulators keep those weights apart and are recombined as
// 16*a1 + 4*a4 + a16 = 16 * (sum of code * q): two shift-adds instead of two
// shifts and an add.  A float scaled by 16 rounds exactly like the unscaled
// value in every later product and sum (no overflow, and the magnitudes here
// never reach the subnormal range), so callers fold the scaled sums and drop
// the factor once per output.
__device__ __forceinline__ int word_code_dot(unsigned w, int4 q, int& a1, int& a4, int& a16) {
  a1 = sdot4(w & 0x03030303u, q.x, a1);
  a4 = sdot4(w & 0x0c0c0c0cu, q.y, a4);
  a16 = sdot4(w & 0x30303030u, q.z, a16);
  a16 = sdot4((w >> 2) & 0x30303030u, q.w, a16);
  return 0;
}

// v_dot4_i32_i8 in its three-operand form, seeded from c or from zero.  The
// compiler prefers v_dot4c, whose accumulator is also its destination, and so
// spends a v_mov per accumulator to seed it (four per row and chunk).
__device__ __forceinline__ int sdot4_seed(unsigned a, int b, int c) {
  int d;
  asm("v_dot4_i32_i8 %0, %1, %2, %3" : "=v"(d) : "v"(a), "v"(b), "v"(c));
  return d;
}
__device__ __forceinline__ int sdot4_zero(unsigned a, int b) {
  int d;
  asm("v_dot4_i32_i8 %0, %1, %2, 0" : "=v"(d) : "v"(a), "v"(b));
  return d;
}

// Nibble-split activations for 4-bit dot products.  A packed word W holds 16
// codes, input 4b + f of its 16 in field f of byte b; W & 0x33333333 keeps
// fields 0 and 2 of every byte as the nibbles 2b and 2b + 1, and
// (W >> 2) & 0x33333333 fields 1 and 3.  The matching activation words split
// each q into q = 16 * hi + lo (hi = q >> 4 in -8..7, lo = q & 15): word 0 of a
// split quad holds hi of inputs 4b and 4b + 2 as nibbles 2b and 2b + 1, word 1
// hi of inputs 4b + 1 and 4b + 3, words 2 and 3 the lo nibbles likewise.  In q8
// terms (word k of a quad holds input 4b + k at byte b), word 0 = hi nibbles of
// q8 words 0 and 2, word 1 = of words 1 and 3, words 2 and 3 the lo nibbles:
// word k of the split quad, from q8 word k and the word of lane k ^ 2.
__device__ __forceinline__ unsigned split_quad_word(unsigned own, unsigned partner, int k) {
  const unsigned a = k < 2 ? own : partner;  // q8 word 0 or 1 (inputs 4b + 0 or 1)
  const unsigned b = k < 2 ? partner : own;  // q8 word 2 or 3 (inputs 4b + 2 or 3)
  return k < 2 ? ((a >> 4) & 0x0F0F0F0Fu) | (b & 0xF0F0F0F0u) : (a & 0x0F0F0F0Fu) | ((b << 4) & 0xF0F0F0F0u);
}

// The split form of a whole q8 quad (words 0..3), as split_quad_word gives it
// word by word.
__device__ __forceinline__ int4 split_quad(int4 q) {
  const unsigned w0 = (unsigned)q.x, w1 = (unsigned)q.y, w2 = (unsigned)q.z, w3 = (unsigned)q.w;
  return make_int4((int)(((w0 >> 4) & 0x0F0F0F0Fu) | (w2 & 0xF0F0F0F0u)),
                   (int)(((w1 >> 4) & 0x0F0F0F0Fu) | (w3 & 0xF0F0F0F0u)),
                   (int)((w0 & 0x0F0F0F0Fu) | ((w2 << 4) & 0xF0F0F0F0u)),
                   (int)((w1 & 0x0F0F0F0Fu) | ((w3 << 4) & 0xF0F0F0F0u)));
}

// v_dot8_i32_i4 seeded from zero and v_dot8_u32_u4 in its three-operand form.
__device__ __forceinline__ int sdot8_zero(unsigned a, unsigned b) {
  int d;
  asm("v_dot8_i32_i4 %0, %1, %2, 0" : "=v"(d) : "v"(a), "v"(b));
  return d;
}
__device__ __forceinline__ unsigned udot8_seed(unsigned a, unsigned b, unsigned c) {
  unsigned d;
  asm("v_dot8_u32_u4 %0, %1, %2, %3" : "=v"(d) : "v"(a), "v"(b), "v"(c));
  return d;
}
// Sum over one 64-input chunk of code * q plus acc, times 16, from the
// nibble-split activations (the value chunk_code_dot returns for the q8 form):
// per packed word two masks and a shift with the four 4-bit dot products, 7
// VALU against chunk_code_dot's 9.  The hi products (signed nibbles) and lo
// products (unsigned, seeded with acc) run in two accumulators; two
// shift-adds give 16 * (16 * sum(code * hi) + sum(code * lo) + acc), exact in
// int32 (the lo accumulator in unsigned arithmetic, modulo 2^32).
__device__ __forceinline__ int chunk_split_dot(const uint4 w, const int4 s0, const int4 s1, const int4 s2,
                                               const int4 s3, int acc) {
  const unsigned words[4] = {w.x, w.y, w.z, w.w};
  const int4 quads[4] = {s0, s1, s2, s3};
  int hi = 0;
  unsigned lo = (unsigned)acc;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const unsigned n0 = words[i] & 0x33333333u, n1 = (words[i] >> 2) & 0x33333333u;
    if (i == 0) {
      hi = sdot8_zero(n0, (unsigned)quads[i].x);
      lo = udot8_seed(n0, (unsigned)quads[i].z, lo);
    } else {
      hi = __builtin_amdgcn_sdot8((int)n0, quads[i].x, hi, false);
      lo = __builtin_amdgcn_udot8(n0, (unsigned)quads[i].z, lo, false);
    }
    hi = __builtin_amdgcn_sdot8((int)n1, quads[i].y, hi, false);
    lo = __builtin_amdgcn_udot8(n1, (unsigned)quads[i].w, lo, false);
  }
  return (int)(((unsigned)hi << 8) + (lo << 4));
}

__device__ __forceinline__ int chunk_code_dot(const uint4 w, const int4 q0, const int4 q1, const int4 q2,
                                              const int4 q3, int acc) {
  int a1 = sdot4_seed(w.x & 0x03030303u, q0.x, acc);
  int a4 = sdot4_zero(w.x & 0x0c0c0c0cu, q0.y);
  int a16 = sdot4_zero(w.x & 0x30303030u, q0.z);
  a16 = sdot4((w.x >> 2) & 0x30303030u, q0.w, a16);
  word_code_dot(w.y, q1, a1, a4, a16);
  word_code_dot(w.z, q2, a1, a4, a16);
  word_code_dot(w.w, q3, a1, a4, a16);
  // Two shift-adds: the empty asm keeps the compiler from merging them into
  // two shifts and a three-way add.
  int t = (a4 << 2) + a16;
  asm("" : "+v"(t));
  return (a1 << 4) + t;
}

// Lane value of the partner in the same lane pair (quad_perm [1,0,3,2]).
__device__ __forceinline__ int pair_swap(int v) { return __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false); }

// Lane L reads lane L + N of its 16-lane row (lanes past the row read 0).
template <int N>
__device__ __forceinline__ int row_shl_int(int v) {
  static_assert(N >= 1 && N <= 15, "DPP row_shl 1..15");
  return __builtin_amdgcn_mov_dpp(v, 0x100 + N, 0xF, 0xF, true);
}
template <int N>
__device__ __forceinline__ float row_shl(float v) {
  return __int_as_float(row_shl_int<N>(__float_as_int(v)));
}

// Lanes of even 16-lane rows read the same lane of the next row; lanes of the
// lower 32 read the same lane of the upper 32 (v_permlane16/32_swap).
__device__ __forceinline__ float row_swap16(float v) {
  const unsigned u = __float_as_uint(v);
  return __uint_as_float(__builtin_amdgcn_permlane16_swap(u, u, false, false)[1]);
}
__device__ __forceinline__ float row_swap32(float v) {
  const unsigned u = __float_as_uint(v);
  return __uint_as_float(__builtin_amdgcn_permlane32_swap(u, u, false, false)[1]);
}

// The xor butterfly over lane pairs, acc += acc of lane L ^ o for o = 2, 4, ..
// lanes/2, evaluated for the lanes that finish a row (L mod lanes < 2) only:
// at stage o such a lane, and every lane its result depends on, has bit o
// clear, so L ^ o = L + o and adding lane L + o is the same operand pair in
// the same order.  DPP row shifts and row swaps instead of LDS permutes.
__device__ __forceinline__ float pair_tree_sum(float acc, int lanes) {
  if (lanes > 2) acc = acc + row_shl<2>(acc);
  if (lanes > 4) acc = acc + row_shl<4>(acc);
  if (lanes > 8) acc = acc + row_shl<8>(acc);
  if (lanes > 16) acc = acc + row_swap16(acc);
  if (lanes > 32) acc = acc + row_swap32(acc);
  return acc;
}

// Max over the wave, complete in lane 0 only (the other lanes hold partial
// maxima): lane 0 at each stage reads a lane that has already folded its
// share, as in pair_tree_sum.  The callers reduce absolute values (no -0),
// whose fmaxf does not depend on the order.
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, row_shl<1>(v));
  v = fmaxf(v, row_shl<2>(v));
  v = fmaxf(v, row_shl<4>(v));
  v = fmaxf(v, row_shl<8>(v));
  v = fmaxf(v, row_swap16(v));
  v = fmaxf(v, row_swap32(v));
  return v;
}

// Block-wide max over the 4 waves; every thread gets the result.  A block
// reduces at most once into the same slots (one token row per block), so
// no barrier follows the slot reads.
__device__ __forceinline__ float block_max(float v, float* slots) {
  v = wave_max(v);
  if ((threadIdx.x & 63) == 0) slots[threadIdx.x >> 6] = v;
  __syncthreads();
  return fmaxf(fmaxf(slots[0], slots[1]), fmaxf(slots[2], slots[3]));
}

// The reference kernel's reduction tree for a sum of squares over a 256-thread
// block (ternary.cu:157-170, :81-84, :101-109): per-thread fma partials over
// i = tid, tid+256, ... in order, xor butterfly inside each 32-lane half
// (offsets 16..1), then the eight half-wave totals added in order.  Loads go
// out in batches of kBatch independent reads (indices clamped, values past
// the row masked to zero, which leaves a non-negative fma chain unchanged).
constexpr int kBatch = 16;

// The block part of that tree, from each thread's fma partial.
// The butterfly (offsets 16, 8, .., 1, s + s of lane L ^ o) is needed in
// lanes 0 and 32 only: at stage o every lane their sums depend on is below o
// within its half, so L ^ o = L + o, the lane a DPP row shift (o < 16) or
// the row swap (o = 16) reads; same operands, same order.
__device__ __forceinline__ float tree_reduce(float s, float* slots) {
  const int tid = threadIdx.x;
  s = s + row_swap16(s);
  s = s + row_shl<8>(s);
  s = s + row_shl<4>(s);
  s = s + row_shl<2>(s);
  s = s + row_shl<1>(s);
  if ((tid & 31) == 0) slots[tid >> 5] = s;
  __syncthreads();
  float total = 0.0f;
  for (int w = 0; w < kThreads / 32; ++w) total = total + slots[w];
  return total;  // used once per block, like block_max: no barrier after the reads
}

template <int NB = kBatch>
__device__ __forceinline__ float tree_sum_squares(const float* __restrict__ x, int n, float* slots) {
  const int tid = threadIdx.x;
  float s = 0.0f;
  for (int base = 0; base < n; base += kThreads * NB) {
    float v[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) v[b] = x[min(base + b * kThreads + tid, n - 1)];
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const float value = base + b * kThreads + tid < n ? v[b] : 0.0f;
      s = __builtin_fmaf(value, value, s);
    }
  }
  return tree_reduce(s, slots);
}

// Source value of input i (ternary.cu:128-146 for the split-softmax merge).
template <int MODE>
__device__ __forceinline__ float source_value(const float* __restrict__ input, int i, int splits, int head_dim) {
  if constexpr (MODE == kAttn) {
    const int stride = head_dim + 2;
    const int head = i / head_dim, dim = i - head * head_dim;
    const float* base = input + (size_t)head * splits * stride;
    float peak = -__builtin_inff();
    for (int s = 0; s < splits; ++s) peak = fmaxf(peak, base[s * stride]);
    float total = 0.0f, value = 0.0f;
    for (int s = 0; s < splits; ++s) {
      const float* part = base + s * stride;
      const float weight = part[0] == -__builtin_inff() ? 0.0f : ivo_expf(part[0] - peak);
      total = __builtin_fmaf(weight, part[1], total);
      value = __builtin_fmaf(weight, part[2 + dim], value);
    }
    return value / total;
  } else {
    return input[i];
  }
}

// Everything a block needs to quantize one token row.
struct RowSource {
  const float* input;  // row start
  const float* aux;    // NORM weights (may be null otherwise)
  int n;
  float eps;
  int splits;
  int head_dim;
};

// Per-row prologue shared by all quantizing kernels: returns the token scale
// and, for NORM, sets inv_rms.  All 256 threads must call it.  amax is
// order-free, so its loads are clamped duplicates rather than masked, and a
// 16-byte aligned PLAIN row is read as float4.
template <int MODE, int NB = kBatch>
__device__ __forceinline__ float row_scale(const RowSource& src, float& inv_rms, float* slots) {
  const int tid = threadIdx.x;
  const int n = src.n;
  inv_rms = 1.0f;
  if constexpr (MODE == kNorm) {
    const float squares = tree_sum_squares<NB>(src.input, n, slots);
    inv_rms = 1.0f / __builtin_sqrtf(squares / (float)n + src.eps);
  }
  float amax = 0.0f;
  if constexpr (MODE == kAttn) {
    for (int i = tid; i < n; i += kThreads)
      amax = fmaxf(amax, fabsf(source_value<MODE>(src.input, i, src.splits, src.head_dim)));
  } else if (MODE == kPlain && (n & 3) == 0 && (((uintptr_t)src.input) & 15) == 0) {
    const float4* x4 = reinterpret_cast<const float4*>(src.input);
    const int n4 = n >> 2;
    for (int base = 0; base < n4; base += kThreads * NB) {
      float4 v[NB];
#pragma unroll
      for (int b = 0; b < NB; ++b) v[b] = x4[min(base + b * kThreads + tid, n4 - 1)];
#pragma unroll
      for (int b = 0; b < NB; ++b)
        amax = fmaxf(fmaxf(amax, fmaxf(fabsf(v[b].x), fabsf(v[b].y))), fmaxf(fabsf(v[b].z), fabsf(v[b].w)));
    }
  } else {
    for (int base = 0; base < n; base += kThreads * NB) {
      float v[NB];
      int idx[NB];
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        idx[b] = min(base + b * kThreads + tid, n - 1);
        v[b] = src.input[idx[b]];
      }
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        float value = v[b];
        if constexpr (MODE == kNorm) value = fminf(fmaxf(value * inv_rms, -8.0f), 8.0f) * src.aux[idx[b]];
        amax = fmaxf(amax, fabsf(value));
      }
    }
  }
  amax = block_max(amax, slots + 32);
  return fmaxf(amax / 127.0f, 1e-5f);
}

// q8 word (chunk u, quad w, field k) of one token: 4 quantized inputs.
template <int MODE>
__device__ __forceinline__ int quantize_word(const RowSource& src, int u, int w, int k, float inv_rms, float scale) {
  unsigned word = 0;
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    const int i = u * kChunk + w * 16 + 4 * b + k;
    int q = 0;
    if (i < src.n) {
      float v = source_value<MODE>(src.input, i, src.splits, src.head_dim);
      if constexpr (MODE == kNorm) v = fminf(fmaxf(v * inv_rms, -8.0f), 8.0f) * src.aux[i];
      q = (int)__builtin_rintf(v / scale);
    }
    word |= ((unsigned)q & 0xffu) << (8 * b);
  }
  return (int)word;
}

// Sum of the four int8 lanes of a word.
__device__ __forceinline__ int word_sum(int word) { return sdot4((unsigned)word, 0x01010101, 0); }

// Sum over the 16 consecutive lanes that hold one chunk's 16 words, complete
// in the first lane of each 16 (DPP row shifts; integer, so exact).
__device__ __forceinline__ int chunk_lane_sum(int v) {
  v += row_shl_int<1>(v);
  v += row_shl_int<2>(v);
  v += row_shl_int<4>(v);
  v += row_shl_int<8>(v);
  return v;
}

// Whole-block quantizer for one PLAIN or NORM token row of at most
// kThreads * NB inputs that reads the row once: thread t holds inputs
// t + 256*b in registers, which is also the reference's order for the
// sum-of-squares partials (so the fp32 result is the same as row_scale's).
// The q8 bytes go to LDS in the quad-planar layout (quad w of chunk u at
// 16-byte slot w*C + u; word k of a quad holds inputs 16w + k + 4b' at byte
// b'), zero past n up to C*64.  Returns the token scale.  All threads of the
// block call it; it ends with the block's writes not yet fenced.
struct NoLoads {
  __device__ void operator()() const {}
};

template <int MODE, int NB = kBatch, typename AfterLoads = NoLoads>
__device__ __forceinline__ float quantize_row_to_lds(const RowSource& src, int chunks, unsigned char* lds_q,
                                                     float* slots, AfterLoads after_loads = AfterLoads{}) {
  static_assert(MODE == kPlain || MODE == kNorm, "register path for PLAIN and NORM rows");
  static_assert(NB >= 1 && NB <= kBatch, "at most kBatch inputs per thread");
  const int tid = threadIdx.x;
  const int n = src.n;
  float v[NB], w[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    const int i = min(b * kThreads + tid, n - 1);
    v[b] = src.input[i];
    w[b] = MODE == kNorm ? src.aux[i] : 1.0f;
  }
  // Loads the caller issues behind the row's (loads return in order, so the
  // row's wait does not include them).
  __builtin_amdgcn_sched_barrier(0);
  after_loads();
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int b = 0; b < NB; ++b)
    if (b * kThreads + tid >= n) v[b] = 0.0f;
  float inv_rms = 1.0f;
  if constexpr (MODE == kNorm) {
    float s = 0.0f;
#pragma unroll
    for (int b = 0; b < NB; ++b) s = __builtin_fmaf(v[b], v[b], s);
    inv_rms = 1.0f / __builtin_sqrtf(tree_reduce(s, slots) / (float)n + src.eps);
  }
  float amax = 0.0f;
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    if constexpr (MODE == kNorm) v[b] = fminf(fmaxf(v[b] * inv_rms, -8.0f), 8.0f) * w[b];
    amax = fmaxf(amax, fabsf(v[b]));
  }
  amax = block_max(amax, slots + 32);
  const float scale = fmaxf(amax / 127.0f, 1e-5f);
  if constexpr (NB % 4 == 0) {
    // Thread t's input t + 256b is byte j = (t >> 2) & 3 of word (chunk
    // (t >> 6) + 4b, quad (t >> 4) & 3, field t & 3): the four bytes of a word
    // sit in lanes 4 apart within a 16-lane row, one per j.  For each four
    // batches b = 4c .. 4c + 3 the lanes rotate their four bytes by 4, 8 and
    // 12 lanes (DPP row_ror) and lane j keeps word b = 4c + j, whose byte i
    // is lane i's byte j; each rotated value's source is found by rotating
    // j the same way.  One word store instead of four byte stores.
    const int j = (tid >> 2) & 3;
    const int ja = __builtin_amdgcn_mov_dpp(j, 0x124, 0xF, 0xF, false);  // row_ror:4
    const int jb = __builtin_amdgcn_mov_dpp(j, 0x128, 0xF, 0xF, false);  // row_ror:8
    const int jc = __builtin_amdgcn_mov_dpp(j, 0x12C, 0xF, 0xF, false);  // row_ror:12
    // v_perm_b32 selectors: 0..3 pick the second operand's bytes, 4..7 the first's, 0x0C zero.
    auto place = [](unsigned sel, int position, unsigned source) {
      return (sel & ~(0xFFu << (8 * position))) | (source << (8 * position));
    };
    const unsigned sel_a = place(place(0x0C0C0C0Cu, j, (unsigned)j), ja, 4u + j);   // own byte j, lane ja's
    const unsigned sel_b = place(place(0x0C0C0C0Cu, jb, (unsigned)j), jc, 4u + j);  // lanes jb and jc
#pragma unroll
    for (int c = 0; c < NB / 4; ++c) {
      unsigned q4 = 0;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int i = (4 * c + e) * kThreads + tid;
        const int q = i < n ? (int)__builtin_rintf(v[4 * c + e] / scale) : 0;
        q4 |= ((unsigned)q & 0xffu) << (8 * e);
      }
      const unsigned pa = (unsigned)__builtin_amdgcn_mov_dpp((int)q4, 0x124, 0xF, 0xF, false);
      const unsigned pb = (unsigned)__builtin_amdgcn_mov_dpp((int)q4, 0x128, 0xF, 0xF, false);
      const unsigned pc = (unsigned)__builtin_amdgcn_mov_dpp((int)q4, 0x12C, 0xF, 0xF, false);
      const unsigned word = __builtin_amdgcn_perm(pa, q4, sel_a) | __builtin_amdgcn_perm(pc, pb, sel_b);
      const int u = (tid >> 6) + 4 * (4 * c + j);
      if (u < chunks)
        reinterpret_cast<unsigned*>(lds_q)[((((tid >> 4) & 3) * chunks + u) << 2) + (tid & 3)] = word;
    }
  } else {
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const int i = b * kThreads + tid;
      if (i < chunks * kChunk) {
        const int q = i < n ? (int)__builtin_rintf(v[b] / scale) : 0;
        const int u = i >> 6, r = i & 63;
        lds_q[((((r >> 4) & 3) * chunks + u) << 4) + ((r & 3) << 2) + ((r >> 2) & 3)] = (unsigned char)(q & 0xff);
      }
    }
  }
  return scale;
}

// quantize_row_to_lds for a 16-byte aligned PLAIN row of n inputs (n a
// multiple of 4): thread t holds float4 t + 256c (inputs 4(t + 256c) .. + 3),
// one load instruction per four inputs instead of one per input.  The
// absmax is order-free and every input is quantized on its own, so the q8
// bytes are the same.
template <int NB, typename AfterLoads = NoLoads>
__device__ __forceinline__ float quantize_plain_row4_to_lds(const RowSource& src, int chunks, unsigned char* lds_q,
                                                            float* slots, AfterLoads after_loads = AfterLoads{}) {
  static_assert(NB % 4 == 0 && NB <= kBatch, "whole float4 per thread");
  constexpr int NC = NB / 4;
  const int tid = threadIdx.x;
  const int n4 = src.n >> 2;
  const float4* x4 = reinterpret_cast<const float4*>(src.input);
  float4 v[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) v[c] = x4[min(c * kThreads + tid, n4 - 1)];
  __builtin_amdgcn_sched_barrier(0);
  after_loads();
  __builtin_amdgcn_sched_barrier(0);
  float amax = 0.0f;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    if (c * kThreads + tid >= n4) v[c] = float4{0.0f, 0.0f, 0.0f, 0.0f};
    amax = fmaxf(fmaxf(amax, fmaxf(fabsf(v[c].x), fabsf(v[c].y))), fmaxf(fabsf(v[c].z), fabsf(v[c].w)));
  }
  amax = block_max(amax, slots + 32);
  const float scale = fmaxf(amax / 127.0f, 1e-5f);
  // The four lanes 4g .. 4g + 3 hold the four float4 of one 16-input quad;
  // word k of the quad takes byte j of lane j's quantized float4 at byte j
  // (inputs 16w + k + 4j), so lane j forms word j with three DPP quad
  // permutations and two v_perm_b32 (the byte transpose of
  // quantize_row_split) and stores it whole.
  const int j = tid & 3;
  unsigned sel_near = 0x0C0C0C0Cu, sel_far = 0x0C0C0C0Cu;
  sel_near = (sel_near & ~(0xFFu << (8 * j))) | ((unsigned)j << (8 * j));
  sel_near = (sel_near & ~(0xFFu << (8 * (j ^ 1)))) | ((unsigned)(4 + j) << (8 * (j ^ 1)));
  sel_far = (sel_far & ~(0xFFu << (8 * (j ^ 2)))) | ((unsigned)j << (8 * (j ^ 2)));
  sel_far = (sel_far & ~(0xFFu << (8 * (j ^ 3)))) | ((unsigned)(4 + j) << (8 * (j ^ 3)));
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int f = c * kThreads + tid;
    const float e[4] = {v[c].x, v[c].y, v[c].z, v[c].w};
    unsigned q4 = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k)  // inputs past the row (f >= n4) hold zeros, which quantize to 0
      q4 |= ((unsigned)(int)__builtin_rintf(e[k] / scale) & 0xffu) << (8 * k);
    const unsigned p1 = (unsigned)__builtin_amdgcn_mov_dpp((int)q4, 0xB1, 0xF, 0xF, false);  // lane ^ 1
    const unsigned p2 = (unsigned)__builtin_amdgcn_mov_dpp((int)q4, 0x4E, 0xF, 0xF, false);  // lane ^ 2
    const unsigned p3 = (unsigned)__builtin_amdgcn_mov_dpp((int)q4, 0x1B, 0xF, 0xF, false);  // lane ^ 3
    const unsigned word = __builtin_amdgcn_perm(p1, q4, sel_near) | __builtin_amdgcn_perm(p3, p2, sel_far);
    if (f < chunks * 16) {  // whole quads: chunks * 16 is a multiple of 4
      const int g = f >> 2;  // quad g: chunk g >> 2, quad g & 3
      reinterpret_cast<unsigned*>(lds_q)[(((g & 3) * chunks + (g >> 2)) << 2) + j] = word;
    }
  }
  return scale;
}

// One block's share of the PLAIN quantizer for a 16-byte aligned row of n
// inputs (n a multiple of 4): T/16 chunks (slice `slice`), one q8 word per
// thread.  Every thread issues all of its loads in one round - its four
// inputs and its share of the row's amax as float4 (a row longer than
// ROUNDS*T float4 takes more rounds) - so the slice costs one memory
// round trip, a block max and the divisions.  Writes the slice's q8 words
// (split_quad_word form if `split`), its chunk sums and, from slice 0, the
// token scale.  slots holds T/64 floats; all threads of the block call it.
template <int T, int ROUNDS = 8>
__device__ __forceinline__ void quantize_plain_slice(const float* __restrict__ row, int n, int slice, bool split,
                                                     int8_t* __restrict__ q8, int32_t* __restrict__ xsum,
                                                     float* __restrict__ scale_out, float* slots) {
  constexpr int kSlice = T / 16;  // chunks per block
  const int tid = threadIdx.x;
  const int n4 = n >> 2;
  const int chunks = (n + kChunk - 1) / kChunk;
  const float4* row4 = reinterpret_cast<const float4*>(row);

  // This thread's q8 word: chunk u, quad w, field k holds inputs
  // u*64 + w*16 + k + 4b for b = 0..3.
  const int u = slice * kSlice + (tid >> 4);
  const int first = u * kChunk + ((tid >> 2) & 3) * 16 + (tid & 3);
  float mine[4];
#pragma unroll
  for (int b = 0; b < 4; ++b) mine[b] = row[min(first + 4 * b, n - 1)];
  float amax = 0.0f;
  for (int base = 0; base < n4; base += ROUNDS * T) {
    float4 v[ROUNDS];
#pragma unroll
    for (int j = 0; j < ROUNDS; ++j) v[j] = row4[min(base + j * T + tid, n4 - 1)];
#pragma unroll
    for (int j = 0; j < ROUNDS; ++j)
      amax = fmaxf(fmaxf(amax, fmaxf(fabsf(v[j].x), fabsf(v[j].y))), fmaxf(fabsf(v[j].z), fabsf(v[j].w)));
  }
  amax = wave_max(amax);
  if ((tid & 63) == 0) slots[tid >> 6] = amax;
  __syncthreads();
  amax = slots[0];
#pragma unroll
  for (int w = 1; w < T / 64; ++w) amax = fmaxf(amax, slots[w]);
  const float scale = fmaxf(amax / 127.0f, 1e-5f);

  unsigned word = 0;
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    const int q = first + 4 * b < n ? (int)__builtin_rintf(mine[b] / scale) : 0;
    word |= ((unsigned)q & 0xffu) << (8 * b);
  }
  const int value = (int)word;
  const int total = chunk_lane_sum(word_sum(value));
  const unsigned partner = (unsigned)__builtin_amdgcn_mov_dpp(value, 0x4E, 0xF, 0xF, false);  // lane ^ 2
  if (u < chunks) {
    int32_t* q8w = reinterpret_cast<int32_t*>(q8);
    q8w[u * 16 + (tid & 15)] = split ? (int)split_quad_word(word, partner, tid & 3) : value;
    if ((tid & 15) == 0) xsum[u] = total;
  }
  if (slice == 0 && tid == 0) *scale_out = scale;
}

// Hand-over between the blocks of one launch (the argmax's per-block pairs,
// the K-sliced token GEMV's chains), without any block waiting for another:
// 1. every value goes out through store_device, an agent-scope store: on
//    gfx950 a global store with the SC1 scope bit, written through the XCD's
//    L2 to the device's coherence point;
// 2. each storing wave waits for vmcnt(0), which counts such a store complete
//    only once it is performed at that point, then the block barrier;
// 3. one thread counts the block in with an agent-scope atomic add (performed
//    at the same point, issued after the wait);
// 4. the block that reads the final count issues its loads of the values only
//    after the count returned, through load_device, agent-scope loads (SC1),
//    served from the coherence point and not from a stale L2 or L1 line;
//    it then resets the count for the next launch.
// So every value is complete device-wide before any reader can learn that it
// exists.  The compiler's full agent-scope release and acquire add an L2
// writeback and invalidate, which matter only for data stored or loaded
// without the scope bit (none is handed over here); one writeback per block
// made such a launch tens of microseconds slower.
template <typename V>
__device__ __forceinline__ void store_device(V* p, V v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename V>
__device__ __forceinline__ V load_device(const V* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace ivo
