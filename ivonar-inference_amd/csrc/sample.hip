// On-device token sampler: temperature, repetition penalty, top-k and an
// inverse-CDF draw from a caller-supplied uniform (reference kernels
// logit_bounds / sample_token, kernels/ternary.cu:984-1337; the sampling rule
// in torch form, decoder.py:324-333; uniform_() per step,
// kernel_decoder.py:669-681).
//
// Sampling rule, element i of the vocabulary:
//   score_i = logits[i] * (1 / temperature)
//   if seen[i]: score_i *= score_i > 0 ? inverse_penalty : penalty
// k = clamp(*top_k, 1, min(MAX_TOPK, vocab)).  The picks are the k largest
// scores, ordered by the 32-bit order key of the float (so +NaN ranks above
// +inf); equal keys at the cut are taken lowest index first.  The picks are
// listed in ascending index order, p_j = exp(score_j - peak) (ivo_expf), the
// running sums form the CDF in a fixed order (a 64-lane Hillis-Steele scan per
// wave, then the wave totals added in wave order), and the token is the first
// pick j with cdf[j-1] <= min(u, 0.99999994) * total < cdf[j] (the last pick
// if none).  The token goes to token[0] (and history[0]); seen[token] = 1.
//
// The reference lists its picks in atomic order, so its draw for a given u
// depends on scheduling; only the distribution is fixed there.  Here the
// order is the index order, so a draw is a function of (logits, seen, rule,
// u) and the CPU oracle restates it exactly.  With k = 1 the token is the
// first index of the maximum score, as torch.topk / argmax give it.
//
// Work split (one GPU, one sequence):
//   logit_bounds  one wave per 64-entry group: the group's largest score
//                 (taken by order key) into bounds[g].
//   sample_token  one 1024-thread block: the k-th largest group bound Tb
//                 (radix select, 4-bit digits counted with wave ballots), the
//                 groups whose bound is >= Tb (every top-k element lives in
//                 one), their elements with key >= Tb compacted in index order
//                 into LDS, the exact k-th key among them by the same radix
//                 select, the picks, then the softmax and the draw.
#include "internal.hpp"
#include "ternary_device.hpp"

namespace ivo {
namespace {

constexpr int kBoundGroup = 64;  // entries per bound: one wave
constexpr int kBoundsBlock = 256;
constexpr int kSampleThreads = 1024;
constexpr int kSampleWaves = kSampleThreads / 64;
constexpr int kMaxGroups = kMaxSampleVocab / kBoundGroup;  // 4096
constexpr int kCandidates = 2048;                          // LDS candidate capacity

static_assert(kMaxTopK <= kSampleThreads, "one thread per pick");

// Max or min of an unsigned key over the wave, complete in lane 0 only: DPP
// row shifts and permlane swaps, each stage reading a lane that has already
// folded its share (max and min do not depend on the order).
template <bool MAX>
__device__ __forceinline__ unsigned wave_extreme(unsigned k) {
  auto pick = [](unsigned a, unsigned b) { return MAX ? max(a, b) : min(a, b); };
  k = pick(k, (unsigned)row_shl_int<1>((int)k));
  k = pick(k, (unsigned)row_shl_int<2>((int)k));
  k = pick(k, (unsigned)row_shl_int<4>((int)k));
  k = pick(k, (unsigned)row_shl_int<8>((int)k));
  k = pick(k, __float_as_uint(row_swap16(__uint_as_float(k))));
  k = pick(k, __float_as_uint(row_swap32(__uint_as_float(k))));
  return k;
}

struct Rule {
  float inv_t, pen, inv_pen;
};

__device__ __forceinline__ Rule load_rule(const float* temperature, const float* penalty,
                                          const float* inverse_penalty) {
  return Rule{1.0f / *temperature, *penalty, *inverse_penalty};
}

// Order key: unsigned compare of keys = numeric compare of the floats
// (-NaN < -inf < ... < -0 < +0 < ... < +inf < +NaN).
__device__ __forceinline__ unsigned order_key(float v) {
  const unsigned u = __float_as_uint(v);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float key_value(unsigned key) {
  return __uint_as_float((key & 0x80000000u) ? (key & 0x7fffffffu) : ~key);
}

__device__ __forceinline__ float score_of(const float* __restrict__ logits, const uint8_t* __restrict__ seen, int i,
                                          const Rule& r) {
  float s = logits[i] * r.inv_t;
  if (seen[i]) s *= s > 0.0f ? r.inv_pen : r.pen;
  return s;
}

__global__ __launch_bounds__(kBoundsBlock) void bounds_kernel(const float* __restrict__ logits,
                                                              const float* __restrict__ temperature,
                                                              const float* __restrict__ penalty,
                                                              const float* __restrict__ inverse_penalty,
                                                              const uint8_t* __restrict__ seen,
                                                              float* __restrict__ bounds, int vocab, int groups) {
  const int g = blockIdx.x * (kBoundsBlock / 64) + (threadIdx.x >> 6);
  if (g >= groups) return;  // whole waves
  const Rule r = load_rule(temperature, penalty, inverse_penalty);
  const int i = g * kBoundGroup + (threadIdx.x & 63);
  unsigned key = i < vocab ? order_key(score_of(logits, seen, i, r)) : 0u;
  key = wave_extreme<true>(key);
  if ((threadIdx.x & 63) == 0) bounds[g] = key_value(key);
}

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }
__device__ __forceinline__ int wave_id() { return threadIdx.x >> 6; }
__device__ __forceinline__ uint64_t lanes_below() { return (1ull << lane_id()) - 1ull; }

struct SampleShared {
  unsigned bound_key[kMaxGroups];  // order keys of the group bounds, read once
  int group_list[kMaxGroups];
  unsigned cand_key[kCandidates];
  int cand_index[kCandidates];
  int pick_index[kSampleThreads];
  float pick_score[kSampleThreads];
  float cdf[kSampleThreads];
  float wave_sum[kSampleWaves];
  int wave_a[kSampleWaves];
  int wave_b[kSampleWaves];
  unsigned wave_key[kSampleWaves];
  unsigned bins[16];
  int sel_digit;
  int sel_remaining;
  int sel_count;
  int chosen;
};

// Exclusive prefix of two per-thread flags over the block in thread order,
// plus the block totals.  Two barriers; every thread must call it.
__device__ void block_scan2(bool fa, bool fb, int& pa, int& pb, int& ta, int& tb, SampleShared& sh) {
  const uint64_t ma = __ballot(fa), mb = __ballot(fb);
  if (lane_id() == 0) {
    sh.wave_a[wave_id()] = __popcll(ma);
    sh.wave_b[wave_id()] = __popcll(mb);
  }
  __syncthreads();
  int oa = 0, ob = 0, sa = 0, sb = 0;
#pragma unroll
  for (int w = 0; w < kSampleWaves; ++w) {
    const int a = sh.wave_a[w], b = sh.wave_b[w];
    if (w < wave_id()) {
      oa += a;
      ob += b;
    }
    sa += a;
    sb += b;
  }
  pa = oa + __popcll(ma & lanes_below());
  pb = ob + __popcll(mb & lanes_below());
  ta = sa;
  tb = sb;
  __syncthreads();
}

__device__ unsigned block_max_key(unsigned key, SampleShared& sh) {
  key = wave_extreme<true>(key);
  if (lane_id() == 0) sh.wave_key[wave_id()] = key;
  __syncthreads();
  unsigned best = 0u;
#pragma unroll
  for (int w = 0; w < kSampleWaves; ++w) best = max(best, sh.wave_key[w]);
  __syncthreads();
  return best;
}

__device__ unsigned block_min_u(unsigned v, SampleShared& sh) {
  v = wave_extreme<false>(v);
  if (lane_id() == 0) sh.wave_key[wave_id()] = v;
  __syncthreads();
  unsigned best = 0xffffffffu;
#pragma unroll
  for (int w = 0; w < kSampleWaves; ++w) best = min(best, sh.wave_key[w]);
  __syncthreads();
  return best;
}

// Element sources for the selection steps: element j of a sequence gives a
// key, an index and whether it takes part.
struct BoundSource {  // the group bounds' keys in LDS, j = group
  const unsigned* keys;
  int count;
  __device__ int size() const { return count; }
  __device__ bool get(int j, unsigned& key, int& index) const {
    key = keys[j];
    index = j;
    return true;
  }
};

struct GroupSource {  // elements of the listed groups with key >= floor
  const float* logits;
  const uint8_t* seen;
  const int* list;
  Rule rule;
  int groups;
  int vocab;
  unsigned floor;
  __device__ int size() const { return groups * kBoundGroup; }
  __device__ bool get(int j, unsigned& key, int& index) const {
    index = list[j >> 6] * kBoundGroup + (j & 63);
    if (index >= vocab) return false;
    key = order_key(score_of(logits, seen, index, rule));
    return key >= floor;
  }
};

struct CandidateSource {  // the compacted candidates in LDS
  const unsigned* keys;
  const int* indices;
  int count;
  __device__ int size() const { return count; }
  __device__ bool get(int j, unsigned& key, int& index) const {
    key = keys[j];
    index = indices[j];
    return true;
  }
};

struct Cut {
  unsigned key;   // the k-th largest key (exact when ties, else a lower bound with exactly k above)
  int ties;       // with `exact`: how many elements equal to `key` are taken (lowest index first)
  bool exact;
};

// k-th largest key among the taking-part elements of `src` (there are at
// least k of them): MSB-first radix select over 4-bit digits.  The wave counts
// per digit come from ballots and are summed in LDS by lane `digit`; a digit
// bin that holds exactly the remaining count ends the search early.
template <class Source>
__device__ Cut kth_largest(const Source& src, int k, SampleShared& sh) {
  unsigned prefix = 0u, mask = 0u;
  int remaining = k;
  if (threadIdx.x < 16) sh.bins[threadIdx.x] = 0u;
  __syncthreads();
  for (int shift = 28; shift >= 0; shift -= 4) {
    unsigned mine = 0u;  // this lane's digit total, lane d < 16 holds digit d
    const int n = src.size();
    for (int base = 0; base < n; base += kSampleThreads) {
      const int j = base + threadIdx.x;
      unsigned key = 0u;
      int index;
      const bool take = j < n && src.get(j, key, index) && (key & mask) == prefix;
      const unsigned digit = take ? (key >> shift) & 15u : 16u;
#pragma unroll
      for (unsigned d = 0; d < 16; ++d) {
        const unsigned count = __popcll(__ballot(digit == d));
        if (lane_id() == (int)d) mine += count;
      }
    }
    if (lane_id() < 16 && mine != 0u) atomicAdd(&sh.bins[lane_id()], mine);
    __syncthreads();
    if (threadIdx.x < 64) {
      const int d = lane_id();
      const unsigned count = d < 16 ? sh.bins[d] : 0u;
      unsigned at_or_above = count;  // digits >= d
#pragma unroll
      for (int offset = 1; offset < 16; offset <<= 1) {
        const unsigned other = (unsigned)__shfl_down((int)at_or_above, offset, 16);
        if (d + offset < 16) at_or_above += other;
      }
      if (d < 16) {
        const unsigned above = at_or_above - count;
        if (above < (unsigned)remaining && (unsigned)remaining <= at_or_above) {
          sh.sel_digit = d;
          sh.sel_remaining = remaining - (int)above;
          sh.sel_count = (int)count;
        }
        sh.bins[d] = 0u;
      }
    }
    __syncthreads();
    prefix |= (unsigned)sh.sel_digit << shift;
    mask |= 15u << shift;
    remaining = sh.sel_remaining;
    const int count = sh.sel_count;
    __syncthreads();  // sel_* is rewritten by the next digit
    if (count == remaining) return Cut{prefix, 0, false};
  }
  return Cut{prefix, remaining, true};
}

// The picks of `cut` from `src`, in the source's order (ascending index),
// into pick_index / pick_score.  Returns how many were written.
template <class Source>
__device__ int collect_picks(const Source& src, const Cut& cut, SampleShared& sh) {
  int written = 0, ties_seen = 0;
  const int n = src.size();
  for (int base = 0; base < n; base += kSampleThreads) {
    const int j = base + threadIdx.x;
    unsigned key = 0u;
    int index = 0;
    const bool valid = j < n && src.get(j, key, index);
    const bool above = valid && (cut.exact ? key > cut.key : key >= cut.key);
    const bool tie = valid && cut.exact && key == cut.key;
    int above_before, ties_before, above_total, ties_total;
    block_scan2(above, tie, above_before, ties_before, above_total, ties_total, sh);
    const int tie_room = max(0, cut.ties - ties_seen);
    const bool taken_tie = tie && ties_before < tie_room;
    const int slot = written + above_before + min(ties_before, tie_room);
    if ((above || taken_tie) && slot < kSampleThreads) {
      sh.pick_index[slot] = index;
      sh.pick_score[slot] = key_value(key);
    }
    written += above_total + min(ties_total, tie_room);
    ties_seen += ties_total;
  }
  __syncthreads();
  return written;
}

__global__ __launch_bounds__(kSampleThreads) void sample_kernel(
    const float* __restrict__ logits, const float* __restrict__ bounds, const float* __restrict__ temperature,
    const float* __restrict__ penalty, const float* __restrict__ inverse_penalty, uint8_t* __restrict__ seen,
    const int64_t* __restrict__ top_k, const float* __restrict__ uniform, int64_t* __restrict__ token,
    int64_t* __restrict__ history, int vocab, int max_topk) {
  __shared__ SampleShared sh;
  const int tid = threadIdx.x;
  sh.pick_index[tid] = 0;
  const Rule rule = load_rule(temperature, penalty, inverse_penalty);
  const int groups = (vocab + kBoundGroup - 1) / kBoundGroup;
  const long long requested = *top_k;
  const int k = (int)max(1LL, min(requested, (long long)min(max_topk, vocab)));

  unsigned peak = 0u;
  for (int g = tid; g < groups; g += kSampleThreads) {
    const unsigned key = order_key(bounds[g]);
    sh.bound_key[g] = key;
    peak = max(peak, key);
  }
  peak = block_max_key(peak, sh);  // its barrier also publishes bound_key

  int count;
  if (k == 1) {
    // First group whose bound is the peak, then the first element in it.
    unsigned first = 0xffffffffu;
    for (int g = tid; g < groups; g += kSampleThreads)
      if (sh.bound_key[g] == peak) first = min(first, (unsigned)g);
    first = block_min_u(first, sh);
    if (first >= (unsigned)groups) first = 0u;  // unreachable: the peak is one of the bounds
    if (tid < 64) {
      const int i = (int)first * kBoundGroup + tid;
      const bool hit = i < vocab && order_key(score_of(logits, seen, i, rule)) == peak;
      const uint64_t m = __ballot(hit);
      if (tid == 0) {
        sh.pick_index[0] = (int)first * kBoundGroup + (m != 0ull ? (int)__ffsll((unsigned long long)m) - 1 : 0);
        sh.pick_score[0] = key_value(peak);
      }
    }
    __syncthreads();
    count = 1;
  } else {
    // Tb: the k-th largest group bound (all groups when there are fewer than k).
    unsigned floor = 0u;
    if (groups >= k) floor = kth_largest(BoundSource{sh.bound_key, groups}, k, sh).key;
    // Groups whose bound is >= Tb, in ascending order.
    int listed = 0;
    for (int base = 0; base < groups; base += kSampleThreads) {
      const int g = base + tid;
      const bool in = g < groups && sh.bound_key[g] >= floor;
      int before, unused, total, unused_total;
      block_scan2(in, false, before, unused, total, unused_total, sh);
      if (in) sh.group_list[listed + before] = g;
      listed += total;
    }
    __syncthreads();
    const GroupSource elements{logits, seen, sh.group_list, rule, listed, vocab, floor};
    // Their elements with key >= Tb, compacted in index order while they fit;
    // the logits of kGather blocks of 1024 elements are read in one round.
    constexpr int kGather = 4;
    int candidates = 0;
    for (int base = 0; base < elements.size(); base += kSampleThreads * kGather) {
      unsigned keys[kGather];
      int indices[kGather];
      bool ins[kGather];
#pragma unroll
      for (int c = 0; c < kGather; ++c) {
        const int j = base + c * kSampleThreads + tid;
        keys[c] = 0u;
        indices[c] = 0;
        ins[c] = j < elements.size() && elements.get(j, keys[c], indices[c]);
      }
#pragma unroll
      for (int c = 0; c < kGather; ++c) {
        int before, unused, total, unused_total;
        block_scan2(ins[c], false, before, unused, total, unused_total, sh);
        if (ins[c] && candidates + before < kCandidates) {
          sh.cand_key[candidates + before] = keys[c];
          sh.cand_index[candidates + before] = indices[c];
        }
        candidates += total;
      }
    }
    __syncthreads();
    if (candidates <= kCandidates) {
      const CandidateSource cached{sh.cand_key, sh.cand_index, candidates};
      count = collect_picks(cached, kth_largest(cached, k, sh), sh);
    } else {
      count = collect_picks(elements, kth_largest(elements, k, sh), sh);
    }
  }

  // count == k by construction; the clamps keep every access inside the
  // buffers whatever the inputs hold.
  count = min(max(count, 1), kSampleThreads);
  // Softmax weights relative to the peak score, CDF in index order.
  const float top = key_value(peak);
  const float p = tid < count ? ivo_expf(sh.pick_score[tid] - top) : 0.0f;
  float running = p;
#pragma unroll
  for (int offset = 1; offset < 64; offset <<= 1) {
    const float other = __shfl_up(running, offset);
    if (lane_id() >= offset) running += other;
  }
  if (lane_id() == 63) sh.wave_sum[wave_id()] = running;
  if (tid == 0) sh.chosen = kSampleThreads;
  __syncthreads();
  float carry = 0.0f;
  for (int w = 0; w < wave_id(); ++w) carry += sh.wave_sum[w];
  sh.cdf[tid] = carry + running;
  __syncthreads();
  const float total = sh.cdf[count - 1];
  const float target = fminf(*uniform, 0.99999994f) * total;
  const float lower = tid > 0 ? sh.cdf[tid - 1] : 0.0f;
  // Rounding can leave the CDF a hair non-monotone, so more than one pick may
  // match: the first one wins.
  if (tid < count && lower <= target && target < sh.cdf[tid]) atomicMin(&sh.chosen, tid);
  __syncthreads();
  if (tid == 0) {
    const int chosen = sh.chosen >= count ? count - 1 : sh.chosen;
    int index = sh.pick_index[chosen];
    if (index < 0 || index >= vocab) index = 0;
    token[0] = index;
    if (history != nullptr) history[0] = index;
    seen[index] = 1;
  }
}

}  // namespace

hipError_t launch_logit_bounds(hipStream_t stream, const float* logits, const float* temperature,
                               const float* penalty, const float* inverse_penalty, const uint8_t* seen,
                               float* bounds, int vocab) {
  if (vocab <= 0 || vocab > kMaxSampleVocab) return hipErrorInvalidValue;
  const int groups = ceil_div(vocab, kBoundGroup);
  hipLaunchKernelGGL(bounds_kernel, dim3(ceil_div(groups, kBoundsBlock / 64)), dim3(kBoundsBlock), 0, stream, logits,
                     temperature, penalty, inverse_penalty, seen, bounds, vocab, groups);
  return hipGetLastError();
}

hipError_t launch_sample_token(hipStream_t stream, const float* logits, const float* bounds, const float* temperature,
                               const float* penalty, const float* inverse_penalty, uint8_t* seen,
                               const int64_t* top_k, const float* uniform, int64_t* token, int64_t* history,
                               int vocab) {
  if (vocab <= 0 || vocab > kMaxSampleVocab) return hipErrorInvalidValue;
  hipLaunchKernelGGL(sample_kernel, dim3(1), dim3(kSampleThreads), 0, stream, logits, bounds, temperature, penalty,
                     inverse_penalty, seen, top_k, uniform, token, history, vocab, defines().max_topk);
  return hipGetLastError();
}

}  // namespace ivo
