// Decode GEMV for one token (reference: kernels/ternary.cu:302-388,
// entry points gemv_* with GEMV_ARGS).
//
// Work split.  A row of the packed matrix is covered by `lanes` lanes of a
// wave (a power of two, 2..64, the smallest that spans the row's chunks); a
// wave holds 64/lanes row slots and every lane streams R rows, so one wave
// step reads R * 64 lanes * 16 bytes with 128-bit loads that are contiguous
// across the lanes of a slot.  Lane `sub` takes chunk u = j*lanes + sub, so
// the two chunks of a 128-input group land on a lane pair: each lane forms
// its chunk's exact int32 sum of code*q minus the chunk's q sum, and one DPP
// swap (quad_perm [1,0,3,2]) adds the pair into the group partial P[r, g].
// The pair folds P * scale[r, g] into an fp32 fma chain over its groups
// (g = pair, pair + lanes/2, ...); an xor butterfly over the pairs, the token
// scale and the bias finish the row.  That order is restated bit for bit by
// the CPU oracle (orc_gemv_pairs).
//
// Activations.  The block keeps the token's q8 row in LDS in a quad-planar
// layout (quad w of chunk u at int4 index w*C + u), so the 16-byte reads of
// one instruction are contiguous across a slot's lanes and identical across
// slots.  For rows up to gemv_fused_limit() inputs the block quantizes the
// fp32 input itself (the fused prologue of gemv_plain_*, gemv_norm_*,
// gemv_attn_*); longer rows are quantized once by the quantizer into the
// device scratch and the blocks copy the result, which keeps the per-block
// prologue short when the GEMV streams tens of megabytes.
#include "internal.hpp"
#include "ternary_device.hpp"

namespace ivo {
namespace {

constexpr int kRowsPerLane = 2;  // even, so a silu pair never straddles lanes
constexpr int kFusedLimit = 4096;
constexpr int kMaxLdsBytes = 64 * 1024;

struct GemvGeometry {
  int lanes;
  int lane_shift;
  int iters;  // row steps of one wave
};

template <int MODE, int EPI, bool FUSED, int JB>
__global__ __launch_bounds__(kThreads) void gemv_kernel(GemvArgs a, GemvGeometry geo) {
  extern __shared__ __align__(16) unsigned char lds_raw[];
  __shared__ float slots[64];
  const int chunks = (a.n + kChunk - 1) / kChunk;
  int4* lds_q = reinterpret_cast<int4*>(lds_raw);
  int* lds_x = reinterpret_cast<int*>(lds_raw + (size_t)chunks * kChunk);

  float sx;
  if constexpr (FUSED) {
    const RowSource src{a.input, a.aux, a.n, a.eps, a.splits, a.head_dim};
    float inv_rms;
    sx = row_scale<MODE>(src, inv_rms, slots);
    for (int d = threadIdx.x; d < chunks * 16; d += kThreads) {
      const int u = d >> 4, w = (d >> 2) & 3, k = d & 3;
      const int value = quantize_word<MODE>(src, u, w, k, inv_rms, sx);
      reinterpret_cast<int*>(lds_q)[(w * chunks + u) * 4 + k] = value;
      const int total = chunk_lane_sum(word_sum(value));
      if ((d & 15) == 0) lds_x[u] = total;
    }
  } else {
    const int4* gq = reinterpret_cast<const int4*>(a.q8_in);
    for (int e = threadIdx.x; e < chunks * 4; e += kThreads) lds_q[(e & 3) * chunks + (e >> 2)] = gq[e];
    for (int u = threadIdx.x; u < chunks; u += kThreads) lds_x[u] = a.xsum_in[u];
    sx = *a.scale_in;
  }
  __syncthreads();

  const int lanes = geo.lanes;
  const int lane = threadIdx.x & 63;
  const int sub = lane & (lanes - 1);
  const int slot = lane >> geo.lane_shift;
  const int rows_per_iter = (64 >> geo.lane_shift) * kRowsPerLane;
  const int waves = gridDim.x * (kThreads / 64);
  const uint4 zero4 = make_uint4(0u, 0u, 0u, 0u);
  const int4 zeroq = make_int4(0, 0, 0, 0);

  for (int it = blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6); it < geo.iters; it += waves) {
    const int row0 = it * rows_per_iter + slot * kRowsPerLane;
    float acc[kRowsPerLane];
#pragma unroll
    for (int r = 0; r < kRowsPerLane; ++r) acc[r] = 0.0f;
    for (int j0 = 0; j0 * lanes < chunks; j0 += JB) {
      uint4 wv[JB][kRowsPerLane];
#pragma unroll
      for (int jb = 0; jb < JB; ++jb) {
        const int u = (j0 + jb) * lanes + sub;
#pragma unroll
        for (int r = 0; r < kRowsPerLane; ++r) {
          const int row = row0 + r;
          wv[jb][r] = (u < chunks && row < a.rows)
                          ? *reinterpret_cast<const uint4*>(a.packed + (size_t)row * a.row_bytes + (size_t)u * 16)
                          : zero4;
        }
      }
#pragma unroll
      for (int jb = 0; jb < JB; ++jb) {
        const int u = (j0 + jb) * lanes + sub;
        const bool live = u < chunks;
        const int4 q0 = live ? lds_q[u] : zeroq;
        const int4 q1 = live ? lds_q[chunks + u] : zeroq;
        const int4 q2 = live ? lds_q[2 * chunks + u] : zeroq;
        const int4 q3 = live ? lds_q[3 * chunks + u] : zeroq;
        const int xs = live ? lds_x[u] : 0;
        const int g = u >> 1;
        const bool group_live = 2 * g < chunks;
#pragma unroll
        for (int r = 0; r < kRowsPerLane; ++r) {
          int d = chunk_code_dot(wv[jb][r], q0, q1, q2, q3, 0) - xs;
          d += pair_swap(d);
          const int row = row0 + r;
          if constexpr (EPI == kPartials) {
            if (group_live && (sub & 1) == 0 && row < a.rows) a.partials[(size_t)row * a.groups + g] = d;
          } else {
            if (group_live && row < a.rows)
              acc[r] = __builtin_fmaf((float)d, h2f(a.scales[(size_t)row * a.groups + g]), acc[r]);
          }
        }
      }
    }
    if constexpr (EPI != kPartials) {
#pragma unroll
      for (int r = 0; r < kRowsPerLane; ++r) {
        for (int offset = 2; offset < lanes; offset <<= 1) acc[r] = acc[r] + __shfl_xor(acc[r], offset);
      }
      if (sub == 0) {
        float y[kRowsPerLane];
#pragma unroll
        for (int r = 0; r < kRowsPerLane; ++r) {
          const int row = row0 + r;
          y[r] = acc[r] * sx;
          if (a.bias != nullptr && row < a.rows) y[r] = y[r] + a.bias[row];
        }
#pragma unroll
        for (int r = 0; r < kRowsPerLane; ++r) {
          const int row = row0 + r;
          if constexpr (EPI == kStore) {
            if (row < a.rows) a.output[row] = y[r];
          } else if constexpr (EPI == kResidual) {
            if (row < a.rows) a.output[row] = a.output[row] + y[r];
          } else if constexpr (EPI == kSiluPair) {
            if ((r & 1) == 0 && row + 1 < a.rows) a.output[row >> 1] = ivo_silu(y[r]) * y[r + 1];
          }
        }
      }
    }
  }
}

template <int MODE, int EPI, bool FUSED>
hipError_t launch_jb(hipStream_t stream, const GemvArgs& a, const GemvGeometry& geo, int blocks, size_t lds, int jb) {
  switch (jb) {
    case 1: hipLaunchKernelGGL((gemv_kernel<MODE, EPI, FUSED, 1>), dim3(blocks), dim3(kThreads), lds, stream, a, geo); break;
    case 2: hipLaunchKernelGGL((gemv_kernel<MODE, EPI, FUSED, 2>), dim3(blocks), dim3(kThreads), lds, stream, a, geo); break;
    default: hipLaunchKernelGGL((gemv_kernel<MODE, EPI, FUSED, 4>), dim3(blocks), dim3(kThreads), lds, stream, a, geo); break;
  }
  return hipGetLastError();
}

template <int MODE>
hipError_t launch_fused(hipStream_t stream, const GemvArgs& a, const GemvGeometry& geo, int blocks, size_t lds, int jb) {
  switch (a.epi) {
    case kStore: return launch_jb<MODE, kStore, true>(stream, a, geo, blocks, lds, jb);
    case kResidual: return launch_jb<MODE, kResidual, true>(stream, a, geo, blocks, lds, jb);
    case kSiluPair: return launch_jb<MODE, kSiluPair, true>(stream, a, geo, blocks, lds, jb);
    default: return hipErrorInvalidValue;
  }
}

int device_cus() {
  static int cached[64] = {0};
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= 64) return 256;
  if (cached[device] == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess || cus <= 0) cus = 256;
    cached[device] = cus;
  }
  return cached[device];
}

}  // namespace

int gemv_fused_limit() { return kFusedLimit; }

void gemv_plan(int rows, int n, int* lanes, int* rows_per_lane) {
  (void)rows;
  const int chunks = ceil_div(n, kChunk);
  int l = 2;
  while (l < 64 && l < chunks) l <<= 1;
  *lanes = l;
  *rows_per_lane = kRowsPerLane;
}

hipError_t launch_gemv(hipStream_t stream, const GemvArgs& in) {
  if (in.rows <= 0) return hipSuccess;
  GemvArgs a = in;
  const int chunks = ceil_div(a.n, kChunk);
  const size_t lds = (size_t)chunks * (kChunk + 4);
  if (lds > (size_t)kMaxLdsBytes) return hipErrorInvalidValue;
  int lanes, rpl;
  gemv_plan(a.rows, a.n, &lanes, &rpl);
  GemvGeometry geo;
  geo.lanes = lanes;
  geo.lane_shift = __builtin_ctz((unsigned)lanes);
  const int rows_per_iter = (64 / lanes) * rpl;
  geo.iters = ceil_div(a.rows, rows_per_iter);
  const int steps = ceil_div(chunks, lanes);
  const int jb = steps >= 4 ? 4 : (steps >= 2 ? 2 : 1);
  const int cus = device_cus();
  const bool fused = a.q8_in == nullptr && a.n <= kFusedLimit;
  const int cap = fused ? 2 * cus : 4 * cus;
  int blocks = ceil_div(geo.iters, kThreads / 64);
  if (blocks > cap) blocks = cap;

  if (fused) {
    if (a.epi == kPartials) return hipErrorInvalidValue;
    switch (a.mode) {
      case kPlain: return launch_fused<kPlain>(stream, a, geo, blocks, lds, jb);
      case kNorm: return launch_fused<kNorm>(stream, a, geo, blocks, lds, jb);
      case kAttn: return launch_fused<kAttn>(stream, a, geo, blocks, lds, jb);
      default: return hipErrorInvalidValue;
    }
  }
  if (a.q8_in == nullptr) {
    Scratch* scratch = nullptr;
    hipError_t status = scratch_for_stream(stream, &scratch);
    if (status != hipSuccess) return status;
    if (chunks > scratch->capacity_chunks) return hipErrorInvalidValue;
    QuantArgs q{a.mode, a.input, a.n, a.aux, a.n, a.eps, a.splits, a.head_dim, 1, scratch->q8, scratch->xsum,
                scratch->scale};
    status = launch_quantize(stream, q);
    if (status != hipSuccess) return status;
    a.q8_in = scratch->q8;
    a.xsum_in = scratch->xsum;
    a.scale_in = scratch->scale;
  }
  switch (a.epi) {
    case kStore: return launch_jb<kPlain, kStore, false>(stream, a, geo, blocks, lds, jb);
    case kResidual: return launch_jb<kPlain, kResidual, false>(stream, a, geo, blocks, lds, jb);
    case kSiluPair: return launch_jb<kPlain, kSiluPair, false>(stream, a, geo, blocks, lds, jb);
    case kPartials: return launch_jb<kPlain, kPartials, false>(stream, a, geo, blocks, lds, jb);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace ivo
