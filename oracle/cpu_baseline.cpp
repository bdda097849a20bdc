// CPU baseline for the ternary linear layer: a C++/OpenMP restatement of the
// reference's numba kernels.  TEST AND BENCHMARK INFRASTRUCTURE ONLY: the
// benchmark times it as the CPU baseline ("port") and the tests compare it
// with the oracle by tolerance; the product never links or calls it.
//
// It follows the reference (paths relative to src/ivonar_inference/):
//   planes_of        cpu_decoder.py:288-312  per 128-input group, 32 bytes;
//                    byte b holds inputs b, b+32, b+64, b+96 (2 bits each),
//                    pad code 1 (value 0)
//   quantize_into    cpu_decoder.py:30-52    clamp to +-127, gsum per group
//   norm_quantize    cpu_decoder.py:55-70    sequential sum of squares,
//                    clip to +-clip*|w| after multiplying by w
//   row_dot          cpu_decoder.py:73-86    int32 per group, fp32 total
//   gemv / normed_gemv / normed_gemv_silu    cpu_decoder.py:89-125
// numba compiles these with fastmath {reassoc, contract, nsz}
// (cpu_decoder.py:27); the Makefile builds this file with the matching gcc
// flags, so results match the oracle only within tolerance.
#include <cmath>
#include <cstdint>
#include <cstring>
#include <omp.h>

namespace {
constexpr int kGroup = 128;
constexpr int kPlane = kGroup / 4;

float quantize_into(const float* values, int n, int8_t* q, int32_t* gsum, int groups) {
  float amax = 0.0f;
  for (int i = 0; i < n; ++i) {
    const float magnitude = std::fabs(values[i]);
    if (magnitude > amax) amax = magnitude;
  }
  float scale = amax / 127.0f;
  if (scale < 1e-5f) scale = 1e-5f;
  for (int g = 0; g < groups; ++g) gsum[g] = 0;
  for (int i = 0; i < n; ++i) {
    float level = std::rint(values[i] / scale);
    if (level > 127.0f) level = 127.0f;
    else if (level < -127.0f) level = -127.0f;
    const int code = static_cast<int>(level);
    q[i] = static_cast<int8_t>(code);
    gsum[i / kGroup] += code;
  }
  for (int i = n; i < groups * kGroup; ++i) q[i] = 0;
  return scale;
}

float norm_quantize(const float* x, const float* weight, float eps, float clip, int n, float* work, int8_t* q,
                    int32_t* gsum, int groups) {
  float squares = 0.0f;
  for (int i = 0; i < n; ++i) squares += x[i] * x[i];
  const float inverse = 1.0f / std::sqrt(squares / static_cast<float>(n) + eps);
  for (int i = 0; i < n; ++i) {
    float value = x[i] * inverse * weight[i];
    const float bound = clip * std::fabs(weight[i]);
    if (value > bound) value = bound;
    else if (value < -bound) value = -bound;
    work[i] = value;
  }
  return quantize_into(work, n, q, gsum, groups);
}

inline float row_dot(const uint8_t* planes, const float* scales, int r, int groups, const int8_t* q,
                     const int32_t* gsum) {
  const uint8_t* row = planes + static_cast<size_t>(r) * groups * kPlane;
  const float* srow = scales + static_cast<size_t>(r) * groups;
  float total = 0.0f;
  for (int g = 0; g < groups; ++g) {
    int32_t acc = 0;
    const int base = g * kGroup;
    const uint8_t* plane = row + g * kPlane;
    for (int b = 0; b < kPlane; ++b) {
      const int32_t byte = plane[b];
      acc += (byte & 3) * q[base + b] + ((byte >> 2) & 3) * q[base + kPlane + b];
      acc += ((byte >> 4) & 3) * q[base + 2 * kPlane + b] + ((byte >> 6) & 3) * q[base + 3 * kPlane + b];
    }
    total += srow[g] * static_cast<float>(acc - gsum[g]);
  }
  return total;
}
}  // namespace

extern "C" {

// Repack reference-layout rows (packed[r*row_bytes + i/4], 2 bits per input)
// into planes [rows, groups*32] (cpu_decoder.py:288-312).
void cb_planes_of(const uint8_t* packed, int rows, int n, int row_bytes, uint8_t* planes) {
  const int groups = (n + kGroup - 1) / kGroup;
#pragma omp parallel for schedule(static)
  for (int r = 0; r < rows; ++r) {
    uint8_t* out = planes + static_cast<size_t>(r) * groups * kPlane;
    for (int g = 0; g < groups; ++g) {
      for (int b = 0; b < kPlane; ++b) {
        int byte = 0;
        for (int k = 0; k < 4; ++k) {
          const int i = g * kGroup + k * kPlane + b;
          int code = 1;
          if (i < n) code = (packed[static_cast<size_t>(r) * row_bytes + (i >> 2)] >> ((i & 3) * 2)) & 3;
          byte |= code << (2 * k);
        }
        out[g * kPlane + b] = static_cast<uint8_t>(byte);
      }
    }
  }
}

void cb_set_threads(int threads) { omp_set_num_threads(threads > 0 ? threads : 1); }
int cb_max_threads(void) { return omp_get_max_threads(); }

// gemv (cpu_decoder.py:89-100): out[r] (+)= row_dot * act_scale (+ bias[r]).
void cb_gemv(const float* values, int n, const uint8_t* planes, const float* scales, const float* bias, int rows,
             int8_t* q, int32_t* gsum, float* out, int accumulate) {
  const int groups = (n + kGroup - 1) / kGroup;
  const float act_scale = quantize_into(values, n, q, gsum, groups);
#pragma omp parallel for schedule(static)
  for (int r = 0; r < rows; ++r) {
    float result = row_dot(planes, scales, r, groups, q, gsum) * act_scale;
    if (bias) result += bias[r];
    if (accumulate) out[r] += result;
    else out[r] = result;
  }
}

// normed_gemv (cpu_decoder.py:103-111).
void cb_normed_gemv(const float* x, const float* weight, float eps, float clip, int n, float* work,
                    const uint8_t* planes, const float* scales, const float* bias, int rows, int8_t* q,
                    int32_t* gsum, float* out) {
  const int groups = (n + kGroup - 1) / kGroup;
  const float act_scale = norm_quantize(x, weight, eps, clip, n, work, q, gsum, groups);
#pragma omp parallel for schedule(static)
  for (int r = 0; r < rows; ++r) {
    float result = row_dot(planes, scales, r, groups, q, gsum) * act_scale;
    if (bias) result += bias[r];
    out[r] = result;
  }
}

// normed_gemv_silu (cpu_decoder.py:114-125): gate rows [0, dense), up rows
// [dense, 2*dense) (concatenated, not interleaved).
void cb_normed_gemv_silu(const float* x, const float* weight, float eps, float clip, int n, float* work,
                         const uint8_t* planes, const float* scales, const float* bias, int dense, int8_t* q,
                         int32_t* gsum, float* out) {
  const int groups = (n + kGroup - 1) / kGroup;
  const float act_scale = norm_quantize(x, weight, eps, clip, n, work, q, gsum, groups);
#pragma omp parallel for schedule(static)
  for (int r = 0; r < dense; ++r) {
    float gate = row_dot(planes, scales, r, groups, q, gsum) * act_scale;
    float up = row_dot(planes, scales, dense + r, groups, q, gsum) * act_scale;
    if (bias) {
      gate += bias[r];
      up += bias[dense + r];
    }
    out[r] = gate / (1.0f + std::exp(-gate)) * up;
  }
}

}  // extern "C"
