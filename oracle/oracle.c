/*
 * CPU oracle for the ternary linear layer.  TEST INFRASTRUCTURE ONLY: the
 * tests, the smoke check and the CPU-baseline leg of the benchmark load this
 * library as the checker.  The product path (the HIP library) never links,
 * loads or calls it.
 *
 * What it restates, with the reference file:line each part follows
 * (paths relative to the reference's src/ivonar_inference/):
 *
 *   packed format      quantization.py:10-18 (byte b of a row holds inputs
 *                      4b+k in bits 2k..2k+1; code = w + 1; code 3 unused),
 *                      one fp16 scale per 128 inputs (quantization.py:21-32).
 *   quantizer          kernels/ternary.cu:148-197 (quantize_source):
 *                      amax -> s = fmaxf(amax/127, 1e-5) -> q = rintf(v/s);
 *                      NORM prologue ternary.cu:163,169-176 with the
 *                      reference kernel's reduction tree for the sum of
 *                      squares (256-thread strided partials, 32-lane xor
 *                      butterfly, sequential sum of the 8 warp totals,
 *                      ternary.cu:157-170, :81-84, :101-109);
 *                      ATTN prologue ternary.cu:128-146 (split-softmax merge).
 *   integer core       ternary.cu:241-258 (sum of code*q minus sum of q).
 *   GEMV epilogues     ternary.cu:343-353 (store / residual / silu pair).
 *   tile GEMM          ternary.cu:688-765.
 *   embedding          ternary.cu:411-419, :613-622.
 *
 * The q8 activation layout is this library's own (see q8_index): inside each
 * 64-input chunk, 16-byte quad w holds inputs 16w..16w+15 ordered so that the
 * 32-bit word k of the quad holds inputs {16w+k, 16w+4+k, 16w+8+k, 16w+12+k},
 * which is what (packed_word >> 2k) & 0x03030303 pairs with.  The reference
 * uses the same pairing plus a bank rotation (ternary.cu:121-126).
 *
 * Floating-point order.  Three fp32 orders are restated bit for bit:
 *   gemv_pairs   the decode GEMV of the HIP library: per 128-input group an
 *                exact int32 partial, groups strided over P lane pairs,
 *                each pair an fmaf chain, then an xor butterfly over pairs;
 *   gemm_seq     the MFMA GEMM of the HIP library: one fmaf chain over the
 *                groups in ascending order per output;
 *   reforder     the reference kernel's own order (per 64-input chunk,
 *                chunks strided over `lanes`, fmaf chains, xor butterfly
 *                over lanes), assuming NVRTC's default contraction of
 *                a*b+c into fma.  That contraction cannot be verified
 *                here, so bit equality with the CUDA build is unpinned;
 *                it is checked against the fp64 truth by tolerance.
 * Transcendentals use ivo_expf (Cody-Waite reduction + degree-7 Taylor
 * polynomial), the same op sequence as the HIP library, so silu and the
 * softmax merge are reproducible bit for bit across CPU and GPU.
 *
 * Build: see oracle/Makefile (gcc -O2 -ffp-contract=off, no fast-math).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define MODE_PLAIN 0
#define MODE_NORM 1
#define MODE_ATTN 2
#define EPI_STORE 0
#define EPI_RESIDUAL 1
#define EPI_SILU_PAIR 2

#define REF_THREADS 256
#define REF_WARP 32

static inline float as_float(uint32_t bits) {
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

/* IEEE binary16 -> binary32, exact for every input. */
float orc_h2f(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t exponent = (h >> 10) & 0x1fu;
  const uint32_t mantissa = h & 0x3ffu;
  if (exponent == 0) {
    const float f = (float)mantissa * 5.9604644775390625e-08f; /* man * 2^-24, exact */
    return sign ? -f : f;
  }
  if (exponent == 31) return as_float(sign | 0x7f800000u | (mantissa << 13));
  return as_float(sign | ((exponent + 112u) << 23) | (mantissa << 13));
}

/* exp(x) in fp32: Cody-Waite reduction x = n*ln2 + r, |r| <= ln2/2, then the
 * degree-7 Taylor polynomial of e^r in Horner form and a two-step scaling by
 * 2^n.  Same sequence of IEEE fp32 operations as ivo_expf in the HIP sources. */
float orc_expf(float x) {
  if (x != x) return x;
  if (x > 88.72283935546875f) return INFINITY;
  if (x < -103.97208404541015625f) return 0.0f;
  const float n = rintf(x * 1.44269502162933349609375f);
  float r = fmaf(n, -0.693145751953125f, x);
  r = fmaf(n, -1.428606765330187045e-06f, r);
  float p = 1.9841270113829523e-04f;      /* 1/5040 */
  p = fmaf(p, r, 1.3888889225199819e-03f); /* 1/720 */
  p = fmaf(p, r, 8.3333337679505348e-03f); /* 1/120 */
  p = fmaf(p, r, 4.1666667908430099e-02f); /* 1/24 */
  p = fmaf(p, r, 1.6666667163372040e-01f); /* 1/6 */
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  const int ni = (int)n;
  const int n1 = ni / 2, n2 = ni - n1;
  const float s1 = as_float((uint32_t)(n1 + 127) << 23);
  const float s2 = as_float((uint32_t)(n2 + 127) << 23);
  return (p * s1) * s2;
}

/* silu(x) = x / (1 + e^-x)  (ternary.cu:74) */
float orc_silu(float x) { return x / (1.0f + orc_expf(-x)); }

/* Byte offset of input i inside a token's q8 row (this library's layout). */
static inline int q8_index(int i) {
  return (i >> 6) * 64 + ((i >> 4) & 3) * 16 + (i & 3) * 4 + ((i >> 2) & 3);
}
int orc_q8_index(int i) { return q8_index(i); }

/* Source value of input i before quantization (ternary.cu:128-146). */
static float attn_value(const float* input, int i, int splits, int head_dim) {
  const int stride = head_dim + 2;
  const int head = i / head_dim, dim = i - head * head_dim;
  const float* base = input + (size_t)head * splits * stride;
  float peak = -INFINITY;
  for (int s = 0; s < splits; ++s) peak = fmaxf(peak, base[s * stride]);
  float total = 0.0f, value = 0.0f;
  for (int s = 0; s < splits; ++s) {
    const float* part = base + s * stride;
    const float weight = part[0] == -INFINITY ? 0.0f : orc_expf(part[0] - peak);
    total = fmaf(weight, part[1], total);
    value = fmaf(weight, part[2 + dim], value);
  }
  return value / total;
}

/* Sum of squares in the reference kernel's tree (ternary.cu:157-170). */
float orc_ref_sum_squares(const float* v, int n) {
  float part[REF_THREADS];
  for (int t = 0; t < REF_THREADS; ++t) {
    float s = 0.0f;
    for (int i = t; i < n; i += REF_THREADS) s = fmaf(v[i], v[i], s);
    part[t] = s;
  }
  for (int offset = REF_WARP / 2; offset > 0; offset >>= 1) {
    float next[REF_THREADS];
    for (int t = 0; t < REF_THREADS; ++t) next[t] = part[t] + part[t ^ offset];
    memcpy(part, next, sizeof(part));
  }
  float total = 0.0f;
  for (int w = 0; w < REF_THREADS / REF_WARP; ++w) total = total + part[w * REF_WARP];
  return total;
}

/* Quantize one token row into this library's q8 layout.
 * Returns the activation scale; writes q8[C*64] (zero padded) and xsum[C]. */
static float quantize_row(int mode, const float* input, const float* aux, int n, float eps, int splits,
                          int head_dim, int8_t* q8, int32_t* xsum) {
  const int chunks = (n + 63) >> 6;
  float* values = (float*)malloc(sizeof(float) * (size_t)(n > 0 ? n : 1));
  for (int i = 0; i < n; ++i) values[i] = mode == MODE_ATTN ? attn_value(input, i, splits, head_dim) : input[i];
  if (mode == MODE_NORM) {
    const float squares = orc_ref_sum_squares(values, n);
    const float inv_rms = 1.0f / sqrtf(squares / (float)n + eps);
    for (int i = 0; i < n; ++i) values[i] = fminf(fmaxf(values[i] * inv_rms, -8.0f), 8.0f) * aux[i];
  }
  float amax = 0.0f;
  for (int i = 0; i < n; ++i) amax = fmaxf(amax, fabsf(values[i]));
  const float scale = fmaxf(amax / 127.0f, 1e-5f);
  memset(q8, 0, (size_t)chunks * 64);
  for (int i = 0; i < n; ++i) q8[q8_index(i)] = (int8_t)(int)rintf(values[i] / scale);
  for (int u = 0; u < chunks; ++u) {
    int total = 0;
    for (int b = 0; b < 64; ++b) total += q8[u * 64 + b];
    xsum[u] = total;
  }
  free(values);
  return scale;
}

/* Quantize m token rows (row t reads input + t*in_stride).  q8 row stride is
 * C*64 bytes, xsum row stride C, one scale per row. */
void orc_quantize_rows(int mode, const float* input, int in_stride, const float* aux, int n, float eps, int splits,
                       int head_dim, int m, int8_t* q8, int32_t* xsum, float* scale) {
  const int chunks = (n + 63) >> 6;
  for (int t = 0; t < m; ++t) {
    scale[t] = quantize_row(mode, input + (size_t)t * in_stride, aux, n, eps, splits, head_dim,
                            q8 + (size_t)t * chunks * 64, xsum + (size_t)t * chunks);
  }
}

/* Exact integer dot of chunk u of one weight row with the q8 chunk, minus xsum. */
static inline int chunk_partial(const uint8_t* wrow, const int8_t* q8row, const int32_t* xsum, int u) {
  const uint8_t* w = wrow + (size_t)u * 16;
  const int8_t* a = q8row + (size_t)u * 64;
  int dot = 0;
  for (int quad = 0; quad < 4; ++quad) {
    for (int b = 0; b < 4; ++b) {
      const int byte = w[quad * 4 + b];
      for (int k = 0; k < 4; ++k) dot += ((byte >> (2 * k)) & 3) * a[quad * 16 + k * 4 + b];
    }
  }
  return dot - xsum[u];
}

/* Per-128-group int32 partials P[row, g] = sum over the group of (code-1)*q. */
void orc_group_partials(const int8_t* q8, const int32_t* xsum, const uint8_t* packed, int rows, int n,
                        int row_bytes, int32_t* out) {
  const int chunks = (n + 63) >> 6, groups = (n + 127) >> 7;
  for (int r = 0; r < rows; ++r) {
    const uint8_t* wrow = packed + (size_t)r * row_bytes;
    for (int g = 0; g < groups; ++g) {
      int total = chunk_partial(wrow, q8, xsum, 2 * g);
      if (2 * g + 1 < chunks) total += chunk_partial(wrow, q8, xsum, 2 * g + 1);
      out[(size_t)r * groups + g] = total;
    }
  }
}

static void epilogue(int epi, float* out, int out_index_row, int row, float y, float partner) {
  (void)row;
  if (epi == EPI_STORE) out[out_index_row] = y;
  else if (epi == EPI_RESIDUAL) out[out_index_row] = out[out_index_row] + y;
  else out[out_index_row] = orc_silu(y) * partner;
}

/* Decode GEMV in the HIP library's order (lane pairs).  `lanes` is the lane
 * count per row the library chose (a power of two >= 2). */
void orc_gemv_pairs(int epi, const int8_t* q8, const int32_t* xsum, float sx, const uint8_t* packed,
                    const uint16_t* scales, const float* bias, float* out, int rows, int n, int row_bytes,
                    int groups, int lanes) {
  const int chunks = (n + 63) >> 6, ngroups = (n + 127) >> 7;
  const int pairs = lanes / 2;
  float* y = (float*)malloc(sizeof(float) * (size_t)(rows > 0 ? rows : 1));
  float* acc = (float*)malloc(sizeof(float) * (size_t)pairs);
  float* next = (float*)malloc(sizeof(float) * (size_t)pairs);
  for (int r = 0; r < rows; ++r) {
    const uint8_t* wrow = packed + (size_t)r * row_bytes;
    for (int p = 0; p < pairs; ++p) acc[p] = 0.0f;
    for (int g = 0; g < ngroups; ++g) {
      int total = chunk_partial(wrow, q8, xsum, 2 * g);
      if (2 * g + 1 < chunks) total += chunk_partial(wrow, q8, xsum, 2 * g + 1);
      acc[g % pairs] = fmaf((float)total, orc_h2f(scales[(size_t)r * groups + g]), acc[g % pairs]);
    }
    for (int offset = 1; offset < pairs; offset <<= 1) {
      for (int p = 0; p < pairs; ++p) next[p] = acc[p] + acc[p ^ offset];
      memcpy(acc, next, sizeof(float) * (size_t)pairs);
    }
    float v = acc[0] * sx;
    if (bias) v = v + bias[r];
    y[r] = v;
  }
  for (int r = 0; r < rows; ++r) {
    if (epi == EPI_SILU_PAIR) {
      if ((r & 1) == 0 && r + 1 < rows) epilogue(epi, out, r >> 1, r, y[r], y[r + 1]);
    } else {
      epilogue(epi, out, r, r, y[r], 0.0f);
    }
  }
  free(next);
  free(acc);
  free(y);
}

/* MFMA GEMM order with K split S ways: groups in S contiguous ranges of
 * ceil(G/S), each range an fmaf chain from zero in ascending order, the S
 * partial sums then added in range order (S = 1: one chain over all groups). */
void orc_gemm_split(int epi, const int8_t* q8, const int32_t* xsum, const float* scale_in, const uint8_t* packed,
                    const uint16_t* scales, const float* bias, float* out, int rows, int n, int row_bytes,
                    int groups, int out_stride, int m, int splits) {
  const int chunks = (n + 63) >> 6, ngroups = (n + 127) >> 7;
  const int per = (ngroups + splits - 1) / splits;
  float* y = (float*)malloc(sizeof(float) * (size_t)(rows > 0 ? rows : 1));
  for (int t = 0; t < m; ++t) {
    const int8_t* qrow = q8 + (size_t)t * chunks * 64;
    const int32_t* xrow = xsum + (size_t)t * chunks;
    for (int r = 0; r < rows; ++r) {
      const uint8_t* wrow = packed + (size_t)r * row_bytes;
      float total = 0.0f;
      for (int s = 0; s < splits; ++s) {
        const int begin = s * per < ngroups ? s * per : ngroups;
        const int end = begin + per < ngroups ? begin + per : ngroups;
        float acc = 0.0f;
        for (int g = begin; g < end; ++g) {
          int p = chunk_partial(wrow, qrow, xrow, 2 * g);
          if (2 * g + 1 < chunks) p += chunk_partial(wrow, qrow, xrow, 2 * g + 1);
          acc = fmaf((float)p, orc_h2f(scales[(size_t)r * groups + g]), acc);
        }
        total = s == 0 ? acc : total + acc;
      }
      float v = total * scale_in[t];
      if (bias) v = v + bias[r];
      y[r] = v;
    }
    float* orow = out + (size_t)t * out_stride;
    for (int r = 0; r < rows; ++r) {
      if (epi == EPI_SILU_PAIR) {
        if ((r & 1) == 0 && r + 1 < rows) epilogue(epi, orow, r >> 1, r, y[r], y[r + 1]);
      } else {
        epilogue(epi, orow, r, r, y[r], 0.0f);
      }
    }
  }
  free(y);
}

/* One fmaf chain over groups per (token, row): the split order with S = 1. */
void orc_gemm_seq(int epi, const int8_t* q8, const int32_t* xsum, const float* scale_in, const uint8_t* packed,
                  const uint16_t* scales, const float* bias, float* out, int rows, int n, int row_bytes, int groups,
                  int out_stride, int m) {
  orc_gemm_split(epi, q8, xsum, scale_in, packed, scales, bias, out, rows, n, row_bytes, groups, out_stride, m, 1);
}

/* The reference kernel's own fp32 order (ternary.cu:330-347 for the GEMV,
 * :709-763 for the tile GEMM), for m token rows.  tile != 0 selects the tile
 * epilogue rounding fmaf(acc, token_scale, bias) (ternary.cu:760); the GEMV
 * rounds acc*scale and then adds the bias (ternary.cu:344-345). */
void orc_reforder(int epi, int tile, const int8_t* q8, const int32_t* xsum, const float* scale_in,
                  const uint8_t* packed, const uint16_t* scales, const float* bias, float* out, int rows, int n,
                  int row_bytes, int groups, int lanes, int out_stride, int m) {
  const int chunks = (n + 63) >> 6;
  float* y = (float*)malloc(sizeof(float) * (size_t)(rows > 0 ? rows : 1));
  float* acc = (float*)malloc(sizeof(float) * (size_t)lanes);
  float* next = (float*)malloc(sizeof(float) * (size_t)lanes);
  for (int t = 0; t < m; ++t) {
    const int8_t* qrow = q8 + (size_t)t * chunks * 64;
    const int32_t* xrow = xsum + (size_t)t * chunks;
    for (int r = 0; r < rows; ++r) {
      const uint8_t* wrow = packed + (size_t)r * row_bytes;
      for (int s = 0; s < lanes; ++s) {
        float a = 0.0f;
        for (int u = s; u < chunks; u += lanes) {
          a = fmaf((float)chunk_partial(wrow, qrow, xrow, u), orc_h2f(scales[(size_t)r * groups + (u >> 1)]), a);
        }
        acc[s] = a;
      }
      for (int offset = 1; offset < lanes; offset <<= 1) {
        for (int s = 0; s < lanes; ++s) next[s] = acc[s] + acc[s ^ offset];
        memcpy(acc, next, sizeof(float) * (size_t)lanes);
      }
      float v;
      if (tile) {
        v = fmaf(acc[0], scale_in[t], bias ? bias[r] : 0.0f);
      } else {
        v = acc[0] * scale_in[t];
        if (bias) v = v + bias[r];
      }
      y[r] = v;
    }
    float* orow = out + (size_t)t * out_stride;
    for (int r = 0; r < rows; ++r) {
      if (epi == EPI_SILU_PAIR) {
        if ((r & 1) == 0 && r + 1 < rows) epilogue(epi, orow, r >> 1, r, y[r], y[r + 1]);
      } else {
        epilogue(epi, orow, r, r, y[r], 0.0f);
      }
    }
  }
  free(next);
  free(acc);
  free(y);
}

/* Decode packed rows tokens[t] into fp32 (ternary.cu:411-419, :613-622). */
void orc_embed(const int64_t* tokens, int m, const uint8_t* packed, const uint16_t* scales, float* out, int n,
               int row_bytes, int groups) {
  for (int t = 0; t < m; ++t) {
    const size_t row = (size_t)tokens[t];
    for (int i = 0; i < n; ++i) {
      const int code = (packed[row * row_bytes + (i >> 2)] >> ((i & 3) * 2)) & 3;
      out[(size_t)t * n + i] = (float)(code - 1) * orc_h2f(scales[row * groups + (i >> 7)]);
    }
  }
}

/* ---------------------------------------------------------------------------
 * Fast paths for whole decoder stacks.  The per-group partials are integers,
 * so they are the same whatever order they are summed in; only the fp32
 * finishing step below follows a kernel's order.  Rows run in parallel
 * (OpenMP), which changes nothing inside a row.
 * ------------------------------------------------------------------------- */

/* w: int8 ternary values [rows, K] (-1, 0, +1); q: int8 activations in input
 * order [K]; out: int32 partials [rows, ceil(K/128)]. */
void orc_partials_i8(const int8_t* w, int rows, int k, const int8_t* q, int32_t* out) {
  const int groups = (k + 127) / 128;
#pragma omp parallel for schedule(static)
  for (int r = 0; r < rows; ++r) {
    const int8_t* wr = w + (size_t)r * k;
    for (int g = 0; g < groups; ++g) {
      const int begin = g * 128, end = begin + 128 < k ? begin + 128 : k;
      int total = 0;
      for (int i = begin; i < end; ++i) total += (int)wr[i] * (int)q[i];
      out[(size_t)r * groups + g] = total;
    }
  }
}

/* fp32 outputs of m x rows from int32 partials [m][rows][G], in one of the
 * kernels' orders: order 0 = GEMV lane pairs (param = lanes), order 1 = GEMM
 * K-split (param = splits).  scale_in: per-token scale; epilogue as above. */
void orc_finish(int order, int param, int epi, const int32_t* partials, const uint16_t* scales, int groups_stride,
                const float* scale_in, const float* bias, float* out, int rows, int k, int out_stride, int m) {
  const int groups = (k + 127) / 128;
  /* Tokens are independent: each thread finishes whole token rows with buffers of its own. */
#pragma omp parallel
  {
    float* y = (float*)malloc(sizeof(float) * (size_t)(rows > 0 ? rows : 1));
    float* acc = (float*)malloc(sizeof(float) * (size_t)(param > 0 ? param : 1));
    float* next = (float*)malloc(sizeof(float) * (size_t)(param > 0 ? param : 1));
#pragma omp for schedule(static)
    for (int t = 0; t < m; ++t) {
      for (int r = 0; r < rows; ++r) {
        const int32_t* p = partials + ((size_t)t * rows + r) * groups;
        const uint16_t* s = scales + (size_t)r * groups_stride;
        float total = 0.0f;
        if (order == 0) {
          const int pairs = param / 2;
          for (int i = 0; i < pairs; ++i) acc[i] = 0.0f;
          for (int g = 0; g < groups; ++g) acc[g % pairs] = fmaf((float)p[g], orc_h2f(s[g]), acc[g % pairs]);
          for (int offset = 1; offset < pairs; offset <<= 1) {
            for (int i = 0; i < pairs; ++i) next[i] = acc[i] + acc[i ^ offset];
            memcpy(acc, next, sizeof(float) * (size_t)pairs);
          }
          total = acc[0];
        } else {
          const int per = (groups + param - 1) / param;
          for (int sp = 0; sp < param; ++sp) {
            const int begin = sp * per < groups ? sp * per : groups;
            const int end = begin + per < groups ? begin + per : groups;
            float a = 0.0f;
            for (int g = begin; g < end; ++g) a = fmaf((float)p[g], orc_h2f(s[g]), a);
            total = sp == 0 ? a : total + a;
          }
        }
        float v = total * scale_in[t];
        if (bias) v = v + bias[r];
        y[r] = v;
      }
      float* orow = out + (size_t)t * out_stride;
      for (int r = 0; r < rows; ++r) {
        if (epi == EPI_SILU_PAIR) {
          if ((r & 1) == 0 && r + 1 < rows) epilogue(epi, orow, r >> 1, r, y[r], y[r + 1]);
        } else {
          epilogue(epi, orow, r, r, y[r], 0.0f);
        }
      }
    }
    free(next);
    free(acc);
    free(y);
  }
}

/* First index of the maximum (greedy decoding). */
int64_t orc_argmax(const float* x, int n) {
  int64_t best = 0;
  for (int i = 1; i < n; ++i)
    if (x[i] > x[best]) best = i;
  return best;
}

/* ------------------------------------------------------------------ sampler
 * The sampling rule of the reference's logit_bounds / sample_token
 * (kernels/ternary.cu:984-1097 scores and bounds, :1098-1337 top-k, softmax
 * and inverse-CDF draw; torch form decoder.py:324-333), with the picks in
 * ascending index order and the fp32 CDF order of the HIP sampler:
 * per 64 picks a Hillis-Steele inclusive scan, wave totals added in wave
 * order.  Keys order floats as numbers with -NaN lowest and +NaN highest;
 * equal keys at the top-k cut are taken lowest index first. */
static inline uint32_t order_key(float v) {
  uint32_t u;
  memcpy(&u, &v, 4);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

static inline float key_value(uint32_t key) {
  return as_float((key & 0x80000000u) ? (key & 0x7fffffffu) : ~key);
}

/* ternary.cu:990-996 */
static inline float sample_score(const float* logits, const uint8_t* seen, int i, float inv_t, float pen,
                                 float inv_pen) {
  float s = logits[i] * inv_t;
  if (seen[i]) s *= s > 0.0f ? inv_pen : pen;
  return s;
}

/* ternary.cu:1083-1092: the largest score of each 64-entry group. */
void orc_logit_bounds(const float* logits, float temperature, float penalty, float inverse_penalty,
                      const uint8_t* seen, float* bounds, int vocab) {
  const float inv_t = 1.0f / temperature;
  const int groups = (vocab + 63) / 64;
  for (int g = 0; g < groups; ++g) {
    uint32_t best = 0u;
    for (int i = g * 64; i < g * 64 + 64 && i < vocab; ++i) {
      const uint32_t key = order_key(sample_score(logits, seen, i, inv_t, penalty, inverse_penalty));
      if (key > best) best = key;
    }
    bounds[g] = key_value(best);
  }
}

typedef struct {
  uint32_t key;
  int index;
} keyed_t;

static int by_rank(const void* a, const void* b) {
  const keyed_t* x = (const keyed_t*)a;
  const keyed_t* y = (const keyed_t*)b;
  if (x->key != y->key) return x->key > y->key ? -1 : 1;
  return x->index < y->index ? -1 : (x->index > y->index);
}

static int by_index(const void* a, const void* b) {
  const keyed_t* x = (const keyed_t*)a;
  const keyed_t* y = (const keyed_t*)b;
  return x->index < y->index ? -1 : (x->index > y->index);
}

/* ternary.cu:1098-1337.  Returns the token and sets seen[token] = 1; picks
 * (ascending index) and their CDF go to picks/cdf (k entries each) when not
 * NULL, k to *count. */
int64_t orc_sample_token(const float* logits, float temperature, float penalty, float inverse_penalty,
                         uint8_t* seen, int64_t top_k, int max_topk, float uniform, int vocab, int* picks, float* cdf,
                         int* count) {
  const float inv_t = 1.0f / temperature;
  int64_t limit = max_topk < vocab ? max_topk : vocab;
  int64_t kk = top_k < limit ? top_k : limit;
  const int k = (int)(kk < 1 ? 1 : kk);
  keyed_t* all = (keyed_t*)malloc(sizeof(keyed_t) * (size_t)vocab);
  for (int i = 0; i < vocab; ++i) {
    all[i].key = order_key(sample_score(logits, seen, i, inv_t, penalty, inverse_penalty));
    all[i].index = i;
  }
  qsort(all, (size_t)vocab, sizeof(keyed_t), by_rank);
  const float peak = key_value(all[0].key);
  qsort(all, (size_t)k, sizeof(keyed_t), by_index);
  /* 1024 slots as in the one-block kernel; slots past k hold 0. */
  float run[1024], wave_sum[16], c[1024];
  for (int j = 0; j < 1024; ++j) run[j] = j < k ? orc_expf(key_value(all[j].key) - peak) : 0.0f;
  for (int w = 0; w < 16; ++w) {
    float* r = run + 64 * w;
    for (int offset = 1; offset < 64; offset <<= 1) {
      float old[64];
      memcpy(old, r, sizeof(old));
      for (int l = offset; l < 64; ++l) r[l] = old[l] + old[l - offset];
    }
    wave_sum[w] = r[63];
  }
  for (int j = 0; j < 1024; ++j) {
    float carry = 0.0f;
    for (int w = 0; w < j / 64; ++w) carry += wave_sum[w];
    c[j] = carry + run[j];
  }
  const float total = c[k - 1];
  const float target = fminf(uniform, 0.99999994f) * total;
  int chosen = -1;
  for (int j = 0; j < k; ++j) {
    const float lower = j > 0 ? c[j - 1] : 0.0f;
    if (lower <= target && target < c[j]) {
      chosen = j;
      break;
    }
  }
  if (chosen < 0) chosen = k - 1;
  const int token = all[chosen].index;
  if (picks != NULL)
    for (int j = 0; j < k; ++j) picks[j] = all[j].index;
  if (cdf != NULL) memcpy(cdf, c, sizeof(float) * (size_t)k);
  if (count != NULL) *count = k;
  free(all);
  seen[token] = 1;
  return token;
}
