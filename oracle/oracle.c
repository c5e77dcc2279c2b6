/*
 * CPU oracle for the logan-hip hot path. TEST INFRASTRUCTURE ONLY: loaded by
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, never by
 * the library. Each function restates the reference CPU arithmetic it cites;
 * compile with -ffp-contract=off so every f32 operation rounds like Rust's.
 */
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

static uint32_t rd_u32le(const uint8_t *p) {
  return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) |
         ((uint32_t)p[3] << 24);
}

static float f32_from_bits(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static uint32_t f32_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}

/* logan-qwen4/src/ggufsource.rs:1968-1991 */
float lo_f16_to_f32(uint16_t bits) {
  uint32_t sign = ((uint32_t)(bits & 0x8000u)) << 16;
  int exp = (bits >> 10) & 0x1f;
  uint32_t frac = bits & 0x03ffu;
  uint32_t out;
  if (exp == 0) {
    if (frac == 0) {
      out = sign;
    } else {
      uint32_t mant = frac;
      int e = -14;
      while ((mant & 0x0400u) == 0) {
        mant <<= 1;
        e -= 1;
      }
      mant &= 0x03ffu;
      out = sign | ((uint32_t)(e + 127) << 23) | (mant << 13);
    }
  } else if (exp == 31) {
    out = sign | 0x7f800000u | (frac << 13);
  } else {
    out = sign | ((uint32_t)(exp - 15 + 127) << 23) | (frac << 13);
  }
  return f32_from_bits(out);
}

/* logan-core/src/math.rs:279-283 */
uint16_t lo_f32_to_bf16(float f) {
  uint32_t bits = f32_bits(f);
  uint32_t rounding = 0x7fffu + ((bits >> 16) & 1u);
  return (uint16_t)((bits + rounding) >> 16);
}

/* logan-core/src/math.rs:289-291 */
float lo_bf16_to_f32(uint16_t b) { return f32_from_bits((uint32_t)b << 16); }

/* logan-qwen4/src/lib.rs:3688-3701 */
uint32_t lo_affine_code(const uint8_t *row, size_t column, int bits) {
  size_t bit = column * (size_t)bits;
  size_t word_index = bit / 32;
  unsigned shift = (unsigned)(bit % 32);
  size_t byte = word_index * 4;
  uint64_t lo = rd_u32le(row + byte);
  uint64_t combined = lo;
  if (shift + (unsigned)bits > 32) {
    uint64_t next = rd_u32le(row + byte + 4);
    combined = lo | (next << 32);
  }
  return (uint32_t)((combined >> shift) & ((1ull << bits) - 1));
}

/* logan-qwen4/src/lib.rs:3678-3686 */
float lo_affine_param(const uint8_t *bytes, size_t index, int fp16) {
  size_t off = index * 2;
  uint16_t bits = (uint16_t)(bytes[off] | (bytes[off + 1] << 8));
  return fp16 ? lo_f16_to_f32(bits) : lo_bf16_to_f32(bits);
}

/* logan-qwen4/src/colisource.rs:779-856 (geometry checks :788-833, element
 * formula :836-852) and lib.rs:3703-3727 (the same formula per row). */
int lo_affine_dequant(float *out, const uint8_t *w, const uint8_t *scales,
                      const uint8_t *biases, size_t rows, size_t cols, int bits,
                      size_t group_size, int fp16, size_t row0, size_t nrows) {
  if (!(bits == 4 || bits == 5 || bits == 6 || bits == 8)) return -1;
  if (rows == 0 || cols == 0 || group_size == 0 || cols % group_size != 0)
    return -1;
  if ((cols * (size_t)bits) % 32 != 0) return -1;
  if (row0 + nrows > rows) return -1;
  size_t row_bytes = cols * (size_t)bits / 8;
  size_t groups = cols / group_size;
  for (size_t r = 0; r < nrows; ++r) {
    size_t row = row0 + r;
    const uint8_t *wr = w + row * row_bytes;
    for (size_t c = 0; c < cols; ++c) {
      size_t g = row * groups + c / group_size;
      float code = (float)lo_affine_code(wr, c, bits);
      float prod = code * lo_affine_param(scales, g, fp16);
      out[r * cols + c] = prod + lo_affine_param(biases, g, fp16);
    }
  }
  return 0;
}

/* One row of logan-qwen4/src/lib.rs:3752-3763. */
static float affine_row_dot(const float *x, const uint8_t *w,
                            const uint8_t *scales, const uint8_t *biases,
                            size_t row, size_t i, int bits, size_t group_size,
                            int fp16) {
  size_t row_bytes = i * (size_t)bits / 8;
  size_t groups = i / group_size;
  const uint8_t *wr = w + row * row_bytes;
  float sum = 0.0f;
  for (size_t column = 0; column < i; ++column) {
    size_t group = row * groups + column / group_size;
    float value = (float)lo_affine_code(wr, column, bits) *
                  lo_affine_param(scales, group, fp16);
    value = value + lo_affine_param(biases, group, fp16);
    float prod = value * x[column];
    sum = sum + prod;
  }
  return sum;
}

/* logan-qwen4/src/lib.rs:3729-3764 */
void lo_affine_gemv(float *y, const float *x, const uint8_t *w,
                    const uint8_t *scales, const uint8_t *biases, size_t o,
                    size_t i, int bits, size_t group_size, int fp16) {
  for (size_t row = 0; row < o; ++row)
    y[row] = affine_row_dot(x, w, scales, biases, row, i, bits, group_size,
                            fp16);
}

/* logan-metal/metal/backend_metal.mm:1480-1560 (spark_qmm_affine8_t16o8):
 * the prefill product with every dequantised weight rounded to bf16 (RNE,
 * logan-core/src/math.rs:279-283) before the products, accumulated in f32.
 * x[m * i + k] are the (bf16-valued) activations; y[m * o + n] f32 before the
 * caller's bf16 rounding. Sequential k order. */
void lo_affine_qmm_bf16(float *y, const float *x, const uint8_t *w,
                        const uint8_t *scales, const uint8_t *biases, size_t m,
                        size_t o, size_t i, int bits, size_t group_size,
                        int fp16) {
  size_t row_bytes = i * (size_t)bits / 8;
  size_t groups = i / group_size;
  float *wq = (float *)malloc(sizeof(float) * i);
  for (size_t n = 0; n < o; ++n) {
    const uint8_t *wr = w + n * row_bytes;
    for (size_t k = 0; k < i; ++k) {
      size_t group = n * groups + k / group_size;
      float value = (float)lo_affine_code(wr, k, bits) *
                    lo_affine_param(scales, group, fp16);
      value = value + lo_affine_param(biases, group, fp16);
      wq[k] = lo_bf16_to_f32(lo_f32_to_bf16(value));
    }
    for (size_t r = 0; r < m; ++r) {
      float sum = 0.0f;
      for (size_t k = 0; k < i; ++k) {
        float prod = wq[k] * x[r * i + k];
        sum = sum + prod;
      }
      y[r * o + n] = sum;
    }
  }
  free(wq);
}

typedef struct gemv_job {
  float *y;
  const float *x;
  const uint8_t *w, *scales, *biases;
  size_t r0, r1, i, group_size;
  int bits, fp16;
} gemv_job;

static void *gemv_worker(void *arg) {
  gemv_job *j = (gemv_job *)arg;
  for (size_t row = j->r0; row < j->r1; ++row)
    j->y[row] = affine_row_dot(j->x, j->w, j->scales, j->biases, row, j->i,
                               j->bits, j->group_size, j->fp16);
  return NULL;
}

/* Row split as logan-qwen4/src/lib.rs:3785-3807 (chunk = ceil(o/workers)). */
void lo_affine_gemv_mt(float *y, const float *x, const uint8_t *w,
                       const uint8_t *scales, const uint8_t *biases, size_t o,
                       size_t i, int bits, size_t group_size, int fp16,
                       int threads) {
  if (threads <= 1 || o < 2) {
    lo_affine_gemv(y, x, w, scales, biases, o, i, bits, group_size, fp16);
    return;
  }
  if ((size_t)threads > o) threads = (int)o;
  size_t chunk = (o + (size_t)threads - 1) / (size_t)threads;
  pthread_t *tid = (pthread_t *)malloc(sizeof(pthread_t) * (size_t)threads);
  gemv_job *jobs = (gemv_job *)malloc(sizeof(gemv_job) * (size_t)threads);
  int n = 0;
  for (int t = 0; t < threads; ++t) {
    size_t r0 = (size_t)t * chunk;
    if (r0 >= o) break;
    size_t r1 = r0 + chunk < o ? r0 + chunk : o;
    jobs[n] = (gemv_job){y, x, w, scales, biases, r0, r1, i, group_size, bits,
                         fp16};
    if (pthread_create(&tid[n], NULL, gemv_worker, &jobs[n]) != 0) {
      gemv_worker(&jobs[n]);
      tid[n] = 0;
    }
    ++n;
  }
  for (int t = 0; t < n; ++t)
    if (tid[t]) pthread_join(tid[t], NULL);
  free(tid);
  free(jobs);
}

/* logan-spark/src/lib.rs:346-367 with f32_to_bf16 of lib.rs:254-258. */
void lo_spark_affine8_gemv(float *y, const float *x, const uint8_t *w,
                           const uint8_t *aux, size_t o, size_t i) {
  const size_t G = 64;
  size_t ng = i / G;
  float *xsum = (float *)calloc(ng ? ng : 1, sizeof(float));
  for (size_t g = 0; g < ng; ++g) {
    float s = 0.0f;
    for (size_t j = 0; j < G; ++j) s = s + x[g * G + j];
    xsum[g] = s;
  }
  for (size_t row = 0; row < o; ++row) {
    const uint8_t *wr = w + row * i;
    float acc = 0.0f;
    for (size_t g = 0; g < ng; ++g) {
      float sc = lo_affine_param(aux, row * ng + g, 0);
      float bi = lo_affine_param(aux, o * ng + row * ng + g, 0);
      size_t start = g * G;
      float dot = 0.0f;
      for (size_t j = 0; j < G; ++j) {
        float p = (float)wr[start + j] * x[start + j];
        dot = dot + p;
      }
      float a = sc * dot;
      float b = bi * xsum[g];
      acc = acc + (a + b);
    }
    uint32_t u = f32_bits(acc);
    uint32_t rounded = u + (0x7fffu + ((u >> 16) & 1u));
    y[row] = f32_from_bits(rounded & 0xffff0000u);
  }
  free(xsum);
}

/* MXFP4 (OCP microscaling FP4, fmt 7): two E2M1 codes per byte, element 2j
 * in the low nibble; one E8M0 scale byte per 32 columns, scale = the f32
 * with bits byte << 23 (logan-qwen4/src/lib.rs:2932-2961, matmul_mxfp4_bytes;
 * nibble order as :17676-17694). */
static const float kMx4[16] = {0.0f,  0.5f,  1.0f,  1.5f,  2.0f,  3.0f,  4.0f,  6.0f,
                               -0.0f, -0.5f, -1.0f, -1.5f, -2.0f, -3.0f, -4.0f, -6.0f};

float lo_mxfp4_value(uint8_t code, uint8_t scale_byte) {
  return kMx4[code & 0xf] * f32_from_bits((uint32_t)scale_byte << 23);
}

/* y[r] = sum_col x[col] * MX4[code] * scale, in column order (lib.rs:2948-2961) */
void lo_mxfp4_gemv(float *y, const float *x, const uint8_t *w, const uint8_t *sc, size_t o,
                   size_t i) {
  size_t rb = (i + 1) / 2, ng = (i + 31) / 32;
  for (size_t row = 0; row < o; ++row) {
    const uint8_t *wr = w + row * rb;
    const uint8_t *sr = sc + row * ng;
    float acc = 0.0f;
    for (size_t col = 0; col < i; ++col) {
      uint8_t packed = wr[col / 2];
      uint8_t code = (col & 1) == 0 ? (packed & 0x0f) : (packed >> 4);
      float scale = f32_from_bits((uint32_t)sr[col / 32] << 23);
      acc = acc + (x[col] * kMx4[code]) * scale;
    }
    y[row] = acc;
  }
}

/* fmt 7 / 9 / 10: one, two or three stacked MXFP4 planes, the later ones
 * residual corrections added to the first plane's result in order
 * (lib.rs:2985-3038, matmul_mxfp4_storage). */
void lo_mxfp4_gemv_stacked(float *y, const float *x, const uint8_t *w, const uint8_t *sc,
                           size_t o, size_t i, int stacks) {
  size_t wb = o * ((i + 1) / 2), sb = o * ((i + 31) / 32);
  lo_mxfp4_gemv(y, x, w, sc, o, i);
  float *r = (float *)malloc(sizeof(float) * (o ? o : 1));
  for (int s = 1; s < stacks; ++s) {
    lo_mxfp4_gemv(r, x, w + (size_t)s * wb, sc + (size_t)s * sb, o, i);
    for (size_t k = 0; k < o; ++k) y[k] = y[k] + r[k];
  }
  free(r);
}

/* In-place RMSNorm of nrows rows of n: the Metal kernel a_rmsnorm
 * (logan-metal/metal/backend_metal.mm:705-714, x * rsqrt(mean(x^2) + eps) *
 * w), with the sum of squares in double and the scale formed as
 * logan-core/src/math.rs:207-216 forms it (that CPU routine multiplies by
 * 1 + w; the Metal kernel that coli_metal_rmsnorm runs multiplies by w). */
void lo_rmsnorm(float *x, const float *w, size_t n, size_t nrows, float eps) {
  for (size_t r = 0; r < nrows; ++r) {
    float *xr = x + r * n;
    double ms = 0.0;
    for (size_t i = 0; i < n; ++i) ms += (double)xr[i] * (double)xr[i];
    float q = (float)ms / (float)n + eps;
    float sc = 1.0f / sqrtf(q);
    for (size_t i = 0; i < n; ++i) xr[i] = xr[i] * sc * w[i];
  }
}

/* y[i] += a[i] (backend_metal.mm:782-783, a_add) */
void lo_add(float *y, const float *a, size_t n) {
  for (size_t i = 0; i < n; ++i) y[i] = y[i] + a[i];
}

/* logan-qwen4/src/lib.rs:4516-4518 */
float lo_silu(float x) {
  float e = expf(-x);
  float d = 1.0f + e;
  return x / d;
}

/* Dense SwiGLU in place, g[i] = silu(g[i]) * u[i]
 * (logan-metal/metal/backend_metal.mm:698-699, moe_silu). */
void lo_silu_mul(float *g, const float *u, size_t n) {
  for (size_t i = 0; i < n; ++i) g[i] = lo_silu(g[i]) * u[i];
}

/* logan-qwen4/src/lib.rs:4558-4574 */
void lo_softmax_row(float *x, size_t n) {
  float m = -1e30f;
  for (size_t i = 0; i < n; ++i)
    if (x[i] > m) m = x[i];
  float s = 0.0f;
  for (size_t i = 0; i < n; ++i) {
    x[i] = expf(x[i] - m);
    s = s + x[i];
  }
  for (size_t i = 0; i < n; ++i) x[i] = x[i] / s;
}

/* logan-qwen4/src/lib.rs:7993-8043 */
float lo_topk(const float *probs, size_t n, size_t k, int32_t *idx_out,
              float *val_out) {
  size_t *idx = (size_t *)malloc(sizeof(size_t) * n);
  float *val = (float *)malloc(sizeof(float) * n);
  for (size_t i = 0; i < n; ++i) {
    idx[i] = i;
    val[i] = probs[i];
  }
  if (k > n) k = n;
  for (size_t i = 0; i < k; ++i) {
    size_t best = i;
    for (size_t j = i + 1; j < n; ++j) {
      if (val[j] > val[best] || (val[j] == val[best] && idx[j] < idx[best]))
        best = j;
    }
    size_t ti = idx[i];
    idx[i] = idx[best];
    idx[best] = ti;
    float tv = val[i];
    val[i] = val[best];
    val[best] = tv;
  }
  float wsum = 0.0f;
  for (size_t i = 0; i < k; ++i) wsum = wsum + val[i];
  for (size_t i = 0; i < k; ++i) {
    idx_out[i] = (int32_t)idx[i];
    val_out[i] = val[i];
  }
  free(idx);
  free(val);
  return wsum;
}

static void bank_gemv(float *y, const float *x, const lo_bank *b, size_t e,
                      int threads) {
  size_t row_bytes = b->i * (size_t)b->bits / 8;
  size_t groups = b->i / b->group_size;
  const uint8_t *w = b->w + e * b->o * row_bytes;
  const uint8_t *sc = b->scales + e * b->o * groups * 2;
  const uint8_t *bi = b->biases + e * b->o * groups * 2;
  lo_affine_gemv_mt(y, x, w, sc, bi, b->o, b->i, b->bits, b->group_size,
                    b->fp16, threads);
}

/* Expert MLP: logan-qwen4/src/lib.rs:8803-8812 (and :7745-7757 for the
 * shared expert): h = silu(gate.x) * (up.x); y = down.h. */
static void expert_mlp(float *y, const float *x, const lo_bank *gate,
                       const lo_bank *up, const lo_bank *down, size_t e,
                       int threads) {
  size_t inter = gate->o;
  float *g = (float *)malloc(sizeof(float) * inter);
  float *u = (float *)malloc(sizeof(float) * inter);
  bank_gemv(g, x, gate, e, threads);
  bank_gemv(u, x, up, e, threads);
  for (size_t ii = 0; ii < inter; ++ii) u[ii] = lo_silu(g[ii]) * u[ii];
  bank_gemv(y, u, down, e, threads);
  free(g);
  free(u);
}

static void moe_token_impl(float *out, const float *x, const float *logits,
                           size_t E, size_t k, size_t D, const lo_bank *gate,
                           const lo_bank *up, const lo_bank *down,
                           const lo_bank *se_gate, const lo_bank *se_up,
                           const lo_bank *se_down, const float *se_g,
                           int32_t *idx_out, float *w_out, int threads) {
  float *probs = (float *)malloc(sizeof(float) * E);
  memcpy(probs, logits, sizeof(float) * E);
  lo_softmax_row(probs, E);
  int32_t *idx = (int32_t *)malloc(sizeof(int32_t) * (k ? k : 1));
  float *val = (float *)malloc(sizeof(float) * (k ? k : 1));
  float wsum = lo_topk(probs, E, k, idx, val);
  float *acc = (float *)calloc(D, sizeof(float));
  float *y = (float *)malloc(sizeof(float) * D);
  /* logan-qwen/src/lib.rs:559-576: rank-ordered accumulation */
  for (size_t r = 0; r < k; ++r) {
    float w = val[r] / wsum;
    if (idx_out) idx_out[r] = idx[r];
    if (w_out) w_out[r] = w;
    expert_mlp(y, x, gate, up, down, (size_t)idx[r], threads);
    for (size_t dd = 0; dd < D; ++dd) acc[dd] = acc[dd] + y[dd] * w;
  }
  if (se_g && se_gate && se_up && se_down) {
    /* logan-qwen4/src/lib.rs:7602-7604: gs = sigmoid(se_g . x) */
    float sg = 0.0f;
    for (size_t j = 0; j < D; ++j) sg = sg + se_g[j] * x[j];
    float gs = 1.0f / (1.0f + expf(-sg));
    expert_mlp(y, x, se_gate, se_up, se_down, 0, threads);
    /* logan-qwen4/src/lib.rs:8708-8710: out = acc + sy*gs */
    for (size_t dd = 0; dd < D; ++dd) out[dd] = acc[dd] + y[dd] * gs;
  } else {
    memcpy(out, acc, sizeof(float) * D);
  }
  free(probs);
  free(idx);
  free(val);
  free(acc);
  free(y);
}

void lo_moe_token(float *out, const float *x, const float *logits, size_t E,
                  size_t k, size_t D, const lo_bank *gate, const lo_bank *up,
                  const lo_bank *down, const lo_bank *se_gate,
                  const lo_bank *se_up, const lo_bank *se_down,
                  const float *se_g, int32_t *idx_out, float *w_out) {
  moe_token_impl(out, x, logits, E, k, D, gate, up, down, se_gate, se_up,
                 se_down, se_g, idx_out, w_out, 1);
}

void lo_moe_token_mt(float *out, const float *x, const float *logits, size_t E,
                     size_t k, size_t D, const lo_bank *gate, const lo_bank *up,
                     const lo_bank *down, const lo_bank *se_gate,
                     const lo_bank *se_up, const lo_bank *se_down,
                     const float *se_g, int32_t *idx_out, float *w_out,
                     int threads) {
  moe_token_impl(out, x, logits, E, k, D, gate, up, down, se_gate, se_up,
                 se_down, se_g, idx_out, w_out, threads);
}

/* ---- dense Llama decode layer (logan-llama/src/model.rs:786-905) ---------- */

/* One bf16-valued weight: fmt 5 holds the bf16 bits (weights dequantised and
 * rounded at load, logan-llama/src/weights.rs:441-516, :548-552); fmt 15
 * forms RNE_bf16(code * scale + bias) from an affine-8 code and its group's
 * bf16 scale/bias (the same value; spark_qmv_affine8_fast,
 * logan-metal/metal/backend_metal.mm:1143-1193). */
static float dense_weight(const void *w, const uint16_t *sc, const uint16_t *bi, int fmt,
                          size_t I, size_t row, size_t col) {
  if (fmt == 5) return lo_bf16_to_f32(((const uint16_t *)w)[row * I + col]);
  const size_t g = row * (I / 64) + col / 64;
  const float code = (float)((const uint8_t *)w)[row * I + col];
  const float v = code * lo_bf16_to_f32(sc[g]) + lo_bf16_to_f32(bi[g]);
  return lo_bf16_to_f32(lo_f32_to_bf16(v));
}

/* linear_cpu_into (model.rs:1025-1033): y[r] = sum_j w[r][j] * x[j], f32 in
 * column order */
void lo_dense_gemv(float *y, const float *x, const void *w, const uint16_t *sc,
                   const uint16_t *bi, int fmt, size_t O, size_t I) {
  for (size_t r = 0; r < O; ++r) {
    float acc = 0.0f;
    for (size_t j = 0; j < I; ++j) acc = acc + dense_weight(w, sc, bi, fmt, I, r, j) * x[j];
    y[r] = acc;
  }
}

/* rms_norm_into (model.rs:1067-1073): f32 sum of squares in order */
static void llama_rms(const float *x, const float *w, float eps, size_t n, float *out) {
  float s = 0.0f;
  for (size_t i = 0; i < n; ++i) s = s + x[i] * x[i];
  const float mean = s / (float)n;
  const float inv = 1.0f / sqrtf(mean + eps);
  for (size_t i = 0; i < n; ++i) out[i] = x[i] * inv * w[i];
}

/* rope (model.rs:1087-1100) with the angles of :790-796 */
static void llama_rope(float *x, int heads, int hd, int pos, float theta) {
  const int half = hd / 2;
  for (int h = 0; h < heads; ++h)
    for (int i = 0; i < half; ++i) {
      const float ang = (float)pos / powf(theta, (float)(2 * i) / (float)hd);
      const float co = cosf(ang), si = sinf(ang);
      const float a = x[h * hd + i], b = x[h * hd + half + i];
      x[h * hd + i] = a * co - b * si;
      x[h * hd + half + i] = a * si + b * co;
    }
}

/* One decode layer at position pos for one token (model.rs:810-905 with
 * rows = 1): kc / vc [pos + 1][kv_heads * hd] hold positions 0..pos-1 on
 * entry; row pos is written (K after RoPE). x[D] is updated in place. mats
 * are q, k, v, o, gate, up, down. Returns 0 on bad arguments. */
int lo_llama_layer(float *x, float *kc, float *vc, int pos, const void *const *w,
                   const uint16_t *const *sc, const uint16_t *const *bi, const int *fmt,
                   const float *in_norm, const float *post_norm, int D, int inter, int H, int KH,
                   int hd, float theta, float eps) {
  if (D <= 0 || inter <= 0 || H <= 0 || KH <= 0 || H % KH != 0 || hd <= 0 || hd % 2 != 0 ||
      pos < 0)
    return 0;
  const int qdim = H * hd, kvdim = KH * hd, T = pos + 1;
  float *norm = malloc(sizeof(float) * D), *q = malloc(sizeof(float) * qdim);
  float *att = calloc((size_t)qdim, sizeof(float)), *proj = malloc(sizeof(float) * D);
  float *g = malloc(sizeof(float) * inter), *u = malloc(sizeof(float) * inter);
  float *scores = malloc(sizeof(float) * T);
  float *krow = kc + (size_t)pos * kvdim, *vrow = vc + (size_t)pos * kvdim;
  llama_rms(x, in_norm, eps, D, norm);
  lo_dense_gemv(q, norm, w[0], sc[0], bi[0], fmt[0], qdim, D);
  lo_dense_gemv(krow, norm, w[1], sc[1], bi[1], fmt[1], kvdim, D);
  lo_dense_gemv(vrow, norm, w[2], sc[2], bi[2], fmt[2], kvdim, D);
  llama_rope(q, H, hd, pos, theta);
  llama_rope(krow, KH, hd, pos, theta);
  /* model.rs:838-869 */
  for (int h = 0; h < H; ++h) {
    const int grp = h / (H / KH);
    const float *qh = q + h * hd;
    for (int t = 0; t < T; ++t) {
      const float *k = kc + (size_t)t * kvdim + grp * hd;
      float s = 0.0f;
      for (int z = 0; z < hd; ++z) s = s + qh[z] * k[z];
      scores[t] = s / sqrtf((float)hd);
    }
    /* softmax, model.rs:1075-1086 */
    float m = -INFINITY, tot = 0.0f;
    for (int t = 0; t < T; ++t) m = fmaxf(m, scores[t]);
    for (int t = 0; t < T; ++t) {
      scores[t] = expf(scores[t] - m);
      tot = tot + scores[t];
    }
    if (tot != 0.0f)
      for (int t = 0; t < T; ++t) scores[t] = scores[t] / tot;
    for (int t = 0; t < T; ++t) {
      const float *v = vc + (size_t)t * kvdim + grp * hd;
      for (int z = 0; z < hd; ++z) att[h * hd + z] = att[h * hd + z] + scores[t] * v[z];
    }
  }
  lo_dense_gemv(proj, att, w[3], sc[3], bi[3], fmt[3], D, qdim);
  for (int z = 0; z < D; ++z) x[z] = x[z] + proj[z];
  llama_rms(x, post_norm, eps, D, norm);
  lo_dense_gemv(g, norm, w[4], sc[4], bi[4], fmt[4], inter, D);
  lo_dense_gemv(u, norm, w[5], sc[5], bi[5], fmt[5], inter, D);
  for (int i = 0; i < inter; ++i) g[i] = g[i] / (1.0f + expf(-g[i])) * u[i];
  lo_dense_gemv(proj, g, w[6], sc[6], bi[6], fmt[6], D, inter);
  for (int z = 0; z < D; ++z) x[z] = x[z] + proj[z];
  free(norm);
  free(q);
  free(att);
  free(proj);
  free(g);
  free(u);
  free(scores);
  return 1;
}
