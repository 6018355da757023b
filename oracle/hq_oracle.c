/*
 * hq_oracle.c -- CPU oracle for the MLX affine group-quantized linear path.
 *
 * TEST INFRASTRUCTURE ONLY (see hq_oracle.h): the checker for the HIP path
 * and the timed CPU baseline, never part of the shipped library.
 *
 * Build: oracle/build_oracle.sh (gcc, -ffp-contract=off so that every
 * multiply and add rounds on its own, as MLX's op-by-op CPU path does).
 */
#include "hq_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------ */
/* scalar conversions                                                        */
/* ------------------------------------------------------------------------ */

static uint32_t f2u(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}

static float u2f(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

uint16_t hqo_f32_to_bf16(float f) {
  uint32_t u = f2u(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

float hqo_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

uint16_t hqo_f32_to_f16(float f) {
  uint32_t u = f2u(f);
  uint32_t sign = (u >> 16) & 0x8000u;
  uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);
  if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 -> inf */
  if (a < 0x38800000u) {                                    /* below 2^-14 */
    uint32_t e = a >> 23;
    if (e < 102u) return (uint16_t)sign; /* < 2^-25 (ties at 2^-25 go to 0) */
    uint32_t m = (a & 0x7fffffu) | 0x800000u;
    uint32_t shift = 126u - e; /* 14..24 */
    uint32_t h = m >> shift;
    uint32_t rem = m & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (h & 1u))) h++;
    return (uint16_t)(sign | h);
  }
  uint32_t h = (((a >> 23) - 112u) << 10) | ((a & 0x7fffffu) >> 13);
  uint32_t rem = a & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
  return (uint16_t)(sign | h);
}

float hqo_f16_to_f32(uint16_t h) {
  uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
  uint32_t e = ((uint32_t)h >> 10) & 0x1fu;
  uint32_t m = (uint32_t)h & 0x3ffu;
  if (e == 0) {
    float v = ldexpf((float)m, -24);
    return sign ? -v : v;
  }
  if (e == 31) return u2f(sign | 0x7f800000u | (m << 13));
  return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

/* Round a float to `dtype` and widen it back. */
static float round_dt(float v, int dtype) {
  if (dtype == HQO_BF16) return hqo_bf16_to_f32(hqo_f32_to_bf16(v));
  if (dtype == HQO_F16) return hqo_f16_to_f32(hqo_f32_to_f16(v));
  return v;
}

/* double -> float with round-to-odd, so that a following RNE to a format with
 * at most 22 significand bits equals a single RNE from the double. */
static float f64_to_f32_odd(double d) {
  float f = (float)d;
  if ((double)f == d || isnan(d) || isinf(f)) return f;
  if (fabs((double)f) > fabs(d)) f = nextafterf(f, 0.0f);
  return u2f(f2u(f) | 1u);
}

float hqo_round_f64(double v, int dtype) {
  if (dtype == HQO_F32) return (float)v;
  return round_dt(f64_to_f32_odd(v), dtype);
}

static float load_dt(const void* p, int dtype, int64_t i) {
  if (dtype == HQO_BF16) return hqo_bf16_to_f32(((const uint16_t*)p)[i]);
  if (dtype == HQO_F16) return hqo_f16_to_f32(((const uint16_t*)p)[i]);
  return ((const float*)p)[i];
}

static void store_dt(void* p, int dtype, int64_t i, float v) {
  if (dtype == HQO_BF16)
    ((uint16_t*)p)[i] = hqo_f32_to_bf16(v);
  else if (dtype == HQO_F16)
    ((uint16_t*)p)[i] = hqo_f32_to_f16(v);
  else
    ((float*)p)[i] = v;
}

void hqo_to_f32(const void* src, int dtype, int64_t n, float* dst) {
  for (int64_t i = 0; i < n; i++) dst[i] = load_dt(src, dtype, i);
}

void hqo_from_f32(const float* src, int64_t n, int dtype, void* dst) {
  for (int64_t i = 0; i < n; i++) store_dt(dst, dtype, i, src[i]);
}

/* MLX type promotion between two floating dtypes: equal stays, any mix of
 * distinct 16-bit types (or with float32) becomes float32. */
static int result_dtype(int a, int b) { return a == b ? a : HQO_F32; }

/* ------------------------------------------------------------------------ */
/* packing (qwen3_next.rs:969-988: nibble i of word j is element 8j+i)       */
/* ------------------------------------------------------------------------ */

static int bits_ok(int bits) {
  return bits == 2 || bits == 3 || bits == 4 || bits == 5 || bits == 6 || bits == 8;
}

static int group_ok(int g) { return g == 32 || g == 64 || g == 128; }

/* Element i of a row: bits [i*bits, i*bits+bits) of the LSB-first stream. */
static inline uint32_t get_q(const uint32_t* row, int64_t i, int bits) {
  int64_t bit = i * (int64_t)bits;
  int64_t wd = bit >> 5;
  int off = (int)(bit & 31);
  uint64_t v = (uint64_t)row[wd] >> off;
  if (off + bits > 32) v |= (uint64_t)row[wd + 1] << (32 - off);
  return (uint32_t)(v & ((1u << bits) - 1u));
}

void hqo_pack(const uint32_t* q, int64_t rows, int64_t cols, int bits, uint32_t* w) {
  int64_t P = cols * bits / 32;
  memset(w, 0, (size_t)(rows * P) * sizeof(uint32_t));
  uint32_t mask = (1u << bits) - 1u;
  for (int64_t r = 0; r < rows; r++) {
    uint32_t* row = w + r * P;
    for (int64_t i = 0; i < cols; i++) {
      uint64_t v = (uint64_t)(q[r * cols + i] & mask);
      int64_t bit = i * (int64_t)bits;
      int64_t wd = bit >> 5;
      int off = (int)(bit & 31);
      row[wd] |= (uint32_t)(v << off);
      if (off + bits > 32) row[wd + 1] |= (uint32_t)(v >> (32 - off));
    }
  }
}

void hqo_unpack(const uint32_t* w, int64_t rows, int64_t cols, int bits, uint32_t* q) {
  int64_t P = cols * bits / 32;
  for (int64_t r = 0; r < rows; r++)
    for (int64_t i = 0; i < cols; i++) q[r * cols + i] = get_q(w + r * P, i, bits);
}

/* ------------------------------------------------------------------------ */
/* dequantize (qwen3_next.rs:308-318 -> ops::dequantize)                     */
/* ------------------------------------------------------------------------ */

int hqo_dequantize(const uint32_t* w, const void* scales, const void* biases,
                   int64_t rows, int64_t K, int group_size, int bits, int dtype,
                   int fused, void* out) {
  if (!bits_ok(bits) || !group_ok(group_size) || K % group_size) return -1;
  int64_t P = K * bits / 32, G = K / group_size;
  for (int64_t r = 0; r < rows; r++) {
    const uint32_t* row = w + r * P;
    for (int64_t k = 0; k < K; k++) {
      uint32_t q = get_q(row, k, bits);
      float s = load_dt(scales, dtype, r * G + k / group_size);
      float b = load_dt(biases, dtype, r * G + k / group_size);
      float o;
      if (fused) {
        o = hqo_round_f64((double)q * (double)s + (double)b, dtype);
      } else {
        float p = round_dt((float)q * s, dtype); /* multiply(w, scales) */
        o = round_dt(p + b, dtype);              /* add(., biases) */
      }
      store_dt(out, dtype, r * K + k, o);
    }
  }
  return 0;
}

/* ------------------------------------------------------------------------ */
/* quantized_matmul, exact (fp64) reference                                  */
/* ------------------------------------------------------------------------ */

/* Dequantize a logical [R, C] quantized matrix (groups along C) to double. */
static void deq_f64(const uint32_t* w, const void* s, const void* b, int sdt,
                    int64_t R, int64_t C, int gs, int bits, double* out) {
  int64_t P = C * bits / 32, G = C / gs;
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < R; r++)
    for (int64_t c = 0; c < C; c++) {
      double sv = load_dt(s, sdt, r * G + c / gs);
      double bv = load_dt(b, sdt, r * G + c / gs);
      out[r * C + c] = sv * (double)get_q(w + r * P, c, bits) + bv;
    }
}

int hqo_qmm_f64(const void* x, int x_dtype, const uint32_t* w,
                const void* scales, const void* biases, int s_dtype,
                int64_t M, int64_t N, int64_t K, int transpose, int group_size,
                int bits, double* y) {
  if (!bits_ok(bits) || !group_ok(group_size)) return -1;
  if (transpose ? (K % group_size) : (N % group_size)) return -1;
  double* wd = (double*)malloc((size_t)(N * K) * sizeof(double));
  double* xd = (double*)malloc((size_t)(M * K) * sizeof(double));
  if (!wd || !xd) {
    free(wd);
    free(xd);
    return -2;
  }
  for (int64_t i = 0; i < M * K; i++) xd[i] = load_dt(x, x_dtype, i);
  if (transpose) {
    deq_f64(w, scales, biases, s_dtype, N, K, group_size, bits, wd); /* [N,K] */
#pragma omp parallel for collapse(2) schedule(static)
    for (int64_t m = 0; m < M; m++)
      for (int64_t n = 0; n < N; n++) {
        const double* xr = xd + m * K;
        const double* wr = wd + n * K;
        double acc = 0.0;
        for (int64_t k = 0; k < K; k++) acc += xr[k] * wr[k];
        y[m * N + n] = acc;
      }
  } else {
    deq_f64(w, scales, biases, s_dtype, K, N, group_size, bits, wd); /* [K,N] */
#pragma omp parallel for schedule(static)
    for (int64_t m = 0; m < M; m++) {
      double* yr = y + m * N;
      for (int64_t n = 0; n < N; n++) yr[n] = 0.0;
      for (int64_t k = 0; k < K; k++) {
        double xv = xd[m * K + k];
        const double* wr = wd + k * N;
        for (int64_t n = 0; n < N; n++) yr[n] += xv * wr[n];
      }
    }
  }
  free(wd);
  free(xd);
  return 0;
}

/* ------------------------------------------------------------------------ */
/* MLX-CPU-style quantized_matmul (the timed CPU baseline)                   */
/* ------------------------------------------------------------------------ */

int hqo_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

#define LANES 8

int hqo_qmm_mlx(const void* x, int x_dtype, const uint32_t* w,
                const void* scales, const void* biases, int s_dtype,
                int64_t M, int64_t N, int64_t K, int group_size, int bits,
                int threads, void* y) {
  if (!bits_ok(bits) || !group_ok(group_size) || K % group_size) return -1;
  int T = result_dtype(x_dtype, s_dtype);
  int64_t P = K * bits / 32, G = K / group_size;
#ifdef _OPENMP
  if (threads > 0) omp_set_num_threads(threads);
#else
  (void)threads;
#endif
  /* astype(x, T): values of x rounded to T (exact when promoting). */
  float* xt = (float*)malloc((size_t)(M * K) * sizeof(float));
  if (!xt) return -2;
  for (int64_t i = 0; i < M * K; i++) xt[i] = round_dt(load_dt(x, x_dtype, i), T);
  int pow2 = (bits == 2 || bits == 4 || bits == 8);

#pragma omp parallel for schedule(static)
  for (int64_t n = 0; n < N; n++) {
    const uint32_t* row = w + n * P;
    float wf[128];
    for (int64_t m = 0; m < M; m++) {
      const float* xr = xt + m * K;
      if (pow2) {
        float acc[LANES] = {0};
        for (int64_t g = 0; g < G; g++) {
          float s = round_dt(load_dt(scales, s_dtype, n * G + g), T);
          float b = round_dt(load_dt(biases, s_dtype, n * G + g), T);
          int64_t k0 = g * group_size;
          for (int i = 0; i < group_size; i++) {
            float v = (float)get_q(row, k0 + i, bits) * s;
            wf[i] = v + b;
          }
          for (int i = 0; i < group_size; i += LANES)
            for (int l = 0; l < LANES; l++) acc[l] = acc[l] + xr[k0 + i + l] * wf[i + l];
        }
        float sum = 0.0f;
        for (int l = 0; l < LANES; l++) sum += acc[l];
        store_dt(y, T, m * N + n, sum);
      } else {
        float sum = 0.0f; /* always holds a value of T */
        for (int64_t g = 0; g < G; g++) {
          float s = round_dt(load_dt(scales, s_dtype, n * G + g), T);
          float b = round_dt(load_dt(biases, s_dtype, n * G + g), T);
          int64_t k0 = g * group_size;
          for (int i = 0; i < group_size; i++) {
            float wq = round_dt(round_dt(s * (float)get_q(row, k0 + i, bits), T) + b, T);
            sum = round_dt(sum + round_dt(xr[k0 + i] * wq, T), T);
          }
        }
        store_dt(y, T, m * N + n, sum);
      }
    }
  }
  free(xt);
  return 0;
}

/* ------------------------------------------------------------------------ */
/* gather_qmm (qwen3_next.rs:509-578)                                        */
/* ------------------------------------------------------------------------ */

int hqo_gather_qmm_f64(const void* x, int x_dtype, const uint32_t* w,
                       const void* scales, const void* biases, int s_dtype,
                       const uint32_t* lhs, const uint32_t* rhs, int64_t batch,
                       int64_t x_batch, int64_t w_batch, int64_t M, int64_t N,
                       int64_t K, int transpose, int group_size, int bits,
                       double* y) {
  if (!bits_ok(bits) || !group_ok(group_size)) return -1;
  if (batch < 0 || x_batch <= 0 || w_batch <= 0) return -1;
  if (!lhs && (batch % x_batch)) return -1;
  if (transpose ? (K % group_size) : (N % group_size)) return -1;
  int64_t rep = lhs ? 1 : (batch / x_batch);
  int64_t wrows = transpose ? N : K, wcols = transpose ? K : N;
  int64_t P = wcols * bits / 32, G = wcols / group_size;
  int esz = (s_dtype == HQO_F32) ? 4 : 2;
  int xsz = (x_dtype == HQO_F32) ? 4 : 2;
  for (int64_t i = 0; i < batch; i++) {
    int64_t xi = lhs ? (int64_t)lhs[i] : i / rep;
    int64_t wi = rhs[i];
    double* yi = y + i * M * N;
    if (xi >= x_batch || wi >= w_batch) {
      for (int64_t j = 0; j < M * N; j++) yi[j] = NAN;
      continue;
    }
    const char* xs = (const char*)x + (size_t)(xi * M * K) * xsz;
    const uint32_t* we = w + wi * wrows * P;
    const char* se = (const char*)scales + (size_t)(wi * wrows * G) * esz;
    const char* be = (const char*)biases + (size_t)(wi * wrows * G) * esz;
    int rc = hqo_qmm_f64(xs, x_dtype, we, se, be, s_dtype, M, N, K, transpose,
                         group_size, bits, yi);
    if (rc) return rc;
  }
  return 0;
}

/* ------------------------------------------------------------------------ */
/* global expert sort (qwen3_next.rs:1748-1761)                              */
/* ------------------------------------------------------------------------ */

typedef struct {
  uint32_t key;
  uint32_t pos;
} kp_t;

static int kp_cmp(const void* a, const void* b) {
  const kp_t* x = (const kp_t*)a;
  const kp_t* y = (const kp_t*)b;
  if (x->key != y->key) return x->key < y->key ? -1 : 1;
  return x->pos < y->pos ? -1 : (x->pos > y->pos ? 1 : 0);
}

void hqo_gather_sort(const uint32_t* idx, int64_t n, int64_t top_k,
                     uint32_t* order, uint32_t* inv_order, uint32_t* idx_sorted,
                     uint32_t* token_idx) {
  kp_t* kp = (kp_t*)malloc((size_t)(n > 0 ? n : 1) * sizeof(kp_t));
  for (int64_t i = 0; i < n; i++) {
    kp[i].key = idx[i];
    kp[i].pos = (uint32_t)i;
  }
  qsort(kp, (size_t)n, sizeof(kp_t), kp_cmp); /* (key, pos) order = stable */
  for (int64_t i = 0; i < n; i++) {
    if (order) order[i] = kp[i].pos;
    if (inv_order) inv_order[kp[i].pos] = (uint32_t)i;
    if (idx_sorted) idx_sorted[i] = kp[i].key;
    if (token_idx) token_idx[i] = (uint32_t)(kp[i].pos / (uint64_t)top_k);
  }
  free(kp);
}

/* ------------------------------------------------------------------------ */
/* SwiGLU (qwen3_next.rs:340-342)                                            */
/* ------------------------------------------------------------------------ */

void hqo_swiglu(const void* gate, const void* up, int dtype, int64_t n, void* out) {
  for (int64_t i = 0; i < n; i++) {
    double g = load_dt(gate, dtype, i), u = load_dt(up, dtype, i);
    store_dt(out, dtype, i, hqo_round_f64(g / (1.0 + exp(-g)) * u, dtype));
  }
}

/* ------------------------------------------------------------------------ */
/* MoE unsort + score-weighted combine (qwen3_next.rs:1802-1808 take of     */
/* inv_order; qwen3_moe.rs:355-357 y * scores summed over top_k)            */
/* ------------------------------------------------------------------------ */

/* out[t, d] = round(sum_j round(scores[t, j] * y[inv[t*k + j], d])): each
 * product rounded to `dtype` (MLX's multiply of two `dtype` arrays), the sum
 * over j in fp64, one final rounding. inv out of range -> NaN row. */
void hqo_moe_combine(const void* y, int dtype, const uint32_t* inv, const void* scores,
                     int sdtype, int64_t tokens, int64_t top_k, int64_t D, void* out) {
  const int64_t rows = tokens * top_k;
  for (int64_t t = 0; t < tokens; t++) {
    int bad = 0;
    for (int64_t j = 0; j < top_k; j++)
      if ((int64_t)inv[t * top_k + j] >= rows) bad = 1;
    for (int64_t d = 0; d < D; d++) {
      double acc = 0.0;
      if (!bad) {
        for (int64_t j = 0; j < top_k; j++) {
          const double sc = load_dt(scores, sdtype, t * top_k + j);
          const double yv = load_dt(y, dtype, (int64_t)inv[t * top_k + j] * D + d);
          acc += hqo_round_f64(sc * yv, dtype);
        }
      }
      store_dt(out, dtype, t * D + d, bad ? (float)NAN : hqo_round_f64(acc, dtype));
    }
  }
}


/* ------------------------------------------------------------------------ */
/* quantize                                                                  */
/* ------------------------------------------------------------------------ */

/*
 * MLX affine quantize, op by op in the weights' dtype T (mlx-rs
 * ops::quantize(w, group_size, bits), called by higgs' tests at
 * crates/higgs-models/src/qwen3_next.rs:4305-4307 and 12942, and by
 * mlx_rs::nn::quantize for float checkpoints, transformer.rs:954-965).
 * The algorithm is MLX's, which is not in /root/reference (PARITY UNPINNED
 * against MLX itself; pinned here by what the mathematics fixes, see
 * tests/test_oracle.py). Per group of group_size consecutive elements, each
 * operation computed in float and rounded to T:
 *   mx = max(w), mn = min(w), n_bins = 2^bits - 1
 *   scale = max((mx - mn) / n_bins, T(1e-7))
 *   if |mn| > |mx|: edge = mn            else: edge = mx, scale = -scale
 *   q0 = rint(edge / scale)
 *   if q0 != 0: scale = edge / q0, bias = edge    else: bias = 0
 *   q = clip(rint((w - bias) / scale), 0, n_bins)   (NaN -> 0)
 * so that w = 0 dequantizes to exactly 0. q is packed LSB-first (hqo_pack).
 */
static float quant_group(const void* w, int dtype, int64_t base, int gs, int bits, uint32_t* q,
                         float* bias_out) {
  const float n_bins = (float)((1 << bits) - 1);
  const float eps = round_dt(1e-7f, dtype);
  float mx = load_dt(w, dtype, base), mn = mx;
  for (int i = 1; i < gs; i++) {
    const float v = load_dt(w, dtype, base + i);
    if (v > mx) mx = v;
    if (v < mn) mn = v;
  }
  float scale = round_dt(round_dt(mx - mn, dtype) / n_bins, dtype);
  if (!(scale > eps)) scale = eps;
  const int side = fabsf(mn) > fabsf(mx);
  if (!side) scale = -scale;
  const float edge = side ? mn : mx;
  const float q0 = rintf(round_dt(edge / scale, dtype));
  float bias = 0.0f;
  if (q0 != 0.0f) {
    scale = round_dt(edge / q0, dtype);
    bias = edge;
  }
  for (int i = 0; i < gs; i++) {
    const float v = load_dt(w, dtype, base + i);
    float t = rintf(round_dt(round_dt(v - bias, dtype) / scale, dtype));
    if (!(t >= 0.0f)) t = 0.0f;
    if (t > n_bins) t = n_bins;
    q[i] = (uint32_t)t;
  }
  *bias_out = bias;
  return scale;
}

int hqo_quantize(const void* w, int dtype, int64_t rows, int64_t K, int group_size, int bits,
                 uint32_t* wq, void* scales, void* biases) {
  if (!(bits == 2 || bits == 3 || bits == 4 || bits == 5 || bits == 6 || bits == 8)) return -1;
  if (!(group_size == 32 || group_size == 64 || group_size == 128)) return -1;
  if (rows < 0 || K <= 0 || K % group_size) return -1;
  const int64_t G = K / group_size;
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; r++) {
    uint32_t* q = (uint32_t*)malloc((size_t)K * sizeof(uint32_t));
    for (int64_t g = 0; g < G; g++) {
      float b;
      const float s = quant_group(w, dtype, r * K + g * group_size, group_size, bits,
                                  q + g * group_size, &b);
      store_dt(scales, dtype, r * G + g, s);
      store_dt(biases, dtype, r * G + g, b);
    }
    hqo_pack(q, 1, K, bits, wq + r * (K * bits / 32));
    free(q);
  }
  return 0;
}
