/*
 * h3oracle.c — CPU restatement of h3-hrx's INT8 attention path. TEST INFRASTRUCTURE ONLY:
 * it checks the HIP kernels and serves as the timed CPU baseline; the shipped library never
 * links or calls it. Build: oracle/Makefile (gcc -O2 -ffp-contract=off, no fast-math, so every
 * float operation below is one IEEE binary32/binary64 operation in the order written).
 * Reference citations are relative to the zacharydenton/h3-hrx tree.
 */
#include "h3oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ---------------------------------------------------------------- 16-bit formats */

float h3o_half_to_float(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1fu;
  uint32_t man = h & 0x3ffu;
  uint32_t bits;
  if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else { /* subnormal: man * 2^-24, exact in binary32 */
      float v = (float)man * 5.9604644775390625e-08f;
      memcpy(&bits, &v, 4);
      bits |= sign;
    }
  } else if (exp == 31) {
    bits = sign | 0x7f800000u | (man << 13);
  } else {
    bits = sign | ((exp + 112u) << 23) | (man << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

uint16_t h3o_float_to_half(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
  uint32_t ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u) { /* inf or nan */
    if (ax == 0x7f800000u) return sign | 0x7c00u;
    return sign | 0x7e00u | (uint16_t)((ax >> 13) & 0x3ffu);
  }
  if (ax >= 0x477ff000u) return sign | 0x7c00u; /* rounds to >= 65520: overflow */
  if (ax < 0x38800000u) {                       /* below 2^-14: subnormal half */
    /* value = ax_float; half subnormal unit 2^-24. Round(value * 2^24) to nearest even. */
    float af;
    memcpy(&af, &ax, 4);
    double scaled = (double)af * 16777216.0; /* exact */
    double r = nearbyint(scaled);            /* ties to even (default rounding mode) */
    return sign | (uint16_t)r;
  }
  uint32_t e = (ax >> 23) - 112u; /* half exponent field, 1..30 */
  uint32_t m = ax & 0x7fffffu;
  uint32_t half = (e << 10) | (m >> 13);
  uint32_t rem = m & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (half & 1u))) half += 1u;
  return sign | (uint16_t)half;
}

float h3o_bf16_to_float(uint16_t h) {
  uint32_t bits = (uint32_t)h << 16;
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

static inline float widen(uint16_t v, int fmt) {
  return fmt == H3O_BF16 ? h3o_bf16_to_float(v) : h3o_half_to_float(v);
}

float h3o_config_f32(double v) {
  char buf[64];
  snprintf(buf, sizeof buf, "%.17g", v);
  return strtof(buf, NULL);
}

/* ---------------------------------------------------------------- quantizer */

/* kernels/prepare_qk_i8.loom:84-156. Element e = 4*lane + j. In-lane stage over bits 0-1,
 * then lane butterflies k = 1, 2, 4, 8, 16: the lane with bit k clear keeps s + partner,
 * the lane with bit k set keeps partner - s. */
void h3o_hadamard128_f32(const float *y, float *r) {
  float s[128], t[128];
  for (int l = 0; l < 32; ++l) {
    float a = y[4 * l], b = y[4 * l + 1], c = y[4 * l + 2], d = y[4 * l + 3];
    float ab_p = a + b, ab_m = a - b, cd_p = c + d, cd_m = c - d;
    s[4 * l + 0] = ab_p + cd_p;
    s[4 * l + 1] = ab_m + cd_m;
    s[4 * l + 2] = ab_p - cd_p;
    s[4 * l + 3] = ab_m - cd_m;
  }
  for (int k = 1; k < 32; k <<= 1) {
    for (int l = 0; l < 32; ++l) {
      int p = l ^ k;
      for (int j = 0; j < 4; ++j)
        t[4 * l + j] = (l & k) ? (s[4 * p + j] - s[4 * l + j]) : (s[4 * l + j] + s[4 * p + j]);
    }
    memcpy(s, t, sizeof s);
  }
  memcpy(r, s, sizeof s);
}

/* kernels/prepare_qk_i8.loom:157-188: amax = max(max|r|, 1e-30); sc = amax/127; inv = 127/amax;
 * q = clamp(roundeven(r*inv), -127, 127); word = bytes low-first; scale = sc * extra. */
void h3o_quantize_row(const float *y, float extra, int32_t *words, float *scale) {
  float r[128];
  h3o_hadamard128_f32(y, r);
  float amax = 0.0f;
  for (int e = 0; e < 128; ++e) amax = fmaxf(amax, fabsf(r[e]));
  amax = fmaxf(amax, 1.0000000000000001e-30f);
  float sc = amax / 127.0f;
  float inv = 127.0f / amax;
  for (int l = 0; l < 32; ++l) {
    uint32_t w = 0;
    for (int j = 0; j < 4; ++j) {
      float qf = r[4 * l + j] * inv;
      float qr = rintf(qf);
      float qc = fminf(fmaxf(qr, -127.0f), 127.0f);
      int32_t qi = (int32_t)qc;
      w |= ((uint32_t)qi & 0xffu) << (8 * j);
    }
    words[l] = (int32_t)w;
  }
  *scale = sc * extra;
}

void h3o_prepare_qk_f32(const uint16_t *x, int fmt, const float *mean, int tokens, int row_stride,
                        int head_offset, int heads, float extra, int head_major, int capacity,
                        int32_t *codes, float *scales) {
  float y[128];
  for (int t = 0; t < tokens; ++t) {
    for (int h = 0; h < heads; ++h) {
      int col0 = head_offset + 128 * h;
      for (int c = 0; c < 128; ++c) {
        float v = widen(x[(size_t)t * row_stride + col0 + c], fmt);
        float m = mean ? mean[col0 + c] : 0.0f;
        y[c] = v - m; /* loom:79-82 */
      }
      int32_t *w;
      float *s;
      if (head_major) { /* prepare_qk_i8hm.loom (in-file 184-191) */
        size_t row = (size_t)h * capacity + t;
        w = codes + row * 32;
        s = scales + row;
      } else { /* prepare_qk_i8.loom:180-188 */
        w = codes + (size_t)t * heads * 32 + (size_t)h * 32;
        s = scales + (size_t)t * heads + h;
      }
      h3o_quantize_row(y, extra, w, s);
    }
  }
}

/* tests/kernels.rs:1704-1741 */
void h3o_prepared_qk_f64(const uint16_t *x, const float *mean, int tokens, int heads, double extra,
                         int32_t *words, float *scales, double *codes_out) {
  const int d = 128, stride = heads * d;
  double centred[128], rotated[128];
  memset(words, 0, sizeof(int32_t) * (size_t)tokens * heads * 32);
  for (int t = 0; t < tokens; ++t) {
    for (int h = 0; h < heads; ++h) {
      for (int c = 0; c < d; ++c)
        centred[c] = (double)h3o_half_to_float(x[(size_t)t * stride + h * d + c]) -
                     (double)mean[h * d + c];
      for (int e = 0; e < d; ++e) {
        double acc = 0.0;
        for (int c = 0; c < d; ++c)
          acc += centred[c] * ((__builtin_popcount((unsigned)(c & e)) & 1) ? -1.0 : 1.0);
        rotated[e] = acc;
      }
      double amax = 0.0;
      for (int e = 0; e < d; ++e) amax = fmax(amax, fabs(rotated[e]));
      amax = fmax(amax, 1e-30);
      double step = amax / 127.0;
      for (int e = 0; e < d; ++e) {
        double code = round(rotated[e] / step);
        code = fmin(fmax(code, -127.0), 127.0);
        if (codes_out) codes_out[(size_t)t * stride + h * d + e] = code;
        int32_t *w = &words[((size_t)t * heads + h) * 32 + e / 4];
        *w = (int32_t)((uint32_t)*w | (((uint32_t)(int32_t)code & 0xffu) << (8 * (e % 4))));
      }
      scales[(size_t)t * heads + h] = (float)(step * extra);
    }
  }
}

/* ---------------------------------------------------------------- colmean */

/* kernels/colmean_f32.loom (in-file 30-40) */
void h3o_colmean_f32(const uint16_t *x, int fmt, int tokens, int width, int row_stride,
                     float *mean) {
  for (int c = 0; c < width; ++c) {
    float acc = 0.0f;
    for (int t = 0; t < tokens; ++t) acc = acc + widen(x[(size_t)t * row_stride + c], fmt);
    mean[c] = acc / (float)tokens;
  }
}

/* ---------------------------------------------------------------- RMSNorm + RoPE */

/* Fixed order of this build's kernel: lane partial ((v0^2+v1^2)+v2^2)+v3^2 for lane l holding
 * channels 4l..4l+3; butterfly over lanes k = 1,2,4,8,16 (x_l + x_{l^k}); mean = ss * (1/128);
 * r = 1 / sqrt(mean + eps) (two IEEE operations); xn = (v * r) * w; rotate-half on c < 96:
 * c < 48: xn_c*cos_c - xn_{c+48}*sin_c; 48 <= c < 96: xn_c*cos_{c-48} + xn_{c-48}*sin_{c-48};
 * then f16 round-to-nearest-even. The maths is kernels/prepare_qk_rope_i8hm.loom:110-130. */
void h3o_rope_qknorm_f16(const uint16_t *x, int fmt, int tokens, int row_stride, int head_offset,
                         int heads, const float *weight, const float *cos_t, const float *sin_t,
                         float eps, uint16_t *out, int out_stride) {
  h3o_rope_qknorm_f16_ulps(x, fmt, tokens, row_stride, head_offset, heads, weight, cos_t, sin_t,
                           eps, out, out_stride, 0);
}

/* The same with r moved by r_ulps units in the last place (nextafterf, r_ulps in [-8, 8]):
 * the sensitivity of the route's outputs to an rsqrt that is not correctly rounded, as the
 * reference's scalar.rsqrtf (prepare_qk_rope_i8hm.loom:117) need not be. */
void h3o_rope_qknorm_f16_ulps(const uint16_t *x, int fmt, int tokens, int row_stride,
                              int head_offset, int heads, const float *weight, const float *cos_t,
                              const float *sin_t, float eps, uint16_t *out, int out_stride,
                              int r_ulps) {
  float v[128], xn[128], part[32], nxt[32];
  for (int t = 0; t < tokens; ++t) {
    const float *cs = cos_t + (size_t)t * 48;
    const float *sn = sin_t + (size_t)t * 48;
    for (int h = 0; h < heads; ++h) {
      int col0 = head_offset + 128 * h;
      for (int c = 0; c < 128; ++c) v[c] = widen(x[(size_t)t * row_stride + col0 + c], fmt);
      for (int l = 0; l < 32; ++l) {
        float a = v[4 * l] * v[4 * l], b = v[4 * l + 1] * v[4 * l + 1];
        float c2 = v[4 * l + 2] * v[4 * l + 2], d = v[4 * l + 3] * v[4 * l + 3];
        part[l] = ((a + b) + c2) + d;
      }
      for (int k = 1; k < 32; k <<= 1) {
        for (int l = 0; l < 32; ++l) nxt[l] = part[l] + part[l ^ k];
        memcpy(part, nxt, sizeof part);
      }
      float ms = part[0] * 0.0078125f;
      float me = ms + eps;
      float sq = sqrtf(me);
      float r = 1.0f / sq;
      for (int u = 0; u < r_ulps && u < 8; ++u) r = nextafterf(r, INFINITY);
      for (int u = 0; u > r_ulps && u > -8; --u) r = nextafterf(r, 0.0f);
      for (int c = 0; c < 128; ++c) {
        float nv = v[c] * r;
        xn[c] = nv * weight[c];
      }
      for (int c = 0; c < 128; ++c) {
        float o;
        if (c < 48) {
          float a = xn[c] * cs[c];
          float b = xn[c + 48] * sn[c];
          o = a - b;
        } else if (c < 96) {
          float a = xn[c] * cs[c - 48];
          float b = xn[c - 48] * sn[c - 48];
          o = a + b;
        } else {
          o = xn[c];
        }
        out[(size_t)t * out_stride + 128 * h + c] = h3o_float_to_half(o);
      }
    }
  }
}

/* tests/kernels.rs:1146-1180 (d = 128, rot = 96) */
void h3o_rope_qknorm_f64(const uint16_t *x, int fmt, int tokens, int row_stride, int head_offset,
                         int heads, const float *weight, const float *cos_t, const float *sin_t,
                         double eps, double *out) {
  const int d = 128, rot = 96, half = 48;
  double xv[128];
  for (int t = 0; t < tokens; ++t) {
    for (int h = 0; h < heads; ++h) {
      const uint16_t *row = x + (size_t)t * row_stride + head_offset + h * d;
      double ss = 0.0;
      for (int c = 0; c < d; ++c) {
        double f = (double)widen(row[c], fmt);
        ss += f * f;
      }
      double norm = sqrt(ss / d + eps);
      for (int c = 0; c < d; ++c) xv[c] = (double)widen(row[c], fmt) / norm * (double)weight[c];
      for (int c = 0; c < d; ++c) {
        double val;
        if (c < rot) {
          int p = c % half;
          double a = cos_t[(size_t)t * half + p], b = sin_t[(size_t)t * half + p];
          val = c < half ? xv[c] * a - xv[c + half] * b : xv[c] * a + xv[c - half] * b;
        } else {
          val = xv[c];
        }
        out[((size_t)t * heads + h) * d + c] = val;
      }
    }
  }
}

/* ---------------------------------------------------------------- transpose */

/* kernels/transpose_f16.loom, transpose_qkv_v_f16.loom: out[c][r] = x[r][c] for r < rows,
 * 0 for rows <= r < clear_to. */
void h3o_transpose_f16(const uint16_t *x, int fmt, int rows, int row_stride, int col_offset,
                       int width, int capacity, int clear_to, uint16_t *out) {
  for (int c = 0; c < width; ++c) {
    for (int r = 0; r < clear_to && r < capacity; ++r) {
      uint16_t v = 0;
      if (r < rows) {
        v = x[(size_t)r * row_stride + col_offset + c];
        if (fmt == H3O_BF16) v = h3o_float_to_half(h3o_bf16_to_float(v));
      }
      out[(size_t)c * capacity + r] = v;
    }
  }
}

/* ---------------------------------------------------------------- attention */

void h3o_unpack_codes(const int32_t *words, size_t n_rows, int8_t *codes) {
  for (size_t i = 0; i < n_rows * 32; ++i) {
    uint32_t w = (uint32_t)words[i];
    for (int j = 0; j < 4; ++j) codes[i * 4 + j] = (int8_t)(w >> (8 * j));
  }
}

int h3o_max_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

/* tests/kernels.rs:1891-1913 and 2084-2111: score(j) = (sum_c qc*kc) * qs * ks in f64,
 * weights exp(score - top), out = sum_j w_j/total * v_j. */
int h3o_attention_f64(const int8_t *qc, const float *qs, const int8_t *kc, const float *ks,
                      const uint16_t *vt, int tokens, int capacity, int heads, const int *rows,
                      int n_rows, double *out, int threads) {
  const int d = 128;
  long total = (long)n_rows * heads;
#ifdef _OPENMP
  if (threads <= 0) threads = omp_get_max_threads();
#pragma omp parallel num_threads(threads)
#endif
  {
    double *score = (double *)malloc(sizeof(double) * (size_t)tokens);
    double acc[128];
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 1)
#endif
    for (long job = 0; job < total; ++job) {
      int ri = (int)(job / heads), h = (int)(job % heads);
      int row = rows[ri];
      const int8_t *q = qc + ((size_t)h * capacity + row) * d;
      double qscale = (double)qs[(size_t)h * capacity + row];
      double top = -INFINITY;
      for (int j = 0; j < tokens; ++j) {
        const int8_t *k = kc + ((size_t)h * capacity + j) * d;
        int32_t dot = 0;
        for (int c = 0; c < d; ++c) dot += (int32_t)q[c] * (int32_t)k[c];
        double s = (double)dot * qscale * (double)ks[(size_t)h * capacity + j];
        score[j] = s;
        if (s > top) top = s;
      }
      double sum = 0.0;
      for (int c = 0; c < d; ++c) acc[c] = 0.0;
      for (int j = 0; j < tokens; ++j) {
        double w = exp(score[j] - top);
        score[j] = w;
        sum += w;
      }
      for (int c = 0; c < d; ++c) {
        const uint16_t *vrow = vt + ((size_t)h * d + c) * capacity;
        double a = 0.0;
        for (int j = 0; j < tokens; ++j) a += score[j] * (double)h3o_half_to_float(vrow[j]);
        acc[c] = a / sum;
      }
      double *o = out + ((size_t)ri * heads + h) * d;
      for (int c = 0; c < d; ++c) o[c] = acc[c];
    }
    free(score);
  }
  return 0;
}

/* The reference's CPU path for one attention call: prepared_qk (tests/kernels.rs:1704-1741) of
 * Q on the sampled rows and of K on every token (K centred on its f32 column mean,
 * tests/kernels.rs:1882-1887), V transposed, then the f64 attention of those operands.
 * q, k, v: f16 [tokens][heads*128]. Returns the wall seconds of the per-row part (Q rows and
 * their attention); *fixed_seconds receives the per-call part (K mean, K operand, V^T). */
double h3o_cpu_baseline(const uint16_t *q, const uint16_t *k, const uint16_t *v, int tokens,
                        int heads, const int *rows, int n_rows, int threads, double *out,
                        double *fixed_seconds) {
  const int d = 128, stride = heads * d;
  double t0 = 0.0;
#ifdef _OPENMP
  if (threads <= 0) threads = omp_get_max_threads();
  t0 = omp_get_wtime();
#endif
  size_t cap = (size_t)tokens;
  float *kmean = (float *)calloc((size_t)stride, sizeof(float));
  float *zmean = (float *)calloc((size_t)stride, sizeof(float));
  int8_t *kc = (int8_t *)malloc((size_t)heads * cap * d);
  int8_t *qc = (int8_t *)malloc((size_t)heads * cap * d);
  float *ks = (float *)malloc(sizeof(float) * heads * cap);
  float *qs = (float *)calloc((size_t)heads * cap, sizeof(float));
  uint16_t *vt = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)stride * cap);
  double extra = 1.0 / sqrt((double)d) / 128.0;
#ifdef _OPENMP
#pragma omp parallel for num_threads(threads) schedule(static)
#endif
  for (int c = 0; c < stride; ++c) {
    float acc = 0.0f;
    for (int t = 0; t < tokens; ++t) acc += h3o_half_to_float(k[(size_t)t * stride + c]);
    kmean[c] = acc / (float)tokens;
  }
  /* K operand on every token, Q operand on the sampled rows */
#ifdef _OPENMP
#pragma omp parallel num_threads(threads)
#endif
  {
    int32_t words[32];
    float scale;
    double codes[128];
    int32_t *wbuf = (int32_t *)malloc(sizeof(int32_t) * 32 * (size_t)heads);
    float *sbuf = (float *)malloc(sizeof(float) * (size_t)heads);
    double *cbuf = (double *)malloc(sizeof(double) * (size_t)stride);
    (void)words; (void)scale; (void)codes;
#ifdef _OPENMP
#pragma omp for schedule(static)
#endif
    for (int t = 0; t < tokens; ++t) {
      h3o_prepared_qk_f64(k + (size_t)t * stride, kmean, 1, heads, 1.0, wbuf, sbuf, cbuf);
      for (int h = 0; h < heads; ++h) {
        ks[(size_t)h * cap + t] = sbuf[h];
        for (int c = 0; c < d; ++c) kc[((size_t)h * cap + t) * d + c] = (int8_t)cbuf[h * d + c];
      }
    }
#ifdef _OPENMP
#pragma omp for schedule(static)
#endif
    for (int i = 0; i < n_rows; ++i) {
      int t = rows[i];
      h3o_prepared_qk_f64(q + (size_t)t * stride, zmean, 1, heads, extra, wbuf, sbuf, cbuf);
      for (int h = 0; h < heads; ++h) {
        qs[(size_t)h * cap + t] = sbuf[h];
        for (int c = 0; c < d; ++c) qc[((size_t)h * cap + t) * d + c] = (int8_t)cbuf[h * d + c];
      }
    }
#ifdef _OPENMP
#pragma omp for schedule(static)
#endif
    for (int c = 0; c < stride; ++c)
      for (int t = 0; t < tokens; ++t) vt[(size_t)c * cap + t] = v[(size_t)t * stride + c];
    free(wbuf);
    free(sbuf);
    free(cbuf);
  }
  double tm = 0.0;
#ifdef _OPENMP
  tm = omp_get_wtime();
#endif
  if (fixed_seconds) *fixed_seconds = tm - t0;
  h3o_attention_f64(qc, qs, kc, ks, vt, tokens, (int)cap, heads, rows, n_rows, out, threads);
  double t1 = 0.0;
#ifdef _OPENMP
  t1 = omp_get_wtime();
#endif
  free(kmean); free(zmean); free(kc); free(qc); free(ks); free(qs); free(vt);
  return t1 - tm;
}

/* kernels/gemm_packed_256.loom:370-397 (the f32 epilogue of one output) in the scalar form of
 * tests/kernels.rs:4436-4441: (dot as f32 * ws) * as + 0, clamped to +-65472 when finite. */
static uint16_t gemm_finish(int32_t dot, float ws, float as) {
  float raw = (float)dot * ws;
  raw = raw * as;
  raw = raw + 0.0f;
  if (isfinite(raw)) raw = raw < -65472.0f ? -65472.0f : (raw > 65472.0f ? 65472.0f : raw);
  return h3o_float_to_half(raw);
}

void h3o_gemm_i8_qkv(const int8_t *a, const int8_t *w, const float *ws, const float *as, int m,
                     int n, int k, int k_stride, uint16_t *out, int threads) {
  const int qk = 2 * (n / 3);
  const size_t cap = ((size_t)m + 255) / 256 * 256;
  uint16_t *vt = out + (size_t)m * qk;
  if (threads <= 0) threads = omp_get_max_threads();
#pragma omp parallel for num_threads(threads) schedule(static)
  for (int r = 0; r < m; ++r) {
    const int8_t *ar = a + (size_t)r * k_stride;
    for (int col = 0; col < n; ++col) {
      const int8_t *wr = w + (size_t)col * k_stride;
      int32_t dot = 0;
      for (int i = 0; i < k; ++i) dot += (int32_t)ar[i] * (int32_t)wr[i];
      const uint16_t h = gemm_finish(dot, ws[col], as[r]);
      if (col < qk)
        out[(size_t)r * qk + col] = h;
      else
        vt[(size_t)(col - qk) * cap + r] = h;
    }
  }
  for (int c = 0; c < n / 3; ++c)
    for (size_t r = (size_t)m; r < cap; ++r) vt[(size_t)c * cap + r] = 0;
}

/* One radix-4 stage of the group-256 rotation on digit `d` (index bits 2d, 2d+1) of a 256-group,
 * in the reference's operation order (kernels/prepare_i8_family.loom:26-43, 93-110):
 *   s01 = x0+x1, s23 = x2+x3, d01 = x0-x1, d23 = x2-x3;
 *   y0 = s01+d23, y1 = s01-d23, y2 = d01+s23, y3 = s23-d01.
 * The stages at strides 4 and 16 exchange operands between lanes (48-51, 62-71) but evaluate the
 * same four expressions (additions commute exactly in IEEE arithmetic). */
static void plain_radix4(float *g, int d) {
  const int stride = 1 << (2 * d);
  for (int base = 0; base < 256; ++base) {
    if ((base >> (2 * d)) & 3) continue;
    float *p0 = g + base, *p1 = p0 + stride, *p2 = p1 + stride, *p3 = p2 + stride;
    const float x0 = *p0, x1 = *p1, x2 = *p2, x3 = *p3;
    const float s01 = x0 + x1, s23 = x2 + x3, d01 = x0 - x1, d23 = x2 - x3;
    *p0 = s01 + d23;
    *p1 = s01 - d23;
    *p2 = d01 + s23;
    *p3 = s23 - d01;
  }
}

void h3o_prepare_plain_i8(const void *x, int fmt, int tokens, int width, int out_stride,
                          int8_t *codes, float *scales) {
  float *row = (float *)malloc(sizeof(float) * (size_t)width);
  for (int t = 0; t < tokens; ++t) {
    for (int c = 0; c < width; ++c) {
      float v;
      if (fmt == 2) {
        v = ((const float *)x)[(size_t)t * width + c] + 0.0f; /* loom:641 addf zero */
      } else {
        const uint16_t b = ((const uint16_t *)x)[(size_t)t * width + c];
        v = fmt == H3O_BF16 ? h3o_bf16_to_float(b) : h3o_half_to_float(b);
      }
      row[c] = v * 1.0f; /* prescale 1.0 (loom:280) */
    }
    float amax = 0.0f;
    for (int g = 0; g < width; g += 256) {
      for (int d = 0; d < 4; ++d) plain_radix4(row + g, d);
      for (int i = 0; i < 256; ++i) { /* loom:126-149: non-finite counts as inf */
        const float a = fabsf(row[g + i]);
        const float checked = a < INFINITY ? a : INFINITY;
        amax = fmaxf(amax, checked);
      }
    }
    /* loom:155-163 */
    const float row_max = amax * 0.0625f;
    const float safe = fmaxf(row_max, 1.0000000000000001e-30f);
    const float s = safe / 127.0f;
    const float inv_s = 0.0625f / s;
    const int valid = s < INFINITY;
    for (int c = 0; c < width; ++c) {
      float q = valid ? row[c] * inv_s : 0.0f;
      q = nearbyintf(q); /* roundeven in the default rounding mode */
      q = fmaxf(q, -127.0f);
      q = fminf(q, 127.0f);
      codes[(size_t)t * out_stride + c] = (int8_t)(int)q;
    }
    scales[t] = s;
  }
  free(row);
}

/* int4 variant of the quantizer (kernels/prepare_qk_i4.loom:73-214): the same H_128 butterfly,
 * amax = max(max|r|, 1e-30), sc = amax/7, inv = 7/amax, q = clamp(rne(r*inv), +-7), code e in
 * nibble e%8 of word e/8 (low nibble first), scale = sc * extra. Token-major only
 * (loom:7-8): codes [tokens][heads*16] i32, scales [tokens][heads]. */
void h3o_quantize_row_i4(const float *y, float extra, int32_t *words, float *scale) {
  float r[128];
  h3o_hadamard128_f32(y, r);
  float amax = 0.0f;
  for (int e = 0; e < 128; ++e) amax = fmaxf(amax, fabsf(r[e]));
  amax = fmaxf(amax, 1.0000000000000001e-30f);
  const float sc = amax / 7.0f;
  const float inv = 7.0f / amax;
  for (int w = 0; w < 16; ++w) words[w] = 0;
  for (int e = 0; e < 128; ++e) {
    float q = rintf(r[e] * inv);
    q = fminf(fmaxf(q, -7.0f), 7.0f);
    words[e / 8] = (int32_t)((uint32_t)words[e / 8] | (((uint32_t)(int32_t)q & 15u) << (4 * (e % 8))));
  }
  *scale = sc * extra;
}

void h3o_prepare_qk_i4_f32(const uint16_t *x, int fmt, const float *mean, int tokens,
                           int row_stride, int head_offset, int heads, float extra,
                           int32_t *codes, float *scales) {
  float y[128];
  for (int t = 0; t < tokens; ++t) {
    for (int h = 0; h < heads; ++h) {
      const int col0 = head_offset + 128 * h;
      for (int c = 0; c < 128; ++c) {
        const float v = widen(x[(size_t)t * row_stride + col0 + c], fmt);
        const float m = mean ? mean[col0 + c] : 0.0f;
        y[c] = v - m;
      }
      h3o_quantize_row_i4(y, extra, codes + ((size_t)t * heads + h) * 16,
                          scales + (size_t)t * heads + h);
    }
  }
}

/* Cross-attention of int8 operands with grouped heads and a key mask, f64 (an extension with no
 * reference kernel; the formula is h3o_attention_f64's over the attended keys): query row t of
 * head h attends to the keys j < kv_tokens with mask[j] != 0 of key/value head h / group.
 *   qc [qh][q_cap][128], qs [qh][q_cap]; kc [kh][kv_cap][128], ks [kh][kv_cap];
 *   vt [kh*128][kv_cap] f16; out f64 [n_rows][qh][128]. */
int h3o_cross_attention_f64(const int8_t *qc, const float *qs, const int8_t *kc, const float *ks,
                            const uint16_t *vt, const uint8_t *mask, int q_cap, int kv_tokens,
                            int kv_cap, int qh, int kh, const int *rows, int n_rows, double *out,
                            int threads) {
  const int d = 128, group = qh / kh;
  long total = (long)n_rows * qh;
#ifdef _OPENMP
  if (threads <= 0) threads = omp_get_max_threads();
#pragma omp parallel num_threads(threads)
#endif
  {
    double *score = (double *)malloc(sizeof(double) * (size_t)(kv_tokens > 0 ? kv_tokens : 1));
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 1)
#endif
    for (long job = 0; job < total; ++job) {
      const int ri = (int)(job / qh), h = (int)(job % qh), g = h / group;
      const int row = rows[ri];
      const int8_t *q = qc + ((size_t)h * q_cap + row) * d;
      const double qscale = (double)qs[(size_t)h * q_cap + row];
      double top = -INFINITY;
      for (int j = 0; j < kv_tokens; ++j) {
        if (!mask[j]) { score[j] = -INFINITY; continue; }
        const int8_t *k = kc + ((size_t)g * kv_cap + j) * d;
        int32_t dot = 0;
        for (int c = 0; c < d; ++c) dot += (int32_t)q[c] * (int32_t)k[c];
        score[j] = (double)dot * qscale * (double)ks[(size_t)g * kv_cap + j];
        if (score[j] > top) top = score[j];
      }
      double sum = 0.0;
      for (int j = 0; j < kv_tokens; ++j) {
        score[j] = mask[j] ? exp(score[j] - top) : 0.0;
        sum += score[j];
      }
      double *o = out + ((size_t)ri * qh + h) * d;
      for (int c = 0; c < d; ++c) {
        const uint16_t *vrow = vt + ((size_t)g * d + c) * kv_cap;
        double a = 0.0;
        for (int j = 0; j < kv_tokens; ++j)
          if (mask[j]) a += score[j] * (double)h3o_half_to_float(vrow[j]);
        o[c] = a / sum;
      }
    }
    free(score);
  }
  return 0;
}
