/*
 * h3oracle_vsa.c — CPU restatement of h3-hrx's VSA (video sparse attention) path: the 64-token
 * cube plan, gather/scatter, block means, block scores, top-k routing, the coarse branch and
 * the block-sparse attention of the INT8 operands. TEST INFRASTRUCTURE ONLY (see h3oracle.h):
 * the shipped library never links or calls it. Built by oracle/Makefile with the same flags as
 * h3oracle.c (-ffp-contract=off, no fast-math): every float operation is one IEEE operation in
 * the order written, fmaf is the fused multiply-add. Citations are relative to the
 * zacharydenton/h3-hrx tree.
 */
#include "h3oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ---------------------------------------------------------------- host policy (src/vsa.rs) */

/* src/vsa.rs:98-106 (segment): every prefix segment is cut into 64-row tiles; the last one is
 * padded with -1. src/vsa.rs:111-130: video cubes of 4x4x4 latent cells (t, h, w), row-major
 * within the cube, padded to 64. src/vsa.rs:131-140: the inverse permutation. */
int h3o_vsa_plan_blocks(const int *seg_rows, int n_segs, int nt, int nh, int nw) {
  int blocks = 0;
  for (int s = 0; s < n_segs; ++s) blocks += (seg_rows[s] + 63) / 64;
  blocks += ((nt + 3) / 4) * ((nh + 3) / 4) * ((nw + 3) / 4);
  return blocks;
}

int h3o_vsa_plan(const int *seg_row0, const int *seg_rows, int n_segs, int seq_len, int nt,
                 int nh, int nw, int32_t *src, int32_t *inverse, int32_t *lengths,
                 int *prefix_blocks) {
  int n = 0, b = 0;
  for (int s = 0; s < n_segs; ++s) {
    const int start = seg_row0[s], len = seg_rows[s];
    for (int row = start; row < start + len; row += 64) {
      const int live = start + len - row < 64 ? start + len - row : 64;
      lengths[b++] = live;
      for (int r = 0; r < 64; ++r) src[n++] = r < live ? row + r : -1;
    }
  }
  *prefix_blocks = b;
  const int video0 = seq_len - nt * nh * nw;
  for (int t = 0; t < nt; t += 4)
    for (int h = 0; h < nh; h += 4)
      for (int w = 0; w < nw; w += 4) {
        const int start = n;
        for (int tt = t; tt < t + 4 && tt < nt; ++tt)
          for (int hh = h; hh < h + 4 && hh < nh; ++hh)
            for (int ww = w; ww < w + 4 && ww < nw; ++ww) src[n++] = video0 + (tt * nh + hh) * nw + ww;
        lengths[b++] = n - start;
        while (n < start + 64) src[n++] = -1;
      }
  for (int r = 0; r < seq_len; ++r) inverse[r] = -1;
  for (int i = 0; i < n; ++i)
    if (src[i] >= 0) inverse[src[i]] = i;
  for (int r = 0; r < seq_len; ++r)
    if (inverse[r] < 0) return -1; /* src/vsa.rs:137-140: the plan must cover every token */
  return b;
}

/* src/vsa.rs:54-59: round half to even of keep_percent/100 * nonprefix, at least 1, at most
 * nonprefix - 1 (saturating). */
int h3o_vsa_topk(double keep_percent, int nonprefix) {
  double r = nearbyint(keep_percent / 100.0 * (double)nonprefix); /* ties to even */
  long k = r > 0 ? (long)r : 0;
  if (k < 1) k = 1;
  long cap = nonprefix > 0 ? nonprefix - 1 : 0;
  if (k > cap) k = cap;
  return (int)k;
}

/* src/vsa.rs:60-72: 0 = sparse, 1 = below_min_tokens, 2 = outside_sigma_window. */
int h3o_vsa_dense_reason(double start, double end, long min_tokens, long tokens, float sigma,
                         double shift) {
  if (tokens < min_tokens) return 1;
  double t0 = 1.0 - start, t1 = 1.0 - end;
  float hi = (float)(shift * t0 / (1.0 + (shift - 1.0) * t0));
  float lo = (float)(shift * t1 / (1.0 + (shift - 1.0) * t1));
  if (sigma > hi || sigma < lo) return 2;
  return 0;
}

/* ---------------------------------------------------------------- data movement (vsa_ops) */

/* kernels/vsa_ops.loom h3_vsa_gather: y[i] = x[src[i]] when src[i] (unsigned) < tokens, else 0. */
void h3o_vsa_gather(const int32_t *src, int padded, int tokens, int width, const uint16_t *x,
                    uint16_t *y) {
  for (int i = 0; i < padded; ++i) {
    const uint32_t s = (uint32_t)src[i];
    for (int c = 0; c < width; ++c)
      y[(size_t)i * width + c] = s < (uint32_t)tokens ? x[(size_t)s * width + c] : 0;
  }
}

/* kernels/vsa_ops.loom h3_vsa_scatter: y[r] = x[inverse[r]]. */
void h3o_vsa_scatter(const int32_t *inverse, int tokens, int width, const uint16_t *x,
                     uint16_t *y) {
  for (int r = 0; r < tokens; ++r)
    memcpy(y + (size_t)r * width, x + (size_t)inverse[r] * width, (size_t)width * 2);
}

/* kernels/vsa_ops.loom h3_vsa_pool: means[b][c] = (sum_{j < len_b} f32(x[64b + j][c])) / len_b,
 * a sequential f32 sum from 0, then one f32 division by the length converted to f32. */
void h3o_vsa_pool(const int32_t *lengths, int blocks, int width, const uint16_t *x,
                  float *means) {
  for (int b = 0; b < blocks; ++b)
    for (int c = 0; c < width; ++c) {
      float acc = 0.0f;
      for (int j = 0; j < lengths[b]; ++j) acc = acc + h3o_half_to_float(x[((size_t)64 * b + j) * width + c]);
      means[(size_t)b * width + c] = acc / (float)lengths[b];
    }
}

/* kernels/vsa_ops.loom h3_vsa_scores: scores[h][q][j] = fma chain over d = 0..127 (from 0) of
 * qm[q][128h + d] * km[j][128h + d]. */
void h3o_vsa_scores(const float *qm, const float *km, int blocks, int heads, float *scores) {
  const int width = heads * 128;
  for (int h = 0; h < heads; ++h)
    for (int q = 0; q < blocks; ++q)
      for (int j = 0; j < blocks; ++j) {
        float acc = 0.0f;
        for (int d = 0; d < 128; ++d)
          acc = fmaf(qm[(size_t)q * width + 128 * h + d], km[(size_t)j * width + 128 * h + d], acc);
        scores[((size_t)h * blocks + q) * blocks + j] = acc;
      }
}

/* kernels/vsa_ops.loom h3_vsa_route, literally: a block pair is forced when either block is a
 * prefix block or |q - j| <= 1; otherwise it is kept when fewer than topk non-prefix scores of
 * row q are strictly greater (ordered comparison: NaN is never greater) than its own. */
void h3o_vsa_route(const float *scores, int blocks, int heads, int prefix, int topk,
                   int32_t *routes) {
  for (int h = 0; h < heads; ++h)
    for (int q = 0; q < blocks; ++q) {
      const float *row = scores + ((size_t)h * blocks + q) * blocks;
      for (int j = 0; j < blocks; ++j) {
        const int forced = (j <= q + 1 && q <= j + 1) || q < prefix || j < prefix;
        int keep = 1;
        if (!forced) {
          const float own = row[j];
          int rank = 0;
          for (int k = prefix; k < blocks; ++k) rank += row[k] > own;
          keep = rank < topk;
        }
        routes[((size_t)h * blocks + q) * blocks + j] = keep;
      }
    }
}

/* kernels/vsa_ops.loom h3_vsa_coarse in f64: coarse[q][128h + c] = sum_j softmax_j(scores[h][q][j]
 * * 0.08838834764831845f) vm[j][128h + c]. The reference evaluates exp with an approximate
 * expf (afn); this restatement is the exact value it approximates. */
void h3o_vsa_coarse_f64(const float *scores, const float *vm, int blocks, int heads,
                        double *coarse) {
  const int width = heads * 128;
  const float scale = 0.08838834764831845f;
  double *w = (double *)malloc(sizeof(double) * (size_t)blocks);
  for (int h = 0; h < heads; ++h)
    for (int q = 0; q < blocks; ++q) {
      const float *row = scores + ((size_t)h * blocks + q) * blocks;
      double top = -1.0e9;
      for (int j = 0; j < blocks; ++j) {
        const double s = (double)(row[j] * scale);
        if (s > top) top = s;
      }
      double sum = 0.0;
      for (int j = 0; j < blocks; ++j) {
        w[j] = exp((double)(row[j] * scale) - top);
        sum += w[j];
      }
      for (int c = 0; c < 128; ++c) {
        double acc = 0.0;
        for (int j = 0; j < blocks; ++j) acc += w[j] * (double)vm[(size_t)j * width + 128 * h + c];
        coarse[(size_t)q * width + 128 * h + c] = acc / sum;
      }
    }
  free(w);
}

/* kernels/vsa_ops.loom h3_vsa_gated_scatter: out[r][c] = f16(fma(f32(gate[r][c]),
 * coarse[inverse[r] / 64][c], f32(fine[inverse[r]][c]))), round to nearest even. */
void h3o_vsa_gated_scatter(const int32_t *inverse, int tokens, int width, const uint16_t *fine,
                           const uint16_t *gate, const float *coarse, uint16_t *out) {
  for (int r = 0; r < tokens; ++r) {
    const int sr = inverse[r], b = sr / 64;
    for (int c = 0; c < width; ++c) {
      const float f = h3o_half_to_float(fine[(size_t)sr * width + c]);
      const float g = h3o_half_to_float(gate[(size_t)r * width + c]);
      out[(size_t)r * width + c] = h3o_float_to_half(fmaf(g, coarse[(size_t)b * width + c], f));
    }
  }
}

/* kernels/vsa_kmean.loom: mean[c] = (sum_t x[t][c]) / tokens, sequential f32 from 0. */
void h3o_vsa_kmean(const float *x, int tokens, int width, float *mean) {
  for (int c = 0; c < width; ++c) {
    float acc = 0.0f;
    for (int t = 0; t < tokens; ++t) acc = acc + x[(size_t)t * width + c];
    mean[c] = acc / (float)tokens;
  }
}

/* ---------------------------------------------------------------- block-sparse attention */

/* kernels/vsa_attention_8.loom (body 1-404) in f64: query row i (gathered layout, cube i/64) of
 * head h attends to the keys j of every cube kb with routes[h][i/64][kb] != 0 and j % 64 <
 * lengths[kb], with logits sum(qc*kc) * qs[i][h] * ks[j][h] (the attention scale is folded
 * into qs) and natural softmax; out = sum_j p_j V[j] with V read from vt [width][capacity].
 *   qc, kc  int8 token-major [capacity][width]; qs, ks [capacity][heads]
 *   rows    the query rows to evaluate; out f64 [n_rows][heads][128]. */
int h3o_vsa_attention_f64(const int8_t *qc, const float *qs, const int8_t *kc, const float *ks,
                          const uint16_t *vt, int tokens, int capacity, int heads,
                          const int32_t *routes, const int32_t *lengths, const int *rows,
                          int n_rows, double *out, int threads) {
  const int d = 128, width = heads * d, blocks = tokens / 64;
  long total = (long)n_rows * heads;
#ifdef _OPENMP
  if (threads <= 0) threads = omp_get_max_threads();
#pragma omp parallel num_threads(threads)
#endif
  {
    double *score = (double *)malloc(sizeof(double) * (size_t)tokens);
    int *key = (int *)malloc(sizeof(int) * (size_t)tokens);
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 1)
#endif
    for (long job = 0; job < total; ++job) {
      const int ri = (int)(job / heads), h = (int)(job % heads);
      const int row = rows[ri], qb = row / 64;
      const int8_t *q = qc + (size_t)row * width + h * d;
      const double qscale = (double)qs[(size_t)row * heads + h];
      int nk = 0;
      double top = -INFINITY;
      for (int kb = 0; kb < blocks; ++kb) {
        if (!routes[((size_t)h * blocks + qb) * blocks + kb]) continue;
        for (int jj = 0; jj < lengths[kb] && jj < 64; ++jj) {
          const int j = 64 * kb + jj;
          const int8_t *k = kc + (size_t)j * width + h * d;
          int32_t dot = 0;
          for (int c = 0; c < d; ++c) dot += (int32_t)q[c] * (int32_t)k[c];
          const double s = (double)dot * qscale * (double)ks[(size_t)j * heads + h];
          score[nk] = s;
          key[nk++] = j;
          if (s > top) top = s;
        }
      }
      double sum = 0.0;
      for (int t = 0; t < nk; ++t) {
        score[t] = exp(score[t] - top);
        sum += score[t];
      }
      double *o = out + ((size_t)ri * heads + h) * d;
      for (int c = 0; c < d; ++c) {
        const uint16_t *vrow = vt + ((size_t)h * d + c) * capacity;
        double a = 0.0;
        for (int t = 0; t < nk; ++t) a += score[t] * (double)h3o_half_to_float(vrow[key[t]]);
        o[c] = a / sum;
      }
    }
    free(score);
    free(key);
  }
  return 0;
}

/* kernels/vsa_attention_16.loom (body 1-555) in f64, as the reference's own test states it
 * (src/vsa/device.rs:565-600): query row i (cube i/64) of head h attends to the keys j of every
 * cube kb with routes[h][i/64][kb] != 0 and j % 64 < lengths[kb], logits (q . k) * scale over the
 * f16 values, natural softmax, out = sum_j p_j v[j] / sum_j p_j.
 *   q, k, v  f16 bits token-major [capacity][heads*128]
 *   rows     the query rows to evaluate; out f64 [n_rows][heads][128]. */
int h3o_vsa_attention_f16_f64(const uint16_t *q, const uint16_t *k, const uint16_t *v, int tokens,
                              int heads, double scale, const int32_t *routes,
                              const int32_t *lengths, const int *rows, int n_rows, double *out,
                              int threads) {
  const int d = 128, width = heads * d, blocks = tokens / 64;
  long total = (long)n_rows * heads;
#ifdef _OPENMP
  if (threads <= 0) threads = omp_get_max_threads();
#pragma omp parallel num_threads(threads)
#endif
  {
    double *score = (double *)malloc(sizeof(double) * (size_t)tokens);
    int *key = (int *)malloc(sizeof(int) * (size_t)tokens);
    double qrow[128];
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 1)
#endif
    for (long job = 0; job < total; ++job) {
      const int ri = (int)(job / heads), h = (int)(job % heads);
      const int row = rows[ri], qb = row / 64;
      for (int c = 0; c < d; ++c)
        qrow[c] = (double)h3o_half_to_float(q[(size_t)row * width + h * d + c]);
      int nk = 0;
      double top = -INFINITY;
      for (int kb = 0; kb < blocks; ++kb) {
        if (!routes[((size_t)h * blocks + qb) * blocks + kb]) continue;
        for (int jj = 0; jj < lengths[kb] && jj < 64; ++jj) {
          const int j = 64 * kb + jj;
          const uint16_t *kr = k + (size_t)j * width + h * d;
          double dot = 0.0;
          for (int c = 0; c < d; ++c) dot += qrow[c] * (double)h3o_half_to_float(kr[c]);
          const double s = dot * scale;
          score[nk] = s;
          key[nk++] = j;
          if (s > top) top = s;
        }
      }
      double sum = 0.0;
      for (int t = 0; t < nk; ++t) {
        score[t] = exp(score[t] - top);
        sum += score[t];
      }
      double *o = out + ((size_t)ri * heads + h) * d;
      for (int c = 0; c < d; ++c) {
        double a = 0.0;
        for (int t = 0; t < nk; ++t)
          a += score[t] * (double)h3o_half_to_float(v[(size_t)key[t] * width + h * d + c]);
        o[c] = a / sum;
      }
    }
    free(score);
    free(key);
  }
  return 0;
}
