/*
 * scalar_backend.c - the kernels.Backend contract restated in C.
 *
 * TEST INFRASTRUCTURE ONLY (see gn_oracle.h).  Each function follows the
 * reference's portable backend, kernels/scalar/ sources, keeping its float32
 * data and its float64 accumulations so the GPU path can be checked against
 * it on identical inputs.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "gn_oracle.h"

/* kernels/scalar/elementwise.go:6-10 */
void orc_add(float *dst, const float *l, const float *r, int64_t n) {
  for (int64_t i = 0; i < n; i++) dst[i] = l[i] + r[i];
}
/* kernels/scalar/elementwise.go:13-17 */
void orc_subtract(float *dst, const float *l, const float *r, int64_t n) {
  for (int64_t i = 0; i < n; i++) dst[i] = l[i] - r[i];
}
/* kernels/scalar/elementwise.go:20-24 */
void orc_multiply(float *dst, const float *l, const float *r, int64_t n) {
  for (int64_t i = 0; i < n; i++) dst[i] = l[i] * r[i];
}
/* kernels/scalar/elementwise.go:27-31 */
void orc_divide(float *dst, const float *l, const float *r, int64_t n) {
  for (int64_t i = 0; i < n; i++) dst[i] = l[i] / r[i];
}
/* kernels/scalar/elementwise.go:34-38 */
void orc_scale(float *dst, const float *s, float f, int64_t n) {
  for (int64_t i = 0; i < n; i++) dst[i] = s[i] * f;
}
/* kernels/scalar/elementwise.go:41-45 */
void orc_add_scaled(float *dst, const float *b, const float *s, float f, int64_t n) {
  for (int64_t i = 0; i < n; i++) dst[i] = b[i] + f * s[i];
}
/* kernels/scalar/elementwise.go:48-52 */
void orc_negate(float *dst, const float *s, int64_t n) {
  for (int64_t i = 0; i < n; i++) dst[i] = -s[i];
}
/* kernels/scalar/elementwise.go:55-63 */
void orc_abs(float *dst, const float *s, int64_t n) {
  for (int64_t i = 0; i < n; i++) dst[i] = s[i] < 0 ? -s[i] : s[i];
}
/* kernels/scalar/elementwise.go:66-70 */
void orc_square(float *dst, const float *s, int64_t n) {
  for (int64_t i = 0; i < n; i++) dst[i] = s[i] * s[i];
}
/* kernels/scalar/elementwise.go:73-80 */
void orc_relu_squared(float *dst, const float *s, int64_t n) {
  for (int64_t i = 0; i < n; i++) {
    float v = s[i] < 0 ? 0.0f : s[i];
    dst[i] = v * v;
  }
}

/* kernels/scalar/elementwise.go:107-112 (clampGate) */
static float clamp_gate(float v, float c, float *mask) {
  if (c > 0 && v >= c) { *mask = 0; return c; }
  *mask = 1;
  return v;
}
/* kernels/scalar/elementwise.go:116-126 (clampUp) */
static float clamp_up(float v, float c, float *mask) {
  if (c > 0) {
    if (v > c) { *mask = 0; return c; }
    if (v < -c) { *mask = 0; return -c; }
  }
  *mask = 1;
  return v;
}
/* kernels/scalar/elementwise.go:85-89,129-134 */
void orc_swiglu(float *dst, const float *gate, const float *up, float clamp, int64_t n) {
  for (int64_t i = 0; i < n; i++) {
    float m;
    float g = clamp_gate(gate[i], clamp, &m);
    float u = clamp_up(up[i], clamp, &m);
    float sg = (float)(1.0 / (1.0 + exp(-(double)g)));
    dst[i] = g * sg * u;
  }
}
/* kernels/scalar/elementwise.go:92-103 */
void orc_swiglu_backward(float *dgate, float *dup, const float *gate, const float *up,
                         const float *dout, float clamp, int64_t n) {
  for (int64_t i = 0; i < n; i++) {
    float gm, um;
    float g = clamp_gate(gate[i], clamp, &gm);
    float u = clamp_up(up[i], clamp, &um);
    float sg = (float)(1.0 / (1.0 + exp(-(double)g)));
    float silu = g * sg;
    float sgrad = sg * (1 + g * (1 - sg));
    float d = dout[i];
    dgate[i] = d * u * sgrad * gm;
    dup[i] = d * silu * um;
  }
}
/* kernels/scalar/elementwise.go:137-141 */
void orc_exp(float *dst, const float *s, int64_t n) {
  for (int64_t i = 0; i < n; i++) dst[i] = (float)exp((double)s[i]);
}
/* kernels/scalar/elementwise.go:144-148 */
void orc_sigmoid(float *dst, const float *s, int64_t n) {
  for (int64_t i = 0; i < n; i++) dst[i] = (float)(1.0 / (1.0 + exp(-(double)s[i])));
}
/* kernels/scalar/elementwise.go:151-155 */
void orc_tanh(float *dst, const float *s, int64_t n) {
  for (int64_t i = 0; i < n; i++) dst[i] = (float)tanh((double)s[i]);
}
/* kernels/scalar/elementwise.go:158-162 */
void orc_rsqrt(float *dst, const float *s, int64_t n) {
  for (int64_t i = 0; i < n; i++) dst[i] = (float)(1.0 / sqrt((double)s[i]));
}

/* kernels/scalar/reduce.go:4-10 (float32 running sum, in order) */
float orc_sum(const float *v, int64_t n) {
  float t = 0;
  for (int64_t i = 0; i < n; i++) t += v[i];
  return t;
}
/* kernels/scalar/reduce.go:13-24 */
float orc_max(const float *v, int64_t n) {
  if (n == 0) return 0;
  float m = v[0];
  for (int64_t i = 1; i < n; i++)
    if (v[i] > m) m = v[i];
  return m;
}
/* kernels/scalar/reduce.go:28-36 */
int64_t orc_argmax(const float *v, int64_t n) {
  int64_t b = 0;
  for (int64_t i = 1; i < n; i++)
    if (v[i] > v[b]) b = i;
  return b;
}

/* kernels/scalar/matmul.go:7-17 (float64 accumulation) */
void orc_matmul(float *dst, const float *l, const float *r, int64_t rows, int64_t cols,
                int64_t inner) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < rows; i++)
    for (int64_t j = 0; j < cols; j++) {
      double a = 0;
      for (int64_t k = 0; k < inner; k++) a += (double)l[i * inner + k] * (double)r[k * cols + j];
      dst[i * cols + j] = (float)a;
    }
}
/* kernels/scalar/matmul.go:22-33 (float64 accumulation) */
void orc_matmul_transposed(float *dst, const float *l, const float *r, int64_t rows, int64_t cols,
                           int64_t inner) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < rows; i++)
    for (int64_t j = 0; j < cols; j++) {
      double a = 0;
      for (int64_t k = 0; k < inner; k++) a += (double)l[i * inner + k] * (double)r[j * inner + k];
      dst[i * cols + j] = (float)a;
    }
}
/* kernels/scalar/matmul.go:35-42 */
float orc_dot(const float *l, const float *r, int64_t n) {
  double a = 0;
  for (int64_t i = 0; i < n; i++) a += (double)l[i] * (double)r[i];
  return (float)a;
}

/* kernels/scalar/norm.go:7-22 */
void orc_softmax_last_dim(float *dst, const float *s, int64_t rows, int64_t cols) {
  for (int64_t r = 0; r < rows; r++) {
    const float *src = s + r * cols;
    float *d = dst + r * cols;
    float m = orc_max(src, cols);
    double total = 0;
    for (int64_t c = 0; c < cols; c++) {
      double e = exp((double)(src[c] - m));
      d[c] = (float)e;
      total += e;
    }
    float inv = (float)(1.0 / total);
    for (int64_t c = 0; c < cols; c++) d[c] = d[c] * inv;
  }
}
/* kernels/scalar/norm.go:26-40 */
void orc_rmsnorm_last_dim(float *dst, const float *s, int64_t rows, int64_t cols, float eps) {
  for (int64_t r = 0; r < rows; r++) {
    const float *src = s + r * cols;
    float *d = dst + r * cols;
    double ss = 0;
    for (int64_t c = 0; c < cols; c++) ss += (double)src[c] * (double)src[c];
    float ms = (float)(ss / (double)cols);
    float inv = (float)(1.0 / sqrt((double)ms + (double)eps));
    for (int64_t c = 0; c < cols; c++) d[c] = src[c] * inv;
  }
}

/* kernels/scalar/indexer.go:11-32 (float32 accumulation) */
void orc_indexer_scores(float *dst, const float *q, const float *k, const float *w, int64_t rows,
                        int64_t blocks, int64_t heads, int64_t dim) {
  for (int64_t r = 0; r < rows; r++)
    for (int64_t b = 0; b < blocks; b++) {
      float total = 0;
      for (int64_t h = 0; h < heads; h++) {
        const float *qh = q + (r * heads + h) * dim;
        const float *kh = k + (b * heads + h) * dim;
        float dot = 0;
        for (int64_t e = 0; e < dim; e++) dot += qh[e] * kh[e];
        if (dot > 0) total += w[h] * dot;
      }
      dst[r * blocks + b] = total;
    }
}
/* kernels/scalar/indexer.go:41-61 */
void orc_indexer_block_max(float *dst, const float *scores, int64_t rows, int64_t blocks,
                           int64_t group) {
  if (group < 1) group = 1;
  int64_t groups = (blocks + group - 1) / group;
  for (int64_t r = 0; r < rows; r++)
    for (int64_t g = 0; g < groups; g++) {
      int64_t s = g * group, e = s + group < blocks ? s + group : blocks;
      float m = -INFINITY;
      for (int64_t i = s; i < e; i++)
        if (scores[r * blocks + i] > m) m = scores[r * blocks + i];
      dst[r * groups + g] = m;
    }
}

/* kernels/scalar/moe.go:8-30 */
void orc_topk_indices(int32_t *dst, const float *scores, int64_t rows, int64_t count, int64_t k) {
  if (count == 0 || k <= 0) return;
  int64_t limit = k < count ? k : count;
  float *work = (float *)malloc(sizeof(float) * count);
  for (int64_t r = 0; r < rows; r++) {
    memcpy(work, scores + r * count, sizeof(float) * count);
    for (int64_t s = 0; s < limit; s++) {
      int64_t best = 0;
      for (int64_t e = 1; e < count; e++)
        if (work[e] > work[best]) best = e;
      dst[r * k + s] = (int32_t)best;
      work[best] = -INFINITY;
    }
  }
  free(work);
}
/* kernels/scalar/moe.go:34-50 */
void orc_moe_gate_topk(const float *logits, const float *bias, float *probs, int32_t *selected,
                       float *weights, int64_t rows, int64_t experts, int64_t k) {
  orc_softmax_last_dim(probs, logits, rows, experts);
  float *scores = (float *)malloc(sizeof(float) * rows * experts);
  for (int64_t i = 0; i < rows * experts; i++) scores[i] = logits[i] + bias[i % experts];
  orc_topk_indices(selected, scores, rows, experts, k);
  int64_t limit = k < experts ? k : experts;
  for (int64_t r = 0; r < rows; r++)
    for (int64_t s = 0; s < limit; s++)
      weights[r * k + s] = probs[r * experts + selected[r * k + s]];
  free(scores);
}
/* kernels/scalar/moe.go:54-73 (float32 accumulation) */
void orc_grouped_matmul_transposed(float *dst, const float *in, const float *w,
                                   const int32_t *counts, int64_t experts, int64_t cols,
                                   int64_t inner) {
  int64_t off = 0;
  for (int64_t e = 0; e < experts; e++) {
    int64_t cnt = counts[e];
    const float *wb = w + e * cols * inner;
    for (int64_t r = 0; r < cnt; r++) {
      const float *ir = in + (off + r) * inner;
      float *dr = dst + (off + r) * cols;
      for (int64_t c = 0; c < cols; c++) {
        const float *wr = wb + c * inner;
        float t = 0;
        for (int64_t i = 0; i < inner; i++) t += ir[i] * wr[i];
        dr[c] = t;
      }
    }
    off += cnt;
  }
}

/* ---------------------------------------------------------------------- */
/* Attention (kernels/scalar/attention.go).                                */
/* ---------------------------------------------------------------------- */
#define MASKED_SCORE (-1e30f) /* kernels/scalar/attention.go:11 */

/* kernels/scalar/attention.go:210-228 (applyAttentionMask) */
static void apply_mask(float *scores, int64_t qlen, int64_t klen, int64_t offset, int64_t window,
                       const int32_t *seg, int64_t nseg) {
  int32_t qseg = 0;
  for (int64_t qi = 0; qi < qlen; qi++) {
    int64_t qpos = offset + qi;
    if (seg && qpos < nseg) qseg = seg[qpos];
    float *row = scores + qi * klen;
    for (int64_t kj = 0; kj < klen; kj++) {
      int masked = kj > qpos || (window >= 0 && qpos - kj > window);
      if (!masked && seg && kj < nseg && seg[kj] != qseg) masked = 1;
      if (masked) row[kj] = MASKED_SCORE;
    }
  }
}

/* kernels/scalar/attention.go:16-49 */
void orc_attention_forward(const float *q, const float *k, const float *v, float *out, float *lse,
                           const int32_t *segment, int64_t nseg, int64_t qlen, int64_t klen,
                           int64_t dim, int64_t offset, int64_t window) {
  float *scores = (float *)malloc(sizeof(float) * (qlen * klen + 1));
  float *probs = (float *)malloc(sizeof(float) * (qlen * klen + 1));
  orc_matmul_transposed(scores, q, k, qlen, klen, dim);
  apply_mask(scores, qlen, klen, offset, window, segment, nseg);
  for (int64_t qi = 0; qi < qlen; qi++) {
    float *rs = scores + qi * klen, *rp = probs + qi * klen;
    float m = orc_max(rs, klen);
    double total = 0;
    for (int64_t kj = 0; kj < klen; kj++) {
      double e = exp((double)(rs[kj] - m));
      rp[kj] = (float)e;
      total += e;
    }
    if (lse) lse[qi] = m + (float)log(total);
    float inv = (float)(1.0 / total);
    for (int64_t d = 0; d < dim; d++) {
      double a = 0;
      for (int64_t kj = 0; kj < klen; kj++) a += (double)rp[kj] * (double)v[kj * dim + d];
      out[qi * dim + d] = (float)a * inv;
    }
  }
  free(scores);
  free(probs);
}

/* kernels/scalar/attention.go:54-103 */
void orc_attention_forward_split(const float *q, const float *k, const float *v, float *acc,
                                 float *mx, float *sum, const int32_t *segment, int64_t nseg,
                                 int64_t qlen, int64_t klen, int64_t dim, int64_t offset,
                                 int64_t window, int64_t kstart, int64_t kend) {
  if (kend > klen) kend = klen;
  int64_t range = kend - kstart;
  if (range < 0) range = 0;
  float *scores = (float *)malloc(sizeof(float) * (range + 1));
  for (int64_t qi = 0; qi < qlen; qi++) {
    const float *qr = q + qi * dim;
    int64_t qpos = offset + qi;
    float *ar = acc + qi * dim;
    memset(ar, 0, sizeof(float) * dim);
    float m = -INFINITY;
    for (int64_t c = 0; c < range; c++) {
      int64_t kj = kstart + c;
      float s = orc_dot(qr, k + kj * dim, dim);
      int masked = kj > qpos || (window >= 0 && qpos - kj > window);
      if (!masked && segment && kj < nseg && qpos < nseg && segment[kj] != segment[qpos])
        masked = 1;
      if (masked) s = MASKED_SCORE;
      scores[c] = s;
      if (s > m) m = s;
    }
    double total = 0;
    for (int64_t c = 0; c < range; c++) {
      double p = exp((double)(scores[c] - m));
      total += p;
      const float *vr = v + (kstart + c) * dim;
      for (int64_t d = 0; d < dim; d++) ar[d] += (float)p * vr[d];
    }
    mx[qi] = m;
    sum[qi] = (float)total;
  }
  free(scores);
}

/* kernels/scalar/attention.go:107-141 */
void orc_attention_combine(const float *acc, const float *mx, const float *sum, int64_t nparts,
                           float *out, float *lse, int64_t qlen, int64_t dim) {
  for (int64_t qi = 0; qi < qlen; qi++) {
    float gm = -INFINITY;
    for (int64_t p = 0; p < nparts; p++)
      if (mx[p * qlen + qi] > gm) gm = mx[p * qlen + qi];
    double total = 0;
    float *o = out + qi * dim;
    memset(o, 0, sizeof(float) * dim);
    for (int64_t p = 0; p < nparts; p++) {
      float scale = 0;
      if (mx[p * qlen + qi] > -INFINITY) scale = (float)exp((double)(mx[p * qlen + qi] - gm));
      total += (double)sum[p * qlen + qi] * (double)scale;
      const float *a = acc + (p * qlen + qi) * dim;
      for (int64_t d = 0; d < dim; d++) o[d] += a[d] * scale;
    }
    if (total > 0) {
      float inv = (float)(1.0 / total);
      for (int64_t d = 0; d < dim; d++) o[d] *= inv;
    }
    if (lse) lse[qi] = gm + (float)log(total);
  }
}

/* kernels/scalar/attention.go:145-205 (gradients accumulate into dq/dk/dv) */
void orc_attention_backward(const float *q, const float *k, const float *v, const float *o,
                            const float *dout, const float *lse, const float *row_correction,
                            const int32_t *segment, int64_t nseg, float *dq, float *dk, float *dv,
                            int64_t qlen, int64_t klen, int64_t dim, int64_t offset,
                            int64_t window) {
  (void)o;
  int64_t qk = qlen * klen;
  float *scores = (float *)malloc(sizeof(float) * (qk + 1));
  float *probs = (float *)malloc(sizeof(float) * (qk + 1));
  float *tmp = (float *)malloc(sizeof(float) * (qk + 1));
  float *dsc = (float *)malloc(sizeof(float) * (qk + 1));
  float *dp = (float *)malloc(sizeof(float) * (qk + 1));
  float *grad = (float *)malloc(sizeof(float) * ((qlen > klen ? qlen : klen) * dim + 1));
  orc_matmul_transposed(scores, q, k, qlen, klen, dim);
  apply_mask(scores, qlen, klen, offset, window, segment, nseg);
  for (int64_t qi = 0; qi < qlen; qi++) {
    float l = lse[qi];
    for (int64_t kj = 0; kj < klen; kj++) {
      float s = scores[qi * klen + kj];
      probs[qi * klen + kj] = s <= MASKED_SCORE ? 0.0f : (float)exp((double)(s - l));
    }
  }
  /* dV += P^T dO */
  for (int64_t qi = 0; qi < qlen; qi++)
    for (int64_t kj = 0; kj < klen; kj++) tmp[kj * qlen + qi] = probs[qi * klen + kj];
  orc_matmul(grad, tmp, dout, klen, dim, qlen);
  for (int64_t i = 0; i < klen * dim; i++) dv[i] += grad[i];
  /* dS = P * (dP - rowsum) */
  orc_matmul_transposed(dp, dout, v, qlen, klen, dim);
  for (int64_t qi = 0; qi < qlen; qi++) {
    double rd = 0;
    if (row_correction) rd = (double)row_correction[qi];
    else
      for (int64_t kj = 0; kj < klen; kj++)
        rd += (double)dp[qi * klen + kj] * (double)probs[qi * klen + kj];
    for (int64_t kj = 0; kj < klen; kj++) {
      double p = (double)probs[qi * klen + kj];
      dsc[qi * klen + kj] = (float)(p * ((double)dp[qi * klen + kj] - rd));
    }
  }
  /* dQ += dS K */
  orc_matmul(grad, dsc, k, qlen, dim, klen);
  for (int64_t i = 0; i < qlen * dim; i++) dq[i] += grad[i];
  /* dK += dS^T Q */
  for (int64_t qi = 0; qi < qlen; qi++)
    for (int64_t kj = 0; kj < klen; kj++) tmp[kj * qlen + qi] = dsc[qi * klen + kj];
  orc_matmul(grad, tmp, q, klen, dim, qlen);
  for (int64_t i = 0; i < klen * dim; i++) dk[i] += grad[i];
  free(scores);
  free(probs);
  free(tmp);
  free(dsc);
  free(dp);
  free(grad);
}
