/*
 * optimizer.c - the MuonAdamW optimizer step restated in C.
 *
 * TEST INFRASTRUCTURE ONLY (see gn_oracle.h): the checker for the GPU
 * optimizer step, never part of the product path.
 *
 * One call applies MuonAdamW.Step (optimizer/optimizer.go:118-137) to a flat
 * float32 parameter vector from its gradient vector.  The parameter groups
 * arrive as a table of tensors (or tensor views: a head or an expert block
 * of a packed weight), each with its group's kind and hyperparameters, in
 * the order MuonAdamW iterates them (groups in SetupOptimizer order,
 * model/optimizer.go:16-181, tensors in group order).  The arithmetic keeps
 * the reference's types: float32 data, float64 where the Go code converts
 * (AdamW moments, Sinkhorn momentum and norms, every norm's sum of squares),
 * float32 elsewhere, no fused multiply-adds (-ffp-contract=off).
 *
 * Optimizer state: every tensor owns a consecutive region of `state`
 * (orc_opt_state_floats gives the size): AdamW expAvg[n], expAvgSq[n];
 * Muon momentum[n], secondMom[max(rows, cols)]; Sinkhorn momentum[n].
 * AdamW step counts live in `steps` (one per table entry).
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "gn_oracle.h"

/* optimizer/muon.go:12-18: quintic Polar Express coefficients (ns_steps <= 5) */
static const double PE_COEFFS[5][3] = {
    {8.156554524902461, -22.48329292557795, 15.878769915207462},
    {4.042929935166739, -2.808917465908714, 0.5000178451051316},
    {3.8916678022926607, -2.772484153217685, 0.5060648178503393},
    {3.285753657755655, -2.3681294933425376, 0.46449024233003106},
    {2.3465413258596377, -1.7097828382687081, 0.42323551169305323},
};

int64_t orc_opt_state_floats(const orc_opt_param *t, int n) {
  int64_t total = 0;
  for (int i = 0; i < n; i++) {
    const int64_t numel = (int64_t)t[i].rows * t[i].cols;
    if (t[i].kind == ORC_OPT_ADAMW) total += 2 * numel;
    else if (t[i].kind == ORC_OPT_MUON) total += numel + (t[i].rows >= t[i].cols ? t[i].rows : t[i].cols);
    else total += numel;
  }
  return total;
}

/* optimizer/optimizer.go:150-174 (adamwStep) */
static void adamw_step(float *p, const float *g, int64_t n, const orc_opt_param *h, float *m,
                       float *v, int32_t *step) {
  (*step)++;
  const double beta1 = h->beta1, beta2 = h->beta2, eps = h->eps, wd = h->weight_decay,
               lr = h->lr;
  const double bias1 = 1 - pow(beta1, (double)*step);
  const double bias2 = 1 - pow(beta2, (double)*step);
  const double decay = 1 - lr * wd;
  const double step_size = lr / bias1;
  for (int64_t i = 0; i < n; i++) {
    p[i] *= (float)decay;
    m[i] = (float)(beta1 * (double)m[i] + (1 - beta1) * (double)g[i]);
    v[i] = (float)(beta2 * (double)v[i] + (1 - beta2) * (double)g[i] * (double)g[i]);
    const double denom = sqrt((double)v[i] / bias2) + eps;
    p[i] -= (float)(step_size * (double)m[i] / denom);
  }
}

/* optimizer/muon.go:176-183 (computeFrobeniusNorm / computeRowL2Norm) */
static float norm_f32(const float *x, int64_t n) {
  double s = 0;
  for (int64_t i = 0; i < n; i++) s += (double)x[i] * (double)x[i];
  return (float)sqrt(s);
}

static void transpose(float *dst, const float *src, int64_t rows, int64_t cols) {
  for (int64_t r = 0; r < rows; r++)
    for (int64_t c = 0; c < cols; c++) dst[c * rows + r] = src[r * cols + c];
}

/* Polar Express orthogonalization of u [rows, cols] in place
 * (optimizer/muon.go:50-74), matmuls through kernels.Backend MatMul. */
void orc_polar_express(float *u, int64_t rows, int64_t cols, int steps) {
  const int64_t n = rows * cols;
  const float norm = norm_f32(u, n);
  const float scale = (float)(1.0 / ((double)norm * 1.01 + 1e-6));
  for (int64_t i = 0; i < n; i++) u[i] *= scale;
  const int tall = rows > cols;
  const int64_t gd = tall ? cols : rows;
  float *ut = malloc(sizeof(float) * n);
  float *gram = malloc(sizeof(float) * gd * gd);
  float *gram2 = malloc(sizeof(float) * gd * gd);
  float *poly = malloc(sizeof(float) * gd * gd);
  float *prod = malloc(sizeof(float) * n);
  for (int s = 0; s < steps; s++) {
    const float a = (float)PE_COEFFS[s][0], b = (float)PE_COEFFS[s][1], c = (float)PE_COEFFS[s][2];
    transpose(ut, u, rows, cols);
    if (tall) orc_matmul(gram, ut, u, cols, cols, rows); /* u^T u */
    else orc_matmul(gram, u, ut, rows, rows, cols);      /* u u^T */
    orc_matmul(gram2, gram, gram, gd, gd, gd);
    for (int64_t i = 0; i < gd * gd; i++) {
      const float t1 = gram[i] * b, t2 = gram2[i] * c; /* tensors.Scale */
      poly[i] = t1 + t2;                               /* tensors.Add */
    }
    if (tall) orc_matmul(prod, u, poly, rows, cols, cols);
    else orc_matmul(prod, poly, u, rows, cols, rows);
    for (int64_t i = 0; i < n; i++) {
      const float t1 = u[i] * a;
      u[i] = t1 + prod[i];
    }
  }
  free(ut);
  free(gram);
  free(gram2);
  free(poly);
  free(prod);
}

/* optimizer/muon.go:23-174 (muonStep) */
static void muon_step(float *p, const float *g, int64_t rows, int64_t cols, const orc_opt_param *h,
                      float *mom, float *second) {
  const int64_t n = rows * cols;
  const float mu = h->momentum;
  float *u = malloc(sizeof(float) * n);
  /* Nesterov momentum (float32) */
  for (int64_t i = 0; i < n; i++) {
    const float keep = mu * mom[i], add = (1 - mu) * g[i];
    mom[i] = keep + add;
    const float t1 = (1 - mu) * g[i], t2 = mu * mom[i];
    u[i] = t1 + t2;
  }
  /* MuonEq row equilibration */
  const float target = norm_f32(u, n) / (float)sqrt((double)rows);
  for (int64_t r = 0; r < rows; r++) {
    float rn = norm_f32(u + r * cols, cols);
    if (rn < 1e-6f) rn = 1e-6f;
    const float sc = target / rn;
    for (int64_t c = 0; c < cols; c++) u[r * cols + c] *= sc;
  }
  orc_polar_express(u, rows, cols, h->ns_steps);
  /* Muon+ renormalization */
  const float tnorm = (float)sqrt((double)(rows < cols ? rows : cols));
  float cur = norm_f32(u, n);
  if (cur < 1e-6f) cur = 1e-6f;
  const float rs = tnorm / cur;
  for (int64_t i = 0; i < n; i++) u[i] *= rs;
  /* variance reduction (NorMuon) */
  const int by_row = rows >= cols;
  const int64_t nm = by_row ? rows : cols, red = by_row ? cols : rows;
  float *mean = malloc(sizeof(float) * nm);
  float *step = malloc(sizeof(float) * nm);
  for (int64_t j = 0; j < nm; j++) {
    double s = 0;
    for (int64_t k = 0; k < red; k++) {
      const double x = by_row ? u[j * cols + k] : u[k * cols + j];
      s += x * x;
    }
    mean[j] = (float)(s / (double)red);
  }
  double vns = 0;
  for (int64_t j = 0; j < nm; j++) vns += (double)mean[j];
  vns *= (double)red;
  const float vnorm = (float)sqrt(vns);
  const float b2 = h->muon_beta2;
  for (int64_t j = 0; j < nm; j++) {
    const float keep = b2 * second[j], add = (1 - b2) * mean[j];
    second[j] = keep + add;
    float sm = second[j];
    if (sm < 1e-10f) sm = 1e-10f;
    step[j] = (float)(1.0 / sqrt((double)sm));
  }
  double nvs = 0;
  for (int64_t j = 0; j < nm; j++)
    nvs += (double)mean[j] * (double)red * (double)step[j] * (double)step[j];
  float nvn = (float)sqrt(nvs);
  if (nvn < 1e-10f) nvn = 1e-10f;
  const float ratio = vnorm / nvn;
  for (int64_t j = 0; j < nm; j++) step[j] = step[j] * ratio;
  for (int64_t r = 0; r < rows; r++)
    for (int64_t c = 0; c < cols; c++) u[r * cols + c] *= step[by_row ? r : c];
  /* cautious weight decay + update */
  const float lr = h->lr, lrwd = h->lr * h->weight_decay;
  for (int64_t i = 0; i < n; i++) {
    const float mask = u[i] * p[i] >= 0 ? 1.f : 0.f;
    const float t1 = lr * u[i];
    const float t2 = lrwd * p[i] * mask;
    p[i] -= t1 + t2;
  }
  free(u);
  free(mean);
  free(step);
}

/* optimizer/sinkhorn.go:26-95 (sinkhornStep) */
static void sinkhorn_step(float *p, const float *g, int64_t rows, int64_t cols,
                          const orc_opt_param *h, float *mom) {
  const int64_t n = rows * cols;
  const double beta = h->momentum;
  float *u = malloc(sizeof(float) * n);
  for (int64_t i = 0; i < n; i++) {
    const double mv = beta * (double)mom[i] + (1 - beta) * (double)g[i];
    mom[i] = (float)mv;
    u[i] = (float)(beta * mv + (1 - beta) * (double)g[i]);
  }
  double *rn = malloc(sizeof(double) * rows);
  double nsum = 0;
  for (int64_t r = 0; r < rows; r++) {
    double s = 0;
    for (int64_t c = 0; c < cols; c++) s += (double)u[r * cols + c] * (double)u[r * cols + c];
    rn[r] = sqrt(s);
    nsum += rn[r];
  }
  const double thr = (double)h->tau * nsum / (double)rows;
  for (int64_t r = 0; r < rows; r++)
    if (rn[r] <= thr) memset(u + r * cols, 0, sizeof(float) * cols);
  const double eps = h->sinkhorn_eps;
  for (int s = 1; s <= h->sinkhorn_steps; s++) {
    if (s % 2 == 1) {
      for (int64_t r = 0; r < rows; r++) {
        float *x = u + r * cols;
        double q = 0;
        for (int64_t c = 0; c < cols; c++) q += (double)x[c] * (double)x[c];
        const double sc = 1.0 / (sqrt(q) + eps);
        for (int64_t c = 0; c < cols; c++) x[c] = (float)((double)x[c] * sc);
      }
    } else {
      for (int64_t c = 0; c < cols; c++) {
        double q = 0;
        for (int64_t r = 0; r < rows; r++) q += (double)u[r * cols + c] * (double)u[r * cols + c];
        const double sc = 1.0 / (sqrt(q) + eps);
        for (int64_t r = 0; r < rows; r++) u[r * cols + c] = (float)((double)u[r * cols + c] * sc);
      }
    }
  }
  const double lr = (double)h->gamma * (double)h->lr * sqrt((double)cols);
  for (int64_t i = 0; i < n; i++) p[i] -= (float)(lr * (double)u[i]);
  free(u);
  free(rn);
}

/* optimizer/optimizer.go:118-137 (MuonAdamW.Step) over the tensor table */
void orc_opt_step(float *params, const float *grads, const orc_opt_param *t, int n, float *state,
                  int32_t *steps) {
  float *st = state;
  for (int i = 0; i < n; i++) {
    const orc_opt_param *h = &t[i];
    const int64_t numel = (int64_t)h->rows * h->cols;
    float *p = params + h->offset;
    const float *g = grads + h->offset;
    if (h->kind == ORC_OPT_ADAMW) {
      adamw_step(p, g, numel, h, st, st + numel, &steps[i]);
      st += 2 * numel;
    } else if (h->kind == ORC_OPT_MUON) {
      muon_step(p, g, h->rows, h->cols, h, st, st + numel);
      st += numel + (h->rows >= h->cols ? h->rows : h->cols);
    } else {
      sinkhorn_step(p, g, h->rows, h->cols, h, st);
      st += numel;
    }
  }
}
