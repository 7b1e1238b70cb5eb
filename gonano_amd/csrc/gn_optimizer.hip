// gn_optimizer.hip - MuonAdamW (optimizer/optimizer.go, muon.go, sinkhorn.go)
// on the device parameters and gradients.
//
//  * AdamW (optimizer.go:150-174): one elementwise pass, float64 moment
//    arithmetic per element as the reference converts it.
//  * Muon (muon.go:23-174): Nesterov momentum, MuonEq row equilibration,
//    Polar Express (5 quintic iterations: Gram matrix, its square and the
//    polynomial product on the fp32 GEMM, the scalings elementwise), Muon+
//    renormalization, NorMuon variance reduction and the cautious update.
//    The matrix products are the dominant cost (MFMA-bound); every other
//    pass streams the matrix once.
//  * Sinkhorn (sinkhorn.go:26-95): Nesterov momentum in float64, near-zero
//    row masking, 11 alternating row/column L2 normalizations and the
//    gamma-scaled update.  HBM-bound: each column normalization is fused
//    into the next row pass (scale on read), the last row pass writes the
//    parameter, so the matrix is streamed 2 + 2 * (K-1)/2 times.
//
// Reductions are deterministic: float64 partial sums in a fixed block
// order, never atomics.  Elementwise float32 arithmetic is not contracted
// into fused multiply-adds (the reference's Go and the C oracle round each
// product and sum).
#include "gn_optimizer.h"

#pragma clang fp contract(off)

namespace gn {

static constexpr int RED_BLOCKS = 256;  // fixed partial count of a full reduction

// ---------------------------------------------------------------------------
// reductions
// ---------------------------------------------------------------------------
// part[block] = sum of x^2 over a grid-stride range (float64)
__global__ __launch_bounds__(256) void sumsq_partials_kernel(const float* __restrict__ x, int64_t n,
                                                             double* __restrict__ part) {
  __shared__ double sc[4];
  double s = 0.0;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const double v = x[i];
    s += v * v;
  }
  s = block_sum<double>(s, sc);
  if (threadIdx.x == 0) part[blockIdx.x] = s;
}
// out[0] = sum of part[0..n) (one block, fixed order)
__global__ __launch_bounds__(256) void sum_f64_block_kernel(const double* __restrict__ part, int n,
                                                            double* __restrict__ out) {
  __shared__ double sc[4];
  double s = 0.0;
  for (int i = threadIdx.x; i < n; i += 256) s += part[i];
  s = block_sum<double>(s, sc);
  if (threadIdx.x == 0) out[0] = s;
}
static void sumsq(const float* x, int64_t n, double* part, double* out, hipStream_t st) {
  hipLaunchKernelGGL(sumsq_partials_kernel, dim3(RED_BLOCKS), dim3(256), 0, st, x, n, part);
  hipLaunchKernelGGL(sum_f64_block_kernel, dim3(1), dim3(256), 0, st, part, RED_BLOCKS, out);
}
// out[r] = sum over the row of x^2 (one block per row)
__global__ __launch_bounds__(256) void row_sumsq_kernel(const float* __restrict__ x, int64_t cols,
                                                        double* __restrict__ out) {
  __shared__ double sc[4];
  const float* row = x + (int64_t)blockIdx.x * cols;
  double s = 0.0;
  for (int64_t c = threadIdx.x; c < cols; c += 256) {
    const double v = row[c];
    s += v * v;
  }
  s = block_sum<double>(s, sc);
  if (threadIdx.x == 0) out[blockIdx.x] = s;
}
// part[chunk][c] = sum over the chunk's rows of x[r][c]^2 (thread per column)
static constexpr int COL_CHUNK = 512;
__global__ __launch_bounds__(256) void col_sumsq_partials_kernel(const float* __restrict__ x,
                                                                 int64_t rows, int64_t cols,
                                                                 double* __restrict__ part) {
  const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (c >= cols) return;
  const int64_t r0 = (int64_t)blockIdx.y * COL_CHUNK, r1 = min(rows, r0 + COL_CHUNK);
  double s = 0.0;
  for (int64_t r = r0; r < r1; r++) {
    const double v = x[r * cols + c];
    s += v * v;
  }
  part[blockIdx.y * cols + c] = s;
}
// out[c] = sum over chunks (chunk order) of part[chunk][c]
__global__ void col_finish_kernel(const double* __restrict__ part, int nchunks, int64_t cols,
                                  double* __restrict__ out) {
  const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (c >= cols) return;
  double s = 0.0;
  for (int k = 0; k < nchunks; k++) s += part[(int64_t)k * cols + c];
  out[c] = s;
}
static void col_sumsq(const float* x, int64_t rows, int64_t cols, double* part, double* out,
                      hipStream_t st) {
  const int nch = (int)ceil_div(rows, COL_CHUNK);
  hipLaunchKernelGGL(col_sumsq_partials_kernel, dim3((unsigned)ceil_div(cols, 256), nch), dim3(256),
                     0, st, x, rows, cols, part);
  hipLaunchKernelGGL(col_finish_kernel, dim3((unsigned)ceil_div(cols, 256)), dim3(256), 0, st, part,
                     nch, cols, out);
}

// ---------------------------------------------------------------------------
// AdamW (optimizer.go:150-174)
// ---------------------------------------------------------------------------
__global__ void adamw_kernel(float* __restrict__ p, const float* __restrict__ g,
                             float* __restrict__ m, float* __restrict__ v, int64_t n, float decay,
                             double beta1, double beta2, double bias2, double step_size,
                             double eps) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const double gi = g[i];
  float pi = p[i] * decay;
  const float mi = (float)(beta1 * (double)m[i] + (1 - beta1) * gi);
  const float vi = (float)(beta2 * (double)v[i] + (1 - beta2) * gi * gi);
  const double denom = sqrt((double)vi / bias2) + eps;
  pi -= (float)(step_size * (double)mi / denom);
  m[i] = mi;
  v[i] = vi;
  p[i] = pi;
}

// ---------------------------------------------------------------------------
// Sinkhorn (sinkhorn.go:26-95)
// ---------------------------------------------------------------------------
__global__ void sk_momentum_kernel(float* __restrict__ mom, const float* __restrict__ g,
                                   float* __restrict__ u, int64_t n, double beta) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const double gi = g[i];
  const double mv = beta * (double)mom[i] + (1 - beta) * gi;
  mom[i] = (float)mv;
  u[i] = (float)(beta * mv + (1 - beta) * gi);
}
// threshold = tau * (sum of row norms) / rows (one block; row norms from
// their sums of squares)
__global__ __launch_bounds__(256) void sk_threshold_kernel(const double* __restrict__ rn2,
                                                           int64_t rows, double tau,
                                                           double* __restrict__ thr) {
  __shared__ double sc[4];
  double s = 0.0;
  for (int64_t r = threadIdx.x; r < rows; r += 256) s += sqrt(rn2[r]);
  s = block_sum<double>(s, sc);
  if (threadIdx.x == 0) thr[0] = tau * s / (double)rows;
}
// One row pass over u: optionally apply a pending column normalization
// (cscale[c] = column sum of squares), then
//   first: zero rows whose norm (rn2) is <= thr, normalize the rest by it;
//   else:  normalize the row by its own norm (if `rownorm`);
// and write u, or (last pass) p -= lr * u.
__global__ __launch_bounds__(256) void sk_row_kernel(float* __restrict__ u, int64_t cols,
                                                     const double* __restrict__ csumsq,
                                                     const double* __restrict__ rn2,
                                                     const double* __restrict__ thr, bool rownorm,
                                                     double eps, float* __restrict__ p, double lr) {
  __shared__ double sc[4];
  float* row = u + (int64_t)blockIdx.x * cols;
  auto value = [&](int64_t c) -> float {
    float v = row[c];
    if (csumsq) v = (float)((double)v * (1.0 / (sqrt(csumsq[c]) + eps)));
    return v;
  };
  double rs = 1.0;
  if (rn2) {
    const double nrm = sqrt(rn2[blockIdx.x]);
    rs = nrm <= thr[0] ? 0.0 : 1.0 / (nrm + eps);
  } else if (rownorm) {
    double s = 0.0;
    for (int64_t c = threadIdx.x; c < cols; c += 256) {
      const double v = value(c);
      s += v * v;
    }
    s = block_sum<double>(s, sc);
    rs = 1.0 / (sqrt(s) + eps);
  }
  for (int64_t c = threadIdx.x; c < cols; c += 256) {
    float v = value(c);
    if (rn2 || rownorm) v = (float)((double)v * rs);
    if (p) {
      float* pr = p + (int64_t)blockIdx.x * cols;
      pr[c] -= (float)(lr * (double)v);
    } else {
      row[c] = v;
    }
  }
}

// ---------------------------------------------------------------------------
// Muon (muon.go:23-174)
// ---------------------------------------------------------------------------
__global__ void mu_nesterov_kernel(float* __restrict__ mom, const float* __restrict__ g,
                                   float* __restrict__ u, int64_t n, float mu) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float gi = g[i], keep = 1.f - mu;
  const float m = mu * mom[i] + keep * gi;
  mom[i] = m;
  u[i] = keep * gi + mu * m;
}
// MuonEq: row r scaled to the mean row norm (target = ||u||_F / sqrt(rows));
// writes the scaled row's sum of squares.
__global__ __launch_bounds__(256) void mu_roweq_kernel(float* __restrict__ u, int64_t rows,
                                                       int64_t cols, const double* __restrict__ fro2,
                                                       double* __restrict__ rowss) {
  __shared__ double sc[4];
  float* row = u + (int64_t)blockIdx.x * cols;
  double s = 0.0;
  for (int64_t c = threadIdx.x; c < cols; c += 256) {
    const double v = row[c];
    s += v * v;
  }
  s = block_sum<double>(s, sc);
  float rn = (float)sqrt(s);
  if (rn < 1e-6f) rn = 1e-6f;
  const float target = (float)sqrt(fro2[0]) / (float)sqrt((double)rows);
  const float scale = target / rn;
  double s2 = 0.0;
  for (int64_t c = threadIdx.x; c < cols; c += 256) {
    const float v = row[c] * scale;
    row[c] = v;
    s2 += (double)v * (double)v;
  }
  s2 = block_sum<double>(s2, sc);
  if (threadIdx.x == 0) rowss[blockIdx.x] = s2;
}
// u *= 1 / (1.01 ||u|| + 1e-6) (Polar Express input scaling)
__global__ void mu_pe_scale_kernel(float* __restrict__ u, int64_t n, const double* __restrict__ fro2) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float norm = (float)sqrt(fro2[0]);
  u[i] *= (float)(1.0 / ((double)norm * 1.01 + 1e-6));
}
// poly = b * gram + c * gram^2 (tensors.Scale, tensors.Add)
__global__ void mu_poly_kernel(const float* __restrict__ gram, const float* __restrict__ gram2,
                               float* __restrict__ poly, int64_t n, float b, float c) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float t1 = gram[i] * b, t2 = gram2[i] * c;
  poly[i] = t1 + t2;
}
// u = a * u + prod
__global__ void mu_combine_kernel(float* __restrict__ u, const float* __restrict__ prod, int64_t n,
                                  float a) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float t1 = u[i] * a;
  u[i] = t1 + prod[i];
}
// Muon+: u *= target / max(||u||, 1e-6)
__global__ void mu_renorm_kernel(float* __restrict__ u, int64_t n, const double* __restrict__ fro2,
                                 float target) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  float cur = (float)sqrt(fro2[0]);
  if (cur < 1e-6f) cur = 1e-6f;
  u[i] *= target / cur;
}
// NorMuon variance reduction statistics (one block): from the per-row
// (rows >= cols) or per-column sums of squares `ss` [nm] over `red` entries:
// means, the second-moment update, the step sizes and their norm-preserving
// ratio; writes the final per-row/column scales fs [nm].
__global__ __launch_bounds__(256) void mu_vr_kernel(const double* __restrict__ ss, int64_t nm,
                                                    int64_t red, float* __restrict__ second,
                                                    float beta2, float* __restrict__ fs) {
  __shared__ double sc[4];
  __shared__ float ratio_s;
  double vn = 0.0, nv = 0.0;
  for (int64_t j = threadIdx.x; j < nm; j += 256) {
    const float mean = (float)(ss[j] / (double)red);
    vn += (double)mean;
    const float keep = beta2 * second[j], add = (1.f - beta2) * mean;
    const float s2 = keep + add;
    second[j] = s2;
    const float sm = s2 < 1e-10f ? 1e-10f : s2;
    const float step = (float)(1.0 / sqrt((double)sm));
    fs[j] = step;
    nv += (double)mean * (double)red * (double)step * (double)step;
  }
  vn = block_sum<double>(vn, sc);
  nv = block_sum<double>(nv, sc);
  if (threadIdx.x == 0) {
    const float vnorm = (float)sqrt(vn * (double)red);
    float nvn = (float)sqrt(nv);
    if (nvn < 1e-10f) nvn = 1e-10f;
    ratio_s = vnorm / nvn;
  }
  __syncthreads();
  const float ratio = ratio_s;
  for (int64_t j = threadIdx.x; j < nm; j += 256) fs[j] = fs[j] * ratio;
}
// cautious weight decay + update with the variance-reduction scales
__global__ void mu_update_kernel(float* __restrict__ p, const float* __restrict__ u,
                                 const float* __restrict__ fs, int64_t rows, int64_t cols,
                                 bool by_row, float lr, float lrwd) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= rows * cols) return;
  const float v = u[i] * fs[by_row ? i / cols : i % cols];
  const float pi = p[i];
  const float mask = v * pi >= 0.f ? 1.f : 0.f;
  const float t1 = lr * v;
  const float t2 = lrwd * pi * mask;
  p[i] = pi - (t1 + t2);
}

// ---------------------------------------------------------------------------
// orchestration
// ---------------------------------------------------------------------------
// Polar Express coefficients (muon.go:12-18)
static const double PE_COEFFS[5][3] = {
    {8.156554524902461, -22.48329292557795, 15.878769915207462},
    {4.042929935166739, -2.808917465908714, 0.5000178451051316},
    {3.8916678022926607, -2.772484153217685, 0.5060648178503393},
    {3.285753657755655, -2.3681294933425376, 0.46449024233003106},
    {2.3465413258596377, -1.7097828382687081, 0.42323551169305323},
};

int64_t opt_state_floats(const gn_opt_param& h) {
  const int64_t n = (int64_t)h.rows * h.cols;
  if (h.kind == GN_OPT_ADAMW) return 2 * n;
  if (h.kind == GN_OPT_MUON) return n + std::max(h.rows, h.cols);
  return n;
}

static dim3 grid1(int64_t n) { return dim3((unsigned)ceil_div(n, 256)); }

struct OptScratch {
  float *u, *gram, *gram2, *poly, *prod, *fs;
  double *part, *scal, *vec, *vec2;
};

static void adamw_tensor(OptTensor& t, hipStream_t st) {
  t.step++;
  const gn_opt_param& h = t.h;
  const double beta1 = h.beta1, beta2 = h.beta2, lr = h.lr, wd = h.weight_decay;
  const double bias1 = 1 - std::pow(beta1, (double)t.step);
  const double bias2 = 1 - std::pow(beta2, (double)t.step);
  const double decay = 1 - lr * wd;
  const int64_t n = t.rows * t.cols;
  hipLaunchKernelGGL(adamw_kernel, grid1(n), dim3(256), 0, st, t.p, t.g, t.st, t.st + n, n,
                     (float)decay, beta1, beta2, bias2, lr / bias1, (double)h.eps);
}

static void sinkhorn_tensor(OptTensor& t, const OptScratch& w, hipStream_t st) {
  const gn_opt_param& h = t.h;
  const int64_t rows = t.rows, cols = t.cols, n = rows * cols;
  const double eps = h.sinkhorn_eps;
  const double lr = (double)h.gamma * (double)h.lr * std::sqrt((double)cols);
  hipLaunchKernelGGL(sk_momentum_kernel, grid1(n), dim3(256), 0, st, t.st, t.g, w.u, n,
                     (double)h.momentum);
  hipLaunchKernelGGL(row_sumsq_kernel, dim3((unsigned)rows), dim3(256), 0, st, w.u, cols, w.vec);
  hipLaunchKernelGGL(sk_threshold_kernel, dim3(1), dim3(256), 0, st, w.vec, rows, (double)h.tau,
                     w.scal);
  const int K = h.sinkhorn_steps;  // >= 1 (checked when the optimizer is built)
  // step 1: mask + row normalization (by the norms just computed)
  hipLaunchKernelGGL(sk_row_kernel, dim3((unsigned)rows), dim3(256), 0, st, w.u, cols,
                     (const double*)nullptr, (const double*)w.vec, w.scal, true, eps,
                     K == 1 ? t.p : (float*)nullptr, lr);
  // steps 2, 3 | 4, 5 | ...: column sums, then the column scaling applied in
  // the next row pass (which normalizes the rows again when that step exists)
  for (int s = 2; s <= K; s += 2) {
    col_sumsq(w.u, rows, cols, w.part, w.vec2, st);
    const bool rownorm = s + 1 <= K;
    const bool last = s + 1 >= K;
    hipLaunchKernelGGL(sk_row_kernel, dim3((unsigned)rows), dim3(256), 0, st, w.u, cols,
                       (const double*)w.vec2, (const double*)nullptr, w.scal, rownorm, eps,
                       last ? t.p : (float*)nullptr, lr);
  }
}

static void muon_tensor(OptTensor& t, const OptScratch& w, hipStream_t st, DeviceArena* ws) {
  const gn_opt_param& h = t.h;
  const int64_t rows = t.rows, cols = t.cols, n = rows * cols;
  float* mom = t.st;
  float* second = t.st + n;
  hipLaunchKernelGGL(mu_nesterov_kernel, grid1(n), dim3(256), 0, st, mom, t.g, w.u, n, h.momentum);
  sumsq(w.u, n, w.part, w.scal, st);
  hipLaunchKernelGGL(mu_roweq_kernel, dim3((unsigned)rows), dim3(256), 0, st, w.u, rows, cols,
                     (const double*)w.scal, w.vec);
  hipLaunchKernelGGL(sum_f64_block_kernel, dim3(1), dim3(256), 0, st, (const double*)w.vec,
                     (int)rows, w.scal + 1);
  hipLaunchKernelGGL(mu_pe_scale_kernel, grid1(n), dim3(256), 0, st, w.u, n,
                     (const double*)(w.scal + 1));
  // Polar Express: tall (rows > cols) works on u^T u, wide on u u^T
  const bool tall = rows > cols;
  const int gd = (int)(tall ? cols : rows);
  const int64_t g2 = (int64_t)gd * gd;
  for (int s = 0; s < h.ns_steps; s++) {
    const float a = (float)PE_COEFFS[s][0], b = (float)PE_COEFFS[s][1], c = (float)PE_COEFFS[s][2];
    GemmDesc d;
    if (tall) {  // gram[i][j] = sum_r u[r][i] u[r][j]
      d.M = gd; d.N = gd; d.K = (int)rows;
      d.A = w.u; d.lda = cols; d.a_kcontig = false;
      d.B = w.u; d.ldb = cols; d.b_kcontig = false;
    } else {  // gram[i][j] = sum_c u[i][c] u[j][c]
      d.M = gd; d.N = gd; d.K = (int)cols;
      d.A = w.u; d.lda = cols; d.a_kcontig = true;
      d.B = w.u; d.ldb = cols; d.b_kcontig = true;
    }
    d.C = w.gram; d.ldc = gd;
    gemm(d, st, ws);
    GemmDesc d2;  // gram2 = gram . gram
    d2.M = gd; d2.N = gd; d2.K = gd;
    d2.A = w.gram; d2.lda = gd; d2.a_kcontig = true;
    d2.B = w.gram; d2.ldb = gd; d2.b_kcontig = false;
    d2.C = w.gram2; d2.ldc = gd;
    gemm(d2, st, ws);
    hipLaunchKernelGGL(mu_poly_kernel, grid1(g2), dim3(256), 0, st, w.gram, w.gram2, w.poly, g2, b, c);
    GemmDesc d3;
    if (tall) {  // prod = u . poly  [rows, cols]
      d3.M = (int)rows; d3.N = (int)cols; d3.K = (int)cols;
      d3.A = w.u; d3.lda = cols; d3.a_kcontig = true;
      d3.B = w.poly; d3.ldb = cols; d3.b_kcontig = false;
    } else {  // prod = poly . u  [rows, cols]
      d3.M = (int)rows; d3.N = (int)cols; d3.K = (int)rows;
      d3.A = w.poly; d3.lda = rows; d3.a_kcontig = true;
      d3.B = w.u; d3.ldb = cols; d3.b_kcontig = false;
    }
    d3.C = w.prod; d3.ldc = cols;
    gemm(d3, st, ws);
    hipLaunchKernelGGL(mu_combine_kernel, grid1(n), dim3(256), 0, st, w.u, (const float*)w.prod, n, a);
  }
  // Muon+ renormalization to sqrt(min(rows, cols))
  sumsq(w.u, n, w.part, w.scal + 2, st);
  hipLaunchKernelGGL(mu_renorm_kernel, grid1(n), dim3(256), 0, st, w.u, n,
                     (const double*)(w.scal + 2), (float)std::sqrt((double)std::min(rows, cols)));
  // variance reduction over the longer side's rows (per row) or columns
  const bool by_row = rows >= cols;
  const int64_t nm = by_row ? rows : cols, red = by_row ? cols : rows;
  if (by_row)
    hipLaunchKernelGGL(row_sumsq_kernel, dim3((unsigned)rows), dim3(256), 0, st, w.u, cols, w.vec);
  else
    col_sumsq(w.u, rows, cols, w.part, w.vec, st);
  hipLaunchKernelGGL(mu_vr_kernel, dim3(1), dim3(256), 0, st, (const double*)w.vec, nm, red, second,
                     h.muon_beta2, w.fs);
  hipLaunchKernelGGL(mu_update_kernel, grid1(n), dim3(256), 0, st, t.p, (const float*)w.u,
                     (const float*)w.fs, rows, cols, by_row, h.lr, h.lr * h.weight_decay);
}

void optimizer_step(std::vector<OptTensor>& ts, hipStream_t st, DeviceArena* ws) {
  int64_t maxn = 1, maxg = 1, maxside = 1, maxparts = RED_BLOCKS;
  for (const OptTensor& t : ts) {
    if (t.h.kind == GN_OPT_ADAMW) continue;
    maxn = std::max<int64_t>(maxn, t.rows * t.cols);
    const int64_t gd = std::min(t.rows, t.cols);
    maxg = std::max<int64_t>(maxg, gd * gd);
    maxside = std::max<int64_t>(maxside, std::max(t.rows, t.cols));
    maxparts = std::max<int64_t>(maxparts, ceil_div(t.rows, COL_CHUNK) * t.cols);
  }
  OptScratch w;
  w.u = ws->get<float>("opt_u", maxn);
  w.prod = ws->get<float>("opt_prod", maxn);
  w.gram = ws->get<float>("opt_gram", maxg);
  w.gram2 = ws->get<float>("opt_gram2", maxg);
  w.poly = ws->get<float>("opt_poly", maxg);
  w.fs = ws->get<float>("opt_fs", maxside);
  w.part = ws->get<double>("opt_part", maxparts);
  w.scal = ws->get<double>("opt_scal", 8);
  w.vec = ws->get<double>("opt_vec", maxside);
  w.vec2 = ws->get<double>("opt_vec2", maxside);
  for (OptTensor& t : ts) {
    if (t.h.kind == GN_OPT_ADAMW) adamw_tensor(t, st);
    else if (t.h.kind == GN_OPT_MUON) muon_tensor(t, w, st, ws);
    else sinkhorn_tensor(t, w, st);
  }
  GN_HIP(hipGetLastError());
}

}  // namespace gn
