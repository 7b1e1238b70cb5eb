// gn_elementwise.hip - kernels behind the kernels.Backend primitives:
// element-wise ops, reductions, row softmax/RMSNorm, the lightning-indexer
// scores, top-k selection and the attention row passes used by the
// single-(batch, head) attention entry points.
//
// Transcendentals follow kernels/scalar/elementwise.go: evaluated in float64
// and rounded to float32.  Reductions accumulate in float64.
#include "gn_kernels.h"
#include "gn_prims.h"

namespace gn {

// ---------------------------------------------------------------------------
// Element-wise (kernels/scalar/elementwise.go)
// ---------------------------------------------------------------------------
__device__ __forceinline__ float clamp_gate(float v, float c, float* mask) {
  if (c > 0.f && v >= c) { *mask = 0.f; return c; }
  *mask = 1.f;
  return v;
}
__device__ __forceinline__ float clamp_up(float v, float c, float* mask) {
  if (c > 0.f) {
    if (v > c) { *mask = 0.f; return c; }
    if (v < -c) { *mask = 0.f; return -c; }
  }
  *mask = 1.f;
  return v;
}

__global__ void ew_binary_kernel(float* __restrict__ d, const float* l, const float* r, int64_t n,
                                 int op, float f) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    float a = l[i], b = r ? r[i] : 0.f, o;
    switch (op) {
      case EW_ADD: o = a + b; break;
      case EW_SUB: o = a - b; break;
      case EW_MUL: o = a * b; break;
      case EW_DIV: o = a / b; break;
      case EW_SCALE: o = a * f; break;
      case EW_ADD_SCALED: o = a + f * b; break;
      case EW_NEG: o = -a; break;
      case EW_ABS: o = a < 0.f ? -a : a; break;
      case EW_SQUARE: o = a * a; break;
      case EW_RELU2: { float t = a < 0.f ? 0.f : a; o = t * t; break; }
      case EW_EXP: o = (float)exp((double)a); break;
      case EW_SIGMOID: o = (float)(1.0 / (1.0 + exp(-(double)a))); break;
      case EW_TANH: o = (float)tanh((double)a); break;
      case EW_RSQRT: o = (float)(1.0 / sqrt((double)a)); break;
      case EW_SWIGLU: {
        float m;
        float g = clamp_gate(a, f, &m), u = clamp_up(b, f, &m);
        float s = (float)(1.0 / (1.0 + exp(-(double)g)));
        o = g * s * u;
        break;
      }
      default: o = 0.f;
    }
    d[i] = o;
  }
}

__global__ void swiglu_backward_kernel(float* dg, float* du, const float* gate, const float* up,
                                       const float* dout, float clamp, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    float gm, um;
    float g = clamp_gate(gate[i], clamp, &gm), u = clamp_up(up[i], clamp, &um);
    float s = (float)(1.0 / (1.0 + exp(-(double)g)));
    float silu = g * s;
    float sg = s * (1.f + g * (1.f - s));
    float d = dout[i];
    dg[i] = d * u * sg * gm;
    du[i] = d * silu * um;
  }
}

static unsigned ew_blocks(int64_t n) {
  return (unsigned)std::min<int64_t>(std::max<int64_t>(ceil_div(n, 256), 1), 65536);
}

void launch_elementwise(float* d, const float* l, const float* r, int64_t n, int op, float f,
                        hipStream_t st) {
  if (n <= 0) return;
  hipLaunchKernelGGL(ew_binary_kernel, dim3(ew_blocks(n)), dim3(256), 0, st, d, l, r, n, op, f);
  GN_HIP(hipGetLastError());
}
void launch_swiglu_backward(float* dg, float* du, const float* g, const float* u, const float* d,
                            float clamp, int64_t n, hipStream_t st) {
  if (n <= 0) return;
  hipLaunchKernelGGL(swiglu_backward_kernel, dim3(ew_blocks(n)), dim3(256), 0, st, dg, du, g, u,
                     d, clamp, n);
  GN_HIP(hipGetLastError());
}

// ---------------------------------------------------------------------------
// Reductions (kernels/scalar/reduce.go): one block of 1024 threads.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(1024) void reduce_kernel(const float* __restrict__ v, int64_t n,
                                                      int op, float* out_f, int64_t* out_i,
                                                      const float* __restrict__ w) {
  __shared__ double sd[16];
  __shared__ float sv[16];
  __shared__ int64_t si[16];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  if (op == RED_SUM || op == RED_DOT) {
    double acc = 0;
    for (int64_t i = tid; i < n; i += blockDim.x)
      acc += op == RED_DOT ? (double)v[i] * (double)w[i] : (double)v[i];
    acc = block_sum<double>(acc, sd);
    if (tid == 0) *out_f = (float)acc;
    return;
  }
  // max / argmax: first index of the largest value
  float best = -INFINITY;
  int64_t bi = -1;
  for (int64_t i = tid; i < n; i += blockDim.x) {
    float x = v[i];
    if (bi < 0 || x > best) { best = x; bi = i; }
  }
  for (int o = 32; o > 0; o >>= 1) {
    float ob = __shfl_xor(best, o, 64);
    int64_t oi = __shfl_xor(bi, o, 64);
    if (oi >= 0 && (bi < 0 || ob > best || (ob == best && oi < bi))) { best = ob; bi = oi; }
  }
  if (lane == 0) { sv[wid] = best; si[wid] = bi; }
  __syncthreads();
  if (tid == 0) {
    for (int i = 1; i < (int)(blockDim.x >> 6); i++) {
      if (si[i] >= 0 && (bi < 0 || sv[i] > best || (sv[i] == best && si[i] < bi))) {
        best = sv[i]; bi = si[i];
      }
    }
    if (op == RED_MAX) *out_f = n > 0 ? best : 0.f;
    else *out_i = n > 0 ? bi : 0;
  }
}

void launch_reduce(const float* v, int64_t n, int op, float* out_f, int64_t* out_i,
                   const float* w, hipStream_t st) {
  hipLaunchKernelGGL(reduce_kernel, dim3(1), dim3(1024), 0, st, v, n, op, out_f, out_i, w);
  GN_HIP(hipGetLastError());
}

// ---------------------------------------------------------------------------
// Rows (kernels/scalar/norm.go): one block per row.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void softmax_rows_kernel(float* __restrict__ d,
                                                           const float* __restrict__ s,
                                                           int64_t cols) {
  __shared__ float sf[4];
  __shared__ double sd[4];
  const float* src = s + blockIdx.x * cols;
  float* dst = d + blockIdx.x * cols;
  float m = -INFINITY;
  for (int64_t c = threadIdx.x; c < cols; c += blockDim.x) m = fmaxf(m, src[c]);
  m = block_max(m, sf);
  double tot = 0;
  for (int64_t c = threadIdx.x; c < cols; c += blockDim.x) {
    double e = exp((double)(src[c] - m));
    dst[c] = (float)e;
    tot += e;
  }
  tot = block_sum<double>(tot, sd);
  float inv = (float)(1.0 / tot);
  for (int64_t c = threadIdx.x; c < cols; c += blockDim.x) dst[c] = dst[c] * inv;
}

__global__ __launch_bounds__(256) void rmsnorm_rows_prim_kernel(float* __restrict__ d,
                                                                const float* __restrict__ s,
                                                                int64_t cols, float eps) {
  __shared__ double sd[4];
  const float* src = s + blockIdx.x * cols;
  float* dst = d + blockIdx.x * cols;
  double ss = 0;
  for (int64_t c = threadIdx.x; c < cols; c += blockDim.x) ss += (double)src[c] * (double)src[c];
  ss = block_sum<double>(ss, sd);
  float ms = (float)(ss / (double)cols);
  float inv = (float)(1.0 / sqrt((double)ms + (double)eps));
  for (int64_t c = threadIdx.x; c < cols; c += blockDim.x) dst[c] = src[c] * inv;
}

void launch_softmax_rows(float* d, const float* s, int64_t rows, int64_t cols, hipStream_t st) {
  if (rows <= 0 || cols <= 0) return;
  hipLaunchKernelGGL(softmax_rows_kernel, dim3((unsigned)rows), dim3(256), 0, st, d, s, cols);
  GN_HIP(hipGetLastError());
}
void launch_rmsnorm_rows_prim(float* d, const float* s, int64_t rows, int64_t cols, float eps,
                              hipStream_t st) {
  if (rows <= 0 || cols <= 0) return;
  hipLaunchKernelGGL(rmsnorm_rows_prim_kernel, dim3((unsigned)rows), dim3(256), 0, st, d, s, cols,
                     eps);
  GN_HIP(hipGetLastError());
}

// ---------------------------------------------------------------------------
// Indexer (kernels/scalar/indexer.go)
// ---------------------------------------------------------------------------
__global__ void indexer_scores_kernel(float* __restrict__ d, const float* __restrict__ q,
                                      const float* __restrict__ k, const float* __restrict__ w,
                                      int64_t rows, int64_t blocks, int64_t heads, int64_t dim) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= rows * blocks) return;
  int64_t r = i / blocks, b = i % blocks;
  float total = 0.f;
  for (int64_t h = 0; h < heads; h++) {
    const float* qh = q + (r * heads + h) * dim;
    const float* kh = k + (b * heads + h) * dim;
    float dot = 0.f;
    for (int64_t e = 0; e < dim; e++) dot += qh[e] * kh[e];
    if (dot > 0.f) total += w[h] * dot;
  }
  d[i] = total;
}
__global__ void indexer_block_max_kernel(float* __restrict__ d, const float* __restrict__ s,
                                         int64_t rows, int64_t blocks, int64_t group) {
  int64_t groups = (blocks + group - 1) / group;
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= rows * groups) return;
  int64_t r = i / groups, g = i % groups;
  int64_t s0 = g * group, e = min(s0 + group, blocks);
  float m = -INFINITY;
  for (int64_t j = s0; j < e; j++) m = fmaxf(m, s[r * blocks + j]);
  d[i] = m;
}
void launch_indexer_scores(float* d, const float* q, const float* k, const float* w, int64_t rows,
                           int64_t blocks, int64_t heads, int64_t dim, hipStream_t st) {
  int64_t n = rows * blocks;
  if (n <= 0) return;
  hipLaunchKernelGGL(indexer_scores_kernel, dim3((unsigned)ceil_div(n, 256)), dim3(256), 0, st, d,
                     q, k, w, rows, blocks, heads, dim);
  GN_HIP(hipGetLastError());
}
void launch_indexer_block_max(float* d, const float* s, int64_t rows, int64_t blocks,
                              int64_t group, hipStream_t st) {
  if (group < 1) group = 1;
  int64_t n = rows * ((blocks + group - 1) / group);
  if (n <= 0) return;
  hipLaunchKernelGGL(indexer_block_max_kernel, dim3((unsigned)ceil_div(n, 256)), dim3(256), 0, st,
                     d, s, rows, blocks, group);
  GN_HIP(hipGetLastError());
}

// ---------------------------------------------------------------------------
// Top-k (kernels/scalar/moe.go:8-50): per row, k rounds of "largest remaining,
// ties to the smaller index"; one block per row.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void topk_rows_kernel(int32_t* __restrict__ out,
                                                        const float* __restrict__ scores,
                                                        const float* __restrict__ bias,
                                                        int64_t count, int64_t k,
                                                        uint8_t* __restrict__ taken_all) {
  __shared__ float sv[4];
  __shared__ int64_t si[4];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const float* row = scores + blockIdx.x * count;
  uint8_t* taken = taken_all + blockIdx.x * count;
  for (int64_t c = tid; c < count; c += blockDim.x) taken[c] = 0;
  __syncthreads();
  const int64_t limit = k < count ? k : count;
  for (int64_t slot = 0; slot < limit; slot++) {
    float best = -INFINITY;
    int64_t bi = -1;
    for (int64_t c = tid; c < count; c += blockDim.x) {
      float x = taken[c] ? -INFINITY : row[c] + (bias ? bias[c] : 0.f);
      if (bi < 0 || x > best) { best = x; bi = c; }
    }
    for (int o = 32; o > 0; o >>= 1) {
      float ob = __shfl_xor(best, o, 64);
      int64_t oi = __shfl_xor(bi, o, 64);
      if (oi >= 0 && (bi < 0 || ob > best || (ob == best && oi < bi))) { best = ob; bi = oi; }
    }
    if (lane == 0) { sv[wid] = best; si[wid] = bi; }
    __syncthreads();
    if (tid == 0) {
      for (int i = 1; i < 4; i++)
        if (si[i] >= 0 && (bi < 0 || sv[i] > best || (sv[i] == best && si[i] < bi))) {
          best = sv[i]; bi = si[i];
        }
      // The reference masks a chosen entry with -Inf and rescans from index 0,
      // so once only -Inf remain the scan returns index 0 again.
      if (best == -INFINITY) bi = 0;
      out[blockIdx.x * k + slot] = (int32_t)bi;
      taken[bi] = 1;
    }
    __syncthreads();
  }
}
void launch_topk_rows(int32_t* out, const float* scores, const float* bias, int64_t rows,
                      int64_t count, int64_t k, uint8_t* taken, hipStream_t st) {
  if (rows <= 0 || count <= 0 || k <= 0) return;
  hipLaunchKernelGGL(topk_rows_kernel, dim3((unsigned)rows), dim3(256), 0, st, out, scores, bias,
                     count, k, taken);
  GN_HIP(hipGetLastError());
}

__global__ void gather_weights_kernel(float* __restrict__ w, const float* __restrict__ probs,
                                      const int32_t* __restrict__ sel, int64_t rows,
                                      int64_t experts, int64_t k, int64_t limit) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= rows * limit) return;
  int64_t r = i / limit, s = i % limit;
  w[r * k + s] = probs[r * experts + sel[r * k + s]];
}
void launch_gather_weights(float* w, const float* probs, const int32_t* sel, int64_t rows,
                           int64_t experts, int64_t k, hipStream_t st) {
  int64_t limit = k < experts ? k : experts;
  int64_t n = rows * limit;
  if (n <= 0) return;
  hipLaunchKernelGGL(gather_weights_kernel, dim3((unsigned)ceil_div(n, 256)), dim3(256), 0, st, w,
                     probs, sel, rows, experts, k, limit);
  GN_HIP(hipGetLastError());
}

// ---------------------------------------------------------------------------
// Attention row passes for the single-(batch, head) entry points
// (kernels/scalar/attention.go).  Scores S [qlen, ncols] come from the GEMM.
// ---------------------------------------------------------------------------
// Segment of query position qpos as applyAttentionMask tracks it
// (kernels/scalar/attention.go:211-216): the last in-range query's segment
// carries over, starting from 0.
__device__ __forceinline__ int32_t query_segment(const int32_t* seg, int64_t nseg, int64_t qpos,
                                                 int64_t offset) {
  if (!seg) return 0;
  if (qpos < nseg) return seg[qpos];
  return offset < nseg ? seg[nseg - 1] : 0;
}

// Forward row pass: mask, max (masked scores included, as backend.Max sees
// them), exp, float64 total; writes normalized (mode 0) or unnormalized
// (mode 1, split shard) probabilities in place, plus lse / max / sum.
__global__ __launch_bounds__(256) void attn_row_fwd_kernel(
    float* __restrict__ S, int64_t ncols, int64_t kstart, int64_t qlen, int64_t offset,
    int64_t window, const int32_t* __restrict__ seg, int64_t nseg, int mode,
    float* __restrict__ lse, float* __restrict__ mx_out, float* __restrict__ sum_out) {
  __shared__ float sf[4];
  __shared__ double sd[4];
  const int64_t qi = blockIdx.x;
  const int64_t qpos = offset + qi;
  float* row = S + qi * ncols;
  const int32_t qseg = query_segment(seg, nseg, qpos, offset);
  float m = -INFINITY;
  for (int64_t c = threadIdx.x; c < ncols; c += blockDim.x) {
    int64_t kj = kstart + c;
    bool masked = kj > qpos || (window >= 0 && qpos - kj > window);
    if (!masked && seg && kj < nseg) {
      if (mode == 0) masked = seg[kj] != qseg;
      else masked = qpos < nseg && seg[kj] != seg[qpos];
    }
    float s = masked ? -1e30f : row[c];
    row[c] = s;
    m = fmaxf(m, s);
  }
  m = block_max(m, sf);
  double tot = 0;
  for (int64_t c = threadIdx.x; c < ncols; c += blockDim.x) {
    double e = exp((double)(row[c] - m));
    row[c] = (float)e;
    tot += e;
  }
  tot = block_sum<double>(tot, sd);
  if (mode == 0) {
    float inv = (float)(1.0 / tot);
    for (int64_t c = threadIdx.x; c < ncols; c += blockDim.x) row[c] = row[c] * inv;
    if (threadIdx.x == 0 && lse) lse[qi] = m + (float)log(tot);
  } else if (threadIdx.x == 0) {
    mx_out[qi] = ncols > 0 ? m : -INFINITY;
    sum_out[qi] = (float)tot;
  }
}

// Backward row pass: P = exp(S - lse) with masked entries 0; dS = P (dP - rd),
// rd = row_correction or sum_j dP P in float64 (kernels/scalar/attention.go:
// 155-192).  P overwrites S and dS overwrites dP.
__global__ __launch_bounds__(256) void attn_row_bwd_kernel(
    float* __restrict__ S, float* __restrict__ dP, int64_t klen, int64_t offset, int64_t window,
    const int32_t* __restrict__ seg, int64_t nseg, const float* __restrict__ lse,
    const float* __restrict__ corr) {
  __shared__ double sd[4];
  const int64_t qi = blockIdx.x;
  const int64_t qpos = offset + qi;
  float* srow = S + qi * klen;
  float* drow = dP + qi * klen;
  const int32_t qseg = query_segment(seg, nseg, qpos, offset);
  const float l = lse[qi];
  double rd = 0;
  for (int64_t c = threadIdx.x; c < klen; c += blockDim.x) {
    bool masked = c > qpos || (window >= 0 && qpos - c > window);
    if (!masked && seg && c < nseg) masked = seg[c] != qseg;
    float s = masked ? -1e30f : srow[c];
    float p = s <= -1e30f ? 0.f : (float)exp((double)(s - l));
    srow[c] = p;
    rd += (double)drow[c] * (double)p;
  }
  rd = block_sum<double>(rd, sd);
  if (corr) rd = (double)corr[qi];
  for (int64_t c = threadIdx.x; c < klen; c += blockDim.x)
    drow[c] = (float)((double)srow[c] * ((double)drow[c] - rd));
}

void launch_attn_row_fwd(float* S, int64_t ncols, int64_t kstart, int64_t qlen, int64_t offset,
                         int64_t window, const int32_t* seg, int64_t nseg, int mode, float* lse,
                         float* mx, float* sum, hipStream_t st) {
  if (qlen <= 0) return;
  hipLaunchKernelGGL(attn_row_fwd_kernel, dim3((unsigned)qlen), dim3(256), 0, st, S, ncols,
                     kstart, qlen, offset, window, seg, nseg, mode, lse, mx, sum);
  GN_HIP(hipGetLastError());
}
void launch_attn_row_bwd(float* S, float* dP, int64_t qlen, int64_t klen, int64_t offset,
                         int64_t window, const int32_t* seg, int64_t nseg, const float* lse,
                         const float* corr, hipStream_t st) {
  if (qlen <= 0) return;
  hipLaunchKernelGGL(attn_row_bwd_kernel, dim3((unsigned)qlen), dim3(256), 0, st, S, dP, klen,
                     offset, window, seg, nseg, lse, corr);
  GN_HIP(hipGetLastError());
}

// AttentionCombine (kernels/scalar/attention.go:107-141) over `parts` shards
// given as device pointer arrays; one block per query row.
__global__ __launch_bounds__(128) void attn_combine_kernel(
    const float* const* __restrict__ accs, const float* const* __restrict__ mxs,
    const float* const* __restrict__ sums, int64_t parts, int64_t dim, float* __restrict__ out,
    float* __restrict__ lse) {
  const int64_t qi = blockIdx.x;
  float gm = -INFINITY;
  for (int64_t p = 0; p < parts; p++) gm = fmaxf(gm, mxs[p][qi]);
  double total = 0;
  for (int64_t p = 0; p < parts; p++) {
    float m = mxs[p][qi];
    float scale = m > -INFINITY ? (float)exp((double)(m - gm)) : 0.f;
    total += (double)sums[p][qi] * (double)scale;
  }
  float inv = total > 0 ? (float)(1.0 / total) : 1.f;
  for (int64_t d = threadIdx.x; d < dim; d += blockDim.x) {
    float o = 0.f;
    for (int64_t p = 0; p < parts; p++) {
      float m = mxs[p][qi];
      float scale = m > -INFINITY ? (float)exp((double)(m - gm)) : 0.f;
      o += accs[p][qi * dim + d] * scale;
    }
    out[qi * dim + d] = total > 0 ? o * inv : o;
  }
  if (threadIdx.x == 0 && lse) lse[qi] = gm + (float)log(total);
}
void launch_attn_combine(const float* const* accs, const float* const* mxs,
                         const float* const* sums, int64_t parts, int64_t qlen, int64_t dim,
                         float* out, float* lse, hipStream_t st) {
  if (qlen <= 0) return;
  hipLaunchKernelGGL(attn_combine_kernel, dim3((unsigned)qlen), dim3(128), 0, st, accs, mxs, sums,
                     parts, dim, out, lse);
  GN_HIP(hipGetLastError());
}

}  // namespace gn
