// gn_model.hip - fused row kernels of the dense transformer's forward and
// backward (model/transformer.go, model/attention.go, model/train.go,
// model/train_transformer.go).  Rows are tokens; one block per row unless
// noted.  Head dimension is 128 (every benchmark config).
#include "gn_model.h"

namespace gn {

typedef float v4f __attribute__((ext_vector_type(4)));

static constexpr int SMEAR_CH = 24;       // model/helpers.go:7


// Sum of a per-thread value over a 256-thread block (float).
__device__ __forceinline__ float bsum256(float v, float* sc) { return block_sum<float>(v, sc); }

// ---------------------------------------------------------------------------
// Embedding + RMSNorm + smear gate (model/transformer.go:255-301,
// model/train_transformer.go:73-87).  Writes raw (optional), embn, and for
// t >= 1 the smear sigmoid.  ids [B*T].
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void embed_norm_kernel(const int32_t* __restrict__ ids,
                                                         const float* __restrict__ wte, int C,
                                                         int T, const float* __restrict__ wsg,
                                                         float* __restrict__ raw,
                                                         float* __restrict__ embn,
                                                         float* __restrict__ smsig,
                                                         float* __restrict__ seedsig) {
  __shared__ float sc[4];
  const int64_t n = blockIdx.x;
  const int t = (int)(n % T);
  const float* src = wte + (int64_t)ids[n] * C;
  float ss = 0.f;
  for (int c = threadIdx.x; c < C; c += 256) {
    float v = src[c];
    if (raw) raw[n * C + c] = v;
    ss += v * v;
  }
  ss = bsum256(ss, sc);
  const float inv = 1.f / sqrtf(ss / (float)C + NORM_EPS);
  for (int c = threadIdx.x; c < C; c += 256) embn[n * C + c] = src[c] * inv;
  if ((t >= 1 && smsig) || (t == 0 && seedsig)) {
    // gate = sigmoid(embn[:24] . w) (smearGate Linear 24 -> 1); at t == 0 the
    // seed gate of a forward that continues a cached prefix (smearSeed)
    float p = 0.f;
    if (threadIdx.x < SMEAR_CH) p = src[threadIdx.x] * inv * wsg[threadIdx.x];
    p = warp_sum(threadIdx.x < 64 ? p : 0.f);
    if (threadIdx.x == 0) {
      if (t >= 1) smsig[(n / T) * (T - 1) + t - 1] = sigmoidf_(p);
      else seedsig[n / T] = sigmoidf_(p);
    }
  }
}

// x[t] = embn[t] + lambda * smsig[t-1] * embn[t-1] (helpers.go:35-48; reads the
// pre-smear embedding of the previous row); with seed_prev, row 0 of each
// sequence adds lambda * seedsig * seed_prev (smearSeed, helpers.go:53-67:
// the previous token's stored embedding of a cached prefix).
__global__ void smear_apply_kernel(const float* __restrict__ embn, const float* __restrict__ smsig,
                                   const float* __restrict__ lam, float* __restrict__ x, int C,
                                   int T, int64_t total, const float* __restrict__ seedsig,
                                   const float* __restrict__ seed_prev) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  int64_t n = i / C;
  int t = (int)(n % T);
  float v = embn[i];
  if (t >= 1) {
    float g = smsig[(n / T) * (T - 1) + t - 1] * lam[0];
    v += g * embn[i - C];
  } else if (seed_prev) {
    const int64_t b = n / T;
    float g = seedsig[b] * lam[0];
    v += g * seed_prev[b * C + (i - n * C)];
  }
  x[i] = v;
}

void launch_embed_smear(const int32_t* ids, const float* wte, const float* wsg, const float* lam,
                        int B, int T, int C, float* raw, float* embn, float* smsig, float* x,
                        hipStream_t st, const float* seed_prev, float* seedsig) {
  GN_CHECK(!seed_prev || seedsig, "embed_smear: a seed needs its gate buffer");
  int64_t N = (int64_t)B * T;
  hipLaunchKernelGGL(embed_norm_kernel, dim3((unsigned)N), dim3(256), 0, st, ids, wte, C, T, wsg,
                     raw, embn, T > 1 ? smsig : nullptr, seed_prev ? seedsig : nullptr);
  GN_HIP(hipGetLastError());
  int64_t tot = N * C;
  hipLaunchKernelGGL(smear_apply_kernel, dim3((unsigned)ceil_div(tot, 256)), dim3(256), 0, st,
                     embn, smsig, lam, x, C, T, tot, seedsig, seed_prev);
  GN_HIP(hipGetLastError());
}

// Decode step embedding (transformer.go:276-300 with T == 1): embn =
// norm(wte[tok]); x = embn + lambda*sigmoid(embn[:24].w)*prev; prev = embn.
// tok [rows] is the column fed; with ovr (nullable) a row whose ovr entry
// is >= 0 is fed that token instead, and it is written back to tok (the
// step's later kernels read the fed token).
__global__ __launch_bounds__(256) void embed_decode_kernel(int32_t* tok,
                                                           const int32_t* __restrict__ ovr,
                                                           const float* __restrict__ wte, int C,
                                                           const float* __restrict__ wsg,
                                                           const float* __restrict__ lam,
                                                           float* __restrict__ prev,
                                                           float* __restrict__ x,
                                                           float* __restrict__ x0) {
  __shared__ float sc[4];
  __shared__ float gate_s;
  const int64_t r = blockIdx.x;
  int32_t t = tok[r];
  if (ovr && ovr[r] >= 0) t = ovr[r];
  const float* src = wte + (int64_t)t * C;
  float ss = 0.f;
  for (int c = threadIdx.x; c < C; c += 256) ss += src[c] * src[c];
  ss = bsum256(ss, sc);
  const float inv = 1.f / sqrtf(ss / (float)C + NORM_EPS);
  if (threadIdx.x < 64) {
    float p = threadIdx.x < SMEAR_CH ? src[threadIdx.x] * inv * wsg[threadIdx.x] : 0.f;
    p = warp_sum(p);
    if (threadIdx.x == 0) gate_s = sigmoidf_(p) * lam[0];
  }
  __syncthreads();  // every thread has read tok[r]
  if (ovr && threadIdx.x == 0) tok[r] = t;
  const float g = gate_s;
  for (int c = threadIdx.x; c < C; c += 256) {
    float e = src[c] * inv;
    float v = e + g * prev[r * C + c];
    prev[r * C + c] = e;
    x[r * C + c] = v;
    x0[r * C + c] = v;
  }
}
void launch_embed_decode(int32_t* tok, const float* wte, const float* wsg, const float* lam,
                         int rows, int C, float* prev, float* x, float* x0, hipStream_t st,
                         const int32_t* ovr) {
  hipLaunchKernelGGL(embed_decode_kernel, dim3(rows), dim3(256), 0, st, tok, ovr, wte, C, wsg,
                     lam, prev, x, x0);
  GN_HIP(hipGetLastError());
}

// embed_decode_kernel followed by layer 0's combineResidual + RMSNorm
// (resid_norm_kernel with no pending sum) in the same block: x0 = the
// smeared embedding v, x = lr[0] v + l0[0] v, h = norm(x).  Element k of a
// thread is column threadIdx.x + 256 k in both steps, as in the two kernels,
// so the sums and the results are the same bits.
template <int NE>
__global__ __launch_bounds__(256) void embed_decode_mix_kernel(
    int32_t* tok, const int32_t* __restrict__ ovr, const float* __restrict__ wte, int C,
    const float* __restrict__ wsg, const float* __restrict__ lam, const float* __restrict__ lr,
    const float* __restrict__ l0, float* __restrict__ prev, float* __restrict__ x,
    float* __restrict__ x0, float* __restrict__ h) {
  __shared__ float sc[4];
  __shared__ float gate_s;
  const int64_t r = blockIdx.x;
  int32_t t = tok[r];
  if (ovr && ovr[r] >= 0) t = ovr[r];
  const float* src = wte + (int64_t)t * C;
  float e[NE];
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < NE; k++) {
    const int c = threadIdx.x + 256 * k;
    e[k] = c < C ? src[c] : 0.f;
    if (c < C) ss += e[k] * e[k];
  }
  ss = bsum256(ss, sc);
  const float inv = 1.f / sqrtf(ss / (float)C + NORM_EPS);
  if (threadIdx.x < 64) {
    float p = threadIdx.x < SMEAR_CH ? src[threadIdx.x] * inv * wsg[threadIdx.x] : 0.f;
    p = warp_sum(p);
    if (threadIdx.x == 0) gate_s = sigmoidf_(p) * lam[0];
  }
  __syncthreads();  // every thread has read tok[r]; sc is free again
  if (ovr && threadIdx.x == 0) tok[r] = t;
  const float g = gate_s, a = lr[0], b = l0[0];
  float vals[NE];
  float ss2 = 0.f;
#pragma unroll
  for (int k = 0; k < NE; k++) {
    const int c = threadIdx.x + 256 * k;
    if (c >= C) continue;
    const int64_t i = r * C + c;
    const float en = e[k] * inv;
    const float v = en + g * prev[i];
    prev[i] = en;
    x0[i] = v;
    const float m = __fmaf_rn(a, v, b * v);  // resid_norm_kernel's mix of x = x0 = v
    vals[k] = m;
    ss2 += m * m;
  }
  ss2 = bsum256(ss2, sc);
  const float inv2 = 1.f / sqrtf(ss2 / (float)C + NORM_EPS);
#pragma unroll
  for (int k = 0; k < NE; k++) {
    const int c = threadIdx.x + 256 * k;
    if (c >= C) continue;
    x[r * C + c] = vals[k];
    h[r * C + c] = vals[k] * inv2;
  }
}

// Deferred split-K products: element i is the float64 sum of its partials
// in split order, rounded once (gemm_reduce_kernel's result).  The row
// kernels are latency-bound (one block per row, a few elements per
// thread), so a thread first issues the loads of all its elements'
// partials (a fixed, unrolled count) and sums them afterwards.
template <int NE>
struct PendingLoad {
  float v[NE][PENDING_MAX_SPLITS];
  // element e (index idx[e], valid[e]) of thread-local slot e
  __device__ __forceinline__ void load(const PendingSum& ps, const int64_t* idx, const bool* valid) {
#pragma unroll
    for (int e = 0; e < NE; e++)
#pragma unroll
      for (int z = 0; z < PENDING_MAX_SPLITS; z++)
        if (valid[e] && z < ps.splits) v[e][z] = ps.part[z * ps.stride + idx[e]];
  }
  __device__ __forceinline__ float sum(const PendingSum& ps, int e) const {
    double s = 0.0;
#pragma unroll
    for (int z = 0; z < PENDING_MAX_SPLITS; z++)
      if (z < ps.splits) s += (double)v[e][z];
    return (float)s;
  }
};

// ---------------------------------------------------------------------------
// combineResidual + RMSNorm (transformer.go:312,544-551; block.go:39):
// xb = lr*xin + l0*x0 ; h = norm(xb).  xb may alias xin.  With a deferred
// residual-add product pending on xin, xin stands for xin + sum.
// ---------------------------------------------------------------------------
template <int NE>
__global__ __launch_bounds__(256) void resid_norm_kernel(const float* xin, const float* __restrict__ x0,
                                                         const float* __restrict__ lr,
                                                         const float* __restrict__ l0, int layer,
                                                         int C, float* xb, float* __restrict__ h,
                                                         PendingSum pend, float* __restrict__ xs) {
  __shared__ float sc[4];
  const int64_t r = blockIdx.x;
  const float a = lr[layer], b = l0[layer];
  // element k of this thread: column threadIdx.x + 256k (C <= 256 * NE)
  int64_t idx[NE];
  bool ok[NE];
  float xi[NE], xz[NE];
#pragma unroll
  for (int k = 0; k < NE; k++) {
    const int c = threadIdx.x + 256 * k;
    ok[k] = c < C;
    idx[k] = r * C + c;
    if (ok[k]) {
      xi[k] = xin[idx[k]];
      xz[k] = x0[idx[k]];
    }
  }
  PendingLoad<NE> pl;
  if (pend.splits > 0) pl.load(pend, idx, ok);
  float vals[NE];
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < NE; k++) {
    if (!ok[k]) continue;
    const float x = pend.splits > 0 ? pl.sum(pend, k) + xi[k] : xi[k];
    if (xs) xs[idx[k]] = x;
    const float v = __fmaf_rn(a, x, b * xz[k]);  // one rounding order on every build
    vals[k] = v;
    ss += v * v;
  }
  ss = bsum256(ss, sc);
  const float inv = 1.f / sqrtf(ss / (float)C + NORM_EPS);
#pragma unroll
  for (int k = 0; k < NE; k++) {
    if (!ok[k]) continue;
    xb[idx[k]] = vals[k];
    h[idx[k]] = vals[k] * inv;
  }
}
// Elements per thread of a 256-thread row kernel over C columns.
#define GN_ROW_NE_DISPATCH(C, KERNEL_LAUNCH)                                        \
  do {                                                                              \
    GN_CHECK((C) >= 1 && (C) <= 2048, "embedding width above 2048 is not supported"); \
    if ((C) <= 768) { constexpr int NE = 3; KERNEL_LAUNCH; }                        \
    else if ((C) <= 1024) { constexpr int NE = 4; KERNEL_LAUNCH; }                  \
    else if ((C) <= 1280) { constexpr int NE = 5; KERNEL_LAUNCH; }                  \
    else if ((C) <= 1536) { constexpr int NE = 6; KERNEL_LAUNCH; }                  \
    else { constexpr int NE = 8; KERNEL_LAUNCH; }                                   \
  } while (0)
void launch_resid_norm(const float* xin, const float* x0, const float* lr, const float* l0,
                       int layer, int64_t rows, int C, float* xb, float* h, hipStream_t st,
                       const PendingSum& pend, float* xs) {
  GN_CHECK(pend.splits == 0 || (pend.stride == rows * (int64_t)C && pend.splits <= PENDING_MAX_SPLITS),
           "resid_norm: pending sum shape");
  GN_ROW_NE_DISPATCH(C, hipLaunchKernelGGL(resid_norm_kernel<NE>, dim3((unsigned)rows), dim3(256),
                                           0, st, xin, x0, lr, l0, layer, C, xb, h, pend, xs));
  GN_HIP(hipGetLastError());
}

void launch_embed_decode_mix(int32_t* tok, const float* wte, const float* wsg, const float* lam,
                             const float* lr, const float* l0, int rows, int C, float* prev,
                             float* x, float* x0, float* h, hipStream_t st, const int32_t* ovr) {
  GN_ROW_NE_DISPATCH(C, hipLaunchKernelGGL(embed_decode_mix_kernel<NE>, dim3((unsigned)rows),
                                           dim3(256), 0, st, tok, ovr, wte, C, wsg, lam, lr, l0,
                                           prev, x, x0, h));
  GN_HIP(hipGetLastError());
}

// y = norm(x - lam*back) (or norm(x) when back is null); pre receives x - lam*back.
// With a deferred residual-add product pending on x, x first becomes
// x + sum (written back).
template <int NE>
__global__ __launch_bounds__(256) void norm_rows_kernel(float* x, const float* __restrict__ back,
                                                        const float* __restrict__ lam, int C,
                                                        float* __restrict__ pre,
                                                        float* __restrict__ y, PendingSum pend) {
  __shared__ float sc[4];
  const int64_t r = blockIdx.x;
  const float nl = back ? -lam[0] : 0.f;
  int64_t idx[NE];
  bool ok[NE];
  float xv[NE], bv[NE];
#pragma unroll
  for (int k = 0; k < NE; k++) {
    const int c = threadIdx.x + 256 * k;
    ok[k] = c < C;
    idx[k] = r * C + c;
    if (ok[k]) {
      xv[k] = x[idx[k]];
      bv[k] = back ? back[idx[k]] : 0.f;
    }
  }
  PendingLoad<NE> pl;
  if (pend.splits > 0) pl.load(pend, idx, ok);
  float vals[NE];
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < NE; k++) {
    if (!ok[k]) continue;
    float v = xv[k];
    if (pend.splits > 0) {
      v = pl.sum(pend, k) + v;
      x[idx[k]] = v;
    }
    if (back) v = v + nl * bv[k];
    vals[k] = v;
    ss += v * v;
  }
  ss = bsum256(ss, sc);
  const float inv = 1.f / sqrtf(ss / (float)C + NORM_EPS);
#pragma unroll
  for (int k = 0; k < NE; k++) {
    if (!ok[k]) continue;
    if (pre) pre[idx[k]] = vals[k];
    y[idx[k]] = vals[k] * inv;
  }
}
void launch_norm_rows(float* x, const float* back, const float* lam, int64_t rows, int C,
                      float* pre, float* y, hipStream_t st, const PendingSum& pend) {
  GN_CHECK(pend.splits == 0 || (pend.stride == rows * (int64_t)C && pend.splits <= PENDING_MAX_SPLITS),
           "norm_rows: pending sum shape");
  GN_ROW_NE_DISPATCH(C, hipLaunchKernelGGL(norm_rows_kernel<NE>, dim3((unsigned)rows), dim3(256),
                                           0, st, x, back, lam, C, pre, y, pend));
  GN_HIP(hipGetLastError());
}

// ---------------------------------------------------------------------------
// Q/K/V post-processing (attention.go:240-256): VE gate on v, RoPE on the
// trailing R dims of q and k, then 1.2 * RMSNorm per head.  One block of 256
// threads per token; each wave handles whole heads (D = 128: two values per
// lane).  Inputs: qkv [N, (Hq+2Hkv)*D] (GEMM output), h [N, C] (VE gate
// reads h[:12]); token n sits at position pos0 + n % T.  The key and value
// of token n land in cache row (n / T) at that position when a cache is
// given (decode: T == 1, one row per token; prefill: one row per prompt).
// ---------------------------------------------------------------------------
// The kernel is latency-bound (one block per token, ~1-2 K floats each), so
// every load that does not depend on another -- the q/k/v row (or its
// split-K partials), the VE gate inputs, the token's VE row and the RoPE
// table entries of this lane's dims -- is issued before the first wait.
// PEND: the q/k/v rows arrive as deferred split-K partials (decode); the
// other instance (prefill, training) holds no partials, a third of the
// registers, so twice the blocks per CU keep loads in flight.
template <bool PEND>
__global__ __launch_bounds__(256) void qkv_post_kernel(QkvPostArgs a) {
  constexpr int D = 128;
  __shared__ __attribute__((aligned(16))) float row[16 * D];  // up to 16 heads of q/k/v
  __shared__ float gate[8];
  const int64_t n = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int H = a.Hq + 2 * a.Hkv;
  const int n4 = H * D / 4;  // <= 512 float4 per token: at most 2 per thread
  const int t = (int)(n % a.T);
  const int pos = (a.pos_dev ? *a.pos_dev : a.pos0) + t;
  // q/k/v row: float4 e of this thread is element (tid + 256e) of the row
  constexpr bool pend = PEND;
  v4f rv[2];
  v4f pv[2][PEND ? PENDING_MAX_SPLITS : 1];
#pragma unroll
  for (int e = 0; e < 2; e++) {
    const int i = tid + 256 * e;
    if (i >= n4) continue;
    if constexpr (pend) {
      const v4f* P = reinterpret_cast<const v4f*>(a.qkv_sum.part) + n * n4 + i;
      const int64_t zs = a.qkv_sum.stride / 4;
#pragma unroll
      for (int z = 0; z < PENDING_MAX_SPLITS; z++)
        if (z < a.qkv_sum.splits) pv[e][z] = P[z * zs];
    } else {
      rv[e] = reinterpret_cast<const v4f*>(a.qkv)[n * n4 + i];
    }
  }
  // VE inputs: h[:12] and the gate weights (wave 0), the token's VE row
  float hv = 0.f, wv[8];
  if (a.ve && wid == 0 && lane < VE_CH) {
    hv = a.h[n * a.C + lane];
#pragma unroll
    for (int hk = 0; hk < 8; hk++)
      if (hk < a.Hkv) wv[hk] = a.wve[hk * VE_CH + lane];
  }
  float vev[4];
  if (a.ve) {
    const float* ver = a.ve + (int64_t)a.ids[n] * a.Hkv * D;
#pragma unroll
    for (int e = 0; e < 4; e++)
      if (tid + 256 * e < a.Hkv * D) vev[e] = ver[tid + 256 * e];
  }
  // RoPE table entries of this lane's two dims (the same for every head)
  const int half = a.R / 2, off = D - a.R;
  float cv[2] = {0.f, 0.f}, sv[2] = {0.f, 0.f};
#pragma unroll
  for (int e = 0; e < 2; e++) {
    const int d = lane + 64 * e;
    if (d >= off) {
      const int j = d - off, jj = j < half ? j : j - half;
      cv[e] = a.cosT[(int64_t)pos * half + jj];
      sv[e] = a.sinT[(int64_t)pos * half + jj];
    }
  }
  // the row into LDS
#pragma unroll
  for (int e = 0; e < 2; e++) {
    const int i = tid + 256 * e;
    if (i >= n4) continue;
    v4f v = rv[e];
    if constexpr (pend) {
#pragma unroll
      for (int c = 0; c < 4; c++) {
        double sum = 0.0;
#pragma unroll
        for (int z = 0; z < PENDING_MAX_SPLITS; z++)
          if (z < a.qkv_sum.splits) sum += (double)pv[e][z][c];
        v[c] = (float)sum;
      }
    }
    *reinterpret_cast<v4f*>(&row[4 * i]) = v;
  }
  if (a.ve && wid == 0) {
    // gate[hk] = 3 * sigmoid(h[:12] . wve[hk]) (attention.go:247-248)
    for (int hk = 0; hk < a.Hkv; hk++) {
      float p = lane < VE_CH ? hv * wv[hk] : 0.f;
      p = warp_sum(p);
      if (lane == 0) {
        float s = sigmoidf_(p);
        gate[hk] = s * VE_SCALE;
        if (a.vesig) a.vesig[n * a.Hkv + hk] = s;
      }
    }
  }
  __syncthreads();
  // v += gate * ve[id] (attention.go:392-405)
  if (a.ve) {
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const int i = tid + 256 * e;
      if (i < a.Hkv * D) row[(a.Hq + a.Hkv) * D + i] += gate[i / D] * vev[e];
    }
  }
  __syncthreads();
  // q and k heads: rotate, then 1.2 * RMSNorm over the head
  for (int hd = wid; hd < a.Hq + a.Hkv; hd += 4) {
    const float* x = row + hd * D;
    float y[2];
#pragma unroll
    for (int e = 0; e < 2; e++) {
      int d = lane + 64 * e;
      float v = x[d];
      if (d >= off) {
        int j = d - off;
        if (j < half) v = x[d] * cv[e] + x[d + half] * sv[e];
        else v = -x[d - half] * sv[e] + x[d] * cv[e];
      }
      y[e] = v;
    }
    float ss = warp_sum(y[0] * y[0] + y[1] * y[1]);
    const float inv = 1.f / sqrtf(ss / (float)D + NORM_EPS);
    const bool isq = hd < a.Hq;
    const int hh = isq ? hd : hd - a.Hq;
#pragma unroll
    for (int e = 0; e < 2; e++) {
      int d = lane + 64 * e;
      float o = y[e] * inv * QK_SCALE;
      if (isq) {
        if (a.qrot) a.qrot[(n * a.Hq + hh) * D + d] = y[e];
        a.qn[(n * a.Hq + hh) * D + d] = o;
      } else {
        if (a.krot) a.krot[(n * a.Hkv + hh) * D + d] = y[e];
        if (a.kn) a.kn[(n * a.Hkv + hh) * D + d] = o;
        if (a.kcache) {
          int64_t crow = (n / a.T) * a.rows_per_seq;
          a.kcache[((crow * a.Hkv + hh) * a.maxSeq + pos) * D + d] = o;
        }
      }
    }
  }
  // v heads
  for (int i = tid; i < a.Hkv * D; i += 256) {
    float v = row[(a.Hq + a.Hkv) * D + i];
    int hh = i / D, d = i % D;
    if (a.vout) a.vout[n * a.Hkv * D + i] = v;
    if (a.vcache) {
      int64_t crow = (n / a.T) * a.rows_per_seq;
      a.vcache[((crow * a.Hkv + hh) * a.maxSeq + pos) * D + d] = v;
    }
  }
}
void launch_qkv_post(const QkvPostArgs& a, int64_t rows, hipStream_t st) {
  GN_CHECK(a.Hq + 2 * a.Hkv <= 16, "qkv_post: at most 16 heads");
  GN_CHECK(((uintptr_t)a.qkv & 15) == 0 && ((uintptr_t)a.qkv_sum.part & 15) == 0,
           "qkv_post: q/k/v rows must be 16-byte aligned");
  GN_CHECK(a.Hkv <= 8, "qkv_post: at most 8 kv heads");
  GN_CHECK(a.R % 2 == 0 && a.R <= 128, "qkv_post: rotary dims must be even and <= 128");
  GN_CHECK(a.qkv_sum.splits == 0 ||
               (a.qkv_sum.stride == rows * (int64_t)(a.Hq + 2 * a.Hkv) * 128 &&
                a.qkv_sum.splits <= PENDING_MAX_SPLITS),
           "qkv_post: pending sum shape");
  if (a.qkv_sum.splits > 0)
    hipLaunchKernelGGL(qkv_post_kernel<true>, dim3((unsigned)rows), dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL(qkv_post_kernel<false>, dim3((unsigned)rows), dim3(256), 0, st, a);
  GN_HIP(hipGetLastError());
}

// Copies a prefill KV cache [G][Hkv][P][D] (per layer) into the decode cache
// [G*S][Hkv][maxSeq][D] (model/kvcache.go:383-448, PrefillFrom), and the
// prefill's last embedding into every row's previous-embedding slot.
__global__ void replicate_kv_kernel(const float* __restrict__ src, float* __restrict__ dst, int G,
                                    int S, int Hkv, int P, int maxSrc, int maxDst, int64_t total) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;  // total = G*S*Hkv*P*D
  constexpr int D = 128;
  int d = (int)(i % D);
  int64_t r = i / D;
  int p = (int)(r % P);
  r /= P;
  int hk = (int)(r % Hkv);
  int64_t row = r / Hkv;
  int g = (int)(row / S);
  dst[((row * Hkv + hk) * maxDst + p) * D + d] = src[(((int64_t)g * Hkv + hk) * maxSrc + p) * D + d];
}
void launch_replicate_kv(const float* src, float* dst, int G, int S, int Hkv, int P, int maxSrc,
                         int maxDst, hipStream_t st) {
  int64_t total = (int64_t)G * S * Hkv * P * 128;
  if (total == 0) return;
  hipLaunchKernelGGL(replicate_kv_kernel, dim3((unsigned)ceil_div(total, 256)), dim3(256), 0, st,
                     src, dst, G, S, Hkv, P, maxSrc, maxDst, total);
  GN_HIP(hipGetLastError());
}

// Gathers row (g*T + T-1) of src [G*T, C] into rows [g*S, (g+1)*S) of dst.
__global__ void expand_last_rows_kernel(const float* __restrict__ src, float* __restrict__ dst,
                                        int G, int T, int S, int C) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  int64_t total = (int64_t)G * S * C;
  if (i >= total) return;
  int c = (int)(i % C);
  int64_t row = i / C;
  int g = (int)(row / S);
  dst[i] = src[((int64_t)g * T + T - 1) * C + c];
}
// One grid row per descriptor; each row's floats are split into chunks of
// COPY_CHUNK spread over the blocks of the grid row, 16-byte moves where the
// addresses, pitches and count allow it.
constexpr int COPY_CHUNK = 4096;
__global__ __launch_bounds__(256) void copy_blocks_kernel(const CopyBlock* __restrict__ descs) {
  const CopyBlock d = descs[blockIdx.y];
  const int64_t chunks = (d.count + COPY_CHUNK - 1) / COPY_CHUNK;
  const int64_t work = chunks * d.outer * d.inner;
  const bool vec = ((reinterpret_cast<uintptr_t>(d.src) | reinterpret_cast<uintptr_t>(d.dst)) & 15) == 0 &&
                   ((d.count | d.s_outer | d.s_inner | d.d_outer | d.d_inner) & 3) == 0;
  for (int64_t w = blockIdx.x; w < work; w += gridDim.x) {
    const int64_t row = w / chunks, c0 = (w % chunks) * COPY_CHUNK;
    const int64_t o = row / d.inner, i = row % d.inner;
    const float* src = d.src + o * d.s_outer + i * d.s_inner + c0;
    float* dst = d.dst + o * d.d_outer + i * d.d_inner + c0;
    const int n = (int)min<int64_t>(COPY_CHUNK, d.count - c0);
    if (vec) {
      for (int k = threadIdx.x; k < n / 4; k += 256)
        reinterpret_cast<float4*>(dst)[k] = reinterpret_cast<const float4*>(src)[k];
    } else {
      for (int k = threadIdx.x; k < n; k += 256) dst[k] = src[k];
    }
  }
}

void launch_copy_blocks(const CopyBlock* descs, int n, hipStream_t st) {
  if (n <= 0) return;
  GN_CHECK(n <= 65535, "copy_blocks: too many descriptors");
  hipLaunchKernelGGL(copy_blocks_kernel, dim3(256, (unsigned)n), dim3(256), 0, st, descs);
  GN_HIP(hipGetLastError());
}

void launch_expand_last_rows(const float* src, float* dst, int G, int T, int S, int C,
                             hipStream_t st) {
  int64_t total = (int64_t)G * S * C;
  if (total == 0) return;
  hipLaunchKernelGGL(expand_last_rows_kernel, dim3((unsigned)ceil_div(total, 256)), dim3(256), 0,
                     st, src, dst, G, T, S, C);
  GN_HIP(hipGetLastError());
}

// ---------------------------------------------------------------------------
// PG loss rows (trainer/rl.go:22-56, tensors/loss.go:16-46,
// tensors/backward.go:108-116).  z [rows, V] holds the lm_head products y
// (row stride ldz); the logits are z = softcap15(y) (transformer.go:538-541,
// applied here on load rather than in the product's epilogue, so the
// product is a plain GEMM), and z is overwritten by dL/dy:
//   g = (softmax(z) - onehot(t)) * (adv/norm) * (1 - (z/15)^2),
// zero for ignored rows.  nll (0 for ignored) and the per-row loss term
// nll*adv/norm (float64) are written per row.  Chunk row r is batch row
// n = rowmap[row0 + r] (rowmap: the rows that have a target, in order) or
// n = row0 + r (rowmap null); targets, the advantage of sequence n / T and
// nll are indexed by n, loss_rows by row0 + r.
//
// When the row fits in registers (V a multiple of 4, at most 1024 * 4 * Q
// floats) one 1024-thread block holds it as Q float4 per thread: the logits
// are read once and the gradient written once (the maximum, the float64
// sum of exponentials and the gradient come from the registers); rows of
// 32,768 entries or more take softcap15_fast / exp_softcapped below.
// Otherwise the row is streamed three times (maximum, sum, gradient).
// ---------------------------------------------------------------------------
__device__ __forceinline__ int64_t loss_row_index(const int32_t* rowmap, int64_t row0, int64_t r) {
  return rowmap ? (int64_t)rowmap[row0 + r] : row0 + r;
}
// Buffer resource over `bytes` bytes from p (gfx9 word 3): loads beyond the
// range return 0.  (Only loads go through it.  A 16-byte buffer store whose
// offset is in an SGPR was measured to have its data registers overwritten
// by the VALU instruction the compiler schedules right after it -- the
// compiler inserts no wait state for that form -- so results are stored
// with global stores, whose wide-store hazard the compiler does cover.)
__device__ __forceinline__ __amdgpu_buffer_rsrc_t row_rsrc(const void* p, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, bytes, 0x00020000);
}
// The register kernel's transcendentals, branch-free and cheaper than
// tanhf / expf (which test ranges and, in tanhf's case, take two paths by
// |x|: lanes of a wave that disagree run both).  The kernel is bound by
// its arithmetic: with a 65,536 row in a whole CU's registers, the memory
// idles while the block computes.
//  * softcap15_fast: 15 tanh(y / 15) with tanh as an odd polynomial of
//    degree 11 (relative minimax fit on [0, 0.55], 1.2 ulp in float32)
//    below |x| = 0.55 and 1 - 2 / (e^(2|x|) + 1) above (hardware exp2 and
//    reciprocal; no cancellation above 0.55): measured on the device
//    within 4 ulp of 15 tanh(y / 15) over |y| <= 45, 2 ulp over |y| <= 8.
//  * exp_softcapped(x) = e^x for x = z - max z of a softcapped row, so
//    x in [-30, 0]: the hardware exp2 of x log2(e) with the product taken
//    in two parts (x times the float nearest log2(e), plus x times the
//    remainder), so the argument is off by its own rounding only and the
//    error has no sign bias.  Measured on the device: 1.4 ulp over
//    [-1, 0] (the terms that carry the sum), 23 ulp at worst near -29
//    (terms below 1e-12 of the largest), mean relative error -3e-9 (expf:
//    0.84 ulp, -2e-9).  With the constant alone the error was biased
//    upward (+2e-7 mean relative over [-30, 0]).
__device__ __forceinline__ float softcap15_fast(float y) {
  const float x = y * (1.0f / 15.0f);
  const float t = fabsf(x), u = t * t;
  float p = fmaf(-0.006235599052160978f, u, 0.021039707586169243f);
  p = fmaf(p, u, -0.05384271591901779f);
  p = fmaf(p, u, 0.13332460820674896f);
  p = fmaf(p, u, -0.3333331048488617f);
  p = fmaf(p, u, 1.0f);
  const float e = __builtin_amdgcn_exp2f(t * 2.8853900817779268f);  // e^(2t)
  const float big = fmaf(-2.0f, __builtin_amdgcn_rcpf(e + 1.0f), 1.0f);
  return copysignf(t < 0.55f ? t * p : big, x) * 15.0f;
}
__device__ __forceinline__ float exp_softcapped(float x) {
  return __builtin_amdgcn_exp2f(fmaf(x, 1.4426950408889634f, x * 1.925963033500011e-08f));
}
template <int Q, bool FULL>
__global__ __launch_bounds__(1024) void pg_loss_rows_reg_kernel(
    float* __restrict__ z, int64_t ldz, int V, int64_t row0, const int32_t* __restrict__ rowmap,
    const int32_t* __restrict__ targets, const float* __restrict__ adv, int T, float norm,
    float* __restrict__ nll, double* __restrict__ loss_rows) {
  __shared__ float sf[16];
  __shared__ double sd[16];
  // rows of 32,768 entries or more take the branch-free softcap and
  // exponential (the arithmetic bounds the kernel there); shorter rows keep
  // tanhf / expf
  constexpr bool FAST = Q >= 8;
  auto sc = [](float y) { return FAST ? softcap15_fast(y) : softcap15(y); };
  auto ex = [](float x) { return FAST ? exp_softcapped(x) : expf(x); };
  const int64_t r = blockIdx.x;
  const int64_t n = loss_row_index(rowmap, row0, r);
  float* zr = z + r * ldz;
  // float4 group k of this thread is row bytes [16 * (tid + 1024 k), +16):
  // one VGPR offset and the group's byte offset as a scalar
  const __amdgpu_buffer_rsrc_t rs = row_rsrc(zr, V * 4);
  const int V4 = V >> 2, tid = threadIdx.x, voff = tid * 16;
  v4f* zr4 = reinterpret_cast<v4f*>(zr);  // 16-byte aligned rows (launcher)
  const int32_t tg = targets[n];
  if (tg < 0) {
    const v4f zero = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int k = 0; k < Q; k++)
      if (FULL || tid + k * 1024 < V4) zr4[tid + k * 1024] = zero;
    if (tid == 0) {
      nll[n] = 0.f;
      loss_rows[row0 + r] = 0.0;
    }
    return;
  }
  const float zt = sc(zr[tg]);
  v4f v[Q];
#pragma unroll
  for (int k = 0; k < Q; k++) {
    v[k] = __builtin_amdgcn_raw_buffer_load_b128(rs, voff, k * 16384, 0);
#pragma unroll
    for (int c = 0; c < 4; c++) v[k][c] = sc(v[k][c]);
  }
  if (!FULL) {
#pragma unroll
    for (int k = 0; k < Q; k++)
      if (tid + k * 1024 >= V4) v[k] = (v4f){-INFINITY, -INFINITY, -INFINITY, -INFINITY};
  }
  float m = -INFINITY;
#pragma unroll
  for (int k = 0; k < Q; k++) m = fmaxf(fmaxf(m, fmaxf(v[k][0], v[k][1])), fmaxf(v[k][2], v[k][3]));
  m = block_max(m, sf);
  double s = 0;
#pragma unroll
  for (int k = 0; k < Q; k++) {
    if (FULL || tid + k * 1024 < V4)
      s += ((double)ex(v[k][0] - m) + (double)ex(v[k][1] - m)) +
           ((double)ex(v[k][2] - m) + (double)ex(v[k][3] - m));
  }
  s = block_sum<double>(s, sd);
  const float a = adv[n / T];
  const float nl = m + (float)log(s) - zt;
  if (tid == 0) {
    nll[n] = nl;
    loss_rows[row0 + r] = (double)nl * (double)a / (double)norm;
  }
  const float inv = (float)(1.0 / s);
  const float scale = a / norm;
  const float ic = 1.0f / 15.0f;
  // the same maximum, hidden from common-subexpression elimination: the
  // exponentials are recomputed here rather than kept live from the sum
  // (64 more registers per thread than the budget holds)
  float mg = m;
  asm volatile("" : "+v"(mg));
#pragma unroll
  for (int k = 0; k < Q; k++) {
    const int j = tid + k * 1024;
    v4f g;
#pragma unroll
    for (int c = 0; c < 4; c++) {
      const float zj = v[k][c];
      float p = ex(zj - mg) * inv;
      if (4 * j + c == tg) p -= 1.f;
      const float sc = zj * ic;
      g[c] = (p * scale) * (1.f - sc * sc);
    }
    if (FULL || j < V4) zr4[j] = g;
  }
}
__global__ __launch_bounds__(256) void pg_loss_rows_kernel(float* __restrict__ z, int64_t ldz,
                                                           int V, int64_t row0,
                                                           const int32_t* __restrict__ rowmap,
                                                           const int32_t* __restrict__ targets,
                                                           const float* __restrict__ adv, int T,
                                                           float norm, float* __restrict__ nll,
                                                           double* __restrict__ loss_rows) {
  __shared__ float sf[4];
  __shared__ double sd[4];
  const int64_t r = blockIdx.x;
  const int64_t n = loss_row_index(rowmap, row0, r);
  float* zr = z + r * ldz;
  const int32_t tg = targets[n];
  if (tg < 0) {
    for (int j = threadIdx.x; j < V; j += 256) zr[j] = 0.f;
    if (threadIdx.x == 0) {
      nll[n] = 0.f;
      loss_rows[row0 + r] = 0.0;
    }
    return;
  }
  float m = -INFINITY;
  for (int j = threadIdx.x; j < V; j += 256) m = fmaxf(m, softcap15(zr[j]));
  m = block_max(m, sf);
  double s = 0;
  for (int j = threadIdx.x; j < V; j += 256) s += (double)expf(softcap15(zr[j]) - m);
  s = block_sum<double>(s, sd);
  const float a = adv[n / T];
  const float nl = m + (float)log(s) - softcap15(zr[tg]);
  if (threadIdx.x == 0) {
    nll[n] = nl;
    loss_rows[row0 + r] = (double)nl * (double)a / (double)norm;
  }
  const float inv = (float)(1.0 / s);
  const float scale = a / norm;
  const float ic = 1.0f / 15.0f;
  __syncthreads();
  for (int j = threadIdx.x; j < V; j += 256) {
    float zj = softcap15(zr[j]);
    float p = expf(zj - m) * inv;
    if (j == tg) p -= 1.f;
    float sc = zj * ic;
    zr[j] = (p * scale) * (1.f - sc * sc);
  }
}
void launch_pg_loss_rows(float* z, int64_t ldz, int V, int64_t row0, int64_t rows,
                         const int32_t* rowmap, const int32_t* targets, const float* adv, int T,
                         float norm, float* nll, double* loss_rows, hipStream_t st) {
  if (rows <= 0) return;
  const bool vec = V % 4 == 0 && ldz % 4 == 0 && (reinterpret_cast<uintptr_t>(z) & 15) == 0;
  const int q = ceil_div(V, 4096);
  const dim3 grid((unsigned)rows);
#define GN_PG_REG(Q)                                                                           \
  do {                                                                                         \
    if (V == 4096 * Q)                                                                         \
      hipLaunchKernelGGL((pg_loss_rows_reg_kernel<Q, true>), grid, dim3(1024), 0, st, z, ldz, V, \
                         row0, rowmap, targets, adv, T, norm, nll, loss_rows);                 \
    else                                                                                       \
      hipLaunchKernelGGL((pg_loss_rows_reg_kernel<Q, false>), grid, dim3(1024), 0, st, z, ldz, \
                         V, row0, rowmap, targets, adv, T, norm, nll, loss_rows);              \
  } while (0)
  if (vec && q <= 1) GN_PG_REG(1);
  else if (vec && q <= 2) GN_PG_REG(2);
  else if (vec && q <= 4) GN_PG_REG(4);
  else if (vec && q <= 8) GN_PG_REG(8);
  else if (vec && q <= 16) GN_PG_REG(16);
  else
    hipLaunchKernelGGL(pg_loss_rows_kernel, grid, dim3(256), 0, st, z, ldz, V, row0, rowmap,
                       targets, adv, T, norm, nll, loss_rows);
#undef GN_PG_REG
  GN_HIP(hipGetLastError());
}

// dst[i, :] = src[idx[i], :] for i < n (rows of C floats)
__global__ __launch_bounds__(256) void gather_rows_kernel(const float* __restrict__ src,
                                                          const int32_t* __restrict__ idx,
                                                          float* __restrict__ dst, int64_t n,
                                                          int C) {
  const int64_t total = n * C;
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < total; e += (int64_t)gridDim.x * 256) {
    const int64_t i = e / C;
    dst[e] = src[(int64_t)idx[i] * C + (e - i * C)];
  }
}
// dst[idx[i], :] = src[i, :] for i < n (rows of C floats; other rows untouched)
__global__ __launch_bounds__(256) void scatter_rows_kernel(const float* __restrict__ src,
                                                           const int32_t* __restrict__ idx,
                                                           float* __restrict__ dst, int64_t n,
                                                           int C) {
  const int64_t total = n * C;
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < total; e += (int64_t)gridDim.x * 256) {
    const int64_t i = e / C;
    dst[(int64_t)idx[i] * C + (e - i * C)] = src[e];
  }
}
void launch_gather_rows(const float* src, const int32_t* idx, float* dst, int64_t n, int C,
                        hipStream_t st) {
  if (n <= 0) return;
  const unsigned blocks = (unsigned)std::min<int64_t>(ceil_div(n * C, 256), 65536);
  hipLaunchKernelGGL(gather_rows_kernel, dim3(blocks), dim3(256), 0, st, src, idx, dst, n, C);
  GN_HIP(hipGetLastError());
}
void launch_scatter_rows(const float* src, const int32_t* idx, float* dst, int64_t n, int C,
                         hipStream_t st) {
  if (n <= 0) return;
  const unsigned blocks = (unsigned)std::min<int64_t>(ceil_div(n * C, 256), 65536);
  hipLaunchKernelGGL(scatter_rows_kernel, dim3(blocks), dim3(256), 0, st, src, idx, dst, n, C);
  GN_HIP(hipGetLastError());
}

// ---------------------------------------------------------------------------
// Distillation rows (tensors/loss.go:84-214, trainer/distill.go:13-46).
// z [rows, V] holds the student's lm_head products y and zt the teacher's
// (row stride ldz); the logits are softcap15 of them, applied on load.  z is
// overwritten by dL/dy:
//   g = (float)((softmax(z/tau) - softmax(zt/tau)) * scale/tau) * (1 - (z/15)^2)
// with z, zt the softcapped logits; the forward-KL loss of the row,
// rounded to float32, is written to loss_rows (float64).  Rows whose target
// slot is negative are masked: zero gradient, zero loss.  The maxima, sums
// and exponentials are float64, as the reference computes them.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void distill_rows_kernel(float* __restrict__ z,
                                                           const float* __restrict__ zt,
                                                           int64_t ldz, int V, int64_t row0,
                                                           const int32_t* __restrict__ rowmap,
                                                           const int32_t* __restrict__ targets,
                                                           double tau, float scale,
                                                           double* __restrict__ loss_rows) {
  __shared__ double sd[4];
  const int64_t r = blockIdx.x;
  const int64_t n = loss_row_index(rowmap, row0, r);
  float* zr = z + r * ldz;
  const float* tr = zt + r * ldz;
  if (targets[n] < 0) {
    for (int j = threadIdx.x; j < V; j += 256) zr[j] = 0.f;
    if (threadIdx.x == 0) loss_rows[row0 + r] = 0.0;
    return;
  }
  double smax = -INFINITY, tmax = -INFINITY;
  for (int j = threadIdx.x; j < V; j += 256) {
    smax = fmax(smax, (double)softcap15(zr[j]) / tau);
    tmax = fmax(tmax, (double)softcap15(tr[j]) / tau);
  }
  // block maxima in float64 (max is exact in any order)
  {
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      smax = fmax(smax, __shfl_xor(smax, o, 64));
      tmax = fmax(tmax, __shfl_xor(tmax, o, 64));
    }
    __shared__ double mx[2][4];
    if (lane == 0) {
      mx[0][wid] = smax;
      mx[1][wid] = tmax;
    }
    __syncthreads();
    smax = fmax(fmax(mx[0][0], mx[0][1]), fmax(mx[0][2], mx[0][3]));
    tmax = fmax(fmax(mx[1][0], mx[1][1]), fmax(mx[1][2], mx[1][3]));
  }
  double ss = 0.0, ts = 0.0, ws = 0.0;
  for (int j = threadIdx.x; j < V; j += 256) {
    const double a = (double)softcap15(zr[j]) / tau, b = (double)softcap15(tr[j]) / tau;
    const double tw = exp(b - tmax);
    ss += exp(a - smax);
    ts += tw;
    ws += tw * a;
  }
  ss = block_sum<double>(ss, sd);
  ts = block_sum<double>(ts, sd);
  ws = block_sum<double>(ws, sd);
  if (threadIdx.x == 0) loss_rows[row0 + r] = (double)(float)(smax + log(ss) - ws / ts);
  const double is = 1.0 / ss, it = 1.0 / ts, gs = (double)scale / tau;
  const float ic = 1.0f / 15.0f;
  __syncthreads();
  for (int j = threadIdx.x; j < V; j += 256) {
    const float zj = softcap15(zr[j]);
    const double ps = exp((double)zj / tau - smax) * is;
    const double pt = exp((double)softcap15(tr[j]) / tau - tmax) * it;
    const float g = (float)((ps - pt) * gs);
    const float sc = zj * ic;
    zr[j] = g * (1.f - sc * sc);
  }
}
void launch_distill_rows(float* z, const float* zt, int64_t ldz, int V, int64_t row0, int64_t rows,
                         const int32_t* rowmap, const int32_t* targets, double tau, float scale,
                         double* loss_rows, hipStream_t st) {
  if (rows <= 0) return;
  hipLaunchKernelGGL(distill_rows_kernel, dim3((unsigned)rows), dim3(256), 0, st, z, zt, ldz, V,
                     row0, rowmap, targets, tau, scale, loss_rows);
  GN_HIP(hipGetLastError());
}

// Ordered float64 sum of n values into out[0] (one block).
__global__ __launch_bounds__(1024) void sum_f64_kernel(const double* __restrict__ v, int64_t n,
                                                       double* __restrict__ out, int accumulate) {
  __shared__ double sd[16];
  double acc = 0;
  for (int64_t i = threadIdx.x; i < n; i += blockDim.x) acc += v[i];
  acc = block_sum<double>(acc, sd);
  if (threadIdx.x == 0) out[0] = accumulate ? out[0] + acc : acc;
}
void launch_sum_f64(const double* v, int64_t n, double* out, bool accumulate, hipStream_t st) {
  hipLaunchKernelGGL(sum_f64_kernel, dim3(1), dim3(1024), 0, st, v, n, out, accumulate ? 1 : 0);
  GN_HIP(hipGetLastError());
}

// ---------------------------------------------------------------------------
// Backward row kernels
// ---------------------------------------------------------------------------
// RMSNorm backward (tensors/backward.go:81-104), float64 row statistics:
// out = g/r - x*(g.x)/(C r^3) [+ extra].  out may alias g or extra.
template <int NE>
__global__ __launch_bounds__(256) void rmsnorm_bwd_kernel(const float* __restrict__ x,
                                                          const float* g, const float* extra,
                                                          int C, float* out) {
  __shared__ double sd[4];
  const int64_t r = blockIdx.x;
  double ss = 0, dot = 0;
  for (int c = threadIdx.x; c < C; c += 256) {
    double xv = x[r * C + c], gv = g[r * C + c];
    ss += xv * xv;
    dot += gv * xv;
  }
  ss = block_sum<double>(ss, sd);
  dot = block_sum<double>(dot, sd);
  const double rms = sqrt(ss / C + (double)NORM_EPS);
  const double inv = 1.0 / rms;
  const double coef = dot / ((double)C * rms * rms * rms);
  float vals[NE];
  int k = 0;
  for (int c = threadIdx.x; c < C; c += 256, k++) {
    float v = (float)((double)g[r * C + c] * inv - coef * (double)x[r * C + c]);
    if (extra) v += extra[r * C + c];
    vals[k] = v;
  }
  __syncthreads();
  k = 0;
  for (int c = threadIdx.x; c < C; c += 256, k++) out[r * C + c] = vals[k];
}
// The same for widths that are a multiple of 256 (d12: 768, d20: 1280): one
// wave per row, four rows per block, the row's x and g read once as float4
// and kept in registers, wave-level float64 reductions (no block barriers).
// The one-block-per-row form reads both rows twice and synchronizes the
// block four times (0.43 of the HBM peak on the d12 training rows).
__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
template <int NV>
__global__ __launch_bounds__(256) void rmsnorm_bwd_wave_kernel(const float* __restrict__ x,
                                                               const float* g, const float* extra,
                                                               int64_t rows, float* out) {
  constexpr int C = 256 * NV;
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;
  const v4f* xr = reinterpret_cast<const v4f*>(x + r * C);
  const v4f* gr = reinterpret_cast<const v4f*>(g + r * C);
  v4f xv[NV], gv[NV], ev[NV];
#pragma unroll
  for (int i = 0; i < NV; i++) {
    xv[i] = xr[lane + 64 * i];
    gv[i] = gr[lane + 64 * i];
  }
  if (extra) {
    const v4f* er = reinterpret_cast<const v4f*>(extra + r * C);
#pragma unroll
    for (int i = 0; i < NV; i++) ev[i] = er[lane + 64 * i];
  }
  double ss = 0, dot = 0;
#pragma unroll
  for (int i = 0; i < NV; i++)
#pragma unroll
    for (int c = 0; c < 4; c++) {
      ss += (double)xv[i][c] * (double)xv[i][c];
      dot += (double)gv[i][c] * (double)xv[i][c];
    }
  ss = wave_sum_f64(ss);
  dot = wave_sum_f64(dot);
  const double rms = sqrt(ss / C + (double)NORM_EPS);
  const double inv = 1.0 / rms;
  const double coef = dot / ((double)C * rms * rms * rms);
  v4f* orow = reinterpret_cast<v4f*>(out + r * C);
#pragma unroll
  for (int i = 0; i < NV; i++) {
    v4f o;
#pragma unroll
    for (int c = 0; c < 4; c++) {
      float v = (float)((double)gv[i][c] * inv - coef * (double)xv[i][c]);
      if (extra) v += ev[i][c];
      o[c] = v;
    }
    orow[lane + 64 * i] = o;
  }
}
void launch_rmsnorm_bwd(const float* x, const float* g, const float* extra, int64_t rows, int C,
                        float* out, hipStream_t st) {
  const bool aligned = ((uintptr_t)x | (uintptr_t)g | (uintptr_t)out |
                        (extra ? (uintptr_t)extra : 0)) % 16 == 0;
  if (aligned && C % 256 == 0 && C <= 2048 && rows > 0) {
    const dim3 grid((unsigned)ceil_div(rows, 4));
    switch (C / 256) {
      case 1: hipLaunchKernelGGL(rmsnorm_bwd_wave_kernel<1>, grid, dim3(256), 0, st, x, g, extra, rows, out); break;
      case 2: hipLaunchKernelGGL(rmsnorm_bwd_wave_kernel<2>, grid, dim3(256), 0, st, x, g, extra, rows, out); break;
      case 3: hipLaunchKernelGGL(rmsnorm_bwd_wave_kernel<3>, grid, dim3(256), 0, st, x, g, extra, rows, out); break;
      case 4: hipLaunchKernelGGL(rmsnorm_bwd_wave_kernel<4>, grid, dim3(256), 0, st, x, g, extra, rows, out); break;
      case 5: hipLaunchKernelGGL(rmsnorm_bwd_wave_kernel<5>, grid, dim3(256), 0, st, x, g, extra, rows, out); break;
      case 6: hipLaunchKernelGGL(rmsnorm_bwd_wave_kernel<6>, grid, dim3(256), 0, st, x, g, extra, rows, out); break;
      case 7: hipLaunchKernelGGL(rmsnorm_bwd_wave_kernel<7>, grid, dim3(256), 0, st, x, g, extra, rows, out); break;
      case 8: hipLaunchKernelGGL(rmsnorm_bwd_wave_kernel<8>, grid, dim3(256), 0, st, x, g, extra, rows, out); break;
    }
    GN_HIP(hipGetLastError());
    return;
  }
  GN_ROW_NE_DISPATCH(C, hipLaunchKernelGGL(rmsnorm_bwd_kernel<NE>, dim3((unsigned)rows), dim3(256),
                                           0, st, x, g, extra, C, out));
  GN_HIP(hipGetLastError());
}

// Per-block float64 partial dot products of a with up to two vectors; the
// partials are reduced in a fixed order afterwards.
__global__ __launch_bounds__(256) void dot_partials_kernel(const float* __restrict__ a,
                                                           const float* __restrict__ b0,
                                                           const float* __restrict__ b1,
                                                           float sign, int64_t n,
                                                           double* __restrict__ part) {
  __shared__ double sd[4];
  double s0 = 0, s1 = 0;
  const bool vec = ((((uintptr_t)a | (uintptr_t)b0 | (uintptr_t)b1) & 15) == 0);
  const int64_t n4 = vec ? n / 4 : 0;
  if (n4 > 0) {
    // float4 loads, one float64 chain per component (summed in component
    // order at the end): four independent dependency chains per thread
    typedef float f4 __attribute__((ext_vector_type(4)));
    const f4* a4 = reinterpret_cast<const f4*>(a);
    const f4* p4 = reinterpret_cast<const f4*>(b0);
    const f4* q4 = reinterpret_cast<const f4*>(b1);
    double c0[4] = {0, 0, 0, 0}, c1[4] = {0, 0, 0, 0};
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += (int64_t)gridDim.x * 256) {
      const f4 x = a4[i], y = p4[i];
      f4 z;
      if (b1) z = q4[i];
#pragma unroll
      for (int c = 0; c < 4; c++) {
        c0[c] += (double)x[c] * (double)(sign * y[c]);
        if (b1) c1[c] += (double)x[c] * (double)z[c];
      }
    }
    s0 = ((c0[0] + c0[1]) + c0[2]) + c0[3];
    s1 = ((c1[0] + c1[1]) + c1[2]) + c1[3];
  }
  for (int64_t i = 4 * n4 + (int64_t)blockIdx.x * 256 + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * 256) {
    s0 += (double)a[i] * (double)(sign * b0[i]);
    if (b1) s1 += (double)a[i] * (double)b1[i];
  }
  s0 = block_sum<double>(s0, sd);
  s1 = block_sum<double>(s1, sd);
  if (threadIdx.x == 0) {
    part[blockIdx.x] = s0;
    if (b1) part[gridDim.x + blockIdx.x] = s1;
  }
}
// Reduces npart partials and adds float32(sum) into dst[0]: one block of
// 256 threads, thread t summing partials t, t + 256, ... in order, then the
// block sum (a fixed order).
__global__ __launch_bounds__(256) void partials_to_grad_kernel(const double* __restrict__ part,
                                                               int npart, float* __restrict__ dst) {
  __shared__ double sd[4];
  double s = 0;
  for (int i = threadIdx.x; i < npart; i += 256) s += part[i];
  s = block_sum<double>(s, sd);
  if (threadIdx.x == 0) dst[0] += (float)s;
}
void launch_dot_into_grad(const float* a, const float* b0, const float* b1, float sign, int64_t n,
                          float* dst0, float* dst1, double* part, hipStream_t st) {
  const int nb = 1024;
  hipLaunchKernelGGL(dot_partials_kernel, dim3(nb), dim3(256), 0, st, a, b0, b1, sign, n, part);
  GN_HIP(hipGetLastError());
  hipLaunchKernelGGL(partials_to_grad_kernel, dim3(1), dim3(256), 0, st, part, nb, dst0);
  if (b1) hipLaunchKernelGGL(partials_to_grad_kernel, dim3(1), dim3(256), 0, st, part + nb, nb, dst1);
  GN_HIP(hipGetLastError());
}

// Layer residual bookkeeping (train_transformer.go:218-230):
// g_next = lr*gb ; gx0 += l0*gb.
__global__ void resid_bwd_kernel(const float* __restrict__ gb, const float* __restrict__ lr,
                                 const float* __restrict__ l0, int layer, float* __restrict__ gnext,
                                 float* __restrict__ gx0, int64_t n) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  float g = gb[i];
  gnext[i] = g * lr[layer];
  gx0[i] = gx0[i] + l0[layer] * g;
}
void launch_resid_bwd(const float* gb, const float* lr, const float* l0, int layer, float* gnext,
                      float* gx0, int64_t n, hipStream_t st) {
  hipLaunchKernelGGL(resid_bwd_kernel, dim3((unsigned)ceil_div(n, 256)), dim3(256), 0, st, gb, lr,
                     l0, layer, gnext, gx0, n);
  GN_HIP(hipGetLastError());
}

// out = a + s*b (element-wise); out may alias a.
__global__ void axpy_kernel(float* out, const float* a, const float* __restrict__ b,
                            const float* __restrict__ sptr, float s, int64_t n) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  float sc = sptr ? -sptr[0] : s;
  out[i] = a[i] + sc * b[i];
}
void launch_axpy(float* out, const float* a, const float* b, const float* neg_scale_ptr, float s,
                 int64_t n, hipStream_t st) {
  hipLaunchKernelGGL(axpy_kernel, dim3((unsigned)ceil_div(n, 256)), dim3(256), 0, st, out, a, b,
                     neg_scale_ptr, s, n);
  GN_HIP(hipGetLastError());
}

// Backward of qkv_post (train.go:331-356 and 369-397) for one token per
// block: dq = rope^T(rmsnorm_bwd(qrot, 1.2*dqn)), likewise k; dv passes
// through; VE gate and value-embedding gradients.  Writes dqkv [N, (Hq+2Hkv)D];
// dpre [N, Hkv] is the VE pre-gate gradient; the value-embedding table
// gradient is scatter-added (repeated ids accumulate, linear.go:90-104).
__global__ __launch_bounds__(256) void qkv_post_bwd_kernel(QkvPostBwdArgs a) {
  constexpr int D = 128;
  const int64_t n = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int H = a.Hq + 2 * a.Hkv;
  const int t = (int)(n % a.T);
  const int half = a.R / 2, off = D - a.R;
  const float* cw = a.cosT + (int64_t)t * half;
  const float* sw = a.sinT + (int64_t)t * half;
  float* out = a.dqkv + n * (int64_t)H * D;
  // every q/k head of this wave (at most 4: <= 16 heads over 4 waves) is
  // requested before the first reduction
  constexpr int MH = 4;
  float xa[MH][2], ga[MH][2];
#pragma unroll
  for (int k = 0; k < MH; k++) {
    const int hd = wid + 4 * k;
    if (hd >= a.Hq + a.Hkv) break;
    const bool isq = hd < a.Hq;
    const int hh = isq ? hd : hd - a.Hq;
    const float* gsrc = isq ? a.dqn + (n * a.Hq + hh) * D : a.dkn + (n * a.Hkv + hh) * D;
    const float* xsrc = isq ? a.qrot + (n * a.Hq + hh) * D : a.krot + (n * a.Hkv + hh) * D;
#pragma unroll
    for (int e = 0; e < 2; e++) {
      xa[k][e] = xsrc[lane + 64 * e];
      ga[k][e] = gsrc[lane + 64 * e];
    }
  }
#pragma unroll
  for (int k = 0; k < MH; k++) {
    const int hd = wid + 4 * k;
    if (hd >= a.Hq + a.Hkv) break;
    float x[2], g[2];
    double ss = 0, dot = 0;
#pragma unroll
    for (int e = 0; e < 2; e++) {
      x[e] = xa[k][e];
      g[e] = ga[k][e] * QK_SCALE;
      ss += (double)x[e] * x[e];
      dot += (double)g[e] * x[e];
    }
    ss = warp_sum_d(ss);
    dot = warp_sum_d(dot);
    const double rms = sqrt(ss / D + (double)NORM_EPS);
    const double inv = 1.0 / rms, coef = dot / ((double)D * rms * rms * rms);
    float gp[2];
#pragma unroll
    for (int e = 0; e < 2; e++) gp[e] = (float)((double)g[e] * inv - coef * (double)x[e]);
    // rotary transpose: negated sine table (train.go:14-20, 334-336).  The
    // partner of dim d is d +- R/2, held by lane (d +- R/2) % 64 in slot
    // (d +- R/2) / 64.
#pragma unroll
    for (int e = 0; e < 2; e++) {
      int d = lane + 64 * e;
      int j = d - off;
      int pd = d >= off ? (j < half ? d + half : d - half) : d;
      float p0 = __shfl(gp[0], pd & 63, 64);
      float p1 = __shfl(gp[1], pd & 63, 64);
      float partner = (pd >> 6) ? p1 : p0;
      float v = gp[e];
      if (d >= off) {
        if (j < half) v = gp[e] * cw[j] - partner * sw[j];
        else v = partner * sw[j - half] + gp[e] * cw[j - half];
      }
      out[hd * D + d] = v;
    }
  }
  // v: gradient passes to the projection; VE pieces
  for (int i = tid; i < a.Hkv * D; i += 256) out[(a.Hq + a.Hkv) * D + i] = a.dv[n * a.Hkv * D + i];
  if (a.vesig) {
    const float* ver = a.ve + (int64_t)a.ids[n] * a.Hkv * D;
    float* gver = a.gve_rows + n * a.Hkv * D;  // this token's row, scattered by id afterwards
    for (int hk = wid; hk < a.Hkv; hk += 4) {
      const float s = a.vesig[n * a.Hkv + hk];
      const float scale = s * VE_SCALE;
      double dot = 0;
#pragma unroll
      for (int e = 0; e < 2; e++) {
        int d = lane + 64 * e;
        float gv = a.dv[(n * a.Hkv + hk) * D + d];
        gver[hk * D + d] = gv * scale;
        dot += (double)gv * (double)ver[hk * D + d];
      }
      dot = warp_sum_d(dot);
      if (lane == 0) {
        float gs = (float)dot * VE_SCALE;
        a.dpre[n * a.Hkv + hk] = gs * s * (1.f - s);
      }
    }
  }
}
void launch_qkv_post_bwd(const QkvPostBwdArgs& a, int64_t rows, hipStream_t st) {
  GN_CHECK(a.Hq + a.Hkv <= 16, "qkv_post backward: at most 16 q/k heads");
  hipLaunchKernelGGL(qkv_post_bwd_kernel, dim3((unsigned)rows), dim3(256), 0, st, a);
  GN_HIP(hipGetLastError());
}

// VE gate backward: dW[hk][c] += sum_n dpre[n,hk] * h[n,c] (c < 12) and
// dh[n, c] += sum_hk dpre[n,hk] * W[hk][c] (train.go:392-396).
__global__ __launch_bounds__(256) void ve_gate_dw_kernel(const float* __restrict__ dpre,
                                                         const float* __restrict__ h, int C,
                                                         int Hkv, int64_t N,
                                                         double* __restrict__ part) {
  // part[block][Hkv*12]
  __shared__ double sd[4];
  for (int hk = 0; hk < Hkv; hk++)
    for (int c = 0; c < VE_CH; c++) {
      double s = 0;
      for (int64_t n = (int64_t)blockIdx.x * 256 + threadIdx.x; n < N; n += (int64_t)gridDim.x * 256)
        s += (double)dpre[n * Hkv + hk] * (double)h[n * C + c];
      s = block_sum<double>(s, sd);
      if (threadIdx.x == 0) part[(int64_t)blockIdx.x * Hkv * VE_CH + hk * VE_CH + c] = s;
    }
}
__global__ void ve_gate_dw_reduce_kernel(const double* __restrict__ part, int nb, int count,
                                         float* __restrict__ dW) {
  int i = threadIdx.x;
  if (i >= count) return;
  double s = 0;
  for (int b = 0; b < nb; b++) s += part[(int64_t)b * count + i];
  dW[i] += (float)s;
}
__global__ void ve_gate_dh_kernel(const float* __restrict__ dpre, const float* __restrict__ W,
                                  int C, int Hkv, int64_t N, float* __restrict__ dh) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= N * VE_CH) return;
  int64_t n = i / VE_CH;
  int c = (int)(i % VE_CH);
  float s = 0.f;
  for (int hk = 0; hk < Hkv; hk++) s += dpre[n * Hkv + hk] * W[hk * VE_CH + c];
  dh[n * C + c] += s;
}
void launch_ve_gate_bwd(const float* dpre, const float* h, const float* W, int C, int Hkv,
                        int64_t N, float* dW, float* dh, double* part, hipStream_t st) {
  const int nb = 256;
  hipLaunchKernelGGL(ve_gate_dw_kernel, dim3(nb), dim3(256), 0, st, dpre, h, C, Hkv, N, part);
  hipLaunchKernelGGL(ve_gate_dw_reduce_kernel, dim3(1), dim3(64), 0, st, part, nb, Hkv * VE_CH, dW);
  hipLaunchKernelGGL(ve_gate_dh_kernel, dim3((unsigned)ceil_div(N * VE_CH, 256)), dim3(256), 0, st,
                     dpre, W, C, Hkv, N, dh);
  GN_HIP(hipGetLastError());
}

// Smear backward (train_transformer.go:269-305) for one token per block:
// ge[t] += ga[t]; ge[t-1] += ga[t]*gate(t); the gate/lambda gradients use the
// pre-smear embedding of t-1.  ge is written for row t only from ga[t] and
// ga[t+1], so blocks do not race.
__global__ __launch_bounds__(256) void smear_bwd_kernel(const float* __restrict__ ga,
                                                        const float* __restrict__ embn,
                                                        const float* __restrict__ smsig,
                                                        const float* __restrict__ lam, int C,
                                                        int T, float* __restrict__ ge,
                                                        float* __restrict__ ggate,
                                                        double* __restrict__ lam_rows) {
  __shared__ double sd[4];
  const int64_t n = blockIdx.x;
  const int t = (int)(n % T);
  const int64_t b = n / T;
  const float l = lam[0];
  // ge[t] = ga[t] + ga[t+1] * gate(t+1)
  float gnext = 0.f;
  if (t + 1 < T) gnext = l * smsig[b * (T - 1) + t];
  for (int c = threadIdx.x; c < C; c += 256) {
    float v = ga[n * C + c];
    if (t + 1 < T) v += ga[(n + 1) * C + c] * gnext;
    ge[n * C + c] = v;
  }
  if (t >= 1) {
    double gs = 0;
    for (int c = threadIdx.x; c < C; c += 256) gs += (double)ga[n * C + c] * (double)embn[(n - 1) * C + c];
    gs = block_sum<double>(gs, sd);
    if (threadIdx.x == 0) {
      const int64_t gi = b * (T - 1) + t - 1;
      const float s = smsig[gi];
      lam_rows[gi] = gs * (double)s;
      ggate[gi] = (float)(gs * (double)l) * s * (1.f - s);
    }
  }
}
// Smear-gate Linear backward (24 -> 1) and scatter of its input gradient into
// the first 24 channels of ge for rows t >= 1.
__global__ void smear_gate_bwd_kernel(const float* __restrict__ ggate,
                                      const float* __restrict__ embn,
                                      const float* __restrict__ wsg, int C, int T, int64_t NS,
                                      float* __restrict__ ge) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= NS * SMEAR_CH) return;
  int64_t gi = i / SMEAR_CH;
  int c = (int)(i % SMEAR_CH);
  int64_t b = gi / (T - 1);
  int t = (int)(gi % (T - 1)) + 1;
  int64_t n = b * T + t;
  ge[n * C + c] += ggate[gi] * wsg[c];
}
__global__ __launch_bounds__(256) void smear_gate_dw_kernel(const float* __restrict__ ggate,
                                                            const float* __restrict__ embn, int C,
                                                            int T, int64_t NS,
                                                            double* __restrict__ part) {
  __shared__ double sd[4];
  for (int c = 0; c < SMEAR_CH; c++) {
    double s = 0;
    for (int64_t gi = (int64_t)blockIdx.x * 256 + threadIdx.x; gi < NS; gi += (int64_t)gridDim.x * 256) {
      int64_t b = gi / (T - 1);
      int t = (int)(gi % (T - 1)) + 1;
      s += (double)ggate[gi] * (double)embn[(b * T + t) * C + c];
    }
    s = block_sum<double>(s, sd);
    if (threadIdx.x == 0) part[(int64_t)blockIdx.x * SMEAR_CH + c] = s;
  }
}
void launch_smear_bwd(const float* ga, const float* embn, const float* smsig, const float* lam,
                      const float* wsg, int B, int T, int C, float* ge, float* ggate,
                      double* lam_rows, double* part, float* dwsg, float* dlam, hipStream_t st) {
  int64_t N = (int64_t)B * T;
  hipLaunchKernelGGL(smear_bwd_kernel, dim3((unsigned)N), dim3(256), 0, st, ga, embn, smsig, lam,
                     C, T, ge, ggate, lam_rows);
  GN_HIP(hipGetLastError());
  if (T <= 1) return;
  int64_t NS = (int64_t)B * (T - 1);
  launch_sum_f64(lam_rows, NS, part, false, st);
  hipLaunchKernelGGL(partials_to_grad_kernel, dim3(1), dim3(64), 0, st, part, 1, dlam);
  const int nb = 128;
  hipLaunchKernelGGL(smear_gate_dw_kernel, dim3(nb), dim3(256), 0, st, ggate, embn, C, T, NS,
                     part + 8);
  hipLaunchKernelGGL(ve_gate_dw_reduce_kernel, dim3(1), dim3(64), 0, st, part + 8, nb, SMEAR_CH,
                     dwsg);
  hipLaunchKernelGGL(smear_gate_bwd_kernel, dim3((unsigned)ceil_div(NS * SMEAR_CH, 256)),
                     dim3(256), 0, st, ggate, embn, wsg, C, T, NS, ge);
  GN_HIP(hipGetLastError());
}

// Embedding backward: scatter-add rows of g into the table at the tokens'
// ids (linear.go:90-104: for n in order, gw[ids[n]] += g[n]).  The tokens
// come grouped by id (ids.perm: token indices, ascending within an id,
// ids.off: each id's range, ids.uid: the ids), so one thread owns each
// (id, column) and adds the id's rows in token order: the reference's
// float32 additions in its order, and the same bits on every run (float
// atomics would add in arrival order).
__global__ __launch_bounds__(256) void rows_scatter_kernel(const float* __restrict__ g, TokenGroups ids,
                                                           int C, float* __restrict__ gw) {
  const int u = blockIdx.x;
  const int c = blockIdx.y * 256 + threadIdx.x;
  if (c >= C) return;
  float* dst = gw + (int64_t)ids.uid[u] * C + c;
  float acc = *dst;
  for (int j = ids.off[u]; j < ids.off[u + 1]; j++) acc += g[(int64_t)ids.perm[j] * C + c];
  *dst = acc;
}
void launch_rows_scatter(const float* g, const TokenGroups& ids, int C, float* gw,
                         hipStream_t st) {
  if (ids.n_ids == 0) return;
  hipLaunchKernelGGL(rows_scatter_kernel, dim3((unsigned)ids.n_ids, (unsigned)ceil_div(C, 256)),
                     dim3(256), 0, st, g, ids, C, gw);
  GN_HIP(hipGetLastError());
}

}  // namespace gn
