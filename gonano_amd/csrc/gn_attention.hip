// gn_attention.hip - causal (sliding-window) attention for the RL step.
//
//  * decode: one new query per row against the KV cache.  Memory-bound: the
//    grid is (row, kv-head) x key-chunks of 64 so K/V of a chunk are read once
//    for all query heads of the GQA group, one key per lane; a combine kernel
//    merges the chunks (model/attention.go:332-387 split-K, with the window
//    applied by skipping keys the reference masks to -1e30, whose softmax
//    weight is exactly zero).
//  * training/prefill: flash-attention forward with the log-sum-exp, and the
//    backward as two kernels (dQ per query block; dK/dV per key block over
//    the whole GQA group), deterministic and atomic-free
//    (kernels/scalar/attention.go:16-49 and 145-205 semantics).
//
// Scores carry no 1/sqrt(D) factor: q and k arrive already multiplied by 1.2
// after their RMSNorm (model/attention.go:252-256).
#include "gn_model.h"

namespace gn {

static constexpr int HD = 128;  // head dim
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v2f __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------------------
// Decode
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(64) void decode_attn_kernel(DecodeAttnArgs a) {
  constexpr int MAXR = 8;
  __shared__ __attribute__((aligned(16))) float qs[MAXR][HD];
  __shared__ float ps[MAXR][64];
  const int lane = threadIdx.x;
  const int bh = blockIdx.x, s = blockIdx.y;
  const int row = bh / a.Hkv, hk = bh % a.Hkv;
  const int r = a.Hq / a.Hkv;
  const int ks = a.kstart + s * 64;
  const int ke = min(a.kend, ks + 64);
  const float* qrow = a.q + ((int64_t)row * a.Hq + hk * r) * HD;
  for (int i = lane; i < r * HD; i += 64) qs[i / HD][i % HD] = qrow[i];
  __syncthreads();
  const int64_t cbase = ((int64_t)row * a.Hkv + hk) * a.maxSeq;
  const int kj = ks + lane;
  const bool valid = kj < ke;
  float sc[MAXR];
#pragma unroll
  for (int h = 0; h < MAXR; h++) sc[h] = 0.f;
  if (valid) {
    const v4f* kp = reinterpret_cast<const v4f*>(a.kc + (cbase + kj) * HD);
#pragma unroll 8
    for (int d4 = 0; d4 < HD / 4; d4++) {
      v4f kv = kp[d4];
#pragma unroll
      for (int h = 0; h < MAXR; h++) {
        if (h < r) {
          v4f qv = *reinterpret_cast<const v4f*>(&qs[h][4 * d4]);
          sc[h] += kv[0] * qv[0] + kv[1] * qv[1] + kv[2] * qv[2] + kv[3] * qv[3];
        }
      }
    }
  }
  float mh[MAXR], lh[MAXR];
#pragma unroll
  for (int h = 0; h < MAXR; h++) {
    if (h < r) {
      float x = valid ? sc[h] : -INFINITY;
      float m = warp_max(x);
      float p = valid ? expf(x - m) : 0.f;
      ps[h][lane] = p;
      mh[h] = m;
      lh[h] = warp_sum(p);
    }
  }
  __syncthreads();
  v2f acc[MAXR];
#pragma unroll
  for (int h = 0; h < MAXR; h++) acc[h] = (v2f){0.f, 0.f};
  const int nk = ke - ks;
  const float* vbase = a.vc + (cbase + ks) * HD + 2 * lane;
  for (int j = 0; j < nk; j++) {
    v2f vv = *reinterpret_cast<const v2f*>(vbase + (int64_t)j * HD);
#pragma unroll
    for (int h = 0; h < MAXR; h++)
      if (h < r) acc[h] += ps[h][j] * vv;
  }
  float* out = a.part + ((int64_t)bh * a.nsplit + s) * r * (HD + 2);
#pragma unroll
  for (int h = 0; h < MAXR; h++) {
    if (h < r) {
      *reinterpret_cast<v2f*>(out + h * (HD + 2) + 2 * lane) = acc[h];
      if (lane == 0) {
        out[h * (HD + 2) + HD] = mh[h];
        out[h * (HD + 2) + HD + 1] = lh[h];
      }
    }
  }
}

__global__ __launch_bounds__(128) void decode_combine_kernel(DecodeAttnArgs a) {
  const int rq = blockIdx.x;  // row * Hq + qh
  const int row = rq / a.Hq, qh = rq % a.Hq;
  const int r = a.Hq / a.Hkv;
  const int hk = qh / r, h = qh % r;
  const float* base = a.part + ((int64_t)(row * a.Hkv + hk) * a.nsplit) * r * (HD + 2) + h * (HD + 2);
  const int64_t stride = (int64_t)r * (HD + 2);
  float gm = -INFINITY;
  for (int s = 0; s < a.nsplit; s++) gm = fmaxf(gm, base[s * stride + HD]);
  float total = 0.f, o = 0.f;
  for (int s = 0; s < a.nsplit; s++) {
    float sc = expf(base[s * stride + HD] - gm);
    total += base[s * stride + HD + 1] * sc;
    o += base[s * stride + threadIdx.x] * sc;
  }
  a.o[(int64_t)rq * HD + threadIdx.x] = o / total;
}

void launch_decode_attention(DecodeAttnArgs a, hipStream_t st) {
  GN_CHECK(a.Hq % a.Hkv == 0 && a.Hq / a.Hkv <= 8, "decode attention: GQA ratio must be <= 8");
  GN_CHECK(a.kend > a.kstart, "decode attention: empty key range");
  a.nsplit = (int)ceil_div(a.kend - a.kstart, 64);
  hipLaunchKernelGGL(decode_attn_kernel, dim3(a.rows * a.Hkv, a.nsplit), dim3(64), 0, st, a);
  GN_HIP(hipGetLastError());
  hipLaunchKernelGGL(decode_combine_kernel, dim3(a.rows * a.Hq), dim3(HD), 0, st, a);
  GN_HIP(hipGetLastError());
}

// ---------------------------------------------------------------------------
// Flash forward (training / prefill).  Block: 32 queries x 8 threads, each
// thread owning 16 of the 128 dims; keys streamed through LDS 32 at a time.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float red8(float v) {
  v += __shfl_xor(v, 1, 64);
  v += __shfl_xor(v, 2, 64);
  v += __shfl_xor(v, 4, 64);
  return v;
}
__device__ __forceinline__ bool key_valid(int kj, int t, int T, int window) {
  return kj < T && kj <= t && (window < 0 || t - kj <= window);
}

__global__ __launch_bounds__(256) void flash_fwd_kernel(FlashArgs a) {
  constexpr int LD = HD + 4;
  __shared__ __attribute__((aligned(16))) float Ks[32 * LD];
  __shared__ __attribute__((aligned(16))) float Vs[32 * LD];
  const int tid = threadIdx.x, qi = tid >> 3, part = tid & 7;
  const int qb = blockIdx.x * 32;
  const int bh = blockIdx.y, b = bh / a.Hq, qh = bh % a.Hq;
  const int hk = qh / (a.Hq / a.Hkv);
  const int t = qb + qi;
  const bool active = t < a.T;
  float q[16];
  {
    const float* qp = a.q + (((int64_t)b * a.T + min(t, a.T - 1)) * a.Hq + qh) * HD + 16 * part;
#pragma unroll
    for (int i = 0; i < 16; i += 4) {
      v4f v = *reinterpret_cast<const v4f*>(qp + i);
      q[i] = v[0]; q[i + 1] = v[1]; q[i + 2] = v[2]; q[i + 3] = v[3];
    }
  }
  const int kmin = a.window >= 0 ? max(0, qb - a.window) : 0;
  const int kmax = min(a.T, qb + 32);
  float m = -INFINITY, l = 0.f;
  float acc[16];
#pragma unroll
  for (int i = 0; i < 16; i++) acc[i] = 0.f;
  for (int kb = (kmin / 32) * 32; kb < kmax; kb += 32) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      int idx = tid + 256 * i;  // 32 rows x 32 float4
      int rr = idx >> 5, c4 = idx & 31;
      int kj = kb + rr;
      v4f kv = {0.f, 0.f, 0.f, 0.f}, vv = {0.f, 0.f, 0.f, 0.f};
      if (kj < a.T) {
        int64_t off = (((int64_t)b * a.T + kj) * a.Hkv + hk) * HD + 4 * c4;
        kv = *reinterpret_cast<const v4f*>(a.k + off);
        vv = *reinterpret_cast<const v4f*>(a.v + off);
      }
      *reinterpret_cast<v4f*>(&Ks[rr * LD + 4 * c4]) = kv;
      *reinterpret_cast<v4f*>(&Vs[rr * LD + 4 * c4]) = vv;
    }
    __syncthreads();
    float s[32];
    float bm = -INFINITY;
#pragma unroll
    for (int j = 0; j < 32; j++) {
      const float* kr = &Ks[j * LD + 16 * part];
      float p = 0.f;
#pragma unroll
      for (int i = 0; i < 16; i += 4) {
        v4f kv = *reinterpret_cast<const v4f*>(kr + i);
        p += q[i] * kv[0] + q[i + 1] * kv[1] + q[i + 2] * kv[2] + q[i + 3] * kv[3];
      }
      p = red8(p);
      s[j] = key_valid(kb + j, t, a.T, a.window) ? p : -INFINITY;
      bm = fmaxf(bm, s[j]);
    }
    if (bm > -INFINITY) {
      const float mn = fmaxf(m, bm);
      const float sc = expf(m - mn);
      l *= sc;
#pragma unroll
      for (int i = 0; i < 16; i++) acc[i] *= sc;
#pragma unroll
      for (int j = 0; j < 32; j++) {
        float p = expf(s[j] - mn);
        l += p;
        const float* vr = &Vs[j * LD + 16 * part];
#pragma unroll
        for (int i = 0; i < 16; i += 4) {
          v4f vv = *reinterpret_cast<const v4f*>(vr + i);
          acc[i] += p * vv[0];
          acc[i + 1] += p * vv[1];
          acc[i + 2] += p * vv[2];
          acc[i + 3] += p * vv[3];
        }
      }
      m = mn;
    }
    __syncthreads();
  }
  if (active) {
    const float inv = 1.f / l;
    float* op = a.o + (((int64_t)b * a.T + t) * a.Hq + qh) * HD + 16 * part;
#pragma unroll
    for (int i = 0; i < 16; i += 4)
      *reinterpret_cast<v4f*>(op + i) = (v4f){acc[i] * inv, acc[i + 1] * inv, acc[i + 2] * inv,
                                               acc[i + 3] * inv};
    if (a.lse && part == 0) a.lse[((int64_t)b * a.T + t) * a.Hq + qh] = m + logf(l);
  }
}

void launch_flash_fwd(const FlashArgs& a, hipStream_t st) {
  hipLaunchKernelGGL(flash_fwd_kernel, dim3((unsigned)ceil_div(a.T, 32), a.B * a.Hq), dim3(256), 0,
                     st, a);
  GN_HIP(hipGetLastError());
}

// delta[n, h] = dO[n, h, :] . O[n, h, :]  (the row correction sum_j dP P)
__global__ __launch_bounds__(256) void flash_delta_kernel(const float* __restrict__ o,
                                                          const float* __restrict__ dout,
                                                          float* __restrict__ delta, int64_t rows) {
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (r >= rows) return;
  v2f x = *reinterpret_cast<const v2f*>(o + r * HD + 2 * lane);
  v2f g = *reinterpret_cast<const v2f*>(dout + r * HD + 2 * lane);
  float s = warp_sum(x[0] * g[0] + x[1] * g[1]);
  if (lane == 0) delta[r] = s;
}

// dQ for 32 queries per block.
__global__ __launch_bounds__(256) void flash_bwd_dq_kernel(FlashBwdArgs a) {
  constexpr int LD = HD + 4;
  __shared__ __attribute__((aligned(16))) float Ks[32 * LD];
  __shared__ __attribute__((aligned(16))) float Vs[32 * LD];
  const int tid = threadIdx.x, qi = tid >> 3, part = tid & 7;
  const int qb = blockIdx.x * 32;
  const int bh = blockIdx.y, b = bh / a.Hq, qh = bh % a.Hq;
  const int hk = qh / (a.Hq / a.Hkv);
  const int t = qb + qi;
  const bool active = t < a.T;
  const int64_t qrow = ((int64_t)b * a.T + min(t, a.T - 1)) * a.Hq + qh;
  float q[16], g[16], dq[16];
#pragma unroll
  for (int i = 0; i < 16; i++) {
    q[i] = a.q[qrow * HD + 16 * part + i];
    g[i] = a.dout[qrow * HD + 16 * part + i];
    dq[i] = 0.f;
  }
  const float lse = a.lse[qrow], dl = a.delta[qrow];
  const int kmin = a.window >= 0 ? max(0, qb - a.window) : 0;
  const int kmax = min(a.T, qb + 32);
  for (int kb = (kmin / 32) * 32; kb < kmax; kb += 32) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      int idx = tid + 256 * i;
      int rr = idx >> 5, c4 = idx & 31;
      int kj = kb + rr;
      v4f kv = {0.f, 0.f, 0.f, 0.f}, vv = {0.f, 0.f, 0.f, 0.f};
      if (kj < a.T) {
        int64_t off = (((int64_t)b * a.T + kj) * a.Hkv + hk) * HD + 4 * c4;
        kv = *reinterpret_cast<const v4f*>(a.k + off);
        vv = *reinterpret_cast<const v4f*>(a.v + off);
      }
      *reinterpret_cast<v4f*>(&Ks[rr * LD + 4 * c4]) = kv;
      *reinterpret_cast<v4f*>(&Vs[rr * LD + 4 * c4]) = vv;
    }
    __syncthreads();
    for (int j = 0; j < 32; j++) {
      const float* kr = &Ks[j * LD + 16 * part];
      const float* vr = &Vs[j * LD + 16 * part];
      float s = 0.f, dp = 0.f;
#pragma unroll
      for (int i = 0; i < 16; i++) {
        s += q[i] * kr[i];
        dp += g[i] * vr[i];
      }
      s = red8(s);
      dp = red8(dp);
      if (key_valid(kb + j, t, a.T, a.window)) {
        float p = expf(s - lse);
        float ds = p * (dp - dl);
#pragma unroll
        for (int i = 0; i < 16; i++) dq[i] += ds * kr[i];
      }
    }
    __syncthreads();
  }
  if (active) {
#pragma unroll
    for (int i = 0; i < 16; i++) a.dq[qrow * HD + 16 * part + i] = dq[i];
  }
}

// dK, dV for 32 keys per block, summed over the query heads of the group.
__global__ __launch_bounds__(256) void flash_bwd_dkdv_kernel(FlashBwdArgs a) {
  constexpr int LD = HD + 4;
  __shared__ __attribute__((aligned(16))) float Qs[32 * LD];
  __shared__ __attribute__((aligned(16))) float Gs[32 * LD];
  __shared__ float Ls[32], Ds[32];
  const int tid = threadIdx.x, ki = tid >> 3, part = tid & 7;
  const int kb = blockIdx.x * 32;
  const int bk = blockIdx.y, b = bk / a.Hkv, hk = bk % a.Hkv;
  const int r = a.Hq / a.Hkv;
  const int kj = kb + ki;
  const bool active = kj < a.T;
  const int64_t krow = ((int64_t)b * a.T + min(kj, a.T - 1)) * a.Hkv + hk;
  float k[16], v[16], dk[16], dv[16];
#pragma unroll
  for (int i = 0; i < 16; i++) {
    k[i] = a.k[krow * HD + 16 * part + i];
    v[i] = a.v[krow * HD + 16 * part + i];
    dk[i] = 0.f;
    dv[i] = 0.f;
  }
  const int qend = a.window >= 0 ? min(a.T, kb + 32 + a.window) : a.T;
  for (int h = 0; h < r; h++) {
    const int qh = hk * r + h;
    for (int qb = kb; qb < qend; qb += 32) {
#pragma unroll
      for (int i = 0; i < 4; i++) {
        int idx = tid + 256 * i;
        int rr = idx >> 5, c4 = idx & 31;
        int t = qb + rr;
        v4f qv = {0.f, 0.f, 0.f, 0.f}, gv = {0.f, 0.f, 0.f, 0.f};
        if (t < a.T) {
          int64_t off = (((int64_t)b * a.T + t) * a.Hq + qh) * HD + 4 * c4;
          qv = *reinterpret_cast<const v4f*>(a.q + off);
          gv = *reinterpret_cast<const v4f*>(a.dout + off);
        }
        *reinterpret_cast<v4f*>(&Qs[rr * LD + 4 * c4]) = qv;
        *reinterpret_cast<v4f*>(&Gs[rr * LD + 4 * c4]) = gv;
      }
      if (tid < 32) {
        int t = qb + tid;
        int64_t qrow = ((int64_t)b * a.T + min(t, a.T - 1)) * a.Hq + qh;
        Ls[tid] = a.lse[qrow];
        Ds[tid] = a.delta[qrow];
      }
      __syncthreads();
      for (int i2 = 0; i2 < 32; i2++) {
        const float* qr = &Qs[i2 * LD + 16 * part];
        const float* gr = &Gs[i2 * LD + 16 * part];
        float s = 0.f, dp = 0.f;
#pragma unroll
        for (int i = 0; i < 16; i++) {
          s += qr[i] * k[i];
          dp += gr[i] * v[i];
        }
        s = red8(s);
        dp = red8(dp);
        const int t = qb + i2;
        if (active && t < a.T && key_valid(kj, t, a.T, a.window)) {
          float p = expf(s - Ls[i2]);
          float ds = p * (dp - Ds[i2]);
#pragma unroll
          for (int i = 0; i < 16; i++) {
            dv[i] += p * gr[i];
            dk[i] += ds * qr[i];
          }
        }
      }
      __syncthreads();
    }
  }
  if (active) {
#pragma unroll
    for (int i = 0; i < 16; i++) {
      a.dk[krow * HD + 16 * part + i] = dk[i];
      a.dv[krow * HD + 16 * part + i] = dv[i];
    }
  }
}

void launch_flash_bwd(const FlashBwdArgs& a, hipStream_t st) {
  int64_t rows = (int64_t)a.B * a.T * a.Hq;
  hipLaunchKernelGGL(flash_delta_kernel, dim3((unsigned)ceil_div(rows, 4)), dim3(256), 0, st, a.o,
                     a.dout, a.delta, rows);
  GN_HIP(hipGetLastError());
  hipLaunchKernelGGL(flash_bwd_dq_kernel, dim3((unsigned)ceil_div(a.T, 32), a.B * a.Hq), dim3(256),
                     0, st, a);
  GN_HIP(hipGetLastError());
  hipLaunchKernelGGL(flash_bwd_dkdv_kernel, dim3((unsigned)ceil_div(a.T, 32), a.B * a.Hkv),
                     dim3(256), 0, st, a);
  GN_HIP(hipGetLastError());
}

}  // namespace gn
