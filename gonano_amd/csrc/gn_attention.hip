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
// Decode: one 256-thread block per (row, kv-head, split of up to 256 keys);
// each wave streams a contiguous quarter of the split.  Lanes form 8 groups
// of 8: group g takes key 8*step + g, lane part p of the group its dims
// [16p, 16p+16), so one step of a wave reads 8 whole K rows and 8 whole V
// rows (64 contiguous bytes per lane), and the next step's rows are loaded
// before the current step is computed.  Scores reduce over the 8 lanes of a
// group; an online softmax per head (running max / sum over the wave's keys)
// rescales the per-lane P.V accumulators; at the end the 8 groups and then
// the 4 waves are merged.  All r query heads of the GQA group share every
// K/V load.  The split's unnormalized output, max and sum go to `part`.
// ---------------------------------------------------------------------------
static constexpr int DEC_KPS = 256;  // keys per split
static constexpr int DEC_MAXR = 8;   // max GQA ratio

__device__ __forceinline__ float xor_groups_max(float v) {
  v = fmaxf(v, __shfl_xor(v, 8, 64));
  v = fmaxf(v, __shfl_xor(v, 16, 64));
  return fmaxf(v, __shfl_xor(v, 32, 64));
}
__device__ __forceinline__ float xor_groups_sum(float v) {
  v += __shfl_xor(v, 8, 64);
  v += __shfl_xor(v, 16, 64);
  return v + __shfl_xor(v, 32, 64);
}

template <int R>
__device__ __forceinline__ void decode_attn_body(const DecodeAttnArgs& a) {
  __shared__ __attribute__((aligned(16))) float qs[R][HD];
  __shared__ __attribute__((aligned(16))) float red[4][R][HD];
  __shared__ float wm[4][R], wl[4][R];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int g = lane >> 3, part = lane & 7;
  const int bh = blockIdx.x, s = blockIdx.y;
  const int row = bh / a.Hkv, hk = bh % a.Hkv;
  const int ks = a.kstart + s * DEC_KPS;
  const int nk = min(a.kend, ks + DEC_KPS) - ks;
  const float* qrow = a.q + ((int64_t)row * a.Hq + hk * R) * HD;
  for (int i = tid; i < R * HD; i += 256) qs[i / HD][i % HD] = qrow[i];
  __syncthreads();
  float qv[R][16];
#pragma unroll
  for (int h = 0; h < R; h++)
#pragma unroll
    for (int i = 0; i < 16; i++) qv[h][i] = qs[h][16 * part + i];

  const int q4 = (nk + 3) / 4;
  const int j0 = wid * q4, j1 = min(nk, j0 + q4);
  const int64_t cbase = ((int64_t)row * a.Hkv + hk) * a.maxSeq + ks;
  const float* kb = a.kc + cbase * HD + 16 * part;
  const float* vb = a.vc + cbase * HD + 16 * part;
  float m[R], l[R], acc[R][16];
#pragma unroll
  for (int h = 0; h < R; h++) {
    m[h] = -INFINITY;
    l[h] = 0.f;
#pragma unroll
    for (int i = 0; i < 16; i++) acc[h][i] = 0.f;
  }
  v4f kc[4], vc[4];
  auto load = [&](int j, v4f* kd, v4f* vd) {
    const int jj = j < j1 ? j : j0;  // clamp (value unused when j >= j1)
    const v4f* kp = reinterpret_cast<const v4f*>(kb + (int64_t)jj * HD);
    const v4f* vp = reinterpret_cast<const v4f*>(vb + (int64_t)jj * HD);
#pragma unroll
    for (int i = 0; i < 4; i++) {
      kd[i] = kp[i];
      vd[i] = vp[i];
    }
  };
  if (j0 < j1) load(j0 + g, kc, vc);
  for (int jb = j0; jb < j1; jb += 8) {
    const int j = jb + g;
    const bool valid = j < j1;
    v4f kn[4], vn[4];
    if (jb + 8 < j1) load(jb + 8 + g, kn, vn);
#pragma unroll
    for (int h = 0; h < R; h++) {
      float d = 0.f;
#pragma unroll
      for (int i = 0; i < 4; i++)
        d += kc[i][0] * qv[h][4 * i] + kc[i][1] * qv[h][4 * i + 1] + kc[i][2] * qv[h][4 * i + 2] +
             kc[i][3] * qv[h][4 * i + 3];
      d += __shfl_xor(d, 1, 64);
      d += __shfl_xor(d, 2, 64);
      d += __shfl_xor(d, 4, 64);
      const float sc = valid ? d : -INFINITY;
      const float mn = fmaxf(m[h], xor_groups_max(sc));
      const float scale = expf(m[h] - mn);  // 0 while m is -inf
      const float p = valid ? expf(sc - mn) : 0.f;
      l[h] = l[h] * scale + xor_groups_sum(p);  // one p per key group
#pragma unroll
      for (int i = 0; i < 4; i++) {
        acc[h][4 * i] = acc[h][4 * i] * scale + p * vc[i][0];
        acc[h][4 * i + 1] = acc[h][4 * i + 1] * scale + p * vc[i][1];
        acc[h][4 * i + 2] = acc[h][4 * i + 2] * scale + p * vc[i][2];
        acc[h][4 * i + 3] = acc[h][4 * i + 3] * scale + p * vc[i][3];
      }
      m[h] = mn;
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
      kc[i] = kn[i];
      vc[i] = vn[i];
    }
  }
  // merge the 8 key groups of the wave, then the 4 waves
#pragma unroll
  for (int h = 0; h < R; h++) {
#pragma unroll
    for (int i = 0; i < 16; i++) acc[h][i] = xor_groups_sum(acc[h][i]);
    if (g == 0)
#pragma unroll
      for (int i = 0; i < 16; i++) red[wid][h][16 * part + i] = acc[h][i];
    if (lane == 0) {
      wm[wid][h] = m[h];
      wl[wid][h] = l[h];
    }
  }
  __syncthreads();
  // One split covers every key of the row: write the normalized output
  // directly (the combine pass is skipped).  Otherwise emit the split's
  // (unnormalized output, max, sum) for decode_combine_kernel.
  const bool whole = a.nsplit == 1;
  float* out = a.part + ((int64_t)bh * a.nsplit + s) * R * (HD + 2);
  for (int i = tid; i < R * HD; i += 256) {
    const int h = i / HD, d = i % HD;
    float M = fmaxf(fmaxf(wm[0][h], wm[1][h]), fmaxf(wm[2][h], wm[3][h]));
    float o = 0.f, L = 0.f;
#pragma unroll
    for (int w = 0; w < 4; w++) {
      float sc = wm[w][h] > -INFINITY ? expf(wm[w][h] - M) : 0.f;
      o += red[w][h][d] * sc;
      L += wl[w][h] * sc;
    }
    if (whole) {
      a.o[((int64_t)row * a.Hq + hk * R + h) * HD + d] = o / L;
    } else {
      out[h * (HD + 2) + d] = o;
      if (d == 0) {
        out[h * (HD + 2) + HD] = M;
        out[h * (HD + 2) + HD + 1] = L;
      }
    }
  }
}

// One kernel per GQA ratio R, so each instance is sized (registers, LDS) for
// its own R rather than for the largest.
template <int R>
__global__ __launch_bounds__(256) void decode_attn_kernel(DecodeAttnArgs a) {
  decode_attn_body<R>(a);
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
  GN_CHECK(a.Hq % a.Hkv == 0 && a.Hq / a.Hkv <= DEC_MAXR, "decode attention: GQA ratio must be <= 8");
  GN_CHECK(a.kend > a.kstart, "decode attention: empty key range");
  a.nsplit = (int)ceil_div(a.kend - a.kstart, DEC_KPS);
  const dim3 grid(a.rows * a.Hkv, a.nsplit);
  switch (a.Hq / a.Hkv) {
    case 1: hipLaunchKernelGGL(decode_attn_kernel<1>, grid, dim3(256), 0, st, a); break;
    case 2: hipLaunchKernelGGL(decode_attn_kernel<2>, grid, dim3(256), 0, st, a); break;
    case 3: hipLaunchKernelGGL(decode_attn_kernel<3>, grid, dim3(256), 0, st, a); break;
    case 4: hipLaunchKernelGGL(decode_attn_kernel<4>, grid, dim3(256), 0, st, a); break;
    case 5: hipLaunchKernelGGL(decode_attn_kernel<5>, grid, dim3(256), 0, st, a); break;
    case 6: hipLaunchKernelGGL(decode_attn_kernel<6>, grid, dim3(256), 0, st, a); break;
    case 7: hipLaunchKernelGGL(decode_attn_kernel<7>, grid, dim3(256), 0, st, a); break;
    case 8: hipLaunchKernelGGL(decode_attn_kernel<8>, grid, dim3(256), 0, st, a); break;
  }
  GN_HIP(hipGetLastError());
  if (a.nsplit == 1) return;
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
