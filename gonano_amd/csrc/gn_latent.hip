// gn_latent.hip - kernels of the latent preset (model/preset.go:120-129):
// multi-head latent attention (model/mla.go) and the DeepSeekMoE
// feed-forward (model/moe.go, model/mlp.go's clamped SwiGLU shared expert).
//
// MLA.  Training and prefill run the non-absorbed form (mlaProjectHeads,
// mla.go:106-122): q = [QueryUp.q_lat | rope(QueryRope.h)] and k = [KeyUp.
// kv_lat | rope(KeyRope.h)] per head, v = ValueUp.kv_lat, then the flash
// kernels with head dim 128 and no QK-norm.  Decode runs the absorbed form
// (mlaForwardInference, mla.go:185-279) against a cache of one latent row
// per token plus the rotary keys; the content key and value up-projections
// are folded into the query and output projections once per weight upload
// (W_qabs = KeyUp^T.QueryUp per head, W_comb = Wo.ValueUp per head), so a
// decode step needs no per-head projection kernels.
//
// MoE.  Routing (softmax, top-k on logits + bias, expert-major placement in
// (token, slot) order) is computed on the device; the expert products are
// the GEMM's expert-grouped modes, so the launch shape never depends on the
// routing and the decode step can be captured in a graph.
#include <hip/hip_ext.h>

#include "gn_model.h"

namespace gn {

typedef float v4f __attribute__((ext_vector_type(4)));
static constexpr int HDIM = 128;

// Rotation of one rotary pair (model/rotary.go:43-75): the first half gets
// x1*cos + x2*sin, the second -x1*sin + x2*cos; sign -1 transposes it (the
// negated sine table of model/train.go:14-20).
__device__ __forceinline__ float rope_elem(const float* x, int j, int rd, const float* cosr,
                                           const float* sinr, float sign) {
  const int half = rd >> 1;
  if (j < half) {
    const float c = cosr[j], s = sign * sinr[j];
    return x[j] * c + x[j + half] * s;
  }
  const int i = j - half;
  const float c = cosr[i], s = sign * sinr[i];
  return -x[i] * s + x[i + half] * c;
}

// ---------------------------------------------------------------------------
// MLA, training / prefill: assemble q, k, v per token (one block per token).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void mla_assemble_kernel(MlaAssembleArgs a) {
  const int64_t n = blockIdx.x;
  const int t = (int)(n % a.T), b = (int)(n / a.T);
  const int pos = a.pos0 + t;
  const int cd = HDIM - a.rd, half = a.rd >> 1;
  const float* cosr = a.cosT + (int64_t)pos * half;
  const float* sinr = a.sinT + (int64_t)pos * half;
  const float* xa = a.xa + n * a.xw;
  const float* qr = xa + 2 * a.lat;
  const float* kr = qr + a.Hq * a.rd;
  const int kvuw = a.Hkv * (cd + HDIM);
  const float* kvu = a.kvu + n * kvuw;
  for (int i = threadIdx.x; i < a.Hq * HDIM; i += blockDim.x) {
    const int h = i / HDIM, d = i % HDIM;
    a.q[n * a.Hq * HDIM + i] = d < cd ? a.qc[(n * a.Hq + h) * cd + d]
                                      : rope_elem(qr + h * a.rd, d - cd, a.rd, cosr, sinr, 1.f);
  }
  for (int i = threadIdx.x; i < a.Hkv * HDIM; i += blockDim.x) {
    const int h = i / HDIM, d = i % HDIM;
    float kv;
    if (d < cd) {
      kv = kvu[h * cd + d];
    } else {
      kv = rope_elem(kr + h * a.rd, d - cd, a.rd, cosr, sinr, 1.f);
      if (a.rk_cache)
        a.rk_cache[((int64_t)b * a.maxSeq + pos) * a.Hkv * a.rd + h * a.rd + (d - cd)] = kv;
    }
    a.k[n * a.Hkv * HDIM + i] = kv;
    a.v[n * a.Hkv * HDIM + i] = kvu[a.Hkv * cd + i];
  }
  if (a.lat_cache)
    for (int i = threadIdx.x; i < a.lat; i += blockDim.x)
      a.lat_cache[((int64_t)b * a.maxSeq + pos) * a.lat + i] = xa[a.lat + i];
}

void launch_mla_assemble(const MlaAssembleArgs& a, int64_t rows, hipStream_t st) {
  GN_CHECK(a.rd > 0 && a.rd < HDIM && a.rd % 2 == 0, "mla: bad rotary width");
  if (rows <= 0) return;
  hipLaunchKernelGGL(mla_assemble_kernel, dim3((unsigned)rows), dim3(256), 0, st, a);
  GN_HIP(hipGetLastError());
}

// ---------------------------------------------------------------------------
// MLA backward glue (model/train.go:414-419, mla.go:126-146): the flash
// gradients dq, dk, dv -> the QueryUp input gradient dqc, the rotary parts of
// dxa (transposed rotation) and dkvu = [dk content | dv].
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void mla_post_bwd_kernel(MlaPostBwdArgs a) {
  const int64_t n = blockIdx.x;
  const int pos = (int)(n % a.T);
  const int cd = HDIM - a.rd, half = a.rd >> 1;
  const float* cosr = a.cosT + (int64_t)pos * half;
  const float* sinr = a.sinT + (int64_t)pos * half;
  float* dxa = a.dxa + n * a.xw;
  float* dqr = dxa + 2 * a.lat;
  float* dkr = dqr + a.Hq * a.rd;
  const int kvuw = a.Hkv * (cd + HDIM);
  float* dkvu = a.dkvu + n * kvuw;
  const float* dq = a.dq + n * a.Hq * HDIM;
  const float* dk = a.dk + n * a.Hkv * HDIM;
  for (int i = threadIdx.x; i < a.Hq * HDIM; i += blockDim.x) {
    const int h = i / HDIM, d = i % HDIM;
    if (d < cd) a.dqc[(n * a.Hq + h) * cd + d] = dq[i];
    else dqr[h * a.rd + d - cd] = rope_elem(dq + h * HDIM + cd, d - cd, a.rd, cosr, sinr, -1.f);
  }
  for (int i = threadIdx.x; i < a.Hkv * HDIM; i += blockDim.x) {
    const int h = i / HDIM, d = i % HDIM;
    if (d < cd) dkvu[h * cd + d] = dk[i];
    else dkr[h * a.rd + d - cd] = rope_elem(dk + h * HDIM + cd, d - cd, a.rd, cosr, sinr, -1.f);
    dkvu[a.Hkv * cd + i] = a.dv[n * a.Hkv * HDIM + i];
  }
}

void launch_mla_post_bwd(const MlaPostBwdArgs& a, int64_t rows, hipStream_t st) {
  if (rows <= 0) return;
  hipLaunchKernelGGL(mla_post_bwd_kernel, dim3((unsigned)rows), dim3(256), 0, st, a);
  GN_HIP(hipGetLastError());
}

// ---------------------------------------------------------------------------
// MLA decode.  mla_decode_prep: rotate the new token's query/key rotary
// parts and append (latent, rotary key) to the cache at the step position
// (kvcache.go:224-274 AppendMLA*).
// ---------------------------------------------------------------------------
__device__ __forceinline__ int decode_pos(const MlaDecodeArgs& a) {
  return a.pos_dev ? *a.pos_dev : a.pos;
}

__global__ __launch_bounds__(256) void mla_decode_prep_kernel(MlaDecodeArgs a) {
  const int row = blockIdx.x;
  if (a.xa_sum.splits > 0) {
    // the input projection's deferred sum: the row of xa, for this kernel
    // and the absorbed-query product after it
    for (int i = threadIdx.x; i < a.xw; i += blockDim.x)
      a.xa_w[(int64_t)row * a.xw + i] = pending_value(a.xa_sum, (int64_t)row * a.xw + i);
    __syncthreads();
  }
  const int pos = decode_pos(a), half = a.rd >> 1;
  const float* cosr = a.cosT + (int64_t)pos * half;
  const float* sinr = a.sinT + (int64_t)pos * half;
  const float* xa = a.xa + (int64_t)row * a.xw;
  const float* qr = xa + 2 * a.lat;
  const float* kr = qr + a.Hq * a.rd;
  for (int i = threadIdx.x; i < a.Hq * a.rd; i += blockDim.x) {
    const int h = i / a.rd, j = i % a.rd;
    a.qrope[(int64_t)row * a.Hq * a.rd + i] = rope_elem(qr + h * a.rd, j, a.rd, cosr, sinr, 1.f);
  }
  float* rk = a.rk_cache + ((int64_t)row * a.maxSeq + pos) * a.Hkv * a.rd;
  for (int i = threadIdx.x; i < a.Hkv * a.rd; i += blockDim.x) {
    const int h = i / a.rd, j = i % a.rd;
    rk[i] = rope_elem(kr + h * a.rd, j, a.rd, cosr, sinr, 1.f);
  }
  float* lc = a.lat_cache + ((int64_t)row * a.maxSeq + pos) * a.lat;
  for (int i = threadIdx.x; i < a.lat; i += blockDim.x) lc[i] = xa[a.lat + i];
}

// Absorbed attention for one row and one split of its key range, all NH
// query heads at once: score(h, j) = q_abs[h] . lat[j] + q_rope[h] .
// rk[j][kv(h)], softmax over the keys, out[h] = sum_j p(h, j) lat[j] (the
// value is [latent | 0], mla.go:249-259).  Three phases, as the dense decode
// kernel:
//  1. scores: each 16-lane quarter-wave takes one key at a time (keys qw,
//     qw + 4 NWV, ... of the split), lane l holds latent float4s l + 16c and
//     rotary-key float4 l of kv head c (rotary width 64: 16 float4 per kv
//     head), the next key is fetched while the current one is reduced
//     (16-lane DPP sums); scores go to LDS;
//  2. softmax per head over the split (each wave reduces the maximum itself);
//  3. P.V: wave w takes keys w, w + NWV, ...; lane l accumulates latent float4
//     l for every head (the rows were just read, so they come from L2);
//     waves are added in LDS.
// A split covering the whole range writes the normalized latent output,
// otherwise (sum, max, total) for mla_decode_combine_kernel.  Splits hold up
// to 132 keys: a 128-token window (129 keys) is one block per row, and the
// blocks of a step (two per CU at this kernel's registers) stay within one
// round; 64-key splits put a 129-key window in three blocks per row (1.5
// rounds) and measured 35.6 us against 24.9 us (d12 latent, cold caches).
static constexpr int MLA_KPS = 132;  // keys per split (at most)
static constexpr int MLA_MAXLAT = 256;
__device__ __forceinline__ float mla_rl(float v, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}
static constexpr int MLA_RD = 64;   // rotary width the kernel is laid out for

__host__ __device__ inline void mla_split(int kstart, int kend, int* kps, int* nsplit) {
  const int n = kend - kstart;
  const int ns = (n + MLA_KPS - 1) / MLA_KPS;
  *kps = (n + ns - 1) / ns;
  *nsplit = (n + *kps - 1) / *kps;
}

template <int NH, int NWV>
__global__ __launch_bounds__(64 * NWV) void mla_decode_attn_kernel(MlaDecodeArgs a) {
  constexpr int NT = 64 * NWV;
  __shared__ float sc[NH][MLA_KPS];
  __shared__ __attribute__((aligned(16))) float wacc[NWV][NH][MLA_MAXLAT];
  __shared__ float wred[NWV][NH];
  __shared__ float stat[2][NH];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int qw = tid >> 4, l16 = tid & 15;
  const int row = blockIdx.x, split = blockIdx.y;
  const int pos = decode_pos(a);
  const int kstart = max(0, pos - a.window), kend = pos + 1;
  int kps, nsplit;
  mla_split(kstart, kend, &kps, &nsplit);
  if (split >= nsplit) return;  // graph launches size the grid for the longest range
  const int ks = kstart + split * kps;
  const int nk = min(kend, ks + kps) - ks;
  const int ratio = NH / a.Hkv;
  const int nl4 = a.lat / 4, nr4 = a.Hkv * (MLA_RD / 4);
  const float* lbase = a.lat_cache + ((int64_t)row * a.maxSeq + ks) * a.lat;
  const float* rbase = a.rk_cache + ((int64_t)row * a.maxSeq + ks) * a.Hkv * MLA_RD;

  // ---- phase 1: scores
  {
    v4f ql[NH][4], qr[NH];
    const float* qa = a.qabs + (int64_t)row * NH * a.lat;
    const float* qp = a.qrope + (int64_t)row * NH * MLA_RD;
#pragma unroll
    for (int h = 0; h < NH; h++) {
#pragma unroll
      for (int c = 0; c < 4; c++) {
        const int f = l16 + 16 * c;
        ql[h][c] = f < nl4 ? *reinterpret_cast<const v4f*>(qa + h * a.lat + 4 * f)
                           : (v4f){0.f, 0.f, 0.f, 0.f};
      }
      qr[h] = *reinterpret_cast<const v4f*>(qp + h * MLA_RD + 4 * l16);
    }
    v4f L[4], K[4];
    auto fetch = [&](int j) {
      const int jj = j < nk ? j : 0;  // clamp (value unused)
#pragma unroll
      for (int c = 0; c < 4; c++) {
        const int f = l16 + 16 * c;
        L[c] = f < nl4 ? *reinterpret_cast<const v4f*>(lbase + (int64_t)jj * a.lat + 4 * f)
                       : (v4f){0.f, 0.f, 0.f, 0.f};
        K[c] = f < nr4 ? *reinterpret_cast<const v4f*>(rbase + (int64_t)jj * a.Hkv * MLA_RD + 4 * f)
                       : (v4f){0.f, 0.f, 0.f, 0.f};
      }
    };
    if (qw < nk) fetch(qw);
    for (int j = qw; j < nk; j += 4 * NWV) {
      v4f Lc[4], Kc[4];
#pragma unroll
      for (int c = 0; c < 4; c++) {
        Lc[c] = L[c];
        Kc[c] = K[c];
      }
      if (j + 4 * NWV < nk) fetch(j + 4 * NWV);
#pragma unroll
      for (int h = 0; h < NH; h++) {
        float t = 0.f;
#pragma unroll
        for (int c = 0; c < 4; c++)
          t += ql[h][c][0] * Lc[c][0] + ql[h][c][1] * Lc[c][1] + ql[h][c][2] * Lc[c][2] +
               ql[h][c][3] * Lc[c][3];
        const int c = h / ratio;  // this head's kv rotary float4 sits in slot c
#pragma unroll
        for (int cc = 0; cc < 4; cc++)
          if (cc == c)
            t += qr[h][0] * Kc[cc][0] + qr[h][1] * Kc[cc][1] + qr[h][2] * Kc[cc][2] +
                 qr[h][3] * Kc[cc][3];
        t = sum16_dpp(t);
        if (l16 == 0) sc[h][j] = t;
      }
    }
  }
  __syncthreads();

  // ---- phase 2: softmax over the split.  Every wave takes the maximum per
  // head itself from the scores in LDS (16-lane DPP + readlane); the thread
  // owning key j writes p = exp(s - max); per-wave sums are added by the
  // first NH threads.
  {
    float mx[NH];
#pragma unroll
    for (int h = 0; h < NH; h++) {
      float m = -INFINITY;
#pragma unroll
      for (int k = 0; k < (MLA_KPS + 63) / 64; k++) {
        const int j = lane + 64 * k;
        if (j < nk) m = fmaxf(m, sc[h][j]);
      }
      m = max16_dpp(m);
      mx[h] = fmaxf(fmaxf(mla_rl(m, 0), mla_rl(m, 16)), fmaxf(mla_rl(m, 32), mla_rl(m, 48)));
    }
    __syncthreads();  // every wave has read the scores before p overwrites them
    float ps[NH];
#pragma unroll
    for (int h = 0; h < NH; h++) ps[h] = 0.f;
    for (int j = tid; j < nk; j += NT)
#pragma unroll
      for (int h = 0; h < NH; h++) {
        const float p = expf(sc[h][j] - mx[h]);
        sc[h][j] = p;
        ps[h] += p;
      }
#pragma unroll
    for (int h = 0; h < NH; h++) {
      const float t = sum16_dpp(ps[h]);
      const float w = (mla_rl(t, 0) + mla_rl(t, 16)) + (mla_rl(t, 32) + mla_rl(t, 48));
      if (lane == 0) wred[wid][h] = w;
    }
    __syncthreads();
    if (tid < NH) {
      stat[0][tid] = mx[tid];
      float l = 0.f;
#pragma unroll
      for (int w = 0; w < NWV; w++) l += wred[w][tid];
      stat[1][tid] = l;
    }
  }

  // ---- phase 3: P.V over the latent rows
  {
    const bool has = lane < nl4;
    v4f acc[NH];
#pragma unroll
    for (int h = 0; h < NH; h++) acc[h] = (v4f){0.f, 0.f, 0.f, 0.f};
    constexpr int PV = (MLA_KPS + NWV - 1) / NWV;  // keys per wave at most
    v4f Lr[PV];
#pragma unroll
    for (int i = 0; i < PV; i++) {
      const int j = wid + NWV * i;
      Lr[i] = (has && j < nk) ? *reinterpret_cast<const v4f*>(lbase + (int64_t)j * a.lat + 4 * lane)
                              : (v4f){0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int i = 0; i < PV; i++) {
      const int j = wid + NWV * i;
      if (j < nk)
#pragma unroll
        for (int h = 0; h < NH; h++) acc[h] += sc[h][j] * Lr[i];
    }
#pragma unroll
    for (int h = 0; h < NH; h++)
      if (has) *reinterpret_cast<v4f*>(&wacc[wid][h][4 * lane]) = acc[h];
  }
  __syncthreads();
  const bool whole = nsplit == 1;
  for (int i = tid; i < NH * a.lat; i += NT) {
    const int h = i / a.lat, d = i % a.lat;
    float o = 0.f;
#pragma unroll
    for (int w = 0; w < NWV; w++) o += wacc[w][h][d];
    if (whole) {
      a.out[((int64_t)row * NH + h) * a.lat + d] = o / stat[1][h];
    } else {
      float* part = a.part + (((int64_t)row * a.nsplit_max + split) * NH + h) * (a.lat + 2);
      part[d] = o;
      if (d == 0) {
        part[a.lat] = stat[0][h];
        part[a.lat + 1] = stat[1][h];
      }
    }
  }
}

__global__ __launch_bounds__(256) void mla_decode_combine_kernel(MlaDecodeArgs a) {
  const int pos = decode_pos(a);
  int kps, nsplit;
  mla_split(max(0, pos - a.window), pos + 1, &kps, &nsplit);
  if (nsplit == 1) return;  // the attention kernel wrote the output
  const int rh = blockIdx.x;  // row * Hq + h
  const int row = rh / a.Hq, h = rh % a.Hq;
  const int64_t stride = (int64_t)a.Hq * (a.lat + 2);
  const float* base = a.part + ((int64_t)row * a.nsplit_max * a.Hq + h) * (a.lat + 2);
  float M = -INFINITY;
  for (int sp = 0; sp < nsplit; sp++) M = fmaxf(M, base[sp * stride + a.lat]);
  for (int d = threadIdx.x; d < a.lat; d += blockDim.x) {
    float tot = 0.f, o = 0.f;
    for (int sp = 0; sp < nsplit; sp++) {
      const float f = expf(base[sp * stride + a.lat] - M);
      tot += base[sp * stride + a.lat + 1] * f;
      o += base[sp * stride + d] * f;
    }
    a.out[(int64_t)rh * a.lat + d] = o / tot;
  }
}

int mla_decode_max_splits(int window, int maxSeq) {
  int kps, ns;
  mla_split(0, std::min(window, maxSeq - 1) + 1, &kps, &ns);
  return ns;
}

void launch_mla_decode_prep(const MlaDecodeArgs& a, hipStream_t st) {
  GN_CHECK(a.rd == MLA_RD && a.Hkv * a.rd <= 256, "mla decode: rotary width must be 64");
  GN_CHECK(a.pos_dev || a.pos < a.maxSeq, "mla decode: position outside the cache");
  GN_CHECK(a.xa_sum.splits == 0 || (a.xa_w == a.xa && a.xa_sum.stride == (int64_t)a.rows * a.xw &&
                                    a.xa_sum.splits <= PENDING_MAX_SPLITS),
           "mla decode: pending input-projection sum shape");
  hipLaunchKernelGGL(mla_decode_prep_kernel, dim3(a.rows), dim3(256), 0, st, a);
  GN_HIP(hipGetLastError());
}

void launch_mla_decode(MlaDecodeArgs a, hipStream_t st) {
  GN_CHECK(a.lat % 4 == 0 && a.lat <= MLA_MAXLAT, "mla decode: latent width must be a multiple "
                                                  "of 4 and at most 256");
  GN_CHECK(a.rd == MLA_RD && a.Hkv * a.rd <= 256,
           "mla decode: rotary width must be 64 and rotary keys at most 256 wide");
  GN_CHECK(a.Hq % a.Hkv == 0 && a.Hq <= 8, "mla decode: at most 8 query heads");
  GN_CHECK(a.window >= 0, "mla decode: bad window");
  const int pos_max = a.pos_dev ? a.maxSeq - 1 : a.pos;
  int kps, ns_max;
  // the longest key range a step of this launch can have
  mla_split(0, std::min(a.window, pos_max) + 1, &kps, &ns_max);
  a.nsplit_max = ns_max;
  GN_CHECK(a.part_splits >= ns_max, "mla decode: split buffer too small");
  GN_CHECK(a.pos_dev || a.pos < a.maxSeq, "mla decode: position outside the cache");
  const dim3 grid(a.rows, ns_max);
  hipEvent_t stop = ns_max > 1 ? nullptr : a.t_stop;
  // One split per row at every step (the sliding windows): 8-wave blocks,
  // twice the loads in flight of the single block per row a CU then holds
  // (d12 latent, 129 keys: 22.9 vs 25.5 us); several splits: 4-wave blocks,
  // two per CU (384 keys: 63.4 vs 66.7 us with 8 waves).
#define GN_MLA_ATTN(H)                                                                        \
  do {                                                                                        \
    if (ns_max == 1) {                                                                        \
      if (a.t_start || stop)                                                                  \
        hipExtLaunchKernelGGL((mla_decode_attn_kernel<H, 8>), grid, dim3(512), 0, st,        \
                              a.t_start, stop, 0, a);                                         \
      else                                                                                    \
        hipLaunchKernelGGL((mla_decode_attn_kernel<H, 8>), grid, dim3(512), 0, st, a);        \
    } else if (a.t_start || stop) {                                                           \
      hipExtLaunchKernelGGL((mla_decode_attn_kernel<H, 4>), grid, dim3(256), 0, st,          \
                            a.t_start, stop, 0, a);                                           \
    } else {                                                                                  \
      hipLaunchKernelGGL((mla_decode_attn_kernel<H, 4>), grid, dim3(256), 0, st, a);          \
    }                                                                                         \
  } while (0)
  switch (a.Hq) {
    case 1: GN_MLA_ATTN(1); break;
    case 2: GN_MLA_ATTN(2); break;
    case 3: GN_MLA_ATTN(3); break;
    case 4: GN_MLA_ATTN(4); break;
    case 5: GN_MLA_ATTN(5); break;
    case 6: GN_MLA_ATTN(6); break;
    case 7: GN_MLA_ATTN(7); break;
    case 8: GN_MLA_ATTN(8); break;
  }
#undef GN_MLA_ATTN
  GN_HIP(hipGetLastError());
  if (ns_max > 1) {
    if (a.t_stop)
      hipExtLaunchKernelGGL(mla_decode_combine_kernel, dim3(a.rows * a.Hq), dim3(256), 0, st,
                            nullptr, a.t_stop, 0, a);
    else
      hipLaunchKernelGGL(mla_decode_combine_kernel, dim3(a.rows * a.Hq), dim3(256), 0, st, a);
    GN_HIP(hipGetLastError());
  }
}

// ---------------------------------------------------------------------------
// Clamped SwiGLU over [gate | up] rows (kernels/scalar/elementwise.go:85-134):
// act[r][j] = silu(min(g, c)) * clamp(u, -c, c), sigmoid in float64.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void swiglu_eval(float g, float u, float c, float* out, float* dg,
                                            float* du, float dout) {
  float gm = 1.f, um = 1.f;
  if (c > 0.f && g >= c) { g = c; gm = 0.f; }
  if (c > 0.f) {
    if (u > c) { u = c; um = 0.f; }
    else if (u < -c) { u = -c; um = 0.f; }
  }
  const float sg = (float)(1.0 / (1.0 + exp(-(double)g)));
  const float silu = g * sg;
  if (out) *out = silu * u;
  if (dg) {
    const float sgrad = sg * (1.f + g * (1.f - sg));
    *dg = dout * u * sgrad * gm;
    *du = dout * silu * um;
  }
}

// With a deferred [gate | up] product pending, gu stands for its sum.
__global__ void swiglu_rows_kernel(const float* __restrict__ gu, int F, int64_t rows, float clamp,
                                   float* __restrict__ act, PendingSum pend) {
  const int64_t n = rows * F;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / F, j = i % F;
    const int64_t ig = r * 2 * F + j, iu = ig + F;
    const float g = pend.splits > 0 ? pending_value(pend, ig) : gu[ig];
    const float u = pend.splits > 0 ? pending_value(pend, iu) : gu[iu];
    float o;
    swiglu_eval(g, u, clamp, &o, nullptr, nullptr, 0.f);
    act[i] = o;
  }
}

__global__ void swiglu_rows_bwd_kernel(const float* __restrict__ gu, const float* __restrict__ dact,
                                       int F, int64_t rows, float clamp, float* __restrict__ dgu) {
  const int64_t n = rows * F;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / F, j = i % F;
    float dg, du;
    swiglu_eval(gu[r * 2 * F + j], gu[r * 2 * F + F + j], clamp, nullptr, &dg, &du, dact[i]);
    dgu[r * 2 * F + j] = dg;
    dgu[r * 2 * F + F + j] = du;
  }
}

static unsigned grid_for(int64_t n) {
  return (unsigned)std::min<int64_t>(std::max<int64_t>(ceil_div(n, 256), 1), 16384);
}

void launch_swiglu_rows(const float* gu, int F, int64_t rows, float clamp, float* act,
                        hipStream_t st, const PendingSum& pend) {
  if (rows <= 0) return;
  GN_CHECK(pend.splits == 0 || (pend.stride == rows * 2 * (int64_t)F && pend.splits <= PENDING_MAX_SPLITS),
           "swiglu: pending sum shape");
  hipLaunchKernelGGL(swiglu_rows_kernel, dim3(grid_for(rows * F)), dim3(256), 0, st, gu, F, rows,
                     clamp, act, pend);
  GN_HIP(hipGetLastError());
}
void launch_swiglu_rows_bwd(const float* gu, const float* dact, int F, int64_t rows, float clamp,
                            float* dgu, hipStream_t st) {
  if (rows <= 0) return;
  hipLaunchKernelGGL(swiglu_rows_bwd_kernel, dim3(grid_for(rows * F)), dim3(256), 0, st, gu, dact,
                     F, rows, clamp, dgu);
  GN_HIP(hipGetLastError());
}

// ---------------------------------------------------------------------------
// MoE routing (moe.go:123-153, kernels/scalar/moe.go:8-52).
// ---------------------------------------------------------------------------
static constexpr int MOE_MAXE = 64;
static constexpr int MOE_MAXK = 8;
static constexpr int MOE_PB = 256;  // (token, slot) pairs per placement block

// One wave per token, lane e = expert e: SoftmaxLastDim of the router
// logits (float64 total, p = float32(exp) * float32(1/total)), top-k of
// logits + bias (largest first, ties to the smaller index), weights = the
// chosen experts' probabilities.
// Softmax and top-k of one token's logits, lane e holding logit e (-inf for
// lanes >= E).
__device__ __forceinline__ void gate_route(float lg, bool on, const float* __restrict__ bias,
                                           int64_t r, int E, int K, float* __restrict__ probs,
                                           int32_t* __restrict__ sel, float* __restrict__ w) {
  const int lane = threadIdx.x & 63;
  float mx = lg;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
  const double x = on ? exp((double)(lg - mx)) : 0.0;
  double tot = x;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) tot += __shfl_xor(tot, o, 64);
  const float inv = (float)(1.0 / tot);
  const float pr = (float)x * inv;
  if (on) probs[r * E + lane] = pr;
  float work = on ? lg + bias[lane] : -INFINITY;
  for (int k = 0; k < K; k++) {
    // largest value, smallest index among equals
    float bv = work;
    int bi = on ? lane : 64;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const float ov = __shfl_xor(bv, o, 64);
      const int oi = __shfl_xor(bi, o, 64);
      if (ov > bv || (ov == bv && oi < bi)) {
        bv = ov;
        bi = oi;
      }
    }
    if (lane == bi) {
      sel[r * K + k] = bi;
      w[r * K + k] = pr;
      work = -INFINITY;
    }
  }
}

__global__ __launch_bounds__(256) void moe_gate_kernel(const float* __restrict__ logits,
                                                       const float* __restrict__ bias,
                                                       int64_t rows, int E, int K,
                                                       float* __restrict__ probs,
                                                       int32_t* __restrict__ sel,
                                                       float* __restrict__ w, PendingSum lsum) {
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;
  const bool on = lane < E;
  const float lg = !on ? -INFINITY
                       : lsum.splits > 0 ? pending_value(lsum, r * E + lane) : logits[r * E + lane];
  gate_route(lg, on, bias, r, E, K, probs, sel, w);
}

// Decode-size batches: one block per token computes the router logits
// x[r] . wr[e] itself (wave v takes experts v, v + 4, ...; the 64 lanes
// split the C columns, every load in flight at once, summed by shuffles --
// another rounding order of the router product's dot product), then wave 0
// routes the token.
static constexpr int MOE_GATE_C4 = 8;  // float4 columns per lane: C <= 2048

__global__ __launch_bounds__(256) void moe_gate_logits_kernel(const float* __restrict__ xin,
                                                              const float* __restrict__ wr, int C,
                                                              const float* __restrict__ bias,
                                                              int E, int K,
                                                              float* __restrict__ probs,
                                                              int32_t* __restrict__ sel,
                                                              float* __restrict__ w) {
  __shared__ float lgs[MOE_MAXE];
  const int lane = threadIdx.x & 63, v = threadIdx.x >> 6;
  const int64_t r = blockIdx.x;
  const int n4 = C / 4;
  const v4f* xv = reinterpret_cast<const v4f*>(xin + r * C);
  v4f xa[MOE_GATE_C4];
#pragma unroll
  for (int i = 0; i < MOE_GATE_C4; i++)
    if (lane + 64 * i < n4) xa[i] = xv[lane + 64 * i];
  for (int e0 = v; e0 < E; e0 += 16) {
    // experts e0, e0 + 4, e0 + 8, e0 + 12 of this wave, loads issued together
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    v4f wa[4][MOE_GATE_C4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int e = e0 + 4 * j;
      const v4f* wv = reinterpret_cast<const v4f*>(wr + (int64_t)min(e, E - 1) * C);
#pragma unroll
      for (int i = 0; i < MOE_GATE_C4; i++)
        if (lane + 64 * i < n4) wa[j][i] = wv[lane + 64 * i];
    }
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
      for (int i = 0; i < MOE_GATE_C4; i++)
        if (lane + 64 * i < n4)
          acc[j] += xa[i][0] * wa[j][i][0] + xa[i][1] * wa[j][i][1] + xa[i][2] * wa[j][i][2] +
                    xa[i][3] * wa[j][i][3];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      float t = acc[j];
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) t += __shfl_xor(t, o, 64);
      if (lane == 0 && e0 + 4 * j < E) lgs[e0 + 4 * j] = t;
    }
  }
  __syncthreads();
  if (v != 0) return;
  const bool on = lane < E;
  gate_route(on ? lgs[lane] : -INFINITY, on, bias, r, E, K, probs, sel, w);
}

// Rank of each pair among the pairs of its block that chose the same expert,
// in pair order, and the block's per-expert counts (wave ballots).
__device__ __forceinline__ int block_rank(int e_mine, bool valid, int E, int* cnt_lds,
                                          int (*wcnt)[MOE_MAXE]) {
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const uint64_t lt = lane ? (~0ull >> (64 - lane)) : 0ull;
  int rank = 0;
  for (int e = 0; e < E; e++) {
    const uint64_t mask = __ballot(valid && e_mine == e);
    if (e == e_mine) rank = __popcll(mask & lt);
    if (lane == 0) wcnt[wid][e] = __popcll(mask);
  }
  __syncthreads();
  if (valid)
    for (int w = 0; w < wid; w++) rank += wcnt[w][e_mine];
  if (tid < E) cnt_lds[tid] = wcnt[0][tid] + wcnt[1][tid] + wcnt[2][tid] + wcnt[3][tid];
  __syncthreads();
  return rank;
}

__global__ __launch_bounds__(MOE_PB) void moe_count_kernel(const int32_t* __restrict__ sel,
                                                           int64_t npairs, int E,
                                                           int* __restrict__ blockcnt) {
  __shared__ int wcnt[4][MOE_MAXE];
  __shared__ int cnt[MOE_MAXE];
  const int64_t p = (int64_t)blockIdx.x * MOE_PB + threadIdx.x;
  const bool valid = p < npairs;
  block_rank(valid ? sel[p] : -1, valid, E, cnt, wcnt);
  if (threadIdx.x < E) blockcnt[(int64_t)blockIdx.x * E + threadIdx.x] = cnt[threadIdx.x];
}

// One block: per-expert exclusive scans over the blocks, expert totals and
// offsets (off[E] = the pair count).
__global__ void moe_scan_kernel(int* __restrict__ blockcnt, int nblk, int E,
                                int* __restrict__ off) {
  __shared__ int tot[MOE_MAXE];
  const int e = threadIdx.x;
  if (e < E) {
    int run = 0;
    for (int b = 0; b < nblk; b++) {
      const int c = blockcnt[(int64_t)b * E + e];
      blockcnt[(int64_t)b * E + e] = run;
      run += c;
    }
    tot[e] = run;
  }
  __syncthreads();
  if (e == 0) {
    int run = 0;
    for (int x = 0; x < E; x++) {
      off[x] = run;
      run += tot[x];
    }
    off[E] = run;
  }
}

// Expert-major placement in (token, slot) order (moe.go:139-153): the pair
// row, weight and position, then the gathered input rows.
__global__ __launch_bounds__(MOE_PB) void moe_place_kernel(MoePlaceArgs a) {
  __shared__ int wcnt[4][MOE_MAXE];
  __shared__ int cnt[MOE_MAXE];
  const int64_t p = (int64_t)blockIdx.x * MOE_PB + threadIdx.x;
  const bool valid = p < a.npairs;
  const int e = valid ? a.sel[p] : -1;
  const int rank = block_rank(e, valid, a.E, cnt, wcnt);
  if (valid) {
    const int pos = a.off[e] + a.blockoff[(int64_t)blockIdx.x * a.E + e] + rank;
    a.perm_row[pos] = (int)(p / a.K);
    a.perm_w[pos] = a.w[p];
    a.inv[p] = pos;
  }
}

// xg[pos] = x[perm_row[pos]], one wave per gathered row.
__global__ __launch_bounds__(256) void moe_gather_kernel(const float* __restrict__ x,
                                                         const int* __restrict__ perm_row,
                                                         int64_t npairs, int C,
                                                         float* __restrict__ xg) {
  const int lane = threadIdx.x & 63;
  const int64_t pos = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (pos >= npairs) return;
  const v4f* src = reinterpret_cast<const v4f*>(x + (int64_t)perm_row[pos] * C);
  v4f* dst = reinterpret_cast<v4f*>(xg + pos * C);
  for (int c = lane; c < C / 4; c += 64) dst[c] = src[c];
}

// Decode-size batches (at most MOE_SMALL_PAIRS pairs): counts, offsets and
// the placement in one block, chunk by chunk in pair order (a pair's
// position is its expert's offset + the pairs of earlier chunks and of
// earlier lanes of its chunk with the same expert -- the multi-block
// placement's order).
static constexpr int MOE_SMALL_PAIRS = 16 * MOE_PB;

__global__ __launch_bounds__(MOE_PB) void moe_route_small_kernel(MoePlaceArgs a, int* __restrict__ off) {
  __shared__ int wcnt[4][MOE_MAXE];
  __shared__ int cnt[MOE_MAXE];
  __shared__ int base[MOE_MAXE];
  __shared__ int offs[MOE_MAXE + 1];
  const int tid = threadIdx.x;
  const int nch = (int)((a.npairs + MOE_PB - 1) / MOE_PB);
  if (tid < a.E) base[tid] = 0;
  __syncthreads();
  for (int c = 0; c < nch; c++) {
    const int64_t p = (int64_t)c * MOE_PB + tid;
    const bool valid = p < a.npairs;
    block_rank(valid ? a.sel[p] : -1, valid, a.E, cnt, wcnt);
    if (tid < a.E) base[tid] += cnt[tid];
    __syncthreads();
  }
  if (tid == 0) {
    int run = 0;
    for (int x = 0; x < a.E; x++) {
      offs[x] = run;
      off[x] = run;
      run += base[x];
    }
    offs[a.E] = run;
    off[a.E] = run;
  }
  __syncthreads();
  if (tid < a.E) base[tid] = 0;
  __syncthreads();
  for (int c = 0; c < nch; c++) {
    const int64_t p = (int64_t)c * MOE_PB + tid;
    const bool valid = p < a.npairs;
    const int e = valid ? a.sel[p] : -1;
    const int rank = block_rank(e, valid, a.E, cnt, wcnt);
    if (valid) {
      const int pos = offs[e] + base[e] + rank;
      a.perm_row[pos] = (int)(p / a.K);
      a.perm_w[pos] = a.w[p];
      a.inv[p] = pos;
    }
    __syncthreads();
    if (tid < a.E) base[tid] += cnt[tid];
    __syncthreads();
  }
}

__global__ __launch_bounds__(MOE_MAXE) void moe_load_accum_kernel(const int* off, int E,
                                                                   double* load) {
  const int e = threadIdx.x;
  if (e < E) load[e] += (double)(off[e + 1] - off[e]);
}
void launch_moe_load_accum(const int* off, int E, double* load, hipStream_t st) {
  GN_CHECK(E >= 1 && E <= MOE_MAXE, "moe: at most 64 experts");
  hipLaunchKernelGGL(moe_load_accum_kernel, dim3(1), dim3(MOE_MAXE), 0, st, off, E, load);
  GN_HIP(hipGetLastError());
}

// The counts are whole numbers (exact in float64), so the total and the mean
// do not depend on the order of the additions.
__global__ __launch_bounds__(MOE_MAXE) void moe_bias_update_kernel(double* load, float* bias,
                                                                   int E, float speed) {
  const int e = threadIdx.x;
  double total = 0.0;
  for (int i = 0; i < E; i++) total += load[i];
  __syncthreads();  // every thread has read the counts before they are cleared
  if (total <= 0.0 || e >= E) return;
  const double diff = total / (double)E - load[e];
  const float sign = diff > 0.0 ? 1.f : diff < 0.0 ? -1.f : 0.f;
  bias[e] += speed * sign;
  load[e] = 0.0;
}
void launch_moe_bias_update(double* load, float* bias, int E, float speed, hipStream_t st) {
  GN_CHECK(E >= 1 && E <= MOE_MAXE, "moe: at most 64 experts");
  hipLaunchKernelGGL(moe_bias_update_kernel, dim3(1), dim3(MOE_MAXE), 0, st, load, bias, E, speed);
  GN_HIP(hipGetLastError());
}

void launch_moe_route(const MoeRouteArgs& a, hipStream_t st) {
  GN_CHECK(a.E <= MOE_MAXE && a.K <= MOE_MAXK && a.K <= a.E, "moe: at most 64 experts, top-8");
  GN_CHECK(a.C % 4 == 0, "moe: model width must be a multiple of 4");
  const int64_t npairs = a.rows * a.K;
  if (a.rows <= 0) return;
  GN_CHECK(a.logits_sum.splits == 0 || (a.logits_sum.stride == a.rows * (int64_t)a.E &&
                                         a.logits_sum.splits <= PENDING_MAX_SPLITS),
           "moe: pending router sum shape");
  if (a.wr) {
    GN_CHECK(a.C % 4 == 0 && a.C <= 256 * MOE_GATE_C4,
             "moe: router in the gate kernel needs a width multiple of 4, at most 2048");
    hipLaunchKernelGGL(moe_gate_logits_kernel, dim3((unsigned)a.rows), dim3(256), 0, st, a.x,
                       a.wr, a.C, a.bias, a.E, a.K, a.probs, a.sel, a.w);
  } else {
    hipLaunchKernelGGL(moe_gate_kernel, dim3((unsigned)ceil_div(a.rows, 4)), dim3(256), 0, st,
                       a.logits, a.bias, a.rows, a.E, a.K, a.probs, a.sel, a.w, a.logits_sum);
  }
  GN_HIP(hipGetLastError());
  if (!a.xg && npairs <= MOE_SMALL_PAIRS) {
    // decode-size batch without a gathered copy: one placement block
    MoePlaceArgs pa{};
    pa.sel = a.sel; pa.w = a.w;
    pa.npairs = npairs; pa.K = a.K; pa.E = a.E; pa.C = a.C;
    pa.perm_row = a.perm_row; pa.perm_w = a.perm_w; pa.inv = a.inv;
    hipLaunchKernelGGL(moe_route_small_kernel, dim3(1), dim3(MOE_PB), 0, st, pa, a.off);
    GN_HIP(hipGetLastError());
    return;
  }
  const int nblk = (int)ceil_div(npairs, MOE_PB);
  hipLaunchKernelGGL(moe_count_kernel, dim3(nblk), dim3(MOE_PB), 0, st, a.sel, npairs, a.E,
                     a.blockcnt);
  GN_HIP(hipGetLastError());
  hipLaunchKernelGGL(moe_scan_kernel, dim3(1), dim3(64), 0, st, a.blockcnt, nblk, a.E, a.off);
  GN_HIP(hipGetLastError());
  MoePlaceArgs pa{};
  pa.sel = a.sel; pa.w = a.w; pa.x = a.x; pa.off = a.off; pa.blockoff = a.blockcnt;
  pa.npairs = npairs; pa.K = a.K; pa.E = a.E; pa.C = a.C;
  pa.perm_row = a.perm_row; pa.perm_w = a.perm_w; pa.inv = a.inv; pa.xg = a.xg;
  hipLaunchKernelGGL(moe_place_kernel, dim3(nblk), dim3(MOE_PB), 0, st, pa);
  GN_HIP(hipGetLastError());
  if (!a.xg) return;  // the expert products read the token rows through perm_row
  hipLaunchKernelGGL(moe_gather_kernel, dim3((unsigned)ceil_div(npairs, 4)), dim3(256), 0, st, a.x,
                     a.perm_row, npairs, a.C, a.xg);
  GN_HIP(hipGetLastError());
}

// The K pairs of a token ordered by expert id: the reference scatters in
// expert-major order (moe.go:161-169, 233-239).
__device__ __forceinline__ int sorted_pairs(const int32_t* sel, const int* inv, int64_t r, int K,
                                            int* pos) {
  int es[MOE_MAXK];
  for (int k = 0; k < K; k++) {
    es[k] = sel[r * K + k];
    pos[k] = inv[r * K + k];
  }
  for (int i = 1; i < K; i++)
    for (int j = i; j > 0 && es[j] < es[j - 1]; j--) {
      int t = es[j]; es[j] = es[j - 1]; es[j - 1] = t;
      t = pos[j]; pos[j] = pos[j - 1]; pos[j - 1] = t;
    }
  return K;
}

// x_next = mid + (shared + routed), routed = sum over the token's pairs in
// expert order of (w * scale) * y (block.go:40-45, moe.go:161-169).
__global__ __launch_bounds__(256) void moe_combine_kernel(MoeCombineArgs a) {
  const int64_t r = blockIdx.x;
  int pos[MOE_MAXK];
  sorted_pairs(a.sel, a.inv, r, a.K, pos);
  float wk[MOE_MAXK];
  for (int k = 0; k < a.K; k++) wk[k] = a.perm_w[pos[k]] * a.scale;
  for (int c = threadIdx.x; c < a.C; c += blockDim.x) {
    float moe = 0.f;
    for (int k = 0; k < a.K; k++) moe += wk[k] * a.yg[(int64_t)pos[k] * a.C + c];
    const float sh = a.shared_sum.splits > 0 ? pending_value(a.shared_sum, r * a.C + c)
                                             : a.shared[r * a.C + c];
    a.out[r * a.C + c] = a.mid[r * a.C + c] + (sh + moe);
  }
}

void launch_moe_combine(const MoeCombineArgs& a, int64_t rows, hipStream_t st) {
  if (rows <= 0) return;
  GN_CHECK(a.shared_sum.splits == 0 || (a.shared_sum.stride == rows * (int64_t)a.C &&
                                         a.shared_sum.splits <= PENDING_MAX_SPLITS),
           "moe: pending shared-expert sum shape");
  hipLaunchKernelGGL(moe_combine_kernel, dim3((unsigned)rows), dim3(256), 0, st, a);
  GN_HIP(hipGetLastError());
}

// ---------------------------------------------------------------------------
// Expert products over decode-size groups.  At decode the pairs per expert
// are few, so an expert's weights are read once per step and the products
// are bound by that stream, not by the matrix cores.  Block (expert e,
// outputs j0..j0+15) of 4 waves: wave w requests its weight fragments (rows
// j0..j0+15 over the w-th quarter of K, kept in registers) before anything
// that depends on the routing, then multiplies the expert's pairs in
// chunks of 64 (four 16-row MFMA tiles, each tile's rows requested while the
// previous one is multiplied), as the weights arrive.  The 4 quarter sums are
// added in LDS in wave order (deterministic) and one wave applies the
// epilogue.  No split-K partial buffers, no reduction launch.  (Chunks of 32
// pairs left every expert with more than 32 -- half of them at d12 decode,
// 256 rows x top-2 over 16 experts -- a second serial pass of loads,
// products, reduction and epilogue: 28 -> 20 us for the d12 gate/up product.)
// ---------------------------------------------------------------------------
// Calls averaging at most 16 pairs per expert (flash d12 decode: 64 rows x
// top-2 over 16 experts) take chunks of two tiles: half the accumulator
// registers, so the down instance at K = 768 runs three waves per SIMD
// (flash d12: its 768 blocks in one round of the CUs instead of 1.5).  The
// gate/up instance holds twice the weights: forced to three waves it
// spills 22 registers to scratch and measured slower (rollout 1080 ->
// 1111 ms), so it keeps two.
static constexpr int MOE_XW = 4;   // waves per block (K quarters)

template <int KH, bool GU, int MOE_CT>
__global__ __launch_bounds__(64 * MOE_XW, (MOE_CT == 2 && !GU) ? 3 : 1) void moe_expert_small_kernel(MoeExpertArgs a) {
  constexpr int NW = GU ? 2 : 1;          // weight matrices (gate, up | down)
  constexpr int JB = KH < 2 ? KH : 2;     // k groups of weights requested before the rows
  constexpr int NB = (NW + 2) * KH <= 40 ? 2 : 1;  // row buffers (double-buffered tiles)
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int nb = a.N / 16;
  const int e = blockIdx.x / nb, j0 = (blockIdx.x - e * nb) * 16;
  const int r = lane & 15, q = lane >> 4;
  const int kq = w * KH * 16 + 4 * q;  // this lane's first k of the wave's quarter
  // B fragments: lane (r, q) holds weight row j0 + r, k = kq + 16 g + c.
  // Loads complete in issue order (vmcnt), so the order of requests sets
  // what the products can start on: the first JB k groups of weights, then
  // the routing-dependent rows of the first tile, then the remaining
  // weights, which the products consume as they arrive.
  v4f f[NW][KH];
  const float* bw[NW];
#pragma unroll
  for (int m = 0; m < NW; m++) bw[m] = (m ? a.w1 : a.w0) + ((int64_t)e * a.N + j0 + r) * a.K + kq;
#pragma unroll
  for (int g = 0; g < JB; g++)
#pragma unroll
    for (int m = 0; m < NW; m++) f[m][g] = *reinterpret_cast<const v4f*>(bw[m] + 16 * g);
  const int beg = a.off[e], cnt = a.off[e + 1] - beg;
  if (cnt < 0) {
    // Never taken (offsets do not decrease).  A use of the first fragments
    // on a path that skips the products keeps their loads above this
    // routing-dependent branch (the compiler would otherwise sink them
    // below it, behind the latency of the offset load).
    float z = 0.f;
#pragma unroll
    for (int m = 0; m < NW; m++)
#pragma unroll
      for (int g = 0; g < JB; g++) z += f[m][g][0] + f[m][g][1] + f[m][g][2] + f[m][g][3];
    a.out[0] = z;
    return;
  }
  const int nchunk = (cnt + 16 * MOE_CT - 1) / (16 * MOE_CT);
  if (nchunk == 0) return;
  // A fragments of tile u of chunk t: lane (r, q) holds pair row
  // t*64 + 16u + r (clamped to the expert's last pair; those outputs are not
  // stored)
  v4f av[NB][KH];
  auto load_rows = [&](int t, int u, v4f(&dst)[KH]) {
    const int pr = beg + min(t * 16 * MOE_CT + 16 * u + r, cnt - 1);
    const int64_t arow = GU ? (int64_t)a.perm_row[pr] : (int64_t)pr;
    const float* ap = a.x + arow * a.K + kq;
#pragma unroll
    for (int g = 0; g < KH; g++) dst[g] = *reinterpret_cast<const v4f*>(ap + 16 * g);
  };
  __shared__ v4f red[MOE_XW][MOE_CT][NW][64];
  auto chunk = [&](int t, bool first) {
    const int tiles = min(MOE_CT, (cnt - t * 16 * MOE_CT + 15) / 16);  // block-uniform
    v4f acc[MOE_CT][NW];
#pragma unroll
    for (int u = 0; u < MOE_CT; u++)
#pragma unroll
      for (int m = 0; m < NW; m++) acc[u][m] = (v4f){0.f, 0.f, 0.f, 0.f};
    if (!first) load_rows(t, 0, av[0]);
#pragma unroll
    for (int u = 0; u < MOE_CT; u++) {
      if (u >= tiles) break;
      v4f(&cur)[KH] = av[NB == 2 ? (u & 1) : 0];
      if (NB == 2 && u + 1 < tiles) {
        load_rows(t, u + 1, av[(u + 1) & 1]);  // the next tile's rows behind this tile's products
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int g = 0; g < KH; g++)
#pragma unroll
        for (int c = 0; c < 4; c++)
#pragma unroll
          for (int m = 0; m < NW; m++)
            acc[u][m] = __builtin_amdgcn_mfma_f32_16x16x4f32(cur[g][c], f[m][g][c], acc[u][m], 0, 0, 0);
      if (NB == 1 && u + 1 < tiles) load_rows(t, u + 1, av[0]);
    }
    if (t > 0) __syncthreads();  // the previous chunk's sums have been read
#pragma unroll
    for (int u = 0; u < MOE_CT; u++)
      if (u < tiles)
#pragma unroll
        for (int m = 0; m < NW; m++) red[w][u][m][lane] = acc[u][m];
    __syncthreads();
    if (w == t % MOE_XW) {
      // D of a 16x16 block: lane holds output j0 + (lane & 15), pair rows 4q + c
#pragma unroll
      for (int u = 0; u < MOE_CT; u++) {
        if (u >= tiles) break;
        v4f sm[NW];
#pragma unroll
        for (int m = 0; m < NW; m++) {
          sm[m] = red[0][u][m][lane];
#pragma unroll
          for (int v = 1; v < MOE_XW; v++) sm[m] += red[v][u][m][lane];
        }
#pragma unroll
        for (int c = 0; c < 4; c++) {
          const int p = t * 16 * MOE_CT + 16 * u + 4 * q + c;
          if (p < cnt) {
            float v = sm[0][c];
            if constexpr (GU) swiglu_eval(sm[0][c], sm[1][c], a.clamp, &v, nullptr, nullptr, 0.f);
            a.out[(int64_t)(beg + p) * a.N + j0 + (lane & 15)] = v;
          }
        }
      }
    }
  };
  load_rows(0, 0, av[0]);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int g = JB; g < KH; g++)
#pragma unroll
    for (int m = 0; m < NW; m++) f[m][g] = *reinterpret_cast<const v4f*>(bw[m] + 16 * g);
  __builtin_amdgcn_sched_barrier(0);
  chunk(0, true);
  for (int t = 1; t < nchunk; t++) chunk(t, false);
}

bool moe_expert_small_supported(int N, int K) {
  if (N <= 0 || N % 16 || K <= 0 || K % (16 * MOE_XW)) return false;
  const int kh = K / (16 * MOE_XW);
  return kh <= 6 || kh == 8 || kh == 10 || kh == 12 || kh == 16;
}

bool launch_moe_expert_small(const MoeExpertArgs& a, hipStream_t st) {
  if (!moe_expert_small_supported(a.N, a.K) || a.E <= 0) return false;
  const int kh = a.K / (16 * MOE_XW);
  GN_CHECK((a.w1 != nullptr) == (a.perm_row != nullptr), "moe expert: gate/up needs both");
  const dim3 grid((unsigned)(a.E * (a.N / 16))), block(64 * MOE_XW);
  const bool small = a.pairs > 0 && a.pairs <= 16 * (int64_t)a.E;
#define GN_MOE_X(KH)                                                                          \
  case KH:                                                                                    \
    if (a.w1 && small) hipLaunchKernelGGL((moe_expert_small_kernel<KH, true, 2>), grid, block, 0, st, a); \
    else if (a.w1) hipLaunchKernelGGL((moe_expert_small_kernel<KH, true, 4>), grid, block, 0, st, a);    \
    else if (small) hipLaunchKernelGGL((moe_expert_small_kernel<KH, false, 2>), grid, block, 0, st, a);  \
    else hipLaunchKernelGGL((moe_expert_small_kernel<KH, false, 4>), grid, block, 0, st, a);             \
    break;
  switch (kh) {
    GN_MOE_X(1) GN_MOE_X(2) GN_MOE_X(3) GN_MOE_X(4) GN_MOE_X(5) GN_MOE_X(6) GN_MOE_X(8)
    GN_MOE_X(10) GN_MOE_X(12) GN_MOE_X(16)
    default:
      return false;
  }
#undef GN_MOE_X
  GN_HIP(hipGetLastError());
  return true;
}

// ---------------------------------------------------------------------------
// MoE backward (moe.go:203-267).
// ---------------------------------------------------------------------------
// Per pair (one wave): gy = g[row] * (w * scale) and the probability
// gradient term <g[row], y> * scale in float64.
__global__ __launch_bounds__(256) void moe_bwd_prep_kernel(const float* __restrict__ g,
                                                           const float* __restrict__ yg,
                                                           const int* __restrict__ perm_row,
                                                           const float* __restrict__ perm_w,
                                                           float scale, int64_t npairs, int C,
                                                           float* __restrict__ gy,
                                                           double* __restrict__ dotp) {
  const int lane = threadIdx.x & 63;
  const int64_t pidx = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (pidx >= npairs) return;
  const int64_t row = perm_row[pidx];
  const float w = perm_w[pidx] * scale;
  double d = 0.0;
  for (int c = lane; c < C; c += 64) {
    const float gv = g[row * C + c];
    gy[pidx * C + c] = gv * w;
    d += (double)gv * (double)yg[pidx * C + c];
  }
  d = warp_sum_d(d);
  if (lane == 0) dotp[pidx] = d * (double)scale;
}

void launch_moe_bwd_prep(const float* g, const float* yg, const int* perm_row, const float* perm_w,
                         float scale, int64_t npairs, int C, float* gy, double* dotp,
                         hipStream_t st) {
  if (npairs <= 0) return;
  hipLaunchKernelGGL(moe_bwd_prep_kernel, dim3((unsigned)ceil_div(npairs, 4)), dim3(256), 0, st, g,
                     yg, perm_row, perm_w, scale, npairs, C, gy, dotp);
  GN_HIP(hipGetLastError());
}

// Sequence-level balance loss (moe.go:276-326): per sequence, the selection
// counts and probability sums per expert; loss_seq = sum_e ss * count *
// sum / T with ss = E / (K T).  One block per sequence.  The probability
// sums are float64: thread (slice j, expert e) adds tokens j, j + S, ... of
// expert e (S = 256 / E slices; neighbouring threads read neighbouring
// floats), then thread e adds the S slice sums in slice order.  (One thread
// per expert walking all T tokens took 1.9 ms per call at T = 8,703.)
__global__ __launch_bounds__(256) void moe_balance_kernel(const float* __restrict__ probs,
                                                          const int32_t* __restrict__ sel, int T,
                                                          int E, int K, float* __restrict__ cnt,
                                                          double* __restrict__ loss_seq) {
  __shared__ int c[MOE_MAXE];
  __shared__ double term[MOE_MAXE];
  __shared__ double part[256];
  const int64_t s = blockIdx.x;
  if (threadIdx.x < E) c[threadIdx.x] = 0;
  __syncthreads();
  for (int i = threadIdx.x; i < T * K; i += blockDim.x) atomicAdd(&c[sel[s * T * K + i]], 1);
  const int S = 256 / E;  // E <= 64: at least 4 slices
  {
    const int e = threadIdx.x % E, j = threadIdx.x / E;
    double acc = 0.0;
    if (j < S)
      for (int t = j; t < T; t += S) acc += (double)probs[(s * T + t) * E + e];
    part[threadIdx.x] = acc;
  }
  __syncthreads();
  if (threadIdx.x < E) {
    const int e = threadIdx.x;
    double sum = 0.0;
    for (int j = 0; j < S; j++) sum += part[j * E + e];
    const double ss = (double)E / ((double)K * (double)T);
    term[e] = ss * (double)c[e] * (sum / (double)T);
    cnt[s * E + e] = (float)c[e];
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    double l = 0.0;
    for (int e = 0; e < E; e++) l += term[e];
    loss_seq[s] = l;
  }
}

void launch_moe_balance(const float* probs, const int32_t* sel, int S, int T, int E, int K,
                        float* cnt, double* loss_seq, hipStream_t st) {
  if (S <= 0) return;
  hipLaunchKernelGGL(moe_balance_kernel, dim3(S), dim3(256), 0, st, probs, sel, T, E, K, cnt,
                     loss_seq);
  GN_HIP(hipGetLastError());
}

// Router softmax backward per token: dProbs[e] = (sum of its pair terms) +
// balance gradient coef * count[seq][e]; dLogits = p * (dProbs - <p, dProbs>)
// in float64 (moe.go:245-263).
__global__ void moe_router_bwd_kernel(MoeRouterBwdArgs a) {
  const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= a.rows) return;
  double gp[MOE_MAXE];
  for (int e = 0; e < a.E; e++) gp[e] = 0.0;
  for (int k = 0; k < a.K; k++) {
    const int e = a.sel[r * a.K + k];
    gp[e] += a.dotp[a.inv[r * a.K + k]];
  }
  if (a.bal_cnt) {
    const float* c = a.bal_cnt + (r / a.T) * a.E;
    for (int e = 0; e < a.E; e++) gp[e] += a.bal_coef * (double)c[e];
  }
  double dot = 0.0;
  for (int e = 0; e < a.E; e++) dot += (double)a.probs[r * a.E + e] * gp[e];
  for (int e = 0; e < a.E; e++) {
    const double p = (double)a.probs[r * a.E + e];
    a.glog[r * a.E + e] = (float)(p * (gp[e] - dot));
  }
}

void launch_moe_router_bwd(const MoeRouterBwdArgs& a, hipStream_t st) {
  if (a.rows <= 0) return;
  hipLaunchKernelGGL(moe_router_bwd_kernel, dim3((unsigned)ceil_div(a.rows, 256)), dim3(256), 0, st,
                     a);
  GN_HIP(hipGetLastError());
}

// dh2 = dshared + ((sum over the token's pairs, expert order, of dxg) +
// drouter) (moe.go:233-266, train.go:561-564).
__global__ __launch_bounds__(256) void moe_bwd_combine_kernel(MoeBwdCombineArgs a) {
  const int64_t r = blockIdx.x;
  int pos[MOE_MAXK];
  sorted_pairs(a.sel, a.inv, r, a.K, pos);
  for (int c = threadIdx.x; c < a.C; c += blockDim.x) {
    float s = 0.f;
    for (int k = 0; k < a.K; k++) s += a.dxg[(int64_t)pos[k] * a.C + c];
    a.out[r * a.C + c] = a.dshared[r * a.C + c] + (s + a.drouter[r * a.C + c]);
  }
}

void launch_moe_bwd_combine(const MoeBwdCombineArgs& a, int64_t rows, hipStream_t st) {
  if (rows <= 0) return;
  hipLaunchKernelGGL(moe_bwd_combine_kernel, dim3((unsigned)rows), dim3(256), 0, st, a);
  GN_HIP(hipGetLastError());
}

// PrefillFrom for position-major caches (kvcache.go:383-448): rows
// [0, P) of src [G][maxSrc][W] are copied to each of the S rows of their
// group in dst [G*S][maxDst][W].
__global__ void replicate_rows_kernel(const float* __restrict__ src, float* __restrict__ dst, int G,
                                      int S, int P, int W, int maxSrc, int maxDst, int64_t total) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;  // total = G*S*P*W
  const int w = (int)(i % W);
  int64_t r = i / W;
  const int p = (int)(r % P);
  const int64_t row = r / P;
  const int64_t g = row / S;
  dst[(row * maxDst + p) * W + w] = src[(g * maxSrc + p) * W + w];
}

void launch_replicate_rows(const float* src, float* dst, int G, int S, int P, int W, int maxSrc,
                           int maxDst, hipStream_t st) {
  const int64_t total = (int64_t)G * S * P * W;
  if (total <= 0) return;
  hipLaunchKernelGGL(replicate_rows_kernel, dim3((unsigned)ceil_div(total, 256)), dim3(256), 0, st,
                     src, dst, G, S, P, W, maxSrc, maxDst, total);
  GN_HIP(hipGetLastError());
}

}  // namespace gn
