// gn_attention.hip - causal (sliding-window) attention for the RL step.
//
//  * decode: one new query per row against the KV cache.  Memory-bound: the
//    grid is (row, kv-head) x splits of up to 256 keys, so K/V are read once
//    for all query heads of the GQA group; a combine kernel merges splits
//    when a window needs more than one (model/attention.go:332-387 split-K,
//    with the window applied by skipping keys the reference masks to -1e30,
//    whose softmax weight is exactly zero).
//  * training/prefill: flash-attention forward with the log-sum-exp, and the
//    backward as two kernels (dQ per query block; dK/dV per key block over
//    the whole GQA group), deterministic and atomic-free
//    (kernels/scalar/attention.go:16-49 and 145-205 semantics).
//
// Scores carry no 1/sqrt(D) factor: q and k arrive already multiplied by 1.2
// after their RMSNorm (model/attention.go:252-256).
#include <hip/hip_ext.h>

#include "gn_model.h"

namespace gn {

static constexpr int HD = 128;  // head dim
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v2f __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------------------
// Decode: one block of NW waves per (row, kv-head, split of up to 256 or 512
// keys), in three phases; all r query heads of the GQA group share every K/V
// load.
//  1. Scores.  Lanes form 8 groups of 8; in each step group g of a wave
//     takes one key, and load i of lane part p of the group reads dims
//     [4(p + 8i), 4(p + 8i) + 4) of it: each of the 4 load instructions of a
//     step covers 128 contiguous bytes of each of 8 whole K rows (one cache
//     line per row, as the P.V loads do), and a step reads the 8 rows whole.
//     An 8-lane reduction gives the r scores, kept in LDS.  Each wave
//     streams a contiguous 1/NW of the split with two steps of K rows in
//     flight.
//  2. Softmax over the split: each wave reduces the block max per head from
//     LDS itself (DPP + readlane, no cross-wave exchange), the owner thread
//     of a key writes p = exp(s - max) back over the score, per-wave sums of
//     p are added at the end; two barriers.
//  3. P.V: thread t reads float4 (t mod 32) of V rows j = t/32 + 2*NW*i,
//     i.e. two whole rows per wave instruction, and accumulates p[h][j] *
//     V[j] for every head; the 2*NW row groups are added in LDS.  The first
//     VP rows per thread are requested right after the first K steps, the
//     rest double-buffered.
// A short split (the 129-key sliding windows) gives one block per (row,
// kv-head) and only 2 blocks per CU, so the waves per block set how many
// loads a CU keeps in flight: r <= 3 runs 8 waves (<= 128 VGPRs, two blocks
// per CU); larger r keep 4 waves to bound registers.  Measured on d12
// shapes: 8 waves beat 4 on long windows (512 keys: 5.6 vs 5.4 TB/s) and
// tie on short ones; deeper per-wave queues at 4 waves (every K and V byte
// of a 129-key split requested before the first wait, 219 VGPRs) were 8 %
// slower; spreading a step's K loads over whole 128-byte lines (instead of
// 64 bytes per lane) gained 3 %.  Per-block phase timestamps (cold caches,
// 129 keys) put ~2 us of the former four-barrier shuffle softmax on every
// block's critical path after its last K row arrived; the present phase 2
// removes most of it (18.2 -> 17.1 us).  The rest of the gap to a plain
// streaming read of the same bytes on the same grid (13.4 us) is the VALU
// work of fp32 attention (768 FMAs per key and block plus reductions, ~4
// cycles per wave instruction) landing after the last rows arrive: variants
// that request every K and V byte up front (16 or 32 lanes per key), that
// keep per-half-wave softmax states merged once, or that stream K and V in
// one online-softmax pass all measured 16.7-18.6 us.
// With the q/k/v post-processing fused in, the position's own key and value
// (the last key of the last split) are not read from the cache: the block
// computes them into LDS, scores that key in one extra step of the last
// wave and adds that value row last, then writes both cache rows at its
// end.  The cached keys split evenly over the waves (a 129-key window: 16
// per wave, every K row requested before the first wait; before, 17 per
// wave left one load behind the first step): d12 in place, 18.7 -> 18.2 us
// per 129-key call, 41.5 -> 41.1 us on the full-context layers.  Copying V
// rows 64..127 into LDS with global_load_lds at the start (so no V load is
// left for phase 3) measured slower, 19.2 us.
// One split covering the whole window writes the normalized output; several
// splits write (unnormalized output, max, sum) for decode_combine_kernel.
// ---------------------------------------------------------------------------
// Keys per split: at most DEC_KPS, balanced (300 keys -> 2 x 150), or up to
// DEC_KPS_WIDE when the (row, kv-head) blocks alone already give two blocks
// per CU (rows * Hkv >= DEC_WIDE_BLOCKS, plain windows): a 257-528-key window
// then runs as one block per (row, kv-head) with no combine pass (d12 full
// layer, 384 keys: 37-40 us against 46.6 us as 2 splits + combine; 512 keys:
// 49 vs 57 us).  Smaller splits were measured slower: the combine pass they
// need costs more than the extra workgroups gain.
static constexpr int DEC_KPS = 256;
static constexpr int DEC_KPS_WIDE = 528;  // 512-token windows admit 513 keys
static constexpr int DEC_WIDE_BLOCKS = 512;
static constexpr int DEC_MAXR = 8;   // max GQA ratio
static constexpr int DEC_POST_SPLITS = DECODE_POST_MAX_SPLITS;
// NW waves per block; the V rows of phase 3 are dealt to 2*NW row groups.
template <int R, int NW>
struct DecDepth {
  static constexpr int KD = 2;                // K steps in flight per wave
  static constexpr int VP = NW == 4 ? 8 : 4;  // V rows per thread requested before phase 1
  static constexpr int RS = 2 * NW;           // V row stride between a thread's rows
};
// waves per block for GQA ratio R
template <int R>
struct DecWaves {
  static constexpr int NW = R <= 3 ? 8 : 4;
};

// The key range of the call and its balanced splits (same arithmetic on the
// host for eager launches).
struct DecSplit {
  int kstart, kend, kps, nsplit;
};
__host__ __device__ inline DecSplit dec_split(int kstart, int kend, int kps_max = DEC_KPS) {
  DecSplit d;
  d.kstart = kstart;
  d.kend = kend;
  const int n = kend - kstart;
  const int ns = (n + kps_max - 1) / kps_max;
  d.kps = (n + ns - 1) / ns;
  d.nsplit = (n + d.kps - 1) / d.kps;  // every split non-empty
  return d;
}
__host__ __device__ inline DecSplit dec_empty() {
  DecSplit d;
  d.kstart = d.kend = 0;
  d.kps = 1;
  d.nsplit = 0;
  return d;
}
// The splits of one step: first those of the compressed blocks (ratio > 1),
// then those of the raw keys.
struct DecPlan {
  DecSplit g, l;
  int nsplit;
};
__host__ __device__ inline DecPlan dec_plan_at(const DecodeAttnArgs& a, int pos, int nsel) {
  DecPlan p;
  if (a.ratio > 1) {
    const int count = a.sel ? nsel : pos / a.ratio;
    p.g = count > 0 ? dec_split(0, count) : dec_empty();
    p.l = a.window > 0 ? dec_split(max(0, pos - a.window), pos + 1) : dec_empty();
  } else {
    const int kps = a.split_keys > 0 ? a.split_keys : DEC_KPS;
    p.g = dec_empty();
    p.l = a.pos_dev ? dec_split(max(0, pos - a.window), pos + 1, kps)
                    : dec_split(a.kstart, a.kend, kps);
  }
  p.nsplit = p.g.nsplit + p.l.nsplit;
  return p;
}
// bk = row * Hkv + kv-head (sparse selection counts are per row and head)
__device__ __forceinline__ DecPlan dec_plan(const DecodeAttnArgs& a, int bk) {
  return dec_plan_at(a, a.pos_dev ? *a.pos_dev : a.kend - 1, a.sel ? a.nsel[bk] : 0);
}

__device__ __forceinline__ float red8_sum(float v) { return sum8_dpp(v); }
__device__ __forceinline__ float readlane_f(float v, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}
// Wave-uniform maximum / sum of the 64 lanes without LDS round trips: a
// 16-lane DPP reduction, then the four row results by readlane (a shuffle
// butterfly is six dependent ds_bpermute/swizzle steps).  Every lane of the
// wave must be active.
__device__ __forceinline__ float wave_max_bcast(float v) {
  v = max16_dpp(v);
  return fmaxf(fmaxf(readlane_f(v, 0), readlane_f(v, 16)), fmaxf(readlane_f(v, 32), readlane_f(v, 48)));
}
__device__ __forceinline__ float wave_sum_bcast(float v) {
  v = sum16_dpp(v);
  return (readlane_f(v, 0) + readlane_f(v, 16)) + (readlane_f(v, 32) + readlane_f(v, 48));
}

// Fused q/k/v post-processing of one block's heads (fuse_post): wave w takes
// heads w, w + NW, ... of the R query heads, the key head (R) and the value
// head (R + 1) of kv-head hk; a lane holds dims lane and lane + 64.  The
// arithmetic is qkv_post_kernel's (split partials summed in float64 in split
// order, the VE gate's butterfly sum, the rotation and the norm as written
// there), so fused and separate launches give the same bits.
template <int R, int NW>
struct DecPost {
  static constexpr int HPW = (R + 2 + NW - 1) / NW;  // heads per wave
  static constexpr int FZ = DEC_POST_SPLITS;         // partials loaded per element
  float v[HPW][2][FZ];                               // raw values / partials
  float cv[2], sv[2];                                // RoPE entries of the lane's dims
  float hv, wv, ve[2];                               // VE gate inputs, the token's VE row

  __device__ __forceinline__ static int col(const QkvPostArgs& p, int hk, int hd) {
    return hd < R ? (hk * R + hd) * HD : hd == R ? (p.Hq + hk) * HD : (p.Hq + p.Hkv + hk) * HD;
  }
  // Every load of the prologue, issued before the attention's own loads and
  // without branches: the token id (the one dependent address) first, then
  // FZ partials per element at clamped split indices (the sum uses the
  // first `splits`), the RoPE entries and the VE inputs.
  __device__ __forceinline__ void load(const QkvPostArgs& p, int row, int hk, int pos, int wid,
                                       int lane) {
    const int vid = p.ve ? p.ids[row] : 0;
    const int64_t rbase = (int64_t)row * (p.Hq + 2 * p.Hkv) * HD;
    const PendingSum& ps = p.qkv_sum;
    const float* src = ps.splits > 0 ? ps.part : p.qkv;
    const int zmax = ps.splits > 0 ? ps.splits - 1 : 0;
#pragma unroll
    for (int u = 0; u < HPW; u++) {
      const int hd = min(wid + NW * u, R + 1);
#pragma unroll
      for (int e = 0; e < 2; e++) {
        const int64_t i = rbase + col(p, hk, hd) + lane + 64 * e;
#pragma unroll
        for (int z = 0; z < FZ; z++) v[u][e][z] = src[min(z, zmax) * ps.stride + i];
      }
    }
    const int half = p.R / 2, off = HD - p.R;
#pragma unroll
    for (int e = 0; e < 2; e++) {
      const int d = lane + 64 * e;
      const int j = max(d - off, 0), jj = j < half ? j : j - half;
      cv[e] = sv[e] = 0.f;
      if (half > 0) {  // uniform
        cv[e] = p.cosT[(int64_t)pos * half + jj];
        sv[e] = p.sinT[(int64_t)pos * half + jj];
      }
    }
    hv = wv = 0.f;
    ve[0] = ve[1] = 0.f;
    if (p.ve) {
      hv = p.h[(int64_t)row * p.C + min(lane, VE_CH - 1)];
      wv = p.wve[hk * VE_CH + min(lane, VE_CH - 1)];
      const float* ver = p.ve + ((int64_t)vid * p.Hkv + hk) * HD;
      ve[0] = ver[lane];
      ve[1] = ver[lane + 64];
    }
  }
  // q heads (rotated, normed, 1.2 x) into out[0..R), the key into out[R], the
  // value into out[R + 1].
  __device__ __forceinline__ void compute(const QkvPostArgs& p, float (*out)[HD], int wid,
                                          int lane) {
    const int half = p.R / 2, off = HD - p.R;
#pragma unroll
    for (int u = 0; u < HPW; u++) {
      const int hd = wid + NW * u;
      if (hd >= R + 2) continue;  // wave-uniform
      float x[2];
#pragma unroll
      for (int e = 0; e < 2; e++) {
        if (p.qkv_sum.splits > 0) {
          double sum = 0.0;
#pragma unroll
          for (int z = 0; z < FZ; z++)
            if (z < p.qkv_sum.splits) sum += (double)v[u][e][z];
          x[e] = (float)sum;
        } else {
          x[e] = v[u][e][0];
        }
      }
      if (hd == R + 1) {  // v += gate * ve[id] (attention.go:247-248, 392-405)
        if (p.ve) {
          const float g = warp_sum(lane < VE_CH ? hv * wv : 0.f);
          const float gate = sigmoidf_(g) * VE_SCALE;
#pragma unroll
          for (int e = 0; e < 2; e++) x[e] += gate * ve[e];
        }
#pragma unroll
        for (int e = 0; e < 2; e++) out[hd][lane + 64 * e] = x[e];
        continue;
      }
      // rotate the trailing R dims (partners through LDS, this wave's own row)
      out[hd][lane] = x[0];
      out[hd][lane + 64] = x[1];
      float y[2];
#pragma unroll
      for (int e = 0; e < 2; e++) {
        const int d = lane + 64 * e;
        float t = out[hd][d];
        if (d >= off) {
          const int j = d - off;
          if (j < half) t = out[hd][d] * cv[e] + out[hd][d + half] * sv[e];
          else t = -out[hd][d - half] * sv[e] + out[hd][d] * cv[e];
        }
        y[e] = t;
      }
      const float ss = warp_sum(y[0] * y[0] + y[1] * y[1]);
      const float inv = 1.f / sqrtf(ss / (float)HD + NORM_EPS);
#pragma unroll
      for (int e = 0; e < 2; e++) {
        out[hd][lane + 64 * e] = y[e] * inv * QK_SCALE;
      }
    }
  }
};

template <int R, int NW, bool FUSE>
__device__ __forceinline__ void decode_attn_body(const DecodeAttnArgs& a) {
  constexpr int NT = 64 * NW;
  constexpr int KD = DecDepth<R, NW>::KD, VP = DecDepth<R, NW>::VP, RS = DecDepth<R, NW>::RS;
  __shared__ float sc[R][DEC_KPS_WIDE];
  __shared__ __attribute__((aligned(16))) float pv[RS][R][HD];
  __shared__ float wred[NW][R];  // per-wave sums of p
  // fused post-processing: q heads, the new key, the new value
  __shared__ __attribute__((aligned(16))) float post[FUSE ? R + 2 : 1][HD];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int bh = blockIdx.x, s = blockIdx.y;
  const DecPlan pl = dec_plan(a, bh);
  if (s >= pl.nsplit) return;  // graph launches size the grid for the longest window
  const int row = bh / a.Hkv, hk = bh % a.Hkv;
  const bool glob = s < pl.g.nsplit;  // a split of compressed blocks
  const DecSplit& sp = glob ? pl.g : pl.l;
  const int ks = sp.kstart + (glob ? s : s - pl.g.nsplit) * sp.kps;
  const int nk = min(sp.kend, ks + sp.kps) - ks;
  const float* kbase = glob ? a.ck : a.kc;
  const float* vbase = glob ? a.cv : a.vc;
  const int64_t cbase = ((int64_t)row * a.Hkv + hk) * (glob ? a.maxBlocks : a.maxSeq) + ks;
  // key j of the split is row (cbase + j), or a gathered block of the selection
  const int* gsel = (glob && a.sel) ? a.sel + (int64_t)bh * a.kcap + ks : nullptr;
  const int64_t gbase = cbase - ks;
  auto krow = [&](int j) -> int64_t { return gsel ? gbase + gsel[j] : cbase + j; };
  // fused: the query position's key is key jn of this split (-1: another
  // split's); the cache holds it only after this block writes it, so the
  // scores and P.V take it from `post`
  int jn = -1, qpos = 0;
  DecPost<R, NW> dp;
  if constexpr (FUSE) {
    qpos = a.pos_dev ? *a.pos_dev : a.kend - 1;
    jn = qpos - ks < nk ? qpos - ks : -1;
    dp.load(a.post, row, hk, qpos, wid, lane);
    __builtin_amdgcn_sched_barrier(0);
  }
  // keys [0, nc) come from the cache; the position's own key, the last of
  // its split, is taken from `post` (not loaded)
  const int nc = jn >= 0 ? nk - 1 : nk;

  const int d4 = tid & 31, jr = tid >> 5;
  const v4f* vrow = reinterpret_cast<const v4f*>(vbase) + d4;
  v4f vpre[VP];

  // ---- phase 1: scores
  {
    const int g = lane >> 3, part = lane & 7;
    float qv[R][16];
    auto read_q = [&](const float* qrow) {
#pragma unroll
      for (int h = 0; h < R; h++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const v4f t = *reinterpret_cast<const v4f*>(qrow + h * HD + 32 * i);
          qv[h][4 * i] = t[0];
          qv[h][4 * i + 1] = t[1];
          qv[h][4 * i + 2] = t[2];
          qv[h][4 * i + 3] = t[3];
        }
    };
    if constexpr (!FUSE) read_q(a.q + ((int64_t)row * a.Hq + hk * R) * HD + 4 * part);
    const int qw = (nc + NW - 1) / NW;
    const int j0 = wid * qw, j1 = min(nc, j0 + qw);
    const v4f* kb = reinterpret_cast<const v4f*>(kbase + 4 * part);
    auto load = [&](int j, v4f* kd) {
      const int jj = j < j1 ? j : j0;  // clamp (value unused when j >= j1)
      const int64_t r = krow(jj) * (HD / 4);
#pragma unroll
      for (int i = 0; i < 4; i++) kd[i] = kb[r + 8 * i];
    };
    // the first KD steps of K, then the V rows of phase 3 (loads complete in
    // issue order, so the K rows the loop needs first are queued first)
    v4f kr[KD][4];
#pragma unroll
    for (int t = 0; t < KD; t++)
      if (j0 + 8 * t < j1) load(j0 + 8 * t + g, kr[t]);
#pragma unroll
    for (int i = 0; i < VP; i++) {
      const int j = jr + RS * i;
      vpre[i] = vrow[krow(j < nc ? j : 0) * (HD / 4)];
    }
    if constexpr (FUSE) {
      __builtin_amdgcn_sched_barrier(0);
      // the new key and value stay in `post` until the end, where they are
      // written to the cache rows of the position
      dp.compute(a.post, post, wid, lane);
      __syncthreads();
      read_q(&post[0][4 * part]);
    }
    // the R scores of the key whose row k holds (8-lane group sums), and
    // their store for key j = jc + g when j < jend
    auto dots = [&](const v4f* k, float* d) {
#pragma unroll
      for (int h = 0; h < R; h++) {
        float x = 0.f;
#pragma unroll
        for (int i = 0; i < 4; i++)
          x += k[i][0] * qv[h][4 * i] + k[i][1] * qv[h][4 * i + 1] + k[i][2] * qv[h][4 * i + 2] +
               k[i][3] * qv[h][4 * i + 3];
        d[h] = red8_sum(x);
      }
    };
    auto store = [&](const float* d, int jc, int jend) {
      const int j = jc + g;
      if (part == 0 && j < jend)
#pragma unroll
        for (int h = 0; h < R; h++) sc[h][j] = d[h];
    };
    for (int jb = j0; jb < j1; jb += 8 * KD) {
#pragma unroll
      for (int t = 0; t < KD; t++) {
        const int jc = jb + 8 * t;  // wave-uniform
        if (jc < j1) {
          float d[R];
          dots(kr[t], d);
          if (jc + 8 * KD < j1) load(jc + 8 * KD + g, kr[t]);
          store(d, jc, j1);
        }
      }
    }
    // the position's own key: group 0 of the last wave (the same arithmetic
    // as a cached key's)
    if (FUSE && jn >= 0 && wid == NW - 1) {
#pragma unroll
      for (int i = 0; i < 4; i++) kr[0][i] = *reinterpret_cast<const v4f*>(&post[R][4 * (part + 8 * i)]);
      float d[R];
      dots(kr[0], d);
      store(d, jn, g == 0 ? jn + 1 : jn);
    }
  }
  __syncthreads();

  // ---- phase 2: softmax over the split.  Every wave takes the block
  // maximum itself from the scores in LDS, so no wave waits on another for
  // it; the thread owning key j writes p = exp(s - max) back over the score;
  // the per-wave sums of p are added at the end.  (The former version, a
  // shuffle-butterfly max and sum per wave merged through LDS over four
  // barriers, cost ~2 us per block on the critical path.)
  float mx[R];
#pragma unroll
  for (int h = 0; h < R; h++) {
    float m = -INFINITY;
#pragma unroll
    for (int k = 0; k < (DEC_KPS_WIDE + 63) / 64; k++)
      if (64 * k < nk) {  // wave-uniform
        const int j = lane + 64 * k;
        if (j < nk) m = fmaxf(m, sc[h][j]);
      }
    mx[h] = wave_max_bcast(m);
  }
  __syncthreads();  // every wave has read the scores before p overwrites them
  {
    float ps[R];
#pragma unroll
    for (int h = 0; h < R; h++) ps[h] = 0.f;
    for (int j = tid; j < nk; j += NT)
#pragma unroll
      for (int h = 0; h < R; h++) {
        const float p = expf(sc[h][j] - mx[h]);
        sc[h][j] = p;
        ps[h] += p;
      }
#pragma unroll
    for (int h = 0; h < R; h++) {
      const float t = wave_sum_bcast(ps[h]);
      if (lane == 0) wred[wid][h] = t;
    }
  }
  __syncthreads();

  // ---- phase 3: P.V
  float acc[R][4];
#pragma unroll
  for (int h = 0; h < R; h++)
#pragma unroll
    for (int c = 0; c < 4; c++) acc[h][c] = 0.f;
  // every thread adds its rows jr, jr + RS, ... in increasing order
  auto accumulate = [&](int j, const v4f& vv) {
#pragma unroll
    for (int h = 0; h < R; h++) {
      const float p = sc[h][j];
#pragma unroll
      for (int c = 0; c < 4; c++) acc[h][c] += p * vv[c];
    }
  };
#pragma unroll
  for (int i = 0; i < VP; i++)
    if (jr + RS * i < nc) accumulate(jr + RS * i, vpre[i]);
  if (RS * VP < nc) {  // block-uniform: the rest of a long split, two sets of 4 rows in flight
    auto load4 = [&](int j, v4f* vv) {
#pragma unroll
      for (int u = 0; u < 4; u++) {
        const int jj = j + RS * u;
        vv[u] = vrow[krow(jj < nc ? jj : 0) * (HD / 4)];
      }
    };
    auto acc4 = [&](int j, const v4f* vv) {
#pragma unroll
      for (int u = 0; u < 4; u++)
        if (j + RS * u < nc) accumulate(j + RS * u, vv[u]);
    };
    v4f va[4], vb[4];
    int jb = jr + RS * VP;
    load4(jb, va);
    for (; jb < nc; jb += 8 * RS) {
      if (jb + 4 * RS < nc) load4(jb + 4 * RS, vb);
      acc4(jb, va);
      if (jb + 4 * RS >= nc) break;
      if (jb + 8 * RS < nc) load4(jb + 8 * RS, va);
      acc4(jb + 4 * RS, vb);
    }
  }
  // the position's own value row, the last row of its thread
  if (FUSE && jn >= 0 && jr == jn % RS)
    accumulate(jn, *reinterpret_cast<const v4f*>(&post[R + 1][4 * d4]));
#pragma unroll
  for (int h = 0; h < R; h++)
    *reinterpret_cast<v4f*>(&pv[jr][h][4 * d4]) = (v4f){acc[h][0], acc[h][1], acc[h][2], acc[h][3]};
  __syncthreads();
  const bool whole = pl.nsplit == 1;
  float* out = a.part + ((int64_t)bh * a.nsplit_max + s) * R * (HD + 2);
  for (int i = tid; i < R * HD; i += NT) {
    const int h = i / HD, dd = i % HD;
    float o = 0.f;
#pragma unroll
    for (int r = 0; r < RS; r++) o += pv[r][h][dd];
    float l = 0.f;
#pragma unroll
    for (int w = 0; w < NW; w++) l += wred[w][h];
    if (whole) {
      a.o[((int64_t)row * a.Hq + hk * R + h) * HD + dd] = o / l;
    } else {
      out[h * (HD + 2) + dd] = o;
      if (dd == 0) {
        out[h * (HD + 2) + HD] = mx[h];
        out[h * (HD + 2) + HD + 1] = l;
      }
    }
  }
  // the cache rows of the position are this block's to write (this layer's
  // attention took them from `post`)
  if (FUSE && jn >= 0) {
    const int64_t crow = ((int64_t)row * a.Hkv + hk) * a.maxSeq + qpos;
    for (int i = tid; i < 2 * HD; i += NT) {
      float* c = const_cast<float*>(i < HD ? a.kc : a.vc);
      c[crow * HD + i % HD] = post[R + i / HD][i % HD];
    }
  }
}

// One kernel per GQA ratio R, so each instance is sized (registers, LDS) for
// its own R rather than for the largest.
template <int R, int NW, bool FUSE>
__global__ __launch_bounds__(64 * NW) void decode_attn_kernel(DecodeAttnArgs a) {
  decode_attn_body<R, NW, FUSE>(a);
}
template <int R, bool FUSE>
static void launch_decode_attn_f(dim3 grid, hipStream_t st, const DecodeAttnArgs& a,
                                 hipEvent_t stop) {
  constexpr int NW = DecWaves<R>::NW;
  if (a.t_start || stop)
    hipExtLaunchKernelGGL((decode_attn_kernel<R, NW, FUSE>), grid, dim3(64 * NW), 0, st,
                          a.t_start, stop, 0, a);
  else
    hipLaunchKernelGGL((decode_attn_kernel<R, NW, FUSE>), grid, dim3(64 * NW), 0, st, a);
}
template <int R>
static void launch_decode_attn(dim3 grid, hipStream_t st, const DecodeAttnArgs& a,
                               hipEvent_t stop) {
  if (a.fuse_post) launch_decode_attn_f<R, true>(grid, st, a, stop);
  else launch_decode_attn_f<R, false>(grid, st, a, stop);
}

__global__ __launch_bounds__(128) void decode_combine_kernel(DecodeAttnArgs a) {
  const int rq = blockIdx.x;  // row * Hq + qh
  const DecPlan pl = dec_plan(a, (rq / a.Hq) * a.Hkv + (rq % a.Hq) / (a.Hq / a.Hkv));
  if (pl.nsplit == 1) return;  // the attention kernel wrote the output
  if (pl.nsplit == 0) {  // compressed attention with nothing visible yet
    a.o[(int64_t)rq * HD + threadIdx.x] = 0.f;
    return;
  }
  const int row = rq / a.Hq, qh = rq % a.Hq;
  const int r = a.Hq / a.Hkv;
  const int hk = qh / r, h = qh % r;
  const float* base =
      a.part + ((int64_t)(row * a.Hkv + hk) * a.nsplit_max) * r * (HD + 2) + h * (HD + 2);
  const int64_t stride = (int64_t)r * (HD + 2);
  float gm = -INFINITY;
  for (int s = 0; s < pl.nsplit; s++) gm = fmaxf(gm, base[s * stride + HD]);
  float total = 0.f, o = 0.f;
  for (int s = 0; s < pl.nsplit; s++) {
    float sc = expf(base[s * stride + HD] - gm);
    total += base[s * stride + HD + 1] * sc;
    o += base[s * stride + threadIdx.x] * sc;
  }
  a.o[(int64_t)rq * HD + threadIdx.x] = o / total;
}

static int decode_attention_max_splits(int window, int maxSeq, int kps = DEC_KPS) {
  return dec_split(0, std::min(window + 1, maxSeq), kps).nsplit;
}

int decode_attention_split_cap(const DecodeAttnArgs& a) {
  if (a.ratio > 1) {
    int n = a.sel ? 1 : a.maxBlocks > 0 ? dec_split(0, a.maxBlocks).nsplit : 0;
    if (a.window > 0) n += decode_attention_max_splits(a.window, a.maxSeq);
    return std::max(n, 1);
  }
  return decode_attention_max_splits(std::max(a.window, 0), a.maxSeq);
}

void launch_decode_attention(DecodeAttnArgs a, hipStream_t st) {
  GN_CHECK(a.Hq % a.Hkv == 0 && a.Hq / a.Hkv <= DEC_MAXR, "decode attention: GQA ratio must be <= 8");
  if (a.fuse_post) {
    const QkvPostArgs& p = a.post;
    GN_CHECK(a.ratio <= 1 && !a.sel && p.Hq == a.Hq && p.Hkv == a.Hkv && p.T == 1 &&
                 p.R % 2 == 0 && p.R <= HD && p.cosT && p.sinT && (p.qkv || p.qkv_sum.splits > 0) &&
                 (!p.ve || (p.h && p.ids && p.wve)),
             "decode attention: bad fused q/k/v arguments");
    GN_CHECK(p.qkv_sum.splits == 0 ||
                 (p.qkv_sum.stride == (int64_t)a.rows * (p.Hq + 2 * p.Hkv) * HD &&
                  p.qkv_sum.splits <= DEC_POST_SPLITS),
             "decode attention: fused q/k/v pending sum shape");
  }
  // wide splits only when the (row, kv-head) blocks fill the CUs on their own
  a.split_keys = a.ratio <= 1 && (int64_t)a.rows * a.Hkv >= DEC_WIDE_BLOCKS ? DEC_KPS_WIDE : DEC_KPS;
  bool combine;
  if (a.ratio > 1) {
    GN_CHECK(a.ck && a.cv && a.maxBlocks > 0 && a.window >= 0, "decode attention: bad compressed cache");
    GN_CHECK(!a.sel || (a.nsel && a.kcap >= 1 && a.kcap <= DEC_KPS), "decode attention: bad selection");
    if (a.pos_dev || a.sel) {
      a.nsplit_max = decode_attention_split_cap(a);
    } else {
      GN_CHECK(a.kend >= 1 && a.kend <= a.maxSeq && (a.kend - 1) / a.ratio <= a.maxBlocks,
               "decode attention: position outside the caches");
      a.nsplit_max = std::max(dec_plan_at(a, a.kend - 1, 0).nsplit, 1);
    }
    combine = true;  // also writes the zero output of a step with no visible key
  } else if (a.pos_dev) {
    // position read on the device: size for the longest key range
    GN_CHECK(a.window >= 0, "decode attention: bad window");
    a.nsplit_max = decode_attention_max_splits(a.window, a.maxSeq, a.split_keys);
    combine = a.nsplit_max > 1;
  } else {
    GN_CHECK(a.kend > a.kstart, "decode attention: empty key range");
    a.nsplit_max = dec_split(a.kstart, a.kend, a.split_keys).nsplit;
    combine = a.nsplit_max > 1;
  }
  // every block that does not cover its whole key range writes its split's
  // partial at (row * Hkv + kv-head, split) with stride nsplit_max
  GN_CHECK(a.nsplit_max <= 1 ||
               (a.part && (int64_t)a.rows * a.Hkv * a.nsplit_max * (a.Hq / a.Hkv) * (HD + 2) <=
                              a.part_floats),
           "decode attention: the split partial buffer is too small for this key range");
  const dim3 grid(a.rows * a.Hkv, a.nsplit_max);
  hipEvent_t stop = combine ? nullptr : a.t_stop;
  switch (a.Hq / a.Hkv) {
    case 1: launch_decode_attn<1>(grid, st, a, stop); break;
    case 2: launch_decode_attn<2>(grid, st, a, stop); break;
    case 3: launch_decode_attn<3>(grid, st, a, stop); break;
    case 4: launch_decode_attn<4>(grid, st, a, stop); break;
    case 5: launch_decode_attn<5>(grid, st, a, stop); break;
    case 6: launch_decode_attn<6>(grid, st, a, stop); break;
    case 7: launch_decode_attn<7>(grid, st, a, stop); break;
    case 8: launch_decode_attn<8>(grid, st, a, stop); break;
  }
  GN_HIP(hipGetLastError());
  if (!combine) return;
  if (a.t_stop)
    hipExtLaunchKernelGGL(decode_combine_kernel, dim3(a.rows * a.Hq), dim3(HD), 0, st, nullptr,
                          a.t_stop, 0, a);
  else
    hipLaunchKernelGGL(decode_combine_kernel, dim3(a.rows * a.Hq), dim3(HD), 0, st, a);
  GN_HIP(hipGetLastError());
}

// Key kj is visible from query t: causal, inside the sliding window (a
// window w admits w + 1 keys, kernels/scalar/attention.go:210-228).
__device__ __forceinline__ bool key_valid(int kj, int t, int T, int window) {
  return kj < T && kj <= t && (window < 0 || t - kj <= window);
}
// The flash kernels' mask: causal/windowed keys, or compressed blocks that
// ended before the query's block (ratio > 1).  Query t sits at position
// t + qoff: a forward that continues a cached prefix of qoff tokens attends
// keys [0, qoff + T) with its queries at the end.
__device__ __forceinline__ bool key_ok(int kj, int t, int Tk, int ratio, int window, int qoff) {
  if (ratio > 1) return kj < Tk && (kj + 1) * ratio <= t + qoff;
  return key_valid(kj, t + qoff, Tk, window);
}
// Key tiles a query block [q0, qlast] needs: [kbeg, kend).
__device__ __forceinline__ void key_range(int q0, int qlast, int Tk, int ratio, int window,
                                          int qoff, int* kbeg, int* kend) {
  if (ratio > 1) {
    *kbeg = 0;
    *kend = min(Tk, (qlast + qoff) / ratio);
  } else {
    *kbeg = window >= 0 ? max(0, q0 + qoff - window) : 0;
    *kend = min(Tk, qlast + qoff + 1);
  }
}

// ---------------------------------------------------------------------------
// Flash attention on the matrix cores (training forward, prefill, backward).
//
// Operand tiles of FS rows x 128 dims (keys, or queries for dK/dV) go from
// global memory straight into a two-stage LDS ring (global_load_lds_dwordx4,
// no VGPR staging; the next tile is in flight while the current one is
// multiplied, one barrier per tile).  A tile row is 32 16-byte slots, the
// slot column XOR-swizzled by (row & 15), so both ways the kernels read it
// are conflict-free ds_read_b128:
//  * row fragments: 16 rows at one slot column (lane (l16, g) reads row
//    R0 + l16, dims 4(4s + g) .. + 3) -- the A operand of S^T = K.Q^T,
//    dP^T = V.dO^T, S = Q.K^T, dP = dO.V^T;
//  * column fragments: one row, 16 consecutive slots (lane (l16, g) reads
//    row R, dims 4(16gi + l16) .. + 3) -- the A operand of O^T += V^T.P^T,
//    dQ^T += K^T.dS^T, dV^T += dO^T.P, dK^T += Q^T.dS.  Component cc of the
//    read feeds output block (gi, cc), whose row i is dim 64 gi + 4 i + cc,
//    so a lane's accumulator (gi, cc) register r holds dim 64 gi + 16 g +
//    4 r + cc: for fixed (gi, r) the four blocks give four consecutive dims,
//    stored as one 16-byte vector.
// Rows past the operand's end are clamped to its last row (finite values
// whose products the mask zeroes).  k order inside a 16-row block: MFMA c
// takes row 4 (lane >> 4) + c, where the S^T / S accumulators leave it.
// ---------------------------------------------------------------------------
static constexpr int FQ = 64;  // queries per forward / dQ block
static constexpr int FK = 64;  // keys per dK/dV block
static constexpr int FS = 32;  // rows per LDS stage

__device__ __forceinline__ void fl_barrier() {
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}
__device__ __forceinline__ void fl_wait_all() {
  __builtin_amdgcn_s_waitcnt((0) | (7 << 4) | (0 << 8));  // vmcnt(0) expcnt(7) lgkmcnt(0)
}

typedef __attribute__((address_space(3))) void fl_lds_void;

// FS rows into stage S by 256 threads: instruction t of wave w fills slots
// (4t + w) 64 .. + 63, i.e. rows 2(4t + w) + (lane >> 5), physical slot
// lane & 31 holding logical slot (lane & 31) ^ (row & 15).  rowptr(r) is
// the first float of tile row r (already clamped).
template <class RowPtr>
__device__ __forceinline__ void fl_stage_load(float* S, RowPtr rowptr, int w, int lane) {
#pragma unroll
  for (int t = 0; t < 4; t++) {
    const int row = 2 * (4 * t + w) + (lane >> 5);
    const int slot = (lane & 31) ^ (row & 15);
    __builtin_amdgcn_global_load_lds((const void*)(rowptr(row) + 4 * slot),
                                     (fl_lds_void*)(S + 4 * ((4 * t + w) * 64)), 16, 0, 0);
  }
}
// Row fragment: row r0 + l16 (r0 % 16 == 0), logical slot 4s + g.
__device__ __forceinline__ v4f fl_row(const float* S, int r0, int s, int l16, int g) {
  return *reinterpret_cast<const v4f*>(&S[(r0 + l16) * HD + 4 * ((4 * s + g) ^ l16)]);
}
// Column fragment: row r, logical slot 16 gi + l16.
__device__ __forceinline__ v4f fl_col(const float* S, int r, int gi, int l16) {
  return *reinterpret_cast<const v4f*>(&S[r * HD + 4 * ((16 * gi + l16) ^ (r & 15))]);
}
// Store a column-fragment accumulator [2][4] of one lane's row at p (the
// row's first dim): dims 64 gi + 16 g + 4 r + cc; add: p[] += acc.
__device__ __forceinline__ void fl_store_cols(float* p, const v4f (&acc)[2][4], int g, bool add,
                                              float scale) {
#pragma unroll
  for (int gi = 0; gi < 2; gi++)
#pragma unroll
    for (int r = 0; r < 4; r++) {
      v4f v = {acc[gi][0][r], acc[gi][1][r], acc[gi][2][r], acc[gi][3][r]};
      float* q = p + 64 * gi + 16 * g + 4 * r;
      v = v * scale;
      if (add) v = *reinterpret_cast<const v4f*>(q) + v;
      *reinterpret_cast<v4f*>(q) = v;
    }
}

// Forward.  Block: 4 waves x 16 queries of one (sequence, query head); each
// wave computes S^T = K.Q^T and O^T += V^T.P^T, a lane's column being its
// query (lane & 15): the running max, the sum and the O rescale stay in the
// lane, and its P values are the B operand of the second product directly.
__global__ __launch_bounds__(256, 2) void flash_fwd_mfma_kernel(FlashArgs a) {
  __shared__ __attribute__((aligned(16))) float Ks0[FS * HD];
  __shared__ __attribute__((aligned(16))) float Vs0[FS * HD];
  __shared__ __attribute__((aligned(16))) float Ks1[FS * HD];
  __shared__ __attribute__((aligned(16))) float Vs1[FS * HD];
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, g = lane >> 4;
  const int q0 = blockIdx.x * FQ;
  const int bh = blockIdx.y, b = bh / a.Hq, qh = bh % a.Hq;
  const int hk = qh / (a.Hq / a.Hkv);
  const int t = q0 + 16 * w + l16;  // this lane's query
  const bool active = t < a.T;

  // Q^T fragments: lane holds Q[t][16s + 4g .. +3], s = 0..7
  v4f qf[8];
  {
    const float* qp = a.q + (((int64_t)b * a.T + min(t, a.T - 1)) * a.Hq + qh) * HD + 4 * g;
#pragma unroll
    for (int s = 0; s < 8; s++) qf[s] = *reinterpret_cast<const v4f*>(qp + 16 * s);
  }
  v4f acc[2][4];  // O^T, column-fragment layout
#pragma unroll
  for (int gi = 0; gi < 2; gi++)
#pragma unroll
    for (int cc = 0; cc < 4; cc++) acc[gi][cc] = (v4f){0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, l = 0.f;

  const int qlast = min(a.T, q0 + FQ) - 1;
  int kmin, kmax;
  key_range(q0, qlast, a.Tk, a.ratio, a.window, a.qoff, &kmin, &kmax);
  const int kt0 = (kmin / FS) * FS;
  const int ntile = kmax > kt0 ? (kmax - kt0 + FS - 1) / FS : 0;
  const float* kbase = a.k + ((int64_t)b * a.Tk * a.Hkv + hk) * HD;
  const float* vbase = a.v + ((int64_t)b * a.Tk * a.Hkv + hk) * HD;
  const int64_t kvstride = (int64_t)a.Hkv * HD;
  auto load = [&](int i, float* KS, float* VS) {
    const int kt = kt0 + i * FS;
    fl_stage_load(KS, [&](int r) { return kbase + min(kt + r, a.Tk - 1) * kvstride; }, w, lane);
    fl_stage_load(VS, [&](int r) { return vbase + min(kt + r, a.Tk - 1) * kvstride; }, w, lane);
  };
  auto tile = [&](int i, const float* KS, const float* VS, float* XK, float* XV) {
    fl_wait_all();  // tile i (the only loads in flight) landed
    fl_barrier();   // ... for every wave; the other stage is no longer read
    if (i + 1 < ntile) load(i + 1, XK, XV);
    const int kt = kt0 + i * FS;
    v4f st[FS / 16];  // S^T[kt + 16kb + 4g + r][t]
#pragma unroll
    for (int kb = 0; kb < FS / 16; kb++) {
      st[kb] = (v4f){0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 8; s++) {
        const v4f kf = fl_row(KS, 16 * kb, s, l16, g);
#pragma unroll
        for (int c = 0; c < 4; c++)
          st[kb] = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[c], qf[s][c], st[kb], 0, 0, 0);
      }
    }
    // mask, online softmax (the lane's column is query t)
    float tmax = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < FS / 16; kb++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int kj = kt + 16 * kb + 4 * g + r;
        if (!key_ok(kj, t, a.Tk, a.ratio, a.window, a.qoff)) st[kb][r] = -INFINITY;
        tmax = fmaxf(tmax, st[kb][r]);
      }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
    if (tmax > -INFINITY) {  // uniform over the 4 lanes of a query
      const float mn = fmaxf(m, tmax);
      const float sc = expf(m - mn);  // 0 while m is -inf
      float ps = 0.f;
#pragma unroll
      for (int kb = 0; kb < FS / 16; kb++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const float p = expf(st[kb][r] - mn);  // masked: exp(-inf) = 0
          st[kb][r] = p;
          ps += p;
        }
      ps += __shfl_xor(ps, 16, 64);
      ps += __shfl_xor(ps, 32, 64);
      l = l * sc + ps;
      m = mn;
#pragma unroll
      for (int gi = 0; gi < 2; gi++)
#pragma unroll
        for (int cc = 0; cc < 4; cc++) acc[gi][cc] *= sc;
    } else {
#pragma unroll
      for (int kb = 0; kb < FS / 16; kb++) st[kb] = (v4f){0.f, 0.f, 0.f, 0.f};
    }
    // O^T += V^T P^T
#pragma unroll
    for (int kb = 0; kb < FS / 16; kb++)
#pragma unroll
      for (int c = 0; c < 4; c++)
#pragma unroll
        for (int gi = 0; gi < 2; gi++) {
          const v4f vf = fl_col(VS, 16 * kb + 4 * g + c, gi, l16);
#pragma unroll
          for (int cc = 0; cc < 4; cc++)
            acc[gi][cc] = __builtin_amdgcn_mfma_f32_16x16x4f32(vf[cc], st[kb][c], acc[gi][cc],
                                                               0, 0, 0);
        }
  };
  if (ntile > 0) load(0, Ks0, Vs0);
  for (int i = 0; i < ntile; i += 2) {
    tile(i, Ks0, Vs0, Ks1, Vs1);
    if (i + 1 < ntile) tile(i + 1, Ks1, Vs1, Ks0, Vs0);
  }
  if (active) {
    // l == 0: no visible key (compressed attention before the first block)
    const float inv = l > 0.f ? 1.f / l : 0.f;
    fl_store_cols(a.o + (((int64_t)b * a.T + t) * a.Hq + qh) * HD, acc, g, false, inv);
    if (a.lse && g == 0)
      a.lse[((int64_t)b * a.T + t) * a.Hq + qh] = l > 0.f ? m + logf(l) : -INFINITY;
  }
}

void launch_flash_fwd(FlashArgs a, hipStream_t st) {
  if (a.Tk <= 0) a.Tk = a.T;
  GN_CHECK(a.ratio <= 1 || a.window < 0, "flash: compressed keys take no window");
  GN_CHECK(a.ratio > 1 || a.qoff + a.T <= a.Tk, "flash: queries past the last key");
  hipLaunchKernelGGL(flash_fwd_mfma_kernel, dim3((unsigned)ceil_div(a.T, FQ), a.B * a.Hq),
                     dim3(256), 0, st, a);
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

// ---------------------------------------------------------------------------
// Flash backward on the matrix cores, deterministic and atomic-free as two
// kernels (kernels/scalar/attention.go:145-205 semantics, from the forward's
// log-sum-exp and delta = rowsum(dO * O)):
//  * dQ: 4 waves x 16 queries per block, keys in tiles of 64.  Per 16-key
//    block a wave forms S^T and dP^T (lane column = its query), dS^T =
//    P^T (dP^T - delta) in the lane, and dQ^T += K^T dS^T.
//  * dK/dV: 4 waves x 16 keys per block, over every query head of the GQA
//    group and query tiles of 64.  Per 16-query block S and dP come out with
//    the lane column = its key, so P and dS feed dV^T += dO^T P and
//    dK^T += Q^T dS as B operands straight from the lane.
// Both use the k order of the forward (k-slot g of MFMA c is element 4g + c
// of a 16 block), so no accumulator is transposed through LDS.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256, 2) void flash_bwd_dq_mfma_kernel(FlashBwdArgs a) {
  __shared__ __attribute__((aligned(16))) float Ks0[FS * HD];
  __shared__ __attribute__((aligned(16))) float Vs0[FS * HD];
  __shared__ __attribute__((aligned(16))) float Ks1[FS * HD];
  __shared__ __attribute__((aligned(16))) float Vs1[FS * HD];
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, g = lane >> 4;
  const int q0 = blockIdx.x * FQ;
  const int bh = blockIdx.y, b = bh / a.Hq, qh = bh % a.Hq;
  const int hk = qh / (a.Hq / a.Hkv);
  const int t = q0 + 16 * w + l16;
  const bool active = t < a.T;
  const int64_t qrow = ((int64_t)b * a.T + min(t, a.T - 1)) * a.Hq + qh;
  v4f qf[8], gf[8];
#pragma unroll
  for (int s = 0; s < 8; s++) {
    qf[s] = *reinterpret_cast<const v4f*>(a.q + qrow * HD + 16 * s + 4 * g);
    gf[s] = *reinterpret_cast<const v4f*>(a.dout + qrow * HD + 16 * s + 4 * g);
  }
  const float lse = a.lse[qrow], dl = a.delta[qrow];
  v4f dq[2][4];  // dQ^T, column-fragment layout
#pragma unroll
  for (int gi = 0; gi < 2; gi++)
#pragma unroll
    for (int cc = 0; cc < 4; cc++) dq[gi][cc] = (v4f){0.f, 0.f, 0.f, 0.f};

  const int qlast = min(a.T, q0 + FQ) - 1;
  int kmin, kmax;
  key_range(q0, qlast, a.Tk, a.ratio, a.window, a.qoff, &kmin, &kmax);
  const int kt0 = (kmin / FS) * FS;
  const int ntile = kmax > kt0 ? (kmax - kt0 + FS - 1) / FS : 0;
  const float* kbase = a.k + ((int64_t)b * a.Tk * a.Hkv + hk) * HD;
  const float* vbase = a.v + ((int64_t)b * a.Tk * a.Hkv + hk) * HD;
  const int64_t kvstride = (int64_t)a.Hkv * HD;
  auto load = [&](int i, float* KS, float* VS) {
    const int kt = kt0 + i * FS;
    fl_stage_load(KS, [&](int r) { return kbase + min(kt + r, a.Tk - 1) * kvstride; }, w, lane);
    fl_stage_load(VS, [&](int r) { return vbase + min(kt + r, a.Tk - 1) * kvstride; }, w, lane);
  };
  auto tile = [&](int i, const float* KS, const float* VS, float* XK, float* XV) {
    fl_wait_all();
    fl_barrier();
    if (i + 1 < ntile) load(i + 1, XK, XV);
    const int kt = kt0 + i * FS;
#pragma unroll
    for (int kb = 0; kb < FS / 16; kb++) {
      v4f st = {0.f, 0.f, 0.f, 0.f}, dpt = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 8; s++) {
        const v4f kf = fl_row(KS, 16 * kb, s, l16, g);
        const v4f vf = fl_row(VS, 16 * kb, s, l16, g);
#pragma unroll
        for (int c = 0; c < 4; c++) {
          st = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[c], qf[s][c], st, 0, 0, 0);
          dpt = __builtin_amdgcn_mfma_f32_16x16x4f32(vf[c], gf[s][c], dpt, 0, 0, 0);
        }
      }
      v4f ds;
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int kj = kt + 16 * kb + 4 * g + r;
        const float p =
            (active && key_ok(kj, t, a.Tk, a.ratio, a.window, a.qoff)) ? expf(st[r] - lse) : 0.f;
        ds[r] = p * (dpt[r] - dl);
      }
      // dQ^T += K^T dS^T: A = K^T, column fragments of key rows 16kb + 4g + c
#pragma unroll
      for (int c = 0; c < 4; c++)
#pragma unroll
        for (int gi = 0; gi < 2; gi++) {
          const v4f kc = fl_col(KS, 16 * kb + 4 * g + c, gi, l16);
#pragma unroll
          for (int cc = 0; cc < 4; cc++)
            dq[gi][cc] = __builtin_amdgcn_mfma_f32_16x16x4f32(kc[cc], ds[c], dq[gi][cc], 0, 0, 0);
        }
    }
  };
  if (ntile > 0) load(0, Ks0, Vs0);
  for (int i = 0; i < ntile; i += 2) {
    tile(i, Ks0, Vs0, Ks1, Vs1);
    if (i + 1 < ntile) tile(i + 1, Ks1, Vs1, Ks0, Vs0);
  }
  if (active) fl_store_cols(a.dq + qrow * HD, dq, g, a.dq_accum, 1.f);
}

// dK/dV.  Block: 4 waves x 16 keys of one (sequence, KV head), over every
// query head of the GQA group and the query tiles that see the keys; S and
// dP come out with the lane's column = its key, so P and dS feed dV^T +=
// dO^T.P and dK^T += Q^T.dS as B operands straight from the lane.
__global__ __launch_bounds__(256, 2) void flash_bwd_dkdv_mfma_kernel(FlashBwdArgs a) {
  __shared__ __attribute__((aligned(16))) float Qs0[FS * HD];
  __shared__ __attribute__((aligned(16))) float Gs0[FS * HD];
  __shared__ __attribute__((aligned(16))) float Qs1[FS * HD];
  __shared__ __attribute__((aligned(16))) float Gs1[FS * HD];
  // per stage: the tile's log-sum-exp [0, FS) and delta [FS, 2 FS)
  __shared__ __attribute__((aligned(16))) float LD[2][2 * FS];
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, g = lane >> 4;
  const int k0 = blockIdx.x * FK;
  const int bk = blockIdx.y, b = bk / a.Hkv, hk = bk % a.Hkv;
  const int r = a.Hq / a.Hkv;
  const int j = k0 + 16 * w + l16;  // this lane's key
  const bool active = j < a.Tk;
  const int64_t krow = ((int64_t)b * a.Tk + min(j, a.Tk - 1)) * a.Hkv + hk;
  v4f kf[8], vf[8];
#pragma unroll
  for (int s = 0; s < 8; s++) {
    kf[s] = *reinterpret_cast<const v4f*>(a.k + krow * HD + 16 * s + 4 * g);
    vf[s] = *reinterpret_cast<const v4f*>(a.v + krow * HD + 16 * s + 4 * g);
  }
  v4f dk[2][4], dv[2][4];  // dK^T, dV^T, column-fragment layout
#pragma unroll
  for (int gi = 0; gi < 2; gi++)
#pragma unroll
    for (int cc = 0; cc < 4; cc++) {
      dk[gi][cc] = (v4f){0.f, 0.f, 0.f, 0.f};
      dv[gi][cc] = (v4f){0.f, 0.f, 0.f, 0.f};
    }
  const int klast = min(a.Tk, k0 + FK) - 1;
  // queries that can see a key of the block: [qbeg, qend)
  int qbeg, qend;
  if (a.ratio > 1) {
    qbeg = min(a.T, max(0, (k0 + 1) * a.ratio - a.qoff));
    qend = a.T;
  } else {
    qbeg = k0;
    qend = a.window >= 0 ? min(a.T, klast + a.window + 1) : a.T;
  }
  const int qt0 = (qbeg / FS) * FS;
  const int nq = qend > qt0 ? (qend - qt0 + FS - 1) / FS : 0;
  const int ntile = nq * r;  // (head, query tile) pairs, head-major
  const int64_t qstride = (int64_t)a.Hq * HD;
  auto load = [&](int i, float* QS, float* GS, int st) {
    const int qh = hk * r + i / nq, qt = qt0 + (i % nq) * FS;
    const float* qb = a.q + ((int64_t)b * a.T * a.Hq + qh) * HD;
    const float* gb = a.dout + ((int64_t)b * a.T * a.Hq + qh) * HD;
    fl_stage_load(QS, [&](int rr) { return qb + min(qt + rr, a.T - 1) * qstride; }, w, lane);
    fl_stage_load(GS, [&](int rr) { return gb + min(qt + rr, a.T - 1) * qstride; }, w, lane);
    if (w == 0) {  // one dword per lane: lse of rows [0, FS), then delta
      const int64_t row = ((int64_t)b * a.T + min(qt + (lane & (FS - 1)), a.T - 1)) * a.Hq + qh;
      __builtin_amdgcn_global_load_lds((const void*)((lane < FS ? a.lse : a.delta) + row),
                                       (fl_lds_void*)&LD[st][0], 4, 0, 0);
    }
  };
  auto tile = [&](int i, const float* QS, const float* GS, int st, float* XQ, float* XG) {
    fl_wait_all();
    fl_barrier();
    if (i + 1 < ntile) load(i + 1, XQ, XG, st ^ 1);
    const int qt = qt0 + (i % nq) * FS;
#pragma unroll
    for (int qb = 0; qb < FS / 16; qb++) {
      v4f sv = {0.f, 0.f, 0.f, 0.f}, dp = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 8; s++) {
        const v4f qv = fl_row(QS, 16 * qb, s, l16, g);
        const v4f gv = fl_row(GS, 16 * qb, s, l16, g);
#pragma unroll
        for (int c = 0; c < 4; c++) {
          sv = __builtin_amdgcn_mfma_f32_16x16x4f32(qv[c], kf[s][c], sv, 0, 0, 0);
          dp = __builtin_amdgcn_mfma_f32_16x16x4f32(gv[c], vf[s][c], dp, 0, 0, 0);
        }
      }
      // S[q][j], dP[q][j] for q = qt + 16qb + 4g + rr
      v4f p, ds;
#pragma unroll
      for (int rr = 0; rr < 4; rr++) {
        const int ql = 16 * qb + 4 * g + rr, tq = qt + ql;
        const bool ok = active && tq < a.T && key_ok(j, tq, a.Tk, a.ratio, a.window, a.qoff);
        p[rr] = ok ? expf(sv[rr] - LD[st][ql]) : 0.f;
        ds[rr] = p[rr] * (dp[rr] - LD[st][FS + ql]);
      }
      // dV^T += dO^T P, dK^T += Q^T dS: column fragments of query rows 16qb + 4g + c
#pragma unroll
      for (int c = 0; c < 4; c++)
#pragma unroll
        for (int gi = 0; gi < 2; gi++) {
          const int row = 16 * qb + 4 * g + c;
          const v4f gc = fl_col(GS, row, gi, l16);
          const v4f qc = fl_col(QS, row, gi, l16);
#pragma unroll
          for (int cc = 0; cc < 4; cc++) {
            dv[gi][cc] = __builtin_amdgcn_mfma_f32_16x16x4f32(gc[cc], p[c], dv[gi][cc], 0, 0, 0);
            dk[gi][cc] = __builtin_amdgcn_mfma_f32_16x16x4f32(qc[cc], ds[c], dk[gi][cc], 0, 0, 0);
          }
        }
    }
  };
  if (ntile > 0) load(0, Qs0, Gs0, 0);
  for (int i = 0; i < ntile; i += 2) {
    tile(i, Qs0, Gs0, 0, Qs1, Gs1);
    if (i + 1 < ntile) tile(i + 1, Qs1, Gs1, 1, Qs0, Gs0);
  }
  if (active) {
    fl_store_cols(a.dk + krow * HD, dk, g, false, 1.f);
    fl_store_cols(a.dv + krow * HD, dv, g, false, 1.f);
  }
}

void launch_row_dot(const float* o, const float* dout, float* delta, int64_t rows, hipStream_t st) {
  hipLaunchKernelGGL(flash_delta_kernel, dim3((unsigned)ceil_div(rows, 4)), dim3(256), 0, st, o,
                     dout, delta, rows);
  GN_HIP(hipGetLastError());
}

void launch_flash_bwd(FlashBwdArgs a, hipStream_t st) {
  if (a.Tk <= 0) a.Tk = a.T;
  GN_CHECK(a.ratio <= 1 || a.window < 0, "flash: compressed keys take no window");
  if (!a.delta_ready) launch_row_dot(a.o, a.dout, a.delta, (int64_t)a.B * a.T * a.Hq, st);
  hipLaunchKernelGGL(flash_bwd_dq_mfma_kernel, dim3((unsigned)ceil_div(a.T, FQ), a.B * a.Hq),
                     dim3(256), 0, st, a);
  GN_HIP(hipGetLastError());
  hipLaunchKernelGGL(flash_bwd_dkdv_mfma_kernel, dim3((unsigned)ceil_div(a.Tk, FK), a.B * a.Hkv),
                     dim3(256), 0, st, a);
  GN_HIP(hipGetLastError());
}

}  // namespace gn
