// gn_sparse.hip - the flash preset's sparse compressed attention (CSA:
// model/indexer.go, model/compress_attention.go).
//
// Every query row (sequence, kv-head, position t) selects at most K of the
// compressed blocks before its own block, allowed(t) = (qoff + t) / ratio,
// by the lightning indexer's score I[t,s] = sum_h w_h ReLU(q_h . k_h[s]):
// blocks are grouped by `pool`, the best groups by their maximum score give
// the candidates, and the top-K candidates by score are attended (ties go to
// the smaller group index, then to the earlier candidate, as topKIndices
// orders them).  The selection is integer work and is exact given the
// scores.
//
// Kernels:
//  * indexer_scores: one 64x64 (t, s) tile per block (4x4 entries per
//    thread) from LDS copies of the query and key projections; tiles past
//    every row's causal limit are skipped (their entries are never read).
//  * csa_select: one wave per row.  Group maxima live in LDS; the chosen
//    groups and the final top-K come from repeated wave-wide argmax
//    reductions over (value desc, index asc).
//  * csa_attn_fwd / _bwd: one block per (token, kv-head) for all query heads
//    of the GQA group, over the <= K gathered compressed rows held in LDS.
//    The backward adds its compressed-key/value gradients with atomics.
//  * distillation: the indexer's softmax against the softmax of the mean
//    main-attention logit (compress_attention.go:133-196), per row, then the
//    per-head ReLU masks that feed the indexer's backward GEMMs.
#include "gn_model.h"

namespace gn {

typedef float v4f __attribute__((ext_vector_type(4)));
static constexpr int SD = 128;   // head dim
static constexpr int ST = 16;    // score tile
static constexpr int HIMAX = 256;

// ---------------------------------------------------------------------------
// Indexer scores
// ---------------------------------------------------------------------------
__device__ __forceinline__ int allowed_blocks(int t, const CsaShape& s) {
  return min(s.blocks, ((s.qoff_dev ? *s.qoff_dev : s.qoff) + t) / s.ratio);
}

static constexpr int IHMAX = 8;  // indexer heads

// Forward (mask_out null): out[z][t][s] = sum_h w_h ReLU(q_h . k_h) for
// s < allowed(t).  Backward (mask_out set): for every s < ldo the per-head
// gradient masks mask_out[h][z][t][s] = gs * w_h * [q_h . k_h > 0] (zero past
// allowed(t)), and this block's partial of each head weight's gradient
// sum gs * dot * [dot > 0] into gw_blocks[h * nblocks + block].
// A block covers a (SR*16) x (SR*16) tile of (t, s); thread (tx, ty) takes
// the SR x SR entries t0 + ty + 16 i, s0 + tx + 16 j, so each LDS value it
// reads feeds SR dot products (one entry per thread read two values per
// multiply-add).  Every entry's dot products run over e in order, as before.
static constexpr int SR = 4;
static constexpr int STT = ST * SR;
// dynamic LDS: the query and key rows of the tile, STT x (H dim + 1) floats each
__global__ __launch_bounds__(256) void indexer_scores_kernel(IndexerScoreArgs a) {
  extern __shared__ float lds_qk[];
  __shared__ float red[4];
  const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
  const CsaShape& sh = a.shape;
  const int HI = sh.H * sh.dim, HP = HI + 1;
  float* qsb = lds_qk;
  float* ksb = lds_qk + STT * HP;
  auto qs_at = [&](int r, int c) -> float& { return qsb[r * HP + c]; };
  auto ks_at = [&](int r, int c) -> float& { return ksb[r * HP + c]; };
  const int s0 = blockIdx.x * STT, t0 = blockIdx.y * STT, z = blockIdx.z;
  const int b = sh.b0 + z / sh.Hkv, hh = z % sh.Hkv;
  const int tl = min(sh.T, t0 + STT) - 1;
  const bool live = s0 < allowed_blocks(tl, sh);
  const bool bwd = a.mask_out != nullptr;
  const int64_t blk = ((int64_t)blockIdx.z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x;
  const int64_t nblk = (int64_t)gridDim.x * gridDim.y * gridDim.z;
  auto entry = [&](int i, int j, int& t, int& s) {
    t = t0 + ty + ST * i;
    s = s0 + tx + ST * j;
    return t < sh.T && s < sh.ldo;
  };
  if (!live) {  // past every row's causal limit: scores unread, masks zero
    if (bwd) {
      for (int i = 0; i < SR; i++)
        for (int j = 0; j < SR; j++) {
          int t, s;
          if (entry(i, j, t, s))
            for (int h = 0; h < sh.H; h++)
              a.mask_out[(int64_t)h * a.mask_stride + ((int64_t)z * sh.T + t) * sh.ldo + s] = 0.f;
        }
      if (tid < sh.H) a.gw_blocks[(int64_t)tid * nblk + blk] = 0.f;
    }
    return;
  }
  for (int i = tid; i < STT * HI; i += 256) {
    const int r = i / HI, c = i % HI;
    const int tt = t0 + r, ss = s0 + r;
    qs_at(r, c) = tt < sh.T ? a.iq[((int64_t)b * sh.T + tt) * HI + c] : 0.f;
    ks_at(r, c) = ss < sh.blocks ? a.ik[(((int64_t)b * sh.blocks + ss) * sh.Hkv + hh) * HI + c] : 0.f;
  }
  __syncthreads();
  bool ok[SR][SR], in[SR][SR];
  float g[SR][SR], total[SR][SR];
#pragma unroll
  for (int i = 0; i < SR; i++)
#pragma unroll
    for (int j = 0; j < SR; j++) {
      int t, s;
      in[i][j] = entry(i, j, t, s);
      ok[i][j] = in[i][j] && s < allowed_blocks(t, sh);
      g[i][j] = (bwd && ok[i][j]) ? a.gs[((int64_t)z * sh.T + t) * sh.ldo + s] : 0.f;
      total[i][j] = 0.f;
    }
  float wpart[IHMAX];
  for (int h = 0; h < sh.H; h++) {
    float dot[SR][SR];
#pragma unroll
    for (int i = 0; i < SR; i++)
#pragma unroll
      for (int j = 0; j < SR; j++) dot[i][j] = 0.f;
    for (int e = 0; e < sh.dim; e++) {
      float qv[SR], kv[SR];
#pragma unroll
      for (int i = 0; i < SR; i++) qv[i] = qs_at(ty + ST * i, h * sh.dim + e);
#pragma unroll
      for (int j = 0; j < SR; j++) kv[j] = ks_at(tx + ST * j, h * sh.dim + e);
#pragma unroll
      for (int i = 0; i < SR; i++)
#pragma unroll
        for (int j = 0; j < SR; j++) dot[i][j] += qv[i] * kv[j];
    }
    float wp = 0.f;
#pragma unroll
    for (int i = 0; i < SR; i++)
#pragma unroll
      for (int j = 0; j < SR; j++) {
        const bool pos = ok[i][j] && dot[i][j] > 0.f;
        if (bwd) {
          if (in[i][j]) {
            const int t = t0 + ty + ST * i, s = s0 + tx + ST * j;
            a.mask_out[(int64_t)h * a.mask_stride + ((int64_t)z * sh.T + t) * sh.ldo + s] =
                pos ? g[i][j] * a.w[h] : 0.f;
          }
          wp += pos ? g[i][j] * dot[i][j] : 0.f;
        } else if (pos) {
          total[i][j] += a.w[h] * dot[i][j];
        }
      }
    if (bwd) wpart[h] = wp;
  }
  if (bwd) {
    for (int h = 0; h < sh.H; h++) {
      const float v = block_sum(wpart[h], red);
      if (tid == 0) a.gw_blocks[(int64_t)h * nblk + blk] = v;
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < SR; i++)
#pragma unroll
    for (int j = 0; j < SR; j++)
      if (ok[i][j]) {
        const int t = t0 + ty + ST * i, s = s0 + tx + ST * j;
        a.out[((int64_t)z * sh.T + t) * sh.ldo + s] = total[i][j];
      }
}

// Decode scores (one query per row, T == 1): the row's keys are streamed
// once, coalesced.  LK = H * dim / 4 lanes share a key, each holding 4
// channels of one head (dim % 4 == 0): the per-head dot is summed over the
// head's dim / 4 lanes, ReLU-weighted by its lane 0, and the heads are
// summed over the key's lanes.  A block covers DEC_IT * 256 / LK keys, every
// thread's DEC_IT loads in flight at once.
static constexpr int DEC_IT = 8;
template <int LK>
__global__ __launch_bounds__(256) void indexer_scores_decode_kernel(IndexerScoreArgs a) {
  constexpr int KPI = 256 / LK;  // keys per block iteration
  const CsaShape& sh = a.shape;
  const int tid = threadIdx.x, kl = tid % LK, ks = tid / LK;
  const int z = blockIdx.y, b = sh.b0 + z / sh.Hkv, hh = z % sh.Hkv;
  const int allowed = allowed_blocks(0, sh);
  const int s0 = blockIdx.x * (DEC_IT * KPI);
  if (s0 >= allowed) return;  // past the causal limit: never read
  const int seg = sh.dim / 4;  // lanes per head
  const v4f q = *reinterpret_cast<const v4f*>(a.iq + (int64_t)b * (LK * 4) + 4 * kl);
  const float wh = a.w[(4 * kl) / sh.dim];
  const v4f* kb = reinterpret_cast<const v4f*>(a.ik + ((int64_t)b * sh.blocks * sh.Hkv + hh) * (LK * 4)) + kl;
  const int64_t kstride = (int64_t)sh.Hkv * LK;  // float4 per block key
  v4f kv[DEC_IT];
#pragma unroll
  for (int i = 0; i < DEC_IT; i++) {
    const int s = s0 + ks + i * KPI;
    kv[i] = s < allowed ? kb[s * kstride] : (v4f){0.f, 0.f, 0.f, 0.f};
  }
#pragma unroll
  for (int i = 0; i < DEC_IT; i++) {
    const int s = s0 + ks + i * KPI;
    float d = q[0] * kv[i][0] + q[1] * kv[i][1] + q[2] * kv[i][2] + q[3] * kv[i][3];
    for (int o = 1; o < seg; o <<= 1) d += __shfl_xor(d, o, 64);
    float v = (kl % seg == 0 && d > 0.f) ? wh * d : 0.f;
    for (int o = seg; o < LK; o <<= 1) v += __shfl_xor(v, o, 64);
    if (kl == 0 && s < allowed) a.out[(int64_t)z * sh.ldo + s] = v;
  }
}

template <int LK>
static void run_scores_decode(const IndexerScoreArgs& a, int chunk_seqs, hipStream_t st) {
  const int per = DEC_IT * (256 / LK);
  hipLaunchKernelGGL(indexer_scores_decode_kernel<LK>,
                     dim3((unsigned)ceil_div(a.shape.ldo, per), (unsigned)(chunk_seqs * a.shape.Hkv)),
                     dim3(256), 0, st, a);
}

void launch_indexer_scores(const IndexerScoreArgs& a, int chunk_seqs, hipStream_t st) {
  const CsaShape& s = a.shape;
  GN_CHECK(s.H * s.dim <= HIMAX && s.H <= IHMAX, "indexer: heads * dim must be <= 256, heads <= 8");
  GN_CHECK(s.ldo >= s.blocks, "indexer: score row stride below the block count");
  const int seg = s.dim / 4, LK = s.H * s.dim / 4;
  if (s.T == 1 && !a.mask_out && s.dim % 4 == 0 && seg > 0 && (seg & (seg - 1)) == 0 &&
      (LK & (LK - 1)) == 0) {
    switch (LK) {  // LK = H * dim / 4 <= 64, a power of two
      case 1: run_scores_decode<1>(a, chunk_seqs, st); break;
      case 2: run_scores_decode<2>(a, chunk_seqs, st); break;
      case 4: run_scores_decode<4>(a, chunk_seqs, st); break;
      case 8: run_scores_decode<8>(a, chunk_seqs, st); break;
      case 16: run_scores_decode<16>(a, chunk_seqs, st); break;
      case 32: run_scores_decode<32>(a, chunk_seqs, st); break;
      case 64: run_scores_decode<64>(a, chunk_seqs, st); break;
    }
    GN_HIP(hipGetLastError());
    return;
  }
  dim3 grid((unsigned)ceil_div(s.ldo, STT), (unsigned)ceil_div(s.T, STT), (unsigned)(chunk_seqs * s.Hkv));
  const size_t lds = sizeof(float) * 2 * STT * (s.H * s.dim + 1);  // <= 132 KB
  static const bool lds_ok = hipFuncSetAttribute((const void*)indexer_scores_kernel,
                                                 hipFuncAttributeMaxDynamicSharedMemorySize,
                                                 (int)(sizeof(float) * 2 * STT * (HIMAX + 1))) ==
                             hipSuccess;
  GN_CHECK(lds_ok, "indexer: the score kernel's LDS size was refused");
  hipLaunchKernelGGL(indexer_scores_kernel, grid, dim3(256), lds, st, a);
  GN_HIP(hipGetLastError());
}

int64_t indexer_mask_blocks(const CsaShape& s, int chunk_seqs) {
  return ceil_div(s.ldo, STT) * ceil_div(s.T, STT) * (int64_t)chunk_seqs * s.Hkv;
}

// ---------------------------------------------------------------------------
// Selection: one wave per row
// ---------------------------------------------------------------------------
// LDS writes of one lane visible to the rest of its wave
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}
// (value desc, index asc): a outranks b
__device__ __forceinline__ bool outranks(float va, int ia, float vb, int ib) {
  return va > vb || (va == vb && ia < ib);
}
__device__ __forceinline__ void wave_best(float& v, int& i) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(v, o, 64);
    const int oi = __shfl_xor(i, o, 64);
    if (outranks(ov, oi, v, i)) {
      v = ov;
      i = oi;
    }
  }
}
// n values in LDS (NaN marks taken entries, which never outrank): take the
// best `count` in rank order into out[].  All lanes return the same count.
// Up to 64 * 8 values: every lane ranks its M = ceil(n / 64) values against
// all n at once -- rank(i) = #{j : (v_j, j) outranks (v_i, i)}, a strict
// total order, so the ranks are distinct and rank r goes to out[r] -- one
// pass over the LDS (broadcast reads) instead of `count` rounds of
// wave-wide argmax.  The order is compared as one 64-bit key: the float
// mapped to an order-preserving unsigned (-0 as +0, so the zeros tie as in
// a float compare) above the complemented index; NaN maps to key 0, which
// outranks nothing.
__device__ __forceinline__ uint64_t rank_key(float v, int i) {
  if (v != v) return 0;
  uint32_t u = __float_as_uint(v == 0.f ? 0.f : v);
  u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((uint64_t)u << 32) | (uint32_t)(0xFFFFFFFFu - (uint32_t)i);
}
template <int M>
__device__ int wave_topk_rank(const float* vals, int n, int count, int* out) {
  const int lane = threadIdx.x & 63;
  uint64_t key[M];
  int r[M];
  int mine = 0;
#pragma unroll
  for (int m = 0; m < M; m++) {
    const int i = lane + 64 * m;
    key[m] = i < n ? rank_key(vals[i], i) : 0;
    r[m] = 0;
    mine += key[m] != 0;
  }
#pragma unroll 4
  for (int j = 0; j < n; j++) {
    const uint64_t kj = rank_key(vals[j], j);
#pragma unroll
    for (int m = 0; m < M; m++) r[m] += kj > key[m];
  }
#pragma unroll
  for (int m = 0; m < M; m++)
    if (key[m] != 0 && r[m] < count) out[r[m]] = lane + 64 * m;
  wave_sync();
  int valid = mine;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) valid += __shfl_xor(valid, o, 64);
  return min(count, valid);
}
__device__ int wave_topk_iter(float* vals, int n, int count, int* out);
__device__ int wave_topk(float* vals, int n, int count, int* out) {
  switch ((n + 63) / 64) {
    case 0:
    case 1: return wave_topk_rank<1>(vals, n, count, out);
    case 2: return wave_topk_rank<2>(vals, n, count, out);
    case 3: return wave_topk_rank<3>(vals, n, count, out);
    case 4: return wave_topk_rank<4>(vals, n, count, out);
    case 5: return wave_topk_rank<5>(vals, n, count, out);
    case 6: return wave_topk_rank<6>(vals, n, count, out);
    case 7: return wave_topk_rank<7>(vals, n, count, out);
    case 8: return wave_topk_rank<8>(vals, n, count, out);
    default: return wave_topk_iter(vals, n, count, out);
  }
}
__device__ int wave_topk_iter(float* vals, int n, int count, int* out) {
  const int lane = threadIdx.x & 63;
  int got = 0;
  for (int r = 0; r < count && r < n; r++) {
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int j = lane; j < n; j += 64) {
      const float v = vals[j];
      if (outranks(v, j, bv, bi)) {
        bv = v;
        bi = j;
      }
    }
    wave_best(bv, bi);
    if (bi == 0x7fffffff) break;  // every remaining entry taken
    if (lane == 0) {
      out[r] = bi;
      vals[bi] = __builtin_nanf("");
    }
    got++;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    wave_sync();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  }
  return got;
}

__global__ __launch_bounds__(256) void csa_select_kernel(CsaSelectArgs a) {
  extern __shared__ float sm[];
  const CsaShape& sh = a.shape;
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int64_t row = (int64_t)blockIdx.x * 4 + wid;  // chunk row (z, t)
  if (row >= (int64_t)a.chunk_seqs * sh.Hkv * sh.T) return;
  const int z = (int)(row / sh.T), t = (int)(row % sh.T);
  const int64_t grow = ((int64_t)(sh.b0 * sh.Hkv) + z) * sh.T + t;  // global row
  float* vals = sm + (int64_t)wid * a.wave_floats;  // groups or candidate scores
  int* cand = reinterpret_cast<int*>(vals + a.groups_cap);  // ccap entries
  int* rank = cand + a.ccap;                                // ranks (<= max(gpt, K))
  const float* score = a.scores + ((int64_t)z * sh.T + t) * sh.ldo;
  const int allowed = allowed_blocks(t, sh);
  int* sel = a.sel + grow * a.K;
  if (allowed <= 0 || a.K <= 0) {
    if (lane == 0) {
      a.nsel[grow] = 0;
      if (a.npool_out) a.npool_out[grow] = 0;
    }
    return;
  }
  int nc = 0;  // candidates (in candidate order) in cand[]
  if (a.pool_in) {  // Reindex: the fine stage within the producer's pool
    const int np = a.npool_in[grow];
    const int* pl = a.pool_in + grow * a.ccap;
    for (int i0 = 0; i0 < np; i0 += 64) {  // the pool's allowed entries, in order
      const int i = i0 + lane;
      const int e = i < np ? pl[i] : -1;
      const bool ok = e >= 0 && e < allowed;
      const uint64_t m = __ballot(ok);
      if (ok) cand[nc + __popcll(m & ((1ull << lane) - 1))] = e;
      nc += __popcll(m);
    }
  } else if (a.pool == 1 && a.gpt >= a.K) {
    // flat: the top-K of the top-budget entries are the top-K entries
    for (int j = lane; j < allowed; j += 64) vals[j] = score[j];
    wave_sync();
    const int n = wave_topk(vals, allowed, a.K, rank);
    if (lane == 0) {
      for (int i = 0; i < n; i++) sel[i] = rank[i];
      a.nsel[grow] = n;
    }
    return;
  } else {
    const int ag = (allowed + a.pool - 1) / a.pool;
    if (a.pool <= 64 && (a.pool & (a.pool - 1)) == 0) {
      // IndexerBlockMax over the allowed entries, coalesced: lane j of a
      // 256-entry stretch reads entry j, a group is `pool` adjacent lanes
      for (int j0 = 0; j0 < allowed; j0 += 256) {
        float v[4];
#pragma unroll
        for (int u = 0; u < 4; u++) {
          const int j = j0 + 64 * u + lane;
          v[u] = j < allowed ? score[j] : -INFINITY;
        }
#pragma unroll
        for (int u = 0; u < 4; u++) {
          const int j = j0 + 64 * u + lane;
          for (int o = 1; o < a.pool; o <<= 1) v[u] = fmaxf(v[u], __shfl_xor(v[u], o, 64));
          if ((lane & (a.pool - 1)) == 0 && j < allowed) vals[j / a.pool] = v[u];
        }
      }
    } else {
      for (int g = lane; g < ag; g += 64) {  // IndexerBlockMax over the allowed entries
        const int st = g * a.pool, en = min(st + a.pool, allowed);
        float mx = -INFINITY;
        for (int e = st; e < en; e++) mx = fmaxf(mx, score[e]);
        vals[g] = mx;
      }
    }
    wave_sync();
    const int ng = wave_topk(vals, ag, a.gpt, rank);
    for (int i0 = 0; i0 < ng * a.pool; i0 += 64) {  // the chosen groups' allowed entries
      const int i = i0 + lane;
      const int e = i < ng * a.pool ? rank[i / a.pool] * a.pool + i % a.pool : allowed;
      const bool ok = e < allowed;
      const uint64_t m = __ballot(ok);
      if (ok) cand[nc + __popcll(m & ((1ull << lane) - 1))] = e;
      nc += __popcll(m);
    }
  }
  wave_sync();
  if (a.pool_out) {
    int* po = a.pool_out + grow * a.ccap;
    for (int i = lane; i < nc; i += 64) po[i] = cand[i];
    if (lane == 0) a.npool_out[grow] = nc;
  }
  for (int i = lane; i < nc; i += 64) vals[i] = score[cand[i]];
  wave_sync();
  const int n = wave_topk(vals, nc, a.K, rank);
  if (lane == 0) {
    for (int i = 0; i < n; i++) sel[i] = cand[rank[i]];
    a.nsel[grow] = n;
  }
}

// ---------------------------------------------------------------------------
// Selection for few rows (decode): one block of CSB_NW waves per row.  The
// rank counts of every top-k stage are split over the block's waves (each
// wave counts, for every value, the values of its own share of the list that
// outrank it; the shares are added in LDS), so a row's selection takes a
// fraction of the serial passes of one wave.  Same strict order (rank_key)
// as the wave kernel, so the same selection.
// ---------------------------------------------------------------------------
static constexpr int CSB_NW = 8, CSB_NT = 64 * CSB_NW, CSB_MAXN = 512;
// rows up to which the block kernel is chosen (fewer rows than CUs: the
// one-wave-per-row grid would leave most of the chip idle)
static constexpr int64_t CSB_ROWS = 128;

// n <= CSB_MAXN values in LDS (NaN never outranks): the best `count` into
// out[] in rank order; rk[] holds n rank counts.  Called by the whole block;
// returns min(count, #non-NaN) and ends with out[] visible to every thread.
template <int M>
__device__ int block_topk_rank(const float* vals, int n, int count, int* out, int* rk,
                               int* nvalid) {
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  for (int i = tid; i < n; i += CSB_NT) rk[i] = 0;
  __syncthreads();
  uint64_t key[M];
  int r[M];
#pragma unroll
  for (int m = 0; m < M; m++) {
    const int i = lane + 64 * m;
    key[m] = i < n ? rank_key(vals[i], i) : 0;
    r[m] = 0;
  }
  const int per = (n + CSB_NW - 1) / CSB_NW, j0 = wid * per, j1 = min(n, j0 + per);
#pragma unroll 4
  for (int j = j0; j < j1; j++) {
    const uint64_t kj = rank_key(vals[j], j);
#pragma unroll
    for (int m = 0; m < M; m++) r[m] += kj > key[m];
  }
#pragma unroll
  for (int m = 0; m < M; m++)
    if (lane + 64 * m < n && r[m] > 0) atomicAdd(&rk[lane + 64 * m], r[m]);
  if (wid == 0) {
    int mine = 0;
#pragma unroll
    for (int m = 0; m < M; m++) mine += key[m] != 0;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mine += __shfl_xor(mine, o, 64);
    if (lane == 0) *nvalid = mine;
  }
  __syncthreads();
  for (int i = tid; i < n; i += CSB_NT)
    if (rank_key(vals[i], i) != 0 && rk[i] < count) out[rk[i]] = i;
  const int valid = *nvalid;
  __syncthreads();
  return min(count, valid);
}
__device__ int block_topk(const float* vals, int n, int count, int* out, int* rk, int* nvalid) {
  switch ((n + 63) / 64) {
    case 0:
    case 1: return block_topk_rank<1>(vals, n, count, out, rk, nvalid);
    case 2: return block_topk_rank<2>(vals, n, count, out, rk, nvalid);
    case 3: return block_topk_rank<3>(vals, n, count, out, rk, nvalid);
    case 4: return block_topk_rank<4>(vals, n, count, out, rk, nvalid);
    case 5: return block_topk_rank<5>(vals, n, count, out, rk, nvalid);
    case 6: return block_topk_rank<6>(vals, n, count, out, rk, nvalid);
    case 7: return block_topk_rank<7>(vals, n, count, out, rk, nvalid);
    default: return block_topk_rank<8>(vals, n, count, out, rk, nvalid);
  }
}

// Wave 0 lists the allowed entries of a candidate list in order into cand[]
// (compaction by ballot); returns the count to every thread.
template <typename F>
__device__ int block_compact(int total, F entry, int allowed, int* cand, int* ncand) {
  const int tid = threadIdx.x, lane = tid & 63;
  if (tid < 64) {
    int nc = 0;
    for (int i0 = 0; i0 < total; i0 += 64) {
      const int i = i0 + lane;
      const int e = i < total ? entry(i) : -1;
      const bool ok = e >= 0 && e < allowed;
      const uint64_t m = __ballot(ok);
      if (ok) cand[nc + __popcll(m & ((1ull << lane) - 1))] = e;
      nc += __popcll(m);
    }
    if (lane == 0) *ncand = nc;
  }
  __syncthreads();
  return *ncand;
}

__global__ __launch_bounds__(CSB_NT) void csa_select_block_kernel(CsaSelectArgs a) {
  extern __shared__ float sm[];
  __shared__ int nvalid, ncand;
  const CsaShape& sh = a.shape;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int64_t row = blockIdx.x;  // chunk row (z, t)
  const int z = (int)(row / sh.T), t = (int)(row % sh.T);
  const int64_t grow = ((int64_t)(sh.b0 * sh.Hkv) + z) * sh.T + t;  // global row
  float* vals = sm;                                         // groups or candidate scores
  int* cand = reinterpret_cast<int*>(vals + a.groups_cap);  // ccap entries
  int* rank = cand + a.ccap;                                // max(gpt, K) + 1
  int* rk = rank + std::max(a.gpt, a.K) + 1;                // CSB_MAXN rank counts
  const float* score = a.scores + ((int64_t)z * sh.T + t) * sh.ldo;
  const int allowed = allowed_blocks(t, sh);
  int* sel = a.sel + grow * a.K;
  if (allowed <= 0 || a.K <= 0) {  // block-uniform
    if (tid == 0) {
      a.nsel[grow] = 0;
      if (a.npool_out) a.npool_out[grow] = 0;
    }
    return;
  }
  int nc;
  if (a.pool_in) {  // Reindex: the fine stage within the producer's pool
    const int* pl = a.pool_in + grow * a.ccap;
    nc = block_compact(a.npool_in[grow], [&](int i) { return pl[i]; }, allowed, cand, &ncand);
  } else if (a.pool == 1 && a.gpt >= a.K) {
    // flat: the top-K of the top-budget entries are the top-K entries
    for (int j = tid; j < allowed; j += CSB_NT) vals[j] = score[j];
    __syncthreads();
    const int n = block_topk(vals, allowed, a.K, rank, rk, &nvalid);
    for (int i = tid; i < n; i += CSB_NT) sel[i] = rank[i];
    if (tid == 0) a.nsel[grow] = n;
    return;
  } else {
    const int ag = (allowed + a.pool - 1) / a.pool;
    if (a.pool <= 64 && (a.pool & (a.pool - 1)) == 0) {
      // IndexerBlockMax, coalesced: a wave takes 256-entry stretches, lane j
      // of a stretch reads entry j, a group is `pool` adjacent lanes
      for (int j0 = 256 * wid; j0 < allowed; j0 += 256 * CSB_NW) {
        float v[4];
#pragma unroll
        for (int u = 0; u < 4; u++) {
          const int j = j0 + 64 * u + lane;
          v[u] = j < allowed ? score[j] : -INFINITY;
        }
#pragma unroll
        for (int u = 0; u < 4; u++) {
          const int j = j0 + 64 * u + lane;
          for (int o = 1; o < a.pool; o <<= 1) v[u] = fmaxf(v[u], __shfl_xor(v[u], o, 64));
          if ((lane & (a.pool - 1)) == 0 && j < allowed) vals[j / a.pool] = v[u];
        }
      }
    } else {
      for (int g = tid; g < ag; g += CSB_NT) {  // IndexerBlockMax over the allowed entries
        const int st = g * a.pool, en = min(st + a.pool, allowed);
        float mx = -INFINITY;
        for (int e = st; e < en; e++) mx = fmaxf(mx, score[e]);
        vals[g] = mx;
      }
    }
    __syncthreads();
    const int ng = block_topk(vals, ag, a.gpt, rank, rk, &nvalid);
    const int pool = a.pool;
    nc = block_compact(ng * pool, [&](int i) { return rank[i / pool] * pool + i % pool; },
                       allowed, cand, &ncand);
  }
  if (a.pool_out) {
    int* po = a.pool_out + grow * a.ccap;
    for (int i = tid; i < nc; i += CSB_NT) po[i] = cand[i];
    if (tid == 0) a.npool_out[grow] = nc;
  }
  for (int i = tid; i < nc; i += CSB_NT) vals[i] = score[cand[i]];
  __syncthreads();
  const int n = block_topk(vals, nc, a.K, rank, rk, &nvalid);
  for (int i = tid; i < n; i += CSB_NT) sel[i] = cand[rank[i]];
  if (tid == 0) a.nsel[grow] = n;
}

void launch_csa_select(CsaSelectArgs a, hipStream_t st) {
  const CsaShape& s = a.shape;
  GN_CHECK(a.pool >= 1 && a.gpt >= 1 && a.K >= 1, "csa select: bad pool / budget / top-k");
  GN_CHECK(a.gpt * a.pool <= a.ccap && a.K <= a.ccap, "csa select: candidate capacity too small");
  GN_CHECK(a.mode >= 0 && a.mode <= 2, "csa select: bad mode");
  a.groups_cap = std::max<int>((s.blocks + a.pool - 1) / a.pool, a.ccap);
  const int64_t nrows = (int64_t)a.chunk_seqs * s.Hkv * s.T;
  // the block kernel ranks lists of at most CSB_MAXN values: the groups (or,
  // flat, the entries) and the candidates
  const bool block_fits = a.groups_cap <= CSB_MAXN && a.ccap <= CSB_MAXN;
  if (block_fits && (a.mode == 2 || (a.mode == 0 && nrows <= CSB_ROWS))) {
    const size_t lds = sizeof(float) * ((size_t)a.groups_cap + a.ccap + std::max(a.gpt, a.K) + 1 +
                                        CSB_MAXN);
    hipLaunchKernelGGL(csa_select_block_kernel, dim3((unsigned)nrows), dim3(CSB_NT), lds, st, a);
    GN_HIP(hipGetLastError());
    return;
  }
  a.wave_floats = a.groups_cap + a.ccap + std::max(a.gpt, a.K) + 1;
  const size_t lds = sizeof(float) * 4 * (size_t)a.wave_floats;
  GN_CHECK(lds <= 160 * 1024, "csa select: too many compressed blocks for one row in LDS");
  hipLaunchKernelGGL(csa_select_kernel, dim3((unsigned)ceil_div(nrows, 4)), dim3(256), lds, st, a);
  GN_HIP(hipGetLastError());
}

// ---------------------------------------------------------------------------
// Attention over the selected compressed rows
// ---------------------------------------------------------------------------
template <bool BWD>
__global__ __launch_bounds__(128) void csa_attn_kernel(CsaAttnArgs a) {
  extern __shared__ float sm[];
  const int tid = threadIdx.x;
  const int64_t n = blockIdx.x;  // token b*T + t
  const int hk = blockIdx.y;
  const int rr = a.Hq / a.Hkv;
  const int b = (int)(n / a.T), t = (int)(n % a.T);
  const int64_t grow = ((int64_t)b * a.Hkv + hk) * a.T + t;
  const int ns = a.nsel[grow];
  const int* sel = a.sel + grow * a.K;
  const int K = a.K;
  float* Ks = sm;                          // [K][SD + 1]
  float* Vs = Ks + K * (SD + 1);           // [K][SD + 1]
  float* Ss = Vs + K * (SD + 1);           // [rr][K] scores -> probabilities
  float* Dp = Ss + rr * K;                 // [rr][K] dP -> dS (backward)
  float* stat = Dp + rr * K;               // [rr][2] max / sum
  const int64_t qbase = (n * a.Hq + (int64_t)hk * rr) * SD;
  if (ns == 0) {
    if (!BWD) {
      for (int i = tid; i < rr * SD; i += 128) a.o[qbase + i] = 0.f;
      if (tid < rr) a.lse[n * a.Hq + hk * rr + tid] = -INFINITY;
    } else {
      for (int i = tid; i < rr * SD; i += 128) a.dq[qbase + i] = 0.f;
    }
    return;
  }
  for (int i = tid; i < ns * SD; i += 128) {
    const int j = i / SD, d = i % SD;
    const int64_t off = (((int64_t)b * a.blocks + sel[j]) * a.Hkv + hk) * SD + d;
    Ks[j * (SD + 1) + d] = a.kc[off];
    Vs[j * (SD + 1) + d] = a.vc[off];
  }
  __syncthreads();
  // scores (and dP): thread per (head, key)
  for (int p = tid; p < rr * ns; p += 128) {
    const int h = p / ns, j = p % ns;
    const float* q = a.q + qbase + (int64_t)h * SD;
    float s = 0.f, dp = 0.f;
    for (int d = 0; d < SD; d++) s += q[d] * Ks[j * (SD + 1) + d];
    if (BWD) {
      const float* g = a.dout + qbase + (int64_t)h * SD;
      for (int d = 0; d < SD; d++) dp += g[d] * Vs[j * (SD + 1) + d];
      const float lse = a.lse[n * a.Hq + hk * rr + h];
      const float pr = expf(s - lse);
      Ss[h * K + j] = pr;
      Dp[h * K + j] = pr * (dp - a.delta[n * a.Hq + hk * rr + h]);
    } else {
      Ss[h * K + j] = s;
    }
  }
  __syncthreads();
  if (!BWD) {
    if (tid < rr) {
      float mx = -INFINITY;
      for (int j = 0; j < ns; j++) mx = fmaxf(mx, Ss[tid * K + j]);
      float sum = 0.f;
      for (int j = 0; j < ns; j++) {
        const float e = expf(Ss[tid * K + j] - mx);
        Ss[tid * K + j] = e;
        sum += e;
      }
      stat[2 * tid] = mx;
      stat[2 * tid + 1] = sum;
      a.lse[n * a.Hq + hk * rr + tid] = mx + logf(sum);
    }
    __syncthreads();
    for (int i = tid; i < rr * SD; i += 128) {
      const int h = i / SD, d = i % SD;
      float acc = 0.f;
      for (int j = 0; j < ns; j++) acc += Ss[h * K + j] * Vs[j * (SD + 1) + d];
      a.o[qbase + i] = acc / stat[2 * h + 1];
    }
    return;
  }
  // backward: dq (overwritten; the local branch adds after), dk/dv scattered
  for (int i = tid; i < rr * SD; i += 128) {
    const int h = i / SD, d = i % SD;
    float acc = 0.f;
    for (int j = 0; j < ns; j++) acc += Dp[h * K + j] * Ks[j * (SD + 1) + d];
    a.dq[qbase + i] = acc;
  }
  for (int i = tid; i < ns * SD; i += 128) {
    const int j = i / SD, d = i % SD;
    float gk = 0.f, gv = 0.f;
    for (int h = 0; h < rr; h++) {
      gk += Dp[h * K + j] * a.q[qbase + (int64_t)h * SD + d];
      gv += Ss[h * K + j] * a.dout[qbase + (int64_t)h * SD + d];
    }
    const int64_t off = (((int64_t)b * a.blocks + sel[j]) * a.Hkv + hk) * SD + d;
    atomicAdd(a.dkc + off, gk);
    atomicAdd(a.dvc + off, gv);
  }
}

static size_t csa_attn_lds(const CsaAttnArgs& a) {
  const int rr = a.Hq / a.Hkv;
  return sizeof(float) * ((size_t)2 * a.K * (SD + 1) + 2 * (size_t)rr * a.K + 2 * rr);
}

void launch_csa_attn_fwd(const CsaAttnArgs& a, hipStream_t st) {
  GN_CHECK(a.K >= 1 && a.K <= 64, "sparse attention: top-k must be in [1, 64]");
  hipLaunchKernelGGL(csa_attn_kernel<false>, dim3((unsigned)((int64_t)a.B * a.T), a.Hkv), dim3(128),
                     csa_attn_lds(a), st, a);
  GN_HIP(hipGetLastError());
}
void launch_csa_attn_bwd(const CsaAttnArgs& a, hipStream_t st) {
  GN_CHECK(a.K >= 1 && a.K <= 64, "sparse attention: top-k must be in [1, 64]");
  hipLaunchKernelGGL(csa_attn_kernel<true>, dim3((unsigned)((int64_t)a.B * a.T), a.Hkv), dim3(128),
                     csa_attn_lds(a), st, a);
  GN_HIP(hipGetLastError());
}

// ---------------------------------------------------------------------------
// Distillation (compress_attention.go:133-196, 199-230, 262-298)
// ---------------------------------------------------------------------------
// qsum[n][hk][:] = sum of the query heads of kv-head hk
__global__ void query_group_sum_kernel(const float* __restrict__ q, int Hq, int Hkv, int64_t N,
                                       float* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= N * Hkv * SD) return;
  const int d = (int)(i % SD);
  const int64_t r = i / SD;
  const int hk = (int)(r % Hkv);
  const int64_t n = r / Hkv;
  const int rr = Hq / Hkv;
  float s = 0.f;
  for (int h = 0; h < rr; h++) s += q[(n * Hq + hk * rr + h) * SD + d];
  out[i] = s;
}
void launch_query_group_sum(const float* q, int Hq, int Hkv, int64_t N, float* out,
                            hipStream_t st) {
  const int64_t total = N * Hkv * SD;
  hipLaunchKernelGGL(query_group_sum_kernel, dim3((unsigned)ceil_div(total, 256)), dim3(256), 0, st,
                     q, Hq, Hkv, N, out);
  GN_HIP(hipGetLastError());
}

// One block per chunk row: gs = (softmax(I) - target) * weight over the
// allowed blocks (zero elsewhere in the row); the target is the softmax of
// the mean main-attention logits tl (already divided by the group size),
// restricted and renormalized to the pool on Reindex layers, whose indexer
// scores outside the pool count as -inf.
__global__ __launch_bounds__(256) void csa_distill_kernel(CsaDistillArgs a) {
  extern __shared__ float sm[];
  __shared__ float red[8];
  const CsaShape& sh = a.shape;
  const int64_t row = blockIdx.x;
  const int z = (int)(row / sh.T), t = (int)(row % sh.T);
  const int64_t grow = ((int64_t)(sh.b0 * sh.Hkv) + z) * sh.T + t;
  const int tid = threadIdx.x;
  const int allowed = allowed_blocks(t, sh);
  const float* sc = a.scores + row * sh.ldo;
  const float* tl = a.tlog + row * sh.ldo;
  float* gs = a.gs + row * sh.ldo;
  unsigned char* inpool = reinterpret_cast<unsigned char*>(sm);
  if (a.pool_in) {
    for (int e = tid; e < allowed; e += 256) inpool[e] = 0;
    __syncthreads();
    const int np = a.npool_in[grow];
    for (int i = tid; i < np; i += 256) {
      const int e = a.pool_in[grow * a.ccap + i];
      if (e >= 0 && e < allowed) inpool[e] = 1;
    }
    __syncthreads();
  }
  auto member = [&](int e) { return !a.pool_in || inpool[e]; };
  float ms = -INFINITY, mt = -INFINITY;
  for (int e = tid; e < allowed; e += 256) {
    if (member(e)) ms = fmaxf(ms, sc[e]);
    mt = fmaxf(mt, tl[e]);
  }
  ms = block_max(ms, red);
  mt = block_max(mt, red);
  float ss = 0.f, st_ = 0.f, sp = 0.f;
  for (int e = tid; e < allowed; e += 256) {
    if (member(e) && ms > -INFINITY) ss += expf(sc[e] - ms);
    const float v = expf(tl[e] - mt);
    st_ += v;
    if (member(e)) sp += v;
  }
  ss = block_sum(ss, red);
  st_ = block_sum(st_, red);
  sp = block_sum(sp, red);
  for (int e = tid; e < sh.ldo; e += 256) {
    float g = 0.f;
    if (e < allowed) {
      const float p = (member(e) && ms > -INFINITY) ? expf(sc[e] - ms) / ss : 0.f;
      float tg = expf(tl[e] - mt) / st_;
      if (a.pool_in) tg = member(e) && sp > 0.f ? expf(tl[e] - mt) / sp : 0.f;
      g = (p - tg) * a.weight;
    }
    gs[e] = g;
  }
}

void launch_csa_distill(const CsaDistillArgs& a, int chunk_seqs, hipStream_t st) {
  const CsaShape& s = a.shape;
  const size_t lds = a.pool_in ? (size_t)s.blocks + 16 : 16;
  GN_CHECK(lds <= 64 * 1024, "distillation: too many compressed blocks");
  hipLaunchKernelGGL(csa_distill_kernel, dim3((unsigned)((int64_t)chunk_seqs * s.Hkv * s.T)),
                     dim3(256), lds, st, a);
  GN_HIP(hipGetLastError());
}

// gw[h] += sum of the per-block partials (fixed order)
__global__ void sum_partials_kernel(const float* __restrict__ part, int64_t n, float* __restrict__ out) {
  __shared__ float red[4];
  float s = 0.f;
  for (int64_t i = threadIdx.x; i < n; i += 256) s += part[i];
  s = block_sum(s, red);
  if (threadIdx.x == 0) *out += s;
}
void launch_sum_partials(const float* part, int64_t n, float* out, hipStream_t st) {
  hipLaunchKernelGGL(sum_partials_kernel, dim3(1), dim3(256), 0, st, part, n, out);
  GN_HIP(hipGetLastError());
}

}  // namespace gn
