// gn_gemm.hip - fp32 GEMM on gfx950 matrix cores (v_mfma_f32_16x16x4_f32).
//
// C(m, n) = epilogue( sum_k A(m, k) * B(n, k) ), where each operand is either
// K-contiguous (A[m*lda + k], the "x" of x.W^T; B[n*ldb + k], a [out, in]
// weight) or M/N-contiguous (A[k*lda + m], B[k*ldb + n]).  One kernel thus
// serves Linear forward (x.W^T), its input gradient (g.W), its weight
// gradient (g^T.x, split over K) and kernels.Backend MatMul/MatMulTransposed.
//
// Tiles are staged through LDS in K-major order ([k][m]) so that the 16 lanes
// feeding one MFMA row block read 16 consecutive floats; rows are padded by
// 16 floats so the four k-rows a wave touches land on disjoint banks.  Two
// LDS buffers alternate so the global loads of tile k+1 overlap the MFMAs of
// tile k with a single barrier per iteration.
#include "gn_kernels.h"

namespace gn {

typedef float v4f __attribute__((ext_vector_type(4)));

struct GemmParams {
  const float* A;
  const float* B;
  float* C;
  const float* aux;  // EPI_ADD_SRC source / EPI_DRELU2 pre-activation
  float* aux_out;    // EPI_RELU2_SAVE pre-activation output
  int64_t lda, ldb, ldc, ldaux;
  int M, N, K;
  int k_per_split;
  int tiles_m;
  int epi;
  float alpha;
};

__device__ __forceinline__ void gemm_epilogue(const GemmParams& p, int row, int col, float v,
                                              int split) {
  if (row >= p.M || col >= p.N) return;
  const int64_t ci = (int64_t)row * p.ldc + col;
  switch (p.epi) {
    case EPI_STORE:
      p.C[ci] = v * p.alpha;
      break;
    case EPI_ADD_SRC:
      p.C[ci] = v + p.aux[(int64_t)row * p.ldaux + col];
      break;
    case EPI_ACCUM:
      p.C[ci] += v;
      break;
    case EPI_SOFTCAP:
      p.C[ci] = softcap15(v);
      break;
    case EPI_RELU2_SAVE: {
      if (p.aux_out) p.aux_out[(int64_t)row * p.ldaux + col] = v;
      float r = v < 0.f ? 0.f : v;
      p.C[ci] = r * r;
      break;
    }
    case EPI_DRELU2: {
      // tensors/backward.go:57-65: gradOut * 2 * value where value > 0
      float u = p.aux[(int64_t)row * p.ldaux + col];
      p.C[ci] = u > 0.f ? (v * 2.f) * u : 0.f;
      break;
    }
    case EPI_PARTIAL:
      p.C[(int64_t)split * p.M * p.N + (int64_t)row * p.N + col] = v;
      break;
  }
}

template <bool VEC>
__device__ __forceinline__ v4f load4(const float* __restrict__ ptr, int valid) {
  v4f r = {0.f, 0.f, 0.f, 0.f};
  if (VEC && valid == 4) {
    r = *reinterpret_cast<const v4f*>(ptr);
  } else {
    if (valid > 0) r[0] = ptr[0];
    if (valid > 1) r[1] = ptr[1];
    if (valid > 2) r[2] = ptr[2];
    if (valid > 3) r[3] = ptr[3];
  }
  return r;
}

// Loads the [BK=16] x [BD] tile of an operand whose logical index is
// (d, k), d in [d0, d0+BD), k in [k0, k0+16), into registers.
template <int BD, int NT, bool KCONTIG, bool VEC>
struct TileLoader {
  static constexpr int NV = (BD * 16 / 4) / NT;  // float4 per thread
  v4f v[NV];
  __device__ __forceinline__ void load(const float* __restrict__ X, int64_t ld, int d0, int dmax,
                                       int k0, int kmax, int tid) {
#pragma unroll
    for (int i = 0; i < NV; i++) {
      int idx = tid + i * NT;
      if (KCONTIG) {
        int d = idx % BD, kq = idx / BD;
        int gd = d0 + d, gk = k0 + 4 * kq;
        int valid = (gd < dmax) ? min(4, kmax - gk) : 0;
        v[i] = load4<VEC>(X + (int64_t)gd * ld + gk, valid);
      } else {
        int k = idx / (BD / 4), dq = idx % (BD / 4);
        int gd = d0 + 4 * dq, gk = k0 + k;
        int valid = (gk < kmax) ? min(4, dmax - gd) : 0;
        v[i] = load4<VEC>(X + (int64_t)gk * ld + gd, valid);
      }
    }
  }
  template <int LD>
  __device__ __forceinline__ void store(float* __restrict__ S, int tid) {
#pragma unroll
    for (int i = 0; i < NV; i++) {
      int idx = tid + i * NT;
      if (KCONTIG) {
        int d = idx % BD, kq = idx / BD;
#pragma unroll
        for (int j = 0; j < 4; j++) S[(4 * kq + j) * LD + d] = v[i][j];
      } else {
        int k = idx / (BD / 4), dq = idx % (BD / 4);
        *reinterpret_cast<v4f*>(&S[k * LD + 4 * dq]) = v[i];
      }
    }
  }
};

template <int BM, int BN, int WM, int WN, bool AK, bool BK, bool VEC>
__global__ __launch_bounds__(64 * WM * WN) void gemm_kernel(GemmParams p) {
  constexpr int NT = 64 * WM * WN;
  constexpr int TM = BM / WM, TN = BN / WN;
  constexpr int MI = TM / 16, NI = TN / 16;
  constexpr int LDA = BM + 16, LDB = BN + 16;
  __shared__ __attribute__((aligned(16))) float As[2][16 * LDA];
  __shared__ __attribute__((aligned(16))) float Bs[2][16 * LDB];

  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int wm = wid % WM, wn = wid / WM;
  const int tile = blockIdx.x;
  const int m0 = (tile % p.tiles_m) * BM, n0 = (tile / p.tiles_m) * BN;
  const int split = blockIdx.z;
  const int kbeg = split * p.k_per_split;
  const int kend = min(p.K, kbeg + p.k_per_split);

  // Two-level summation: MFMAs accumulate one 64-deep K block into `blk`,
  // which is folded into `acc` between blocks.  Rounding error then grows
  // with 64 + K/64 instead of K, which matters for the weight gradients (K =
  // tokens) and the logits-gradient contraction (K = vocabulary).
  constexpr int FOLD = 4;  // K tiles of 16 per block
  v4f acc[MI][NI], blk[MI][NI];
#pragma unroll
  for (int i = 0; i < MI; i++)
#pragma unroll
    for (int j = 0; j < NI; j++) {
      acc[i][j] = (v4f){0.f, 0.f, 0.f, 0.f};
      blk[i][j] = (v4f){0.f, 0.f, 0.f, 0.f};
    }

  TileLoader<BM, NT, AK, VEC> la;
  TileLoader<BN, NT, BK, VEC> lb;
  const int nkt = kend > kbeg ? (kend - kbeg + 15) / 16 : 0;
  if (nkt > 0) {
    la.load(p.A, p.lda, m0, p.M, kbeg, kend, tid);
    lb.load(p.B, p.ldb, n0, p.N, kbeg, kend, tid);
    la.template store<LDA>(As[0], tid);
    lb.template store<LDB>(Bs[0], tid);
  }
  __syncthreads();
  for (int kt = 0; kt < nkt; kt++) {
    const int cur = kt & 1;
    const bool more = kt + 1 < nkt;
    if (more) {
      la.load(p.A, p.lda, m0, p.M, kbeg + (kt + 1) * 16, kend, tid);
      lb.load(p.B, p.ldb, n0, p.N, kbeg + (kt + 1) * 16, kend, tid);
    }
    const float* as = As[cur];
    const float* bs = Bs[cur];
#pragma unroll
    for (int kk = 0; kk < 4; kk++) {
      const int k = 4 * kk + (lane >> 4);
      float a[MI], b[NI];
#pragma unroll
      for (int i = 0; i < MI; i++) a[i] = as[k * LDA + wm * TM + i * 16 + (lane & 15)];
#pragma unroll
      for (int j = 0; j < NI; j++) b[j] = bs[k * LDB + wn * TN + j * 16 + (lane & 15)];
#pragma unroll
      for (int i = 0; i < MI; i++)
#pragma unroll
        for (int j = 0; j < NI; j++)
          blk[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i], b[j], blk[i][j], 0, 0, 0);
    }
    if ((kt % FOLD) == FOLD - 1 || !more) {
#pragma unroll
      for (int i = 0; i < MI; i++)
#pragma unroll
        for (int j = 0; j < NI; j++) {
          acc[i][j] += blk[i][j];
          blk[i][j] = (v4f){0.f, 0.f, 0.f, 0.f};
        }
    }
    if (more) {
      la.template store<LDA>(As[cur ^ 1], tid);
      lb.template store<LDB>(Bs[cur ^ 1], tid);
    }
    __syncthreads();
  }
  // D[i][j] of a 16x16 block: lane holds column (lane & 15), rows 4*(lane>>4)+r.
#pragma unroll
  for (int i = 0; i < MI; i++)
#pragma unroll
    for (int j = 0; j < NI; j++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        int row = m0 + wm * TM + i * 16 + 4 * (lane >> 4) + r;
        int col = n0 + wn * TN + j * 16 + (lane & 15);
        gemm_epilogue(p, row, col, acc[i][j][r], split);
      }
}

// Sums split-K partials in split order in float64 (deterministic) and applies
// the real epilogue.
__global__ void gemm_reduce_kernel(GemmParams p, const float* __restrict__ part, int splits) {
  int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  int64_t total = (int64_t)p.M * p.N;
  if (idx >= total) return;
  double s = 0.0;
  for (int z = 0; z < splits; z++) s += (double)part[(int64_t)z * total + idx];
  int row = (int)(idx / p.N), col = (int)(idx % p.N);
  gemm_epilogue(p, row, col, (float)s, 0);
}

template <int BM, int BN, int WM, int WN>
static void launch_cfg(const GemmParams& p, bool ak, bool bk, bool vec, int splits,
                       hipStream_t st) {
  dim3 grid(p.tiles_m * (int)ceil_div(p.N, BN), 1, splits);
  dim3 block(64 * WM * WN);
#define GN_GEMM_LAUNCH(AK, BK, V) \
  hipLaunchKernelGGL((gemm_kernel<BM, BN, WM, WN, AK, BK, V>), grid, block, 0, st, p)
  if (vec) {
    if (ak && bk) GN_GEMM_LAUNCH(true, true, true);
    else if (ak && !bk) GN_GEMM_LAUNCH(true, false, true);
    else if (!ak && bk) GN_GEMM_LAUNCH(false, true, true);
    else GN_GEMM_LAUNCH(false, false, true);
  } else {
    if (ak && bk) GN_GEMM_LAUNCH(true, true, false);
    else if (ak && !bk) GN_GEMM_LAUNCH(true, false, false);
    else if (!ak && bk) GN_GEMM_LAUNCH(false, true, false);
    else GN_GEMM_LAUNCH(false, false, false);
  }
#undef GN_GEMM_LAUNCH
  GN_HIP(hipGetLastError());
}

static bool aligned16(const void* ptr) { return ((uintptr_t)ptr & 15) == 0; }

void gemm(const GemmDesc& d, hipStream_t st, DeviceArena* ws) {
  GN_CHECK(d.M >= 0 && d.N >= 0 && d.K >= 0, "gemm: negative extent");
  if (d.M == 0 || d.N == 0) return;
  GemmParams p{};
  p.A = d.A; p.B = d.B; p.C = d.C; p.aux = d.aux; p.aux_out = d.aux_out;
  p.lda = d.lda; p.ldb = d.ldb; p.ldc = d.ldc; p.ldaux = d.ldaux;
  p.M = d.M; p.N = d.N; p.K = d.K;
  p.epi = d.epi;
  p.alpha = d.alpha;
  const bool vec = aligned16(d.A) && aligned16(d.B) && d.lda % 4 == 0 && d.ldb % 4 == 0;

  // Tile choice: the 128x128 tile when it yields enough workgroups to cover
  // the 256 CUs, otherwise 64x64; split K when even that underfills the chip
  // and K is long enough to share.
  // Long-K products (weight gradients, K = tokens) keep the 128x128 tile and
  // split K instead, since each split still has thousands of K steps.
  const int64_t cus = 256;
  const int64_t big = ceil_div(d.M, 128) * ceil_div(d.N, 128);
  const bool long_k = d.K >= 4096;
  const bool use_big = big >= cus || long_k;
  const int bm = use_big ? 128 : 64, bn = use_big ? 128 : 64;
  const int64_t tiles = ceil_div(d.M, bm) * ceil_div(d.N, bn);
  int splits = 1;
  if (d.force_splits > 0) {
    splits = d.force_splits;
  } else if (tiles < 2 * cus && d.K >= 512) {
    splits = (int)std::min<int64_t>(ceil_div(2 * cus, tiles), d.K / (long_k ? 1024 : 256));
    splits = std::max(1, std::min(splits, 64));
  }
  int kps = (int)ceil_div(ceil_div(d.K, splits), 16) * 16;
  splits = d.K > 0 ? (int)ceil_div(d.K, kps) : 1;
  p.tiles_m = (int)ceil_div(d.M, bm);

  if (splits > 1) {
    GN_CHECK(ws != nullptr, "gemm: split-K needs a workspace");
    float* part = ws->get<float>("gemm_splitk", (size_t)splits * d.M * d.N);
    GemmParams q = p;
    q.C = part;
    q.epi = EPI_PARTIAL;
    q.k_per_split = kps;
    if (use_big) launch_cfg<128, 128, 2, 2>(q, d.a_kcontig, d.b_kcontig, vec, splits, st);
    else launch_cfg<64, 64, 2, 2>(q, d.a_kcontig, d.b_kcontig, vec, splits, st);
    int64_t total = (int64_t)d.M * d.N;
    hipLaunchKernelGGL(gemm_reduce_kernel, dim3((unsigned)ceil_div(total, 256)), dim3(256), 0, st,
                       p, part, splits);
    GN_HIP(hipGetLastError());
  } else {
    p.k_per_split = d.K > 0 ? kps : 0;
    if (use_big) launch_cfg<128, 128, 2, 2>(p, d.a_kcontig, d.b_kcontig, vec, 1, st);
    else launch_cfg<64, 64, 2, 2>(p, d.a_kcontig, d.b_kcontig, vec, 1, st);
  }
}

}  // namespace gn
