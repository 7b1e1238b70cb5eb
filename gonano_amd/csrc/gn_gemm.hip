// gn_gemm.hip - fp32 GEMM on gfx950 matrix cores (v_mfma_f32_16x16x4_f32).
//
// C(m, n) = epilogue( sum_k A(m, k) * B(n, k) ), where each operand is either
// K-contiguous (A[m*lda + k], the "x" of x.W^T; B[n*ldb + k], a [out, in]
// weight) or M/N-contiguous (A[k*lda + m], B[k*ldb + n]).  One kernel thus
// serves Linear forward (x.W^T), its input gradient (g.W), its weight
// gradient (g^T.x, split over K) and kernels.Backend MatMul/MatMulTransposed.
//
// Operand tiles go from global memory straight into a ring of LDS stages
// (global_load_lds_dwordx4, no VGPR staging), laid out so that MFMA fragments
// are read with conflict-free LDS accesses; see TileIO.  One barrier per K
// tile; the loads of the next S-1 tiles stay in flight behind the MFMAs.
#include <cstdlib>
#include <type_traits>

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
  int tiles_m, tiles_n, splits;
  int epi;
  float alpha;
  float* part;  // split-K: [splits][M][N] partial sums
  // Expert-grouped products (GEMM_GROUP_ROWS / GEMM_GROUP_K): goff[0..groups]
  // are row offsets on the device; gstride is the per-group element offset
  // of B (rows mode) or of C (K mode).
  const int* goff;
  int groups;
  int64_t gstride;
  int a_pad;  // rows mode: A is readable for at least 128 rows past its last row
  // batched products (grid y): product y reads A + y*bsa, B + y*bsb and
  // writes C + y*bsc, its split partials [splits][M][N] at part + y*splits*M*N
  int64_t bsa, bsb, bsc;
};

__device__ __forceinline__ void gemm_epilogue(const GemmParams& p, int row, int col, float v) {
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
  }
}

// Epilogue of a whole BM x BN tile inside C with the epilogue kind fixed at
// compile time (E; E == EPI_RELU2_SAVE + 16: ReLU^2 without the saved
// pre-activation): the same arithmetic as gemm_epilogue, without its
// per-element bounds check and dispatch, which compile to a branch around
// every single store.  D of a 16x16 block: lane holds column (lane & 15),
// rows 4*(lane>>4)+r.
template <int E, int MI, int NI>
__device__ __forceinline__ void store_tile(const GemmParams& p, const v4f (&acc)[MI][NI], int r0,
                                           int c0, int lane) {
#pragma unroll
  for (int i = 0; i < MI; i++)
#pragma unroll
    for (int j = 0; j < NI; j++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int row = r0 + i * 16 + 4 * (lane >> 4) + r;
        const int col = c0 + j * 16 + (lane & 15);
        const int64_t ci = (int64_t)row * p.ldc + col;
        const float v = acc[i][j][r];
        if constexpr (E == EPI_STORE) {
          p.C[ci] = v * p.alpha;
        } else if constexpr (E == EPI_ADD_SRC) {
          p.C[ci] = v + p.aux[(int64_t)row * p.ldaux + col];
        } else if constexpr (E == EPI_ACCUM) {
          p.C[ci] += v;
        } else if constexpr (E == EPI_SOFTCAP) {
          p.C[ci] = softcap15(v);
        } else if constexpr (E == EPI_RELU2_SAVE || E == EPI_RELU2_SAVE + 16) {
          if constexpr (E == EPI_RELU2_SAVE) p.aux_out[(int64_t)row * p.ldaux + col] = v;
          const float u = v < 0.f ? 0.f : v;
          p.C[ci] = u * u;
        } else {
          static_assert(E == EPI_DRELU2, "epilogue kind");
          const float u = p.aux[(int64_t)row * p.ldaux + col];
          p.C[ci] = u > 0.f ? (v * 2.f) * u : 0.f;
        }
      }
}

// A 64 x 64 wave tile (MI = NI = 4) through the wave's 16 KB LDS region S,
// so that each store instruction writes four whole 256-byte row pieces
// instead of 4 rows x 64 bytes one float per lane; same arithmetic as
// store_tile.  D of a 16x16 block (lane: column lane & 15, rows
// 4 (lane >> 4) + r) goes to S row-major with the column XOR 16 ((row >> 2)
// & 3), which spreads the four row groups of one ds_write over all banks;
// the reads take 16 bytes of one row per lane, the epilogue applied on the
// way out, the reading epilogues' operand fetched in that pattern before
// the staging writes.  Needs 16-byte aligned rows (ldc, ldaux % 4 == 0).
template <int E, int MI, int NI>
__device__ __forceinline__ void store_tile_staged(const GemmParams& p, const v4f (&acc)[MI][NI],
                                                  int r0, int c0, int lane, float* S) {
  static_assert(MI == 4 && NI == 4, "64 x 64 wave tiles");
  const int q = lane >> 4, cl = lane & 15;
  constexpr bool READS = E == EPI_ADD_SRC || E == EPI_ACCUM || E == EPI_DRELU2;
  v4f xs[READS ? 16 : 1];
  if constexpr (READS) {
    const float* src = E == EPI_ACCUM ? p.C : p.aux;
    const int64_t ld = E == EPI_ACCUM ? p.ldc : p.ldaux;
#pragma unroll
    for (int t = 0; t < 16; t++)
      xs[t] = *reinterpret_cast<const v4f*>(&src[(int64_t)(r0 + 4 * t + q) * ld + c0 + 4 * cl]);
  }
#pragma unroll
  for (int i = 0; i < MI; i++)
#pragma unroll
    for (int j = 0; j < NI; j++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int row = 16 * i + 4 * q + r;
        S[row * 64 + ((16 * j + cl) ^ (((row >> 2) & 3) << 4))] = acc[i][j][r];
      }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
  for (int t = 0; t < 16; t++) {
    const int row = 4 * t + q;
    const v4f v = *reinterpret_cast<const v4f*>(&S[row * 64 + ((4 * cl) ^ ((t & 3) << 4))]);
    const int64_t ci = (int64_t)(r0 + row) * p.ldc + c0 + 4 * cl;
    v4f o;
    if constexpr (E == EPI_STORE) {
      o = v * p.alpha;
    } else if constexpr (E == EPI_ADD_SRC || E == EPI_ACCUM) {
      o = E == EPI_ADD_SRC ? v + xs[t] : xs[t] + v;
    } else if constexpr (E == EPI_SOFTCAP) {
#pragma unroll
      for (int c = 0; c < 4; c++) o[c] = softcap15(v[c]);
    } else if constexpr (E == EPI_RELU2_SAVE || E == EPI_RELU2_SAVE + 16) {
      if constexpr (E == EPI_RELU2_SAVE)
        *reinterpret_cast<v4f*>(&p.aux_out[(int64_t)(r0 + row) * p.ldaux + c0 + 4 * cl]) = v;
#pragma unroll
      for (int c = 0; c < 4; c++) {
        const float u = v[c] < 0.f ? 0.f : v[c];
        o[c] = u * u;
      }
    } else {
      static_assert(E == EPI_DRELU2, "epilogue kind");
#pragma unroll
      for (int c = 0; c < 4; c++) o[c] = xs[t][c] > 0.f ? (v[c] * 2.f) * xs[t][c] : 0.f;
    }
    *reinterpret_cast<v4f*>(&p.C[ci]) = o;
  }
}

template <int MI, int NI>
__device__ __forceinline__ void store_tile_staged_any(const GemmParams& p,
                                                      const v4f (&acc)[MI][NI], int r0, int c0,
                                                      int lane, float* S) {
  switch (p.epi) {
    case EPI_STORE: store_tile_staged<EPI_STORE>(p, acc, r0, c0, lane, S); break;
    case EPI_ADD_SRC: store_tile_staged<EPI_ADD_SRC>(p, acc, r0, c0, lane, S); break;
    case EPI_ACCUM: store_tile_staged<EPI_ACCUM>(p, acc, r0, c0, lane, S); break;
    case EPI_SOFTCAP: store_tile_staged<EPI_SOFTCAP>(p, acc, r0, c0, lane, S); break;
    case EPI_RELU2_SAVE:
      if (p.aux_out) store_tile_staged<EPI_RELU2_SAVE>(p, acc, r0, c0, lane, S);
      else store_tile_staged<EPI_RELU2_SAVE + 16>(p, acc, r0, c0, lane, S);
      break;
    case EPI_DRELU2: store_tile_staged<EPI_DRELU2>(p, acc, r0, c0, lane, S); break;
  }
}

// Whole-tile epilogue: one dispatch on the (uniform) epilogue kind.
template <int MI, int NI>
__device__ __forceinline__ void store_tile_any(const GemmParams& p, const v4f (&acc)[MI][NI],
                                               int r0, int c0, int lane) {
  switch (p.epi) {
    case EPI_STORE: store_tile<EPI_STORE>(p, acc, r0, c0, lane); break;
    case EPI_ADD_SRC: store_tile<EPI_ADD_SRC>(p, acc, r0, c0, lane); break;
    case EPI_ACCUM: store_tile<EPI_ACCUM>(p, acc, r0, c0, lane); break;
    case EPI_SOFTCAP: store_tile<EPI_SOFTCAP>(p, acc, r0, c0, lane); break;
    case EPI_RELU2_SAVE:
      if (p.aux_out) store_tile<EPI_RELU2_SAVE>(p, acc, r0, c0, lane);
      else store_tile<EPI_RELU2_SAVE + 16>(p, acc, r0, c0, lane);
      break;
    case EPI_DRELU2: store_tile<EPI_DRELU2>(p, acc, r0, c0, lane); break;
  }
}

template <bool VEC>
__device__ __forceinline__ v4f load4(const float* __restrict__ ptr, int valid) {
  v4f r = {0.f, 0.f, 0.f, 0.f};
  if (VEC && valid >= 4) {
    r = *reinterpret_cast<const v4f*>(ptr);
  } else {
    if (valid > 0) r[0] = ptr[0];
    if (valid > 1) r[1] = ptr[1];
    if (valid > 2) r[2] = ptr[2];
    if (valid > 3) r[3] = ptr[3];
  }
  return r;
}

static constexpr int GK = 32;  // K depth of one LDS tile

typedef __attribute__((address_space(3))) void lds_void;

// One operand tile of BD rows (the M or N extent) by GK k values, moved from
// global memory into LDS by a workgroup of NT threads.
//
// Interior tiles use global_load_lds_dwordx4: each lane's 16 bytes land in
// LDS at (wave-uniform base) + lane * 16 without passing through VGPRs, so
// the LDS image is a sequence of 16-byte slots, slot s filled by thread
// s mod NT of instruction s / NT.  Which global float4 a lane fetches is free,
// so the layout is chosen by the addresses: a K-contiguous operand
// (X[d*ld + k]) is stored as [d][k] rows of GK floats (8 slots), an operand
// contiguous in d (X[k*ld + d]) as [k][d] rows of BD floats, and the slot
// column is XOR-swizzled with the row (row & 7, resp. row & 4) so the MFMA
// fragment reads below hit distinct banks.  Edge tiles (rows past the
// operand end, a partial last K tile, unaligned operands) go through VGPRs
// with zero fill and store to the same slots.
//
// MFMA k order: for the 16-deep k group g, lane (r = lane & 15, q = lane >> 4)
// holds k = 16g + 4q + c in component c, and MFMA c of the group consumes
// component c of both operands.  Every k is paired with itself in A and B,
// so the products summed are the same as in natural order.
template <int BD, int NT, bool KCONTIG, int TK = GK>
struct TileIO {
  static constexpr int ROWSLOTS = KCONTIG ? TK / 4 : BD / 4;  // 16-byte slots per LDS row
  static constexpr int SIZE = BD * TK;                         // floats
  static constexpr int NV = SIZE / 4 / NT;                     // slots per thread
  static constexpr int RSTEP = NT / ROWSLOTS;                  // LDS rows per instruction
  static_assert(NV >= 1 && NT % ROWSLOTS == 0 && RSTEP % 8 == 0, "tile shape");
  int row0, col;  // the thread's first LDS row and logical slot column

  static __device__ __forceinline__ int swz(int row) { return KCONTIG ? (row & 7) : (row & 4); }

  __device__ __forceinline__ void init(int tid) {
    row0 = tid / ROWSLOTS;
    col = (tid % ROWSLOTS) ^ swz(row0);  // swz(row0 + i * RSTEP) == swz(row0)
  }
  __device__ __forceinline__ const float* src(const float* X, int64_t ld, int d0, int k0,
                                              int i) const {
    const int row = row0 + i * RSTEP;
    return KCONTIG ? X + (int64_t)(d0 + row) * ld + (k0 + 4 * col)
                   : X + (int64_t)(k0 + row) * ld + (d0 + 4 * col);
  }
  // The whole tile lies inside the operand and is 16-byte aligned.
  __device__ __forceinline__ void load_direct(const float* __restrict__ X, int64_t ld, int d0,
                                              int k0, float* S, int wave) const {
#pragma unroll
    for (int i = 0; i < NV; i++)
      __builtin_amdgcn_global_load_lds((const void*)src(X, ld, d0, k0, i),
                                       (lds_void*)(S + 4 * (i * NT + 64 * wave)), 16, 0, 0);
  }
  // Edge tiles: zero outside d < dmax, k < kmax.
  template <bool VEC>
  __device__ __forceinline__ void load_edge(const float* __restrict__ X, int64_t ld, int d0,
                                            int dmax, int k0, int kmax, float* S, int tid) const {
#pragma unroll
    for (int i = 0; i < NV; i++) {
      const int row = row0 + i * RSTEP;
      int valid;
      if (KCONTIG) valid = d0 + row < dmax ? kmax - (k0 + 4 * col) : 0;
      else valid = k0 + row < kmax ? dmax - (d0 + 4 * col) : 0;
      *reinterpret_cast<v4f*>(&S[4 * (i * NT + tid)]) = load4<VEC>(src(X, ld, d0, k0, i), valid);
    }
  }
  // MFMA operand for the 16 rows starting at tile row d (a multiple of 16),
  // k group g.
  static __device__ __forceinline__ v4f frag(const float* __restrict__ S, int d, int g, int lane) {
    const int r = lane & 15, q = lane >> 4;
    if (KCONTIG) {
      const int row = d + r;
      return *reinterpret_cast<const v4f*>(&S[4 * (row * ROWSLOTS + ((4 * g + q) ^ swz(row)))]);
    }
    v4f f;
    const int dd = d + r;
#pragma unroll
    for (int c = 0; c < 4; c++) {
      const int k = 16 * g + 4 * q + c;
      f[c] = S[4 * (k * ROWSLOTS + ((dd >> 2) ^ swz(k))) + (dd & 3)];
    }
    return f;
  }
};

// Workgroup -> (tile row, tile column, split).  Workgroups are dealt to the
// 8 XCDs round-robin; renumbering gives each XCD a contiguous range of the
// logical order, so the tiles that share operand rows share one L2.  The
// logical order walks groups of 8 tile rows, column by column, so a group's
// A rows and the B columns in flight stay cache-resident.
__device__ __forceinline__ void tile_coords(const GemmParams& p, int& tm, int& tn, int& split) {
  const int total = p.tiles_m * p.tiles_n * p.splits;
  const int bid = blockIdx.x;
  const int x = bid % 8, q = total / 8, rem = total % 8;
  const int logical = x * q + min(x, rem) + bid / 8;
  const int T = p.tiles_m * p.tiles_n;
  split = logical / T;
  const int t = logical - split * T;
  constexpr int GM = 8;
  const int per_group = GM * p.tiles_n;
  const int first = (t / per_group) * GM;
  const int gsz = min(p.tiles_m - first, GM);
  const int r = t % per_group;
  tm = first + r % gsz;
  tn = r / gsz;
}

// s_waitcnt vmcnt(N) lgkmcnt(0) (gfx9 encoding: vmcnt[3:0] and [15:14],
// expcnt[6:4], lgkmcnt[11:8]).
template <int N>
__device__ __forceinline__ void wait_vm_lgkm0() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | ((N >> 4) << 14));
}

// Waits until at most `ahead` tiles of PT LDS-DMA instructions each are
// still in flight (ahead <= MAXA), with every LDS access of this wave done.
template <int PT, int MAXA>
__device__ __forceinline__ void wait_tiles(int ahead) {
  if constexpr (MAXA > 0) {
    if (ahead >= MAXA) {
      wait_vm_lgkm0<PT * MAXA>();
      return;
    }
    wait_tiles<PT, MAXA - 1>(ahead);
  } else {
    wait_vm_lgkm0<0>();
  }
}

// Workgroup barrier for the tile pipeline.  No release fence: a fence would
// make the compiler wait for every outstanding LDS-DMA load (vmcnt(0)) and
// defeat the prefetch; the explicit wait before it covers this wave's own
// accesses.  The acquire fence keeps LDS reads below the barrier.
__device__ __forceinline__ void tile_barrier() {
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// C tile of BM x BN per workgroup of WM x WN x WK waves, K in TK-deep tiles (GK unless given)
// through an S-stage LDS ring: tile kt + S - 1 is in flight while tile kt
// is multiplied.  The WK wave groups take alternate 16-deep k groups of
// every tile (more waves per SIMD for small grids) and are added in LDS at
// the end.  With p.splits > 1 each workgroup sums one K range into p.part
// and gemm_reduce_kernel applies the epilogue.
template <int BM, int BN, int WM, int WN, int WK, int S, bool FOLD, bool AK, bool BK, bool VEC,
          int GRP, int TK = GK>
__global__ __launch_bounds__(64 * WM * WN * WK, 2) void gemm_kernel(GemmParams p0) {
  constexpr int NT = 64 * WM * WN * WK;
  constexpr int TM = BM / WM, TN = BN / WN;
  constexpr int MI = TM / 16, NI = TN / 16;
  static_assert((TK / 16) % WK == 0, "k groups per wave group");
  static_assert(TK == GK || (AK && BK), "deep K tiles: K-contiguous operands");
  using LA = TileIO<BM, NT, AK, TK>;
  using LB = TileIO<BN, NT, BK, TK>;
  constexpr int PT = LA::NV + LB::NV;  // LDS-DMA instructions per tile and thread
  static_assert(S >= 2 && PT * (S - 2) < 64, "pipeline depth");
  static_assert((WK - 1) * WM * WN * MI * NI * 256 <= S * LA::SIZE,
                "wave-group partials fit in the A stage buffers");
  __shared__ __attribute__((aligned(16))) float As[S][LA::SIZE];
  __shared__ __attribute__((aligned(16))) float Bs[S][LB::SIZE];

  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int wmn = wid % (WM * WN), wk = wid / (WM * WN);
  const int wm = wmn % WM, wn = wmn / WM;
  int tm, tn, split;
  tile_coords(p0, tm, tn, split);
  GemmParams p = p0;
  if constexpr (GRP == GEMM_GROUP_NONE) {
    const int64_t y = blockIdx.y;  // batched products
    p.A += y * p.bsa;
    p.B += y * p.bsb;
    p.C += y * p.bsc;
    if (p.part) p.part += y * (int64_t)p.splits * p.M * p.N;
  }
  int m0 = tm * BM, kbeg, kend;
  const int n0 = tn * BN;
  if constexpr (GRP == GEMM_GROUP_ROWS) {
    // Rows grouped by expert: logical tile row tm walks each group's tiles
    // in turn (the grid is sized for the worst case; spare tiles exit).
    int base = 0, g = -1, mt = 0;
    for (int e = 0; e < p.groups; e++) {
      const int nt = (p.goff[e + 1] - p.goff[e] + BM - 1) / BM;
      if (tm < base + nt) {
        g = e;
        mt = tm - base;
        break;
      }
      base += nt;
    }
    if (g < 0) return;
    m0 = p.goff[g] + mt * BM;
    p.M = p.goff[g + 1];
    p.B += g * p.gstride;
    kbeg = split * p.k_per_split;  // optional split-K (small decode groups)
    kend = min(p.K, kbeg + p.k_per_split);
  } else if constexpr (GRP == GEMM_GROUP_K) {
    // The reduction runs over one group's rows; group g owns C + g*gstride.
    kbeg = p.goff[split];
    kend = p.goff[split + 1];
    p.C += split * p.gstride;
  } else {
    kbeg = split * p.k_per_split;
    kend = min(p.K, kbeg + p.k_per_split);
  }
  const int nkt = kend > kbeg ? (kend - kbeg + TK - 1) / TK : 0;
  // Rows mode with a padded A (a_pad): a tile may read up to BM rows past
  // its group's end (the next group's rows or the padding); those rows only
  // feed output rows >= p.M, which the epilogue discards, so partial groups
  // still take the direct path.
  const bool interior = VEC && (m0 + BM <= p.M || (GRP == GEMM_GROUP_ROWS && p.a_pad)) &&
                        n0 + BN <= p.N;
  const int nfull = interior ? (kend - kbeg) / TK : 0;

  LA la;
  LB lb;
  la.init(tid);
  lb.init(tid);
  // Fills LDS stage `buf` with K tile kt; readable after wait_tiles and
  // tile_barrier.
  auto load = [&](int kt, int buf) {
    const int k0 = kbeg + kt * TK;
    if (kt < nfull) {
      la.load_direct(p.A, p.lda, m0, k0, As[buf], wid);
      lb.load_direct(p.B, p.ldb, n0, k0, Bs[buf], wid);
    } else {
      la.template load_edge<VEC>(p.A, p.lda, m0, p.M, k0, kend, As[buf], tid);
      lb.template load_edge<VEC>(p.B, p.ldb, n0, p.N, k0, kend, Bs[buf], tid);
    }
  };

  // FOLD (two-level summation): the MFMAs of one GK-deep tile accumulate
  // into `blk`, which is added to `acc` after the tile, so rounding error
  // grows with GK + K/GK rather than K.  It is used for long K ranges (the
  // weight gradients, K = tokens, and the logits-gradient contraction, K =
  // vocabulary); it costs 5-9 % of throughput, so short-K products
  // accumulate in `acc` directly.
  v4f acc[MI][NI];
#pragma unroll
  for (int i = 0; i < MI; i++)
#pragma unroll
    for (int j = 0; j < NI; j++) acc[i][j] = (v4f){0.f, 0.f, 0.f, 0.f};

#pragma unroll
  for (int s = 0; s < S - 1; s++)
    if (s < nkt) load(s, s);
  for (int kt = 0; kt < nkt; kt++) {
    const int cur = kt % S;
    // Tiles kt+1 .. kt+S-2 may stay in flight.  (A tile loaded through
    // VGPRs completes before its LDS stores, which waits for everything
    // issued before it.)
    wait_tiles<PT, S - 2>(min(S - 2, nkt - 1 - kt));
    tile_barrier();
    // Stage (kt - 1) % S was last read in iteration kt - 1, before the barrier.
    if (kt + S - 1 < nkt) load(kt + S - 1, (kt + S - 1) % S);
    // one tile's MFMAs into t; `fresh`: the first MFMA starts from zero
    auto tile_mma = [&](v4f(&t)[MI][NI], auto fresh) {
#pragma unroll
      for (int gi = 0; gi < TK / 16 / WK; gi++) {
        const int g = gi * WK + wk;
        v4f fa[MI], fb[NI];
#pragma unroll
        for (int i = 0; i < MI; i++) fa[i] = LA::frag(As[cur], wm * TM + 16 * i, g, lane);
#pragma unroll
        for (int j = 0; j < NI; j++) fb[j] = LB::frag(Bs[cur], wn * TN + 16 * j, g, lane);
#pragma unroll
        for (int c = 0; c < 4; c++)
#pragma unroll
          for (int i = 0; i < MI; i++)
#pragma unroll
            for (int j = 0; j < NI; j++)
              t[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(
                  fa[i][c], fb[j][c],
                  (decltype(fresh)::value && gi == 0 && c == 0) ? (v4f){0.f, 0.f, 0.f, 0.f}
                                                                : t[i][j],
                  0, 0, 0);
      }
    };
    if constexpr (FOLD) {
      v4f blk[MI][NI];
      tile_mma(blk, std::true_type{});
#pragma unroll
      for (int i = 0; i < MI; i++)
#pragma unroll
        for (int j = 0; j < NI; j++) acc[i][j] += blk[i][j];
    } else {
      tile_mma(acc, std::false_type{});
    }
  }
  if constexpr (WK > 1) {
    // Wave groups 1..WK-1 park their sums in the (now idle) stage buffers;
    // group 0 adds them in group order.  The last iteration waited for all
    // loads (vmcnt(0)), so no LDS-DMA write is still in flight.
    float* red = &As[0][0];
    tile_barrier();
    if (wk > 0) {
#pragma unroll
      for (int i = 0; i < MI; i++)
#pragma unroll
        for (int j = 0; j < NI; j++)
#pragma unroll
          for (int r = 0; r < 4; r++)
            red[((((wk - 1) * WM * WN + wmn) * MI + i) * NI + j) * 256 + r * 64 + lane] =
                acc[i][j][r];
    }
    wait_vm_lgkm0<0>();
    tile_barrier();
    if (wk > 0) return;
#pragma unroll
    for (int v = 1; v < WK; v++)
#pragma unroll
      for (int i = 0; i < MI; i++)
#pragma unroll
        for (int j = 0; j < NI; j++)
#pragma unroll
          for (int r = 0; r < 4; r++)
            acc[i][j][r] += red[((((v - 1) * WM * WN + wmn) * MI + i) * NI + j) * 256 + r * 64 + lane];
  }
  // D of a 16x16 block: lane holds column (lane & 15), rows 4*(lane>>4)+r.
  if (GRP == GEMM_GROUP_K || p.splits == 1) {
    if (m0 + BM <= p.M && n0 + BN <= p.N) {
      if constexpr (MI == 4 && NI == 4 && WM * WN == 4 && WK == 1 && S == 2 &&
                    LA::SIZE == 4096 && LB::SIZE == 4096) {
        // 128 x 128 tiles: each wave stages its 64 x 64 outputs in one of
        // the four (idle) 16 KB stage buffers
        const bool rows16 = p.ldc % 4 == 0 && ((uintptr_t)p.C & 15) == 0 &&
                            (p.epi == EPI_STORE || p.epi == EPI_SOFTCAP ||
                             p.epi == EPI_ACCUM ||
                             (p.epi == EPI_RELU2_SAVE && !p.aux_out) ||
                             (p.ldaux % 4 == 0 &&
                              ((uintptr_t)(p.epi == EPI_RELU2_SAVE ? p.aux_out : p.aux) & 15) == 0));
        if (rows16) {
          tile_barrier();  // every wave's fragment reads of the stages are done
          float* Sw = wmn < 2 ? &As[wmn][0] : &Bs[wmn - 2][0];
          store_tile_staged_any(p, acc, m0 + wm * TM, n0 + wn * TN, lane, Sw);
          return;
        }
      }
      store_tile_any(p, acc, m0 + wm * TM, n0 + wn * TN, lane);
      return;
    }
#pragma unroll
    for (int i = 0; i < MI; i++)
#pragma unroll
      for (int j = 0; j < NI; j++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const int row = m0 + wm * TM + i * 16 + 4 * (lane >> 4) + r;
          const int col = n0 + wn * TN + j * 16 + (lane & 15);
          gemm_epilogue(p, row, col, acc[i][j][r]);
        }
    return;
  }
  // Split-K: this workgroup's partial sums; gemm_reduce_kernel adds them.
  // (rows mode: p.M is this group's end row; the partial buffer spans all rows)
  float* mine = p.part + (int64_t)split * p0.M * p.N;
  if (m0 + BM <= p.M && n0 + BN <= p.N) {
#pragma unroll
    for (int i = 0; i < MI; i++)
#pragma unroll
      for (int j = 0; j < NI; j++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const int row = m0 + wm * TM + i * 16 + 4 * (lane >> 4) + r;
          const int col = n0 + wn * TN + j * 16 + (lane & 15);
          mine[(int64_t)row * p.N + col] = acc[i][j][r];
        }
    return;
  }
#pragma unroll
  for (int i = 0; i < MI; i++)
#pragma unroll
    for (int j = 0; j < NI; j++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int row = m0 + wm * TM + i * 16 + 4 * (lane >> 4) + r;
        const int col = n0 + wn * TN + j * 16 + (lane & 15);
        if (row < p.M && col < p.N) mine[(int64_t)row * p.N + col] = acc[i][j][r];
      }
}

// Sums split-K partials in split order in float64 (deterministic) and applies
// the epilogue.
__global__ void gemm_reduce_kernel(GemmParams p) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = (int64_t)p.M * p.N;
  if (idx >= total) return;
  p.C += (int64_t)blockIdx.y * p.bsc;  // batched products
  p.part += (int64_t)blockIdx.y * p.splits * total;
  double s = 0.0;
  for (int z = 0; z < p.splits; z++) s += (double)p.part[(int64_t)z * total + idx];
  gemm_epilogue(p, (int)(idx / p.N), (int)(idx % p.N), (float)s);
}

template <int BM, int BN, int WM, int WN, int WK, int S, bool FOLD>
static void launch_cfg(const GemmParams& p, bool ak, bool bk, bool vec, int splits,
                       hipStream_t st, int batch = 1) {
  GemmParams q = p;
  q.tiles_m = (int)ceil_div(p.M, BM);
  q.tiles_n = (int)ceil_div(p.N, BN);
  q.splits = splits;
  dim3 grid(q.tiles_m * q.tiles_n * splits, batch);
  dim3 block(64 * WM * WN * WK);
#define GN_GEMM_LAUNCH(AK, BK, V)                                                             \
  hipLaunchKernelGGL((gemm_kernel<BM, BN, WM, WN, WK, S, FOLD, AK, BK, V, GEMM_GROUP_NONE>), \
                     grid, block, 0, st, q)
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

// Both operands K-contiguous only (x.W^T): tile shapes whose M/N-contiguous
// LDS layout would not divide into the workgroup's slots.
template <int BM, int BN, int WM, int WN, int WK, int S, int TK = GK>
static void launch_cfg_kk(const GemmParams& p, bool vec, int splits, hipStream_t st) {
  GemmParams q = p;
  q.tiles_m = (int)ceil_div(p.M, BM);
  q.tiles_n = (int)ceil_div(p.N, BN);
  q.splits = splits;
  dim3 grid(q.tiles_m * q.tiles_n * splits);
  dim3 block(64 * WM * WN * WK);
  if (vec)
    hipLaunchKernelGGL((gemm_kernel<BM, BN, WM, WN, WK, S, false, true, true, true, GEMM_GROUP_NONE, TK>),
                       grid, block, 0, st, q);
  else
    hipLaunchKernelGGL((gemm_kernel<BM, BN, WM, WN, WK, S, false, true, true, false, GEMM_GROUP_NONE, TK>),
                       grid, block, 0, st, q);
  GN_HIP(hipGetLastError());
}

// Expert-grouped launches.  Rows mode: p.M is the total row count (the sum
// over groups); the grid has one tile row per BM rows plus one per group
// (each group's last tile may be partial).  K mode: one "split" per group.
template <int BM, int BN, int WM, int WN, int WK, int S, bool FOLD, int GRP>
static void launch_grouped(const GemmParams& p, bool ak, bool bk, bool vec, hipStream_t st) {
  GemmParams q = p;
  q.tiles_m = GRP == GEMM_GROUP_ROWS ? (int)ceil_div(p.M, BM) + p.groups : (int)ceil_div(p.M, BM);
  q.tiles_n = (int)ceil_div(p.N, BN);
  if (GRP == GEMM_GROUP_K) {
    q.splits = p.groups;
    q.k_per_split = p.K;
  }
  dim3 grid(q.tiles_m * q.tiles_n * q.splits);
  dim3 block(64 * WM * WN * WK);
#define GN_GEMM_LAUNCH(AK, BK, V) \
  hipLaunchKernelGGL((gemm_kernel<BM, BN, WM, WN, WK, S, FOLD, AK, BK, V, GRP>), grid, block, 0, st, q)
  if constexpr (GRP == GEMM_GROUP_ROWS) {
    GN_CHECK(ak, "grouped gemm: rows mode needs a K-contiguous A");
    if (vec) {
      if (bk) GN_GEMM_LAUNCH(true, true, true);
      else GN_GEMM_LAUNCH(true, false, true);
    } else {
      if (bk) GN_GEMM_LAUNCH(true, true, false);
      else GN_GEMM_LAUNCH(true, false, false);
    }
  } else {
    GN_CHECK(!ak && !bk, "grouped gemm: K mode needs M- and N-contiguous operands");
    if (vec) GN_GEMM_LAUNCH(false, false, true);
    else GN_GEMM_LAUNCH(false, false, false);
  }
#undef GN_GEMM_LAUNCH
  GN_HIP(hipGetLastError());
}

static bool aligned16(const void* ptr) { return ((uintptr_t)ptr & 15) == 0; }

// ---------------------------------------------------------------------------
// Wide-tile engine for the large products: the train phase's Linear
// forward and backward products and the lm_head (training and rollout).
//
// One 256 x 256 output tile per workgroup of four waves (2 x 2), each wave
// owning 128 x 128 outputs: 256 accumulators per lane, held in the AGPR half
// of gfx950's 512-entry register file (one wave per SIMD).  K runs in
// 32-deep tiles through a two-stage LDS ring (2 x 64 KB of the 160 KB).
// The wave tile sets the operand traffic: a 16-deep k group is 16
// ds_read_b128 per wave for 256 MFMAs.
//
// The MFMA's row operand (src A, whose rows a lane's four D registers walk)
// is the N side of the product and the column operand the M side, so a
// lane's four results of a block are four consecutive columns of one row of
// C: the epilogue stores 16-byte vectors.
//
// Pipeline, K tile kt in stage kt & 1:
//   issue the group-1 fragment reads of tile kt
//   256 MFMAs on the group-0 fragments of tile kt
//   wait (own LDS reads, tile kt+1's loads), barrier
//   issue tile kt+2's loads into stage kt & 1 (every wave holds group 1)
//   issue the group-0 fragment reads of tile kt+1
//   256 MFMAs on the group-1 fragments of tile kt
// LDS latency hides behind MFMAs, a tile's loads have two tiles of MFMAs
// (16384 cycles) to land, and there is one barrier per tile.
//
// Long K ranges are split (at most KCHUNK deep per workgroup) and the
// partials summed in float64 in split order by gemm_reduce_kernel, which
// bounds float32 rounding growth as the two-level summation of gemm_kernel
// does.
// ---------------------------------------------------------------------------
namespace wide {

constexpr int TILE = 256;      // output tile edge (M and N)
constexpr int TK = 32;         // K depth of one LDS stage
constexpr int SZ = TILE * TK;  // floats per operand stage (32 KB)
constexpr int KCHUNK = 8192;   // deepest K range of one workgroup

// Zeros read in place of the K rows past a grouped K range (one row of a
// tile, 16 bytes per lane); never written.
__device__ __attribute__((aligned(16))) float zero_row[TILE];

// One operand of a workgroup of NW waves: its K tile moved into an LDS
// stage and read back as MFMA fragments.
//
// K-contiguous (X[d*ld + k]): LDS [256 d][32 k], 8 16-byte slots per row,
// slot column XOR-swizzled by (row & 7).  A fragment is one ds_read_b128 of
// 16 rows x 4 consecutive k per lane: lane (i, q) = (lane & 15, lane >> 4)
// reads row d + i, k = 16 g + 4 q .. + 3, and MFMA step c of the group
// takes component c (every k meets itself in both operands).
//
// Contiguous in d (X[k*ld + d]): LDS [32 k][256 d].  A read takes four
// consecutive d at one k: lane (i, q) reads k = 16 g + 4 q + c, d = base +
// 4 i .. + 3, for MFMA step c; component c' feeds block 4 b' + c', whose row
// i is d = 64 b' + 4 i + c'.  The 16 lanes of a q read 256 contiguous bytes.
//
// Global -> LDS: global_load_lds_dwordx4 drops lane l's 16 bytes at (wave
// base) + 16 l, so instruction t of wave w fills slots (t NW + w) 64 .. + 63
// and the lane -> address map places them.  The map is the same for every
// instruction up to a uniform row step, so a lane keeps one 32-bit offset
// and the instructions add scalar steps.  Tiles are never partial: a tile
// that would run past the operand's extent D (>= 256) is shifted back to
// end at D, and the epilogue skips the rows it shares with the tile before.
template <bool KC, int NW>
struct WOp {
  static constexpr int NI = SZ / 4 / (64 * NW);  // LDS-DMA instructions per thread and stage
  uint32_t loff;  // the lane's byte offset from the tile corner (d0, k0), instruction 0

  __device__ __forceinline__ void init(int64_t ld, int tid) {
    const int w = tid >> 6, l = tid & 63;
    if constexpr (KC)  // row w*8 + l/8, slot (l & 7) ^ (row & 7) = (l & 7) ^ (l >> 3)
      loff = (uint32_t)(((int64_t)(w * 8 + (l >> 3)) * ld + 4 * ((l & 7) ^ (l >> 3))) * 4);
    else  // row w, columns 4 l .. 4 l + 3
      loff = (uint32_t)(((int64_t)w * ld + 4 * l) * 4);
  }
  // bytes between the rows of instructions t and t + 1
  static __device__ __forceinline__ int64_t tstep(int64_t ld) {
    return (KC ? (int64_t)NW * 8 * ld : (int64_t)NW * ld) * 4;
  }
  static __device__ __forceinline__ const char* corner(const float* X, int64_t ld, int d0, int k0) {
    return reinterpret_cast<const char*>(KC ? X + (int64_t)d0 * ld + k0 : X + (int64_t)k0 * ld + d0);
  }
  // Instruction t of the K tile whose corner is at base.
  __device__ __forceinline__ void dma_one(const char* base, int64_t step, float* S, int w,
                                          int t) const {
    __builtin_amdgcn_global_load_lds((const void*)(base + t * step + loff),
                                     (lds_void*)(S + 4 * ((t * NW + w) * 64)), 16, 0, 0);
  }
  // As dma_one for a d-contiguous operand whose instruction t is K row
  // (tile's first row) + t NW + w: the row is read when ok, else the 16
  // bytes come from zl (the lane's slot of a zero row), so a K range may end
  // anywhere inside the tile.
  __device__ __forceinline__ void dma_one_k(const char* base, int64_t step, float* S, int w, int t,
                                            bool ok, const char* zl) const {
    static_assert(!KC, "K-row masking: d-contiguous operands");
    const char* a = ok ? base + t * step + loff : zl;
    __builtin_amdgcn_global_load_lds((const void*)a, (lds_void*)(S + 4 * ((t * NW + w) * 64)), 16,
                                     0, 0);
  }
  // Whole K tile at k0 of the tile starting at row d0.
  __device__ __forceinline__ void dma(const float* __restrict__ X, int64_t ld, int d0, int k0,
                                      float* S, int w) const {
    const char* base = corner(X, ld, d0, k0);
    const int64_t step = tstep(ld);
#pragma unroll
    for (int t = 0; t < NI; t++) dma_one(base, step, S, w, t);
  }
  // LDS float offset of the lane's first fragment read of k group g for
  // the rows starting at d (a multiple of 64); the others are immediates.
  static __device__ __forceinline__ int frag_base(int d, int g, int lane) {
    const int i = lane & 15, q = lane >> 4;
    if constexpr (KC) return (d + i) * TK + 4 * ((4 * g + q) ^ (i & 7));
    else return (16 * g + 4 * q) * TILE + d + 4 * i;
  }
  // The R/16 fragments of the R rows whose first read is at S + base.
  template <int R>
  static __device__ __forceinline__ void frags(const float* __restrict__ S, int base,
                                               v4f (&F)[R / 16]) {
    if constexpr (KC) {
#pragma unroll
      for (int b = 0; b < R / 16; b++)
        F[b] = *reinterpret_cast<const v4f*>(&S[base + 16 * b * TK]);
    } else {
#pragma unroll
      for (int bb = 0; bb < R / 64; bb++)
#pragma unroll
        for (int c = 0; c < 4; c++)
          F[4 * bb + c] = *reinterpret_cast<const v4f*>(&S[base + c * TILE + 64 * bb]);
    }
  }
  // Fragment j of the R/16 that frags() reads.
  template <int R>
  static __device__ __forceinline__ v4f frag(const float* __restrict__ S, int base, int j) {
    if constexpr (KC) return *reinterpret_cast<const v4f*>(&S[base + 16 * j * TK]);
    else return *reinterpret_cast<const v4f*>(&S[base + (j & 3) * TILE + 64 * (j >> 2)]);
  }
  // Operand of block b at MFMA step c.
  template <int N>
  static __device__ __forceinline__ float elem(const v4f (&F)[N], int b, int c) {
    if constexpr (KC) return F[b][c];
    else return F[(b >> 2) * 4 + c][b & 3];
  }
  // Row (within the wave's rows) of block b's MFMA row/column index i.
  static __device__ __forceinline__ int row(int b, int i) {
    if constexpr (KC) return 16 * b + i;
    else return 64 * (b >> 2) + 4 * i + (b & 3);
  }
};

// One MFMA accumulating in place in an AGPR quad.  Written as inline asm so
// that the accumulators are tied to their registers across the K loop (the
// builtin's untied destination let register allocation rotate the 256
// accumulators through copies inside the loop), and volatile so that the
// memory operations placed between MFMAs keep their source order.  No
// hazard needs wait states here: the fragments come from LDS (lgkmcnt waits
// are inserted for the asm's operands), the accumulators are written by
// nothing but these MFMAs, each accumulator is reused 64 MFMAs later, and
// the epilogue reads them after a vmcnt wait and s_nops (see the kernel).
__device__ __forceinline__ void mfma_acc(v4f& acc, float a, float b) {
  asm volatile("v_mfma_f32_16x16x4_f32 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}

// The MFMAs of one 16-deep k group: acc[J][I], J over the wave's M blocks,
// I over its N blocks.  after(n) runs after MFMA n (0-based) and issues
// the memory operations spread over the group.
template <bool AK, bool BK, int NW, int MI, int NI, class After>
__device__ __forceinline__ void group_mma(v4f (&acc)[MI][NI], const v4f (&fa)[MI],
                                          const v4f (&fb)[NI], After&& after) {
#pragma unroll
  for (int c = 0; c < 4; c++)
#pragma unroll
    for (int J = 0; J < MI; J++)
#pragma unroll
      for (int I = 0; I < NI; I++) {
        mfma_acc(acc[J][I], WOp<BK, NW>::elem(fb, I, c), WOp<AK, NW>::elem(fa, J, c));
        after((c * MI + J) * NI + I);
      }
}

// Four consecutive outputs (row m, columns n .. n + 3) through epilogue E;
// E == -1 stores split-K partials.  Same arithmetic as gemm_epilogue.
template <int E>
__device__ __forceinline__ void store4(const GemmParams& p, float* part, int m, int n, v4f v) {
  if constexpr (E == -1) {
    *reinterpret_cast<v4f*>(&part[(int64_t)m * p.N + n]) = v;
  } else {
    float* c = &p.C[(int64_t)m * p.ldc + n];
    if constexpr (E == EPI_STORE) {
      *reinterpret_cast<v4f*>(c) = v * p.alpha;
    } else if constexpr (E == EPI_ADD_SRC) {
      *reinterpret_cast<v4f*>(c) =
          v + *reinterpret_cast<const v4f*>(&p.aux[(int64_t)m * p.ldaux + n]);
    } else if constexpr (E == EPI_ACCUM) {
      *reinterpret_cast<v4f*>(c) = *reinterpret_cast<const v4f*>(c) + v;
    } else if constexpr (E == EPI_SOFTCAP) {
      v4f o;
#pragma unroll
      for (int r = 0; r < 4; r++) o[r] = softcap15(v[r]);
      *reinterpret_cast<v4f*>(c) = o;
    } else if constexpr (E == EPI_RELU2_SAVE || E == EPI_RELU2_SAVE + 16) {
      if constexpr (E == EPI_RELU2_SAVE)
        *reinterpret_cast<v4f*>(&p.aux_out[(int64_t)m * p.ldaux + n]) = v;
      v4f o;
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const float u = v[r] < 0.f ? 0.f : v[r];
        o[r] = u * u;
      }
      *reinterpret_cast<v4f*>(c) = o;
    } else {
      static_assert(E == EPI_DRELU2, "epilogue kind");
      const v4f u = *reinterpret_cast<const v4f*>(&p.aux[(int64_t)m * p.ldaux + n]);
      v4f o;
#pragma unroll
      for (int r = 0; r < 4; r++) o[r] = u[r] > 0.f ? (v[r] * 2.f) * u[r] : 0.f;
      *reinterpret_cast<v4f*>(c) = o;
    }
  }
}

// The wave's outputs, whose first row and column are mw, nw; rows before m0
// and columns before n0 (a shifted tile's overlap with the tile before) are
// skipped.  N % 4 == 0, and nw, n0 are multiples of 4.  Epilogues that read
// (the residual add, the ReLU^2 backward, the accumulate) load one block
// row ahead: row J+1's 16-byte reads are in flight while row J is combined
// and stored, instead of a full memory round trip per store.
template <int E, bool AK, bool BK, int NW, int MI, int NI>
__device__ __forceinline__ void store_wave(const GemmParams& p, float* part,
                                           const v4f (&acc)[MI][NI], int mw, int nw, int m0,
                                           int n0, int lane) {
  const int q = lane >> 4;
  const bool full = mw >= m0 && nw >= n0;
  auto row = [&](int J) { return mw + WOp<AK, NW>::row(J, lane & 15); };
  auto col = [&](int u) {
    return BK ? nw + 16 * u + 4 * q : nw + 64 * (u >> 2) + 16 * q + 4 * (u & 3);
  };
  auto val = [&](int J, int u) {
    v4f v;
    if constexpr (BK) {
      v = acc[J][u];
    } else {
#pragma unroll
      for (int c = 0; c < 4; c++) v[c] = acc[J][4 * (u >> 2) + c][u & 3];
    }
    return v;
  };
  constexpr bool READS = E == EPI_ADD_SRC || E == EPI_DRELU2 || E == EPI_ACCUM;
  if constexpr (READS) {
    const float* src = E == EPI_ACCUM ? p.C : p.aux;
    const int64_t ld = E == EPI_ACCUM ? p.ldc : p.ldaux;
    v4f cur[NI], nxt[NI];
#pragma unroll
    for (int u = 0; u < NI; u++)
      cur[u] = *reinterpret_cast<const v4f*>(&src[(int64_t)row(0) * ld + col(u)]);
#pragma unroll
    for (int J = 0; J < MI; J++) {
      const int m = row(J);
      if (J + 1 < MI) {
#pragma unroll
        for (int u = 0; u < NI; u++)
          nxt[u] = *reinterpret_cast<const v4f*>(&src[(int64_t)row(J + 1) * ld + col(u)]);
      }
#pragma unroll
      for (int u = 0; u < NI; u++) {
        const int n = col(u);
        const v4f v = val(J, u), x = cur[u];
        v4f o;
        if constexpr (E == EPI_DRELU2) {
#pragma unroll
          for (int r = 0; r < 4; r++) o[r] = x[r] > 0.f ? (v[r] * 2.f) * x[r] : 0.f;
        } else {
          o = x + v;  // ADD_SRC: acc + aux; ACCUM: C + acc (same sum)
        }
        if (full || (m >= m0 && n >= n0))
          *reinterpret_cast<v4f*>(&p.C[(int64_t)m * p.ldc + n]) = o;
      }
#pragma unroll
      for (int u = 0; u < NI; u++) cur[u] = nxt[u];
    }
  } else {
#pragma unroll
    for (int J = 0; J < MI; J++) {
      const int m = row(J);
#pragma unroll
      for (int u = 0; u < NI; u++) {
        const int n = col(u);
        if (full || (m >= m0 && n >= n0)) store4<E>(p, part, m, n, val(J, u));
      }
    }
  }
}

// As store_wave for a 128 x 128 wave tile (MI = NI = 8), the stores going
// through the wave's own 32 KB LDS region S, 64 rows at a time, so that each
// store instruction writes two whole 512-byte row pieces instead of 16 rows
// x 64 bytes (a 256 x 256 tile's epilogue: 8.2 -> 5.9 us, same bits).  The
// products of (row, 4 columns) go straight from the accumulators to row
// `row` of S, 16-byte slot (column / 4) ^ sw(row), sw a bijection on the 16
// rows that one ds_write_b128 pass touches; they are read back two rows per
// instruction and the epilogue is applied there, the reading epilogues'
// operand (aux or C) fetched in the same row-wise pattern before the phase's
// staging writes, so that its latency overlaps them.  Each wave reads back
// only what it wrote, in order, so a wave-scope fence (compiler ordering)
// separates the passes.
template <int E, bool AK, bool BK, int NW, int MI, int NI>
__device__ __forceinline__ void store_wave_staged(const GemmParams& p, float* part,
                                                  const v4f (&acc)[MI][NI], int mw, int nw,
                                                  int m0, int n0, int lane, float* S) {
  static_assert(MI == 8 && NI == 8, "128 x 128 wave tiles");
  const int q = lane >> 4, i = lane & 15;
  const bool full = mw >= m0 && nw >= n0;
  auto sw = [](int lr) { return AK ? (lr & 15) : ((lr >> 2) & 15); };
  auto lcol = [&](int u) { return BK ? 16 * u + 4 * q : 64 * (u >> 2) + 16 * q + 4 * (u & 3); };
  auto val = [&](int J, int u) {
    v4f v;
    if constexpr (BK) {
      v = acc[J][u];
    } else {
#pragma unroll
      for (int c = 0; c < 4; c++) v[c] = acc[J][4 * (u >> 2) + c][u & 3];
    }
    return v;
  };
  auto wave_fence = [] {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  };
  constexpr bool READS = E == EPI_ADD_SRC || E == EPI_DRELU2 || E == EPI_ACCUM;
  const float* src = E == EPI_ACCUM ? p.C : p.aux;
  const int64_t lds = E == EPI_ACCUM ? p.ldc : p.ldaux;
  const int ls = lane & 31;
#pragma unroll
  for (int ph = 0; ph < 2; ph++) {
    // the reading epilogues' operand for this phase's rows, requested before
    // the staging writes so that its latency overlaps them
    v4f xs[READS ? 32 : 1];
    if constexpr (READS) {
#pragma unroll
      for (int t = 0; t < 32; t++)
        xs[t] = *reinterpret_cast<const v4f*>(
            &src[(int64_t)(mw + 64 * ph + 2 * t + (lane >> 5)) * lds + nw + 4 * ls]);
    }
#pragma unroll
    for (int J = 4 * ph; J < 4 * ph + 4; J++) {
      const int lr = WOp<AK, NW>::row(J, i) & 63;
#pragma unroll
      for (int u = 0; u < NI; u++)
        *reinterpret_cast<v4f*>(&S[lr * 128 + 4 * ((lcol(u) >> 2) ^ sw(lr))]) = val(J, u);
    }
    wave_fence();
#pragma unroll
    for (int t = 0; t < 32; t++) {
      const int lr = 2 * t + (lane >> 5);
      const v4f v = *reinterpret_cast<const v4f*>(&S[lr * 128 + 4 * (ls ^ sw(lr))]);
      const int m = mw + 64 * ph + lr, n = nw + 4 * ls;
      if (full || (m >= m0 && n >= n0)) {
        float* c = &p.C[(int64_t)m * p.ldc + n];
        if constexpr (E == -1) {
          *reinterpret_cast<v4f*>(&part[(int64_t)m * p.N + n]) = v;
        } else if constexpr (E == EPI_RELU2_SAVE || E == EPI_RELU2_SAVE + 16) {
          if constexpr (E == EPI_RELU2_SAVE)
            *reinterpret_cast<v4f*>(&p.aux_out[(int64_t)m * p.ldaux + n]) = v;
          v4f o;
#pragma unroll
          for (int r = 0; r < 4; r++) {
            const float u = v[r] < 0.f ? 0.f : v[r];
            o[r] = u * u;
          }
          *reinterpret_cast<v4f*>(c) = o;
        } else if constexpr (E == EPI_STORE) {
          *reinterpret_cast<v4f*>(c) = v * p.alpha;
        } else if constexpr (E == EPI_DRELU2) {
          v4f o;
#pragma unroll
          for (int r = 0; r < 4; r++) o[r] = xs[t][r] > 0.f ? (v[r] * 2.f) * xs[t][r] : 0.f;
          *reinterpret_cast<v4f*>(c) = o;
        } else {
          static_assert(E == EPI_ADD_SRC || E == EPI_ACCUM, "epilogue kind");
          *reinterpret_cast<v4f*>(c) = xs[t] + v;  // ADD_SRC: aux + acc; ACCUM: C + acc
        }
      }
    }
    wave_fence();
  }
}

// 256 x 256 tile per workgroup of WM x WN waves (wave tile 256/WM rows of M
// by 256/WN columns of N), epilogue E (-1: split-K partials).  Every K range
// is a whole number of tile pairs (K and k_per_split multiples of 2 TK), so
// the loop body is two tiles, one per stage, and every LDS address is an
// immediate from a per-lane base.  The stages are separate arrays: the LDS
// reads of one stage provably do not alias the loads in flight into the
// other.
//
// GKM (expert-grouped K, GEMM_GROUP_K, both operands d-contiguous): split z
// is (group g, part c) of the p.splits / p.groups parts of group g's rows
// goff[g] .. goff[g+1], cut evenly; the range starts at its first row (no
// alignment needed: every DMA instruction is one K row) and the rows of its
// last tile pair past the range read zeros.  Partials land at split z, so
// gemm_reduce_kernel sums group g's parts over grid y.
template <bool AK, bool BK, int WM, int WN, int E, bool GKM = false>
__global__ __launch_bounds__(64 * WM * WN, (WM * WN) / 4) void gemm_wide_kernel(GemmParams p) {
  static_assert(!GKM || (!AK && !BK && E == -1), "grouped K: d-contiguous operands, partials");
  constexpr int NW = WM * WN, TM = TILE / WM, TN = TILE / WN, MI = TM / 16, NI = TN / 16;
  using LA = WOp<AK, NW>;
  using LB = WOp<BK, NW>;
  constexpr int PT = LA::NI + LB::NI;  // LDS-DMA instructions per thread and K tile
  __shared__ __attribute__((aligned(16))) float As0[SZ];
  __shared__ __attribute__((aligned(16))) float Bs0[SZ];
  __shared__ __attribute__((aligned(16))) float As1[SZ];
  __shared__ __attribute__((aligned(16))) float Bs1[SZ];
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = w % WM, wn = w / WM;
  int tm, tn, split;
  tile_coords(p, tm, tn, split);
  // the tile's first row and column, and where it is loaded from (a tile
  // past the end is shifted back to end at M resp. N)
  const int m0 = tm * TILE, n0 = tn * TILE;
  const int ms = min(m0, p.M - TILE), ns = min(n0, p.N - TILE);
  int kbeg = split * p.k_per_split, kend = min(p.K, kbeg + p.k_per_split);
  if constexpr (GKM) {
    const int parts = p.splits / p.groups, g = split / parts, c = split - g * parts;
    const int b = p.goff[g], cnt = p.goff[g + 1] - b, per = (cnt + parts - 1) / parts;
    kbeg = b + min(c * per, cnt);
    kend = b + min(c * per + per, cnt);
  }
  // even (GKM: rounded up to a tile pair, the rows past kend masked)
  const int nkt = kend <= kbeg ? 0 : GKM ? 2 * ((kend - kbeg + 2 * TK - 1) / (2 * TK))
                                         : (kend - kbeg) / TK;
  const char* zl = reinterpret_cast<const char*>(zero_row) + 16 * lane;
  LA la;
  LB lb;
  la.init(p.lda, tid);
  lb.init(p.ldb, tid);
  // the first two K tiles (the loop issues the others; those past the end
  // re-read the last tile into a stage nobody reads again)
  auto load = [&](int kt, float* sa, float* sb) {
    const int k0 = kbeg + kt * TK;
    if constexpr (GKM) {
      const char* ga = LA::corner(p.A, p.lda, ms, k0);
      const char* gb = LB::corner(p.B, p.ldb, ns, k0);
      const int64_t sa_ = LA::tstep(p.lda), sb_ = LB::tstep(p.ldb);
#pragma unroll
      for (int t = 0; t < LA::NI; t++) la.dma_one_k(ga, sa_, sa, w, t, k0 + t * NW + w < kend, zl);
#pragma unroll
      for (int t = 0; t < LB::NI; t++) lb.dma_one_k(gb, sb_, sb, w, t, k0 + t * NW + w < kend, zl);
    } else {
      la.dma(p.A, p.lda, ms, k0, sa, w);
      lb.dma(p.B, p.ldb, ns, k0, sb, w);
    }
  };
  const int ab0 = LA::frag_base(wm * TM, 0, lane), ab1 = LA::frag_base(wm * TM, 1, lane);
  const int bb0 = LB::frag_base(wn * TN, 0, lane), bb1 = LB::frag_base(wn * TN, 1, lane);

  v4f acc[MI][NI];
#pragma unroll
  for (int J = 0; J < MI; J++)
#pragma unroll
    for (int I = 0; I < NI; I++) acc[J][I] = (v4f){0.f, 0.f, 0.f, 0.f};
  v4f fa0[MI], fb0[NI], fa1[MI], fb1[NI];
  if (nkt > 0) {
    load(0, As0, Bs0);
    load(1, As1, Bs1);
    wait_vm_lgkm0<PT>();
    tile_barrier();
    LA::template frags<TM>(As0, ab0, fa0);
    LB::template frags<TN>(Bs0, bb0, fb0);
  }
  // One K tile kt in stage (CA, CB); (XA, XB) holds tile kt+1.  MFMA n of a
  // group is followed by memory operation n - 1 (n >= 1) of that group's
  // list: first half, the group-1 fragment reads of tile kt; second half,
  // the loads of tile kt+2 into (CA, CB), then the group-0 fragment reads
  // of tile kt+1.
  auto tile = [&](int kt, float* CA, float* CB, float* XA, float* XB) {
    group_mma<AK, BK, NW>(acc, fa0, fb0, [&](int n) {
      const int o = n - 1;
      if (o >= 0 && o < MI) fa1[o] = LA::template frag<TM>(CA, ab1, o);
      else if (o >= MI && o < MI + NI) fb1[o - MI] = LB::template frag<TN>(CB, bb1, o - MI);
    });
    // own fragment reads done; tile kt+1 (the only loads in flight) landed
    wait_vm_lgkm0<0>();
    tile_barrier();
    // stage (CA, CB) is free: every wave holds its group-1 fragments
    const int k2 = kbeg + min(kt + 2, nkt - 1) * TK;
    const char* ga = LA::corner(p.A, p.lda, ms, k2);
    const char* gb = LB::corner(p.B, p.ldb, ns, k2);
    const int64_t sa = LA::tstep(p.lda), sb = LB::tstep(p.ldb);
    group_mma<AK, BK, NW>(acc, fa1, fb1, [&](int n) {
      const int o = n - 1;
      if (o >= 0 && o < PT) {
        if constexpr (GKM) {
          if (o < LA::NI) la.dma_one_k(ga, sa, CA, w, o, k2 + o * NW + w < kend, zl);
          else lb.dma_one_k(gb, sb, CB, w, o - LA::NI, k2 + (o - LA::NI) * NW + w < kend, zl);
        } else {
          if (o < LA::NI) la.dma_one(ga, sa, CA, w, o);
          else lb.dma_one(gb, sb, CB, w, o - LA::NI);
        }
      } else if (o >= PT && o < PT + MI) fa0[o - PT] = LA::template frag<TM>(XA, ab0, o - PT);
      else if (o >= PT + MI && o < PT + MI + NI)
        fb0[o - PT - MI] = LB::template frag<TN>(XB, bb0, o - PT - MI);
    });
  };
  for (int kt = 0; kt < nkt; kt += 2) {
    tile(kt, As0, Bs0, As1, Bs1);
    tile(kt + 1, As1, Bs1, As0, Bs0);
    // wait states between the last MFMAs and any accumulator copy the
    // compiler places at the loop's head (gonano_amd/isa_check checks the
    // gap)
    asm volatile("s_nop 7\n\ts_nop 7");
  }
  // the loads issued past the last tile; then 24 wait states before the
  // accumulators are read (at least what an MFMA's result needs)
  wait_vm_lgkm0<0>();
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7");

  float* part = E == -1 ? p.part + (int64_t)split * p.M * p.N : nullptr;
  // every wave's loads into the stages have landed and its fragment reads
  // are done: each wave takes one stage array as its store staging region
  tile_barrier();
  float* S = w == 0 ? As0 : w == 1 ? Bs0 : w == 2 ? As1 : Bs1;
  store_wave_staged<E, AK, BK, NW>(p, part, acc, ms + wm * TM, ns + wn * TN, m0, n0, lane, S);
}

}  // namespace wide

// The wide kernel for operand layouts (AK, BK) and epilogue E, or null
// when that combination has no instance (gemm_kernel takes it).  The
// instances are those the session's products use: x.W^T (forward,
// lm_head), g.W (input gradients), g^T.x (weight gradients), and the
// split-K partials (E == -1) of each.
typedef void (*WideKernel)(GemmParams);
static WideKernel wide_kernel(bool ak, bool bk, int e) {
  using namespace wide;
  constexpr int WM = 2, WN = 2;
  if (ak && bk) {
    switch (e) {
      case -1: return gemm_wide_kernel<true, true, WM, WN, -1>;
      case EPI_STORE: return gemm_wide_kernel<true, true, WM, WN, EPI_STORE>;
      case EPI_ADD_SRC: return gemm_wide_kernel<true, true, WM, WN, EPI_ADD_SRC>;
      case EPI_RELU2_SAVE: return gemm_wide_kernel<true, true, WM, WN, EPI_RELU2_SAVE>;
      case EPI_RELU2_SAVE + 16: return gemm_wide_kernel<true, true, WM, WN, EPI_RELU2_SAVE + 16>;
    }
  } else if (ak && !bk) {
    switch (e) {
      case -1: return gemm_wide_kernel<true, false, WM, WN, -1>;
      case EPI_STORE: return gemm_wide_kernel<true, false, WM, WN, EPI_STORE>;
      case EPI_ACCUM: return gemm_wide_kernel<true, false, WM, WN, EPI_ACCUM>;
      case EPI_DRELU2: return gemm_wide_kernel<true, false, WM, WN, EPI_DRELU2>;
    }
  } else if (!ak && !bk) {
    switch (e) {
      case -1: return gemm_wide_kernel<false, false, WM, WN, -1>;
      case EPI_STORE: return gemm_wide_kernel<false, false, WM, WN, EPI_STORE>;
      case EPI_ACCUM: return gemm_wide_kernel<false, false, WM, WN, EPI_ACCUM>;
    }
  }
  return nullptr;
}

// Expert-grouped K (GEMM_GROUP_K: the MoE experts' weight gradients, each a
// reduction over its expert's rows) on the wide-tile engine: each group's
// rows are cut into `parts` even ranges, one workgroup per (tile, group,
// part) writing a partial; gemm_reduce_kernel sums each group's parts
// (float64, part order) into its output over grid y and applies the
// epilogue.  parts gives whole rounds of the CUs with ranges of about 1024
// rows or more on average.  The group sizes live on the device, so a range
// may be empty (its partial is zero) or shorter than a tile pair (masked).
static bool gemm_wide_grouped_k(const GemmDesc& d, GemmParams p, bool vec, hipStream_t st,
                                DeviceArena* ws) {
  using namespace wide;
  if (d.group != GEMM_GROUP_K || d.defer || d.force_splits > 0 || !vec) return false;
  if (d.a_kcontig || d.b_kcontig || (d.epi != EPI_STORE && d.epi != EPI_ACCUM)) return false;
  if (d.M < TILE || d.N < TILE || d.M % 4 || d.N % 4) return false;
  // GN_GEMM_WIDE_GROUPED_K=0 keeps these products on gemm_kernel (A/B runs)
  if (const char* e = std::getenv("GN_GEMM_WIDE_GROUPED_K"); e && std::atoi(e) == 0) return false;
  const int64_t tm = ceil_div(d.M, TILE), tn = ceil_div(d.N, TILE), tiles = tm * tn;
  // padding: at most 1/8 of the MFMA work on rows or columns past the product
  if ((double)(tm * TILE) * (double)(tn * TILE) > 1.125 * (double)d.M * (double)d.N) return false;
  const int64_t cus = 256, per_group = tiles * d.groups;
  int64_t min_wg = (3 * cus) / 4;
  if (const char* e = std::getenv("GN_GEMM_WIDE_MIN")) {
    min_wg = std::max(1, std::atoi(e));
  } else if ((double)d.M * d.N * d.K < (double)(1 << 28)) {
    return false;
  }
  const int64_t avg = d.K / d.groups;
  const int pmax = (int)std::max<int64_t>(1, std::min<int64_t>(64, avg / 1024));
  int parts = 1;
  double best = -1.0;
  for (int s = 1; s <= pmax; s++) {
    const int64_t wg = per_group * s;
    const double eff = (double)wg / (double)(ceil_div(wg, cus) * cus);
    if (eff > best + 1e-9) {
      best = eff;
      parts = s;
    }
    if (eff >= 0.999) break;
  }
  // GN_GEMM_WIDE_PARTS: another part count (tests: several parts of small
  // groups, so that ranges end inside a tile pair or are empty)
  if (const char* e = std::getenv("GN_GEMM_WIDE_PARTS")) parts = std::min(64, std::max(1, std::atoi(e)));
  if (per_group * parts < min_wg) return false;
  GN_CHECK(ws != nullptr, "gemm: grouped split-K needs a workspace");
  p.part = ws->get<float>("gemm_splitk", (size_t)parts * d.groups * d.M * d.N);
  p.tiles_m = (int)tm;
  p.tiles_n = (int)tn;
  p.splits = parts * d.groups;
  p.k_per_split = d.K;
  hipLaunchKernelGGL((gemm_wide_kernel<false, false, 2, 2, -1, true>),
                     dim3((unsigned)(per_group * parts)), dim3(256), 0, st, p);
  GN_HIP(hipGetLastError());
  p.splits = parts;
  p.bsc = d.group_stride;
  const int64_t total = (int64_t)d.M * d.N;
  hipLaunchKernelGGL(gemm_reduce_kernel, dim3((unsigned)ceil_div(total, 256), (unsigned)d.groups),
                     dim3(256), 0, st, p);
  GN_HIP(hipGetLastError());
  return true;
}

// Runs d on the wide-tile engine when it suits the product: large enough to
// fill the chip with 256 x 256 tiles (after K splits), little padding, K at
// least 64, and the 16-byte alignment its vector loads and stores need.
// Returns false otherwise (gemm_kernel takes it).
static bool gemm_wide(const GemmDesc& d, GemmParams p, bool vec, hipStream_t st,
                      DeviceArena* ws) {
  using namespace wide;
  if (d.group != GEMM_GROUP_NONE || d.defer || d.force_splits > 0 || !vec) return false;
  // GN_GEMM_WIDE=0 leaves every plain product to gemm_kernel (tests)
  if (const char* e = std::getenv("GN_GEMM_WIDE"); e && std::atoi(e) == 0) return false;
  if ((double)d.M * d.N * d.K < (double)(1 << 28)) return false;
  if (d.M < TILE || d.N < TILE) return false;
  if (d.N % 4 || d.ldc % 4 || !aligned16(d.C)) return false;
  if (!d.a_kcontig && d.M % 4) return false;
  const bool uses_aux = d.epi == EPI_ADD_SRC || d.epi == EPI_DRELU2;
  if (uses_aux && (!aligned16(d.aux) || d.ldaux % 4)) return false;
  if (d.epi == EPI_RELU2_SAVE && d.aux_out && (!aligned16(d.aux_out) || d.ldaux % 4)) return false;
  // The engine runs K in whole 64-deep tile pairs: a K that is not a
  // multiple of 64 (the weight gradients' token counts, 16 x 8703 or
  // B x 1535) leaves its last K % 64 values to one more split, a
  // gemm_kernel launch over the whole output writing that split's partial;
  // gemm_reduce_kernel adds it after the engine's splits.
  const int rem = d.K % (2 * TK), Kw = d.K - rem;
  if (Kw < 2 * TK) return false;
  const int64_t tm = ceil_div(d.M, TILE), tn = ceil_div(d.N, TILE), tiles = tm * tn;
  // padding: at most 1/8 of the MFMA work on rows or columns past the product
  if ((double)(tm * TILE) * (double)(tn * TILE) > 1.125 * (double)d.M * (double)d.N) return false;
  const int64_t cus = 256;
  int splits = (int)ceil_div(Kw, KCHUNK);
  {
    // more splits (each at least 1024 deep) while that makes whole rounds
    // of the CUs fuller
    const int smin = splits, smax = std::max<int>(smin, (int)std::min<int64_t>(64, Kw / 1024));
    double best = -1.0;
    for (int s = smin; s <= smax; s++) {
      const int64_t wg = tiles * s;
      const double eff = (double)wg / (double)(ceil_div(wg, cus) * cus);
      if (eff > best + 1e-9) {
        best = eff;
        splits = s;
      }
      if (eff >= 0.999) break;
    }
  }
  const int kps = (int)ceil_div(ceil_div(Kw, splits), 2 * TK) * 2 * TK;
  splits = (int)ceil_div(Kw, kps);
  // at least 3/4 of a round of the CUs (GN_GEMM_WIDE_MIN: another minimum
  // workgroup count; tests take every eligible product with 1)
  int64_t min_wg = (3 * cus) / 4;
  if (const char* e = std::getenv("GN_GEMM_WIDE_MIN")) min_wg = std::max(1, std::atoi(e));
  if (tiles * splits < min_wg) return false;
  const int parts = splits + (rem > 0 ? 1 : 0);  // partial sums, the remainder's last
  int e = parts > 1 ? -1 : d.epi;
  if (e == EPI_RELU2_SAVE && !d.aux_out) e = EPI_RELU2_SAVE + 16;
  const WideKernel kern = wide_kernel(d.a_kcontig, d.b_kcontig, e);
  if (!kern) return false;
  p.tiles_m = (int)tm;
  p.tiles_n = (int)tn;
  p.splits = splits;
  p.k_per_split = kps;
  p.K = Kw;
  if (parts > 1) {
    GN_CHECK(ws != nullptr, "gemm: split-K needs a workspace");
    p.part = ws->get<float>("gemm_splitk", (size_t)parts * d.M * d.N);
  }
  hipLaunchKernelGGL(kern, dim3((unsigned)(tiles * splits)), dim3(256), 0, st, p);
  GN_HIP(hipGetLastError());
  if (rem > 0) {  // K values [Kw, K): a plain product into the last partial
    GemmParams q = p;
    q.A = d.a_kcontig ? d.A + Kw : d.A + (int64_t)Kw * d.lda;
    q.B = d.b_kcontig ? d.B + Kw : d.B + (int64_t)Kw * d.ldb;
    q.K = rem;
    q.k_per_split = rem;
    q.C = p.part + (int64_t)splits * d.M * d.N;
    q.ldc = d.N;
    q.epi = EPI_STORE;
    q.alpha = 1.f;
    q.aux = nullptr;
    q.aux_out = nullptr;
    q.part = nullptr;
    launch_cfg<128, 128, 2, 2, 1, 2, false>(q, d.a_kcontig, d.b_kcontig, vec, 1, st);
  }
  if (parts > 1) {
    p.splits = parts;
    const int64_t total = (int64_t)d.M * d.N;
    hipLaunchKernelGGL(gemm_reduce_kernel, dim3((unsigned)ceil_div(total, 256)), dim3(256), 0, st,
                       p);
    GN_HIP(hipGetLastError());
  }
  return true;
}

// ---------------------------------------------------------------------------
// Slim-tile engine for the decode projections: x.W^T (both operands
// K-contiguous) with M the decode batch (a few hundred rows), where the
// whole product is a few microseconds of MFMA work spread over 256 CUs.
//
// One 32 x BN output tile (BN = 96, 128 or 160) per workgroup of four waves
// (2 x 2), each wave owning 16 rows x BN/2 columns: BN/32 accumulator
// blocks, in AGPRs, by the same in-place inline-asm MFMAs as the wide
// engine.  A workgroup's K range is short (a few dozen 32-deep tiles), so
// what bounds it is the latency of the first loads and of every tile's
// loads behind the MFMAs: the tiles go through an S-stage LDS ring (S - 1
// tiles in flight, one 16-24 KB stage each, up to 144 KB), enough to cover
// ~2 us of load latency with MFMA work at one workgroup per CU.
//
// Pipeline, K tile kt in stage kt % S (its group-0 fragments in registers):
//   the group-0 MFMAs, with the group-1 fragment reads of tile kt between
//   wait (own LDS reads; tile kt+1's loads), barrier
//   the group-1 MFMAs, with the loads of tile kt+S into stage kt % S and
//   the group-0 fragment reads of tile kt+1 between
// Every stage is its own LDS array (the loop is unrolled S times), so the
// compiler can tell that the reads of one stage do not alias the loads in
// flight into the others and inserts no wait for them.
//
// Split K ranges either go to a consumer that sums them (deferred sums,
// PendingSum) or to gemm_reduce_kernel, both in float64 in split order.
// ---------------------------------------------------------------------------
namespace slim {

constexpr int BM = 32;  // tile rows
constexpr int TK = 32;  // K depth of one LDS stage
constexpr int NW = 4;   // waves per workgroup (2 x 2)
constexpr int MAXS = 8;  // deepest ring

// One K-contiguous operand of R rows (R a multiple of 32) in an LDS stage:
// [R][TK] floats, 8 16-byte slots per row, the slot column XOR-swizzled by
// (row & 7) so that the fragment reads (16 rows x 4 k per 16 lanes) hit
// distinct banks.  DMA instruction t of wave w fills slots (t NW + w) 64 ..
// + 63, i.e. rows 8 (t NW + w) .. + 7, lane l taking row + (l >> 3) and
// logical slot (l & 7) ^ (l >> 3); one 32-bit lane offset from the tile
// corner serves every instruction (a uniform row step apart).
template <int R>
struct SOp {
  static_assert(R % 32 == 0, "operand rows");
  static constexpr int NI = R / 32;  // DMA instructions per thread and stage
  static __device__ __forceinline__ uint32_t lane_off(int64_t ld, int tid) {
    const int w = tid >> 6, l = tid & 63;
    return (uint32_t)(((int64_t)(w * 8 + (l >> 3)) * ld + 4 * ((l & 7) ^ (l >> 3))) * 4);
  }
  static __device__ __forceinline__ void dma_one(const char* corner, uint32_t off, int64_t step,
                                                 float* S, int w, int t) {
    __builtin_amdgcn_global_load_lds((const void*)(corner + t * step + off),
                                     (lds_void*)(S + 4 * ((t * NW + w) * 64)), 16, 0, 0);
  }
  // LDS float offset of lane's fragment read of k group g, rows d .. d + 15
  // (d a multiple of 16)
  static __device__ __forceinline__ int frag_off(int d, int g, int lane) {
    const int i = lane & 15, q = lane >> 4;
    return (d + i) * TK + 4 * ((4 * g + q) ^ (i & 7));
  }
};

// Zeros standing in for the K tiles past the end of a workgroup's range (up
// to 160 rows of one TK-deep tile, row stride TK); never written.
__device__ __attribute__((aligned(16))) float zero_tile[160 * TK];

// Calls f(integral_constant<I>) for I = 0 .. N-1.
template <int I, int N, class F>
__device__ __forceinline__ void unroll(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    unroll<I + 1, N>(f);
  }
}

// The K loop runs a whole number of rounds of S tiles with no branch inside
// (a branch between the loads and the reads of the ring would make the
// compiler wait for every load in flight before the reads); the tiles past
// the workgroup's range are loaded from zero_tile and add nothing.
template <int BN, int S, int E>
__global__ __launch_bounds__(64 * NW, 1) void gemm_slim_kernel(GemmParams p) {
  constexpr int NB = BN / 32;  // accumulator blocks per wave (16 x 16 NB wave tile)
  constexpr int SZ = (BM + BN) * TK;
  using LA = SOp<BM>;
  using LB = SOp<BN>;
  constexpr int PT = LA::NI + LB::NI;  // DMA instructions per thread and stage
  static_assert(S >= 2 && S <= MAXS && PT * (S - 1) < 64, "ring depth");
  static_assert(BN <= 160, "zero tile rows");
  static_assert(4 * NB - 1 >= PT + 1 + NB, "memory operations fit between the group's MFMAs");
  __shared__ __attribute__((aligned(16))) float S0[SZ], S1[SZ], S2[SZ], S3[SZ], S4[SZ], S5[SZ],
      S6[SZ], S7[SZ];
  auto stage = [&](auto I) -> float* {
    constexpr int i = decltype(I)::value % S;
    if constexpr (i == 0) return S0;
    else if constexpr (i == 1) return S1;
    else if constexpr (i == 2) return S2;
    else if constexpr (i == 3) return S3;
    else if constexpr (i == 4) return S4;
    else if constexpr (i == 5) return S5;
    else if constexpr (i == 6) return S6;
    else return S7;
  };
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = w & 1, wn = w >> 1;
  int tm, tn, split;
  tile_coords(p, tm, tn, split);
  const int m0 = tm * BM, n0 = tn * BN;
  const int kbeg = split * p.k_per_split, kend = min(p.K, kbeg + p.k_per_split);
  const int nkt = (kend - kbeg) / TK;  // >= 1 (host)
  const uint32_t offa = LA::lane_off(p.lda, tid), offb = LB::lane_off(p.ldb, tid);
  const uint32_t offz = LA::lane_off(TK, tid);  // the same map over zero_tile
  const int64_t sa = (int64_t)NW * 8 * p.lda * 4, sb = (int64_t)NW * 8 * p.ldb * 4;
  constexpr int64_t sz = (int64_t)NW * 8 * TK * 4;
  const char* zero = reinterpret_cast<const char*>(zero_tile);
  // DMA instruction o (< PT) of K tile kt into stage X: selects, not
  // branches, between the operands and the zeros
  auto dma = [&](int kt, float* X, int o) {
    const bool real = kt < nkt;
    if (o < LA::NI) {
      const char* c = reinterpret_cast<const char*>(p.A + (int64_t)m0 * p.lda + kbeg + kt * TK);
      LA::dma_one(real ? c : zero, real ? offa : offz, real ? sa : sz, X, w, o);
    } else {
      const char* c = reinterpret_cast<const char*>(p.B + (int64_t)n0 * p.ldb + kbeg + kt * TK);
      LB::dma_one(real ? c : zero, real ? offb : offz, real ? sb : sz, X + BM * TK, w,
                  o - LA::NI);
    }
  };
  const int fa_0 = LA::frag_off(16 * wm, 0, lane), fa_1 = LA::frag_off(16 * wm, 1, lane);
  const int fb_0 = BM * TK + LB::frag_off(16 * NB * wn, 0, lane);
  const int fb_1 = BM * TK + LB::frag_off(16 * NB * wn, 1, lane);

  v4f acc[1][NB];
#pragma unroll
  for (int I = 0; I < NB; I++) acc[0][I] = (v4f){0.f, 0.f, 0.f, 0.f};
  v4f fa0[1], fb0[NB], fa1[1], fb1[NB];
  // the first S tiles
  unroll<0, S>([&](auto I) {
#pragma unroll
    for (int o = 0; o < PT; o++) dma(decltype(I)::value, stage(I), o);
  });
  wait_vm_lgkm0<PT * (S - 1)>();
  tile_barrier();
  {
    const float* X = stage(std::integral_constant<int, 0>{});
    fa0[0] = *reinterpret_cast<const v4f*>(&X[fa_0]);
#pragma unroll
    for (int u = 0; u < NB; u++) fb0[u] = *reinterpret_cast<const v4f*>(&X[fb_0 + 16 * u * TK]);
  }
  for (int kt0 = 0; kt0 < nkt; kt0 += S) {
    unroll<0, S>([&](auto I) {
      const int kt = kt0 + decltype(I)::value;
      float* C = stage(I);
      const float* X = stage(std::integral_constant<int, decltype(I)::value + 1>{});
      wide::group_mma<true, true, NW>(acc, fa0, fb0, [&](int n) {
        const int o = n - 1;
        if (o == 0) fa1[0] = *reinterpret_cast<const v4f*>(&C[fa_1]);
        else if (o >= 1 && o <= NB)
          fb1[o - 1] = *reinterpret_cast<const v4f*>(&C[fb_1 + 16 * (o - 1) * TK]);
      });
      // own fragment reads done; tile kt+1 landed (tiles kt+2 .. kt+S-1 may
      // still be in flight)
      wait_vm_lgkm0<PT * (S - 2)>();
      tile_barrier();
      // stage C is free: every wave holds tile kt's group-1 fragments
      wide::group_mma<true, true, NW>(acc, fa1, fb1, [&](int n) {
        const int o = n - 1;
        if (o >= 0 && o < PT) dma(kt + S, C, o);
        else if (o == PT) fa0[0] = *reinterpret_cast<const v4f*>(&X[fa_0]);
        else if (o > PT && o <= PT + NB)
          fb0[o - PT - 1] = *reinterpret_cast<const v4f*>(&X[fb_0 + 16 * (o - PT - 1) * TK]);
      });
    });
    // wait states between the last MFMAs and any accumulator copy the
    // compiler places at the loop's head
    asm volatile("s_nop 7\n\ts_nop 7");
  }
  // the loads issued past the last round (a workgroup must not end with LDS
  // writes in flight); then wait states before the accumulators are read
  wait_vm_lgkm0<0>();
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7");
  float* part = E == -1 ? p.part + (int64_t)split * p.M * p.N : nullptr;
  const int mw = m0 + 16 * wm, nw = n0 + 16 * NB * wn;
  wide::store_wave<E, true, true, NW>(p, part, acc, mw, nw, mw, nw, lane);
}

}  // namespace slim

typedef void (*SlimKernel)(GemmParams);
template <int BN, int S>
static SlimKernel slim_kernel_s(int e) {
  using namespace slim;
  switch (e) {
    case -1: return gemm_slim_kernel<BN, S, -1>;
    case EPI_STORE: return gemm_slim_kernel<BN, S, EPI_STORE>;
    case EPI_ADD_SRC: return gemm_slim_kernel<BN, S, EPI_ADD_SRC>;
    case EPI_RELU2_SAVE: return gemm_slim_kernel<BN, S, EPI_RELU2_SAVE>;
    case EPI_RELU2_SAVE + 16: return gemm_slim_kernel<BN, S, EPI_RELU2_SAVE + 16>;
  }
  return nullptr;
}
// Ring depth per tile width: the deepest that fits 160 KB of LDS (16, 20
// and 24 KB stages).
static int slim_depth(int bn) { return bn == 96 ? 8 : bn == 128 ? 7 : 6; }
static SlimKernel slim_kernel(int bn, int e) {
  switch (bn) {
    case 96: return slim_kernel_s<96, 8>(e);
    case 128: return slim_kernel_s<128, 7>(e);
    case 160: return slim_kernel_s<160, 6>(e);
  }
  return nullptr;
}

// Runs d on the slim-tile engine when it suits: x.W^T with M a multiple of
// 32 and at most 1024, N a multiple of one of the tile widths, K a multiple
// of 32, a grid of at most ~1.5 rounds of the CUs even unsplit.  The tile
// width and K split come from a cost model: rounds of workgroups times
// (MFMA cycles of one workgroup's K range + the latency of its first
// loads), plus a reduction launch when the split sums cannot be deferred.
static bool gemm_slim(const GemmDesc& d, GemmParams p, bool vec, hipStream_t st,
                      DeviceArena* ws) {
  if (d.group != GEMM_GROUP_NONE || d.force_splits > 0 || !vec) return false;
  if (!d.a_kcontig || !d.b_kcontig || d.M % slim::BM || d.M > 1024 || d.K % slim::TK) return false;
  if (d.ldc % 4 || !aligned16(d.C)) return false;
  if (d.epi == EPI_ADD_SRC && (!aligned16(d.aux) || d.ldaux % 4)) return false;
  if (d.epi == EPI_RELU2_SAVE && d.aux_out && (!aligned16(d.aux_out) || d.ldaux % 4)) return false;
  if (d.epi != EPI_STORE && d.epi != EPI_ADD_SRC && d.epi != EPI_RELU2_SAVE) return false;
  // GN_GEMM_SLIM: 0 turns the engine off, 1 takes every eligible product
  // (tests), unset: the products the cost model and the latency floor give it
  const char* env = std::getenv("GN_GEMM_SLIM");
  const int mode = env ? std::atoi(env) : -1;
  if (mode == 0) return false;
  const bool can_defer = d.defer && ((d.epi == EPI_STORE && d.alpha == 1.f) || d.epi == EPI_ADD_SRC);
  const int64_t cus = 256;
  const double lat = 4800.0;     // first-load latency, cycles (~2 us)
  const double reduce = 9600.0;  // a reduction launch
  double best = 0.0;
  int bn = 0, splits = 1;
  for (int w : {96, 128, 160}) {
    if (d.N % w) continue;
    const int64_t tiles = (int64_t)(d.M / slim::BM) * (d.N / w);
    if (tiles > (3 * cus) / 2) continue;
    const int smax = std::min<int>(can_defer ? PENDING_MAX_SPLITS : 16, d.K / 128);
    for (int s = 1; s <= std::max(1, smax); s++) {
      const int kps = (int)ceil_div(ceil_div(d.K, s), slim::TK) * slim::TK;
      if ((int)ceil_div(d.K, kps) != s) continue;
      const int64_t wg = tiles * s;
      const int ring = slim_depth(w);  // the K loop runs whole rounds of `ring` tiles
      const double kt = (double)ceil_div(kps / slim::TK, ring) * ring * slim::TK;
      const double t = (double)ceil_div(wg, cus) * (kt * w / 4.0 + lat) +
                       (s > 1 && !can_defer ? reduce : 0.0);
      if (bn == 0 || t < best - 1e-9) {
        best = t;
        bn = w;
        splits = s;
      }
    }
  }
  if (bn == 0) return false;
  const int kps = (int)ceil_div(ceil_div(d.K, splits), slim::TK) * slim::TK;
  // Short K ranges per workgroup are dominated by the first loads' latency,
  // which gemm_kernel's smaller tiles (two workgroups per CU) hide as well:
  // measured at M = 256, the slim engine wins from 16 K tiles per workgroup
  // (MLP products: 768-deep ranges, 15.5 -> 14.1 us and 15.1 -> 13.0 us)
  // but not at 6 (qkv 8.8 vs 8.9 us, attention output 5.8 vs 7.2 us).
  if (mode != 1 && kps < 16 * slim::TK) return false;
  int e = splits > 1 ? -1 : d.epi;
  if (e == EPI_RELU2_SAVE && !d.aux_out) e = EPI_RELU2_SAVE + 16;
  const SlimKernel kern = slim_kernel(bn, e);
  if (!kern) return false;
  p.tiles_m = d.M / slim::BM;
  p.tiles_n = d.N / bn;
  p.splits = splits;
  p.k_per_split = kps;
  const bool defer = can_defer && splits > 1;
  if (d.defer) {
    GN_CHECK(d.ldc == d.N && ((d.epi == EPI_STORE && d.alpha == 1.f) ||
                              (d.epi == EPI_ADD_SRC && d.aux == d.C && d.ldaux == d.N)),
             "gemm: a deferred split-K sum needs a plain or in-place residual product");
    *d.defer = PendingSum{};
  }
  if (splits > 1) {
    GN_CHECK(ws != nullptr, "gemm: split-K needs a workspace");
    p.part = ws->get<float>(defer ? "gemm_splitk_defer" + std::to_string(d.defer_slot)
                                  : std::string("gemm_splitk"),
                            (size_t)splits * d.M * d.N);
  }
  hipLaunchKernelGGL(kern, dim3((unsigned)(p.tiles_m * p.tiles_n * splits)), dim3(64 * slim::NW),
                     0, st, p);
  GN_HIP(hipGetLastError());
  if (defer) {
    d.defer->part = p.part;
    d.defer->splits = splits;
    d.defer->stride = (int64_t)d.M * d.N;
  } else if (splits > 1) {
    const int64_t total = (int64_t)d.M * d.N;
    hipLaunchKernelGGL(gemm_reduce_kernel, dim3((unsigned)ceil_div(total, 256)), dim3(256), 0, st,
                       p);
    GN_HIP(hipGetLastError());
  }
  return true;
}

GemmEngine gemm(const GemmDesc& d, hipStream_t st, DeviceArena* ws) {
  GN_CHECK(d.M >= 0 && d.N >= 0 && d.K >= 0, "gemm: negative extent");
  if (d.M == 0 || d.N == 0) return GEMM_ENGINE_TILE;
  GemmParams p{};
  p.A = d.A; p.B = d.B; p.C = d.C; p.aux = d.aux; p.aux_out = d.aux_out;
  p.lda = d.lda; p.ldb = d.ldb; p.ldc = d.ldc; p.ldaux = d.ldaux;
  p.M = d.M; p.N = d.N; p.K = d.K;
  p.epi = d.epi;
  p.alpha = d.alpha;
  const bool vec = aligned16(d.A) && aligned16(d.B) && d.lda % 4 == 0 && d.ldb % 4 == 0 &&
                   d.group_stride % 4 == 0;
  if (d.group != GEMM_GROUP_NONE) {
    GN_CHECK(d.group_off != nullptr && d.groups > 0, "grouped gemm: missing group offsets");
    p.goff = d.group_off;
    p.groups = d.groups;
    p.gstride = d.group_stride;
    p.a_pad = d.a_pad_rows >= 128;
    p.splits = 1;
    p.k_per_split = d.K;
    if (d.group == GEMM_GROUP_ROWS) {
      // per-group tiles: large tiles once the average group fills them
      if (d.M / d.groups >= 1024) {
        launch_grouped<128, 128, 2, 2, 1, 2, false, GEMM_GROUP_ROWS>(p, d.a_kcontig, d.b_kcontig,
                                                                     vec, st);
        return GEMM_ENGINE_TILE;
      }
      // Small groups (decode: a few to tens of rows per expert) stream each
      // expert's weights once; split K so that enough workgroups keep loads
      // in flight, summed by gemm_reduce_kernel.  Tile rows follow the
      // average group: 16 or 32 rows with 2-wave workgroups (about 4 per
      // CU) when groups are that small, else 64 rows with 8 waves (about 2
      // per CU) -- taller tiles would multiply mostly padding rows.
      const int64_t avg = ceil_div(d.M, d.groups);
      const int bm = avg <= 16 ? 16 : avg <= 32 ? 32 : 64;
      const int64_t want = bm < 64 ? 4 * 256 : 2 * 256;
      const int64_t tiles = (ceil_div(d.M, bm) + d.groups) * ceil_div(d.N, 64);
      int splits = 1;
      if (tiles < want && d.K >= 256)
        splits = (int)std::max<int64_t>(1, std::min<int64_t>(ceil_div(want, tiles), d.K / 128));
      const int kps = (int)ceil_div(ceil_div(d.K, splits), GK) * GK;
      splits = (int)ceil_div(d.K, kps);
      p.k_per_split = kps;
      p.splits = splits;
      if (splits > 1) {
        GN_CHECK(ws != nullptr, "gemm: split-K needs a workspace");
        p.part = ws->get<float>("gemm_splitk", (size_t)splits * d.M * d.N);
      }
      if (bm == 16)
        launch_grouped<16, 64, 1, 2, 1, 4, false, GEMM_GROUP_ROWS>(p, d.a_kcontig, d.b_kcontig, vec,
                                                                   st);
      else if (bm == 32)
        launch_grouped<32, 64, 1, 2, 1, 4, false, GEMM_GROUP_ROWS>(p, d.a_kcontig, d.b_kcontig, vec,
                                                                   st);
      else
        launch_grouped<64, 64, 2, 2, 2, 4, false, GEMM_GROUP_ROWS>(p, d.a_kcontig, d.b_kcontig, vec,
                                                                   st);
      if (splits > 1) {
        const int64_t total = (int64_t)d.M * d.N;
        hipLaunchKernelGGL(gemm_reduce_kernel, dim3((unsigned)ceil_div(total, 256)), dim3(256), 0,
                           st, p);
        GN_HIP(hipGetLastError());
      }
    } else {
      if (gemm_wide_grouped_k(d, p, vec, st, ws)) return GEMM_ENGINE_WIDE;
      // K mode: a group's whole row range per workgroup, two-level summation
      launch_grouped<128, 128, 2, 2, 1, 2, true, GEMM_GROUP_K>(p, d.a_kcontig, d.b_kcontig, vec,
                                                               st);
    }
    return GEMM_ENGINE_TILE;
  }
  if (d.batch > 1) {
    // batched products of one shape (the compressed attention's per-sequence
    // products): one launch, the batch on grid y; 128 x 128 tiles unless a
    // side is at most 64 (then 64 x 64: no half-empty tiles); K split only
    // while the batch leaves the CUs short of two workgroups each
    GN_CHECK(d.group == GEMM_GROUP_NONE && !d.defer && (d.epi == EPI_STORE || d.epi == EPI_ACCUM),
             "gemm: batched products store or accumulate");
    p.bsa = d.batch_sa;
    p.bsb = d.batch_sb;
    p.bsc = d.batch_sc;
    const int64_t cus = 256;
    const bool big = d.M > 64 && d.N > 64;
    const int bm = big ? 128 : 64, bn = big ? 128 : 64;
    const int64_t tiles = ceil_div(d.M, bm) * ceil_div(d.N, bn) * d.batch;
    int splits = 1;
    if (tiles < 2 * cus && d.K >= 2048)
      splits = (int)std::max<int64_t>(1, std::min<int64_t>(ceil_div(2 * cus, tiles), d.K / 1024));
    splits = std::min(splits, 64);
    if (const char* e = std::getenv("GN_GEMM_BATCH_SPLITS"))  // tests: force the split path
      splits = std::max(1, std::min(std::atoi(e), 64));
    const int kps = d.K > 0 ? (int)ceil_div(ceil_div(d.K, splits), GK) * GK : 0;
    splits = d.K > 0 ? (int)ceil_div(d.K, kps) : 1;
    p.k_per_split = kps;
    p.splits = splits;
    if (splits > 1) {
      GN_CHECK(ws != nullptr, "gemm: split-K needs a workspace");
      p.part = ws->get<float>("gemm_splitk", (size_t)splits * d.M * d.N * d.batch);
    }
    const bool fold = kps >= 4096;
    if (big && fold)
      launch_cfg<128, 128, 2, 2, 1, 2, true>(p, d.a_kcontig, d.b_kcontig, vec, splits, st, d.batch);
    else if (big)
      launch_cfg<128, 128, 2, 2, 1, 2, false>(p, d.a_kcontig, d.b_kcontig, vec, splits, st, d.batch);
    else if (fold)
      launch_cfg<64, 64, 2, 2, 2, 4, true>(p, d.a_kcontig, d.b_kcontig, vec, splits, st, d.batch);
    else
      launch_cfg<64, 64, 2, 2, 2, 4, false>(p, d.a_kcontig, d.b_kcontig, vec, splits, st, d.batch);
    if (splits > 1) {
      const int64_t total = (int64_t)d.M * d.N;
      hipLaunchKernelGGL(gemm_reduce_kernel, dim3((unsigned)ceil_div(total, 256), (unsigned)d.batch),
                         dim3(256), 0, st, p);
      GN_HIP(hipGetLastError());
    }
    return GEMM_ENGINE_TILE;
  }
  if (gemm_wide(d, p, vec, st, ws)) return GEMM_ENGINE_WIDE;
  if (gemm_slim(d, p, vec, st, ws)) return GEMM_ENGINE_SLIM;

  // Tile choice: the 128x128 tile when it yields enough workgroups to cover
  // the 256 CUs, otherwise 64x64; split K when even that underfills the chip
  // and K is long enough to share.
  // Long-K products (weight gradients, K = tokens) keep the 128x128 tile and
  // split K instead, since each split still has thousands of K steps.
  const int64_t cus = 256;
  const int64_t big = ceil_div(d.M, 128) * ceil_div(d.N, 128);
  const bool long_k = d.K >= 4096;
  // at most 64 rows (the flash decode's 64 rows: its lm_head, N = 65,536):
  // 64 x 64 tiles, not half-empty 128-row ones
  const bool use_big = (big >= cus && d.M > 64) || long_k;
  const int bm = use_big ? 128 : 64, bn = use_big ? 128 : 64;
  const int64_t tiles = ceil_div(d.M, bm) * ceil_div(d.N, bn);
  int splits = 1;
  if (d.force_splits > 0) {
    splits = d.force_splits;
  } else if (long_k && tiles < 8 * cus) {
    // Aim for >= 9 workgroups per CU and prefer a total that is a multiple
    // of the CU count, so the last round of workgroups is not a partial one.
    const int smax = (int)std::max<int64_t>(1, std::min<int64_t>(64, d.K / 1024));
    const int smin = (int)std::min<int64_t>(smax, ceil_div(9 * cus, tiles));
    double best = -1.0;
    for (int s = smin; s <= smax; s++) {
      const int64_t wg = tiles * s;
      const double eff = (double)wg / (double)(ceil_div(wg, cus) * cus);
      if (eff > best + 1e-9) {
        best = eff;
        splits = s;
      }
      if (eff >= 0.999) break;
    }
  } else if (tiles < cus && d.K >= 512) {
    // Small grids (the M = 256 decode projections): about 200 workgroups
    // (25/32 of a workgroup per CU) measured fastest; more splits cost more
    // in the reduction than they gain in parallelism.
    // Few-row products (M <= 128: the flash decode's 64 rows, 8 to 24 tiles)
    // take K splits down to 64 deep, so their serial K loop shortens too
    // (flash d12 rollout 1080 -> 1013 ms at 128 deep, 1004 ms at 64; at
    // M = 256, 128-deep splits left the latent and d12 rollouts unchanged).
    const int kmin = d.M <= 128 ? 64 : 256;
    splits = (int)std::min<int64_t>((25 * cus / 32 + tiles / 2) / tiles, d.K / kmin);
    splits = std::max(1, std::min(splits, d.defer ? PENDING_MAX_SPLITS : 64));
  }
  // Narrow tiles for small grids whose N is a multiple of 96 (the d12 decode
  // projections, N = 768 or 3072 at M = 256): 32x96 tiles with a split
  // count that makes the workgroups fill whole rounds of the CUs (the MLP
  // input projection: exactly 256 tiles; the output projections: 64 tiles
  // x 4 splits), where 64x64 tiles leave a quarter of the CUs idle.  Their
  // K tiles are 64 deep (half the barriers of 32-deep ones; 128-deep and
  // deeper rings measured no faster).
  int narrow = 0;  // narrow tile width (0: none)
  if (!use_big && !long_k && d.force_splits == 0 && d.N % 96 == 0 && d.a_kcontig && d.b_kcontig) {
    const int64_t nt = ceil_div(d.M, 32) * (d.N / 96);
    double best = 0.0;
    int bs = 1;
    for (int s = 1; s <= PENDING_MAX_SPLITS && (s == 1 || d.K / s >= 128); s++) {
      const int64_t wg = nt * s;
      const double eff = (double)wg / (double)(ceil_div(wg, cus) * cus);
      if (eff > best + 1e-9) {
        best = eff;
        bs = s;
      }
    }
    if (best >= 0.9) {
      narrow = 96;
      splits = bs;
    }
  }
  // 32 x 80 and 32 x 112 tiles (N a multiple of 80 or 112, not of 96) when
  // the 64 x 64 tiling leaves CUs idle (the d20 decode projections at M =
  // 512: N = 1280 gives 160 tiles, N = 1792 224).  A product whose split
  // sums can be deferred takes the split count nearest two workgroups per
  // CU (wo 31.9 -> 22.5 us, qkv 34.2 -> 29.6 us cold); others stay unsplit
  // (fc with its ReLU^2 epilogue: 79.5 -> 73.2 us).
  const bool can_defer = d.defer && ((d.epi == EPI_STORE && d.alpha == 1.f) || d.epi == EPI_ADD_SRC);
  if (!narrow && !use_big && !long_k && d.force_splits == 0 && d.a_kcontig && d.b_kcontig &&
      tiles * splits < (9 * cus) / 10) {
    for (int bn : {80, 112}) {
      if (d.N % bn) continue;
      const int64_t nt = ceil_div(d.M, 32) * (d.N / bn);
      if (nt < cus / 2) continue;
      int bs = 1;
      if (can_defer)
        for (int s = 2; s <= PENDING_MAX_SPLITS && d.K / s >= 512; s++)
          if (std::llabs(nt * s - 2 * cus) < std::llabs(nt * bs - 2 * cus)) bs = s;
      narrow = bn;
      splits = bs;
      break;
    }
  }
  // k_per_split is a whole number of LDS tiles so that every split but the
  // last starts and ends on a tile boundary.
  int kps = (int)ceil_div(ceil_div(d.K, splits), GK) * GK;
  splits = d.K > 0 ? (int)ceil_div(d.K, kps) : 1;

  p.k_per_split = d.K > 0 ? kps : 0;
  p.splits = splits;
  const bool defer = d.defer && splits > 1 && splits <= PENDING_MAX_SPLITS;
  if (d.defer) {
    GN_CHECK(d.ldc == d.N && ((d.epi == EPI_STORE && d.alpha == 1.f) ||
                              (d.epi == EPI_ADD_SRC && d.aux == d.C && d.ldaux == d.N)),
             "gemm: a deferred split-K sum needs a plain or in-place residual product");
    *d.defer = PendingSum{};
  }
  if (splits > 1) {
    GN_CHECK(ws != nullptr, "gemm: split-K needs a workspace");
    // deferred partials live until their consumer runs, past later GEMMs'
    p.part = ws->get<float>(defer ? "gemm_splitk_defer" + std::to_string(d.defer_slot)
                                  : std::string("gemm_splitk"),
                            (size_t)splits * d.M * d.N);
  }
  // two-level summation for long K ranges per workgroup (see gemm_kernel)
  const bool fold = kps >= 4096;
  if (use_big && fold)
    launch_cfg<128, 128, 2, 2, 1, 2, true>(p, d.a_kcontig, d.b_kcontig, vec, splits, st);
  else if (use_big)
    launch_cfg<128, 128, 2, 2, 1, 2, false>(p, d.a_kcontig, d.b_kcontig, vec, splits, st);
  else if (fold)
    launch_cfg<64, 64, 2, 2, 2, 4, true>(p, d.a_kcontig, d.b_kcontig, vec, splits, st);
  else if (narrow == 96 && kps <= 3 * 64)  // every K tile of the split in flight at once
    launch_cfg_kk<32, 96, 1, 2, 2, 4, 64>(p, vec, splits, st);  // (d12 wo: 7.51 -> 7.29 us)
  else if (narrow == 96)  // 64-deep K tiles, two stages (fc 21.3 -> 19.4 us, proj 18.7 -> 17.7 us)
    launch_cfg_kk<32, 96, 1, 2, 2, 2, 64>(p, vec, splits, st);
  else if (narrow == 80)
    launch_cfg_kk<32, 80, 2, 1, 2, 2, 64>(p, vec, splits, st);
  else if (narrow == 112)
    launch_cfg_kk<32, 112, 2, 1, 2, 2, 64>(p, vec, splits, st);
  else
    launch_cfg<64, 64, 2, 2, 2, 4, false>(p, d.a_kcontig, d.b_kcontig, vec, splits, st);
  if (defer) {
    d.defer->part = p.part;
    d.defer->splits = splits;
    d.defer->stride = (int64_t)d.M * d.N;
  } else if (splits > 1) {
    const int64_t total = (int64_t)d.M * d.N;
    hipLaunchKernelGGL(gemm_reduce_kernel, dim3((unsigned)ceil_div(total, 256)), dim3(256), 0, st,
                       p);
    GN_HIP(hipGetLastError());
  }
  return GEMM_ENGINE_TILE;
}

}  // namespace gn
