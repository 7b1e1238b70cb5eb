// gn_sampler.hip - inference.SampleNextToken (inference/sampler.go:16-60) on
// device, bit-exact with the reference given the same logits and stream.
//
// The reference draws one tensors.RNG Float32 for EVERY vocabulary entry of
// every row, masked or not (tensors/random.go:66-78), so draw v of row i of a
// call is the (i*V + v + 1)-th step of the group's stream.  Go's PCG is a
// 128-bit LCG, so any step is reachable in O(log n) by squaring the affine
// map; the DXSM output, the Float32 mapping and the float64 Gumbel transform
// are evaluated only for entries that survive the top-k mask.
//
// Top-k threshold (the k-th largest value of the row, ties kept):
//  1. one coalesced pass over the row computes the maxima of ngroups strided
//     groups (float4 c, or entry c when the row is not float4-aligned, in
//     group c mod ngroups);
//  2. the k-th largest group maximum L is a lower bound of the k-th largest
//     value (each of the k groups holds a value >= L);
//  3. the values >= L (a few hundred at most for real logits) are compacted
//     into LDS and bitonic-sorted; the k-th of them is the threshold.
// When the row fits in the block's registers (V <= 16 float4 per thread,
// V = 65,536 at 1024 threads) it is read from memory once: the group maxima,
// the candidates and their values all come from registers and LDS.
// If the candidates overflow the LDS buffer (e.g. massively tied logits) the
// row falls back to an exact 4-pass 8-bit radix select over the whole row.
//
// Softcapped rows (the decode path hands over lm_head products y; the logits
// are softcap15(y)): softcap15 is non-decreasing over every float (checked
// exhaustively on the device by count_softcap_order_violations), so the
// k-th largest logit is softcap15 of the k-th largest product, and steps 1-2
// run on the raw products; only the candidates are softcapped.  Entries
// below the bound L are dropped, which is exact when softcap15 of the float
// below L is under the threshold (no dropped entry can tie it); otherwise
// (a flat, saturated softcap across L) the row takes the radix select.
// This keeps the tanh off all but a few hundred entries of a row.
#include "gn_model.h"

namespace gn {

typedef float v4f __attribute__((ext_vector_type(4)));

struct u128 {
  uint64_t hi, lo;
};
__device__ __forceinline__ u128 mul128(u128 a, u128 b) {
  u128 r;
  r.lo = a.lo * b.lo;
  r.hi = __umul64hi(a.lo, b.lo) + a.hi * b.lo + a.lo * b.hi;
  return r;
}
__device__ __forceinline__ u128 add128(u128 a, u128 b) {
  u128 r;
  r.lo = a.lo + b.lo;
  r.hi = a.hi + b.hi + (r.lo < a.lo ? 1ull : 0ull);
  return r;
}
// Go math/rand/v2 PCG constants (multiplier and increment of the LCG).
__device__ __forceinline__ u128 pcg_mul() { return {0x2360ED051FC65DA4ull, 0x4385DF649FCCF645ull}; }
__device__ __forceinline__ u128 pcg_inc() { return {6364136223846793005ull, 1442695040888963407ull}; }
__device__ __forceinline__ u128 pcg_step(u128 s) { return add128(mul128(s, pcg_mul()), pcg_inc()); }

// Jumps of 2^j LCG steps (j = 0..63) as affine maps s -> a s + c, built at
// compile time: f^(2^(j+1)) = f^(2^j) o f^(2^j), i.e. a' = a^2, c' = a c + c.
struct PcgJump {
  uint64_t ahi, alo, chi, clo;
};
struct PcgJumps {
  PcgJump j[64];
};
constexpr PcgJumps make_pcg_jumps() {
  PcgJumps t{};
  unsigned __int128 a = ((unsigned __int128)0x2360ED051FC65DA4ull << 64) | 0x4385DF649FCCF645ull;
  unsigned __int128 c = ((unsigned __int128)6364136223846793005ull << 64) | 1442695040888963407ull;
  for (int i = 0; i < 64; i++) {
    t.j[i] = {(uint64_t)(a >> 64), (uint64_t)a, (uint64_t)(c >> 64), (uint64_t)c};
    c = a * c + c;
    a = a * a;
  }
  return t;
}
__constant__ PcgJumps kPcgJumps = make_pcg_jumps();

// State after n further LCG steps: the jumps of n's set bits (powers of one
// map commute), one 128-bit multiply-add per set bit.
__device__ u128 pcg_advance(u128 s, uint64_t n) {
  for (int j = 0; n; j++, n >>= 1)
    if (n & 1) {
      const PcgJump& J = kPcgJumps.j[j];
      s = add128(mul128(u128{J.ahi, J.alo}, s), u128{J.chi, J.clo});
    }
  return s;
}

// DXSM permutation of the (post-step) state -> Uint64 -> Float32.
__device__ __forceinline__ float pcg_float32(u128 s) {
  uint64_t hi = s.hi;
  hi ^= hi >> 32;
  hi *= 0xda942042e4dd58b5ull;
  hi ^= hi >> 48;
  hi *= (s.lo | 1ull);
  uint32_t u = (uint32_t)(hi >> 32);
  return (float)((u << 8) >> 8) / 16777216.0f;
}

// Gumbel score of entry v whose draw state is s (tensors/random.go:68-73).
__device__ __forceinline__ float gumbel_score(float zv, float T, u128 s) {
  float u = pcg_float32(s);
  if (u <= 0.f) u = 1e-12f;
  float gum = -(float)log(-log((double)u));
  return __fadd_rn(__fdiv_rn(zv, T), gum);
}

__device__ __forceinline__ uint32_t order_key(float f) {
  uint32_t b = __float_as_uint(f);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float key_float(uint32_t u) {
  uint32_t b = (u & 0x80000000u) ? (u & 0x7fffffffu) : ~u;
  return __uint_as_float(b);
}

// Merges per-thread (score, index) winners: larger score, ties to the
// smaller index; index -1 means "none".
__device__ __forceinline__ void better(float& bv, int& bi, float ov, int oi) {
  if (oi >= 0 && (bi < 0 || ov > bv || (ov == bv && oi < bi))) {
    bv = ov;
    bi = oi;
  }
}

// Descending bitonic sort of n (power of two) floats in LDS by all threads.
__device__ void bitonic_desc(float* a, int n) {
  for (int k = 2; k <= n; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = threadIdx.x; i < n; i += blockDim.x) {
        int ixj = i ^ j;
        if (ixj > i) {
          bool desc = (i & k) == 0;
          float x = a[i], y = a[ixj];
          if (desc ? (x < y) : (x > y)) {
            a[i] = y;
            a[ixj] = x;
          }
        }
      }
      __syncthreads();
    }
  }
}

static constexpr int NT = 1024;  // 16 waves per row: loads of a pass in flight together
static constexpr int MAXG = 4096;  // group maxima
static constexpr int MAXC = 2048;  // candidates
static constexpr int REGV = 16;    // float4 per thread of a row held in registers

__global__ __launch_bounds__(NT) void sampler_kernel(SamplerArgs a) {
  __shared__ float buf[MAXG];
  __shared__ int cand_i[MAXC];
  __shared__ float cand_v[MAXC];
  __shared__ uint32_t hist[4][256];
  __shared__ uint32_t sel_prefix, sel_k;
  __shared__ int ncand;
  __shared__ float thr_s;
  __shared__ float best_v[NT / 64];
  __shared__ int best_i[NT / 64];
  __shared__ uint64_t base_s[2];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int row = blockIdx.x;
  const float* z = a.logits + (int64_t)row * a.ldl;
  const int V = a.V;
  const bool sc = a.softcap != 0;
  auto zl = [&](int v) { return sc ? softcap15(z[v]) : z[v]; };  // logit v
  auto zl4 = [&](v4f t) {
    if (sc)
#pragma unroll
      for (int c = 0; c < 4; c++) t[c] = softcap15(t[c]);
    return t;
  };
  float bv = -INFINITY;
  int bi = -1;

  if (a.temperature <= 0.f) {
    // argMax: first index of the largest value (sampler.go:37-45)
    for (int v = tid; v < V; v += NT) better(bv, bi, zl(v), v);
  } else {
    const int g = row / a.samples_per_group, ig = row % a.samples_per_group;
    const int k = a.top_k;
    const bool masking = k > 0 && k < V;
    const float T = a.temperature;
    const bool vec = V % 4 == 0 && a.ldl % 4 == 0 && ((uintptr_t)a.logits & 15) == 0;
    const v4f* z4 = reinterpret_cast<const v4f*>(z);
    const int V4 = V / 4;
    // the row in registers: float4 c = tid + u * NT of thread tid, requested
    // before the stream jump below so the two overlap
    const bool inreg = masking && vec && V4 <= REGV * NT;
    int ngroups = NT;  // a power of two >= 4k (at most MAXG)
    while (ngroups < MAXG && ngroups < 4 * k) ngroups <<= 1;
    const bool fast = inreg && ngroups == NT;  // k <= 256: one group per thread
    // raw: the registers hold the products y and the selection runs on them
    const bool raw = fast && sc;
    v4f zr[REGV];
    if (inreg) {
#pragma unroll
      for (int u = 0; u < REGV; u++) {
        const int c = tid + u * NT;
        zr[u] = c < V4 ? (raw ? z4[c] : zl4(z4[c]))
                       : (v4f){-INFINITY, -INFINITY, -INFINITY, -INFINITY};
      }
    }
    if (tid == 0) {
      u128 s = {a.base_states[2 * g], a.base_states[2 * g + 1]};
      s = pcg_advance(s, (uint64_t)ig * (uint64_t)V);
      base_s[0] = s.hi;
      base_s[1] = s.lo;
      ncand = 0;
      thr_s = -INFINITY;
    }
    __syncthreads();
    const u128 rowbase = {base_s[0], base_s[1]};
    if (!masking) {
      // every entry is a candidate: walk the stream sequentially per chunk
      const int chunk = (V + NT - 1) / NT;
      const int v0 = tid * chunk, v1 = min(V, v0 + chunk);
      u128 s = pcg_advance(rowbase, (uint64_t)v0);
      for (int v = v0; v < v1; v++) {
        s = pcg_step(s);
        better(bv, bi, gumbel_score(zl(v), T, s), v);
      }
    } else {
      // 1) a lower bound of the k-th largest value.  The maxima of any
      //    partition of the row bound it: the k-th largest of them is one
      //    (each of the k groups holds a value >= it).  The groups are
      //    strided (entry v belongs to group v mod ngroups) so the pass
      //    reads the row with coalesced loads.
      float lower;
      if (fast) {
        // One group per thread (its 64 registers).  Each of the 16 waves
        // ranks its 64 maxima (value, then lane) and offers its m-th
        // largest, m = ceil(k / 16); the smallest offer L bounds the k-th
        // largest value: the 16 m >= k maxima ranked at or above m in their
        // waves are all >= L.  No barrier-synchronized sort.
        float mx = -INFINITY;
#pragma unroll
        for (int u = 0; u < REGV; u++)
          mx = fmaxf(mx, fmaxf(fmaxf(zr[u][0], zr[u][1]), fmaxf(zr[u][2], zr[u][3])));
        if (mx != mx) mx = -INFINITY;  // an all-NaN group offers nothing
        const int mrank = (k + NT / 64 - 1) / (NT / 64);
        int rank = 0;
        for (int o = 0; o < 64; o++) {
          const float ov = __shfl(mx, o, 64);
          rank += (ov > mx || (ov == mx && o < lane)) ? 1 : 0;
        }
        if (rank == mrank - 1) buf[wid] = mx;  // one lane per wave: ranks are a permutation
        __syncthreads();
        lower = buf[0];
#pragma unroll
        for (int w = 1; w < NT / 64; w++) lower = fminf(lower, buf[w]);
      } else {
        if (inreg) {
          // float4 c is in group c mod ngroups = tid + (u mod gpt) * NT
          const int gpt = ngroups / NT;
          for (int j = 0; j < gpt; j++) {
            float m = -INFINITY;
#pragma unroll
            for (int u = 0; u < REGV; u++)
              if ((u & (gpt - 1)) == j)
                m = fmaxf(m, fmaxf(fmaxf(zr[u][0], zr[u][1]), fmaxf(zr[u][2], zr[u][3])));
            buf[tid + j * NT] = m;
          }
        } else if (vec) {
          // float4 c belongs to group c mod ngroups
          for (int gi = tid; gi < ngroups; gi += NT) {
            float m = -INFINITY;
#pragma unroll 16
            for (int c = gi; c < V4; c += ngroups) {
              const v4f t = zl4(z4[c]);
              m = fmaxf(m, fmaxf(fmaxf(t[0], t[1]), fmaxf(t[2], t[3])));
            }
            buf[gi] = m;
          }
        } else {
          for (int gi = tid; gi < ngroups; gi += NT) {
            float m = -INFINITY;
            for (int v = gi; v < V; v += ngroups) m = fmaxf(m, zl(v));
            buf[gi] = m;
          }
        }
        __syncthreads();
        bitonic_desc(buf, ngroups);
        lower = k <= ngroups ? buf[k - 1] : -INFINITY;
      }
      __syncthreads();
      // 2) compact candidates >= lower (the row is read 8 float4 per thread
      //    at a time so the loads overlap)
      auto keep = [&](int v, float zv) {
        if (v < V && zv >= lower) {  // (padding past the row is -inf, and lower may be too)
          const int slot = atomicAdd(&ncand, 1);
          if (slot < MAXC) {
            cand_i[slot] = v;
            cand_v[slot] = raw ? softcap15(zv) : zv;
          }
        }
      };
      if (inreg) {
#pragma unroll
        for (int u = 0; u < REGV; u++)
#pragma unroll
          for (int j = 0; j < 4; j++) keep(4 * (tid + u * NT) + j, zr[u][j]);
      } else if (vec) {
        for (int c0 = tid; c0 < V4; c0 += 8 * NT) {
          v4f t[8];
#pragma unroll
          for (int u = 0; u < 8; u++) {
            const int c = c0 + u * NT;
            t[u] = c < V4 ? zl4(z4[c]) : (v4f){-INFINITY, -INFINITY, -INFINITY, -INFINITY};
          }
#pragma unroll
          for (int u = 0; u < 8; u++)
#pragma unroll
            for (int j = 0; j < 4; j++) keep(4 * (c0 + u * NT) + j, t[u][j]);
        }
      } else {
        for (int v = tid; v < V; v += NT) keep(v, zl(v));
      }
      __syncthreads();
      const int nc = ncand;
      float thr = 0.f;
      bool small = nc <= MAXC;
      if (small) {
        if (fast) {
          // the k-th largest candidate value: the one with fewer than k
          // candidates above it and at least k at or above it (all such
          // candidates hold that same value)
          for (int i = tid; i < nc; i += NT) {
            const float x = cand_v[i];
            int gt = 0, ge = 0;
            for (int j = 0; j < nc; j++) {
              const float y = cand_v[j];
              gt += y > x ? 1 : 0;
              ge += y >= x ? 1 : 0;
            }
            if (gt < k && k <= ge) thr_s = x;
          }
          __syncthreads();
          thr = thr_s;
        } else {
          int cp2 = 1;
          while (cp2 < nc) cp2 <<= 1;
          for (int i = tid; i < cp2; i += NT) buf[i] = i < nc ? cand_v[i] : -INFINITY;
          __syncthreads();
          bitonic_desc(buf, cp2);
          thr = buf[k - 1];
          __syncthreads();
        }
        // Raw selection: every entry below the bound must stay below the
        // threshold (thr and lower are the same in every thread).
        if (raw && !(softcap15(nextafterf(lower, -INFINITY)) < thr)) small = false;
      }
      if (small) {
        // 3) Gumbel-max over the survivors, in index order per thread
        for (int i = tid; i < nc; i += NT) {
          const int v = cand_i[i];
          const float zv = cand_v[i];
          if (zv >= thr) {
            float sc = gumbel_score(zv, T, pcg_advance(rowbase, (uint64_t)v + 1));
            better(bv, bi, sc, v);
          }
        }
      } else {
        // exact fallback: radix select of the k-th largest over the row
        uint32_t prefix = 0, pmask = 0, kk = (uint32_t)k;
        for (int pass = 0; pass < 4; pass++) {
          const int shift = 24 - 8 * pass;
          for (int i = tid; i < 4 * 256; i += NT) (&hist[0][0])[i] = 0;
          __syncthreads();
          for (int v = tid; v < V; v += NT) {
            uint32_t u = order_key(zl(v));
            if ((u & pmask) == prefix) atomicAdd(&hist[wid & 3][(u >> shift) & 255u], 1u);
          }
          __syncthreads();
          if (tid == 0) {
            uint32_t cum = 0;
            int bin = 0;
            for (int bb = 255; bb >= 0; bb--) {
              uint32_t c = hist[0][bb] + hist[1][bb] + hist[2][bb] + hist[3][bb];
              if (cum + c >= kk) { bin = bb; break; }
              cum += c;
            }
            sel_prefix = prefix | ((uint32_t)bin << shift);
            sel_k = kk - cum;
          }
          __syncthreads();
          prefix = sel_prefix;
          kk = sel_k;
          pmask |= 255u << shift;
          __syncthreads();
        }
        thr = key_float(prefix);
        for (int v = tid; v < V; v += NT) {
          const float zv = zl(v);
          if (zv >= thr) {
            float sc = gumbel_score(zv, T, pcg_advance(rowbase, (uint64_t)v + 1));
            better(bv, bi, sc, v);
          }
        }
      }
    }
  }
  for (int o = 32; o > 0; o >>= 1) {
    float ov = __shfl_xor(bv, o, 64);
    int oi = __shfl_xor(bi, o, 64);
    better(bv, bi, ov, oi);
  }
  if (lane == 0) {
    best_v[wid] = bv;
    best_i[wid] = bi;
  }
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < NT / 64; w++) better(bv, bi, best_v[w], best_i[w]);
    a.out[row] = bi < 0 ? 0 : bi;
  }
}

// Order check of softcap15 over every float, which the raw selection above
// relies on: the floats are walked in increasing order (key k holds
// key_float(k)), each thread a contiguous run of keys overlapping the next
// run by one, and every neighbour pair whose softcap decreases (or is NaN
// for a non-NaN input) is counted.  NaN bit patterns are skipped.
__global__ __launch_bounds__(256) void softcap_order_kernel(unsigned long long* bad) {
  const uint64_t nthreads = (uint64_t)gridDim.x * blockDim.x;
  const uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const uint64_t total = 1ull << 32;
  const uint64_t per = (total + nthreads - 1) / nthreads;
  const uint64_t k0 = t * per, k1 = k0 + per + 1 < total ? k0 + per + 1 : total;
  unsigned long long n = 0;
  float prev = 0.f;
  bool have = false;
  for (uint64_t k = k0; k < k1; k++) {
    const float x = key_float((uint32_t)k);
    if (x != x) {
      have = false;
      continue;
    }
    const float y = softcap15(x);
    if (y != y || (have && y < prev)) n++;
    prev = y;
    have = true;
  }
  if (n) atomicAdd(bad, n);
}

uint64_t count_softcap_order_violations() {
  unsigned long long* bad = nullptr;
  GN_HIP(hipMalloc(&bad, sizeof(unsigned long long)));
  unsigned long long h = 0;
  hipError_t e = hipMemset(bad, 0, sizeof(h));
  if (e == hipSuccess) {
    hipLaunchKernelGGL(softcap_order_kernel, dim3(1024), dim3(256), 0, 0, bad);
    e = hipGetLastError();
  }
  if (e == hipSuccess) e = hipMemcpy(&h, bad, sizeof(h), hipMemcpyDeviceToHost);
  (void)hipFree(bad);
  GN_HIP(e);
  return h;
}

void launch_sampler(const SamplerArgs& a, hipStream_t st) {
  if (a.rows <= 0) return;
  GN_CHECK(a.V > 0, "sampler: empty vocabulary");
  hipLaunchKernelGGL(sampler_kernel, dim3(a.rows), dim3(NT), 0, st, a);
  GN_HIP(hipGetLastError());
}

}  // namespace gn
