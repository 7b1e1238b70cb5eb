// gn_sampler.hip - inference.SampleNextToken (inference/sampler.go:16-60) on
// device, bit-exact with the reference given the same logits and stream.
//
// The reference draws one tensors.RNG Float32 for EVERY vocabulary entry of
// every row, masked or not (tensors/random.go:66-78), so draw v of row i of a
// call starts at stream offset i*V + v.  Each thread owns a contiguous chunk
// of the row, jumps Go's 128-bit PCG LCG to its chunk start in O(log n)
// (affine-map squaring), and steps sequentially; the DXSM output, the
// Float32 mapping and the float64 Gumbel transform are evaluated only for
// entries that survive the top-k mask (value >= k-th largest, ties kept).
// The k-th largest comes from a 4-pass 8-bit radix select over the
// order-preserving integer image of the floats.
#include "gn_model.h"

namespace gn {

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

// state after n further LCG steps
__device__ u128 pcg_advance(u128 s, uint64_t n) {
  u128 cm = pcg_mul(), cp = pcg_inc();
  u128 am = {0, 1}, ap = {0, 0};
  while (n) {
    if (n & 1) {
      am = mul128(am, cm);
      ap = add128(mul128(ap, cm), cp);
    }
    u128 cm1 = add128(cm, u128{0, 1});
    cp = mul128(cm1, cp);
    cm = mul128(cm, cm);
    n >>= 1;
  }
  return add128(mul128(am, s), ap);
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

__device__ __forceinline__ uint32_t order_key(float f) {
  uint32_t b = __float_as_uint(f);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float key_float(uint32_t u) {
  uint32_t b = (u & 0x80000000u) ? (u & 0x7fffffffu) : ~u;
  return __uint_as_float(b);
}

__global__ __launch_bounds__(256) void sampler_kernel(SamplerArgs a) {
  __shared__ uint32_t hist[4][256];
  __shared__ uint32_t sel_prefix, sel_k;
  __shared__ float best_v[4];
  __shared__ int best_i[4];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int row = blockIdx.x;
  const float* z = a.logits + (int64_t)row * a.ldl;
  const int V = a.V;

  if (a.temperature <= 0.f) {
    // argMax: first index of the largest value (sampler.go:37-45)
    float bv = -INFINITY;
    int bi = -1;
    for (int v = tid; v < V; v += 256)
      if (bi < 0 || z[v] > bv) { bv = z[v]; bi = v; }
    for (int o = 32; o > 0; o >>= 1) {
      float ov = __shfl_xor(bv, o, 64);
      int oi = __shfl_xor(bi, o, 64);
      if (oi >= 0 && (bi < 0 || ov > bv || (ov == bv && oi < bi))) { bv = ov; bi = oi; }
    }
    if (lane == 0) { best_v[wid] = bv; best_i[wid] = bi; }
    __syncthreads();
    if (tid == 0) {
      for (int w = 1; w < 4; w++)
        if (best_i[w] >= 0 && (bi < 0 || best_v[w] > bv || (best_v[w] == bv && best_i[w] < bi))) {
          bv = best_v[w]; bi = best_i[w];
        }
      a.out[row] = bi < 0 ? 0 : bi;
    }
    return;
  }

  // ---- threshold: k-th largest (multiset), or -inf when no top-k mask -----
  float thr = -INFINITY;
  const bool masking = a.top_k > 0 && a.top_k < V;
  if (masking) {
    uint32_t prefix = 0, pmask = 0, kk = (uint32_t)a.top_k;
    for (int pass = 0; pass < 4; pass++) {
      const int shift = 24 - 8 * pass;
      for (int i = tid; i < 4 * 256; i += 256) (&hist[0][0])[i] = 0;
      __syncthreads();
      for (int v = tid; v < V; v += 256) {
        uint32_t u = order_key(z[v]);
        if ((u & pmask) == prefix) atomicAdd(&hist[wid][(u >> shift) & 255u], 1u);
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
  }

  // ---- Gumbel-max over the surviving entries ------------------------------
  const int g = row / a.samples_per_group, i = row % a.samples_per_group;
  const int chunk = (V + 255) / 256;
  const int v0 = tid * chunk, v1 = min(V, v0 + chunk);
  u128 s = {a.base_states[2 * g], a.base_states[2 * g + 1]};
  s = pcg_advance(s, (uint64_t)i * (uint64_t)V + (uint64_t)v0);
  float bv = -INFINITY;
  int bi = -1;
  const float T = a.temperature;
  for (int v = v0; v < v1; v++) {
    s = pcg_step(s);
    const float zv = z[v];
    if (zv >= thr) {
      float u = pcg_float32(s);
      if (u <= 0.f) u = 1e-12f;
      float gum = -(float)log(-log((double)u));
      float sc = __fadd_rn(__fdiv_rn(zv, T), gum);
      if (sc > bv) { bv = sc; bi = v; }
    }
  }
  for (int o = 32; o > 0; o >>= 1) {
    float ov = __shfl_xor(bv, o, 64);
    int oi = __shfl_xor(bi, o, 64);
    if (oi >= 0 && (bi < 0 || ov > bv || (ov == bv && oi < bi))) { bv = ov; bi = oi; }
  }
  if (lane == 0) { best_v[wid] = bv; best_i[wid] = bi; }
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < 4; w++)
      if (best_i[w] >= 0 && (bi < 0 || best_v[w] > bv || (best_v[w] == bv && best_i[w] < bi))) {
        bv = best_v[w]; bi = best_i[w];
      }
    a.out[row] = bi < 0 ? 0 : bi;
  }
}

void launch_sampler(const SamplerArgs& a, hipStream_t st) {
  if (a.rows <= 0) return;
  GN_CHECK(a.V > 0, "sampler: empty vocabulary");
  hipLaunchKernelGGL(sampler_kernel, dim3(a.rows), dim3(256), 0, st, a);
  GN_HIP(hipGetLastError());
}

}  // namespace gn
