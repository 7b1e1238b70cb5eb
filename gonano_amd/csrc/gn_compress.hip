// gn_compress.hip - the flash preset's compressed attention (HCA,
// model/compress.go, model/compress_attention.go): the channel compressor,
// the merge of the global (compressed) and local (sliding-window) branches,
// their backward, and the decode-time compression of each completed block.
//
// The compressor reduces each block of `ratio` positions of a sequence to
// one key and one value row: per channel d, a softmax over the block's rows
// of the logits Wl.h + bias[t % ratio] (ChannelCompressor.Forward,
// compress.go:110-164) weights the rows' keys (and values).  The logits are
// shared by every KV head and by K and V, so the kernels take one thread per
// (sequence, block, channel) and loop over heads: the logits are read once,
// the K/V rows of a block are read once, and every access is a contiguous
// 512-byte row across the 128 threads of a channel group.  Block rows are
// compile-time (RT = ratio) so the per-row values stay in registers.
//
// The logit GEMM (h . Wl^T) and its two backward GEMMs run on the matrix
// cores through gemm(); the kernels here are HBM-bound elementwise passes.
#include "gn_model.h"

namespace gn {

static constexpr int CD = 128;  // channels = head dim

// ---------------------------------------------------------------------------
// Training / prefill compressor
// ---------------------------------------------------------------------------
template <int RT>
__global__ __launch_bounds__(256) void hca_compress_kernel(HcaCompressArgs a) {
  const int d = threadIdx.x & (CD - 1);
  const int blocks = (a.T + RT - 1) / RT;
  const int64_t pair = (int64_t)blockIdx.x * 2 + (threadIdx.x >> 7);  // (b, block)
  if (pair >= (int64_t)a.B * blocks) return;
  const int b = (int)(pair / blocks), bl = (int)(pair % blocks);
  const int t0 = bl * RT, n = min(RT, a.T - t0);
  const int64_t row0 = (int64_t)b * a.T + t0;
  float lg[RT], p[RT];
  float mx = -INFINITY;
#pragma unroll
  for (int r = 0; r < RT; r++) {
    lg[r] = r < n ? a.clog[(row0 + r) * CD + d] + a.bias[r * CD + d] : -INFINITY;
    mx = fmaxf(mx, lg[r]);
  }
  float tot = 0.f;
#pragma unroll
  for (int r = 0; r < RT; r++) {
    p[r] = r < n ? expf(lg[r] - mx) : 0.f;
    tot += p[r];
  }
  const float inv = 1.f / tot;
#pragma unroll
  for (int r = 0; r < RT; r++) {
    p[r] *= inv;
    a.probs[(pair * RT + r) * CD + d] = p[r];
  }
  const int full = a.T / RT;  // complete blocks of the sequence
  for (int hk = 0; hk < a.Hkv; hk++) {
    float ak = 0.f, av = 0.f;
#pragma unroll
    for (int r = 0; r < RT; r++)
      if (r < n) {
        const int64_t off = ((row0 + r) * a.Hkv + hk) * CD + d;
        ak += p[r] * a.k[off];
        av += p[r] * a.v[off];
      }
    const int64_t co = (pair * a.Hkv + hk) * CD + d;
    a.kc[co] = ak;
    a.vc[co] = av;
    if (a.ck_pf && bl < full) {
      const int64_t po = (((int64_t)b * a.Hkv + hk) * full + bl) * CD + d;
      a.ck_pf[po] = ak;
      a.cv_pf[po] = av;
    }
  }
  // the logits (and, in tail mode, keys/values) of an incomplete last block
  // wait in the decode ring
  if (a.ring_pf && n < RT)
#pragma unroll
    for (int r = 0; r < RT; r++)
      if (r < n) a.ring_pf[((int64_t)b * RT + r) * CD + d] = lg[r];
  if (a.tailk_pf && n < RT)
    for (int hk = 0; hk < a.Hkv; hk++)
      for (int r = 0; r < n; r++) {
        const int64_t off = ((row0 + r) * a.Hkv + hk) * CD + d;
        const int64_t to = (((int64_t)b * a.Hkv + hk) * RT + r) * CD + d;
        a.tailk_pf[to] = a.k[off];
        a.tailv_pf[to] = a.v[off];
      }
}

#define GN_RATIO_SWITCH(ratio, KERNEL, ...)                                 \
  switch (ratio) {                                                          \
    case 2: KERNEL<2>(__VA_ARGS__); break;                                  \
    case 3: KERNEL<3>(__VA_ARGS__); break;                                  \
    case 4: KERNEL<4>(__VA_ARGS__); break;                                  \
    case 5: KERNEL<5>(__VA_ARGS__); break;                                  \
    case 6: KERNEL<6>(__VA_ARGS__); break;                                  \
    case 7: KERNEL<7>(__VA_ARGS__); break;                                  \
    case 8: KERNEL<8>(__VA_ARGS__); break;                                  \
    case 16: KERNEL<16>(__VA_ARGS__); break;                                \
    default: throw Error(GN_ERR_INVALID, "compression ratio must be 2..8 or 16"); \
  }

bool hca_ratio_supported(int ratio) { return (ratio >= 2 && ratio <= 8) || ratio == 16; }

template <int RT>
static void run_compress(const HcaCompressArgs& a, hipStream_t st) {
  const int64_t pairs = (int64_t)a.B * ((a.T + RT - 1) / RT);
  hipLaunchKernelGGL(hca_compress_kernel<RT>, dim3((unsigned)ceil_div(pairs, 2)), dim3(256), 0, st,
                     a);
}

void launch_hca_compress(const HcaCompressArgs& a, hipStream_t st) {
  GN_CHECK(a.B > 0 && a.T > 0 && a.Hkv > 0, "compressor: empty input");
  GN_CHECK((a.ck_pf == nullptr) == (a.cv_pf == nullptr), "compressor: prefill caches come in pairs");
  GN_RATIO_SWITCH(a.ratio, run_compress, a, st);
  GN_HIP(hipGetLastError());
}

// ---------------------------------------------------------------------------
// Branch merge (mergeAttentionBranches, compress_attention.go:440-466): one
// wave per (token, head) row of 128.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void merge_branches_kernel(const float* __restrict__ oa,
                                                             const float* __restrict__ la,
                                                             const float* __restrict__ ob,
                                                             const float* __restrict__ lb,
                                                             float* __restrict__ out,
                                                             float* __restrict__ lse,
                                                             int64_t rows) {
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (r >= rows) return;
  const float a = la[r], b = lb[r];
  const float mx = fmaxf(a, b);
  float2* op = reinterpret_cast<float2*>(out + r * CD) + lane;
  if (mx == -INFINITY) {
    *op = make_float2(0.f, 0.f);
    if (lse && lane == 0) lse[r] = -INFINITY;
    return;
  }
  const float wa = expf(a - mx), wb = expf(b - mx);
  const float tot = wa + wb, inv = 1.f / tot;
  const float2 x = reinterpret_cast<const float2*>(oa + r * CD)[lane];
  const float2 y = reinterpret_cast<const float2*>(ob + r * CD)[lane];
  *op = make_float2((wa * x.x + wb * y.x) * inv, (wa * x.y + wb * y.y) * inv);
  if (lse && lane == 0) lse[r] = mx + logf(tot);
}

void launch_merge_branches(const float* oa, const float* la, const float* ob, const float* lb,
                           float* out, float* lse, int64_t rows, hipStream_t st) {
  hipLaunchKernelGGL(merge_branches_kernel, dim3((unsigned)ceil_div(rows, 4)), dim3(256), 0, st,
                     oa, la, ob, lb, out, lse, rows);
  GN_HIP(hipGetLastError());
}

// ---------------------------------------------------------------------------
// Compressor backward (ChannelCompressor.Backward's softmax part,
// compress.go:199-222): for a block's row t and channel d,
//   dlogit[t][d] = sum over heads, K and V of p * g * (x[t] - compressed)
//   dx[t][d]    += p * g
// The logit gradient of all heads and of K and V is summed here, so one GEMM
// pair gives the weight gradient and the input gradient.
// ---------------------------------------------------------------------------
template <int RT>
__global__ __launch_bounds__(256) void hca_compress_bwd_kernel(HcaCompressBwdArgs a) {
  const int d = threadIdx.x & (CD - 1);
  const int blocks = (a.T + RT - 1) / RT;
  const int64_t pair = (int64_t)blockIdx.x * 2 + (threadIdx.x >> 7);
  if (pair >= (int64_t)a.B * blocks) return;
  const int b = (int)(pair / blocks), bl = (int)(pair % blocks);
  const int t0 = bl * RT, n = min(RT, a.T - t0);
  const int64_t row0 = (int64_t)b * a.T + t0;
  float p[RT], gl[RT];
#pragma unroll
  for (int r = 0; r < RT; r++) {
    p[r] = a.probs[(pair * RT + r) * CD + d];
    gl[r] = 0.f;
  }
  for (int hk = 0; hk < a.Hkv; hk++) {
    const int64_t co = (pair * a.Hkv + hk) * CD + d;
    const float gk = a.dkc[co], ck = a.kc[co], gv = a.dvc[co], cv = a.vc[co];
#pragma unroll
    for (int r = 0; r < RT; r++)
      if (r < n) {
        const int64_t off = ((row0 + r) * a.Hkv + hk) * CD + d;
        const float pk = p[r] * gk, pv = p[r] * gv;
        gl[r] += pk * (a.k[off] - ck) + pv * (a.v[off] - cv);
        a.dk[off] += pk;
        a.dv[off] += pv;
      }
  }
#pragma unroll
  for (int r = 0; r < RT; r++)
    if (r < n) a.glog[(row0 + r) * CD + d] = gl[r];
}

// Bias gradient: gbias[r][d] += sum of glog over the rows at position
// r (mod ratio) of every sequence, in two deterministic passes (partials per
// chunk of blocks, then a fixed-order sum).
static constexpr int BIAS_CHUNKS = 256;

__global__ __launch_bounds__(128) void hca_bias_partial_kernel(const float* __restrict__ glog,
                                                               int B, int T, int ratio,
                                                               float* __restrict__ part) {
  const int d = threadIdx.x, r = blockIdx.y, c = blockIdx.x;
  const int blocks = (T + ratio - 1) / ratio;
  const int64_t pairs = (int64_t)B * blocks;
  const int64_t per = (pairs + BIAS_CHUNKS - 1) / BIAS_CHUNKS;
  const int64_t p0 = c * per, p1 = min(pairs, p0 + per);
  float acc = 0.f;
  for (int64_t pr = p0; pr < p1; pr++) {
    const int b = (int)(pr / blocks), t = (int)(pr % blocks) * ratio + r;
    if (t < T) acc += glog[((int64_t)b * T + t) * CD + d];
  }
  part[((int64_t)c * ratio + r) * CD + d] = acc;
}

__global__ __launch_bounds__(128) void hca_bias_sum_kernel(const float* __restrict__ part,
                                                           int ratio, float* __restrict__ gbias) {
  const int d = threadIdx.x, r = blockIdx.x;
  float acc = 0.f;
  for (int c = 0; c < BIAS_CHUNKS; c++) acc += part[((int64_t)c * ratio + r) * CD + d];
  gbias[r * CD + d] += acc;
}

template <int RT>
static void run_compress_bwd(const HcaCompressBwdArgs& a, hipStream_t st) {
  const int64_t pairs = (int64_t)a.B * ((a.T + RT - 1) / RT);
  hipLaunchKernelGGL(hca_compress_bwd_kernel<RT>, dim3((unsigned)ceil_div(pairs, 2)), dim3(256), 0,
                     st, a);
}

void launch_hca_compress_bwd(const HcaCompressBwdArgs& a, hipStream_t st) {
  GN_CHECK(a.B > 0 && a.T > 0 && a.Hkv > 0, "compressor backward: empty input");
  GN_RATIO_SWITCH(a.ratio, run_compress_bwd, a, st);
  GN_HIP(hipGetLastError());
  hipLaunchKernelGGL(hca_bias_partial_kernel, dim3(BIAS_CHUNKS, a.ratio), dim3(CD), 0, st, a.glog,
                     a.B, a.T, a.ratio, a.bias_part);
  GN_HIP(hipGetLastError());
  hipLaunchKernelGGL(hca_bias_sum_kernel, dim3(a.ratio), dim3(CD), 0, st, a.bias_part, a.ratio,
                     a.gbias);
  GN_HIP(hipGetLastError());
}

size_t hca_bias_part_floats(int ratio) { return (size_t)BIAS_CHUNKS * ratio * CD; }

// ---------------------------------------------------------------------------
// Decode (appendGlobalTail / compressTail, compress_attention.go:848-890):
// the current token's logits (+ bias of its slot) enter the row's ring; the
// token that completes a block compresses the block's raw cached keys and
// values into compressed slot pos / ratio.  One block of 128 threads per
// row; the position may be read on the device (captured decode graphs).
// ---------------------------------------------------------------------------
template <int RT>
__global__ __launch_bounds__(128) void hca_decode_compress_kernel(HcaDecodeArgs a) {
  const int d = threadIdx.x, row = blockIdx.x;
  const int pos = a.pos_dev ? *a.pos_dev : a.pos;
  const int slot = pos % RT;
  float* ring = a.ring + (int64_t)row * RT * CD + d;
  const float cur = a.clog[(int64_t)row * CD + d] + a.bias[slot * CD + d];
  ring[slot * CD] = cur;
  if (a.tailk)  // this token's keys/values into its tail slot
    for (int hk = 0; hk < a.Hkv; hk++) {
      const int64_t tb = (((int64_t)row * a.Hkv + hk) * RT + slot) * CD + d;
      a.tailk[tb] = a.knew[((int64_t)row * a.Hkv + hk) * CD + d];
      a.tailv[tb] = a.vnew[((int64_t)row * a.Hkv + hk) * CD + d];
    }
  if (slot != RT - 1) return;
  const int blk = pos / RT;
  if (blk >= a.maxBlocks) return;  // the host sizes maxBlocks past every position
  float p[RT];
  float mx = -INFINITY;
#pragma unroll
  for (int r = 0; r < RT; r++) {
    p[r] = r == RT - 1 ? cur : ring[r * CD];  // written by this thread in earlier steps
    mx = fmaxf(mx, p[r]);
  }
  float tot = 0.f;
#pragma unroll
  for (int r = 0; r < RT; r++) {
    p[r] = expf(p[r] - mx);
    tot += p[r];
  }
  const float inv = 1.f / tot;
#pragma unroll
  for (int r = 0; r < RT; r++) p[r] *= inv;
  const int start = pos - RT + 1;
  for (int hk = 0; hk < a.Hkv; hk++) {
    const float* ksrc = a.tailk ? a.tailk + ((int64_t)row * a.Hkv + hk) * RT * CD + d
                                : a.kc + (((int64_t)row * a.Hkv + hk) * a.maxSeq + start) * CD + d;
    const float* vsrc = a.tailk ? a.tailv + ((int64_t)row * a.Hkv + hk) * RT * CD + d
                                : a.vc + (((int64_t)row * a.Hkv + hk) * a.maxSeq + start) * CD + d;
    float ak = 0.f, av = 0.f;
#pragma unroll
    for (int r = 0; r < RT; r++) {
      ak += p[r] * ksrc[(int64_t)r * CD];
      av += p[r] * vsrc[(int64_t)r * CD];
    }
    const int64_t co = (((int64_t)row * a.Hkv + hk) * a.maxBlocks + blk) * CD + d;
    a.ck[co] = ak;
    a.cv[co] = av;
  }
}

template <int RT>
static void run_decode_compress(const HcaDecodeArgs& a, hipStream_t st) {
  hipLaunchKernelGGL(hca_decode_compress_kernel<RT>, dim3(a.rows), dim3(CD), 0, st, a);
}

// The indexer key of the block completed at this step (one block per
// (row, kv-head), one thread per output, 128-term dot in order).
__global__ __launch_bounds__(256) void indexer_key_step_kernel(const float* __restrict__ ck,
                                                               const float* __restrict__ wik,
                                                               float* __restrict__ ik, int Hkv,
                                                               int maxBlocks, int HI, int ratio,
                                                               int pos0, const int* pos_dev) {
  const int pos = pos_dev ? *pos_dev : pos0;
  if (pos % ratio != ratio - 1) return;
  const int blk = pos / ratio;
  if (blk >= maxBlocks) return;
  const int row = blockIdx.x / Hkv, hk = blockIdx.x % Hkv;
  __shared__ float crow[CD];
  const float* src = ck + (((int64_t)row * Hkv + hk) * maxBlocks + blk) * CD;
  for (int i = threadIdx.x; i < CD; i += blockDim.x) crow[i] = src[i];
  __syncthreads();
  for (int o = threadIdx.x; o < HI; o += blockDim.x) {
    const float* w = wik + (int64_t)o * CD;
    float acc = 0.f;
    for (int i = 0; i < CD; i++) acc += crow[i] * w[i];
    ik[(((int64_t)row * maxBlocks + blk) * Hkv + hk) * HI + o] = acc;
  }
}
void launch_indexer_key_step(const float* ck, const float* wik, float* ik, int rows, int Hkv,
                             int maxBlocks, int HI, int ratio, int pos, const int* pos_dev,
                             hipStream_t st) {
  hipLaunchKernelGGL(indexer_key_step_kernel, dim3(rows * Hkv), dim3(256), 0, st, ck, wik, ik, Hkv,
                     maxBlocks, HI, ratio, pos, pos_dev);
  GN_HIP(hipGetLastError());
}

void launch_hca_decode_compress(const HcaDecodeArgs& a, hipStream_t st) {
  GN_CHECK(a.rows > 0 && a.maxBlocks * a.ratio > a.maxSeq - 1, "decode compressor: cache too small");
  if (!a.pos_dev) GN_CHECK(a.pos >= 0 && a.pos < a.maxSeq, "decode compressor: position outside the cache");
  GN_RATIO_SWITCH(a.ratio, run_decode_compress, a, st);
  GN_HIP(hipGetLastError());
}

}  // namespace gn
