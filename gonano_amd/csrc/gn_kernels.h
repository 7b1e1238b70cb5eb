// gn_kernels.h - launchers shared between the backend primitives and the
// session.  All launchers enqueue on the given stream and never synchronize.
#pragma once

#include <algorithm>
#include <map>
#include <string>

#include "gn_common.h"

namespace gn {

// ---------------------------------------------------------------------------
// Grow-only named device buffers.  Growing synchronizes the owning stream
// first so no in-flight kernel still reads the old allocation.
// ---------------------------------------------------------------------------
class DeviceArena {
 public:
  explicit DeviceArena(hipStream_t s = nullptr) : stream_(s) {}
  ~DeviceArena() { release(); }
  DeviceArena(const DeviceArena&) = delete;
  DeviceArena& operator=(const DeviceArena&) = delete;
  void set_stream(hipStream_t s) { stream_ = s; }

  template <typename T>
  T* get(const std::string& name, size_t count) {
    size_t bytes = std::max<size_t>(count * sizeof(T), 256);
    auto it = bufs_.find(name);
    if (it != bufs_.end() && it->second.bytes >= bytes) return static_cast<T*>(it->second.ptr);
    if (it != bufs_.end()) {
      GN_HIP(hipStreamSynchronize(stream_));
      GN_HIP(hipFree(it->second.ptr));
      bufs_.erase(it);
    }
    void* p = nullptr;
    GN_HIP(hipMalloc(&p, bytes));
    bufs_[name] = Buf{p, bytes};
    return static_cast<T*>(p);
  }
  void release() {
    for (auto& kv : bufs_) (void)hipFree(kv.second.ptr);
    bufs_.clear();
  }
  size_t bytes() const {
    size_t t = 0;
    for (auto& kv : bufs_) t += kv.second.bytes;
    return t;
  }

 private:
  struct Buf {
    void* ptr;
    size_t bytes;
  };
  hipStream_t stream_;
  std::map<std::string, Buf> bufs_;
};

// ---------------------------------------------------------------------------
// GEMM
// ---------------------------------------------------------------------------
enum GemmEpilogue {
  EPI_STORE = 0,      // C = alpha * acc
  EPI_ADD_SRC = 1,    // C = acc + aux            (residual add; aux may alias C)
  EPI_ACCUM = 2,      // C += acc                 (gradient accumulation)
  EPI_SOFTCAP = 3,    // C = 15 tanh(acc / 15)    (logits)
  EPI_RELU2_SAVE = 4, // aux_out = acc, C = relu(acc)^2
  EPI_DRELU2 = 5      // C = acc * 2 * relu(aux)  (ReluSquared backward)
};

// Expert-grouped GEMM modes (the MoE feed-forward): rows of A and C, or the
// reduction rows, are concatenated groups whose offsets live on the device,
// so the launch shape does not depend on how tokens were routed.
enum GemmGroup {
  GEMM_GROUP_NONE = 0,
  GEMM_GROUP_ROWS = 1,  // C[goff[g]:goff[g+1]] = A[same rows] . B_g^T, B_g = B + g*group_stride
  GEMM_GROUP_K = 2      // C_g (= C + g*group_stride) op= sum over k in [goff[g], goff[g+1])
};

// Split-K partial sums left for the kernel that reads the product next:
// value (m, n) = (float) sum over z < splits, in z order, of (double)
// part[z * stride + m * N + n] -- what gemm_reduce_kernel computes.
// splits == 0: the GEMM wrote its output itself.
struct PendingSum {
  const float* part = nullptr;
  int splits = 0;
  int64_t stride = 0;
};
// Consumers hold every partial of their elements in registers (all loads in
// flight at once), so a GEMM defers its sum only up to this many splits.
constexpr int PENDING_MAX_SPLITS = 8;
// Element i of a deferred product: its partials summed in split order in
// float64 and rounded once (gemm_reduce_kernel's result before its epilogue).
__device__ __forceinline__ float pending_value(const PendingSum& ps, int64_t i) {
  float v[PENDING_MAX_SPLITS];
#pragma unroll
  for (int z = 0; z < PENDING_MAX_SPLITS; z++)
    if (z < ps.splits) v[z] = ps.part[z * ps.stride + i];  // every load before the sum
  double s = 0.0;
#pragma unroll
  for (int z = 0; z < PENDING_MAX_SPLITS; z++)
    if (z < ps.splits) s += (double)v[z];
  return (float)s;
}

struct GemmDesc {
  int M = 0, N = 0, K = 0;
  const float* A = nullptr;
  int64_t lda = 0;
  bool a_kcontig = true;  // A(m,k) = a_kcontig ? A[m*lda+k] : A[k*lda+m]
  const float* B = nullptr;
  int64_t ldb = 0;
  bool b_kcontig = true;  // B(n,k) = b_kcontig ? B[n*ldb+k] : B[k*ldb+n]
  float* C = nullptr;
  int64_t ldc = 0;
  int epi = EPI_STORE;
  const float* aux = nullptr;
  float* aux_out = nullptr;
  int64_t ldaux = 0;
  float alpha = 1.f;
  int force_splits = 0;
  int group = GEMM_GROUP_NONE;
  const int* group_off = nullptr;  // device [groups + 1]
  int groups = 0;
  int64_t group_stride = 0;
  int a_pad_rows = 0;  // rows mode: readable rows of A past row M (>= 128 enables full tiles)
  // Plain products only (EPI_STORE with alpha 1, or EPI_ADD_SRC with aux ==
  // C, ldc == ldaux == N): when the product splits K, leave the partials in
  // *defer instead of launching the reduction; the consumer applies the sum
  // (and the residual add) as gemm_reduce_kernel would.
  PendingSum* defer = nullptr;
  // partial buffer of a deferred sum: products whose sums are pending at the
  // same time use different slots
  int defer_slot = 0;
  // batch products of one shape (gemm_kernel only; EPI_STORE or EPI_ACCUM):
  // product i takes A + i*batch_sa, B + i*batch_sb, C + i*batch_sc
  int batch = 1;
  int64_t batch_sa = 0, batch_sb = 0, batch_sc = 0;
};

// Which kernel ran a product: gemm_kernel (tiles up to 128 x 128, fused
// epilogues, grouped and deferred products), the wide-tile engine (256 x
// 256 tiles for the large products) or the slim-tile engine (32-row tiles
// for the decode projections); all in gn_gemm.hip.
enum GemmEngine { GEMM_ENGINE_TILE = 0, GEMM_ENGINE_WIDE = 1, GEMM_ENGINE_SLIM = 2 };

GemmEngine gemm(const GemmDesc& d, hipStream_t st, DeviceArena* ws);

// y[rows, out] = x[rows, in] . W[out, in]^T   (model/layers/linear.go:32-40)
inline GemmDesc linear_fwd_desc(const float* x, const float* W, float* y, int rows, int in,
                                int out, int epi = EPI_STORE) {
  GemmDesc d;
  d.M = rows; d.N = out; d.K = in;
  d.A = x; d.lda = in; d.a_kcontig = true;
  d.B = W; d.ldb = in; d.b_kcontig = true;
  d.C = y; d.ldc = out; d.epi = epi;
  return d;
}
// dx[rows, in] = g[rows, out] . W[out, in]    (linear.go:51)
inline GemmDesc linear_dx_desc(const float* g, const float* W, float* dx, int rows, int in,
                               int out, int epi = EPI_STORE) {
  GemmDesc d;
  d.M = rows; d.N = in; d.K = out;
  d.A = g; d.lda = out; d.a_kcontig = true;
  d.B = W; d.ldb = in; d.b_kcontig = false;
  d.C = dx; d.ldc = in; d.epi = epi;
  return d;
}
// dW[out, in] += g[rows, out]^T . x[rows, in]  (linear.go:49-50)
inline GemmDesc linear_dw_desc(const float* g, const float* x, float* dW, int rows, int in,
                               int out) {
  GemmDesc d;
  d.M = out; d.N = in; d.K = rows;
  d.A = g; d.lda = out; d.a_kcontig = false;
  d.B = x; d.ldb = in; d.b_kcontig = false;
  d.C = dW; d.ldc = in; d.epi = EPI_ACCUM;
  return d;
}

}  // namespace gn
