// gn_blaslt.cpp - plain fp32 products through hipBLASLt (see gn_blaslt.h).
#include "gn_blaslt.h"

#include <hipblaslt/hipblaslt.h>

#include <map>
#include <memory>
#include <string>
#include <tuple>

namespace gn {

namespace {

constexpr size_t kWorkspace = 64u << 20;
// below this many multiply-adds gemm_kernel is as fast (the M = 256 decode
// projections) and keeps its fused epilogues
constexpr double kMinMacs = 268435456.0;
constexpr double kDeferMacs = 1073741824.0;

#define GN_LT(expr)                                                                          \
  do {                                                                                       \
    hipblasStatus_t _s = (expr);                                                             \
    if (_s != HIPBLAS_STATUS_SUCCESS)                                                        \
      throw ::gn::Error(GN_ERR_HIP, std::string("hipBLASLt: ") + #expr + " failed (status " + \
                                        std::to_string((int)_s) + ")");                      \
  } while (0)

// (M, N, K, a_kcontig, b_kcontig, lda, ldb, ldc, ldcin, has Cin)
using Key = std::tuple<int, int, int, bool, bool, int64_t, int64_t, int64_t, int64_t, bool>;

struct Plan {
  bool ok = false;
  hipblasLtMatmulDesc_t op = nullptr;
  hipblasLtMatrixLayout_t la = nullptr, lb = nullptr, lc = nullptr, ld = nullptr;
  hipblasLtMatmulAlgo_t algo{};
};

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace

struct BlasLt {
  hipblasLtHandle_t h = nullptr;
  void* ws = nullptr;
  std::map<Key, Plan> plans;
};

BlasLt* blaslt_create() {
  auto b = std::make_unique<BlasLt>();
  GN_LT(hipblasLtCreate(&b->h));
  GN_HIP(hipMalloc(&b->ws, kWorkspace));
  return b.release();
}

void blaslt_destroy(BlasLt* b) {
  if (!b) return;
  for (auto& kv : b->plans) {
    Plan& p = kv.second;
    if (p.la) (void)hipblasLtMatrixLayoutDestroy(p.la);
    if (p.lb) (void)hipblasLtMatrixLayoutDestroy(p.lb);
    if (p.lc) (void)hipblasLtMatrixLayoutDestroy(p.lc);
    if (p.ld) (void)hipblasLtMatrixLayoutDestroy(p.ld);
    if (p.op) (void)hipblasLtMatmulDescDestroy(p.op);
  }
  if (b->ws) (void)hipFree(b->ws);
  if (b->h) (void)hipblasLtDestroy(b->h);
  delete b;
}

// hipBLASLt is column-major: the row-major C[M][N] is the column-major
// N x M matrix D = op(Bm) . op(Am), where Bm is our B (N x K operand) and
// Am our A (M x K operand) read as column-major matrices.
static Plan make_plan(BlasLt* b, const GemmDesc& d, int64_t ldcin, bool has_cin) {
  Plan p;
  GN_LT(hipblasLtMatmulDescCreate(&p.op, HIPBLAS_COMPUTE_32F, HIP_R_32F));
  const hipblasOperation_t ta = d.b_kcontig ? HIPBLAS_OP_T : HIPBLAS_OP_N;
  const hipblasOperation_t tb = d.a_kcontig ? HIPBLAS_OP_N : HIPBLAS_OP_T;
  GN_LT(hipblasLtMatmulDescSetAttribute(p.op, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof(ta)));
  GN_LT(hipblasLtMatmulDescSetAttribute(p.op, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof(tb)));
  // B(n, k) = b_kcontig ? B[n*ldb + k] (column-major K x N) : B[k*ldb + n] (N x K)
  GN_LT(hipblasLtMatrixLayoutCreate(&p.la, HIP_R_32F, d.b_kcontig ? d.K : d.N,
                                    d.b_kcontig ? d.N : d.K, d.ldb));
  // A(m, k) = a_kcontig ? A[m*lda + k] (column-major K x M) : A[k*lda + m] (M x K)
  GN_LT(hipblasLtMatrixLayoutCreate(&p.lb, HIP_R_32F, d.a_kcontig ? d.K : d.M,
                                    d.a_kcontig ? d.M : d.K, d.lda));
  GN_LT(hipblasLtMatrixLayoutCreate(&p.lc, HIP_R_32F, d.N, d.M, has_cin ? ldcin : d.ldc));
  GN_LT(hipblasLtMatrixLayoutCreate(&p.ld, HIP_R_32F, d.N, d.M, d.ldc));
  hipblasLtMatmulPreference_t pref;
  GN_LT(hipblasLtMatmulPreferenceCreate(&pref));
  size_t wsb = kWorkspace;
  hipblasStatus_t st = hipblasLtMatmulPreferenceSetAttribute(
      pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &wsb, sizeof(wsb));
  hipblasLtMatmulHeuristicResult_t res[1];
  int nres = 0;
  if (st == HIPBLAS_STATUS_SUCCESS)
    st = hipblasLtMatmulAlgoGetHeuristic(b->h, p.op, p.la, p.lb, p.lc, p.ld, pref, 1, res, &nres);
  (void)hipblasLtMatmulPreferenceDestroy(pref);
  if (st == HIPBLAS_STATUS_SUCCESS && nres > 0 && res[0].workspaceSize <= kWorkspace) {
    p.algo = res[0].algo;
    p.ok = true;
  }
  return p;
}

bool blaslt_gemm(BlasLt* b, const GemmDesc& d, hipStream_t st) {
  if (!b || d.group != GEMM_GROUP_NONE || d.force_splits > 0) return false;
  if (d.M <= 0 || d.N <= 0 || d.K <= 0) return false;
  // A product whose split-K sum its consumer could take (d.defer) stays on
  // gemm_kernel below kDeferMacs (d12 decode at M = 256: its deferred split
  // sums are as fast or faster, proj 17.7 vs 20.3 us); above it hipBLASLt
  // runs it whole and leaves nothing pending (d20 decode at M = 512: proj
  // 59 vs 67 us).
  if ((double)d.M * d.N * d.K < (d.defer ? kDeferMacs : kMinMacs)) return false;
  float alpha = 1.f, beta = 0.f;
  const float* cin = nullptr;
  int64_t ldcin = d.ldc;
  switch (d.epi) {
    case EPI_STORE:
      alpha = d.alpha;
      break;
    case EPI_ACCUM:
      beta = 1.f;
      cin = d.C;
      break;
    case EPI_ADD_SRC:
      beta = 1.f;
      cin = d.aux;
      ldcin = d.ldaux;
      break;
    default:
      return false;  // fused epilogues stay on gemm_kernel
  }
  if (!aligned16(d.A) || !aligned16(d.B) || !aligned16(d.C) || (cin && !aligned16(cin)) ||
      d.lda % 4 || d.ldb % 4 || d.ldc % 4 || ldcin % 4)
    return false;
  const Key key{d.M, d.N, d.K, d.a_kcontig, d.b_kcontig, d.lda, d.ldb, d.ldc, ldcin, cin != nullptr};
  auto it = b->plans.find(key);
  if (it == b->plans.end()) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    GN_HIP(hipStreamIsCapturing(st, &cs));
    if (cs != hipStreamCaptureStatusNone) return false;  // choose algorithms outside captures
    it = b->plans.emplace(key, make_plan(b, d, ldcin, cin != nullptr)).first;
  }
  const Plan& p = it->second;
  if (!p.ok) return false;
  if (d.defer) *d.defer = PendingSum{};  // the whole sum, nothing left pending
  GN_LT(hipblasLtMatmul(b->h, p.op, &alpha, d.B, p.la, d.A, p.lb, &beta, cin ? cin : d.C, p.lc,
                        d.C, p.ld, &p.algo, b->ws, kWorkspace, st));
  return true;
}

}  // namespace gn
