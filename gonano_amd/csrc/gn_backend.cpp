// gn_backend.cpp - the kernels.Backend methods (kernels/backend.go:21-297)
// as extern "C" entry points on host pointers.
//
// Each calling thread owns a stream and a grow-only device arena, so calls
// from concurrent goroutines never share state.  Operands are staged into
// device memory before any result is written back, which makes every
// destination/source aliasing pattern the interface allows safe.
#include <cmath>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include "gn_kernels.h"
#include "gn_prims.h"

namespace gn {

static thread_local std::string t_last_error;
void set_last_error(const std::string& msg) { t_last_error = msg; }

struct ThreadCtx {
  int device = -1;
  hipStream_t stream = nullptr;
  std::unique_ptr<DeviceArena> arena;
  ~ThreadCtx() {
    arena.reset();
    if (stream) (void)hipStreamDestroy(stream);
  }
};
static thread_local int t_device = 0;
static thread_local std::unique_ptr<ThreadCtx> t_ctx;

static ThreadCtx& ctx() {
  if (!t_ctx || t_ctx->device != t_device) {
    t_ctx.reset();
    auto c = std::make_unique<ThreadCtx>();
    int n = 0;
    GN_HIP(hipGetDeviceCount(&n));
    GN_CHECK(n > 0, "no HIP device visible");
    GN_CHECK(t_device >= 0 && t_device < n, "device index out of range");
    GN_HIP(hipSetDevice(t_device));
    GN_HIP(hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking));
    c->arena = std::make_unique<DeviceArena>(c->stream);
    c->device = t_device;
    t_ctx = std::move(c);
  }
  GN_HIP(hipSetDevice(t_ctx->device));
  return *t_ctx;
}

template <typename T>
static T* up(ThreadCtx& c, const char* name, const T* host, int64_t n) {
  T* d = c.arena->get<T>(name, (size_t)std::max<int64_t>(n, 1));
  if (n > 0 && host) GN_HIP(hipMemcpyAsync(d, host, sizeof(T) * n, hipMemcpyHostToDevice, c.stream));
  return d;
}
template <typename T>
static T* dev(ThreadCtx& c, const char* name, int64_t n) {
  return c.arena->get<T>(name, (size_t)std::max<int64_t>(n, 1));
}
template <typename T>
static void down(ThreadCtx& c, T* host, const T* d, int64_t n) {
  if (n > 0) GN_HIP(hipMemcpyAsync(host, d, sizeof(T) * n, hipMemcpyDeviceToHost, c.stream));
}
static void sync(ThreadCtx& c) { GN_HIP(hipStreamSynchronize(c.stream)); }

static void check_ptrs(int64_t n, std::initializer_list<const void*> ps) {
  GN_CHECK(n >= 0, "negative length");
  if (n == 0) return;
  for (auto p : ps) GN_CHECK(p != nullptr, "null pointer with non-zero length");
}

static int ew(float* d, const float* l, const float* r, int64_t n, int op, float f) {
  return guard([&] {
    check_ptrs(n, {d, l});
    if (n == 0) return;
    ThreadCtx& c = ctx();
    float* dl = up(c, "a", l, n);
    float* dr = r ? up(c, "b", r, n) : nullptr;
    float* dd = dev<float>(c, "d", n);
    launch_elementwise(dd, dl, dr, n, op, f, c.stream);
    down(c, d, dd, n);
    sync(c);
  });
}

}  // namespace gn

using namespace gn;

extern "C" {

const char* gn_last_error(void) { return gn::t_last_error.c_str(); }

int gn_device_count(void) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) return 0;
  return n;
}

int gn_set_device(int device) {
  return guard([&] {
    int n = 0;
    GN_HIP(hipGetDeviceCount(&n));
    GN_CHECK(device >= 0 && device < n, "device index out of range");
    gn::t_device = device;
  });
}

int gn_synchronize(void) {
  return guard([&] { sync(ctx()); });
}

// kernels/backend.go:23-66 -------------------------------------------------
int gn_add(float* d, const float* l, const float* r, int64_t n) { return ew(d, l, r, n, EW_ADD, 0); }
int gn_subtract(float* d, const float* l, const float* r, int64_t n) { return ew(d, l, r, n, EW_SUB, 0); }
int gn_multiply(float* d, const float* l, const float* r, int64_t n) { return ew(d, l, r, n, EW_MUL, 0); }
int gn_divide(float* d, const float* l, const float* r, int64_t n) { return ew(d, l, r, n, EW_DIV, 0); }
int gn_scale(float* d, const float* s, float f, int64_t n) { return ew(d, s, nullptr, n, EW_SCALE, f); }
int gn_add_scaled(float* d, const float* b, const float* s, float f, int64_t n) {
  return ew(d, b, s, n, EW_ADD_SCALED, f);
}
int gn_negate(float* d, const float* s, int64_t n) { return ew(d, s, nullptr, n, EW_NEG, 0); }
int gn_abs(float* d, const float* s, int64_t n) { return ew(d, s, nullptr, n, EW_ABS, 0); }
int gn_square(float* d, const float* s, int64_t n) { return ew(d, s, nullptr, n, EW_SQUARE, 0); }
int gn_relu_squared(float* d, const float* s, int64_t n) { return ew(d, s, nullptr, n, EW_RELU2, 0); }
int gn_swiglu(float* d, const float* g, const float* u, float clamp, int64_t n) {
  return ew(d, g, u, n, EW_SWIGLU, clamp);
}
int gn_exp(float* d, const float* s, int64_t n) { return ew(d, s, nullptr, n, EW_EXP, 0); }
int gn_sigmoid(float* d, const float* s, int64_t n) { return ew(d, s, nullptr, n, EW_SIGMOID, 0); }
int gn_tanh(float* d, const float* s, int64_t n) { return ew(d, s, nullptr, n, EW_TANH, 0); }
int gn_rsqrt(float* d, const float* s, int64_t n) { return ew(d, s, nullptr, n, EW_RSQRT, 0); }

int gn_swiglu_backward(float* dg, float* du, const float* g, const float* u, const float* dout,
                       float clamp, int64_t n) {
  return guard([&] {
    check_ptrs(n, {dg, du, g, u, dout});
    if (n == 0) return;
    ThreadCtx& c = ctx();
    float* a = up(c, "a", g, n);
    float* b = up(c, "b", u, n);
    float* o = up(c, "c", dout, n);
    float* x = dev<float>(c, "d", n);
    float* y = dev<float>(c, "e", n);
    launch_swiglu_backward(x, y, a, b, o, clamp, n, c.stream);
    down(c, dg, x, n);
    down(c, du, y, n);
    sync(c);
  });
}

// kernels/backend.go:70-78 -------------------------------------------------
static int reduce_call(const float* v, int64_t n, int op, float* rf, int64_t* ri,
                       const float* w) {
  return guard([&] {
    check_ptrs(n, {v});
    GN_CHECK(rf || ri, "null result pointer");
    ThreadCtx& c = ctx();
    float* dv = up(c, "a", v, n);
    float* dw = w ? up(c, "b", w, n) : nullptr;
    float* of = dev<float>(c, "rf", 1);
    int64_t* oi = dev<int64_t>(c, "ri", 1);
    launch_reduce(dv, n, op, of, oi, dw, c.stream);
    if (rf) down(c, rf, of, 1);
    if (ri) down(c, ri, oi, 1);
    sync(c);
  });
}
int gn_sum(const float* v, int64_t n, float* out) { return reduce_call(v, n, RED_SUM, out, nullptr, nullptr); }
int gn_max(const float* v, int64_t n, float* out) { return reduce_call(v, n, RED_MAX, out, nullptr, nullptr); }
int gn_argmax(const float* v, int64_t n, int64_t* out) {
  return reduce_call(v, n, RED_ARGMAX, nullptr, out, nullptr);
}
// DotProduct sums over the shorter input (kernels/scalar/matmul.go:35-42).
int gn_dot_product(const float* l, int64_t ln, const float* r, int64_t rn, float* out) {
  return reduce_call(l, std::min(ln, rn), RED_DOT, out, nullptr, r);
}

// kernels/backend.go:82-90 -------------------------------------------------
static int matmul_call(float* d, const float* l, const float* r, int64_t rows, int64_t cols,
                       int64_t inner, bool transposed) {
  return guard([&] {
    GN_CHECK(rows >= 0 && cols >= 0 && inner >= 0, "negative extent");
    GN_CHECK(rows < (1ll << 31) && cols < (1ll << 31) && inner < (1ll << 31), "extent too large");
    if (rows * cols == 0) return;
    check_ptrs(rows * cols, {d});
    check_ptrs(rows * inner, {l});
    check_ptrs(cols * inner, {r});
    ThreadCtx& c = ctx();
    float* dl = up(c, "a", l, rows * inner);
    float* dr = up(c, "b", r, cols * inner);
    float* dd = dev<float>(c, "d", rows * cols);
    GemmDesc g;
    g.M = (int)rows; g.N = (int)cols; g.K = (int)inner;
    g.A = dl; g.lda = inner; g.a_kcontig = true;
    g.B = dr;
    if (transposed) { g.ldb = inner; g.b_kcontig = true; }
    else { g.ldb = cols; g.b_kcontig = false; }
    g.C = dd; g.ldc = cols;
    gemm(g, c.stream, c.arena.get());
    down(c, d, dd, rows * cols);
    sync(c);
  });
}
int gn_matmul(float* d, const float* l, const float* r, int64_t rows, int64_t cols, int64_t inner) {
  return matmul_call(d, l, r, rows, cols, inner, false);
}
int gn_matmul_transposed(float* d, const float* l, const float* r, int64_t rows, int64_t cols,
                         int64_t inner) {
  return matmul_call(d, l, r, rows, cols, inner, true);
}

// kernels/backend.go:106-115 -----------------------------------------------
int gn_indexer_scores(float* d, const float* q, const float* k, const float* w, int64_t rows,
                      int64_t blocks, int64_t heads, int64_t dim) {
  return guard([&] {
    GN_CHECK(rows >= 0 && blocks >= 0 && heads >= 0 && dim >= 0, "negative extent");
    if (rows * blocks == 0) return;
    ThreadCtx& c = ctx();
    float* dq = up(c, "a", q, rows * heads * dim);
    float* dk = up(c, "b", k, blocks * heads * dim);
    float* dw = up(c, "c", w, heads);
    float* dd = dev<float>(c, "d", rows * blocks);
    launch_indexer_scores(dd, dq, dk, dw, rows, blocks, heads, dim, c.stream);
    down(c, d, dd, rows * blocks);
    sync(c);
  });
}
int gn_indexer_block_max(float* d, const float* s, int64_t rows, int64_t blocks, int64_t group) {
  return guard([&] {
    GN_CHECK(rows >= 0 && blocks >= 0, "negative extent");
    if (group < 1) group = 1;
    int64_t groups = (blocks + group - 1) / group;
    if (rows * groups == 0) return;
    ThreadCtx& c = ctx();
    float* ds = up(c, "a", s, rows * blocks);
    float* dd = dev<float>(c, "d", rows * groups);
    launch_indexer_block_max(dd, ds, rows, blocks, group, c.stream);
    down(c, d, dd, rows * groups);
    sync(c);
  });
}

// kernels/backend.go:125-140 -----------------------------------------------
int gn_topk_indices(int32_t* d, const float* scores, int64_t rows, int64_t count, int64_t k) {
  return guard([&] {
    GN_CHECK(rows >= 0 && count >= 0 && k >= 0, "negative extent");
    if (count == 0 || k == 0 || rows == 0) return;
    check_ptrs(rows * count, {scores});
    check_ptrs(rows * k, {d});
    ThreadCtx& c = ctx();
    float* ds = up(c, "a", scores, rows * count);
    int32_t* dd = dev<int32_t>(c, "i", rows * k);
    // slots the reference leaves untouched (k > count) keep their contents
    GN_HIP(hipMemcpyAsync(dd, d, sizeof(int32_t) * rows * k, hipMemcpyHostToDevice, c.stream));
    uint8_t* taken = dev<uint8_t>(c, "t", rows * count);
    launch_topk_rows(dd, ds, nullptr, rows, count, k, taken, c.stream);
    down(c, d, dd, rows * k);
    sync(c);
  });
}
int gn_moe_gate_topk(const float* logits, const float* bias, float* probs, int32_t* selected,
                     float* weights, int64_t rows, int64_t experts, int64_t k) {
  return guard([&] {
    GN_CHECK(rows >= 0 && experts >= 0 && k >= 0, "negative extent");
    if (rows == 0 || experts == 0) return;
    check_ptrs(rows * experts, {logits, probs});
    check_ptrs(experts, {bias});
    check_ptrs(rows * k, {selected, weights});
    ThreadCtx& c = ctx();
    float* dl = up(c, "a", logits, rows * experts);
    float* db = up(c, "b", bias, experts);
    float* dp = dev<float>(c, "p", rows * experts);
    launch_softmax_rows(dp, dl, rows, experts, c.stream);
    down(c, probs, dp, rows * experts);
    if (k > 0) {
      int32_t* ds = dev<int32_t>(c, "i", rows * k);
      float* dw = dev<float>(c, "w", rows * k);
      GN_HIP(hipMemcpyAsync(ds, selected, sizeof(int32_t) * rows * k, hipMemcpyHostToDevice, c.stream));
      GN_HIP(hipMemcpyAsync(dw, weights, sizeof(float) * rows * k, hipMemcpyHostToDevice, c.stream));
      uint8_t* taken = dev<uint8_t>(c, "t", rows * experts);
      launch_topk_rows(ds, dl, db, rows, experts, k, taken, c.stream);
      launch_gather_weights(dw, dp, ds, rows, experts, k, c.stream);
      down(c, selected, ds, rows * k);
      down(c, weights, dw, rows * k);
    }
    sync(c);
  });
}
int gn_grouped_matmul_transposed(float* d, const float* in, const float* w, const int32_t* counts,
                                 int64_t experts, int64_t cols, int64_t inner) {
  return guard([&] {
    GN_CHECK(experts >= 0 && cols >= 0 && inner >= 0, "negative extent");
    int64_t rows = 0;
    for (int64_t e = 0; e < experts; e++) {
      GN_CHECK(counts[e] >= 0, "negative token count");
      rows += counts[e];
    }
    if (rows == 0 || cols == 0) return;
    ThreadCtx& c = ctx();
    float* di = up(c, "a", in, rows * inner);
    float* dw = up(c, "b", w, experts * cols * inner);
    float* dd = dev<float>(c, "d", rows * cols);
    int64_t off = 0;
    for (int64_t e = 0; e < experts; e++) {
      if (counts[e] > 0) {
        GemmDesc g = linear_fwd_desc(di + off * inner, dw + e * cols * inner, dd + off * cols,
                                     counts[e], (int)inner, (int)cols);
        gemm(g, c.stream, c.arena.get());
      }
      off += counts[e];
    }
    down(c, d, dd, rows * cols);
    sync(c);
  });
}

// kernels/backend.go:146-152 -----------------------------------------------
int gn_softmax_last_dim(float* d, const float* s, int64_t rows, int64_t cols) {
  return guard([&] {
    GN_CHECK(rows >= 0 && cols >= 0, "negative extent");
    if (rows == 0 || cols == 0) return;
    check_ptrs(rows * cols, {d, s});
    ThreadCtx& c = ctx();
    float* ds = up(c, "a", s, rows * cols);
    float* dd = dev<float>(c, "d", rows * cols);
    launch_softmax_rows(dd, ds, rows, cols, c.stream);
    down(c, d, dd, rows * cols);
    sync(c);
  });
}
int gn_rmsnorm_last_dim(float* d, const float* s, int64_t rows, int64_t cols, float eps) {
  return guard([&] {
    GN_CHECK(rows >= 0 && cols >= 0, "negative extent");
    if (rows == 0 || cols == 0) return;
    check_ptrs(rows * cols, {d, s});
    ThreadCtx& c = ctx();
    float* ds = up(c, "a", s, rows * cols);
    float* dd = dev<float>(c, "d", rows * cols);
    launch_rmsnorm_rows_prim(dd, ds, rows, cols, eps, c.stream);
    down(c, d, dd, rows * cols);
    sync(c);
  });
}

// kernels/backend.go:267-283 -----------------------------------------------
// Scores are computed with the MFMA GEMM, masked and normalized by a row pass,
// and contracted with V by the GEMM again.
int gn_attention_forward(const float* q, const float* k, const float* v, const int32_t* seg,
                         int64_t nseg, int64_t qlen, int64_t klen, int64_t dim, int64_t offset,
                         int64_t window, float* out, float* lse) {
  return guard([&] {
    GN_CHECK(qlen >= 0 && klen >= 0 && dim >= 0, "negative extent");
    GN_CHECK(qlen * klen < (1ll << 31), "attention: score matrix too large");
    if (qlen == 0) return;
    ThreadCtx& c = ctx();
    float* dq = up(c, "q", q, qlen * dim);
    float* dk = up(c, "k", k, klen * dim);
    float* dv = up(c, "v", v, klen * dim);
    int32_t* ds = seg ? up(c, "seg", seg, nseg) : nullptr;
    float* S = dev<float>(c, "S", qlen * klen);
    float* dout = dev<float>(c, "o", qlen * dim);
    float* dl = dev<float>(c, "lse", qlen);
    GemmDesc g;
    g.M = (int)qlen; g.N = (int)klen; g.K = (int)dim;
    g.A = dq; g.lda = dim; g.B = dk; g.ldb = dim; g.C = S; g.ldc = klen;
    gemm(g, c.stream, c.arena.get());
    launch_attn_row_fwd(S, klen, 0, qlen, offset, window, ds, nseg, 0, dl, nullptr, nullptr,
                        c.stream);
    GemmDesc h;
    h.M = (int)qlen; h.N = (int)dim; h.K = (int)klen;
    h.A = S; h.lda = klen; h.B = dv; h.ldb = dim; h.b_kcontig = false; h.C = dout; h.ldc = dim;
    gemm(h, c.stream, c.arena.get());
    down(c, out, dout, qlen * dim);
    if (lse) down(c, lse, dl, qlen);
    sync(c);
  });
}

int gn_attention_forward_split(const float* q, const float* k, const float* v, const int32_t* seg,
                               int64_t nseg, int64_t qlen, int64_t klen, int64_t dim,
                               int64_t offset, int64_t window, int64_t kstart, int64_t kend,
                               float* acc, float* mx, float* sum) {
  return guard([&] {
    GN_CHECK(qlen >= 0 && klen >= 0 && dim >= 0 && kstart >= 0, "negative extent");
    if (kend > klen) kend = klen;
    int64_t range = std::max<int64_t>(kend - kstart, 0);
    if (qlen == 0) return;
    ThreadCtx& c = ctx();
    float* dq = up(c, "q", q, qlen * dim);
    float* dk = up(c, "k", k + kstart * dim, range * dim);
    float* dv = up(c, "v", v + kstart * dim, range * dim);
    int32_t* ds = seg ? up(c, "seg", seg, nseg) : nullptr;
    float* S = dev<float>(c, "S", qlen * std::max<int64_t>(range, 1));
    float* da = dev<float>(c, "o", qlen * dim);
    float* dm = dev<float>(c, "m", qlen);
    float* dsum = dev<float>(c, "s", qlen);
    GemmDesc g;
    g.M = (int)qlen; g.N = (int)range; g.K = (int)dim;
    g.A = dq; g.lda = dim; g.B = dk; g.ldb = dim; g.C = S; g.ldc = range;
    gemm(g, c.stream, c.arena.get());
    launch_attn_row_fwd(S, range, kstart, qlen, offset, window, ds, nseg, 1, nullptr, dm, dsum,
                        c.stream);
    GemmDesc h;
    h.M = (int)qlen; h.N = (int)dim; h.K = (int)range;
    h.A = S; h.lda = range; h.B = dv; h.ldb = dim; h.b_kcontig = false; h.C = da; h.ldc = dim;
    gemm(h, c.stream, c.arena.get());
    down(c, acc, da, qlen * dim);
    down(c, mx, dm, qlen);
    down(c, sum, dsum, qlen);
    sync(c);
  });
}

int gn_attention_combine(const float* const* accs, const float* const* mxs, const float* const* sums,
                         int64_t parts, int64_t qlen, int64_t dim, float* out, float* lse) {
  return guard([&] {
    GN_CHECK(parts >= 0 && qlen >= 0 && dim >= 0, "negative extent");
    if (qlen == 0) return;
    ThreadCtx& c = ctx();
    std::vector<const float*> pa(parts), pm(parts), ps(parts);
    float* buf = dev<float>(c, "parts", parts * (qlen * dim + 2 * qlen));
    for (int64_t p = 0; p < parts; p++) {
      float* a = buf + p * (qlen * dim + 2 * qlen);
      GN_HIP(hipMemcpyAsync(a, accs[p], sizeof(float) * qlen * dim, hipMemcpyHostToDevice, c.stream));
      GN_HIP(hipMemcpyAsync(a + qlen * dim, mxs[p], sizeof(float) * qlen, hipMemcpyHostToDevice, c.stream));
      GN_HIP(hipMemcpyAsync(a + qlen * dim + qlen, sums[p], sizeof(float) * qlen, hipMemcpyHostToDevice, c.stream));
      pa[p] = a; pm[p] = a + qlen * dim; ps[p] = a + qlen * dim + qlen;
    }
    const float** tab = dev<const float*>(c, "tab", 3 * parts);
    std::vector<const float*> all;
    all.insert(all.end(), pa.begin(), pa.end());
    all.insert(all.end(), pm.begin(), pm.end());
    all.insert(all.end(), ps.begin(), ps.end());
    if (parts > 0)
      GN_HIP(hipMemcpyAsync(tab, all.data(), sizeof(float*) * 3 * parts, hipMemcpyHostToDevice, c.stream));
    float* dout = dev<float>(c, "o", qlen * dim);
    float* dl = dev<float>(c, "lse", qlen);
    launch_attn_combine(tab, tab + parts, tab + 2 * parts, parts, qlen, dim, dout, dl, c.stream);
    down(c, out, dout, qlen * dim);
    if (lse) down(c, lse, dl, qlen);
    sync(c);
  });
}

int gn_attention_backward(const float* q, const float* k, const float* v, const float* o,
                          const float* dout, const float* lse, const float* corr, const int32_t* seg,
                          int64_t nseg, int64_t qlen, int64_t klen, int64_t dim, int64_t offset,
                          int64_t window, float* dq, float* dk, float* dv) {
  (void)o;
  return guard([&] {
    GN_CHECK(qlen >= 0 && klen >= 0 && dim >= 0, "negative extent");
    GN_CHECK(qlen * klen < (1ll << 31), "attention: score matrix too large");
    if (qlen == 0 || klen == 0) return;
    ThreadCtx& c = ctx();
    float* Q = up(c, "q", q, qlen * dim);
    float* K = up(c, "k", k, klen * dim);
    float* V = up(c, "v", v, klen * dim);
    float* dO = up(c, "do", dout, qlen * dim);
    float* L = up(c, "lse", lse, qlen);
    float* Cr = corr ? up(c, "corr", corr, qlen) : nullptr;
    int32_t* ds = seg ? up(c, "seg", seg, nseg) : nullptr;
    float* dQ = up(c, "dq", dq, qlen * dim);
    float* dK = up(c, "dk", dk, klen * dim);
    float* dV = up(c, "dv", dv, klen * dim);
    float* S = dev<float>(c, "S", qlen * klen);
    float* dP = dev<float>(c, "dP", qlen * klen);
    GemmDesc g;  // S = Q K^T
    g.M = (int)qlen; g.N = (int)klen; g.K = (int)dim;
    g.A = Q; g.lda = dim; g.B = K; g.ldb = dim; g.C = S; g.ldc = klen;
    gemm(g, c.stream, c.arena.get());
    GemmDesc h = g;  // dP = dO V^T
    h.A = dO; h.B = V; h.C = dP;
    gemm(h, c.stream, c.arena.get());
    launch_attn_row_bwd(S, dP, qlen, klen, offset, window, ds, nseg, L, Cr, c.stream);
    GemmDesc gv;  // dV += P^T dO
    gv.M = (int)klen; gv.N = (int)dim; gv.K = (int)qlen;
    gv.A = S; gv.lda = klen; gv.a_kcontig = false;
    gv.B = dO; gv.ldb = dim; gv.b_kcontig = false;
    gv.C = dV; gv.ldc = dim; gv.epi = EPI_ACCUM;
    gemm(gv, c.stream, c.arena.get());
    GemmDesc gk = gv;  // dK += dS^T Q
    gk.A = dP; gk.B = Q; gk.C = dK;
    gemm(gk, c.stream, c.arena.get());
    GemmDesc gq;  // dQ += dS K
    gq.M = (int)qlen; gq.N = (int)dim; gq.K = (int)klen;
    gq.A = dP; gq.lda = klen; gq.B = K; gq.ldb = dim; gq.b_kcontig = false;
    gq.C = dQ; gq.ldc = dim; gq.epi = EPI_ACCUM;
    gemm(gq, c.stream, c.arena.get());
    down(c, dq, dQ, qlen * dim);
    down(c, dk, dK, klen * dim);
    down(c, dv, dV, klen * dim);
    sync(c);
  });
}

}  // extern "C"
