// gn_model.h - launchers of the transformer kernels used by the session.
#pragma once

#include "gn_kernels.h"

namespace gn {

static constexpr float NORM_EPS = 1e-6f;  // model/attention.go:11
static constexpr float QK_SCALE = 1.2f;   // model/attention.go:14
static constexpr int VE_CH = 12;          // model/attention.go:18
static constexpr float VE_SCALE = 3.f;    // model/attention.go:21
__device__ __forceinline__ float sigmoidf_(float x) { return 1.f / (1.f + expf(-x)); }

// ---- embedding / norms --------------------------------------------------
void launch_embed_smear(const int32_t* ids, const float* wte, const float* wsg, const float* lam,
                        int B, int T, int C, float* raw, float* embn, float* smsig, float* x,
                        hipStream_t st, const float* seed_prev = nullptr,
                        float* seedsig = nullptr);
// A batch of strided copies in one launch: block `d` copies outer x inner
// rows of `count` floats, row (o, i) at src + o*s_outer + i*s_inner to
// dst + o*d_outer + i*d_inner.  The descriptors live in device memory.
struct CopyBlock {
  const float* src;
  float* dst;
  int64_t count, s_outer, s_inner, d_outer, d_inner;
  int32_t outer, inner;
};
void launch_copy_blocks(const CopyBlock* descs, int n, hipStream_t st);
// ovr (nullable): per row, a token fed instead of tok's (>= 0) or -1; the
// fed token is written back to tok.
void launch_embed_decode(int32_t* tok, const float* wte, const float* wsg, const float* lam,
                         int rows, int C, float* prev, float* x, float* x0, hipStream_t st,
                         const int32_t* ovr = nullptr);
// launch_embed_decode followed by layer 0's residual mix and norm
// (launch_resid_norm with no pending sum) in one launch: x0 = the embedding,
// x = the mixed row, h = its norm.
void launch_embed_decode_mix(int32_t* tok, const float* wte, const float* wsg, const float* lam,
                             const float* lr, const float* l0, int rows, int C, float* prev,
                             float* x, float* x0, float* h, hipStream_t st,
                             const int32_t* ovr = nullptr);
// xin (resp. x) may be the target of a residual-add GEMM whose split-K sum
// was deferred (pend): the kernels then read xin + sum, and norm_rows
// writes that value back to x.  resid_norm writes it (xin + sum, before the
// residual mix) to xs when xs is given.
void launch_resid_norm(const float* xin, const float* x0, const float* lr, const float* l0,
                       int layer, int64_t rows, int C, float* xb, float* h, hipStream_t st,
                       const PendingSum& pend = PendingSum{}, float* xs = nullptr);
void launch_norm_rows(float* x, const float* back, const float* lam, int64_t rows, int C,
                      float* pre, float* y, hipStream_t st, const PendingSum& pend = PendingSum{});

// ---- q/k/v post-processing ----------------------------------------------
struct QkvPostArgs {
  const float* qkv;
  const float* h;
  const int32_t* ids;
  const float* ve;
  const float* wve;
  const float* cosT;
  const float* sinT;
  int C, Hq, Hkv, R, T;
  int pos0;
  const int* pos_dev;  // when set, pos0 is read from the device instead
  float* qn;
  float* kn;
  float* vout;
  float* qrot;
  float* krot;
  float* vesig;
  float* kcache;
  float* vcache;
  int maxSeq;
  int rows_per_seq;
  PendingSum qkv_sum;  // qkv is a deferred split-K product (its partials)
};
void launch_qkv_post(const QkvPostArgs& a, int64_t rows, hipStream_t st);
void launch_replicate_kv(const float* src, float* dst, int G, int S, int Hkv, int P, int maxSrc,
                         int maxDst, hipStream_t st);
void launch_expand_last_rows(const float* src, float* dst, int G, int T, int S, int C,
                             hipStream_t st);

// ---- attention -----------------------------------------------------------
struct DecodeAttnArgs {
  const float* q;   // [rows, Hq, 128]
  const float* kc;  // layer base of the K cache [rows][Hkv][maxSeq][128]
  const float* vc;
  float* part;      // [rows*Hkv][nsplit][Hq/Hkv][130]
  float* o;         // [rows, Hq, 128]
  int rows, Hq, Hkv, maxSeq;
  int kstart, kend;    // keys [kstart, kend) when pos_dev is null; else
  const int* pos_dev;  // the query position is *pos_dev (read on the device,
  int window;          // so a captured graph serves every step) and the keys
                       // are [max(0, pos - window), pos]
  // Compressed attention (ratio > 1): the keys are the compressed blocks
  // [0, pos / ratio) of ck/cv ([rows][Hkv][maxBlocks][128]) followed, when
  // window > 0, by the raw keys [max(0, pos - window), pos] of kc/vc: one
  // softmax over both, which is the log-sum-exp merge of the global and
  // local branches (model/compress_attention.go:440-484, 543-560).  With
  // neither (pos < ratio, no window) the output is zero.  kend - 1 is the
  // query position of eager launches.
  const float* ck = nullptr;
  const float* cv = nullptr;
  int maxBlocks = 0;
  int ratio = 0;
  // sparse selection (ratio > 1): the compressed keys are only the selected
  // blocks sel[(row*Hkv + hk)*kcap + j], j < nsel[row*Hkv + hk] (<= 256)
  const int* sel = nullptr;
  const int* nsel = nullptr;
  int kcap = 0;
  int nsplit_max;      // set by the launcher: grid.y and the split stride of part
  int split_keys = 0;  // set by the launcher: most keys per split of a plain window
  int64_t part_floats = 0;  // capacity of part in floats; the launcher rejects a
                            // grid whose split layout would not fit
  // optional events recorded by the dispatch itself (hipExtLaunchKernelGGL):
  // t_start when the attention kernel starts, t_stop when the last kernel of
  // the call (the combine, when launched) ends -- the calls' own duration
  hipEvent_t t_start = nullptr, t_stop = nullptr;
  // Fused q/k/v post-processing (plain windows, one token per row): with
  // fuse_post set, q is not read from `q`.  Each block computes its R query
  // heads and its kv head from post.qkv (or the pending split-K partials
  // post.qkv_sum) exactly as qkv_post_kernel does -- VE gate on v, RoPE on
  // the trailing post.R dims, 1.2 * RMSNorm per head -- the block whose
  // split holds the query position writes the new key and value to kc/vc,
  // and the new key/value enter the block's scores and P.V from its own
  // copy.  Read: post.{qkv | qkv_sum}, h, ids, ve, wve, cosT, sinT, C, R.
  bool fuse_post = false;
  QkvPostArgs post{};
};
// Most split-K partials of the q/k/v product a fused launch sums.
constexpr int DECODE_POST_MAX_SPLITS = 4;
// Split capacity a part buffer needs for launches with these arguments
// (window, maxSeq, ratio, maxBlocks).
int decode_attention_split_cap(const DecodeAttnArgs& a);
void launch_decode_attention(DecodeAttnArgs a, hipStream_t st);

// Key masks of the flash kernels.  ratio <= 1: causal with a sliding window
// (key j visible from query t when j <= t and t - j <= window, window < 0:
// none).  ratio > 1: the keys are compressed blocks of `ratio` positions and
// query t (at position qoff + t) sees the blocks that ended before its own,
// j < (qoff + t) / ratio (model/compress_attention.go:562-677); a query with
// no visible key gets a zero output and log-sum-exp -inf.
struct FlashArgs {
  const float* q;  // [B*T, Hq, 128]
  const float* k;  // [B*Tk, Hkv, 128]
  const float* v;
  float* o;        // [B*T, Hq, 128]
  float* lse;      // [B*T, Hq] or null
  int B, T, Hq, Hkv, window;
  int Tk = 0;      // keys per sequence (0: T)
  int ratio = 0;
  int qoff = 0;    // compressed keys: position of the first query
};
void launch_flash_fwd(FlashArgs a, hipStream_t st);

struct FlashBwdArgs {
  const float* q;
  const float* k;
  const float* v;
  const float* o;
  const float* dout;
  const float* lse;
  float* delta;  // [B*T, Hq]: rowsum(dO * O), computed here unless delta_ready
  float* dq;     // [B*T, Hq, 128] (overwritten, or accumulated with dq_accum)
  float* dk;     // [B*Tk, Hkv, 128] (overwritten)
  float* dv;
  int B, T, Hq, Hkv, window;
  int Tk = 0;
  int ratio = 0;
  int qoff = 0;
  bool delta_ready = false;  // branches of a merged softmax share the merged
  bool dq_accum = false;     // log-sum-exp and row correction dO . O_merged
};
void launch_flash_bwd(FlashBwdArgs a, hipStream_t st);
// delta[r] = dO[r, :] . O[r, :] over rows of 128
void launch_row_dot(const float* o, const float* dout, float* delta, int64_t rows, hipStream_t st);

// ---- loss ----------------------------------------------------------------
// Loss rows of one logits chunk: chunk row r is batch row rowmap[row0 + r]
// (rowmap null: row0 + r); loss_rows is indexed by row0 + r.
void launch_distill_rows(float* z, const float* zt, int64_t ldz, int V, int64_t row0, int64_t rows,
                         const int32_t* rowmap, const int32_t* targets, double tau, float scale,
                         double* loss_rows, hipStream_t st);
void launch_pg_loss_rows(float* z, int64_t ldz, int V, int64_t row0, int64_t rows,
                         const int32_t* rowmap, const int32_t* targets, const float* adv, int T,
                         float norm, float* nll, double* loss_rows, hipStream_t st);
// dst[i] = src[idx[i]] / dst[idx[i]] = src[i] for rows of C floats, i < n
void launch_gather_rows(const float* src, const int32_t* idx, float* dst, int64_t n, int C,
                        hipStream_t st);
void launch_scatter_rows(const float* src, const int32_t* idx, float* dst, int64_t n, int C,
                         hipStream_t st);
void launch_sum_f64(const double* v, int64_t n, double* out, bool accumulate, hipStream_t st);

// ---- backward helpers -----------------------------------------------------
void launch_rmsnorm_bwd(const float* x, const float* g, const float* extra, int64_t rows, int C,
                        float* out, hipStream_t st);
void launch_dot_into_grad(const float* a, const float* b0, const float* b1, float sign, int64_t n,
                          float* dst0, float* dst1, double* part, hipStream_t st);
void launch_resid_bwd(const float* gb, const float* lr, const float* l0, int layer, float* gnext,
                      float* gx0, int64_t n, hipStream_t st);
void launch_axpy(float* out, const float* a, const float* b, const float* neg_scale_ptr, float s,
                 int64_t n, hipStream_t st);

struct QkvPostBwdArgs {
  const float* dqn;
  const float* dkn;
  const float* dv;
  const float* qrot;
  const float* krot;
  const float* vesig;
  const float* ve;
  const int32_t* ids;
  const float* cosT;
  const float* sinT;
  int Hq, Hkv, R, T;
  float* dqkv;
  float* dpre;
  float* gve_rows;  // [rows][Hkv*128] the value-embedding gradient of each token's row
};
void launch_qkv_post_bwd(const QkvPostBwdArgs& a, int64_t rows, hipStream_t st);
void launch_ve_gate_bwd(const float* dpre, const float* h, const float* W, int C, int Hkv,
                        int64_t N, float* dW, float* dh, double* part, hipStream_t st);
void launch_smear_bwd(const float* ga, const float* embn, const float* smsig, const float* lam,
                      const float* wsg, int B, int T, int C, float* ge, float* ggate,
                      double* lam_rows, double* part, float* dwsg, float* dlam, hipStream_t st);
// A batch's tokens grouped by id (host-built, on the device): perm lists
// token indices, ascending within each id; id u (of n_ids, ascending) owns
// perm[off[u] .. off[u+1]) and is uid[u].
struct TokenGroups {
  const int32_t* perm = nullptr;
  const int32_t* off = nullptr;
  const int32_t* uid = nullptr;
  int n_ids = 0;
};
// gw[id] += the rows g[n] of the tokens with that id, added in token order
// (embedding and value-embedding backward).
void launch_rows_scatter(const float* g, const TokenGroups& ids, int C, float* gw,
                         hipStream_t st);

// ---- latent preset: MLA (model/mla.go) ------------------------------------
// xa rows are [q_lat (lat) | kv_lat (lat) | q_rope (Hq*rd) | k_rope (Hkv*rd)]
// (one GEMM of h against the stacked QueryDown, KVDown, QueryRope, KeyRope);
// kvu rows are [k_content (Hkv*cd) | v (Hkv*128)] (KeyUp and ValueUp on
// kv_lat); cd = 128 - rd.
struct MlaAssembleArgs {
  const float* xa;
  int xw;
  const float* qc;  // [N, Hq*cd] = QueryUp . q_lat
  const float* kvu;
  const float* cosT;
  const float* sinT;
  int Hq, Hkv, lat, rd, T, pos0;
  float* q;  // [N, Hq, 128]
  float* k;  // [N, Hkv, 128]
  float* v;
  float* lat_cache;  // prefill: [B][maxSeq][lat] (or null)
  float* rk_cache;   // prefill: [B][maxSeq][Hkv*rd]
  int maxSeq;
};
void launch_mla_assemble(const MlaAssembleArgs& a, int64_t rows, hipStream_t st);

struct MlaPostBwdArgs {
  const float* dq;  // [N, Hq, 128]
  const float* dk;  // [N, Hkv, 128]
  const float* dv;
  const float* cosT;
  const float* sinT;
  int Hq, Hkv, lat, rd, T, xw;
  float* dqc;   // [N, Hq*cd]
  float* dxa;   // rotary parts written: [N, xw] columns 2*lat ..
  float* dkvu;  // [N, Hkv*(cd+128)]
};
void launch_mla_post_bwd(const MlaPostBwdArgs& a, int64_t rows, hipStream_t st);

struct MlaDecodeArgs {
  const float* xa;    // [rows, xw]
  int xw;
  // a deferred input projection: the prep kernel writes its sum into xa_w
  // (== xa) before anything reads xa
  PendingSum xa_sum;
  float* xa_w = nullptr;
  const float* qabs;  // [rows, Hq, lat] absorbed content queries
  float* qrope;       // [rows, Hq, rd] (written by the prep kernel)
  float* lat_cache;   // layer base [rows][maxSeq][lat]
  float* rk_cache;    // layer base [rows][maxSeq][Hkv*rd]
  const float* cosT;
  const float* sinT;
  float* out;         // [rows, Hq, lat] attention-weighted latents
  float* part;        // [rows][nsplit_max][Hq][lat + 2] split partials
  int rows, Hq, Hkv, lat, rd, maxSeq, window;
  int pos;            // query position (eager launches)
  const int* pos_dev; // when set, the position is read on the device
  int part_splits;    // splits the part buffer holds per row
  int nsplit_max;     // set by the launcher
  // optional events recorded by the dispatch (hipExtLaunchKernelGGL): at the
  // start of the attention kernel and the end of the call's last kernel
  hipEvent_t t_start = nullptr, t_stop = nullptr;
};
// Largest number of key splits a decode step with this window and cache
// length can use (sizes MlaDecodeArgs::part).
int mla_decode_max_splits(int window, int maxSeq);
// Rotates the new token's query/key rotary parts and appends (latent,
// rotary key) to the caches; runs before the absorbed-query product.
void launch_mla_decode_prep(const MlaDecodeArgs& a, hipStream_t st);
// Absorbed attention over the caches (+ the split combine).
void launch_mla_decode(MlaDecodeArgs a, hipStream_t st);
void launch_replicate_rows(const float* src, float* dst, int G, int S, int P, int W, int maxSrc,
                           int maxDst, hipStream_t st);

// ---- latent preset: DeepSeekMoE (model/moe.go) ---------------------------
void launch_swiglu_rows(const float* gu, int F, int64_t rows, float clamp, float* act,
                        hipStream_t st, const PendingSum& pend = PendingSum{});
void launch_swiglu_rows_bwd(const float* gu, const float* dact, int F, int64_t rows, float clamp,
                            float* dgu, hipStream_t st);

struct MoeRouteArgs {
  const float* logits;  // [rows, E] router logits
  const float* bias;    // [E] router correction bias
  const float* x;       // [rows, C] MoE input (gathered into xg)
  int64_t rows;
  int E, K, C;
  float* probs;     // [rows, E]
  int32_t* sel;     // [rows*K]
  float* w;         // [rows*K]
  int* blockcnt;    // [ceil(rows*K/256)][E] scratch
  int* off;         // [E+1] expert offsets into the gathered rows
  int* perm_row;    // [rows*K] gathered pair -> token
  float* perm_w;    // [rows*K] gathered pair -> router weight
  int* inv;         // [rows*K] (token, slot) -> gathered pair
  float* xg;        // [rows*K, C]; null: no gathered copy (the decode expert kernels read x)
  PendingSum logits_sum;  // a deferred router product (then `logits` is unused)
  const float* wr = nullptr;  // [E, C] router weights: logits computed from x in the gate kernel
};
void launch_moe_route(const MoeRouteArgs& a, hipStream_t st);
// MoE.forwardTraining's load counts (moe.go:192-193): load[e] += the tokens
// the routing placed with expert e (off[e + 1] - off[e]).
void launch_moe_load_accum(const int* off, int E, double* load, hipStream_t st);
// MoE.updateRouterBias (moe.go:330-341): bias[e] += speed * sign(mean - load[e])
// over one layer's counts, which are then cleared; no change while no token
// was counted.
void launch_moe_bias_update(double* load, float* bias, int E, float speed, hipStream_t st);
struct MoePlaceArgs {
  const int32_t* sel;
  const float* w;
  const float* x;
  const int* off;
  const int* blockoff;
  int64_t npairs;
  int K, E, C;
  int* perm_row;
  float* perm_w;
  int* inv;
  float* xg;
};

struct MoeCombineArgs {
  const float* mid;     // residual stream after attention
  const float* shared;  // shared-expert output
  const float* yg;      // [rows*K, C] expert outputs (gathered order)
  const float* perm_w;
  const int32_t* sel;
  const int* inv;
  float scale;
  int K, C;
  float* out;
  PendingSum shared_sum;  // a deferred shared-expert product (then `shared` is unused)
};
void launch_moe_combine(const MoeCombineArgs& a, int64_t rows, hipStream_t st);

// Expert products over decode-size groups (a few to tens of pairs per
// expert): gate and up with the clamped SwiGLU fused (x: token rows read
// through perm_row; w0 = gate, w1 = up weights [E][N][K]; out = SwiGLU
// [pairs][N]), or down (x: SwiGLU rows in pair order; w0 = down weights
// [E][N][K]; w1 = null; out [pairs][N]).  Returns false (nothing launched)
// for shapes it does not take (N % 16, K % 64, K / 64 outside 1..16).
struct MoeExpertArgs {
  const float* x;
  const int* perm_row;  // gate/up only
  const int* off;       // [E + 1] pair offsets of the experts (device)
  const float* w0;
  const float* w1;
  float* out;
  int E, N, K;
  float clamp;
  int64_t pairs = 0;  // token-expert pairs of the call (chooses the chunk size)
};
bool launch_moe_expert_small(const MoeExpertArgs& a, hipStream_t st);
bool moe_expert_small_supported(int N, int K);

void launch_moe_bwd_prep(const float* g, const float* yg, const int* perm_row, const float* perm_w,
                         float scale, int64_t npairs, int C, float* gy, double* dotp,
                         hipStream_t st);
void launch_moe_balance(const float* probs, const int32_t* sel, int S, int T, int E, int K,
                        float* cnt, double* loss_seq, hipStream_t st);
struct MoeRouterBwdArgs {
  const float* probs;
  const int32_t* sel;
  const int* inv;
  const double* dotp;
  const float* bal_cnt;  // [S][E] or null
  double bal_coef;       // weight / (S T) * E / (K T)
  int64_t rows;
  int E, K, T;
  float* glog;           // [rows, E]
};
void launch_moe_router_bwd(const MoeRouterBwdArgs& a, hipStream_t st);
struct MoeBwdCombineArgs {
  const float* dshared;
  const float* dxg;
  const float* drouter;
  const int32_t* sel;
  const int* inv;
  int K, C;
  float* out;
};
void launch_moe_bwd_combine(const MoeBwdCombineArgs& a, int64_t rows, hipStream_t st);

// ---- flash preset: compressed attention (model/compress*.go) --------------
bool hca_ratio_supported(int ratio);
struct HcaCompressArgs {
  const float* clog;  // [B*T, 128] h . Wl^T (the bias is added here)
  const float* bias;  // [ratio, 128]
  const float* k;     // [B*T, Hkv, 128] keys after norm and rotary
  const float* v;     // [B*T, Hkv, 128]
  int B, T, Hkv, ratio;
  float* probs;       // [B*blocks][ratio][128] softmax weights (saved for the backward)
  float* kc;          // [B*blocks, Hkv, 128] compressed keys
  float* vc;
  // prefill (optional): compressed keys/values of the complete blocks as a
  // cache [B][Hkv][T / ratio][128], and the logits of an incomplete last
  // block into its ring [B][ratio][128] (slot = position % ratio)
  float* ck_pf = nullptr;
  float* cv_pf = nullptr;
  float* ring_pf = nullptr;
  float* tailk_pf = nullptr;  // [B][Hkv][ratio][128] keys/values of that block
  float* tailv_pf = nullptr;
};
void launch_hca_compress(const HcaCompressArgs& a, hipStream_t st);
void launch_merge_branches(const float* oa, const float* la, const float* ob, const float* lb,
                           float* out, float* lse, int64_t rows, hipStream_t st);
struct HcaCompressBwdArgs {
  const float* probs;
  const float* k;
  const float* v;
  const float* kc;
  const float* vc;
  const float* dkc;  // [B*blocks, Hkv, 128] gradients of the compressed keys/values
  const float* dvc;
  int B, T, Hkv, ratio;
  float* glog;       // [B*T, 128] logit gradient (overwritten)
  float* dk;         // [B*T, Hkv, 128] accumulated
  float* dv;
  float* gbias;      // [ratio, 128] accumulated
  float* bias_part;  // hca_bias_part_floats(ratio) scratch
};
size_t hca_bias_part_floats(int ratio);
void launch_hca_compress_bwd(const HcaCompressBwdArgs& a, hipStream_t st);
struct HcaDecodeArgs {
  const float* clog;  // [rows, 128] this token's h . Wl^T
  const float* bias;
  float* ring;        // [rows][ratio][128] logits of the current block
  const float* kc;    // layer base of the raw caches [rows][Hkv][maxSeq][128]
  const float* vc;
  // tail mode (CED decoder layers, whose compressed keys/values are not the
  // raw cache rows): knew/vnew [rows][Hkv][128] enter tail slots
  // [rows][Hkv][ratio][128] and complete blocks compress from there
  const float* knew = nullptr;
  const float* vnew = nullptr;
  float* tailk = nullptr;
  float* tailv = nullptr;
  float* ck;          // layer base of the compressed caches [rows][Hkv][maxBlocks][128]
  float* cv;
  int rows, Hkv, ratio, maxSeq, maxBlocks;
  int pos;             // position of this token (eager launches)
  const int* pos_dev;  // when set, read on the device
};
void launch_hca_decode_compress(const HcaDecodeArgs& a, hipStream_t st);
// The indexer key of a block completed at this step (pos % ratio == ratio - 1):
// ik[row][blk][hk][:] = ck[row][hk][blk][:] . Wik^T, blk = pos / ratio;
// ck layer base [rows][Hkv][maxBlocks][128], ik [rows][maxBlocks][Hkv][HI].
void launch_indexer_key_step(const float* ck, const float* wik, float* ik, int rows, int Hkv,
                             int maxBlocks, int HI, int ratio, int pos, const int* pos_dev,
                             hipStream_t st);

// ---- flash preset: sparse compressed attention (model/indexer.go) ---------
// A chunk of sequences [b0, b0 + chunk) of one layer: rows (z, t) with
// z = (b - b0) * Hkv + hk; row t may select compressed blocks
// s < min(blocks, (qoff + t) / ratio).
struct CsaShape {
  int T, blocks, Hkv, ratio, qoff, b0;
  int ldo;      // row stride of the chunk's score-like matrices (>= blocks)
  int H, dim;   // indexer heads and head dim
  const int* qoff_dev = nullptr;  // decode: qoff read on the device
};
struct IndexerScoreArgs {
  CsaShape shape;
  const float* iq;  // [B*T][H*dim] indexer queries
  const float* ik;  // [B*blocks][Hkv][H*dim] indexer keys of the compressed blocks
  const float* w;   // [H] head weights
  float* out;       // forward: chunk scores [chunk*Hkv][T][ldo]
  // backward (mask_out set): per-head masks [H][chunk*Hkv][T][ldo] (stride
  // mask_stride between heads) from the row gradient gs, and per-block
  // partials of the head-weight gradient [H][indexer_mask_blocks()]
  const float* gs;
  float* mask_out;
  int64_t mask_stride;
  float* gw_blocks;
};
void launch_indexer_scores(const IndexerScoreArgs& a, int chunk_seqs, hipStream_t st);
int64_t indexer_mask_blocks(const CsaShape& s, int chunk_seqs);

struct CsaSelectArgs {
  CsaShape shape;
  int chunk_seqs;
  const float* scores;    // chunk scores
  int K, pool, gpt, ccap; // top-k, group size, groups kept, candidate capacity
  const int* pool_in;     // Reindex: the producer's candidates [B*Hkv][T][ccap] (or null)
  const int* npool_in;
  int* sel;               // [B*Hkv][T][K]
  int* nsel;              // [B*Hkv][T]
  int* pool_out;          // Full with pool > 1: candidates published, or null
  int* npool_out;
  int groups_cap, wave_floats;  // set by the launcher
  // 0: one block of 8 waves per row when the rows are few (decode), one wave
  // per row otherwise; 1: one wave per row; 2: one block per row where the
  // shapes allow.  Same selection either way.
  int mode;
};
void launch_csa_select(CsaSelectArgs a, hipStream_t st);

struct CsaAttnArgs {
  const float* q;   // [B*T, Hq, 128]
  const float* kc;  // [B*blocks, Hkv, 128]
  const float* vc;
  const int* sel;   // [B*Hkv][T][K]
  const int* nsel;
  int B, T, blocks, Hq, Hkv, K;
  float* o;         // forward: [B*T, Hq, 128] and lse [B*T, Hq]
  float* lse;
  const float* dout;   // backward: with the merged lse and delta (dO . O)
  const float* delta;
  float* dq;           // overwritten
  float* dkc;          // accumulated (atomics)
  float* dvc;
};
void launch_csa_attn_fwd(const CsaAttnArgs& a, hipStream_t st);
void launch_csa_attn_bwd(const CsaAttnArgs& a, hipStream_t st);
void launch_query_group_sum(const float* q, int Hq, int Hkv, int64_t N, float* out,
                            hipStream_t st);
struct CsaDistillArgs {
  CsaShape shape;
  const float* scores;  // chunk indexer scores
  const float* tlog;    // chunk mean main-attention logits
  const int* pool_in;   // Reindex restriction (or null)
  const int* npool_in;
  int ccap;
  float weight;
  float* gs;            // chunk (softmax(I) - target) * weight
};
void launch_csa_distill(const CsaDistillArgs& a, int chunk_seqs, hipStream_t st);
void launch_sum_partials(const float* part, int64_t n, float* out, hipStream_t st);

// ---- sampler (inference/sampler.go + tensors/random.go) -------------------
struct SamplerArgs {
  const float* logits;          // [rows, V]
  int64_t ldl;
  int rows, V;
  int samples_per_group;        // S: row r is index r % S of group r / S
  const uint64_t* base_states;  // [groups][2] {hi, lo}: each group's stream before this call
  float temperature;
  int top_k;
  int32_t* out;                 // [rows]
  // logits holds lm_head products y: the logits are softcap15(y), applied on
  // load (transformer.go:538-541); 0: logits holds the logits themselves
  int softcap = 0;
};
void launch_sampler(const SamplerArgs& a, hipStream_t st);
// Neighbouring floats (in increasing order) whose softcap15 decreases, over
// all 2^32 bit patterns but NaNs: 0 when softcap15 is non-decreasing, which
// the sampler's selection on raw lm_head products assumes.
uint64_t count_softcap_order_violations();
// Advances the Go PCG state {hi, lo} by n draws (tensors.RNG after n Float32
// calls, tensors/random.go:66-78).
void advance_rng_state(uint64_t* state, uint64_t n);

}  // namespace gn
