// gn_model.h - launchers of the transformer kernels used by the session.
#pragma once

#include "gn_kernels.h"

namespace gn {

// ---- embedding / norms --------------------------------------------------
void launch_embed_smear(const int32_t* ids, const float* wte, const float* wsg, const float* lam,
                        int B, int T, int C, float* raw, float* embn, float* smsig, float* x,
                        hipStream_t st);
void launch_embed_decode(const int32_t* tok, const float* wte, const float* wsg, const float* lam,
                         int rows, int C, float* prev, float* x, float* x0, hipStream_t st);
void launch_resid_norm(const float* xin, const float* x0, const float* lr, const float* l0,
                       int layer, int64_t rows, int C, float* xb, float* h, hipStream_t st);
void launch_norm_rows(const float* x, const float* back, const float* lam, int64_t rows, int C,
                      float* pre, float* y, hipStream_t st);

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
  int nsplit_max;      // set by the launcher: grid.y and the split stride of part
};
void launch_decode_attention(DecodeAttnArgs a, hipStream_t st);

struct FlashArgs {
  const float* q;  // [B*T, Hq, 128]
  const float* k;  // [B*T, Hkv, 128]
  const float* v;
  float* o;        // [B*T, Hq, 128]
  float* lse;      // [B*T, Hq] or null
  int B, T, Hq, Hkv, window;
};
void launch_flash_fwd(const FlashArgs& a, hipStream_t st);

struct FlashBwdArgs {
  const float* q;
  const float* k;
  const float* v;
  const float* o;
  const float* dout;
  const float* lse;
  float* delta;  // [B*T, Hq] scratch
  float* dq;     // [B*T, Hq, 128] (overwritten)
  float* dk;     // [B*T, Hkv, 128] (overwritten)
  float* dv;
  int B, T, Hq, Hkv, window;
};
void launch_flash_bwd(const FlashBwdArgs& a, hipStream_t st);

// ---- loss ----------------------------------------------------------------
void launch_pg_loss_rows(float* z, int64_t ldz, int V, int64_t row0, int64_t rows,
                         const int32_t* targets, const float* adv, int T, float norm, float* nll,
                         double* loss_rows, hipStream_t st);
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
  float* gve;
};
void launch_qkv_post_bwd(const QkvPostBwdArgs& a, int64_t rows, hipStream_t st);
void launch_ve_gate_bwd(const float* dpre, const float* h, const float* W, int C, int Hkv,
                        int64_t N, float* dW, float* dh, double* part, hipStream_t st);
void launch_smear_bwd(const float* ga, const float* embn, const float* smsig, const float* lam,
                      const float* wsg, int B, int T, int C, float* ge, float* ggate,
                      double* lam_rows, double* part, float* dwsg, float* dlam, hipStream_t st);
void launch_embed_scatter(const float* g, const int32_t* ids, int C, int64_t N, float* gw,
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
};
// Largest number of key splits a decode step with this window and cache
// length can use (sizes MlaDecodeArgs::part).
int mla_decode_max_splits(int window, int maxSeq);
void launch_mla_decode(MlaDecodeArgs a, hipStream_t st);
void launch_replicate_rows(const float* src, float* dst, int G, int S, int P, int W, int maxSrc,
                           int maxDst, hipStream_t st);

// ---- latent preset: DeepSeekMoE (model/moe.go) ---------------------------
void launch_swiglu_rows(const float* gu, int F, int64_t rows, float clamp, float* act,
                        hipStream_t st);
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
  float* xg;        // [rows*K, C]
};
void launch_moe_route(const MoeRouteArgs& a, hipStream_t st);
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
};
void launch_moe_combine(const MoeCombineArgs& a, int64_t rows, hipStream_t st);

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
};
void launch_sampler(const SamplerArgs& a, hipStream_t st);

}  // namespace gn
