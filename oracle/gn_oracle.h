/*
 * gn_oracle.h - CPU restatement of gonano's RL-step arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (libgnhip.so, the
 * gonano_amd package) may link, load or call this code; only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg use it, and only
 * as the checker.
 *
 * Every function states the reference file:line it restates
 * (paths relative to the gonano source tree).  Floating-point formulas keep
 * the reference's float32 data and its float64 accumulations.
 */
#ifndef GN_ORACLE_H
#define GN_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------------- */
/* kernels.Backend restated (kernels/scalar/ sources).                          */
/* ---------------------------------------------------------------------- */
void orc_add(float *dst, const float *l, const float *r, int64_t n);
void orc_subtract(float *dst, const float *l, const float *r, int64_t n);
void orc_multiply(float *dst, const float *l, const float *r, int64_t n);
void orc_divide(float *dst, const float *l, const float *r, int64_t n);
void orc_scale(float *dst, const float *s, float f, int64_t n);
void orc_add_scaled(float *dst, const float *b, const float *s, float f, int64_t n);
void orc_negate(float *dst, const float *s, int64_t n);
void orc_abs(float *dst, const float *s, int64_t n);
void orc_square(float *dst, const float *s, int64_t n);
void orc_relu_squared(float *dst, const float *s, int64_t n);
void orc_swiglu(float *dst, const float *gate, const float *up, float clamp, int64_t n);
void orc_swiglu_backward(float *dgate, float *dup, const float *gate, const float *up,
                         const float *dout, float clamp, int64_t n);
void orc_exp(float *dst, const float *s, int64_t n);
void orc_sigmoid(float *dst, const float *s, int64_t n);
void orc_tanh(float *dst, const float *s, int64_t n);
void orc_rsqrt(float *dst, const float *s, int64_t n);
float orc_sum(const float *v, int64_t n);
float orc_max(const float *v, int64_t n);
int64_t orc_argmax(const float *v, int64_t n);
void orc_matmul(float *dst, const float *l, const float *r, int64_t rows, int64_t cols, int64_t inner);
void orc_matmul_transposed(float *dst, const float *l, const float *r, int64_t rows, int64_t cols,
                           int64_t inner);
float orc_dot(const float *l, const float *r, int64_t n);
void orc_softmax_last_dim(float *dst, const float *s, int64_t rows, int64_t cols);
void orc_rmsnorm_last_dim(float *dst, const float *s, int64_t rows, int64_t cols, float eps);
void orc_indexer_scores(float *dst, const float *q, const float *k, const float *w, int64_t rows,
                        int64_t blocks, int64_t heads, int64_t dim);
void orc_indexer_block_max(float *dst, const float *scores, int64_t rows, int64_t blocks,
                           int64_t group);
void orc_topk_indices(int32_t *dst, const float *scores, int64_t rows, int64_t count, int64_t k);
void orc_moe_gate_topk(const float *logits, const float *bias, float *probs, int32_t *selected,
                       float *weights, int64_t rows, int64_t experts, int64_t k);
void orc_grouped_matmul_transposed(float *dst, const float *in, const float *w,
                                   const int32_t *counts, int64_t experts, int64_t cols,
                                   int64_t inner);
/* AttentionForward: lse may be NULL; segment may be NULL. */
void orc_attention_forward(const float *q, const float *k, const float *v, float *out, float *lse,
                           const int32_t *segment, int64_t nseg, int64_t qlen, int64_t klen,
                           int64_t dim, int64_t offset, int64_t window);
void orc_attention_backward(const float *q, const float *k, const float *v, const float *o,
                            const float *dout, const float *lse, const float *row_correction,
                            const int32_t *segment, int64_t nseg, float *dq, float *dk, float *dv,
                            int64_t qlen, int64_t klen, int64_t dim, int64_t offset,
                            int64_t window);
void orc_attention_forward_split(const float *q, const float *k, const float *v, float *acc,
                                 float *mx, float *sum, const int32_t *segment, int64_t nseg,
                                 int64_t qlen, int64_t klen, int64_t dim, int64_t offset,
                                 int64_t window, int64_t kstart, int64_t kend);
/* partials: nparts accumulators [qlen*dim], maxima [qlen], sums [qlen] laid
 * out contiguously (part-major). */
void orc_attention_combine(const float *acc, const float *mx, const float *sum, int64_t nparts,
                           float *out, float *lse, int64_t qlen, int64_t dim);

/* ---------------------------------------------------------------------- */
/* Go math/rand/v2 PCG + tensors.RNG + the top-k Gumbel sampler.           */
/* ---------------------------------------------------------------------- */
typedef struct {
  uint64_t hi, lo;
} orc_pcg;
void orc_rng_new(orc_pcg *g, uint64_t seed);           /* tensors/random.go:16-18 */
uint64_t orc_rng_uint64(orc_pcg *g);                    /* PCG.Uint64 (DXSM) */
float orc_rng_float32(orc_pcg *g);                      /* Rand.Float32 */
void orc_rng_advance(orc_pcg *g, uint64_t delta_hi, uint64_t delta_lo); /* jump ahead */
float orc_kth_largest(const float *v, int64_t n, int64_t rank);
int64_t orc_sample_multinomial(orc_pcg *g, const float *logits, int64_t n, float temperature);
void orc_sample_next_token(const float *logits, int64_t rows, int64_t vocab, orc_pcg *g,
                           float temperature, int64_t top_k, int32_t *out);
float orc_gumbel_from_uniform(float u);

/* ---------------------------------------------------------------------- */
/* Calculator tool + byte-level tokenizer (inference/tooluse.go,           */
/* tokenizer/tokenizer.go).                                               */
/* ---------------------------------------------------------------------- */
/* Returns 1 and writes a NUL-terminated result when the calculator
 * understands expr; 0 otherwise. */
int orc_calculator(const char *expr, char *out, size_t out_cap);

/* ---------------------------------------------------------------------- */
/* Dense transformer (model/ sources) in float32 and float64 builds.           */
/* ---------------------------------------------------------------------- */
typedef struct {
  int32_t sequence_len, vocab_size, n_layer, n_head, n_kv_head, n_embd, rotary_dims;
  char window_pattern[16];
  /* Latent preset (model/preset.go:122-129), resolved by the caller; zeros
   * select the dense model.  mla_latent > 0 enables absorbed MLA
   * (Config.MLALatent) with mla_rope_dims decoupled rotary dims
   * (Config.MLARotaryDimension); n_experts > 0 enables the DeepSeekMoE
   * feed-forward: a shared SwiGLU expert of shared_hidden plus n_experts
   * routed experts of expert_hidden, experts_per_token selected
   * (model/config.go:138-227). */
  int32_t mla_latent, mla_rope_dims;
  int32_t n_experts, experts_per_token, expert_hidden, shared_hidden;
  float moe_clamp, moe_scale, balance_weight;
  /* Flash preset (model/preset.go:93-118): KV compression ratio > 1 makes
   * every layer an HCA compressed-attention layer (model/compress.go,
   * model/compress_attention.go) with a local sliding window of swa_window
   * keys merged in (0: none).  The sparse indexer, cross-layer reuse and
   * CED fields are reserved: this restatement requires them to be zero. */
  int32_t compression_ratio, swa_window;
  int32_t sparse_topk, indexer_dim, indexer_heads, indexer_pool, indexer_candidates;
  float indexer_weight;
  char reuse_pattern[16];
  int32_t ced;
} orc_config;

/* Sorted-name parameter table (model/params.go:14-85). */
int orc_param_count(const orc_config *cfg);
/* Writes name into name_out (cap 96) and returns numel; shape in rows/cols. */
int64_t orc_param_info(const orc_config *cfg, int index, char *name_out, int64_t *rows,
                       int64_t *cols);
int64_t orc_param_total(const orc_config *cfg);

#define ORC_MODEL_DECL(SFX, REAL)                                                                \
  typedef struct orc_model##SFX orc_model##SFX;                                                  \
  orc_model##SFX *orc_model_new##SFX(const orc_config *cfg, const REAL *params);                 \
  void orc_model_free##SFX(orc_model##SFX *m);                                                   \
  /* Inference forward without cache: logits [B,T,V]. */                                        \
  void orc_forward##SFX(orc_model##SFX *m, const int32_t *ids, int B, int T, REAL *logits);     \
  /* Token-by-token KV-cache decode of the same ids; logits [B,T,V]. */                          \
  void orc_forward_decode##SFX(orc_model##SFX *m, const int32_t *ids, int B, int T, int chunk,   \
                               REAL *logits);                                                    \
  /* PolicyGradientStep (trainer/rl.go:14-60): returns loss; writes nll[B*T] and the           \
   * parameter gradients grads[param_total] (overwritten). */                                   \
  double orc_pg_step##SFX(orc_model##SFX *m, const int32_t *inputs, const int32_t *targets,     \
                          int B, int T, const float *adv, float norm, REAL *nll, REAL *grads);   \
  /* trainer.DistillStep given the teacher's logits (trainer/distill.go:13-46). */                \
  double orc_distill_step##SFX(orc_model##SFX *m, const float *teacher, const int32_t *inputs,   \
                               const int32_t *mask, int B, int T, float temperature, int accum,  \
                               REAL *grads);                                                      \
  /* Mean cross-entropy with the gradcheck weighting (model/gradcheck_test.go:94-110). */         \
  double orc_ce_loss##SFX(orc_model##SFX *m, const int32_t *inputs, const int32_t *targets,     \
                          int B, int T, REAL *grads);                                            \
  /* Engine.GenerateBatchWith (inference/engine.go:336-369) for one prompt.  rows_out is         \
   * [S, P+max_tokens] (prompt + completion, terminal excluded); lens_out[S]. */                \
  void orc_generate_batch##SFX(orc_model##SFX *m, const int32_t *prompt, int P, int S,          \
                               int max_tokens, float temperature, int top_k, uint64_t seed,     \
                               int32_t *rows_out, int32_t *lens_out);                           \
  /* precomputeRotary (model/rotary.go:16-30) and ApplyRotary for one token's heads           \
   * (model/rotary.go:43-75), the functions the model uses. */                                   \
  void orc_rotary_table##SFX(int npos, int R, REAL *cosT, REAL *sinT);                          \
  void orc_apply_rotary##SFX(REAL *dst, const REAL *src, int heads, int D, int R,               \
                             const REAL *cw, const REAL *sw);                                    \
  /* GenerateWith's logits for one group with the fed columns given: out [ncols+1][S][V]      \
   * (the prefill's last logits, then those after each column cols[t][S]). */                    \
  void orc_decode_forced##SFX(orc_model##SFX *m, const int32_t *prompt, int P, int S,           \
                              const int32_t *cols, int ncols, REAL *out);                       \
  /* One chat_rl step (cmd/chat_rl/main.go:101-183) over G groups of S rollouts with           \
   * precomputed rewards.  Outputs: rollouts/lengths as generate; adv[G*S]; maxLen;              \
   * inputs/targets [G*S, maxLen-1]; nll; grads; returns loss. */                                \
  double orc_rl_step##SFX(orc_model##SFX *m, const int32_t *prompts, int G, int P, int S,       \
                          int max_tokens, float temperature, int top_k, const uint64_t *seeds,  \
                          const float *rewards, int32_t *rows_out, int32_t *lens_out,           \
                          float *adv_out, int32_t *max_len_out, int32_t *inputs_out,            \
                          int32_t *targets_out, REAL *nll, REAL *grads);

ORC_MODEL_DECL(_f32, float)
ORC_MODEL_DECL(_f64, double)
/* Sequence-level MoE balance loss of the last training forward
 * (model/train_transformer.go:121-123; 0 without MoE). */
double orc_aux_loss_f32(const orc_model_f32 *m);
double orc_aux_loss_f64(const orc_model_f64 *m);
/* The CSA indexer's distillation (compress_attention.go:133-147): its
 * gradient holds the targets constant, so finite-difference checks freeze
 * them -- mode 1 records every layer's targets at the next training
 * forward, 2 reuses them, 0 computes them -- and differentiate CE plus
 * orc_distill_loss (weight * sum of -target . log softmax(I) of the last
 * forward). */
void orc_set_freeze_targets_f32(orc_model_f32 *m, int mode);
void orc_set_freeze_targets_f64(orc_model_f64 *m, int mode);
double orc_distill_loss_f32(const orc_model_f32 *m);
void orc_model_set_params_f32(orc_model_f32 *m, const float *params);
/* PrefillCED (model/transformer.go:363-449) of a batch-1 prompt into a fresh
 * cache: the last replayed row's logits [vocab]. */
void orc_prefill_ced_f32(orc_model_f32 *m, const int32_t *ids, int T, float *last_logits);
void orc_prefill_ced_f64(orc_model_f64 *m, const int32_t *ids, int T, double *last_logits);
void orc_model_set_params_f64(orc_model_f64 *m, const double *params);
double orc_distill_loss_f64(const orc_model_f64 *m);

/* ChannelCompressor.Forward of one sequence (model/compress.go:110-164):
 * logits [T][D] (bias added), value [T][D] -> comp [ceil(T/ratio)][D],
 * probs [blocks][ratio][D]. */
void orc_channel_compress(int T, int D, int ratio, const float *logits, const float *value,
                          float *comp, float *probs);
/* mergeAttentionBranches (model/compress_attention.go:440-466). */
void orc_merge_attention_rows(float *out, float *lse, const float *oa, const float *la,
                              const float *ob, const float *lb, int rows, int D);

/* CSA lightning-indexer pieces (model/indexer.go), float32 build:
 * topKIndices (:226-268, returns the count); IndexerScores
 * (kernels/scalar/indexer.go:11-34); the hierarchical selection of T rows at
 * positions offset.. (selectFromScoreMatrix / selectRows /
 * selectRowBlockMax, indexer.go:378-530; sel rows of kcap, candidate rows of
 * ccap, may be NULL); fineSelect (:560-606); restrictIndexerToPool
 * (compress_attention.go:199-230). */
int orc_indexer_topk(const float *values, int n, int k, int32_t *out);
void orc_indexer_scores_rows(const float *iq, const float *ik, const float *w, int rows, int blocks,
                             int heads, int dim, float *out);
void orc_select_rows(const float *scores, int T, int blocks, int offset, int ratio, int topk,
                     int pool, int budget, int kcap, int ccap, int32_t *sel, int32_t *nsel,
                     int32_t *cand, int32_t *ncand);
void orc_fine_select(const float *iq_row, const float *ik, const float *w, int heads, int dim,
                     const int32_t *cand, int nc, int topk, int max_block, int32_t *sel,
                     int32_t *nsel);
void orc_restrict_to_pool(float *scores, float *target, int T, int blocks, const int32_t *pool,
                          const int32_t *npool, int ccap);

/* Window sizes (model/config.go:629-645): writes n_layer left widths. */
void orc_window_sizes(const orc_config *cfg, int32_t *out);

/* Number of OpenMP threads the oracle uses (for the CPU baseline report). */
int orc_num_threads(void);

/* ---- MuonAdamW optimizer step (optimizer.c) ------------------------------
 * One table entry per optimized tensor or tensor view, in MuonAdamW's
 * iteration order; same layout as gn_opt_param in include/gonano_hip.h. */
enum { ORC_OPT_ADAMW = 0, ORC_OPT_MUON = 1, ORC_OPT_SINKHORN = 2 };
typedef struct {
  int64_t offset; /* into the flat parameter / gradient vectors */
  int32_t rows, cols;
  int32_t kind;
  float lr, beta1, beta2, eps, weight_decay; /* AdamW (lr, weight_decay: all kinds) */
  float momentum;                            /* Muon, Sinkhorn */
  int32_t ns_steps;                          /* Muon */
  float muon_beta2;                          /* Muon */
  float gamma;                               /* Sinkhorn */
  int32_t sinkhorn_steps;
  float tau, sinkhorn_eps;
} orc_opt_param;
int64_t orc_opt_state_floats(const orc_opt_param *t, int n);
void orc_opt_step(float *params, const float *grads, const orc_opt_param *t, int n, float *state,
                  int32_t *steps);
void orc_polar_express(float *u, int64_t rows, int64_t cols, int steps);

#ifdef __cplusplus
}
#endif
#endif
