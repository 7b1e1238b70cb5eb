/*
 * gonano_hip.h - C ABI of libgnhip.so, the MI355X (gfx950) HIP backend for
 * gonano's RL step.
 *
 * Two groups of entry points:
 *
 *  1. gn_<method>: the 33 methods of gonano's numeric plugin interface
 *     kernels.Backend (kernels/backend.go:21-297), one C function each, on
 *     host pointers with the same argument meaning.  They stage the operands
 *     through device memory on a per-thread stream and are re-entrant, since
 *     the reference calls its backend concurrently from goroutines
 *     (model/attention.go:311-320, tensors/loss.go:30-37).  Lengths are the
 *     Go slice lengths; destinations may alias sources.
 *
 *  2. gn_session_* / gn_generate_batch / gn_policy_gradient_step /
 *     gn_rl_step: a device-resident session that runs the fused hot path the
 *     interface cannot carry (in the reference the sampler, the PG loss
 *     loops, softcap backward, smear and embedding scatter are Go loops
 *     outside kernels.Backend).  They replace Engine.GenerateBatchWith
 *     (inference/engine.go:336-369), trainer.PolicyGradientStep
 *     (trainer/rl.go:14-60) and the body of cmd/chat_rl's step loop
 *     (cmd/chat_rl/main.go:101-183).
 *
 * Every function returns a gn_status; on failure gn_last_error() gives the
 * message for the calling thread.  Pointers are borrowed for the call only.
 */
#ifndef GONANO_HIP_H
#define GONANO_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
  GN_OK = 0,
  GN_ERR_INVALID = 1,     /* bad shape or argument (the reference panics) */
  GN_ERR_HIP = 2,         /* a HIP runtime call failed */
  GN_ERR_OOM = 3,         /* device or host allocation failed */
  GN_ERR_UNSUPPORTED = 4, /* configuration not built for this device */
  GN_ERR_INTERNAL = 5
} gn_status;

/* Message of the last failure on the calling thread ("" if none). */
const char *gn_last_error(void);
/* Number of visible HIP devices (0 when none); never fails. */
int gn_device_count(void);
/* Selects the device the calling thread's backend calls run on (default 0). */
int gn_set_device(int device);
/* Waits for all work the calling thread queued. */
int gn_synchronize(void);

/* ---- kernels.Backend: Elementwise (kernels/backend.go:21-67) ------------- */
int gn_add(float *destination, const float *left, const float *right, int64_t n);
int gn_subtract(float *destination, const float *left, const float *right, int64_t n);
int gn_multiply(float *destination, const float *left, const float *right, int64_t n);
int gn_divide(float *destination, const float *left, const float *right, int64_t n);
int gn_scale(float *destination, const float *source, float factor, int64_t n);
int gn_add_scaled(float *destination, const float *base, const float *scaled, float factor,
                  int64_t n);
int gn_negate(float *destination, const float *source, int64_t n);
int gn_abs(float *destination, const float *source, int64_t n);
int gn_square(float *destination, const float *source, int64_t n);
int gn_relu_squared(float *destination, const float *source, int64_t n);
int gn_swiglu(float *destination, const float *gate, const float *up, float clamp, int64_t n);
int gn_swiglu_backward(float *gate_gradient, float *up_gradient, const float *gate,
                       const float *up, const float *output_gradient, float clamp, int64_t n);
int gn_exp(float *destination, const float *source, int64_t n);
int gn_sigmoid(float *destination, const float *source, int64_t n);
int gn_tanh(float *destination, const float *source, int64_t n);
int gn_rsqrt(float *destination, const float *source, int64_t n);

/* ---- Reductions (kernels/backend.go:70-78) ------------------------------- */
int gn_sum(const float *values, int64_t n, float *result);
int gn_max(const float *values, int64_t n, float *result);
int gn_argmax(const float *values, int64_t n, int64_t *result);

/* ---- LinearAlgebra (kernels/backend.go:82-93) ---------------------------- */
int gn_matmul(float *destination, const float *left, const float *right, int64_t row_count,
              int64_t column_count, int64_t inner_count);
int gn_matmul_transposed(float *destination, const float *left, const float *right,
                         int64_t row_count, int64_t column_count, int64_t inner_count);
int gn_dot_product(const float *left, int64_t left_len, const float *right, int64_t right_len,
                   float *result);

/* ---- Indexer (kernels/backend.go:103-116) -------------------------------- */
int gn_indexer_scores(float *destination, const float *query, const float *key,
                      const float *weight, int64_t row_count, int64_t block_count,
                      int64_t head_count, int64_t dim);
int gn_indexer_block_max(float *destination, const float *scores, int64_t row_count,
                         int64_t block_count, int64_t group_size);

/* ---- MoE (kernels/backend.go:119-141) ------------------------------------ */
int gn_topk_indices(int32_t *destination, const float *scores, int64_t row_count,
                    int64_t count, int64_t k);
int gn_moe_gate_topk(const float *logits, const float *bias, float *probs, int32_t *selected,
                     float *selected_weights, int64_t row_count, int64_t expert_count,
                     int64_t k);
int gn_grouped_matmul_transposed(float *destination, const float *input, const float *weight,
                                 const int32_t *token_counts, int64_t expert_count,
                                 int64_t column_count, int64_t inner_count);

/* ---- Rows (kernels/backend.go:145-153) ----------------------------------- */
int gn_softmax_last_dim(float *destination, const float *source, int64_t row_count,
                        int64_t column_count);
int gn_rmsnorm_last_dim(float *destination, const float *source, int64_t row_count,
                        int64_t column_count, float epsilon);

/* ---- Attention (kernels/backend.go:155-283) ------------------------------ */
/* AttentionForward: query [query_length, head_dim], key/value
 * [key_length, head_dim]; window < 0 is full causal context; segment_ids
 * (nullable, segment_count entries) is the sample-level mask; log_sum_exp is
 * nullable. */
int gn_attention_forward(const float *query, const float *key, const float *value,
                         const int32_t *segment_ids, int64_t segment_count, int64_t query_length,
                         int64_t key_length, int64_t head_dim, int64_t position_offset,
                         int64_t window, float *output, float *log_sum_exp);
/* AttentionBackward: gradients ACCUMULATE into query/key/value_gradient;
 * row_correction and segment_ids are nullable. */
int gn_attention_backward(const float *query, const float *key, const float *value,
                          const float *output, const float *output_gradient,
                          const float *log_sum_exp, const float *row_correction,
                          const int32_t *segment_ids, int64_t segment_count,
                          int64_t query_length, int64_t key_length, int64_t head_dim,
                          int64_t position_offset, int64_t window, float *query_gradient,
                          float *key_gradient, float *value_gradient);
/* AttentionForwardSplit over keys [key_start, key_end); overwrites
 * accumulator [query_length, head_dim], maximum and sum [query_length]. */
int gn_attention_forward_split(const float *query, const float *key, const float *value,
                               const int32_t *segment_ids, int64_t segment_count,
                               int64_t query_length, int64_t key_length, int64_t head_dim,
                               int64_t position_offset, int64_t window, int64_t key_start,
                               int64_t key_end, float *accumulator, float *maximum, float *sum);
/* AttentionCombine of part_count shards given as pointer arrays. */
int gn_attention_combine(const float *const *accumulators, const float *const *maxima,
                         const float *const *sums, int64_t part_count, int64_t query_length,
                         int64_t head_dim, float *output, float *log_sum_exp);

/* ---- Session: device-resident model for the fused RL step --------------- */
/* model.Config (model/config.go:9-124): the dense fields, then the latent
 * preset's (model/preset.go:120-129) with resolved values; zeros keep the
 * dense model.  mla_latent > 0 selects absorbed multi-head latent attention
 * (Config.MLALatent) with mla_rope_dims decoupled rotary dims
 * (Config.MLARotaryDimension()); n_experts > 0 selects the DeepSeekMoE
 * feed-forward: a clamped-SwiGLU shared expert of shared_hidden plus
 * n_experts routed experts of expert_hidden, experts_per_token chosen per
 * token, outputs scaled by moe_scale, SwiGLU clamp moe_clamp and the
 * sequence-level balance loss weight balance_weight
 * (Config.MoEActiveExperts / MoEExpertHidden / MoESharedHidden /
 * MoEEffectiveScale / MoEEffectiveClamp / MoEBalanceLossWeight).
 *
 * The flash preset's fields (model/preset.go:93-118, model/config.go:9-124):
 * compression_ratio > 1 makes every layer's attention compressed (HCA,
 * Config.Compression(): a channel compressor per layer reduces each block of
 * compression_ratio positions to one key/value row; queries attend to the
 * blocks before their own) merged with a sliding-window local branch of
 * swa_window keys (Config.SWAWindowSize(); 0: none).  sparse_topk,
 * indexer_dim, indexer_heads, indexer_pool, indexer_candidates,
 * indexer_weight (the CSA lightning indexer: top-k compressed blocks per
 * query, hierarchical over groups of indexer_pool blocks within a budget of
 * indexer_candidates, trained by its distillation loss of weight
 * indexer_weight), reuse_pattern (FRU cross-layer reuse, e.g. "FRU") and
 * ced (the causal encoder-decoder split at n_layer / 2) take the
 * reference's resolved values (Config.Compression, SWAWindowSize,
 * SparseTopK, indexerDefaults, IndexerPool, IndexerCandidateBudget,
 * IndexerWeight, ReusePattern, CEDEnabled; model/config.go:282-420).
 * compression_ratio 0 turns the preset off; zero indexer_dim,
 * indexer_heads, indexer_candidates and indexer_weight take the reference's
 * defaults (64, 1, max(8 * sparse_topk, 64), 1).  gn_session_create returns
 * a non-zero status for the combinations Config.Validate rejects and for
 * shapes the kernels do not cover (ratio 2..8 or 16, top-k <= 64, indexer
 * heads * dim <= 256). */
typedef struct gn_config {
  int32_t sequence_len;
  int32_t vocab_size;
  int32_t n_layer;
  int32_t n_head;
  int32_t n_kv_head;
  int32_t n_embd;
  int32_t rotary_dims;
  char window_pattern[16];
  int32_t mla_latent;
  int32_t mla_rope_dims;
  int32_t n_experts;
  int32_t experts_per_token;
  int32_t expert_hidden;
  int32_t shared_hidden;
  float moe_clamp;
  float moe_scale;
  float balance_weight;
  int32_t compression_ratio;
  int32_t swa_window;
  int32_t sparse_topk;
  int32_t indexer_dim;
  int32_t indexer_heads;
  int32_t indexer_pool;
  int32_t indexer_candidates;
  float indexer_weight;
  char reuse_pattern[16];
  int32_t ced;
} gn_config;

typedef struct gn_session gn_session;

/* model.NewTransformer (model/transformer.go:50-80) on `device`. */
int gn_session_create(const gn_config *config, int device, gn_session **out);
int gn_session_destroy(gn_session *session);
/* Total float count of the flat parameter vector: every tensor of
 * Transformer.NamedParameters in ParameterNames (sorted) order
 * (model/params.go:14-113). */
int gn_session_param_total(const gn_session *session, int64_t *total);
/* Name, shape and offset of the index-th parameter in that order. */
int gn_session_param_info(const gn_session *session, int32_t index, char *name, size_t name_cap,
                          int64_t *rows, int64_t *cols, int64_t *offset);
int gn_session_param_count(const gn_session *session, int32_t *count);
int gn_session_set_params(gn_session *session, const float *params, int64_t count);
int gn_session_get_params(const gn_session *session, float *params, int64_t count);
/* Parameter gradients (Tensor.Grad of every parameter) in the same layout. */
int gn_session_get_grads(const gn_session *session, float *grads, int64_t count);
/* Transformer.ZeroGrad (model/params.go:97-101). */
int gn_session_zero_grads(gn_session *session);
/* Transformer.UpdateRouterBias (model/transformer.go:121-131, moe.go:330-341)
 * with speed = Config.MoERouterBiasUpdate(): every MoE layer's router bias
 * moves by +-speed toward balance from the tokens its training forwards
 * (gn_rl_step / gn_pg_step / gn_distill_step, MoE.forwardTraining,
 * moe.go:192-193) routed to each expert since the last update, and the
 * counts are cleared.  No MoE: nothing to do. */
int gn_session_update_router_bias(gn_session *session, float speed);
/* Those counts (MoE.loadCounts), [n_layer][n_experts] in float64; count
 * must be n_layer * n_experts (0 without MoE). */
int gn_session_moe_loads(const gn_session *session, double *loads, int64_t count);

/* trainer.DistillStep (trainer/distill.go:13-46) for one micro-batch:
 * the frozen `teacher` session (same device and vocabulary, any
 * architecture) scores inputs [batch, seq_len]; the student `session`'s
 * gradients accumulate (d/dθ of) the forward-KL loss
 * (tensors/loss.go:84-214) of every position whose mask entry is non-zero
 * (mask NULL: every position), scaled by 1 / (valid positions *
 * grad_accum_steps).  loss_out: the mean per-position loss. */
int gn_distill_step(gn_session *session, gn_session *teacher, const int32_t *inputs,
                    const int32_t *mask, int32_t batch, int32_t seq_len, float temperature,
                    int32_t grad_accum_steps, float *loss_out);

/* ---- optimizer step (optimizer/optimizer.go, muon.go, sinkhorn.go) -------
 * MuonAdamW (optimizer/optimizer.go:72-137) over the session's parameters
 * and gradients.  The host builds the parameter groups exactly as
 * Transformer.SetupOptimizer (model/optimizer.go:16-181) and passes one
 * entry per optimized tensor or tensor view (a head of c_q/c_k under
 * head-wise Muon, one expert of a packed expert weight), in the order
 * MuonAdamW.Step visits them; `offset` indexes the flat parameter vector
 * (gn_session_param_info) and the view is rows x cols floats from there.
 * Fields a kind does not use are ignored. */
enum { GN_OPT_ADAMW = 0, GN_OPT_MUON = 1, GN_OPT_SINKHORN = 2 };
typedef struct {
  int64_t offset;
  int32_t rows, cols;
  int32_t kind;
  float lr, beta1, beta2, eps, weight_decay; /* ParamGroup.LR .. WeightDecay */
  float momentum;                            /* ParamGroup.Momentum */
  int32_t ns_steps;                          /* ParamGroup.NSSteps (<= 5) */
  float muon_beta2;                          /* ParamGroup.MuonBeta2 */
  float gamma;                               /* ParamGroup.Gamma */
  int32_t sinkhorn_steps;                    /* ParamGroup.SinkhornSteps */
  float tau, sinkhorn_eps;                   /* ParamGroup.SinkhornTau, SinkhornEps */
} gn_opt_param;
typedef struct gn_optimizer gn_optimizer;
/* optimizer.NewMuonAdamW (optimizer/optimizer.go:81-110): zeroed state. */
int gn_optimizer_create(gn_session *session, const gn_opt_param *table, int32_t count,
                        gn_optimizer **out);
/* MuonAdamW.Step (optimizer/optimizer.go:118-137) on the device parameters,
 * consuming the accumulated gradients (which stay as they are; ZeroGrad is
 * gn_session_zero_grads). */
int gn_optimizer_step(gn_optimizer *optimizer);
/* Trainer.StepOptimizer's schedules (trainer/trainer.go:80-102) set each
 * group's LR, Momentum and WeightDecay before every Step: one value per
 * table entry (the entry's group's value), in table order; a NULL array
 * leaves that field as it is.  The state is kept. */
int gn_optimizer_set_hyper(gn_optimizer *optimizer, const float *lr, const float *momentum,
                           const float *weight_decay, int32_t count);
/* The optimizer state, entry by entry: AdamW expAvg[n] expAvgSq[n]; Muon
 * momentum[n] secondMom[max(rows, cols)]; Sinkhorn momentum[n]. */
int gn_optimizer_state_size(const gn_optimizer *optimizer, int64_t *count);
int gn_optimizer_get_state(const gn_optimizer *optimizer, float *state, int64_t count);
int gn_optimizer_destroy(gn_optimizer *optimizer);

/* Transformer.Forward without a cache (model/transformer.go:211-214):
 * logits [batch, seq_len, vocab] of ids [batch, seq_len]. */
int gn_forward(gn_session *session, const int32_t *ids, int32_t batch, int32_t seq_len,
               float *logits);

/* Engine.GenerateBatchWith (inference/engine.go:336-369) for `groups`
 * prompts at once, each expanded to `samples` rows and sampled from its own
 * tensors.RNG stream seeds[g].  rows_out is [groups*samples,
 * prompt_len+max_tokens] (prompt + completion, terminal token excluded),
 * lengths_out [groups*samples]. */
int gn_generate_batch(gn_session *session, const int32_t *prompts, int32_t groups,
                      int32_t prompt_len, int32_t samples, int32_t max_tokens, float temperature,
                      int32_t top_k, const uint64_t *seeds, int32_t *rows_out,
                      int32_t *lengths_out);

/* inference.GenerateOptions (inference/engine.go:25-34) together with what
 * GenerateWith takes from the engine's tokenizer and tool registry
 * (engine.go:215-224, 282-296): the ids Tokenizer.EncodeSpecial /
 * BOSTokenID return for the host's tokenizer, and the tool call.
 *
 * tool, when set, is Registry.Execute(Tokenizer.Decode(call)) followed by
 * Tokenizer.Encode of the result, run on the host: it receives the n ids
 * between <|tool_start|> and <|tool_end|>, writes at most cap result ids
 * into out and returns their count, or -1 when no tool understands the
 * call (no output is forced then).  It is called from the calling thread
 * during gn_generate_batch_with / gn_rl_step_with.  tool NULL uses the
 * built-in calculator (inference/tooluse.go:27-90) over the byte-level
 * tokenizer's Decode/Encode (tokenizer/special.go:19-31). */
typedef struct gn_generate_options {
  int32_t thinking;        /* GenerateOptions.Thinking */
  int32_t thinking_budget; /* GenerateOptions.ThinkingBudget (<= 0: no budget) */
  int32_t bos;             /* Tokenizer.BOSTokenID() */
  int32_t assistant_end;   /* EncodeSpecial("<|assistant_end|>") (also chat_rl's padding) */
  int32_t tool_start, tool_end, tool_output_start, tool_output_end;
  int32_t think_start, think_end;
  int32_t (*tool)(void *user, const int32_t *call, int32_t n, int32_t *out, int32_t cap);
  void *tool_user;
} gn_generate_options;
/* The byte-level tokenizer's ids, thinking off, the built-in calculator:
 * what gn_generate_batch and gn_rl_step use. */
int gn_generate_options_default(gn_generate_options *out);
/* Engine.GenerateBatchWith (inference/engine.go:336-369) with options
 * (NULL: the defaults); masks_out (nullable, [groups*samples,
 * prompt_len+max_tokens]) is GenerateBatchWith's masks: 0 for prompt and
 * forced tokens, 1 for sampled ones. */
int gn_generate_batch_with(gn_session *session, const int32_t *prompts, int32_t groups,
                           int32_t prompt_len, int32_t samples, int32_t max_tokens,
                           float temperature, int32_t top_k, const uint64_t *seeds,
                           const gn_generate_options *options, int32_t *rows_out,
                           int32_t *lengths_out, int32_t *masks_out);

/* trainer.PolicyGradientStep (trainer/rl.go:14-60): teacher-forced
 * recompute of inputs [batch, seq_len], per-token NLL (nll_out, nullable,
 * [batch*seq_len]; logp = -nll), loss = sum_valid nll*adv/norm, and the
 * backward of that loss ACCUMULATED into the session's parameter gradients. */
int gn_policy_gradient_step(gn_session *session, const int32_t *inputs, const int32_t *targets,
                            int32_t batch, int32_t seq_len, const float *advantages, float norm,
                            float *loss_out, float *nll_out);

/* One cmd/chat_rl step (cmd/chat_rl/main.go:101-183) without the optimizer:
 * rollouts of every group, group-mean advantages of the supplied rewards,
 * padding/masking, and PolicyGradientStep.  Outputs as gn_generate_batch plus
 * advantages_out [groups*samples], max_len_out and loss_out. */
int gn_rl_step(gn_session *session, const int32_t *prompts, int32_t groups, int32_t prompt_len,
               int32_t samples, int32_t max_tokens, float temperature, int32_t top_k,
               const uint64_t *seeds, const float *rewards, int32_t *rows_out,
               int32_t *lengths_out, float *advantages_out, int32_t *max_len_out,
               float *loss_out);
/* gn_rl_step with generation options (NULL: the defaults); rows are padded
 * with options->assistant_end (cmd/chat_rl/main.go:157-180). */
int gn_rl_step_with(gn_session *session, const int32_t *prompts, int32_t groups,
                    int32_t prompt_len, int32_t samples, int32_t max_tokens, float temperature,
                    int32_t top_k, const uint64_t *seeds, const gn_generate_options *options,
                    const float *rewards, int32_t *rows_out, int32_t *lengths_out,
                    float *advantages_out, int32_t *max_len_out, float *loss_out);
/* inference.UseCalculator (inference/tooluse.go:83-90), the built-in tool:
 * *ok = 1 and the NUL-terminated result in out (cap bytes), or *ok = 0 when
 * the expression is rejected.  Host code; needs no device. */
int gn_use_calculator(const char *expression, char *out, size_t cap, int32_t *ok);

/* inference.SampleNextToken (inference/sampler.go:16-60) on host logits
 * [rows, vocab] with the tensors.RNG state rng_state = {hi, lo} of Go's PCG,
 * which is advanced past the rows*vocab draws consumed. */
int gn_sample_next_token(const float *logits, int64_t rows, int64_t vocab, uint64_t *rng_state,
                         float temperature, int64_t top_k, int32_t *out);
/* gn_sample_next_token without any device allocation.  No counterpart in
 * the reference: for callers that cannot allocate device memory (tight
 * serving loops, harnesses that forbid hipMalloc).  The logits, the RNG
 * state and the sampled ids are staged through one fixed 65 MiB array in the
 * library's device memory (per GPU, held until the process ends) on the
 * calling thread's per-thread stream, so rows <= 65536 and rows * vocab <=
 * 16,777,216 (GN_ERR_INVALID otherwise).  Results equal
 * gn_sample_next_token's.  Calls on one device are serialized by a lock the
 * library holds from the first copy to the final stream synchronization
 * (calls on different devices run concurrently).  The call copies from
 * pageable host memory and synchronizes, so it cannot be captured into a
 * HIP graph. */
int gn_sample_next_token_static(const float *logits, int64_t rows, int64_t vocab,
                                uint64_t *rng_state, float temperature, int64_t top_k,
                                int32_t *out);

/* Self-check of the decode sampler's softcap handling.  No counterpart in the
 * reference: the decode sampler selects the top-k candidates on the raw
 * lm_head products and softcaps only the candidates, which equals softcapping
 * every logit first when softcap (15 tanh(y/15), transformer.go:538-541) is
 * non-decreasing over floats.  *violations = the number of neighbouring
 * floats, over all 2^32 bit patterns but NaNs, whose softcap decreases (or
 * is NaN) as computed on the device; 0 confirms the assumption. */
int gn_softcap_order_check(uint64_t *violations);

/* Device time (ms) the session spent in its most recent calls, by phase, and
 * the average duration of the named kernel class measured with HIP events on
 * the session stream.  Enabled by gn_session_set_timing(session, 1). */
typedef struct gn_timing {
  double rollout_ms;        /* gn_generate_batch wall time on device */
  double decode_attn_ms;    /* sum over decode-attention launches */
  int64_t decode_attn_launches;
  double decode_attn_bytes; /* algorithmic K/V bytes those launches read */
  double train_ms;          /* gn_policy_gradient_step on device */
  double gemm_ms;           /* GEMM launches inside the train step */
  double gemm_flops;        /* algorithmic flops of those launches */
  int64_t gemm_launches;
  double gemm_wide_ms;      /* the part of them run by the wide-tile engine (256x256 tiles) */
  double gemm_wide_flops;
  int64_t gemm_wide_launches;
  double loss_ms;           /* policy-gradient loss launches inside the train step */
  double loss_bytes;        /* algorithmic bytes of those launches: logits read + gradient written */
  int64_t loss_launches;
} gn_timing;
int gn_session_set_timing(gn_session *session, int enabled);
int gn_session_get_timing(const gn_session *session, gn_timing *out);
/* Rollout decode steps are captured once per gn_generate_batch / gn_rl_step
 * call as a HIP graph and replayed (default 1); 0 launches every kernel of
 * every step.  Results are identical either way.  No reference counterpart
 * (an execution knob of this backend). */
int gn_session_set_decode_graph(gn_session *session, int enabled);
/* Transformer.AuxiliaryLoss (model/transformer.go:108-116): the MoE
 * sequence-level balance loss of the most recent gn_policy_gradient_step /
 * gn_rl_step (0 without MoE); its gradient is already in the session's
 * parameter gradients. */
int gn_session_aux_loss(const gn_session *session, double *out);
/* Waits until the session stream is idle (no reference counterpart: the Go
 * backends are synchronous; used to bracket timed regions). */
int gn_session_synchronize(gn_session *session);

/* ---- prefix cache (inference/cache.go CacheManager, inference/prefix.go
 * PrefixCache) -------------------------------------------------------------
 * Engine.Cache / Engine.Prefix (inference/engine.go:44-51, 120-173) kept in
 * device memory: gn_generate_batch(_with) and gn_rl_step(_with) look every
 * prompt up and store its prefill state; a prompt whose longest stored strict
 * prefix has m tokens prefills only its last prompt_len - m tokens against
 * the stored keys/values.  A batch of groups sees the cache as that many
 * successive GenerateWith calls would (an earlier group's entry can serve a
 * later group).  An entry holds every layer's keys/values of its prompt, its
 * decode-cache rows, its last token embedding (KVBuffer.PrevEmbedding) and,
 * for compressed attention, the Full layers' compressor logits of every
 * position (a continuation recompresses the whole sequence from them, so the
 * raw sliding-window rows are kept and CacheOptions.StripSWA's bounded replay
 * is never needed); `bytes` counts that device memory (not the reference's
 * KVBuffer.BytesAllocated).  Entries are dropped whenever the parameters
 * change (gn_session_set_params, gn_optimizer_step): their state would no
 * longer equal a full prefill.  Not for CED models (GN_ERR_UNSUPPORTED; the
 * reference's engine skips them, inference/engine.go:128-140,
 * inference/prefix.go:17-19).  A call that fails leaves the cache as it
 * found it.  The on-disk tier is `disk_dir` below. */
typedef struct gn_prefix_cache_options {
  int32_t max_entries; /* CacheOptions.MaxEntries; 0: unbounded */
  int32_t max_prefix;  /* NewPrefixCache(maxPrefix): longer entries never hit; 0: any */
  int64_t max_bytes;   /* CacheOptions.MaxBytes (entry bytes, either tier); 0: unbounded */
  double ttl_seconds;  /* CacheOptions.TTL from storage; 0: no expiry */
  /* CacheOptions.DiskDir: entries are written to this directory (created if
   * missing; if that fails, or for an entry whose file cannot be written,
   * device memory is used) and read back for the call that hits them; a file
   * that cannot be read drops its entry and misses.  Files are deleted with
   * their entries (eviction, expiry, invalidation, new parameters, the
   * session's end).  NULL or "": device memory only. */
  const char *disk_dir;
} gn_prefix_cache_options;
/* NewCacheManager (cache.go:64-77) on the session: turns the cache on with
 * these limits (evicting to fit), or off with options NULL (dropping every
 * entry).  max_entries 1 with max_prefix is NewPrefixCache(maxPrefix). */
int gn_session_set_prefix_cache(gn_session *session, const gn_prefix_cache_options *options);
/* CacheManager.Invalidate (cache.go:162-174). */
int gn_session_prefix_cache_invalidate(gn_session *session);
/* CacheManager.Len (cache.go:176-180) after expiry, and the entries' device
 * bytes (bytes nullable). */
int gn_session_prefix_cache_len(gn_session *session, int32_t *entries, int64_t *bytes);
/* Per group of the last generate call, the prompt tokens taken from the
 * cache (Lookup's matched length; 0 for a miss or with the cache off).
 * groups must equal that call's. */
int gn_session_prefix_cache_hits(const gn_session *session, int32_t *hits, int32_t groups);

#ifdef __cplusplus
}
#endif
#endif
