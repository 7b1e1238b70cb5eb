/*
 * model.c - the gonano transformer's inference forward, KV-cache decode,
 * training forward/backward, policy-gradient step, batched generation and
 * one chat_rl step, restated in C: the dense preset, the latent preset
 * (MLA attention, DeepSeekMoE feed-forward) and the flash preset's
 * attention: compressed attention (HCA: channel compressor, block-causal
 * attention over compressed keys, sliding-window local branch merged by
 * log-sum-exp), sparse selection of compressed blocks (CSA: lightning
 * indexer, hierarchical top-k, distillation gradient), cross-layer reuse
 * (Full / Reindex / Reuse layers) and the causal encoder-decoder split (CED,
 * with its bounded-replay prefill).
 *
 * TEST INFRASTRUCTURE ONLY (see gn_oracle.h).
 *
 * This file is compiled twice: with REAL=float (SFX=_f32), the parity
 * oracle, which rounds to float32 where the reference does and accumulates
 * matmuls/softmax sums in float64 like kernels/scalar; and with REAL=double
 * (SFX=_f64), used by the finite-difference checks that pin the backward.
 */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "gn_oracle.h"

#ifndef REAL
#define REAL float
#define SFX _f32
#endif

#define CAT2(a, b) a##b
#define CAT(a, b) CAT2(a, b)
#define FN(name) CAT(name, SFX)
#define MODEL CAT(orc_model, SFX)
#define R(x) ((REAL)(x))

/* model/attention.go:11-21, model/helpers.go:7, model/transformer.go:11,15 */
#define NORM_EPS 1e-6f
#define QK_SCALE 1.2f
#define VE_GATE_CH 12
#define VE_GATE_SCALE 3.0f
#define SMEAR_CH 24
#define SOFTCAP 15.0f
#define ROT_OVER 10
#define MASKED (-1e30f)
#define MAXL 64

/* ---------------------------------------------------------------------- */
/* Parameter table shared by both builds (defined once, in the f32 build). */
/* ---------------------------------------------------------------------- */
typedef struct {
  char name[96];
  int64_t rows, cols, offset;
} param_entry;

static int has_value_embedding(int layer, int n_layer) { /* model/helpers.go:69-71 */
  return layer % 2 == (n_layer - 1) % 2;
}
static int padded_vocab(const orc_config *c) { /* model/config.go:622-624 */
  return ((c->vocab_size + 63) / 64) * 64;
}
/* precomputeRotary (model/rotary.go:16-30): cos/sin [npos][R/2] of
 * position * base^(-2j/R), base 100000, in float64 rounded once. */
void FN(orc_rotary_table)(int npos, int R, REAL *cosT, REAL *sinT) {
  int half = R / 2;
  for (int p = 0; p < npos; p++)
    for (int j = 0; j < half; j++) {
      double inv = pow(100000.0, -2.0 * (double)j / (double)R);
      double f = (double)p * inv;
      cosT[(int64_t)p * half + j] = R(cos(f));
      sinT[(int64_t)p * half + j] = R(sin(f));
    }
}

static int rotary_dim(const orc_config *c) { /* model/config.go:430-444 */
  int hd = c->n_embd / c->n_head;
  if (c->mla_latent > 0) return c->mla_rope_dims; /* MLARotaryDimension */
  return c->rotary_dims <= 0 ? hd : c->rotary_dims;
}
static int mlp_hidden(const orc_config *c) { /* model/block.go:23-28 */
  return c->n_experts > 0 ? c->shared_hidden : 4 * c->n_embd;
}
#define TABLE_MAX (24 * MAXL)

/* Flash preset layer roles (model/config.go:282-381). */
enum { REUSE_FULL = 0, REUSE_REINDEX = 1, REUSE_REUSE = 2 };
static int ced_split(const orc_config *c) { return c->ced ? c->n_layer / 2 : 0; }
static int reuse_half_start(const orc_config *c, int layer) {
  int split = ced_split(c);
  return (c->ced && split > 0 && layer >= split) ? split : 0;
}
static int reuse_mode_at(const orc_config *c, int layer) { /* config.go:326-344 */
  size_t n = strnlen(c->reuse_pattern, sizeof c->reuse_pattern);
  if (n == 0) return REUSE_FULL;
  char ch = c->reuse_pattern[(layer - reuse_half_start(c, layer)) % n];
  if (ch == 'R' || ch == 'r') return REUSE_REINDEX;
  if (ch == 'U' || ch == 'u') return REUSE_REUSE;
  return REUSE_FULL;
}
static int reuse_producer(const orc_config *c, int layer) { /* config.go:357-370 */
  if (reuse_mode_at(c, layer) == REUSE_FULL) return layer;
  for (int i = layer - 1; i >= reuse_half_start(c, layer); i--)
    if (reuse_mode_at(c, i) == REUSE_FULL) return i;
  return layer;
}
static void indexer_dims(const orc_config *c, int *dim, int *heads) { /* config.go:391-402 */
  *dim = c->indexer_dim > 0 ? c->indexer_dim : 64;
  *heads = c->indexer_heads > 0 ? c->indexer_heads : 1;
}
static int indexer_budget(const orc_config *c) { /* config.go:372-381 */
  if (c->indexer_candidates > 0) return c->indexer_candidates;
  int b = 8 * c->sparse_topk;
  return b < 64 ? 64 : b;
}

#if defined(ORC_DEFINE_SHARED)
static int cmp_entry(const void *a, const void *b) {
  return strcmp(((const param_entry *)a)->name, ((const param_entry *)b)->name);
}
/* model/params.go:14-85 (dense and latent presets), sorted as ParameterNames
 * does.  Packed expert tensors [E, H, C] / [E, C, H] are listed as rows E*H
 * (resp. E*C) by cols C (resp. H). */
static int build_table(const orc_config *c, param_entry *t) {
  int n = 0, C = c->n_embd, D = C / c->n_head, PV = padded_vocab(c);
  int Hq = c->n_head, Hkv = c->n_kv_head, L = c->n_layer;
#define ADD(nm, r, cc)                         \
  do {                                         \
    snprintf(t[n].name, 96, "%s", nm);         \
    t[n].rows = (r);                           \
    t[n].cols = (cc);                          \
    n++;                                       \
  } while (0)
  char nm[96];
  ADD("transformer.wte.weight", PV, C);
  ADD("lm_head.weight", PV, C);
  const int mla = c->mla_latent > 0, F = mlp_hidden(c);
  const int lat = c->mla_latent, rd = c->mla_rope_dims, cd = D - rd;
  const int E = c->n_experts, EH = c->expert_hidden;
  for (int l = 0; l < L; l++) {
    if (mla) { /* params.go:19-27, mla.go:41-58 */
      snprintf(nm, 96, "transformer.h.%d.attn.mla_q_down.weight", l); ADD(nm, lat, C);
      snprintf(nm, 96, "transformer.h.%d.attn.mla_q_up.weight", l); ADD(nm, Hq * cd, lat);
      snprintf(nm, 96, "transformer.h.%d.attn.mla_q_rope.weight", l); ADD(nm, Hq * rd, C);
      snprintf(nm, 96, "transformer.h.%d.attn.mla_kv_down.weight", l); ADD(nm, lat, C);
      snprintf(nm, 96, "transformer.h.%d.attn.mla_k_up.weight", l); ADD(nm, Hkv * cd, lat);
      snprintf(nm, 96, "transformer.h.%d.attn.mla_v_up.weight", l); ADD(nm, Hkv * D, lat);
      snprintf(nm, 96, "transformer.h.%d.attn.mla_k_rope.weight", l); ADD(nm, Hkv * rd, C);
    } else {
      snprintf(nm, 96, "transformer.h.%d.attn.c_q.weight", l); ADD(nm, Hq * D, C);
      snprintf(nm, 96, "transformer.h.%d.attn.c_k.weight", l); ADD(nm, Hkv * D, C);
      snprintf(nm, 96, "transformer.h.%d.attn.c_v.weight", l); ADD(nm, Hkv * D, C);
    }
    snprintf(nm, 96, "transformer.h.%d.attn.c_proj.weight", l); ADD(nm, C, C);
    if (c->compression_ratio > 1) {
      /* params.go:43-51: Full layers own a compressor (compress.go:33-43),
       * Full and Reindex layers an indexer when sparse (indexer.go:33-43,
       * attention.go:210-226) */
      int mode = reuse_mode_at(c, l);
      if (mode == REUSE_FULL) {
        snprintf(nm, 96, "transformer.h.%d.attn.compress_logits.weight", l); ADD(nm, D, C);
        snprintf(nm, 96, "transformer.h.%d.attn.compress_bias", l); ADD(nm, c->compression_ratio, D);
      }
      if (c->sparse_topk > 0 && mode != REUSE_REUSE) {
        int idim, ih;
        indexer_dims(c, &idim, &ih);
        snprintf(nm, 96, "transformer.h.%d.attn.indexer_query.weight", l); ADD(nm, ih * idim, C);
        snprintf(nm, 96, "transformer.h.%d.attn.indexer_key.weight", l); ADD(nm, ih * idim, D);
        snprintf(nm, 96, "transformer.h.%d.attn.indexer_heads", l); ADD(nm, ih, 1);
      }
    }
    if (!mla && has_value_embedding(l, L)) { /* transformer.go:72-78: no VE under MLA */
      snprintf(nm, 96, "transformer.h.%d.attn.ve_gate.weight", l); ADD(nm, Hkv, VE_GATE_CH);
      snprintf(nm, 96, "value_embeds.%d.weight", l); ADD(nm, PV, Hkv * D);
    }
    snprintf(nm, 96, "transformer.h.%d.mlp.c_fc.weight", l); ADD(nm, F, C);
    if (E > 0) { snprintf(nm, 96, "transformer.h.%d.mlp.c_gate.weight", l); ADD(nm, F, C); }
    snprintf(nm, 96, "transformer.h.%d.mlp.c_proj.weight", l); ADD(nm, C, F);
    if (E > 0) { /* params.go:57-63, moe.go:49-69 */
      snprintf(nm, 96, "transformer.h.%d.moe.router.weight", l); ADD(nm, E, C);
      snprintf(nm, 96, "transformer.h.%d.moe.router_bias", l); ADD(nm, E, 1);
      snprintf(nm, 96, "transformer.h.%d.moe.experts.gate.weight", l); ADD(nm, E * EH, C);
      snprintf(nm, 96, "transformer.h.%d.moe.experts.up.weight", l); ADD(nm, E * EH, C);
      snprintf(nm, 96, "transformer.h.%d.moe.experts.down.weight", l); ADD(nm, E * C, EH);
    }
  }
  ADD("resid_lambdas", L, 1);
  ADD("x0_lambdas", L, 1);
  ADD("smear_gate.weight", 1, SMEAR_CH);
  ADD("smear_lambda", 1, 1);
  ADD("backout_lambda", 1, 1);
#undef ADD
  qsort(t, n, sizeof(param_entry), cmp_entry);
  int64_t off = 0;
  for (int i = 0; i < n; i++) {
    t[i].offset = off;
    off += t[i].rows * t[i].cols;
  }
  return n;
}
int orc_param_count(const orc_config *c) {
  param_entry t[TABLE_MAX];
  return build_table(c, t);
}
int64_t orc_param_info(const orc_config *c, int index, char *name_out, int64_t *rows,
                       int64_t *cols) {
  param_entry t[TABLE_MAX];
  int n = build_table(c, t);
  if (index < 0 || index >= n) return -1;
  snprintf(name_out, 96, "%s", t[index].name);
  *rows = t[index].rows;
  *cols = t[index].cols;
  return t[index].rows * t[index].cols;
}
int64_t orc_param_total(const orc_config *c) {
  param_entry t[TABLE_MAX];
  int n = build_table(c, t);
  return t[n - 1].offset + t[n - 1].rows * t[n - 1].cols;
}
/* model/config.go:629-645: S = -((-T/4)/128)*128 in Go integer arithmetic
 * (truncating division), L = T; the last layer is always long. */
void orc_window_sizes(const orc_config *c, int32_t *out) {
  int T = c->sequence_len;
  int shortw = -((-T / 4) / 128) * 128;
  size_t plen = strlen(c->window_pattern);
  for (int l = 0; l < c->n_layer; l++) {
    char p = c->window_pattern[l % plen];
    out[l] = (p == 'L' || p == 'l') ? T : shortw;
  }
  out[c->n_layer - 1] = T;
}
int orc_num_threads(void) {
#ifdef _OPENMP
  extern int omp_get_max_threads(void);
  return omp_get_max_threads();
#else
  return 1;
#endif
}
#else
int orc_param_count(const orc_config *c);
#endif

static int64_t param_offset(const orc_config *c, const char *name) {
  char nm[96];
  int64_t r, cc, off = 0;
  int n = orc_param_count(c);
  for (int i = 0; i < n; i++) {
    int64_t numel = orc_param_info(c, i, nm, &r, &cc);
    if (strcmp(nm, name) == 0) return off;
    off += numel;
  }
  fprintf(stderr, "oracle: unknown parameter %s\n", name);
  abort();
}

/* ---------------------------------------------------------------------- */
/* Model                                                                   */
/* ---------------------------------------------------------------------- */
typedef struct {
  int64_t wq, wk, wv, wo, wve, wfc, wproj, ve;
  /* latent preset: MLA projections, shared-expert gate, router, experts */
  int64_t wqd, wqu, wqr, wkvd, wku, wvu, wkr, wgate, wr, rbias, eg, eu, ed;
  int64_t wcl, cbias; /* HCA compressor logit weight [D, C] and bias [ratio, D] */
  int64_t wiq, wik, wih; /* CSA indexer query [HI, C], key [HI, D], head weights [ih] */
  int has_ve, window;
  int mode, producer, has_idx; /* reuse role, producing Full layer, owns an indexer */
} layer_off;

struct MODEL {
  orc_config cfg;
  int C, Hq, Hkv, D, R, F, L, V, PV, S, KVW;
  /* latent preset: MLA latent width, rope/content widths, experts */
  int mla, lat, rd, cd, E, K, EH;
  int ratio, swa; /* HCA compression ratio (> 1 = compressed layers) and SWA width */
  /* CSA: top-k, indexer head dim / heads / width, hierarchical pool, candidate
   * budget, distillation weight; CED encoder/decoder split (0: off) */
  int topk, idim, ih, HI, ipool, ibudget, split;
  REAL iw;
  /* Test hook for finite differences of the indexer's distillation: the
   * reference's gradient treats the targets as constants, so a check freezes
   * them (1: record each layer's final targets, 2: use the recorded ones)
   * and differentiates CE + weight * sum over rows of -target . log softmax(I),
   * accumulated here by every training forward. */
  int freeze;
  REAL *ftarget[MAXL];
  int64_t ftarget_n[MAXL];
  double distill_loss;
  REAL clamp, mscale, bw;
  double aux_loss;
  int64_t total;
  REAL *p;
  int64_t wte, lm, rl, x0l, smg, sml, bkl;
  layer_off lay[MAXL];
  REAL *cosT, *sinT; /* [S*10][R/2] */
};

MODEL *FN(orc_model_new)(const orc_config *cfg, const REAL *params) {
  MODEL *m = (MODEL *)calloc(1, sizeof(MODEL));
  m->cfg = *cfg;
  m->C = cfg->n_embd;
  m->Hq = cfg->n_head;
  m->Hkv = cfg->n_kv_head;
  m->D = m->C / m->Hq;
  m->R = rotary_dim(cfg);
  m->F = mlp_hidden(cfg);
  m->mla = cfg->mla_latent > 0;
  m->lat = cfg->mla_latent;
  m->rd = cfg->mla_rope_dims;
  m->cd = m->D - m->rd;
  m->E = cfg->n_experts;
  m->K = cfg->experts_per_token;
  m->EH = cfg->expert_hidden;
  m->clamp = R(cfg->moe_clamp);
  m->mscale = R(cfg->moe_scale);
  m->bw = R(cfg->balance_weight);
  m->ratio = cfg->compression_ratio > 1 ? cfg->compression_ratio : 1;
  m->swa = cfg->swa_window > 0 ? cfg->swa_window : 0;
  m->topk = m->ratio > 1 && cfg->sparse_topk > 0 ? cfg->sparse_topk : 0;
  indexer_dims(cfg, &m->idim, &m->ih);
  m->HI = m->idim * m->ih;
  m->ipool = cfg->indexer_pool;
  m->ibudget = indexer_budget(cfg);
  m->iw = R(cfg->indexer_weight > 0 ? cfg->indexer_weight : 1.0f); /* config.go:383-389 */
  m->split = m->ratio > 1 ? ced_split(cfg) : 0;
  m->L = cfg->n_layer;
  m->V = cfg->vocab_size;
  m->PV = padded_vocab(cfg);
  m->S = cfg->sequence_len;
  m->KVW = m->Hkv * m->D;
  m->total = orc_param_total(cfg);
  m->p = (REAL *)malloc(sizeof(REAL) * m->total);
  memcpy(m->p, params, sizeof(REAL) * m->total);
  m->wte = param_offset(cfg, "transformer.wte.weight");
  m->lm = param_offset(cfg, "lm_head.weight");
  m->rl = param_offset(cfg, "resid_lambdas");
  m->x0l = param_offset(cfg, "x0_lambdas");
  m->smg = param_offset(cfg, "smear_gate.weight");
  m->sml = param_offset(cfg, "smear_lambda");
  m->bkl = param_offset(cfg, "backout_lambda");
  int32_t win[MAXL];
  orc_window_sizes(cfg, win);
  char nm[96];
  for (int l = 0; l < m->L; l++) {
    layer_off *o = &m->lay[l];
#define OFF(field, fmt)                      \
  snprintf(nm, 96, fmt, l);                  \
  o->field = param_offset(cfg, nm);
    if (m->mla) {
      OFF(wqd, "transformer.h.%d.attn.mla_q_down.weight");
      OFF(wqu, "transformer.h.%d.attn.mla_q_up.weight");
      OFF(wqr, "transformer.h.%d.attn.mla_q_rope.weight");
      OFF(wkvd, "transformer.h.%d.attn.mla_kv_down.weight");
      OFF(wku, "transformer.h.%d.attn.mla_k_up.weight");
      OFF(wvu, "transformer.h.%d.attn.mla_v_up.weight");
      OFF(wkr, "transformer.h.%d.attn.mla_k_rope.weight");
    } else {
      OFF(wq, "transformer.h.%d.attn.c_q.weight");
      OFF(wk, "transformer.h.%d.attn.c_k.weight");
      OFF(wv, "transformer.h.%d.attn.c_v.weight");
    }
    OFF(wo, "transformer.h.%d.attn.c_proj.weight");
    OFF(wfc, "transformer.h.%d.mlp.c_fc.weight");
    OFF(wproj, "transformer.h.%d.mlp.c_proj.weight");
    if (m->E > 0) {
      OFF(wgate, "transformer.h.%d.mlp.c_gate.weight");
      OFF(wr, "transformer.h.%d.moe.router.weight");
      OFF(rbias, "transformer.h.%d.moe.router_bias");
      OFF(eg, "transformer.h.%d.moe.experts.gate.weight");
      OFF(eu, "transformer.h.%d.moe.experts.up.weight");
      OFF(ed, "transformer.h.%d.moe.experts.down.weight");
    }
    o->mode = m->ratio > 1 ? reuse_mode_at(cfg, l) : REUSE_FULL;
    o->producer = m->ratio > 1 ? reuse_producer(cfg, l) : l;
    if (m->ratio > 1 && o->mode == REUSE_FULL) {
      OFF(wcl, "transformer.h.%d.attn.compress_logits.weight");
      OFF(cbias, "transformer.h.%d.attn.compress_bias");
    }
    o->has_idx = m->topk > 0 && o->mode != REUSE_REUSE;
    if (o->has_idx) {
      OFF(wiq, "transformer.h.%d.attn.indexer_query.weight");
      OFF(wik, "transformer.h.%d.attn.indexer_key.weight");
      OFF(wih, "transformer.h.%d.attn.indexer_heads");
    }
    o->has_ve = !m->mla && has_value_embedding(l, m->L);
    if (o->has_ve) {
      OFF(wve, "transformer.h.%d.attn.ve_gate.weight");
      OFF(ve, "value_embeds.%d.weight");
    }
#undef OFF
    o->window = win[l];
  }
  /* model/rotary.go:16-30 with SequenceLen*10 positions (transformer.go:54) */
  int half = m->R / 2, npos = m->S * ROT_OVER;
  m->cosT = (REAL *)malloc(sizeof(REAL) * npos * half);
  m->sinT = (REAL *)malloc(sizeof(REAL) * npos * half);
  FN(orc_rotary_table)(npos, m->R, m->cosT, m->sinT);
  return m;
}

void FN(orc_model_free)(MODEL *m) {
  if (!m) return;
  for (int l = 0; l < MAXL; l++) free(m->ftarget[l]);
  free(m->p);
  free(m->cosT);
  free(m->sinT);
  free(m);
}

/* ---- primitives ------------------------------------------------------- */

/* kernels/scalar/norm.go:26-40 applied row-wise (model/attention.go:25-29) */
static void rmsnorm_rows(REAL *dst, const REAL *src, int64_t rows, int cols) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; r++) {
    const REAL *s = src + r * cols;
    REAL *d = dst + r * cols;
    double ss = 0;
    for (int c = 0; c < cols; c++) ss += (double)s[c] * (double)s[c];
    REAL ms = R(ss / (double)cols);
    REAL inv = R(1.0 / sqrt((double)ms + (double)NORM_EPS));
    for (int c = 0; c < cols; c++) d[c] = s[c] * inv;
  }
}
/* tensors/backward.go:81-104 */
static void rmsnorm_backward_rows(REAL *dst, const REAL *x, const REAL *g, int64_t rows, int cols) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; r++) {
    const REAL *xr = x + r * cols, *gr = g + r * cols;
    REAL *d = dst + r * cols;
    double ss = 0, dot = 0;
    for (int c = 0; c < cols; c++) {
      ss += (double)xr[c] * (double)xr[c];
      dot += (double)gr[c] * (double)xr[c];
    }
    double ms = ss / (double)cols;
    double rms = sqrt(ms + (double)NORM_EPS);
    double inv = 1.0 / rms;
    double coef = dot / ((double)cols * rms * rms * rms);
    for (int c = 0; c < cols; c++) d[c] = R((double)gr[c] * inv - coef * (double)xr[c]);
  }
}
/* dst[r][o] (= or +=) sum over k ascending of a[r][k] * b[o][k] in float64,
 * for r < rows, o < cols, k < inner (a, b row-major with row lengths lda,
 * ldb; dst row length ldd).  Every entry is one in-order float64 sum; tiles
 * of 64 x 64 entries keep their operand rows in cache, and 2 x 4 entries
 * are summed side by side so that independent adds overlap. */
static void dot_rows(REAL *dst, int64_t ldd, int accumulate, const REAL *a, int64_t lda,
                     const REAL *b, int64_t ldb, int64_t rows, int64_t cols, int64_t inner) {
  const int64_t TR = 64, TC = 64;
  const int64_t nrt = (rows + TR - 1) / TR, nct = (cols + TC - 1) / TC;
#pragma omp parallel for schedule(dynamic)
  for (int64_t t = 0; t < nrt * nct; t++) {
    const int64_t rb = (t / nct) * TR, cb = (t % nct) * TC;
    const int64_t re = rb + TR < rows ? rb + TR : rows, ce = cb + TC < cols ? cb + TC : cols;
    for (int64_t r0 = rb; r0 < re; r0 += 2) {
      const int64_t r1 = r0 + 1 < re ? r0 + 1 : r0;
      const REAL *x0 = a + r0 * lda, *x1 = a + r1 * lda;
      int64_t o = cb;
      for (; o + 4 <= ce; o += 4) {
        const REAL *w0 = b + o * ldb, *w1 = w0 + ldb, *w2 = w1 + ldb, *w3 = w2 + ldb;
        double a00 = 0, a01 = 0, a02 = 0, a03 = 0, a10 = 0, a11 = 0, a12 = 0, a13 = 0;
        for (int64_t k = 0; k < inner; k++) {
          const double u = (double)x0[k], v = (double)x1[k];
          const double b0 = (double)w0[k], b1 = (double)w1[k], b2 = (double)w2[k], b3 = (double)w3[k];
          a00 += u * b0; a01 += u * b1; a02 += u * b2; a03 += u * b3;
          a10 += v * b0; a11 += v * b1; a12 += v * b2; a13 += v * b3;
        }
        REAL *d0 = dst + r0 * ldd + o, *d1 = dst + r1 * ldd + o;
        if (accumulate) {
          d0[0] += R(a00); d0[1] += R(a01); d0[2] += R(a02); d0[3] += R(a03);
          if (r1 != r0) { d1[0] += R(a10); d1[1] += R(a11); d1[2] += R(a12); d1[3] += R(a13); }
        } else {
          d0[0] = R(a00); d0[1] = R(a01); d0[2] = R(a02); d0[3] = R(a03);
          if (r1 != r0) { d1[0] = R(a10); d1[1] = R(a11); d1[2] = R(a12); d1[3] = R(a13); }
        }
      }
      for (; o < ce; o++) {
        const REAL *w = b + o * ldb;
        double a0 = 0, a1 = 0;
        for (int64_t k = 0; k < inner; k++) {
          a0 += (double)x0[k] * (double)w[k];
          a1 += (double)x1[k] * (double)w[k];
        }
        if (accumulate) {
          dst[r0 * ldd + o] += R(a0);
          if (r1 != r0) dst[r1 * ldd + o] += R(a1);
        } else {
          dst[r0 * ldd + o] = R(a0);
          if (r1 != r0) dst[r1 * ldd + o] = R(a1);
        }
      }
    }
  }
}
/* out[rows][outF] = in[rows][inF] . W[outF][inF]^T, float64 accumulation
 * (model/layers/linear.go:32-40 -> kernels/scalar/matmul.go:22-33): each
 * output is one float64 sum over i ascending. */
static void linear_fwd(REAL *out, const REAL *in, const REAL *W, int64_t rows, int inF, int outF) {
  dot_rows(out, outF, 0, in, inF, W, inF, rows, outF, inF);
}
/* dst[cols][rows] = src[rows][cols] */
static void transpose_rows(REAL *dst, const REAL *src, int64_t rows, int64_t cols) {
#pragma omp parallel for schedule(static)
  for (int64_t c0 = 0; c0 < cols; c0 += 32)
    for (int64_t r0 = 0; r0 < rows; r0 += 32)
      for (int64_t c = c0; c < c0 + 32 && c < cols; c++)
        for (int64_t r = r0; r < r0 + 32 && r < rows; r++) dst[c * rows + r] = src[r * cols + c];
}
/* model/layers/linear.go:45-53: dW += g^T x ; dx = g W (float64 accumulation).
 * Each dW entry is one float64 sum over r ascending and each dx entry one
 * over o ascending, as in the reference's loops; transposed copies of g, x
 * and W let those sums run over contiguous memory. */
static void linear_bwd(REAL *dx, REAL *dW, const REAL *x, const REAL *g, const REAL *W,
                       int64_t rows, int inF, int outF) {
  REAL *gT = (REAL *)malloc(sizeof(REAL) * (size_t)rows * outF);
  REAL *xT = (REAL *)malloc(sizeof(REAL) * (size_t)rows * inF);
  if (!gT || !xT) abort();
  transpose_rows(gT, g, rows, outF);
  transpose_rows(xT, x, rows, inF);
  dot_rows(dW, inF, 1, gT, rows, xT, rows, outF, inF, rows);
  free(xT);
  free(gT);
  if (dx) {
    REAL *WT = (REAL *)malloc(sizeof(REAL) * (size_t)outF * inF);
    if (!WT) abort();
    transpose_rows(WT, W, outF, inF);
    dot_rows(dx, inF, 0, g, outF, WT, outF, rows, inF, outF);
    free(WT);
  }
}
static REAL sigmoidR(REAL x) { return R(1.0 / (1.0 + exp(-(double)x))); }

/* model/rotary.go:43-75 (ApplyRotary) for the heads of one token: the
 * trailing R of each head's D channels rotate pairwise with the table row
 * cw/sw (R/2 entries), y1 = x1 cos + x2 sin, y2 = -x1 sin + x2 cos; the
 * leading D-R channels are copied.  sign -1 uses the negated sine table
 * (model/train.go:14-20).  dst may alias src. */
static void rotary_apply(REAL *dst, const REAL *src, int heads, int D, int R, const REAL *cw,
                         const REAL *sw, int sign) {
  int half = R / 2, off = D - R;
  for (int h = 0; h < heads; h++) {
    const REAL *s = src + h * D;
    REAL *d = dst + h * D;
    REAL tmp[1024];
    memcpy(tmp, s, sizeof(REAL) * D);
    for (int j = 0; j < half; j++) {
      REAL x1 = tmp[off + j], x2 = tmp[off + half + j];
      REAL c = cw[j], sn = sign > 0 ? sw[j] : -sw[j];
      d[j + off] = x1 * c + x2 * sn;
      d[off + half + j] = -x1 * sn + x2 * c;
    }
    for (int j = 0; j < off; j++) d[j] = tmp[j];
  }
}
/* The same, exported: the function the model rotates with (pinned by the
 * reference's known answers, model/model_test.go:196-211,283-311). */
void FN(orc_apply_rotary)(REAL *dst, const REAL *src, int heads, int D, int R, const REAL *cw,
                          const REAL *sw) {
  rotary_apply(dst, src, heads, D, R, cw, sw, 1);
}
/* rows of [heads][D] at the given position of the model's table */
static void rope_rows_w(MODEL *m, REAL *dst, const REAL *src, int heads, int D, int pos,
                        int sign) {
  int half = m->R / 2;
  rotary_apply(dst, src, heads, D, m->R, m->cosT + (int64_t)pos * half,
               m->sinT + (int64_t)pos * half, sign);
}
static void rope_row(MODEL *m, REAL *dst, const REAL *src, int heads, int pos, int sign) {
  rope_rows_w(m, dst, src, heads, m->D, pos, sign);
}

/* One (batch, head) attention with the reference mask; scores and
 * probabilities materialized (kernels/scalar/attention.go:16-49). */
static void attn_fwd_full(const REAL *q, const REAL *k, const REAL *v, REAL *out, REAL *lse,
                          int qlen, int klen, int D, int offset, int window) {
  REAL *sc = (REAL *)malloc(sizeof(REAL) * klen);
  for (int qi = 0; qi < qlen; qi++) {
    int qpos = offset + qi;
    REAL mx = 0;
    for (int kj = 0; kj < klen; kj++) {
      double a = 0;
      for (int d = 0; d < D; d++) a += (double)q[qi * D + d] * (double)k[(int64_t)kj * D + d];
      REAL s = R(a);
      if (kj > qpos || (window >= 0 && qpos - kj > window)) s = R(MASKED);
      sc[kj] = s;
      if (kj == 0 || s > mx) mx = s;
    }
    double tot = 0;
    for (int kj = 0; kj < klen; kj++) {
      double e = exp((double)(sc[kj] - mx));
      sc[kj] = R(e);
      tot += e;
    }
    if (lse) lse[qi] = mx + R(log(tot));
    REAL inv = R(1.0 / tot);
    for (int d = 0; d < D; d++) {
      double a = 0;
      for (int kj = 0; kj < klen; kj++) a += (double)sc[kj] * (double)v[(int64_t)kj * D + d];
      out[qi * D + d] = R(a) * inv;
    }
  }
  free(sc);
}
static void attn_key_range(int qpos, int klen, int window, int *lo, int *hi) {
  *hi = qpos < klen - 1 ? qpos : klen - 1;
  *lo = (window >= 0 && qpos - window > 0) ? qpos - window : 0;
}
/* The same over each query's valid keys [lo, hi] only: a masked score is
 * -1e30, below every valid one (the maximum is unchanged), and its
 * exponential and probability are exactly 0, so the sums skip exact zeros.
 * Same results, O(T x window) work. */
static void attn_fwd(const REAL *q, const REAL *k, const REAL *v, REAL *out, REAL *lse, int qlen,
                     int klen, int D, int offset, int window) {
  for (int qi = 0; qi < qlen; qi++) {
    int lo, hi;
    attn_key_range(offset + qi, klen, window, &lo, &hi);
    if (lo > hi) { /* a row with no valid key: the reference's arithmetic */
      attn_fwd_full(q, k, v, out, lse, qlen, klen, D, offset, window);
      return;
    }
  }
  REAL *sc = (REAL *)malloc(sizeof(REAL) * klen);
  for (int qi = 0; qi < qlen; qi++) {
    int lo, hi;
    attn_key_range(offset + qi, klen, window, &lo, &hi);
    REAL mx = 0;
    for (int kj = lo; kj <= hi; kj++) {
      double a = 0;
      for (int d = 0; d < D; d++) a += (double)q[qi * D + d] * (double)k[(int64_t)kj * D + d];
      REAL s = R(a);
      sc[kj] = s;
      if (kj == lo || s > mx) mx = s;
    }
    double tot = 0;
    for (int kj = lo; kj <= hi; kj++) {
      double e = exp((double)(sc[kj] - mx));
      sc[kj] = R(e);
      tot += e;
    }
    if (lse) lse[qi] = mx + R(log(tot));
    REAL inv = R(1.0 / tot);
    for (int d = 0; d < D; d++) {
      double a = 0;
      for (int kj = lo; kj <= hi; kj++) a += (double)sc[kj] * (double)v[(int64_t)kj * D + d];
      out[qi * D + d] = R(a) * inv;
    }
  }
  free(sc);
}
/* kernels/scalar/attention.go:145-205, gradients accumulated. */
static void attn_bwd_corr(const REAL *q, const REAL *k, const REAL *v, const REAL *dout,
                          const REAL *lse, const REAL *corr, REAL *dq, REAL *dk, REAL *dv,
                          int qlen, int klen, int D, int offset, int window);
static void attn_bwd(const REAL *q, const REAL *k, const REAL *v, const REAL *dout,
                     const REAL *lse, REAL *dq, REAL *dk, REAL *dv, int qlen, int klen, int D,
                     int offset, int window) {
  attn_bwd_corr(q, k, v, dout, lse, NULL, dq, dk, dv, qlen, klen, D, offset, window);
}
/* kernels/scalar/attention.go:145-205 over every (query, key) pair, the
 * masked ones included; corr, when given, replaces the row sum of dP*P (the
 * merged-branch row correction dO.O, model/train.go:211-226). */
static void attn_bwd_full(const REAL *q, const REAL *k, const REAL *v, const REAL *dout,
                          const REAL *lse, const REAL *corr, REAL *dq, REAL *dk, REAL *dv,
                          int qlen, int klen, int D, int offset, int window) {
  REAL *P = (REAL *)malloc(sizeof(REAL) * (int64_t)qlen * klen);
  REAL *dS = (REAL *)malloc(sizeof(REAL) * (int64_t)qlen * klen);
  for (int qi = 0; qi < qlen; qi++) {
    int qpos = offset + qi;
    for (int kj = 0; kj < klen; kj++) {
      double a = 0;
      for (int d = 0; d < D; d++) a += (double)q[qi * D + d] * (double)k[(int64_t)kj * D + d];
      REAL s = R(a);
      if (kj > qpos || (window >= 0 && qpos - kj > window)) s = R(MASKED);
      P[(int64_t)qi * klen + kj] = s <= R(MASKED) ? R(0) : R(exp((double)(s - lse[qi])));
    }
  }
  for (int kj = 0; kj < klen; kj++)
    for (int d = 0; d < D; d++) {
      double a = 0;
      for (int qi = 0; qi < qlen; qi++) a += (double)P[(int64_t)qi * klen + kj] * (double)dout[qi * D + d];
      dv[(int64_t)kj * D + d] += R(a);
    }
  for (int qi = 0; qi < qlen; qi++) {
    double rd = 0;
    REAL *dp = dS + (int64_t)qi * klen;
    for (int kj = 0; kj < klen; kj++) {
      double a = 0;
      for (int d = 0; d < D; d++) a += (double)dout[qi * D + d] * (double)v[(int64_t)kj * D + d];
      dp[kj] = R(a);
      rd += (double)dp[kj] * (double)P[(int64_t)qi * klen + kj];
    }
    if (corr) rd = (double)corr[qi];
    for (int kj = 0; kj < klen; kj++)
      dp[kj] = R((double)P[(int64_t)qi * klen + kj] * ((double)dp[kj] - rd));
  }
  for (int qi = 0; qi < qlen; qi++)
    for (int d = 0; d < D; d++) {
      double a = 0;
      for (int kj = 0; kj < klen; kj++) a += (double)dS[(int64_t)qi * klen + kj] * (double)k[(int64_t)kj * D + d];
      dq[qi * D + d] += R(a);
    }
  for (int kj = 0; kj < klen; kj++)
    for (int d = 0; d < D; d++) {
      double a = 0;
      for (int qi = 0; qi < qlen; qi++) a += (double)dS[(int64_t)qi * klen + kj] * (double)q[qi * D + d];
      dk[(int64_t)kj * D + d] += R(a);
    }
  free(P);
  free(dS);
}

/* corr, when given, replaces the row sum of dP*P (the merged-branch row
 * correction dO.O, model/train.go:211-226).
 * The reference computes every (query, key) pair and masks the invalid ones
 * to -1e30, whose probability is exactly 0, so every sum below gets exact
 * zeros from them; those terms are skipped here (each query's valid keys
 * are the range [lo, hi]), and the sums over queries (dv, dk) accumulate in
 * float64 per element with the queries in ascending order, as the
 * reference's loops add them.  Same results, O(T x window) work. */
static void attn_bwd_corr(const REAL *q, const REAL *k, const REAL *v, const REAL *dout,
                          const REAL *lse, const REAL *corr, REAL *dq, REAL *dk, REAL *dv,
                          int qlen, int klen, int D, int offset, int window) {
  for (int qi = 0; qi < qlen; qi++) {
    int lo, hi;
    attn_key_range(offset + qi, klen, window, &lo, &hi);
    if (lo > hi) { /* no valid key: the reference's arithmetic on the masked row */
      attn_bwd_full(q, k, v, dout, lse, corr, dq, dk, dv, qlen, klen, D, offset, window);
      return;
    }
  }
  double *adv = (double *)calloc((size_t)klen * D, sizeof(double));
  double *adk = (double *)calloc((size_t)klen * D, sizeof(double));
  double *P = (double *)malloc(sizeof(double) * klen);
  double *dp = (double *)malloc(sizeof(double) * klen);
  for (int qi = 0; qi < qlen; qi++) {
    int lo, hi;
    attn_key_range(offset + qi, klen, window, &lo, &hi);
    for (int kj = lo; kj <= hi; kj++) {
      double a = 0;
      for (int d = 0; d < D; d++) a += (double)q[qi * D + d] * (double)k[(int64_t)kj * D + d];
      REAL s = R(a);
      P[kj] = (double)(s <= R(MASKED) ? R(0) : R(exp((double)(s - lse[qi]))));
    }
    for (int kj = lo; kj <= hi; kj++)
      for (int d = 0; d < D; d++) adv[(int64_t)kj * D + d] += P[kj] * (double)dout[qi * D + d];
    double rd = 0;
    for (int kj = lo; kj <= hi; kj++) {
      double a = 0;
      for (int d = 0; d < D; d++) a += (double)dout[qi * D + d] * (double)v[(int64_t)kj * D + d];
      dp[kj] = (double)R(a);
      rd += dp[kj] * P[kj];
    }
    if (corr) rd = (double)corr[qi];
    for (int kj = lo; kj <= hi; kj++) dp[kj] = (double)R(P[kj] * (dp[kj] - rd));
    for (int d = 0; d < D; d++) {
      double a = 0;
      for (int kj = lo; kj <= hi; kj++) a += dp[kj] * (double)k[(int64_t)kj * D + d];
      dq[qi * D + d] += R(a);
    }
    for (int kj = lo; kj <= hi; kj++)
      for (int d = 0; d < D; d++) adk[(int64_t)kj * D + d] += dp[kj] * (double)q[qi * D + d];
  }
  for (int64_t i = 0; i < (int64_t)klen * D; i++) {
    dv[i] += R(adv[i]);
    dk[i] += R(adk[i]);
  }
  free(adv);
  free(adk);
  free(P);
  free(dp);
}
/* tensors/math.go:38-45: z = 15*tanh(y*(1/15)) with the float32 reciprocal. */
static REAL softcap(REAL y) {
  REAL inv = R(1) / R(SOFTCAP);
  REAL t = y * inv;
  return R(tanh((double)t)) * R(SOFTCAP);
}

/* ---- KV cache (model/kvcache.go:10-140) -------------------------------- */
typedef struct {
  int B, maxSeq, pos, has_prev;
  REAL *k, *v;  /* [L][B][Hkv][maxSeq][D] (dense) */
  REAL *lat;    /* [L][B][maxSeq][lat]      (MLA latent, kvcache.go:224-274) */
  REAL *rk;     /* [L][B][maxSeq][Hkv*rd]   (MLA rotary key) */
  REAL *prev;   /* [B][C] */
  /* HCA (kvcache.go:142-220): tail buffer of the current block (hidden,
   * key and value rows), compressed blocks and counts; CSA indexer key
   * projections of the compressed blocks (kvcache.go:197-220) */
  int maxBlocks;
  REAL *tailh;  /* [L][B][ratio][C] */
  REAL *tailk, *tailv; /* [L][B][Hkv][ratio][D] */
  int *taillen; /* [L] (all rows advance together) */
  REAL *ck, *cv;  /* [L][B][Hkv][maxBlocks][D] */
  int *ccount;  /* [L][B] (a Reindex layer counts its cached indexer keys) */
  REAL *ikc;    /* [L][B][Hkv][maxBlocks][HI] */
} kvcache;

static kvcache *cache_new(MODEL *m, int B, int maxSeq) {
  kvcache *c = (kvcache *)calloc(1, sizeof(kvcache));
  c->B = B;
  c->maxSeq = maxSeq;
  if (m->ratio > 1) {
    c->maxBlocks = maxSeq / m->ratio + 1;
    c->tailh = (REAL *)calloc((size_t)m->L * B * m->ratio * m->C, sizeof(REAL));
    c->tailk = (REAL *)calloc((size_t)m->L * B * m->Hkv * m->ratio * m->D, sizeof(REAL));
    c->tailv = (REAL *)calloc((size_t)m->L * B * m->Hkv * m->ratio * m->D, sizeof(REAL));
    c->taillen = (int *)calloc(m->L, sizeof(int));
    if (m->topk > 0)
      c->ikc = (REAL *)calloc((size_t)m->L * B * m->Hkv * c->maxBlocks * m->HI, sizeof(REAL));
    c->ck = (REAL *)calloc((size_t)m->L * B * m->Hkv * c->maxBlocks * m->D, sizeof(REAL));
    c->cv = (REAL *)calloc((size_t)m->L * B * m->Hkv * c->maxBlocks * m->D, sizeof(REAL));
    c->ccount = (int *)calloc((size_t)m->L * B, sizeof(int));
  }
  if (m->mla) {
    c->lat = (REAL *)calloc((size_t)m->L * B * maxSeq * m->lat, sizeof(REAL));
    c->rk = (REAL *)calloc((size_t)m->L * B * maxSeq * m->Hkv * m->rd, sizeof(REAL));
  } else {
    size_t n = (size_t)m->L * B * m->Hkv * maxSeq * m->D;
    c->k = (REAL *)calloc(n, sizeof(REAL));
    c->v = (REAL *)calloc(n, sizeof(REAL));
  }
  c->prev = (REAL *)calloc((size_t)B * m->C, sizeof(REAL));
  return c;
}
static void cache_free(kvcache *c) {
  free(c->k);
  free(c->v);
  free(c->lat);
  free(c->rk);
  free(c->tailh); free(c->tailk); free(c->tailv); free(c->taillen); free(c->ck); free(c->cv);
  free(c->ccount); free(c->ikc);
  free(c->prev);
  free(c);
}
static REAL *cache_k(MODEL *m, kvcache *c, int l, int b, int h) {
  return c->k + ((((size_t)l * c->B + b) * m->Hkv + h) * c->maxSeq) * m->D;
}
static REAL *cache_v(MODEL *m, kvcache *c, int l, int b, int h) {
  return c->v + ((((size_t)l * c->B + b) * m->Hkv + h) * c->maxSeq) * m->D;
}
static REAL *cache_lat(MODEL *m, kvcache *c, int l, int b) {
  return c->lat + (((size_t)l * c->B + b) * c->maxSeq) * m->lat;
}
static REAL *cache_rk(MODEL *m, kvcache *c, int l, int b) {
  return c->rk + (((size_t)l * c->B + b) * c->maxSeq) * m->Hkv * m->rd;
}
/* model/kvcache.go:383-448 (PrefillFrom) for a batch-1 source. */
static void prefill_from(MODEL *m, kvcache *dst, kvcache *src) {
  int pos = src->pos;
  for (int l = 0; l < m->L && m->mla; l++)
    for (int b = 0; b < dst->B; b++) {
      memcpy(cache_lat(m, dst, l, b), cache_lat(m, src, l, 0), sizeof(REAL) * pos * m->lat);
      memcpy(cache_rk(m, dst, l, b), cache_rk(m, src, l, 0), sizeof(REAL) * pos * m->Hkv * m->rd);
    }
  for (int l = 0; l < m->L && !m->mla; l++)
    for (int b = 0; b < dst->B; b++)
      for (int h = 0; h < m->Hkv; h++) {
        memcpy(cache_k(m, dst, l, b, h), cache_k(m, src, l, 0, h), sizeof(REAL) * pos * m->D);
        memcpy(cache_v(m, dst, l, b, h), cache_v(m, src, l, 0, h), sizeof(REAL) * pos * m->D);
      }
  if (m->ratio > 1) { /* PrefillFrom copies the compression state too */
    const int RD = m->ratio * m->D;
    for (int l = 0; l < m->L; l++) {
      dst->taillen[l] = src->taillen[l];
      for (int b = 0; b < dst->B; b++) {
        memcpy(dst->tailh + ((size_t)l * dst->B + b) * m->ratio * m->C,
               src->tailh + (size_t)l * m->ratio * m->C, sizeof(REAL) * m->ratio * m->C);
        dst->ccount[l * dst->B + b] = src->ccount[l];
        for (int h = 0; h < m->Hkv; h++) {
          size_t so = (((size_t)l * src->B) * m->Hkv + h) * src->maxBlocks;
          size_t dd = (((size_t)l * dst->B + b) * m->Hkv + h) * dst->maxBlocks;
          size_t to = ((size_t)l * src->B * m->Hkv + h) * RD;
          size_t td = (((size_t)l * dst->B + b) * m->Hkv + h) * RD;
          memcpy(dst->tailk + td, src->tailk + to, sizeof(REAL) * RD);
          memcpy(dst->tailv + td, src->tailv + to, sizeof(REAL) * RD);
          memcpy(dst->ck + dd * m->D, src->ck + so * m->D, sizeof(REAL) * src->ccount[l] * m->D);
          memcpy(dst->cv + dd * m->D, src->cv + so * m->D, sizeof(REAL) * src->ccount[l] * m->D);
          if (m->topk > 0)
            memcpy(dst->ikc + dd * m->HI, src->ikc + so * m->HI, sizeof(REAL) * src->ccount[l] * m->HI);
        }
      }
    }
  }
  dst->pos = pos;
  if (src->has_prev) {
    for (int b = 0; b < dst->B; b++) memcpy(dst->prev + (size_t)b * m->C, src->prev, sizeof(REAL) * m->C);
    dst->has_prev = 1;
  }
}

/* ---- DeepSeekMoE routed experts (model/moe.go) ----------------------- */
typedef struct moe_ctx {
  int64_t rows, NK;
  REAL *probs;       /* [rows][E] router softmax */
  int64_t *counts;   /* [E] tokens per expert */
  int64_t *offsets;  /* [E] first gathered row of each expert */
  int64_t *grow;     /* [NK] gathered pair -> token row */
  REAL *gw;          /* [NK] router probability of the pair */
  REAL *xg, *gg, *ug, *hg, *yg; /* gathered input, gate, up, hidden, output */
  double *bal_gp;    /* [rows][E] balance-loss gradient wrt probs, or NULL */
  double bal_loss;
} moe_ctx;

static void moe_ctx_free(moe_ctx *c) {
  if (!c) return;
  free(c->probs); free(c->counts); free(c->offsets); free(c->grow); free(c->gw);
  free(c->xg); free(c->gg); free(c->ug); free(c->hg); free(c->yg); free(c->bal_gp);
  free(c);
}

/* kernels/scalar/elementwise.go:85-134 (clamped SwiGLU and its backward) */
static REAL swiglu_value(REAL g, REAL u, REAL clamp, REAL *gm, REAL *um, REAL *sg_out) {
  *gm = R(1);
  *um = R(1);
  if (clamp > 0 && g >= clamp) { g = clamp; *gm = R(0); }
  if (clamp > 0) {
    if (u > clamp) { u = clamp; *um = R(0); }
    else if (u < -clamp) { u = -clamp; *um = R(0); }
  }
  REAL sg = R(1.0 / (1.0 + exp(-(double)g)));
  if (sg_out) *sg_out = sg;
  return g * sg * u;
}
static void swiglu_fwd(REAL *dst, const REAL *g, const REAL *u, REAL clamp, int64_t n) {
  for (int64_t i = 0; i < n; i++) {
    REAL gm, um;
    dst[i] = swiglu_value(g[i], u[i], clamp, &gm, &um, NULL);
  }
}
static void swiglu_bwd(REAL *dg, REAL *du, const REAL *g, const REAL *u, const REAL *dout,
                       REAL clamp, int64_t n) {
  for (int64_t i = 0; i < n; i++) {
    REAL gm, um, sg;
    REAL gv = g[i], uv = u[i];
    swiglu_value(gv, uv, clamp, &gm, &um, &sg);
    if (clamp > 0 && gv >= clamp) gv = clamp;
    if (clamp > 0) uv = uv > clamp ? clamp : (uv < -clamp ? -clamp : uv);
    REAL silu = gv * sg;
    REAL sgrad = sg * (R(1) + gv * (R(1) - sg));
    dg[i] = dout[i] * uv * sgrad * gm;
    du[i] = dout[i] * silu * um;
  }
}

/* GroupedMatMulTransposed for one expert's rows (kernels/scalar/moe.go:54-73,
 * a running REAL sum in inner order). */
static void expert_matmul(REAL *dst, const REAL *in, const REAL *W, int64_t rows, int cols,
                          int inner) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; r++)
    for (int c = 0; c < cols; c++) {
      REAL t = 0;
      const REAL *x = in + r * inner, *w = W + (int64_t)c * inner;
      for (int i = 0; i < inner; i++) t += x[i] * w[i];
      dst[r * cols + c] = t;
    }
}

/* MoE.forward (model/moe.go:118-198) with MoEGateTopK (kernels/scalar/moe.go:
 * 8-52) and sequenceBalance (moe.go:276-326).  out[rows][C] is overwritten
 * with the routed contribution; seqlen > 0 (training) also computes the
 * balance loss; ctx_out, when given, keeps the activations. */
static void moe_forward(MODEL *m, const layer_off *lo, const REAL *x, int64_t rows, int seqlen,
                        REAL *out, moe_ctx **ctx_out) {
  const int C = m->C, E = m->E, K = m->K, EH = m->EH;
  const REAL *P = m->p;
  moe_ctx *c = (moe_ctx *)calloc(1, sizeof(moe_ctx));
  c->rows = rows;
  c->NK = rows * K;
  REAL *logits = (REAL *)malloc(sizeof(REAL) * rows * E);
  linear_fwd(logits, x, P + lo->wr, rows, C, E);
  c->probs = (REAL *)malloc(sizeof(REAL) * rows * E);
  int32_t *sel = (int32_t *)malloc(sizeof(int32_t) * rows * K);
  for (int64_t r = 0; r < rows; r++) {
    const REAL *lg = logits + r * E;
    REAL *pr = c->probs + r * E;
    REAL mx = lg[0]; /* SoftmaxLastDim (scalar/norm.go:7-23) */
    for (int e = 1; e < E; e++)
      if (lg[e] > mx) mx = lg[e];
    double tot = 0;
    for (int e = 0; e < E; e++) {
      double ex = exp((double)(lg[e] - mx));
      pr[e] = R(ex);
      tot += ex;
    }
    REAL inv = R(1.0 / tot);
    for (int e = 0; e < E; e++) pr[e] = pr[e] * inv;
    REAL work[256]; /* TopKIndices on logits + bias, ties to the smaller index */
    for (int e = 0; e < E; e++) work[e] = lg[e] + P[lo->rbias + e];
    for (int k = 0; k < K; k++) {
      int best = 0;
      for (int e = 1; e < E; e++)
        if (work[e] > work[best]) best = e;
      sel[r * K + k] = best;
      work[best] = R(-INFINITY);
    }
  }
  free(logits);
  c->counts = (int64_t *)calloc(E, sizeof(int64_t));
  c->offsets = (int64_t *)calloc(E, sizeof(int64_t));
  for (int64_t i = 0; i < rows * K; i++) c->counts[sel[i]]++;
  for (int e = 1; e < E; e++) c->offsets[e] = c->offsets[e - 1] + c->counts[e - 1];
  int64_t NK = c->NK, *fill = (int64_t *)calloc(E, sizeof(int64_t));
  c->grow = (int64_t *)malloc(sizeof(int64_t) * NK);
  c->gw = (REAL *)malloc(sizeof(REAL) * NK);
  c->xg = (REAL *)malloc(sizeof(REAL) * NK * C);
  for (int64_t r = 0; r < rows; r++)
    for (int k = 0; k < K; k++) {
      int e = sel[r * K + k];
      int64_t pos = c->offsets[e] + fill[e]++;
      memcpy(c->xg + pos * C, x + r * C, sizeof(REAL) * C);
      c->grow[pos] = r;
      c->gw[pos] = c->probs[r * E + e];
    }
  free(fill);
  c->gg = (REAL *)malloc(sizeof(REAL) * NK * EH);
  c->ug = (REAL *)malloc(sizeof(REAL) * NK * EH);
  c->hg = (REAL *)malloc(sizeof(REAL) * NK * EH);
  c->yg = (REAL *)malloc(sizeof(REAL) * NK * C);
  for (int e = 0; e < E; e++) {
    int64_t o = c->offsets[e], n = c->counts[e];
    if (!n) continue;
    expert_matmul(c->gg + o * EH, c->xg + o * C, P + lo->eg + (int64_t)e * EH * C, n, EH, C);
    expert_matmul(c->ug + o * EH, c->xg + o * C, P + lo->eu + (int64_t)e * EH * C, n, EH, C);
  }
  swiglu_fwd(c->hg, c->gg, c->ug, m->clamp, NK * EH);
  for (int e = 0; e < E; e++) {
    int64_t o = c->offsets[e], n = c->counts[e];
    if (!n) continue;
    expert_matmul(c->yg + o * C, c->hg + o * EH, P + lo->ed + (int64_t)e * C * EH, n, C, EH);
  }
  memset(out, 0, sizeof(REAL) * rows * C);
  for (int64_t i = 0; i < NK; i++) {
    REAL w = c->gw[i] * m->mscale;
    REAL *dst = out + c->grow[i] * C;
    const REAL *y = c->yg + i * C;
    for (int j = 0; j < C; j++) dst[j] += w * y[j];
  }
  /* sequenceBalance (moe.go:276-326) */
  if (m->bw > 0 && seqlen > 0 && rows > 0 && rows % seqlen == 0) {
    int64_t S = rows / seqlen;
    double tc = (double)seqlen;
    double *cnt = (double *)calloc((size_t)S * E, sizeof(double));
    double *sum = (double *)calloc((size_t)S * E, sizeof(double));
    for (int64_t i = 0; i < rows * K; i++) cnt[((i / K) / seqlen) * E + sel[i]] += 1.0;
    for (int64_t r = 0; r < rows; r++)
      for (int e = 0; e < E; e++) sum[(r / seqlen) * E + e] += (double)c->probs[r * E + e];
    double ss = (double)E / ((double)K * tc), loss = 0;
    for (int64_t sq = 0; sq < S; sq++)
      for (int e = 0; e < E; e++) loss += ss * cnt[sq * E + e] * (sum[sq * E + e] / tc);
    c->bal_loss = (double)m->bw * loss / (double)S;
    double coef = (double)m->bw / ((double)S * tc);
    c->bal_gp = (double *)malloc(sizeof(double) * rows * E);
    for (int64_t r = 0; r < rows; r++)
      for (int e = 0; e < E; e++) c->bal_gp[r * E + e] = coef * ss * cnt[(r / seqlen) * E + e];
    free(cnt);
    free(sum);
  }
  free(sel);
  if (ctx_out) *ctx_out = c;
  else moe_ctx_free(c);
}

/* MoE.backwardTraining (model/moe.go:203-267): gx[rows][C] is overwritten with
 * the gradient wrt the MoE input; expert and router gradients accumulate. */
static void moe_backward(MODEL *m, const layer_off *lo, const moe_ctx *c, const REAL *x,
                         const REAL *gout, REAL *gx, REAL *G) {
  const int C = m->C, E = m->E, EH = m->EH;
  const int64_t rows = c->rows;
  const REAL *P = m->p;
  memset(gx, 0, sizeof(REAL) * rows * C);
  double *gp = (double *)calloc((size_t)rows * E, sizeof(double));
  for (int e = 0; e < E; e++) {
    int64_t o = c->offsets[e], n = c->counts[e];
    if (!n) continue;
    REAL *gy = (REAL *)malloc(sizeof(REAL) * n * C);
    for (int64_t i = 0; i < n; i++) {
      int64_t row = c->grow[o + i];
      REAL w = c->gw[o + i] * m->mscale;
      double dot = 0;
      for (int j = 0; j < C; j++) {
        REAL g = gout[row * C + j];
        gy[i * C + j] = g * w;
        dot += (double)g * (double)c->yg[(o + i) * C + j];
      }
      gp[row * E + e] += dot * (double)m->mscale;
    }
    REAL *gh = (REAL *)malloc(sizeof(REAL) * n * EH);
    linear_bwd(gh, G + lo->ed + (int64_t)e * C * EH, c->hg + o * EH, gy, P + lo->ed + (int64_t)e * C * EH,
               n, EH, C);
    REAL *dg = (REAL *)malloc(sizeof(REAL) * n * EH), *du = (REAL *)malloc(sizeof(REAL) * n * EH);
    swiglu_bwd(dg, du, c->gg + o * EH, c->ug + o * EH, gh, m->clamp, n * EH);
    REAL *fg = (REAL *)malloc(sizeof(REAL) * n * C), *fu = (REAL *)malloc(sizeof(REAL) * n * C);
    linear_bwd(fg, G + lo->eg + (int64_t)e * EH * C, c->xg + o * C, dg, P + lo->eg + (int64_t)e * EH * C,
               n, C, EH);
    linear_bwd(fu, G + lo->eu + (int64_t)e * EH * C, c->xg + o * C, du, P + lo->eu + (int64_t)e * EH * C,
               n, C, EH);
    for (int64_t i = 0; i < n; i++) {
      REAL *dst = gx + c->grow[o + i] * C;
      for (int j = 0; j < C; j++) dst[j] += fg[i * C + j] + fu[i * C + j];
    }
    free(gy); free(gh); free(dg); free(du); free(fg); free(fu);
  }
  if (c->bal_gp)
    for (int64_t i = 0; i < rows * E; i++) gp[i] += c->bal_gp[i];
  REAL *gl = (REAL *)malloc(sizeof(REAL) * rows * E);
  for (int64_t r = 0; r < rows; r++) {
    double dot = 0;
    for (int e = 0; e < E; e++) dot += (double)c->probs[r * E + e] * gp[r * E + e];
    for (int e = 0; e < E; e++) {
      double p = (double)c->probs[r * E + e];
      gl[r * E + e] = R(p * (gp[r * E + e] - dot));
    }
  }
  REAL *gr = (REAL *)malloc(sizeof(REAL) * rows * C);
  linear_bwd(gr, G + lo->wr, x, gl, P + lo->wr, rows, C, E);
  for (int64_t i = 0; i < rows * C; i++) gx[i] = gx[i] + gr[i];
  free(gr); free(gl); free(gp);
}

/* ---- Multi-head latent attention (model/mla.go) ------------------------ */

/* mlaProjectHeads (mla.go:106-122): q [N][Hq][D] = [QueryUp.QueryDown.h |
 * QueryRope.h], k [N][Hkv][D] = [KeyUp.KVDown.h | KeyRope.h], v = ValueUp.
 * KVDown.h; the query and key latents are returned for the backward. */
static void mla_project(MODEL *m, const layer_off *lo, const REAL *h, int64_t N, REAL *q, REAL *k,
                        REAL *v, REAL **ql_out, REAL **kvl_out) {
  const int C = m->C, Hq = m->Hq, Hkv = m->Hkv, D = m->D, lat = m->lat, rd = m->rd, cd = m->cd;
  const REAL *P = m->p;
  REAL *ql = (REAL *)malloc(sizeof(REAL) * N * lat), *kvl = (REAL *)malloc(sizeof(REAL) * N * lat);
  REAL *qc = (REAL *)malloc(sizeof(REAL) * N * Hq * cd), *qr = (REAL *)malloc(sizeof(REAL) * N * Hq * rd);
  REAL *kc = (REAL *)malloc(sizeof(REAL) * N * Hkv * cd), *kr = (REAL *)malloc(sizeof(REAL) * N * Hkv * rd);
  linear_fwd(ql, h, P + lo->wqd, N, C, lat);
  linear_fwd(qc, ql, P + lo->wqu, N, lat, Hq * cd);
  linear_fwd(qr, h, P + lo->wqr, N, C, Hq * rd);
  linear_fwd(kvl, h, P + lo->wkvd, N, C, lat);
  linear_fwd(kc, kvl, P + lo->wku, N, lat, Hkv * cd);
  linear_fwd(kr, h, P + lo->wkr, N, C, Hkv * rd);
  linear_fwd(v, kvl, P + lo->wvu, N, lat, Hkv * D);
  for (int64_t n = 0; n < N; n++) { /* concatHeads (mla.go:150-160) */
    for (int hh = 0; hh < Hq; hh++) {
      memcpy(q + (n * Hq + hh) * D, qc + (n * Hq + hh) * cd, sizeof(REAL) * cd);
      memcpy(q + (n * Hq + hh) * D + cd, qr + (n * Hq + hh) * rd, sizeof(REAL) * rd);
    }
    for (int hh = 0; hh < Hkv; hh++) {
      memcpy(k + (n * Hkv + hh) * D, kc + (n * Hkv + hh) * cd, sizeof(REAL) * cd);
      memcpy(k + (n * Hkv + hh) * D + cd, kr + (n * Hkv + hh) * rd, sizeof(REAL) * rd);
    }
  }
  free(qc); free(qr); free(kc); free(kr);
  *ql_out = ql;
  *kvl_out = kvl;
}

/* mlaProjectBackward (mla.go:126-146) from the post-rotary-backward q/k
 * gradients dq [N][Hq][D], dk [N][Hkv][D] and dv [N][Hkv][D]; dh is
 * overwritten with the gradient wrt the attention input. */
static void mla_project_backward(MODEL *m, const layer_off *lo, const REAL *h, const REAL *ql,
                                 const REAL *kvl, const REAL *dq, const REAL *dk, const REAL *dv,
                                 int64_t N, REAL *dh, REAL *G) {
  const int C = m->C, Hq = m->Hq, Hkv = m->Hkv, D = m->D, lat = m->lat, rd = m->rd, cd = m->cd;
  const REAL *P = m->p;
  REAL *qc = (REAL *)malloc(sizeof(REAL) * N * Hq * cd), *qr = (REAL *)malloc(sizeof(REAL) * N * Hq * rd);
  REAL *kc = (REAL *)malloc(sizeof(REAL) * N * Hkv * cd), *kr = (REAL *)malloc(sizeof(REAL) * N * Hkv * rd);
  for (int64_t n = 0; n < N; n++) { /* splitHeads (mla.go:163-170) */
    for (int hh = 0; hh < Hq; hh++) {
      memcpy(qc + (n * Hq + hh) * cd, dq + (n * Hq + hh) * D, sizeof(REAL) * cd);
      memcpy(qr + (n * Hq + hh) * rd, dq + (n * Hq + hh) * D + cd, sizeof(REAL) * rd);
    }
    for (int hh = 0; hh < Hkv; hh++) {
      memcpy(kc + (n * Hkv + hh) * cd, dk + (n * Hkv + hh) * D, sizeof(REAL) * cd);
      memcpy(kr + (n * Hkv + hh) * rd, dk + (n * Hkv + hh) * D + cd, sizeof(REAL) * rd);
    }
  }
  REAL *dql = (REAL *)malloc(sizeof(REAL) * N * lat), *dkvl = (REAL *)malloc(sizeof(REAL) * N * lat);
  REAL *t = (REAL *)malloc(sizeof(REAL) * N * (lat > C ? lat : C));
  linear_bwd(dql, G + lo->wqu, ql, qc, P + lo->wqu, N, lat, Hq * cd);
  linear_bwd(dh, G + lo->wqd, h, dql, P + lo->wqd, N, C, lat);
  linear_bwd(t, G + lo->wqr, h, qr, P + lo->wqr, N, C, Hq * rd);
  for (int64_t i = 0; i < N * C; i++) dh[i] = dh[i] + t[i];
  linear_bwd(dkvl, G + lo->wku, kvl, kc, P + lo->wku, N, lat, Hkv * cd);
  linear_bwd(t, G + lo->wvu, kvl, dv, P + lo->wvu, N, lat, Hkv * D);
  for (int64_t i = 0; i < N * lat; i++) dkvl[i] = dkvl[i] + t[i];
  linear_bwd(t, G + lo->wkvd, h, dkvl, P + lo->wkvd, N, C, lat);
  for (int64_t i = 0; i < N * C; i++) dh[i] = dh[i] + t[i];
  linear_bwd(t, G + lo->wkr, h, kr, P + lo->wkr, N, C, Hkv * rd);
  for (int64_t i = 0; i < N * C; i++) dh[i] = dh[i] + t[i];
  free(qc); free(qr); free(kc); free(kr); free(dql); free(dkvl); free(t);
}

/* mlaForwardInference (mla.go:185-279): absorbed attention against the
 * latent cache for T new tokens at cache->pos; o [N][Hq][D] receives the
 * per-head outputs before the output projection. */
static void mla_decode_attention(MODEL *m, const layer_off *lo, int l, const REAL *h, int B, int T,
                                 kvcache *cache, REAL *o) {
  const int C = m->C, Hq = m->Hq, Hkv = m->Hkv, D = m->D, lat = m->lat, rd = m->rd, cd = m->cd;
  const int64_t N = (int64_t)B * T;
  const int hd = lat + rd, ratio = Hq / Hkv, offset = cache->pos, count = cache->pos + T;
  const REAL *P = m->p;
  REAL *ql = (REAL *)malloc(sizeof(REAL) * N * lat), *kvl = (REAL *)malloc(sizeof(REAL) * N * lat);
  REAL *qc = (REAL *)malloc(sizeof(REAL) * N * Hq * cd), *qr = (REAL *)malloc(sizeof(REAL) * N * Hq * rd);
  REAL *kr = (REAL *)malloc(sizeof(REAL) * N * Hkv * rd);
  linear_fwd(ql, h, P + lo->wqd, N, C, lat);
  linear_fwd(qc, ql, P + lo->wqu, N, lat, Hq * cd);
  linear_fwd(qr, h, P + lo->wqr, N, C, Hq * rd);
  linear_fwd(kvl, h, P + lo->wkvd, N, C, lat);
  linear_fwd(kr, h, P + lo->wkr, N, C, Hkv * rd);
  for (int b = 0; b < B; b++)
    for (int t = 0; t < T; t++) {
      int64_t n = (int64_t)b * T + t;
      rope_rows_w(m, qr + n * Hq * rd, qr + n * Hq * rd, Hq, rd, offset + t, 1);
      rope_rows_w(m, kr + n * Hkv * rd, kr + n * Hkv * rd, Hkv, rd, offset + t, 1);
      memcpy(cache_lat(m, cache, l, b) + (int64_t)(offset + t) * lat, kvl + n * lat, sizeof(REAL) * lat);
      memcpy(cache_rk(m, cache, l, b) + (int64_t)(offset + t) * Hkv * rd, kr + n * Hkv * rd,
             sizeof(REAL) * Hkv * rd);
    }
  const REAL *ku = P + lo->wku, *vu = P + lo->wvu;
#pragma omp parallel for schedule(dynamic)
  for (int bh = 0; bh < B * Hq; bh++) {
    int b = bh / Hq, hq = bh % Hq, hk = hq / ratio;
    REAL *query = (REAL *)malloc(sizeof(REAL) * T * hd);
    REAL *key = (REAL *)malloc(sizeof(REAL) * (int64_t)count * hd);
    REAL *val = (REAL *)malloc(sizeof(REAL) * (int64_t)count * hd);
    REAL *ao = (REAL *)malloc(sizeof(REAL) * T * hd);
    REAL *lse = (REAL *)malloc(sizeof(REAL) * T);
    for (int t = 0; t < T; t++) {
      const REAL *qcr = qc + (((int64_t)b * T + t) * Hq + hq) * cd;
      for (int rk = 0; rk < lat; rk++) {
        REAL sum = 0; /* a running float32 sum, as mla.go:239-242 */
        for (int ch = 0; ch < cd; ch++) sum += qcr[ch] * ku[(int64_t)(hk * cd + ch) * lat + rk];
        query[t * hd + rk] = sum;
      }
      memcpy(query + t * hd + lat, qr + (((int64_t)b * T + t) * Hq + hq) * rd, sizeof(REAL) * rd);
    }
    const REAL *lc = cache_lat(m, cache, l, b), *rc = cache_rk(m, cache, l, b);
    for (int j = 0; j < count; j++) {
      memcpy(key + (int64_t)j * hd, lc + (int64_t)j * lat, sizeof(REAL) * lat);
      memcpy(key + (int64_t)j * hd + lat, rc + (int64_t)j * Hkv * rd + hk * rd, sizeof(REAL) * rd);
      memcpy(val + (int64_t)j * hd, lc + (int64_t)j * lat, sizeof(REAL) * lat);
      memset(val + (int64_t)j * hd + lat, 0, sizeof(REAL) * rd);
    }
    attn_fwd(query, key, val, ao, lse, T, count, hd, offset, lo->window);
    for (int t = 0; t < T; t++)
      for (int d = 0; d < D; d++) {
        REAL sum = 0; /* mla.go:266-273 */
        for (int rk = 0; rk < lat; rk++) sum += ao[t * hd + rk] * vu[(int64_t)(hk * D + d) * lat + rk];
        o[(((int64_t)b * T + t) * Hq + hq) * D + d] = sum;
      }
    free(query); free(key); free(val); free(ao); free(lse);
  }
  free(ql); free(kvl); free(qc); free(qr); free(kr);
  (void)C;
}

/* ---- HCA compressed attention (model/compress.go, compress_attention.go) ---- */

/* Compression logits of rows [T][C]: logitWeight.Forward then + bias[row %
 * ratio] (compress.go:98-109). */
static void compress_logits(MODEL *m, const layer_off *lo, const REAL *h, int T, REAL *out) {
  const int D = m->D, ratio = m->ratio;
  linear_fwd(out, h, m->p + lo->wcl, T, m->C, D);
  for (int t = 0; t < T; t++)
    for (int d = 0; d < D; d++) out[(int64_t)t * D + d] += m->p[lo->cbias + (t % ratio) * D + d];
}

/* ChannelCompressor.Forward (compress.go:110-164) of one sequence: per block
 * and channel, softmax over the block's rows of the logits, weighted sum of
 * value [T][D]; compressed [blocks][D], probabilities [blocks][ratio][D]. */
static void compress_seq(int T, int D, int ratio, const REAL *logits, const REAL *value,
                         REAL *comp, REAL *probs) {
  const int blocks = (T + ratio - 1) / ratio;
  for (int bl = 0; bl < blocks; bl++)
    for (int d = 0; d < D; d++) {
      REAL mx = R(-INFINITY);
      for (int r = 0; r < ratio; r++) {
        int t = bl * ratio + r;
        if (t < T && logits[(int64_t)t * D + d] > mx) mx = logits[(int64_t)t * D + d];
      }
      double tot = 0;
      REAL *pr = probs + (int64_t)bl * ratio * D;
      for (int r = 0; r < ratio; r++) {
        int t = bl * ratio + r;
        REAL p = R(0);
        if (t < T && mx > R(-INFINITY)) p = R(exp((double)(logits[(int64_t)t * D + d] - mx)));
        pr[r * D + d] = p;
        tot += (double)p;
      }
      REAL acc = 0;
      if (tot > 0) {
        REAL inv = R(1.0 / tot);
        for (int r = 0; r < ratio; r++) {
          pr[r * D + d] *= inv;
          int t = bl * ratio + r;
          if (t < T) acc += pr[r * D + d] * value[(int64_t)t * D + d];
        }
      }
      comp[(int64_t)bl * D + d] = acc;
    }
}

/* ChannelCompressor.Backward's softmax part (compress.go:199-222): gradients
 * of the logits and of value, accumulated. */
static void compress_seq_bwd(int T, int D, int ratio, const REAL *probs, const REAL *value,
                             const REAL *comp, const REAL *g, REAL *glog, REAL *gval) {
  const int blocks = (T + ratio - 1) / ratio;
  for (int bl = 0; bl < blocks; bl++)
    for (int d = 0; d < D; d++) {
      REAL gr = g[(int64_t)bl * D + d], cv = comp[(int64_t)bl * D + d];
      for (int r = 0; r < ratio; r++) {
        int t = bl * ratio + r;
        if (t >= T) continue;
        REAL p = probs[((int64_t)bl * ratio + r) * D + d], v = value[(int64_t)t * D + d];
        glog[(int64_t)t * D + d] += p * gr * (v - cv);
        gval[(int64_t)t * D + d] += p * gr;
      }
    }
}

/* mergeAttentionBranches / mergeAttentionRow (compress_attention.go:440-486). */
static void merge_rows(REAL *out, REAL *lse, const REAL *oa, const REAL *la, const REAL *ob,
                       const REAL *lb, int rows, int D) {
  for (int i = 0; i < rows; i++) {
    REAL mx = la[i] > lb[i] ? la[i] : lb[i];
    if (mx == R(-INFINITY)) {
      for (int d = 0; d < D; d++) out[(int64_t)i * D + d] = 0;
      if (lse) lse[i] = mx;
      continue;
    }
    REAL wa = R(exp((double)(la[i] - mx))), wb = R(exp((double)(lb[i] - mx)));
    REAL tot = wa + wb;
    REAL inv = R(1.0 / (double)tot);
    for (int d = 0; d < D; d++)
      out[(int64_t)i * D + d] = (wa * oa[(int64_t)i * D + d] + wb * ob[(int64_t)i * D + d]) * inv;
    if (lse) lse[i] = mx + R(log((double)tot));
  }
}

/* ---- CSA lightning indexer (model/indexer.go) --------------------------- */

/* IndexerScores (kernels/scalar/indexer.go:11-34): out[r][s] = sum over heads
 * of w_h * ReLU(q[r,h] . k[s,h]), float32 dot products summed in order. */
static void indexer_scores(const REAL *iq, const REAL *ik, const REAL *w, int rows, int blocks,
                           int H, int dim, REAL *out) {
  const int HI = H * dim;
#pragma omp parallel for schedule(static)
  for (int r = 0; r < rows; r++)
    for (int s = 0; s < blocks; s++) {
      REAL total = 0;
      for (int h = 0; h < H; h++) {
        REAL dot = 0;
        const REAL *a = iq + (int64_t)r * HI + h * dim, *b = ik + (int64_t)s * HI + h * dim;
        for (int e = 0; e < dim; e++) dot += a[e] * b[e];
        if (dot > 0) total += w[h] * dot;
      }
      out[(int64_t)r * blocks + s] = total;
    }
}

/* topKIndices (indexer.go:226-268): the k largest values in descending
 * order, ties toward the smaller index; returns the count. */
static int topk_indices(const REAL *v, int n, int k, int *out) {
  if (k > n) k = n;
  if (k <= 0) return 0;
  int cnt = 0;
  for (int i = 0; i < n; i++) {
    int pos = cnt;
    while (pos > 0 && v[i] > v[out[pos - 1]]) pos--; /* equal values keep index order */
    if (pos >= k) continue;
    int last = cnt < k ? cnt : k - 1;
    for (int j = last; j > pos; j--) out[j] = out[j - 1];
    out[pos] = i;
    if (cnt < k) cnt++;
  }
  return cnt;
}

/* selectRowBlockMax + topKFromScoreRow (indexer.go:476-530): groups of
 * `pool` entries scored by their maximum (the trailing partially allowed
 * group over its allowed entries only), the best ceil(budget/pool) groups
 * give the candidates, and the final top-k is taken over the candidates'
 * scores in candidate order.  gmax is the row's group maxima (modified). */
static void select_row_block_max(const REAL *score, REAL *gmax, int allowed, int topk, int pool,
                                 int budget, int *sel, int *nsel, int *cand, int *ncand) {
  *nsel = 0;
  if (ncand) *ncand = 0;
  if (allowed <= 0 || topk <= 0) return;
  if (pool < 1) pool = 1;
  int gpt = (budget + pool - 1) / pool;
  if (gpt < 1) gpt = 1;
  int ag = (allowed + pool - 1) / pool;
  if (allowed % pool != 0 && ag > 0) {
    REAL mx = R(-INFINITY);
    for (int e = (ag - 1) * pool; e < allowed; e++)
      if (score[e] > mx) mx = score[e];
    gmax[ag - 1] = mx;
  }
  int *chosen = (int *)malloc(sizeof(int) * (gpt < ag ? gpt : ag) + sizeof(int));
  int nch = topk_indices(gmax, ag, gpt, chosen);
  int *c = (int *)malloc(sizeof(int) * (nch * pool + 1));
  int nc = 0;
  for (int i = 0; i < nch; i++) {
    int st = chosen[i] * pool, en = st + pool < allowed ? st + pool : allowed;
    for (int e = st; e < en; e++) c[nc++] = e;
  }
  REAL *fine = (REAL *)malloc(sizeof(REAL) * (nc + 1));
  for (int i = 0; i < nc; i++) fine[i] = score[c[i]];
  int *order = (int *)malloc(sizeof(int) * (nc + 1));
  int n = topk_indices(fine, nc, topk, order);
  for (int i = 0; i < n; i++) sel[i] = c[order[i]];
  *nsel = n;
  if (cand) {
    memcpy(cand, c, sizeof(int) * nc);
    *ncand = nc;
  }
  free(chosen); free(c); free(fine); free(order);
}

/* selectFromScoreMatrix / selectRows (indexer.go:378-474) for T rows at
 * positions offset.. of one (sequence, kv-head): IndexerBlockMax over all
 * `blocks` entries, then the per-row selection with allowed = pos / ratio. */
static void select_rows(const REAL *scores, int T, int blocks, int offset, int ratio, int topk,
                        int pool, int budget, int kcap, int ccap, int *sel, int *nsel, int *cand,
                        int *ncand) {
  if (pool < 1) pool = 1;
  const int groups = (blocks + pool - 1) / pool;
#pragma omp parallel for schedule(dynamic)
  for (int t = 0; t < T; t++) {
    const REAL *row = scores + (int64_t)t * blocks;
    REAL *gmax = (REAL *)malloc(sizeof(REAL) * (groups + 1));
    for (int g = 0; g < groups; g++) { /* IndexerBlockMax (scalar/indexer.go:44-61) */
      REAL mx = R(-INFINITY);
      int en = (g + 1) * pool < blocks ? (g + 1) * pool : blocks;
      for (int e = g * pool; e < en; e++)
        if (row[e] > mx) mx = row[e];
      gmax[g] = mx;
    }
    int allowed = (offset + t) / ratio;
    if (allowed > blocks) allowed = blocks;
    select_row_block_max(row, gmax, allowed, topk, pool, budget, sel + (int64_t)t * kcap,
                         nsel + t, cand ? cand + (int64_t)t * ccap : NULL, cand ? ncand + t : NULL);
    free(gmax);
  }
}

/* fineSelect (indexer.go:560-606): score the candidate entries below
 * maxBlock and take their top-k in candidate order. */
static void fine_select(const REAL *iq_row, const REAL *ik, const REAL *w, int H, int dim,
                        const int *cand, int nc, int topk, int maxBlock, int *sel, int *nsel) {
  *nsel = 0;
  if (nc <= 0 || topk <= 0) return;
  int *kept = (int *)malloc(sizeof(int) * nc);
  REAL *fine = (REAL *)malloc(sizeof(REAL) * nc);
  int nk = 0;
  for (int i = 0; i < nc; i++) {
    int e = cand[i];
    if (e < 0 || e >= maxBlock) continue;
    indexer_scores(iq_row, ik + (int64_t)e * H * dim, w, 1, 1, H, dim, fine + nk);
    kept[nk++] = e;
  }
  int *order = (int *)malloc(sizeof(int) * (nk + 1));
  int n = topk_indices(fine, nk, topk, order);
  for (int i = 0; i < n; i++) sel[i] = kept[order[i]];
  *nsel = n;
  free(kept); free(fine); free(order);
}

/* distillationTarget (compress_attention.go:149-196): per query the softmax
 * over its allowed blocks of the mean main attention logit of the query heads
 * sharing kv-head hh.  qh [B][Hq][T][D], kc of (b, hh) [blocks][D]. */
static void distill_target(const REAL *qh, const REAL *kcb, int b, int hh, int Hq, int rr,
                           int ratio, int T, int blocks, int D, REAL *target) {
#pragma omp parallel for schedule(dynamic)
  for (int t = 0; t < T; t++) {
    REAL *trow = target + (int64_t)t * blocks;
    memset(trow, 0, sizeof(REAL) * blocks);
    int allowed = t / ratio;
    if (allowed > blocks) allowed = blocks;
    if (allowed == 0) continue;
    REAL *lg = (REAL *)malloc(sizeof(REAL) * allowed);
    REAL mx = R(-INFINITY);
    for (int s = 0; s < allowed; s++) {
      REAL sum = 0;
      for (int r = 0; r < rr; r++) {
        const REAL *q = qh + (((int64_t)b * Hq + hh * rr + r) * T + t) * D, *k = kcb + (int64_t)s * D;
        REAL dot = 0;
        for (int e = 0; e < D; e++) dot += q[e] * k[e];
        sum += dot;
      }
      lg[s] = sum / R(rr);
      if (lg[s] > mx) mx = lg[s];
    }
    double total = 0;
    for (int s = 0; s < allowed; s++) {
      double v = exp((double)(lg[s] - mx));
      trow[s] = R(v);
      total += v;
    }
    for (int s = 0; s < allowed; s++) trow[s] /= R(total);
    free(lg);
  }
}

/* restrictIndexerToPool (compress_attention.go:199-230). */
static void restrict_to_pool(REAL *scores, REAL *target, int T, int blocks, const int *pool,
                             const int *npool, int ccap) {
  char *in = (char *)malloc(blocks + 1);
  for (int t = 0; t < T; t++) {
    memset(in, 0, blocks + 1);
    for (int i = 0; i < npool[t]; i++) in[pool[(int64_t)t * ccap + i]] = 1;
    REAL *sr = scores + (int64_t)t * blocks, *tr = target + (int64_t)t * blocks;
    double total = 0;
    for (int e = 0; e < blocks; e++) {
      if (!in[e]) {
        sr[e] = R(-INFINITY);
        tr[e] = 0;
        continue;
      }
      total += (double)tr[e];
    }
    if (total > 0)
      for (int e = 0; e < blocks; e++)
        if (in[e]) tr[e] = R((double)tr[e] / total);
  }
  free(in);
}

/* maskedIndexerSoftmax (compress_attention.go:262-298). */
static void masked_softmax(const REAL *scores, int T, int blocks, int ratio, REAL *probs) {
  for (int t = 0; t < T; t++) {
    const REAL *sr = scores + (int64_t)t * blocks;
    REAL *pr = probs + (int64_t)t * blocks;
    memset(pr, 0, sizeof(REAL) * blocks);
    int allowed = t / ratio;
    if (allowed > blocks) allowed = blocks;
    if (allowed == 0) continue;
    REAL mx = sr[0];
    for (int s = 1; s < allowed; s++)
      if (sr[s] > mx) mx = sr[s];
    if (isinf((double)mx) && mx < 0) continue;
    double total = 0;
    for (int s = 0; s < allowed; s++) {
      double v = exp((double)(sr[s] - mx));
      pr[s] = R(v);
      total += v;
    }
    for (int s = 0; s < allowed; s++) pr[s] /= R(total);
  }
}

/* ---- compressed attention (model/compress_attention.go) ----------------- */

/* Group state shared by a Full layer and the Reindex/Reuse layers after it
 * (model/share.go:16-42). */
typedef struct hca_share {
  int producer, blocks;
  REAL *kc, *vc;        /* the producer's compressed keys/values (borrowed) */
  REAL *gkc, *gvc;      /* training: the group's compressed-KV gradients (owned) */
  int *sel, *nsel;      /* most recently published selection (borrowed) */
  int *pool, *npool;    /* the producer's candidate pool (borrowed), or NULL */
} hca_share;

/* One layer's training context.  kc/vc/probs are owned by Full layers (the
 * others point at the producer's); the indexer arrays belong to layers with
 * an indexer. */
typedef struct {
  int blocks, owns, own_sel, kcap, ccap;
  REAL *kc, *vc, *probs;  /* [B][Hkv][blocks][D], probs [B][blocks][ratio][D] */
  int *sel, *nsel;        /* [B*Hkv][T][kcap], [B*Hkv][T] */
  int *pool, *npool;      /* [B*Hkv][T][ccap] (Full layer, pool > 1) */
  REAL *iq, *ik;          /* [B*T][HI], [B*Hkv][blocks][HI] */
  REAL *scores, *target;  /* [B*Hkv][T][blocks] */
  hca_share *share;
  /* CED decoder Full layer: the compressor reads the encoder hidden state
   * (borrowed) and compresses its own projections of it, kg/vg [B][Hkv][T][D]
   * (keys after RoPE and QK norm), ced_krot the post-RoPE pre-norm keys
   * [B*T][Hkv][D] */
  const REAL *enc;
  REAL *kg, *vg, *ced_krot;
} hca_ctx;

static void hca_ctx_free(hca_ctx *hc) {
  if (!hc) return;
  if (hc->owns) { free(hc->kc); free(hc->vc); free(hc->probs); }
  if (hc->own_sel) { free(hc->sel); free(hc->nsel); }
  free(hc->pool); free(hc->npool);
  free(hc->iq); free(hc->ik); free(hc->scores); free(hc->target);
  free(hc->kg); free(hc->vg); free(hc->ced_krot);
  free(hc);
}

/* cedGlobalKeyValue (attention.go:156-171): a CED decoder layer's global keys
 * and values, its own key and value projections of the encoder hidden state
 * (no value embedding); RoPE at positions offset.. and the 1.2 QK norm on
 * the keys.  Sequence layout [B*T][Hkv][D]; krot (optional) receives the
 * post-RoPE pre-norm keys. */
static void ced_kv(MODEL *m, const layer_off *lo, const REAL *enc, int B, int T, int offset,
                   REAL *kseq, REAL *vseq, REAL *krot) {
  const int Hkv = m->Hkv, D = m->D, C = m->C;
  const int64_t N = (int64_t)B * T;
  linear_fwd(kseq, enc, m->p + lo->wk, N, C, Hkv * D);
  linear_fwd(vseq, enc, m->p + lo->wv, N, C, Hkv * D);
  for (int b = 0; b < B; b++)
    for (int t = 0; t < T; t++) {
      int64_t n = (int64_t)b * T + t;
      rope_row(m, kseq + n * Hkv * D, kseq + n * Hkv * D, Hkv, offset + t, 1);
    }
  if (krot) memcpy(krot, kseq, sizeof(REAL) * N * Hkv * D);
  rmsnorm_rows(kseq, kseq, N * Hkv, D);
  for (int64_t i = 0; i < N * Hkv * D; i++) kseq[i] *= R(QK_SCALE);
}
static void hca_share_free(hca_share *sh) {
  if (!sh) return;
  free(sh->gkc); free(sh->gvc);
  free(sh);
}
static int candidate_cap(const MODEL *m) {
  int pool = m->ipool < 1 ? 1 : m->ipool;
  int gpt = (m->ibudget + pool - 1) / pool;
  return (gpt < 1 ? 1 : gpt) * pool;
}

/* sparseTrainingPlan (compress_attention.go:45-131) of a layer with an
 * indexer: indexer projections, scores, distillation targets and the top-k
 * selection (within the producer's candidate pool on a Reindex layer). */
static void sparse_training_plan(MODEL *m, const layer_off *lo, const REAL *h, const REAL *qh,
                                 int B, int T, hca_ctx *hc, hca_share *sh) {
  const int Hkv = m->Hkv, D = m->D, HI = m->HI, blocks = hc->blocks, rr = m->Hq / Hkv;
  const REAL *P = m->p;
  hc->kcap = m->topk;
  hc->ccap = candidate_cap(m);
  hc->sel = (int *)calloc((size_t)B * Hkv * T * hc->kcap, sizeof(int));
  hc->nsel = (int *)calloc((size_t)B * Hkv * T, sizeof(int));
  hc->own_sel = 1;
  const int produce_pool = lo->mode == REUSE_FULL && m->ipool > 1;
  const int use_pool = lo->mode == REUSE_REINDEX && m->ipool > 1 && sh->pool;
  if (produce_pool) {
    hc->pool = (int *)calloc((size_t)B * Hkv * T * hc->ccap, sizeof(int));
    hc->npool = (int *)calloc((size_t)B * Hkv * T, sizeof(int));
  }
  hc->iq = (REAL *)malloc(sizeof(REAL) * (int64_t)B * T * HI);
  linear_fwd(hc->iq, h, P + lo->wiq, (int64_t)B * T, m->C, HI);
  hc->ik = (REAL *)malloc(sizeof(REAL) * (int64_t)B * Hkv * blocks * HI);
  linear_fwd(hc->ik, hc->kc, P + lo->wik, (int64_t)B * Hkv * blocks, D, HI);
  hc->scores = (REAL *)malloc(sizeof(REAL) * (int64_t)B * Hkv * T * blocks);
  hc->target = (REAL *)malloc(sizeof(REAL) * (int64_t)B * Hkv * T * blocks);
  for (int b = 0; b < B; b++)
    for (int hh = 0; hh < Hkv; hh++) {
      const int64_t bk = (int64_t)b * Hkv + hh;
      REAL *sc = hc->scores + bk * T * blocks, *tg = hc->target + bk * T * blocks;
      const REAL *iqb = hc->iq + (int64_t)b * T * HI, *ikb = hc->ik + bk * blocks * HI;
      indexer_scores(iqb, ikb, P + lo->wih, T, blocks, m->ih, m->idim, sc);
      distill_target(qh, hc->kc + bk * blocks * D, b, hh, m->Hq, rr, m->ratio, T, blocks, D, tg);
      int *sel = hc->sel + bk * T * hc->kcap, *nsel = hc->nsel + bk * T;
      if (use_pool) {
        const int *pl = sh->pool + bk * T * hc->ccap, *npl = sh->npool + bk * T;
        for (int t = 0; t < T; t++) {
          int allowed = t / m->ratio;
          if (allowed > blocks) allowed = blocks;
          fine_select(iqb + (int64_t)t * HI, ikb, P + lo->wih, m->ih, m->idim,
                      pl + (int64_t)t * hc->ccap, npl[t], m->topk, allowed,
                      sel + (int64_t)t * hc->kcap, nsel + t);
        }
        restrict_to_pool(sc, tg, T, blocks, pl, npl, hc->ccap);
      } else {
        select_rows(sc, T, blocks, 0, m->ratio, m->topk, m->ipool < 1 ? 1 : m->ipool, m->ibudget,
                    hc->kcap, hc->ccap, sel, nsel, produce_pool ? hc->pool + bk * T * hc->ccap : NULL,
                    produce_pool ? hc->npool + bk * T : NULL);
      }
    }
  const int l = (int)(lo - m->lay);
  const int64_t nt = (int64_t)B * Hkv * T * blocks;
  if (m->freeze == 1) {
    free(m->ftarget[l]);
    m->ftarget[l] = (REAL *)malloc(sizeof(REAL) * nt);
    memcpy(m->ftarget[l], hc->target, sizeof(REAL) * nt);
    m->ftarget_n[l] = nt;
  } else if (m->freeze == 2 && m->ftarget[l] && m->ftarget_n[l] == nt) {
    memcpy(hc->target, m->ftarget[l], sizeof(REAL) * nt);
  }
  /* the distillation objective whose gradient the backward takes */
  REAL *pr = (REAL *)malloc(sizeof(REAL) * (int64_t)T * blocks);
  double dl = 0;
  for (int64_t bk = 0; bk < (int64_t)B * Hkv; bk++) {
    const REAL *sc = hc->scores + bk * T * blocks, *tg = hc->target + bk * T * blocks;
    masked_softmax(sc, T, blocks, m->ratio, pr);
    for (int64_t i = 0; i < (int64_t)T * blocks; i++)
      if (tg[i] > 0) dl -= (double)tg[i] * log((double)pr[i]);
  }
  m->distill_loss += (double)m->iw * dl;
  free(pr);
}

/* Training-side compressed attention (model/train.go:99-169 with
 * compressForward, sparseTrainingPlan, compressedAttentionForward[Sparse],
 * attentionForwardWindowed and mergeAttentionBranches): qh [B][Hq][T][D],
 * kh/vh [B][Hkv][T][D] (post-norm keys, gated values), h [B*T][C]; writes oh
 * and lse.  A Full layer starts a new group share (*shp); the others use the
 * group's compressed keys/values and, for Reuse, its selection. */
static void hca_train_forward(MODEL *m, const layer_off *lo, const REAL *qh, const REAL *kh,
                              const REAL *vh, const REAL *h, const REAL *enc, int B, int T,
                              REAL *oh, REAL *lse, hca_ctx *hc, hca_share **shp) {
  const int D = m->D, Hq = m->Hq, Hkv = m->Hkv, ratio = m->ratio, rr = Hq / Hkv;
  const int blocks = (T + ratio - 1) / ratio;
  hc->blocks = blocks;
  if (lo->mode == REUSE_FULL) {
    hc->owns = 1;
    const REAL *hin = h, *kin = kh, *vin = vh;
    if (enc) { /* CED decoder (train.go:104-111): global KV from the encoder */
      const int64_t N = (int64_t)B * T;
      REAL *ks = (REAL *)malloc(sizeof(REAL) * N * Hkv * D);
      REAL *vs = (REAL *)malloc(sizeof(REAL) * N * Hkv * D);
      hc->ced_krot = (REAL *)malloc(sizeof(REAL) * N * Hkv * D);
      ced_kv(m, lo, enc, B, T, 0, ks, vs, hc->ced_krot);
      hc->kg = (REAL *)malloc(sizeof(REAL) * N * Hkv * D);
      hc->vg = (REAL *)malloc(sizeof(REAL) * N * Hkv * D);
      for (int b = 0; b < B; b++)
        for (int t = 0; t < T; t++)
          for (int hh = 0; hh < Hkv; hh++) {
            memcpy(hc->kg + (((int64_t)b * Hkv + hh) * T + t) * D, ks + (((int64_t)b * T + t) * Hkv + hh) * D, sizeof(REAL) * D);
            memcpy(hc->vg + (((int64_t)b * Hkv + hh) * T + t) * D, vs + (((int64_t)b * T + t) * Hkv + hh) * D, sizeof(REAL) * D);
          }
      free(ks); free(vs);
      hc->enc = enc;
      hin = enc;
      kin = hc->kg;
      vin = hc->vg;
    }
    hc->kc = (REAL *)calloc((size_t)B * Hkv * blocks * D, sizeof(REAL));
    hc->vc = (REAL *)calloc((size_t)B * Hkv * blocks * D, sizeof(REAL));
    hc->probs = (REAL *)calloc((size_t)B * blocks * ratio * D, sizeof(REAL));
    REAL *logits = (REAL *)malloc(sizeof(REAL) * (int64_t)T * D);
    for (int b = 0; b < B; b++) {
      compress_logits(m, lo, hin + (int64_t)b * T * m->C, T, logits);
      REAL *pb = hc->probs + (int64_t)b * blocks * ratio * D;
      for (int hh = 0; hh < Hkv; hh++) {
        int64_t bk = (int64_t)b * Hkv + hh;
        compress_seq(T, D, ratio, logits, kin + bk * T * D, hc->kc + bk * blocks * D, pb);
        compress_seq(T, D, ratio, logits, vin + bk * T * D, hc->vc + bk * blocks * D, pb);
      }
    }
    free(logits);
    hca_share *sh = (hca_share *)calloc(1, sizeof(hca_share));
    sh->blocks = blocks;
    sh->kc = hc->kc;
    sh->vc = hc->vc;
    sh->gkc = (REAL *)calloc((size_t)B * Hkv * blocks * D, sizeof(REAL));
    sh->gvc = (REAL *)calloc((size_t)B * Hkv * blocks * D, sizeof(REAL));
    *shp = sh;
  } else {
    hc->kc = (*shp)->kc;
    hc->vc = (*shp)->vc;
  }
  hca_share *sh = *shp;
  hc->share = sh;
  if (m->topk > 0) {
    if (lo->mode == REUSE_REUSE) {
      hc->sel = sh->sel;
      hc->nsel = sh->nsel;
      hc->kcap = m->topk;
    } else {
      sparse_training_plan(m, lo, h, qh, B, T, hc, sh);
      sh->sel = hc->sel;
      sh->nsel = hc->nsel;
      if (lo->mode == REUSE_FULL) {
        sh->pool = hc->pool;
        sh->npool = hc->npool;
      }
    }
  }
#pragma omp parallel for schedule(dynamic)
  for (int bh = 0; bh < B * Hq; bh++) {
    int b = bh / Hq, hq = bh % Hq;
    int64_t bk = (int64_t)b * Hkv + hq / rr;
    const REAL *q = qh + (int64_t)bh * T * D;
    const REAL *kcb = hc->kc + bk * blocks * D, *vcb = hc->vc + bk * blocks * D;
    REAL *go = (REAL *)calloc((size_t)T * D, sizeof(REAL));
    REAL *gl = (REAL *)malloc(sizeof(REAL) * T);
    if (m->topk > 0) { /* compressedAttentionForwardSparse (:326-373) */
      REAL *kg = (REAL *)malloc(sizeof(REAL) * hc->kcap * D), *vg = (REAL *)malloc(sizeof(REAL) * hc->kcap * D);
      for (int t = 0; t < T; t++) {
        const int *sel = hc->sel + (bk * T + t) * hc->kcap;
        int n = hc->nsel[bk * T + t];
        if (n == 0) {
          gl[t] = R(-INFINITY);
          continue;
        }
        for (int i = 0; i < n; i++) {
          memcpy(kg + (int64_t)i * D, kcb + (int64_t)sel[i] * D, sizeof(REAL) * D);
          memcpy(vg + (int64_t)i * D, vcb + (int64_t)sel[i] * D, sizeof(REAL) * D);
        }
        attn_fwd(q + (int64_t)t * D, kg, vg, go + (int64_t)t * D, gl + t, 1, n, D, n, -1);
      }
      free(kg); free(vg);
    } else { /* compressedAttentionForward (:603-650): queries of block bl see blocks < bl */
      for (int bl = 0; bl < blocks; bl++) {
        int t0 = bl * ratio, t1 = t0 + ratio < T ? t0 + ratio : T;
        if (bl == 0) {
          for (int t = t0; t < t1; t++) gl[t] = R(-INFINITY);
          continue;
        }
        attn_fwd(q + (int64_t)t0 * D, kcb, vcb, go + (int64_t)t0 * D, gl + t0, t1 - t0, bl, D, bl, -1);
      }
    }
    if (m->swa > 0) {
      REAL *loc = (REAL *)malloc(sizeof(REAL) * (int64_t)T * D);
      REAL *ll = (REAL *)malloc(sizeof(REAL) * T);
      attn_fwd(q, kh + bk * T * D, vh + bk * T * D, loc, ll, T, T, D, 0, m->swa);
      merge_rows(oh + (int64_t)bh * T * D, lse + (int64_t)bh * T, go, gl, loc, ll, T, D);
      free(loc); free(ll);
    } else {
      memcpy(oh + (int64_t)bh * T * D, go, sizeof(REAL) * T * D);
      memcpy(lse + (int64_t)bh * T, gl, sizeof(REAL) * T);
    }
    free(go); free(gl);
  }
}

/* indexerDistillationGradient (compress_attention.go:133-147) with
 * SparseIndexer.Backward (indexer.go:107-151): gradient (softmax(I) - target)
 * * weight of the index scores into the indexer weights, the attention input
 * (dh, [B*T][C], accumulated) and the compressed keys (dkc, accumulated). */
static void indexer_distill_backward(MODEL *m, const layer_off *lo, const hca_ctx *hc,
                                     const REAL *h, int B, int T, REAL *dh, REAL *dkc, REAL *G) {
  const int Hkv = m->Hkv, D = m->D, C = m->C, HI = m->HI, H = m->ih, dim = m->idim;
  const int blocks = hc->blocks;
  const REAL *P = m->p, *w = P + lo->wih;
  REAL *probs = (REAL *)malloc(sizeof(REAL) * (int64_t)T * blocks);
  REAL *gq = (REAL *)malloc(sizeof(REAL) * (int64_t)T * HI);
  REAL *gk = (REAL *)malloc(sizeof(REAL) * (int64_t)blocks * HI);
  REAL *dhb = (REAL *)malloc(sizeof(REAL) * (int64_t)T * C);
  REAL *dkb = (REAL *)malloc(sizeof(REAL) * (int64_t)blocks * D);
  for (int b = 0; b < B; b++)
    for (int hh = 0; hh < Hkv; hh++) {
      const int64_t bk = (int64_t)b * Hkv + hh;
      const REAL *sc = hc->scores + bk * T * blocks, *tg = hc->target + bk * T * blocks;
      const REAL *q = hc->iq + (int64_t)b * T * HI, *k = hc->ik + bk * blocks * HI;
      masked_softmax(sc, T, blocks, m->ratio, probs);
      memset(gq, 0, sizeof(REAL) * (int64_t)T * HI);
      memset(gk, 0, sizeof(REAL) * (int64_t)blocks * HI);
      for (int t = 0; t < T; t++)
        for (int s = 0; s < blocks; s++) {
          const REAL gs = (probs[(int64_t)t * blocks + s] - tg[(int64_t)t * blocks + s]) * m->iw;
          for (int hd = 0; hd < H; hd++) {
            const REAL *qa = q + (int64_t)t * HI + hd * dim, *ka = k + (int64_t)s * HI + hd * dim;
            REAL dot = 0;
            for (int e = 0; e < dim; e++) dot += qa[e] * ka[e];
            if (dot <= 0) continue;
            G[lo->wih + hd] += gs * dot;
            const REAL wt = gs * w[hd];
            REAL *gqa = gq + (int64_t)t * HI + hd * dim, *gka = gk + (int64_t)s * HI + hd * dim;
            for (int e = 0; e < dim; e++) {
              gqa[e] += wt * ka[e];
              gka[e] += wt * qa[e];
            }
          }
        }
      linear_bwd(dhb, G + lo->wiq, h + (int64_t)b * T * C, gq, P + lo->wiq, T, C, HI);
      linear_bwd(dkb, G + lo->wik, hc->kc + bk * blocks * D, gk, P + lo->wik, blocks, D, HI);
      for (int64_t i = 0; i < (int64_t)T * C; i++) dh[(int64_t)b * T * C + i] += dhb[i];
      for (int64_t i = 0; i < (int64_t)blocks * D; i++) dkc[bk * blocks * D + i] += dkb[i];
    }
  free(probs); free(gq); free(gk); free(dhb); free(dkb);
}

/* Training-side compressed attention backward (model/train.go:211-303 with
 * compressedAttentionBackward[Sparse], indexerDistillationGradient,
 * attentionBackwardWindowed and compressBackward): dqh/dkh/dvh (head-major,
 * zeroed by the caller) receive the query and raw key/value gradients,
 * dhin_c [B*T][C] the gradient wrt the attention input from the compressor
 * and the indexer (zero on Reuse layers); parameter gradients accumulate in
 * G.  Compressed-KV gradients accumulate in the group share; the Full layer,
 * visited last in the backward, runs the compressor backward on the sum. */
static void hca_train_backward(MODEL *m, const layer_off *lo, const hca_ctx *hc, const REAL *qh,
                               const REAL *kh, const REAL *vh, const REAL *oh, const REAL *doh,
                               const REAL *lse, const REAL *h, int B, int T, REAL *dqh,
                               REAL *dkh, REAL *dvh, REAL *dhin_c, REAL *genc, REAL *G) {
  const int D = m->D, C = m->C, Hq = m->Hq, Hkv = m->Hkv, ratio = m->ratio, rr = Hq / Hkv;
  const int blocks = hc->blocks;
  hca_share *sh = hc->share;
  REAL *corr = NULL;
  if (m->swa > 0) { /* merged row correction dO.O (train.go:211-226) */
    corr = (REAL *)malloc(sizeof(REAL) * (int64_t)B * Hq * T);
    for (int64_t row = 0; row < (int64_t)B * Hq * T; row++) {
      double dot = 0;
      for (int d = 0; d < D; d++) dot += (double)doh[row * D + d] * (double)oh[row * D + d];
      corr[row] = R(dot);
    }
  }
  REAL *dkc = sh->gkc, *dvc = sh->gvc;
  REAL *dkl = (REAL *)calloc((size_t)B * Hkv * T * D, sizeof(REAL));
  REAL *dvl = (REAL *)calloc((size_t)B * Hkv * T * D, sizeof(REAL));
  /* serial over query heads so GQA accumulation into the shared K/V is race-free */
  for (int b = 0; b < B; b++)
#pragma omp parallel for schedule(dynamic)
    for (int hh = 0; hh < Hkv; hh++) {
      REAL *kg = NULL, *vg = NULL, *dkg = NULL, *dvg = NULL;
      if (m->topk > 0) {
        kg = (REAL *)malloc(sizeof(REAL) * hc->kcap * D); vg = (REAL *)malloc(sizeof(REAL) * hc->kcap * D);
        dkg = (REAL *)malloc(sizeof(REAL) * hc->kcap * D); dvg = (REAL *)malloc(sizeof(REAL) * hc->kcap * D);
      }
      int64_t bk = (int64_t)b * Hkv + hh;
      REAL *kcb = hc->kc + bk * blocks * D, *vcb = hc->vc + bk * blocks * D;
      for (int r = 0; r < rr; r++) {
        int hq = hh * rr + r;
        int64_t bh = (int64_t)b * Hq + hq;
        if (m->topk > 0) { /* compressedAttentionBackwardSparse (:376-433) */
          for (int t = 0; t < T; t++) {
            const int *sel = hc->sel + (bk * T + t) * hc->kcap;
            int n = hc->nsel[bk * T + t];
            if (n == 0) continue;
            for (int i = 0; i < n; i++) {
              memcpy(kg + (int64_t)i * D, kcb + (int64_t)sel[i] * D, sizeof(REAL) * D);
              memcpy(vg + (int64_t)i * D, vcb + (int64_t)sel[i] * D, sizeof(REAL) * D);
            }
            memset(dkg, 0, sizeof(REAL) * n * D);
            memset(dvg, 0, sizeof(REAL) * n * D);
            attn_bwd_corr(qh + (bh * T + t) * D, kg, vg, doh + (bh * T + t) * D, lse + bh * T + t,
                          corr ? corr + bh * T + t : NULL, dqh + (bh * T + t) * D, dkg, dvg, 1, n,
                          D, n, -1);
            for (int i = 0; i < n; i++)
              for (int d = 0; d < D; d++) {
                dkc[(bk * blocks + sel[i]) * D + d] += dkg[(int64_t)i * D + d];
                dvc[(bk * blocks + sel[i]) * D + d] += dvg[(int64_t)i * D + d];
              }
          }
        } else {
          for (int bl = 1; bl < blocks; bl++) {
            int t0 = bl * ratio, t1 = t0 + ratio < T ? t0 + ratio : T;
            attn_bwd_corr(qh + (bh * T + t0) * D, kcb, vcb, doh + (bh * T + t0) * D,
                          lse + bh * T + t0, corr ? corr + bh * T + t0 : NULL,
                          dqh + (bh * T + t0) * D, dkc + bk * blocks * D, dvc + bk * blocks * D,
                          t1 - t0, bl, D, bl, -1);
          }
        }
        if (m->swa > 0)
          attn_bwd_corr(qh + bh * T * D, kh + bk * T * D, vh + bk * T * D, doh + bh * T * D,
                        lse + bh * T, corr + bh * T, dqh + bh * T * D, dkl + bk * T * D,
                        dvl + bk * T * D, T, T, D, 0, m->swa);
      }
      free(kg); free(vg); free(dkg); free(dvg);
    }
  memset(dhin_c, 0, sizeof(REAL) * (int64_t)B * T * C);
  REAL *dh_idx = NULL;
  if (lo->has_idx) { /* the indexer's distillation into the group's key gradient */
    dh_idx = (REAL *)calloc((size_t)B * T * C, sizeof(REAL));
    indexer_distill_backward(m, lo, hc, h, B, T, dh_idx, dkc, G);
  }
  if (lo->mode == REUSE_FULL) { /* compressBackward (compress_attention.go:1182-1209) */
    /* a CED decoder layer compresses its projections of the encoder hidden
     * state: those gradients flow to the encoder (train.go:249-262) */
    const int ced = hc->enc != NULL;
    const REAL *hin = ced ? hc->enc : h, *kin = ced ? hc->kg : kh, *vin = ced ? hc->vg : vh;
    REAL *dkin = dkh, *dvin = dvh, *dhc = dhin_c;
    if (ced) {
      dkin = (REAL *)calloc((size_t)B * Hkv * T * D, sizeof(REAL));
      dvin = (REAL *)calloc((size_t)B * Hkv * T * D, sizeof(REAL));
      dhc = (REAL *)calloc((size_t)B * T * C, sizeof(REAL));
    }
    REAL *glk = (REAL *)malloc(sizeof(REAL) * (int64_t)T * D);
    REAL *glv = (REAL *)malloc(sizeof(REAL) * (int64_t)T * D);
    REAL *dhk = (REAL *)malloc(sizeof(REAL) * (int64_t)T * C);
    REAL *dhv = (REAL *)malloc(sizeof(REAL) * (int64_t)T * C);
    for (int b = 0; b < B; b++) {
      const REAL *pb = hc->probs + (int64_t)b * blocks * ratio * D;
      const REAL *hb = hin + (int64_t)b * T * C;
      for (int hh = 0; hh < Hkv; hh++) {
        int64_t bk = (int64_t)b * Hkv + hh;
        memset(glk, 0, sizeof(REAL) * (int64_t)T * D);
        memset(glv, 0, sizeof(REAL) * (int64_t)T * D);
        compress_seq_bwd(T, D, ratio, pb, kin + bk * T * D, hc->kc + bk * blocks * D,
                         dkc + bk * blocks * D, glk, dkin + bk * T * D);
        linear_bwd(dhk, G + lo->wcl, hb, glk, m->p + lo->wcl, T, C, D);
        for (int t = 0; t < T; t++)
          for (int d = 0; d < D; d++) G[lo->cbias + (t % ratio) * D + d] += glk[(int64_t)t * D + d];
        compress_seq_bwd(T, D, ratio, pb, vin + bk * T * D, hc->vc + bk * blocks * D,
                         dvc + bk * blocks * D, glv, dvin + bk * T * D);
        linear_bwd(dhv, G + lo->wcl, hb, glv, m->p + lo->wcl, T, C, D);
        for (int t = 0; t < T; t++)
          for (int d = 0; d < D; d++) G[lo->cbias + (t % ratio) * D + d] += glv[(int64_t)t * D + d];
        for (int64_t i = 0; i < (int64_t)T * C; i++) dhc[(int64_t)b * T * C + i] += dhk[i] + dhv[i];
      }
    }
    free(glk); free(glv); free(dhk); free(dhv);
    if (ced) { /* cedKey/ValueProjectionBackward (train.go:454-479) */
      const int64_t N = (int64_t)B * T;
      REAL *gs = (REAL *)malloc(sizeof(REAL) * N * Hkv * D);
      REAL *gpre = (REAL *)malloc(sizeof(REAL) * N * Hkv * D);
      REAL *tmp = (REAL *)malloc(sizeof(REAL) * N * C);
      for (int b = 0; b < B; b++)
        for (int t = 0; t < T; t++)
          for (int hh = 0; hh < Hkv; hh++)
            for (int d = 0; d < D; d++)
              gs[(((int64_t)b * T + t) * Hkv + hh) * D + d] = dkin[(((int64_t)b * Hkv + hh) * T + t) * D + d] * R(QK_SCALE);
      rmsnorm_backward_rows(gpre, hc->ced_krot, gs, N * Hkv, D);
      for (int b = 0; b < B; b++)
        for (int t = 0; t < T; t++) {
          int64_t n = (int64_t)b * T + t;
          rope_row(m, gpre + n * Hkv * D, gpre + n * Hkv * D, Hkv, t, -1);
        }
      linear_bwd(tmp, G + lo->wk, hc->enc, gpre, m->p + lo->wk, N, C, Hkv * D);
      for (int64_t i = 0; i < N * C; i++) dhc[i] = dhc[i] + tmp[i];
      for (int b = 0; b < B; b++)
        for (int t = 0; t < T; t++)
          for (int hh = 0; hh < Hkv; hh++)
            memcpy(gs + (((int64_t)b * T + t) * Hkv + hh) * D, dvin + (((int64_t)b * Hkv + hh) * T + t) * D, sizeof(REAL) * D);
      linear_bwd(tmp, G + lo->wv, hc->enc, gs, m->p + lo->wv, N, C, Hkv * D);
      for (int64_t i = 0; i < N * C; i++) dhc[i] = dhc[i] + tmp[i];
      for (int64_t i = 0; i < N * C; i++) genc[i] += dhc[i];
      free(gs); free(gpre); free(tmp); free(dkin); free(dvin); free(dhc);
    }
  }
  if (dh_idx) {
    for (int64_t i = 0; i < (int64_t)B * T * C; i++) dhin_c[i] = dhin_c[i] + dh_idx[i];
    free(dh_idx);
  }
  /* raw key/value gradients: compressor part + local branch */
  for (int64_t i = 0; i < (int64_t)B * Hkv * T * D; i++) {
    dkh[i] = dkh[i] + dkl[i];
    dvh[i] = dvh[i] + dvl[i];
  }
  free(dkl); free(dvl); free(corr);
}

/* Per-forward-call group state of inference: the most recent selection and
 * the producer's candidate pool for the call's T rows. */
typedef struct {
  int *sel, *nsel, *pool, *npool;
} dec_share;

/* compressTail (compress_attention.go:848-866) of layer l for every row:
 * compress the buffered block, cache its indexer key projections. */
static void compress_tail(MODEL *m, const layer_off *lo, int l, kvcache *cache, int B) {
  const int D = m->D, C = m->C, ratio = m->ratio, Hkv = m->Hkv;
  REAL *logits = (REAL *)malloc(sizeof(REAL) * (int64_t)ratio * D);
  REAL *probs = (REAL *)malloc(sizeof(REAL) * (int64_t)ratio * D);
  for (int b = 0; b < B; b++) {
    compress_logits(m, lo, cache->tailh + ((size_t)l * B + b) * ratio * C, ratio, logits);
    int slot = cache->ccount[l * B + b];
    for (int hh = 0; hh < Hkv; hh++) {
      size_t cb = ((((size_t)l * B + b) * Hkv + hh) * cache->maxBlocks + slot);
      size_t tb = (((size_t)l * B + b) * Hkv + hh) * ratio * D;
      compress_seq(ratio, D, ratio, logits, cache->tailk + tb, cache->ck + cb * D, probs);
      compress_seq(ratio, D, ratio, logits, cache->tailv + tb, cache->cv + cb * D, probs);
      if (lo->has_idx)
        linear_fwd(cache->ikc + cb * m->HI, cache->ck + cb * D, m->p + lo->wik, 1, D, m->HI);
    }
    cache->ccount[l * B + b]++;
  }
  cache->taillen[l] = 0;
  free(logits); free(probs);
}

/* Inference compressed attention (forwardCompressed / forwardCompressedSparse,
 * compress_attention.go:895-1146): a Full layer buffers the T new rows and
 * compresses each completed block (appendGlobalTail); a Reindex layer caches
 * its own indexer keys of the producer's new blocks (cacheReusedIndexerKeys,
 * :1160-1176); every query attends to the compressed blocks before its own
 * block of the producer's cache -- all of them, or the indexer's top-k --
 * merged with the local window branch. */
/* appendGlobalTail (compress_attention.go:868-890): rows of hid [B*T][C]
 * and their keys/values [B*T][Hkv][D] enter layer l's tail, each completed
 * block is compressed. */
static void append_global_tail(MODEL *m, const layer_off *lo, int l, kvcache *cache,
                               const REAL *hid, const REAL *kseq, const REAL *vseq, int B, int T) {
  const int D = m->D, C = m->C, Hkv = m->Hkv, ratio = m->ratio;
  for (int t = 0; t < T; t++) {
    for (int b = 0; b < B; b++) {
      int slot = cache->taillen[l];
      memcpy(cache->tailh + (((size_t)l * B + b) * ratio + slot) * C, hid + ((int64_t)b * T + t) * C,
             sizeof(REAL) * C);
      for (int hh = 0; hh < Hkv; hh++) {
        size_t tb = ((((size_t)l * B + b) * Hkv + hh) * ratio + slot) * D;
        memcpy(cache->tailk + tb, kseq + (((int64_t)b * T + t) * Hkv + hh) * D, sizeof(REAL) * D);
        memcpy(cache->tailv + tb, vseq + (((int64_t)b * T + t) * Hkv + hh) * D, sizeof(REAL) * D);
      }
    }
    cache->taillen[l]++;
    if (cache->taillen[l] == ratio) compress_tail(m, lo, l, cache, B);
  }
}

/* cacheReusedIndexerKeys (compress_attention.go:1160-1176): a Reindex layer
 * projects the producer's new compressed blocks with its own indexer key. */
static void cache_reused_indexer_keys(MODEL *m, const layer_off *lo, int l, kvcache *cache, int B) {
  const int D = m->D, Hkv = m->Hkv, HI = m->HI, cl = lo->producer;
  int own = cache->ccount[l * B], prod = cache->ccount[cl * B];
  for (int blk = own; blk < prod; blk++) {
    for (int b = 0; b < B; b++)
      for (int hh = 0; hh < Hkv; hh++) {
        size_t pc = (((size_t)cl * B + b) * Hkv + hh) * cache->maxBlocks + blk;
        size_t oc = (((size_t)l * B + b) * Hkv + hh) * cache->maxBlocks + blk;
        linear_fwd(cache->ikc + oc * HI, cache->ck + pc * D, m->p + lo->wik, 1, D, HI);
      }
    for (int b = 0; b < B; b++) cache->ccount[l * B + b]++;
  }
}

/* enc: the encoder hidden state of the T rows for a CED decoder layer (its
 * global tail buffers enc and its own projections of it), else NULL.
 * replay: CED bounded replay (the global caches are already filled; the
 * local window does not reach before the replay start). */
static void hca_decode(MODEL *m, const layer_off *lo, int l, kvcache *cache, const REAL *h,
                       const REAL *qh, const REAL *kn, const REAL *vn, const REAL *enc, int replay,
                       int B, int T, REAL *oh, dec_share *ds) {
  const int D = m->D, C = m->C, Hq = m->Hq, Hkv = m->Hkv, ratio = m->ratio, rr = Hq / Hkv;
  const int offset = cache->pos, cl = lo->producer, HI = m->HI;
  const int floor_pos = replay ? offset : 0;
  if (lo->mode == REUSE_FULL && !replay) {
    if (enc) {
      REAL *ks = (REAL *)malloc(sizeof(REAL) * (int64_t)B * T * Hkv * D);
      REAL *vs = (REAL *)malloc(sizeof(REAL) * (int64_t)B * T * Hkv * D);
      ced_kv(m, lo, enc, B, T, offset, ks, vs, NULL);
      append_global_tail(m, lo, l, cache, enc, ks, vs, B, T);
      free(ks); free(vs);
    } else {
      append_global_tail(m, lo, l, cache, h, kn, vn, B, T);
    }
  } else if (lo->mode == REUSE_REINDEX && m->topk > 0 && !replay) {
    cache_reused_indexer_keys(m, lo, l, cache, B);
  }
  const int kcap = m->topk, ccap = candidate_cap(m);
  int *lsel = NULL, *lnsel = NULL;
  if (m->topk > 0 && lo->mode != REUSE_REUSE) { /* this layer's selection */
    lsel = (int *)calloc((size_t)B * Hkv * T * kcap + 1, sizeof(int));
    lnsel = (int *)calloc((size_t)B * Hkv * T, sizeof(int));
    const int produce_pool = lo->mode == REUSE_FULL && m->ipool > 1;
    const int use_pool = lo->mode == REUSE_REINDEX && m->ipool > 1 && ds->pool;
    if (produce_pool) {
      free(ds->pool); free(ds->npool);
      ds->pool = (int *)calloc((size_t)B * Hkv * T * ccap, sizeof(int));
      ds->npool = (int *)calloc((size_t)B * Hkv * T, sizeof(int));
    }
    REAL *iq = (REAL *)malloc(sizeof(REAL) * (int64_t)B * T * HI);
    linear_fwd(iq, h, m->p + lo->wiq, (int64_t)B * T, C, HI);
    for (int b = 0; b < B; b++) {
      const int avail = cache->ccount[cl * B + b];
      if (avail == 0) continue;
      for (int hh = 0; hh < Hkv; hh++) {
        const int64_t bk = (int64_t)b * Hkv + hh;
        const REAL *keys = cache->ikc + (((size_t)l * B + b) * Hkv + hh) * cache->maxBlocks * HI;
        int *sel = lsel + bk * T * kcap, *nsel = lnsel + bk * T;
        if (use_pool) { /* SelectWithinPool (indexer.go:532-558) */
          for (int t = 0; t < T; t++) {
            int allowed = (offset + t) / ratio;
            if (allowed > avail) allowed = avail;
            fine_select(iq + ((int64_t)b * T + t) * HI, keys, m->p + lo->wih, m->ih, m->idim,
                        ds->pool + (bk * T + t) * ccap, ds->npool[bk * T + t], m->topk, allowed,
                        sel + (int64_t)t * kcap, nsel + t);
          }
        } else { /* SelectProjectedWithCandidates (indexer.go:337-376) */
          const int pool = m->ipool < 1 ? 1 : m->ipool;
          const int budget = pool == 1 ? avail : m->ibudget;
          REAL *sc = (REAL *)malloc(sizeof(REAL) * (int64_t)T * avail);
          indexer_scores(iq + (int64_t)b * T * HI, keys, m->p + lo->wih, T, avail, m->ih, m->idim, sc);
          select_rows(sc, T, avail, offset, ratio, m->topk, pool, budget, kcap, ccap, sel, nsel,
                      produce_pool ? ds->pool + bk * T * ccap : NULL,
                      produce_pool ? ds->npool + bk * T : NULL);
          free(sc);
        }
      }
    }
    free(iq);
    free(ds->sel); free(ds->nsel);
    ds->sel = lsel;
    ds->nsel = lnsel;
  }
#pragma omp parallel for schedule(dynamic)
  for (int bh = 0; bh < B * Hq; bh++) {
    int b = bh / Hq, hq = bh % Hq, hh = hq / rr;
    const int64_t bk = (int64_t)b * Hkv + hh;
    REAL go[1024], lo_[1024], gl, ll;
    REAL *kg = (REAL *)malloc(sizeof(REAL) * (kcap + 1) * D), *vg = (REAL *)malloc(sizeof(REAL) * (kcap + 1) * D);
    const int avail = cache->ccount[cl * B + b];
    size_t cb = (((size_t)cl * B + b) * Hkv + hh) * cache->maxBlocks * D;
    for (int t = 0; t < T; t++) {
      int pos = offset + t;
      const REAL *q = qh + ((int64_t)bh * T + t) * D;
      REAL *out = oh + ((int64_t)bh * T + t) * D;
      gl = R(-INFINITY);
      memset(go, 0, sizeof(REAL) * D);
      if (m->topk > 0) {
        int n = avail > 0 ? ds->nsel[bk * T + t] : 0;
        const int *sel = ds->sel + (bk * T + t) * kcap;
        if (n > 0) {
          for (int i = 0; i < n; i++) {
            memcpy(kg + (int64_t)i * D, cache->ck + cb + (int64_t)sel[i] * D, sizeof(REAL) * D);
            memcpy(vg + (int64_t)i * D, cache->cv + cb + (int64_t)sel[i] * D, sizeof(REAL) * D);
          }
          attn_fwd(q, kg, vg, go, &gl, 1, n, D, n, -1);
        }
      } else {
        int count = pos / ratio;
        if (count > avail) count = avail;
        if (count > 0) attn_fwd(q, cache->ck + cb, cache->cv + cb, go, &gl, 1, count, D, count, -1);
      }
      if (m->swa > 0) { /* localAttentionRow (compress_attention.go:543-560) */
        int ls = pos - m->swa < floor_pos ? floor_pos : pos - m->swa;
        if (ls < 0) ls = 0;
        int n = pos - ls + 1;
        attn_fwd(q, cache_k(m, cache, l, b, hh) + (int64_t)ls * D,
                 cache_v(m, cache, l, b, hh) + (int64_t)ls * D, lo_, &ll, 1, n, D, n - 1, -1);
        merge_rows(out, NULL, go, &gl, lo_, &ll, 1, D);
      } else {
        memcpy(out, go, sizeof(REAL) * D);
      }
    }
    free(kg); free(vg);
  }
}

void FN(orc_set_freeze_targets)(MODEL *m, int mode) { m->freeze = mode; }
void FN(orc_model_set_params)(MODEL *m, const REAL *params) {
  memcpy(m->p, params, sizeof(REAL) * m->total);
}
double FN(orc_distill_loss)(const MODEL *m) { return m->distill_loss; }

#if defined(ORC_DEFINE_SHARED)
/* Test entry points for the HCA pieces (float32 build). */
void orc_channel_compress(int T, int D, int ratio, const float *logits, const float *value,
                          float *comp, float *probs) {
  compress_seq(T, D, ratio, logits, value, comp, probs);
}
void orc_merge_attention_rows(float *out, float *lse, const float *oa, const float *la,
                              const float *ob, const float *lb, int rows, int D) {
  merge_rows(out, lse, oa, la, ob, lb, rows, D);
}
int orc_indexer_topk(const float *values, int n, int k, int32_t *out) {
  return topk_indices(values, n, k, out);
}
void orc_indexer_scores_rows(const float *iq, const float *ik, const float *w, int rows, int blocks,
                             int heads, int dim, float *out) {
  indexer_scores(iq, ik, w, rows, blocks, heads, dim, out);
}
void orc_select_rows(const float *scores, int T, int blocks, int offset, int ratio, int topk,
                     int pool, int budget, int kcap, int ccap, int32_t *sel, int32_t *nsel,
                     int32_t *cand, int32_t *ncand) {
  select_rows(scores, T, blocks, offset, ratio, topk, pool, budget, kcap, ccap, sel, nsel, cand,
              ncand);
}
void orc_fine_select(const float *iq_row, const float *ik, const float *w, int heads, int dim,
                     const int32_t *cand, int nc, int topk, int max_block, int32_t *sel,
                     int32_t *nsel) {
  fine_select(iq_row, ik, w, heads, dim, cand, nc, topk, max_block, sel, nsel);
}
void orc_restrict_to_pool(float *scores, float *target, int T, int blocks, const int32_t *pool,
                          const int32_t *npool, int ccap) {
  restrict_to_pool(scores, target, T, blocks, pool, npool, ccap);
}
#endif

/* ---- forward ---------------------------------------------------------- */
typedef struct {
  REAL *xin, *xb, *h, *qrot, *krot, *qn, *kn, *vh, *lse, *o, *vesig, *ve, *mid, *h2, *u, *act;
  /* latent preset: MLA latents, shared-expert gate, MoE routing and experts */
  REAL *ql, *kvl, *g2;
  struct moe_ctx *moe;
  hca_ctx *hca;
} layer_ctx;

typedef struct {
  int B, T;
  int32_t *ids;
  REAL *raw, *embn, *smsig, *x0;
  layer_ctx lc[MAXL];
  hca_share *shares[MAXL]; /* compressed-attention groups, by producing layer */
  REAL *enc, *ced_genc;    /* CED: encoder hidden state and its decoder gradient */
  REAL *backout, *final_pre, *final_norm, *logits;
} train_ctx;

static void ctx_free(train_ctx *c, int L) {
  if (!c) return;
  free(c->ids);
  free(c->raw); free(c->embn); free(c->smsig); free(c->x0);
  for (int l = 0; l < L; l++) {
    layer_ctx *x = &c->lc[l];
    free(x->xin); free(x->xb); free(x->h); free(x->qrot); free(x->krot); free(x->qn);
    free(x->kn); free(x->vh); free(x->lse); free(x->o); free(x->vesig); free(x->ve);
    free(x->mid); free(x->h2); free(x->u); free(x->act);
    free(x->ql); free(x->kvl); free(x->g2);
    moe_ctx_free(x->moe);
    hca_ctx_free(x->hca);
    hca_share_free(c->shares[l]);
  }
  free(c->enc); free(c->ced_genc);
  free(c->backout); free(c->final_pre); free(c->final_norm); free(c->logits);
  free(c);
}

static REAL *dup_arr(const REAL *a, size_t n) {
  REAL *b = (REAL *)malloc(sizeof(REAL) * n);
  memcpy(b, a, sizeof(REAL) * n);
  return b;
}

/*
 * model/transformer.go:243-342 (forward) with model/block.go:38-47,
 * model/attention.go:235-324 and model/mlp.go:62-77.  With cache == NULL it
 * is also the training forward (model/train_transformer.go:63-142); ctx, when
 * given, receives the saved activations.
 */
/* Options of a partial forward (PrefillCED's phases): a layer range, given
 * activations and initial residual instead of the embedding, bounded replay,
 * the final activations out, and no cache advance. */
typedef struct {
  int l0, l1, replay, no_advance;
  const REAL *x_in, *x0_in;
  REAL *x_out;
} fwd_opts;

static void forward_run(MODEL *m, const int32_t *ids, int B, int T, kvcache *cache, REAL *logits,
                        train_ctx *ctx, const fwd_opts *op);
static void forward_impl(MODEL *m, const int32_t *ids, int B, int T, kvcache *cache, REAL *logits,
                         train_ctx *ctx) {
  forward_run(m, ids, B, T, cache, logits, ctx, NULL);
}

static void forward_run(MODEL *m, const int32_t *ids, int B, int T, kvcache *cache, REAL *logits,
                        train_ctx *ctx, const fwd_opts *op) {
  int C = m->C, Hq = m->Hq, Hkv = m->Hkv, D = m->D, F = m->F, V = m->V, PV = m->PV;
  int64_t N = (int64_t)B * T;
  const REAL *P = m->p;
  /* compressed attention: the current group's share (training) or its
   * per-call selection state (inference); contexts not kept by ctx */
  hca_share *cur_share = NULL, *shares[MAXL] = {0};
  hca_ctx *hcs[MAXL] = {0};
  dec_share ds;
  memset(&ds, 0, sizeof ds);
  m->distill_loss = 0;
  const int l_begin = op ? op->l0 : 0, l_end = op ? op->l1 : m->L;
  const int replay = op ? op->replay : 0;
  REAL *enc = NULL; /* CED: the input of the first decoder layer */
  REAL *x = (REAL *)malloc(sizeof(REAL) * N * C);
  REAL *x0 = NULL;
  if (op && op->x_in) {
    memcpy(x, op->x_in, sizeof(REAL) * N * C);
    x0 = dup_arr(op->x0_in, (size_t)N * C);
    goto layers;
  }
  REAL *raw = (REAL *)malloc(sizeof(REAL) * N * C);
  for (int64_t n = 0; n < N; n++) memcpy(raw + n * C, P + m->wte + (int64_t)ids[n] * C, sizeof(REAL) * C);
  rmsnorm_rows(x, raw, N, C);
  REAL lam_s = P[m->sml];
  const REAL *wsg = P + m->smg;
  REAL *smsig = NULL;
  if (ctx) {
    ctx->raw = raw;
    ctx->embn = dup_arr(x, (size_t)N * C);
    smsig = (REAL *)calloc((size_t)B * (T > 1 ? T - 1 : 1), sizeof(REAL));
    ctx->smsig = smsig;
  }
  /* smear (transformer.go:266-301, helpers.go:35-65) */
  {
    REAL *gate = (REAL *)calloc((size_t)B * (T > 1 ? T - 1 : 1), sizeof(REAL));
    for (int b = 0; b < B; b++)
      for (int t = 1; t < T; t++) {
        double a = 0;
        for (int c = 0; c < SMEAR_CH; c++) a += (double)x[((int64_t)b * T + t) * C + c] * (double)wsg[c];
        REAL sg = sigmoidR(R(a));
        if (smsig) smsig[b * (T - 1) + t - 1] = sg;
        gate[b * (T - 1) + t - 1] = sg * lam_s;
      }
    REAL *seed = NULL;
    int use_prev = cache && cache->has_prev;
    REAL *newprev = NULL;
    if (cache) {
      newprev = (REAL *)malloc(sizeof(REAL) * B * C);
      for (int b = 0; b < B; b++) memcpy(newprev + (int64_t)b * C, x + ((int64_t)b * T + T - 1) * C, sizeof(REAL) * C);
    }
    if (use_prev) {
      seed = (REAL *)malloc(sizeof(REAL) * B);
      for (int b = 0; b < B; b++) {
        double a = 0;
        for (int c = 0; c < SMEAR_CH; c++) a += (double)x[((int64_t)b * T) * C + c] * (double)wsg[c];
        seed[b] = sigmoidR(R(a)) * lam_s;
      }
    }
    if (!cache && T <= 1) { fprintf(stderr, "oracle: training forward requires T > 1\n"); abort(); }
    for (int b = 0; b < B; b++)
      for (int t = T - 1; t >= 1; t--) {
        REAL gv = gate[b * (T - 1) + t - 1];
        REAL *cur = x + ((int64_t)b * T + t) * C, *prv = x + ((int64_t)b * T + t - 1) * C;
        for (int c = 0; c < C; c++) cur[c] += gv * prv[c];
      }
    if (seed)
      for (int b = 0; b < B; b++) {
        REAL *cur = x + ((int64_t)b * T) * C;
        for (int c = 0; c < C; c++) cur[c] += seed[b] * cache->prev[(int64_t)b * C + c];
      }
    if (cache) {
      memcpy(cache->prev, newprev, sizeof(REAL) * B * C);
      cache->has_prev = 1;
      free(newprev);
    }
    free(seed);
    free(gate);
  }
  if (!ctx) free(raw);
  x0 = dup_arr(x, (size_t)N * C);
  if (ctx) ctx->x0 = x0;
layers:;

  int offset = cache ? cache->pos : 0;
  int klen = cache ? cache->pos + T : T;
  int ratio = Hq / Hkv;
  int bkidx = m->L / 2;
  REAL *backout = NULL;
  REAL *h = (REAL *)malloc(sizeof(REAL) * N * C);
  REAL *q = (REAL *)malloc(sizeof(REAL) * N * Hq * D);
  REAL *k = (REAL *)malloc(sizeof(REAL) * N * Hkv * D);
  REAL *v = (REAL *)malloc(sizeof(REAL) * N * Hkv * D);
  REAL *o = (REAL *)malloc(sizeof(REAL) * N * Hq * D);
  REAL *a = (REAL *)malloc(sizeof(REAL) * N * C);
  REAL *u = (REAL *)malloc(sizeof(REAL) * N * F);
  REAL *act = (REAL *)malloc(sizeof(REAL) * N * F);
  REAL *qn = (REAL *)malloc(sizeof(REAL) * N * Hq * D);
  REAL *kn = (REAL *)malloc(sizeof(REAL) * N * Hkv * D);
  REAL *vesig = (REAL *)malloc(sizeof(REAL) * N * Hkv);
  REAL *vev = (REAL *)malloc(sizeof(REAL) * N * Hkv * D);
  REAL *lseb = (REAL *)malloc(sizeof(REAL) * N * Hq);
  for (int l = l_begin; l < l_end; l++) {
    const layer_off *lo = &m->lay[l];
    layer_ctx *lc = ctx ? &ctx->lc[l] : NULL;
    if (m->split > 0 && l == m->split) { /* encoderHidden (transformer.go:310-312) */
      enc = dup_arr(x, (size_t)N * C);
      if (ctx) ctx->enc = enc;
    }
    const REAL *enc_l = (m->split > 0 && l >= m->split) ? enc : NULL;
    if (lc) lc->xin = dup_arr(x, (size_t)N * C);
    /* combineResidual (transformer.go:544-551) */
    REAL lr = P[m->rl + l], l0 = P[m->x0l + l];
    for (int64_t i = 0; i < N * C; i++) x[i] = lr * x[i] + l0 * x0[i];
    if (lc) lc->xb = dup_arr(x, (size_t)N * C);
    /* attention on norm(x) */
    rmsnorm_rows(h, x, N, C);
    if (lc) lc->h = dup_arr(h, (size_t)N * C);
    if (m->mla && cache) { /* absorbed MLA against the latent cache */
      mla_decode_attention(m, lo, l, h, B, T, cache, o);
      goto attn_out;
    }
    if (m->mla) {
      REAL *ql, *kvl;
      mla_project(m, lo, h, N, q, k, v, &ql, &kvl);
      if (lc) { lc->ql = ql; lc->kvl = kvl; } else { free(ql); free(kvl); }
    } else {
      linear_fwd(q, h, P + lo->wq, N, C, Hq * D);
      linear_fwd(k, h, P + lo->wk, N, C, Hkv * D);
      linear_fwd(v, h, P + lo->wv, N, C, Hkv * D);
    }
    if (lo->has_ve) { /* attention.go:245-250, 392-405 */
      for (int64_t n = 0; n < N; n++) memcpy(vev + n * Hkv * D, P + lo->ve + (int64_t)ids[n] * Hkv * D, sizeof(REAL) * Hkv * D);
      for (int64_t n = 0; n < N; n++)
        for (int hh = 0; hh < Hkv; hh++) {
          double acc = 0;
          for (int c = 0; c < VE_GATE_CH; c++) acc += (double)h[n * C + c] * (double)P[lo->wve + hh * VE_GATE_CH + c];
          REAL sg = sigmoidR(R(acc));
          vesig[n * Hkv + hh] = sg;
          REAL g = sg * R(VE_GATE_SCALE);
          for (int d = 0; d < D; d++) v[(n * Hkv + hh) * D + d] += g * vev[(n * Hkv + hh) * D + d];
        }
      if (lc) { lc->vesig = dup_arr(vesig, (size_t)N * Hkv); lc->ve = dup_arr(vev, (size_t)N * Hkv * D); }
    }
    /* rotary then 1.2*RMSNorm per head (attention.go:252-256) */
    for (int b = 0; b < B; b++)
      for (int t = 0; t < T; t++) {
        int64_t n = (int64_t)b * T + t;
        rope_row(m, q + n * Hq * D, q + n * Hq * D, Hq, offset + t, 1);
        rope_row(m, k + n * Hkv * D, k + n * Hkv * D, Hkv, offset + t, 1);
      }
    if (m->mla) { /* no QK-norm under MLA (train.go:82-85) */
      memcpy(qn, q, sizeof(REAL) * N * Hq * D);
      memcpy(kn, k, sizeof(REAL) * N * Hkv * D);
    } else {
      if (lc) { lc->qrot = dup_arr(q, (size_t)N * Hq * D); lc->krot = dup_arr(k, (size_t)N * Hkv * D); }
      rmsnorm_rows(qn, q, N * Hq, D);
      rmsnorm_rows(kn, k, N * Hkv, D);
      for (int64_t i = 0; i < N * Hq * D; i++) qn[i] *= R(QK_SCALE);
      for (int64_t i = 0; i < N * Hkv * D; i++) kn[i] *= R(QK_SCALE);
    }
    /* head-major copies and KV-cache write (attention.go:277-303) */
    REAL *qh = (REAL *)malloc(sizeof(REAL) * N * Hq * D);
    REAL *oh = (REAL *)malloc(sizeof(REAL) * N * Hq * D);
    REAL *kh = (REAL *)malloc(sizeof(REAL) * (int64_t)B * Hkv * klen * D);
    REAL *vh = (REAL *)malloc(sizeof(REAL) * (int64_t)B * Hkv * klen * D);
    for (int b = 0; b < B; b++)
      for (int t = 0; t < T; t++)
        for (int hh = 0; hh < Hq; hh++)
          memcpy(qh + (((int64_t)b * Hq + hh) * T + t) * D, qn + (((int64_t)b * T + t) * Hq + hh) * D, sizeof(REAL) * D);
    for (int b = 0; b < B; b++)
      for (int hh = 0; hh < Hkv; hh++) {
        REAL *kd = kh + ((int64_t)b * Hkv + hh) * klen * D, *vd = vh + ((int64_t)b * Hkv + hh) * klen * D;
        if (cache) {
          REAL *ck = cache_k(m, cache, l, b, hh), *cv = cache_v(m, cache, l, b, hh);
          for (int t = 0; t < T; t++) {
            memcpy(ck + (int64_t)(offset + t) * D, kn + (((int64_t)b * T + t) * Hkv + hh) * D, sizeof(REAL) * D);
            memcpy(cv + (int64_t)(offset + t) * D, v + (((int64_t)b * T + t) * Hkv + hh) * D, sizeof(REAL) * D);
          }
          memcpy(kd, ck, sizeof(REAL) * klen * D);
          memcpy(vd, cv, sizeof(REAL) * klen * D);
        } else {
          for (int t = 0; t < T; t++) {
            memcpy(kd + (int64_t)t * D, kn + (((int64_t)b * T + t) * Hkv + hh) * D, sizeof(REAL) * D);
            memcpy(vd + (int64_t)t * D, v + (((int64_t)b * T + t) * Hkv + hh) * D, sizeof(REAL) * D);
          }
        }
      }
    if (m->ratio > 1 && cache) {
      if (lo->mode == REUSE_FULL) { /* a new group: fresh share (transformer.go:320-325) */
        free(ds.sel); free(ds.nsel); free(ds.pool); free(ds.npool);
        memset(&ds, 0, sizeof ds);
      }
      hca_decode(m, lo, l, cache, h, qh, kn, v, enc_l, replay, B, T, oh, &ds);
    } else if (m->ratio > 1) {
      hca_ctx *hc = (hca_ctx *)calloc(1, sizeof(hca_ctx));
      hca_train_forward(m, lo, qh, kh, vh, h, enc_l, B, T, oh, lseb, hc, &cur_share);
      if (lo->mode == REUSE_FULL) shares[l] = cur_share;
      if (lc) lc->hca = hc;
      else hcs[l] = hc;
    } else {
#pragma omp parallel for schedule(dynamic)
    for (int bh = 0; bh < B * Hq; bh++) {
      int b = bh / Hq, hq = bh % Hq, hk = hq / ratio;
      attn_fwd(qh + (int64_t)bh * T * D, kh + ((int64_t)b * Hkv + hk) * klen * D,
               vh + ((int64_t)b * Hkv + hk) * klen * D, oh + (int64_t)bh * T * D,
               lseb + (int64_t)bh * T, T, klen, D, offset, lo->window);
    }
    }
    if (lc) {
      lc->qn = qh; lc->kn = kh; lc->vh = vh;
      lc->o = dup_arr(oh, (size_t)N * Hq * D);
      lc->lse = dup_arr(lseb, (size_t)N * Hq);
    } else {
      free(qh); free(kh); free(vh);
    }
    /* back to sequence layout, output projection, residual */
    for (int b = 0; b < B; b++)
      for (int t = 0; t < T; t++)
        for (int hh = 0; hh < Hq; hh++)
          memcpy(o + (((int64_t)b * T + t) * Hq + hh) * D, oh + (((int64_t)b * Hq + hh) * T + t) * D, sizeof(REAL) * D);
    free(oh);
  attn_out:
    linear_fwd(a, o, P + lo->wo, N, Hq * D, C);
    for (int64_t i = 0; i < N * C; i++) x[i] = x[i] + a[i];
    if (lc) lc->mid = dup_arr(x, (size_t)N * C);
    /* MLP (mlp.go:62-77) */
    rmsnorm_rows(h, x, N, C);
    if (lc) lc->h2 = dup_arr(h, (size_t)N * C);
    linear_fwd(u, h, P + lo->wfc, N, C, F);
    if (m->E > 0) { /* shared SwiGLU expert (mlp.go:62-76) + routed experts (block.go:40-45) */
      REAL *g2 = (REAL *)malloc(sizeof(REAL) * N * F);
      linear_fwd(g2, h, P + lo->wgate, N, C, F);
      swiglu_fwd(act, g2, u, m->clamp, N * F);
      if (lc) lc->g2 = g2; else free(g2);
    } else {
      for (int64_t i = 0; i < N * F; i++) {
        REAL t = u[i] < 0 ? R(0) : u[i];
        act[i] = t * t;
      }
    }
    if (lc) { lc->u = dup_arr(u, (size_t)N * F); lc->act = dup_arr(act, (size_t)N * F); }
    linear_fwd(a, act, P + lo->wproj, N, F, C);
    if (m->E > 0) {
      REAL *mo = (REAL *)malloc(sizeof(REAL) * N * C);
      moe_forward(m, lo, h, N, lc ? T : 0, mo, lc ? &lc->moe : NULL);
      if (lc) m->aux_loss += lc->moe->bal_loss;
      for (int64_t i = 0; i < N * C; i++) a[i] = a[i] + mo[i];
      free(mo);
    }
    for (int64_t i = 0; i < N * C; i++) x[i] = x[i] + a[i];
    if (l == bkidx) backout = dup_arr(x, (size_t)N * C);
  }
  if (cache && !(op && op->no_advance)) cache->pos += T;
  for (int l = 0; l < m->L; l++) {
    hca_ctx_free(hcs[l]);
    if (ctx) ctx->shares[l] = shares[l];
    else hca_share_free(shares[l]);
  }
  free(ds.sel); free(ds.nsel); free(ds.pool); free(ds.npool);
  if (!ctx) free(enc);
  if (op && op->x_out) memcpy(op->x_out, x, sizeof(REAL) * N * C);
  if (!logits) {
    free(backout);
    goto done;
  }
  /* backout, final norm, lm_head, trimVocab, softcap (transformer.go:333-341) */
  if (backout) {
    REAL nb = -P[m->bkl];
    for (int64_t i = 0; i < N * C; i++) x[i] = x[i] + nb * backout[i];
  }
  if (ctx) { ctx->backout = backout; ctx->final_pre = dup_arr(x, (size_t)N * C); } else free(backout);
  rmsnorm_rows(h, x, N, C);
  if (ctx) ctx->final_norm = dup_arr(h, (size_t)N * C);
#pragma omp parallel for schedule(static)
  for (int64_t n = 0; n < N; n++)
    for (int j = 0; j < V; j++) {
      double acc = 0;
      const REAL *w = P + m->lm + (int64_t)j * C;
      for (int c = 0; c < C; c++) acc += (double)h[n * C + c] * (double)w[c];
      logits[n * V + j] = softcap(R(acc));
    }
  (void)PV;
done:
  if (!ctx) free(x0);
  free(x); free(h); free(q); free(k); free(v); free(o); free(a); free(u); free(act);
  free(qn); free(kn); free(vesig); free(vev); free(lseb);
}

/* PrefillCED (transformer.go:363-449) of a batch-1 prompt: the encoder over
 * the full prompt; every decoder Full layer's global compressed cache filled
 * from its projections of the encoder's final hidden state (Reindex layers
 * cache their indexer keys); the decoder replayed over the last SWA-window
 * tokens from the encoder rows, with embedAndSmear's smear (the first
 * replayed row is not mixed with the previous token; a single replayed row
 * is mixed with the cached previous embedding, which is its own).  Writes
 * the last replayed row's logits; the cache ends at the prompt length. */
static void prefill_ced(MODEL *m, const int32_t *ids, int T, kvcache *cache, REAL *last_logits) {
  const int C = m->C, split = m->split, V = m->V, D = m->D, Hkv = m->Hkv;
  int replay_len = m->swa < T ? m->swa : T;
  const int rstart = T - replay_len;
  /* phase 1: the encoder (embedAndSmear with a fresh cache: smearAdd) */
  REAL *enc = (REAL *)malloc(sizeof(REAL) * (int64_t)T * C);
  fwd_opts op1 = {0, split, 0, 1, NULL, NULL, enc};
  forward_run(m, ids, 1, T, cache, NULL, NULL, &op1);
  /* phase 2: decoder global caches from the encoder hidden state */
  REAL *ks = (REAL *)malloc(sizeof(REAL) * (int64_t)T * Hkv * D);
  REAL *vs = (REAL *)malloc(sizeof(REAL) * (int64_t)T * Hkv * D);
  for (int l = split; l < m->L; l++) {
    const layer_off *lo = &m->lay[l];
    if (lo->mode == REUSE_FULL) {
      ced_kv(m, lo, enc, 1, T, 0, ks, vs, NULL);
      append_global_tail(m, lo, l, cache, enc, ks, vs, 1, T);
    } else if (lo->mode == REUSE_REINDEX && m->topk > 0) {
      cache_reused_indexer_keys(m, lo, l, cache, 1);
    }
  }
  free(ks); free(vs);
  /* phase 3: bounded replay (embedAndSmear, transformer.go:452-477) */
  const int32_t *rids = ids + rstart;
  REAL *xr = (REAL *)malloc(sizeof(REAL) * (int64_t)replay_len * C);
  const REAL *P = m->p, *wsg = P + m->smg;
  const REAL lam = P[m->sml];
  for (int t = 0; t < replay_len; t++) {
    REAL *row = xr + (int64_t)t * C;
    memcpy(row, P + m->wte + (int64_t)rids[t] * C, sizeof(REAL) * C);
    rmsnorm_rows(row, row, 1, C);
  }
  REAL *prev = cache->has_prev ? dup_arr(cache->prev, (size_t)C) : NULL;
  memcpy(cache->prev, xr + (int64_t)(replay_len - 1) * C, sizeof(REAL) * C);
  cache->has_prev = 1;
  if (replay_len > 1) {
    REAL *gate = (REAL *)malloc(sizeof(REAL) * replay_len);
    for (int t = 1; t < replay_len; t++) {
      double a = 0;
      for (int c = 0; c < SMEAR_CH; c++) a += (double)xr[(int64_t)t * C + c] * (double)wsg[c];
      gate[t] = sigmoidR(R(a)) * lam;
    }
    for (int t = replay_len - 1; t >= 1; t--)
      for (int c = 0; c < C; c++) xr[(int64_t)t * C + c] += gate[t] * xr[(int64_t)(t - 1) * C + c];
    free(gate);
  } else if (prev) {
    double a = 0;
    for (int c = 0; c < SMEAR_CH; c++) a += (double)xr[c] * (double)wsg[c];
    REAL g = sigmoidR(R(a)) * lam;
    for (int c = 0; c < C; c++) xr[c] += g * prev[c];
  }
  free(prev);
  cache->pos = rstart;
  REAL *lg = (REAL *)malloc(sizeof(REAL) * (int64_t)replay_len * V);
  fwd_opts op3 = {split, m->L, 1, 1, enc + (int64_t)rstart * C, xr, NULL};
  forward_run(m, rids, 1, replay_len, cache, lg, NULL, &op3);
  memcpy(last_logits, lg + (int64_t)(replay_len - 1) * V, sizeof(REAL) * V);
  cache->pos = T;
  free(lg); free(xr); free(enc);
}

void FN(orc_forward)(MODEL *m, const int32_t *ids, int B, int T, REAL *logits) {
  forward_impl(m, ids, B, T, NULL, logits, NULL);
}

/* PrefillCED of a batch-1 prompt into a fresh cache; the last replayed row's
 * logits [V] (the row Engine.GenerateWith samples from). */
void FN(orc_prefill_ced)(MODEL *m, const int32_t *ids, int T, REAL *last_logits) {
  kvcache *c = cache_new(m, 1, T);
  prefill_ced(m, ids, T, c, last_logits);
  cache_free(c);
}

/* Token-by-token (or chunked) KV-cache decode, the invariant
 * model/smear_test.go:30-82 checks against the full forward. */
void FN(orc_forward_decode)(MODEL *m, const int32_t *ids, int B, int T, int chunk, REAL *logits) {
  kvcache *c = cache_new(m, B, T);
  if (chunk < 1) chunk = 1;
  int32_t *col = (int32_t *)malloc(sizeof(int32_t) * B * chunk);
  REAL *lg = (REAL *)malloc(sizeof(REAL) * (int64_t)B * chunk * m->V);
  for (int t0 = 0; t0 < T; t0 += chunk) {
    int n = T - t0 < chunk ? T - t0 : chunk;
    for (int b = 0; b < B; b++)
      for (int j = 0; j < n; j++) col[b * n + j] = ids[b * T + t0 + j];
    forward_impl(m, col, B, n, c, lg, NULL);
    for (int b = 0; b < B; b++)
      for (int j = 0; j < n; j++)
        memcpy(logits + ((int64_t)b * T + t0 + j) * m->V, lg + ((int64_t)b * n + j) * m->V, sizeof(REAL) * m->V);
  }
  free(col);
  free(lg);
  cache_free(c);
}

/* ---- backward (model/train_transformer.go:147-320, model/train.go) ---- */

/* Block backward (model/train.go:554-572 with 198-427 and 505-514). Returns
 * the gradient with respect to the block input in gx; parameter gradients
 * accumulate into G. */
static void block_backward(MODEL *m, const layer_ctx *lc, const layer_off *lo, const int32_t *ids,
                           int B, int T, const REAL *gout, REAL *gx, REAL *genc, REAL *G) {
  int C = m->C, Hq = m->Hq, Hkv = m->Hkv, D = m->D, F = m->F, ratio = Hq / Hkv;
  int64_t N = (int64_t)B * T;
  const REAL *P = m->p;
  REAL *gmid = dup_arr(gout, (size_t)N * C);
  /* MLP backward */
  REAL *dact = (REAL *)malloc(sizeof(REAL) * N * F);
  linear_bwd(dact, G + lo->wproj, lc->act, gout, P + lo->wproj, N, F, C);
  REAL *dh = (REAL *)malloc(sizeof(REAL) * N * C);
  REAL *tmp = (REAL *)malloc(sizeof(REAL) * N * C);
  if (m->E > 0) { /* train.go:505-511 (SwiGLU shared expert), then moe.go:203-267 */
    REAL *dg = (REAL *)malloc(sizeof(REAL) * N * F), *du = (REAL *)malloc(sizeof(REAL) * N * F);
    swiglu_bwd(dg, du, lc->g2, lc->u, dact, m->clamp, N * F);
    linear_bwd(dh, G + lo->wgate, lc->h2, dg, P + lo->wgate, N, C, F);
    linear_bwd(tmp, G + lo->wfc, lc->h2, du, P + lo->wfc, N, C, F);
    for (int64_t i = 0; i < N * C; i++) dh[i] = dh[i] + tmp[i];
    moe_backward(m, lo, lc->moe, lc->h2, gout, tmp, G);
    for (int64_t i = 0; i < N * C; i++) dh[i] = dh[i] + tmp[i];
    free(dg); free(du);
  } else {
    for (int64_t i = 0; i < N * F; i++) dact[i] = lc->u[i] > 0 ? dact[i] * R(2) * lc->u[i] : R(0);
    linear_bwd(dh, G + lo->wfc, lc->h2, dact, P + lo->wfc, N, C, F);
  }
  free(dact);
  rmsnorm_backward_rows(tmp, lc->mid, dh, N, C);
  for (int64_t i = 0; i < N * C; i++) gmid[i] = gmid[i] + tmp[i];
  /* attention backward */
  REAL *oseq = (REAL *)malloc(sizeof(REAL) * N * Hq * D);
  for (int b = 0; b < B; b++)
    for (int t = 0; t < T; t++)
      for (int hh = 0; hh < Hq; hh++)
        memcpy(oseq + (((int64_t)b * T + t) * Hq + hh) * D, lc->o + (((int64_t)b * Hq + hh) * T + t) * D, sizeof(REAL) * D);
  REAL *dos = (REAL *)malloc(sizeof(REAL) * N * Hq * D);
  linear_bwd(dos, G + lo->wo, oseq, gmid, P + lo->wo, N, Hq * D, C);
  free(oseq);
  REAL *doh = (REAL *)malloc(sizeof(REAL) * N * Hq * D);
  for (int b = 0; b < B; b++)
    for (int t = 0; t < T; t++)
      for (int hh = 0; hh < Hq; hh++)
        memcpy(doh + (((int64_t)b * Hq + hh) * T + t) * D, dos + (((int64_t)b * T + t) * Hq + hh) * D, sizeof(REAL) * D);
  free(dos);
  REAL *dqh = (REAL *)calloc((size_t)N * Hq * D, sizeof(REAL));
  REAL *dkh = (REAL *)calloc((size_t)N * Hkv * D, sizeof(REAL));
  REAL *dvh = (REAL *)calloc((size_t)N * Hkv * D, sizeof(REAL));
  REAL *dhin_c = NULL;
  if (m->ratio > 1) {
    dhin_c = (REAL *)malloc(sizeof(REAL) * N * C);
    hca_train_backward(m, lo, lc->hca, lc->qn, lc->kn, lc->vh, lc->o, doh, lc->lse, lc->h, B, T,
                       dqh, dkh, dvh, dhin_c, genc, G);
  } else {
  /* serial (b, qh) loop as train.go:305-326 so GQA accumulation is race-free */
  for (int b = 0; b < B; b++)
#pragma omp parallel for schedule(dynamic)
    for (int hk = 0; hk < Hkv; hk++)
      for (int r = 0; r < ratio; r++) {
        int hq = hk * ratio + r;
        int64_t bh = (int64_t)b * Hq + hq, bk = (int64_t)b * Hkv + hk;
        attn_bwd(lc->qn + bh * T * D, lc->kn + bk * T * D, lc->vh + bk * T * D, doh + bh * T * D,
                 lc->lse + bh * T, dqh + bh * T * D, dkh + bk * T * D, dvh + bk * T * D, T, T, D, 0,
                 lo->window);
      }
  }
  free(doh);
  if (!m->mla) { /* unscale QK (train.go:331-333); MLA has no QK norm */
    for (int64_t i = 0; i < N * Hq * D; i++) dqh[i] *= R(QK_SCALE);
    for (int64_t i = 0; i < N * Hkv * D; i++) dkh[i] *= R(QK_SCALE);
  }
  REAL *dqs = (REAL *)malloc(sizeof(REAL) * N * Hq * D);
  REAL *dks = (REAL *)malloc(sizeof(REAL) * N * Hkv * D);
  REAL *dvs = (REAL *)malloc(sizeof(REAL) * N * Hkv * D);
  for (int b = 0; b < B; b++)
    for (int t = 0; t < T; t++) {
      for (int hh = 0; hh < Hq; hh++)
        memcpy(dqs + (((int64_t)b * T + t) * Hq + hh) * D, dqh + (((int64_t)b * Hq + hh) * T + t) * D, sizeof(REAL) * D);
      for (int hh = 0; hh < Hkv; hh++) {
        memcpy(dks + (((int64_t)b * T + t) * Hkv + hh) * D, dkh + (((int64_t)b * Hkv + hh) * T + t) * D, sizeof(REAL) * D);
        memcpy(dvs + (((int64_t)b * T + t) * Hkv + hh) * D, dvh + (((int64_t)b * Hkv + hh) * T + t) * D, sizeof(REAL) * D);
      }
    }
  free(dqh); free(dkh); free(dvh);
  REAL *dq = (REAL *)malloc(sizeof(REAL) * N * Hq * D);
  REAL *dk = (REAL *)malloc(sizeof(REAL) * N * Hkv * D);
  if (m->mla) {
    memcpy(dq, dqs, sizeof(REAL) * N * Hq * D);
    memcpy(dk, dks, sizeof(REAL) * N * Hkv * D);
  } else {
    rmsnorm_backward_rows(dq, lc->qrot, dqs, N * Hq, D);
    rmsnorm_backward_rows(dk, lc->krot, dks, N * Hkv, D);
  }
  for (int b = 0; b < B; b++)
    for (int t = 0; t < T; t++) {
      int64_t n = (int64_t)b * T + t;
      rope_row(m, dq + n * Hq * D, dq + n * Hq * D, Hq, t, -1);
      rope_row(m, dk + n * Hkv * D, dk + n * Hkv * D, Hkv, t, -1);
    }
  REAL *dhin = (REAL *)malloc(sizeof(REAL) * N * C);
  if (m->mla) { /* train.go:371-419: zero, then the MLA projection backward */
    mla_project_backward(m, lo, lc->h, lc->ql, lc->kvl, dq, dk, dvs, N, tmp, G);
    for (int64_t i = 0; i < N * C; i++) dhin[i] = R(0) + tmp[i];
  } else {
    linear_bwd(dhin, G + lo->wq, lc->h, dq, P + lo->wq, N, C, Hq * D);
    linear_bwd(tmp, G + lo->wk, lc->h, dk, P + lo->wk, N, C, Hkv * D);
    for (int64_t i = 0; i < N * C; i++) dhin[i] = dhin[i] + tmp[i];
    linear_bwd(tmp, G + lo->wv, lc->h, dvs, P + lo->wv, N, C, Hkv * D);
    for (int64_t i = 0; i < N * C; i++) dhin[i] = dhin[i] + tmp[i];
  }
  free(dq); free(dk);
  if (lo->has_ve) { /* model/train.go:369-397 */
    REAL *dpre = (REAL *)malloc(sizeof(REAL) * N * Hkv);
    for (int64_t n = 0; n < N; n++)
      for (int hh = 0; hh < Hkv; hh++) {
        int64_t row = n * Hkv + hh;
        REAL sg = lc->vesig[row];
        REAL scale = sg * R(VE_GATE_SCALE);
        double dot = 0;
        for (int d = 0; d < D; d++) {
          REAL gvd = dvs[row * D + d];
          /* value_embeds gradient scatter (Embedding.Backward, linear.go:90-104) */
          G[lo->ve + (int64_t)ids[n] * Hkv * D + hh * D + d] += gvd * scale;
          dot += (double)gvd * (double)lc->ve[row * D + d];
        }
        REAL gsig = R(dot) * R(VE_GATE_SCALE);
        dpre[row] = gsig * sg * (R(1) - sg);
      }
    REAL *slice = (REAL *)malloc(sizeof(REAL) * N * VE_GATE_CH);
    for (int64_t n = 0; n < N; n++) memcpy(slice + n * VE_GATE_CH, lc->h + n * C, sizeof(REAL) * VE_GATE_CH);
    REAL *dslice = (REAL *)malloc(sizeof(REAL) * N * VE_GATE_CH);
    linear_bwd(dslice, G + lo->wve, slice, dpre, P + lo->wve, N, VE_GATE_CH, Hkv);
    for (int64_t n = 0; n < N; n++)
      for (int c = 0; c < VE_GATE_CH; c++) dhin[n * C + c] += dslice[n * VE_GATE_CH + c];
    free(dpre); free(slice); free(dslice);
  }
  free(dvs);
  if (dhin_c) { /* the compressor's logit projection reads the attention input (train.go:421-424) */
    for (int64_t i = 0; i < N * C; i++) dhin[i] = dhin[i] + dhin_c[i];
    free(dhin_c);
  }
  rmsnorm_backward_rows(gx, lc->xb, dhin, N, C);
  for (int64_t i = 0; i < N * C; i++) gx[i] = gx[i] + gmid[i];
  free(dhin); free(tmp); free(gmid); free(dh);
}

/* TrainBackward (train_transformer.go:147-156) from dL/d(softcapped logits). */
static void train_backward(MODEL *m, train_ctx *ctx, const REAL *glogits, REAL *G) {
  int B = ctx->B, T = ctx->T, C = m->C, V = m->V, PV = m->PV, L = m->L;
  int64_t N = (int64_t)B * T;
  const REAL *P = m->p;
  /* SoftcapBackward (tensors/backward.go:108-116) and vocab padding */
  REAL *gp = (REAL *)calloc((size_t)N * PV, sizeof(REAL));
  REAL inv = R(1) / R(SOFTCAP);
#pragma omp parallel for schedule(static)
  for (int64_t n = 0; n < N; n++)
    for (int j = 0; j < V; j++) {
      double s = (double)ctx->logits[n * V + j] * (double)inv;
      gp[n * PV + j] = glogits[n * V + j] * R(1 - s * s);
    }
  REAL *g = (REAL *)malloc(sizeof(REAL) * N * C);
  linear_bwd(g, G + m->lm, ctx->final_norm, gp, P + m->lm, N, C, PV);
  free(gp);
  /* trainBackwardFromHidden (train_transformer.go:176-265) */
  REAL *ga = (REAL *)malloc(sizeof(REAL) * N * C);
  rmsnorm_backward_rows(ga, ctx->final_pre, g, N, C);
  REAL *gback = NULL;
  if (ctx->backout) {
    gback = (REAL *)malloc(sizeof(REAL) * N * C);
    REAL nb = -P[m->bkl];
    double dot = 0;
    for (int64_t i = 0; i < N * C; i++) {
      gback[i] = ga[i] * nb;
      dot += (double)ga[i] * (double)(-ctx->backout[i]);
    }
    G[m->bkl] += R(dot);
  }
  int bkidx = L / 2;
  if (m->split > 0) ctx->ced_genc = (REAL *)calloc((size_t)N * C, sizeof(REAL));
  REAL *gx0 = (REAL *)calloc((size_t)N * C, sizeof(REAL));
  REAL *gb = (REAL *)malloc(sizeof(REAL) * N * C);
  REAL *lg = (REAL *)malloc(sizeof(REAL) * N * C);
  for (int l = L - 1; l >= 0; l--) {
    memcpy(lg, ga, sizeof(REAL) * N * C);
    if (l == bkidx && gback)
      for (int64_t i = 0; i < N * C; i++) lg[i] = lg[i] + gback[i];
    block_backward(m, &ctx->lc[l], &m->lay[l], ctx->ids, B, T, lg, gb, ctx->ced_genc, G);
    REAL lr = P[m->rl + l], l0 = P[m->x0l + l];
    double rdot = 0, idot = 0;
    for (int64_t i = 0; i < N * C; i++) {
      ga[i] = gb[i] * lr;
      gx0[i] = gx0[i] + l0 * gb[i];
      rdot += (double)gb[i] * (double)ctx->lc[l].xin[i];
      idot += (double)gb[i] * (double)ctx->x0[i];
    }
    if (m->split > 0 && l == m->split) /* the decoder's global-KV gradient (:221-229) */
      for (int64_t i = 0; i < N * C; i++) ga[i] = ga[i] + ctx->ced_genc[i];
    G[m->rl + l] += R(rdot);
    G[m->x0l + l] += R(idot);
  }
  for (int64_t i = 0; i < N * C; i++) ga[i] = ga[i] + gx0[i];
  /* smearBackward (train_transformer.go:269-305) */
  REAL *ge = (REAL *)calloc((size_t)N * C, sizeof(REAL));
  int Tm = T > 1 ? T - 1 : 1;
  REAL *ggate = (REAL *)calloc((size_t)B * Tm, sizeof(REAL));
  REAL lam = P[m->sml];
  double dlam = 0;
  for (int b = 0; b < B; b++)
    for (int t = 0; t < T; t++) {
      int64_t base = ((int64_t)b * T + t) * C;
      if (t == 0) {
        for (int c = 0; c < C; c++) ge[base + c] += ga[base + c];
        continue;
      }
      int gi = b * (T - 1) + t - 1;
      REAL sg = ctx->smsig[gi];
      REAL gv = lam * sg;
      int64_t pb = ((int64_t)b * T + t - 1) * C;
      double gs = 0;
      for (int c = 0; c < C; c++) {
        ge[base + c] += ga[base + c];
        ge[pb + c] += ga[base + c] * gv;
        gs += (double)ga[base + c] * (double)ctx->embn[pb + c];
      }
      dlam += gs * (double)sg;
      ggate[gi] = R(gs * (double)lam) * sg * (R(1) - sg);
    }
  G[m->sml] += R(dlam);
  if (T > 1) {
    int64_t NS = (int64_t)B * (T - 1);
    REAL *slice = (REAL *)malloc(sizeof(REAL) * NS * SMEAR_CH);
    REAL *gsl = (REAL *)malloc(sizeof(REAL) * NS * SMEAR_CH);
    for (int b = 0; b < B; b++)
      for (int t = 1; t < T; t++)
        memcpy(slice + ((int64_t)b * (T - 1) + t - 1) * SMEAR_CH, ctx->embn + ((int64_t)b * T + t) * C, sizeof(REAL) * SMEAR_CH);
    linear_bwd(gsl, G + m->smg, slice, ggate, P + m->smg, NS, SMEAR_CH, 1);
    for (int b = 0; b < B; b++)
      for (int t = 1; t < T; t++)
        for (int c = 0; c < SMEAR_CH; c++)
          ge[((int64_t)b * T + t) * C + c] += gsl[((int64_t)b * (T - 1) + t - 1) * SMEAR_CH + c];
    free(slice); free(gsl);
  }
  /* embedding norm backward, then the wte scatter-add (linear.go:90-104) */
  REAL *graw = (REAL *)malloc(sizeof(REAL) * N * C);
  rmsnorm_backward_rows(graw, ctx->raw, ge, N, C);
  for (int64_t n = 0; n < N; n++)
    for (int c = 0; c < C; c++) G[m->wte + (int64_t)ctx->ids[n] * C + c] += graw[n * C + c];
  free(graw); free(ge); free(ggate); free(gx0); free(gb); free(lg); free(ga); free(gback); free(g);
}

static train_ctx *train_forward(MODEL *m, const int32_t *ids, int B, int T) {
  train_ctx *ctx = (train_ctx *)calloc(1, sizeof(train_ctx));
  ctx->B = B;
  ctx->T = T;
  ctx->ids = (int32_t *)malloc(sizeof(int32_t) * B * T);
  memcpy(ctx->ids, ids, sizeof(int32_t) * B * T);
  ctx->logits = (REAL *)malloc(sizeof(REAL) * (int64_t)B * T * m->V);
  m->aux_loss = 0;
  forward_impl(m, ids, B, T, NULL, ctx->logits, ctx);
  return ctx;
}

/* trainer/rl.go:14-60 with tensors/loss.go:16-46 and tensors/norm.go:5-10. */
double FN(orc_pg_step)(MODEL *m, const int32_t *inputs, const int32_t *targets, int B, int T,
                        const float *adv, float norm, REAL *nll, REAL *grads) {
  int V = m->V;
  int64_t N = (int64_t)B * T;
  train_ctx *ctx = train_forward(m, inputs, B, T);
  REAL *glog = (REAL *)calloc((size_t)N * V, sizeof(REAL));
  double loss = 0;
#pragma omp parallel for schedule(static)
  for (int64_t n = 0; n < N; n++) {
    const REAL *row = ctx->logits + n * V;
    REAL mx = row[0];
    for (int j = 1; j < V; j++)
      if (row[j] > mx) mx = row[j];
    double s = 0;
    for (int j = 0; j < V; j++) s += exp((double)(row[j] - mx));
    int32_t tg = targets[n];
    nll[n] = tg == -1 ? R(0) : mx + R(log(s)) - row[tg];
    if (tg == -1) continue;
    /* SoftmaxLastDim then (p - onehot) * adv/norm with a float32 scale */
    REAL inv = R(1.0 / s);
    REAL scale = R(adv[n / T]) / R(norm);
    for (int j = 0; j < V; j++) {
      REAL p = R(exp((double)(row[j] - mx))) * inv;
      if (j == tg) p -= R(1);
      glog[n * V + j] = p * scale;
    }
  }
  for (int b = 0; b < B; b++)
    for (int t = 0; t < T; t++) {
      int64_t n = (int64_t)b * T + t;
      if (targets[n] == -1) continue;
      loss += (double)nll[n] * (double)adv[b] / (double)norm;
    }
  memset(grads, 0, sizeof(REAL) * m->total);
  train_backward(m, ctx, glog, grads);
  free(glog);
  ctx_free(ctx, m->L);
  return loss;
}

/* trainer.DistillStep (trainer/distill.go:13-46) for one micro-batch with
 * GradAccumSteps = accum, given the frozen teacher's logits [N, V]
 * (teacher.Forward): the forward-KL loss of every position whose mask is
 * non-zero (mask NULL: every position) and its gradient
 * (softmax(s/tau) - softmax(t/tau)) * scale / tau into the student's
 * parameters (tensors/loss.go:84-214, float64 exp and sums; losses float32
 * per row).  Returns the mean loss over the valid positions. */
double FN(orc_distill_step)(MODEL *m, const float *teacher, const int32_t *inputs,
                            const int32_t *mask, int B, int T, float temperature, int accum,
                            REAL *grads) {
  int V = m->V;
  int64_t N = (int64_t)B * T;
  train_ctx *ctx = train_forward(m, inputs, B, T);
  const double tau = temperature <= 0 ? 1.0 : (double)temperature;
  int valid = 0;
  for (int64_t n = 0; n < N; n++) valid += !mask || mask[n] != 0;
  const int vt = valid == 0 ? 1 : valid;
  const float scale = 1.0f / ((float)vt * (float)accum);
  REAL *losses = (REAL *)calloc((size_t)N, sizeof(REAL));
  REAL *glog = (REAL *)calloc((size_t)N * V, sizeof(REAL));
#pragma omp parallel for schedule(static)
  for (int64_t n = 0; n < N; n++) {
    if (mask && mask[n] == 0) continue;
    const REAL *sr = ctx->logits + n * V;
    const float *tr = teacher + n * V;
    double smax = -INFINITY, tmax = -INFINITY;
    for (int j = 0; j < V; j++) {
      const double a = (double)sr[j] / tau, b = (double)tr[j] / tau;
      if (a > smax) smax = a;
      if (b > tmax) tmax = b;
    }
    double ssum = 0, tsum = 0, wsum = 0;
    for (int j = 0; j < V; j++) {
      const double a = (double)sr[j] / tau, b = (double)tr[j] / tau;
      const double sw = exp(a - smax), tw = exp(b - tmax);
      ssum += sw;
      tsum += tw;
      wsum += tw * a;
    }
    losses[n] = (REAL)(smax + log(ssum) - wsum / tsum);
    const double is = 1.0 / ssum, it = 1.0 / tsum, gs = (double)scale / tau;
    for (int j = 0; j < V; j++) {
      const double ps = exp((double)sr[j] / tau - smax) * is;
      const double pt = exp((double)tr[j] / tau - tmax) * it;
      glog[n * V + j] = (REAL)((ps - pt) * gs);
    }
  }
  double sum = 0;
  for (int64_t n = 0; n < N; n++) sum += (double)losses[n];
  memset(grads, 0, sizeof(REAL) * m->total);
  train_backward(m, ctx, glog, grads);
  free(glog);
  free(losses);
  ctx_free(ctx, m->L);
  return (double)(REAL)(sum / (double)vt);
}

/* Mean cross-entropy and its gradient (model/gradcheck_test.go:94-110). */
double FN(orc_ce_loss)(MODEL *m, const int32_t *inputs, const int32_t *targets, int B, int T,
                        REAL *grads) {
  int V = m->V;
  int64_t N = (int64_t)B * T;
  train_ctx *ctx = train_forward(m, inputs, B, T);
  int valid = 0;
  for (int64_t n = 0; n < N; n++) valid += targets[n] != -1;
  double sum = 0;
  REAL *glog = grads ? (REAL *)calloc((size_t)N * V, sizeof(REAL)) : NULL;
  for (int64_t n = 0; n < N; n++) {
    if (targets[n] == -1) continue;
    const REAL *row = ctx->logits + n * V;
    REAL mx = row[0];
    for (int j = 1; j < V; j++)
      if (row[j] > mx) mx = row[j];
    double s = 0;
    for (int j = 0; j < V; j++) s += exp((double)(row[j] - mx));
    sum += (double)(mx + R(log(s)) - row[targets[n]]);
    if (glog) { /* tensors/backward.go:11-38 */
      double invs = 1.0 / s;
      REAL scale = R(1) / R(valid);
      for (int j = 0; j < V; j++) {
        REAL p = R(exp((double)(row[j] - mx)) * invs);
        if (j == targets[n]) p -= R(1);
        glog[n * V + j] = p * scale;
      }
    }
  }
  if (grads) {
    memset(grads, 0, sizeof(REAL) * m->total);
    train_backward(m, ctx, glog, grads);
    free(glog);
  }
  ctx_free(ctx, m->L);
  return valid ? sum / valid : 0;
}

/* ---- generation (inference/engine.go:112-369) -------------------------- */
enum { TOK_BOS = 256, TOK_ASSISTANT_END = 260, TOK_TOOL_START = 261, TOK_TOOL_END = 262,
       TOK_TOOL_OUT_START = 263, TOK_TOOL_OUT_END = 264 };

/* tokenizer.Decode for the byte-level tokenizer (tokenizer/tokenizer.go:110-118,
 * tokenizer/special.go:19-31): bytes, then special names, unknown ids skipped. */
static const char *SPECIAL_NAMES[11] = {
    "<|bos|>", "<|user_start|>", "<|user_end|>", "<|assistant_start|>", "<|assistant_end|>",
    "<|tool_start|>", "<|tool_end|>", "<|tool_output_start|>", "<|tool_output_end|>",
    "<|think_start|>", "<|think_end|>"};

typedef struct {
  int *forced, nforced, cap_forced;
  int in_tool, *tool, ntool, cap_tool;
  int completed;
} row_state;

void FN(orc_generate_batch)(MODEL *m, const int32_t *prompt, int P, int S, int max_tokens,
                            float temperature, int top_k, uint64_t seed, int32_t *rows_out,
                            int32_t *lens_out) {
  int V = m->V;
  kvcache *pre = cache_new(m, 1, P);
  REAL *lg = (REAL *)malloc(sizeof(REAL) * (int64_t)P * V);
  if (m->split > 0) /* engine.go:164-173 */
    prefill_ced(m, prompt, P, pre, lg + (int64_t)(P - 1) * V);
  else
    forward_impl(m, prompt, 1, P, pre, lg, NULL);
  float *logits = (float *)malloc(sizeof(float) * (int64_t)S * V);
  for (int s = 0; s < S; s++)
    for (int j = 0; j < V; j++) logits[(int64_t)s * V + j] = (float)lg[(int64_t)(P - 1) * V + j];
  free(lg);
  int cache_len = P + (max_tokens > 0 ? max_tokens : 0);
  kvcache *dec = cache_new(m, S, cache_len);
  prefill_from(m, dec, pre);
  cache_free(pre);
  row_state *st = (row_state *)calloc(S, sizeof(row_state));
  int W = P + max_tokens;
  int done_rows = 0;
  int *completed_out = (int *)calloc(S, sizeof(int));
  for (int s = 0; s < S; s++) {
    memcpy(rows_out + (int64_t)s * W, prompt, sizeof(int32_t) * P);
    lens_out[s] = P;
  }
  orc_pcg rng;
  orc_rng_new(&rng, seed);
  int32_t *next = (int32_t *)malloc(sizeof(int32_t) * S);
  int32_t *col = (int32_t *)malloc(sizeof(int32_t) * S);
  REAL *lg1 = (REAL *)malloc(sizeof(REAL) * (int64_t)S * V);
  int generated = 0;
  for (;;) {
    if (max_tokens > 0 && generated >= max_tokens) break;
    int all = 1;
    for (int s = 0; s < S; s++)
      if (!st[s].completed) { all = 0; break; }
    if (all) break;
    orc_sample_next_token(logits, S, V, &rng, temperature, top_k, next);
    for (int s = 0; s < S; s++) {
      row_state *r = &st[s];
      int tok;
      if (r->nforced > 0) {
        tok = r->forced[0];
        memmove(r->forced, r->forced + 1, sizeof(int) * (r->nforced - 1));
        r->nforced--;
      } else
        tok = next[s];
      col[s] = tok;
      if (tok == TOK_ASSISTANT_END || tok == TOK_BOS) r->completed = 1;
      if (tok == TOK_TOOL_START) {
        r->in_tool = 1;
        r->ntool = 0;
      } else if (tok == TOK_TOOL_END && r->in_tool) {
        r->in_tool = 0;
        if (r->ntool > 0) {
          char expr[8192];
          size_t e = 0;
          for (int i = 0; i < r->ntool; i++) {
            int id = r->tool[i];
            if (id >= 0 && id < 256) { if (e + 1 < sizeof expr) expr[e++] = (char)id; }
            else if (id >= 256 && id < 267) {
              const char *nm = SPECIAL_NAMES[id - 256];
              for (size_t k = 0; nm[k] && e + 1 < sizeof expr; k++) expr[e++] = nm[k];
            }
          }
          expr[e] = 0;
          char res[512];
          if (orc_calculator(expr, res, sizeof res)) {
            size_t rl = strlen(res);
            int need = r->nforced + (int)rl + 2;
            if (need > r->cap_forced) {
              r->cap_forced = need * 2;
              r->forced = (int *)realloc(r->forced, sizeof(int) * r->cap_forced);
            }
            r->forced[r->nforced++] = TOK_TOOL_OUT_START;
            for (size_t k = 0; k < rl; k++) r->forced[r->nforced++] = (unsigned char)res[k];
            r->forced[r->nforced++] = TOK_TOOL_OUT_END;
          }
        }
        r->ntool = 0;
      } else if (r->in_tool) {
        if (r->ntool + 1 > r->cap_tool) {
          r->cap_tool = (r->ntool + 1) * 2;
          r->tool = (int *)realloc(r->tool, sizeof(int) * r->cap_tool);
        }
        r->tool[r->ntool++] = tok;
      }
    }
    /* GenerateBatchWith's yield (engine.go:349-366) */
    for (int s = 0; s < S; s++) {
      if (completed_out[s]) continue;
      if (col[s] == TOK_ASSISTANT_END || col[s] == TOK_BOS) {
        completed_out[s] = 1;
        done_rows++;
      } else
        rows_out[(int64_t)s * W + lens_out[s]++] = col[s];
    }
    if (done_rows == S) break;
    generated++;
    forward_impl(m, col, S, 1, dec, lg1, NULL);
    for (int64_t i = 0; i < (int64_t)S * V; i++) logits[i] = (float)lg1[i];
  }
  for (int s = 0; s < S; s++) { free(st[s].forced); free(st[s].tool); }
  free(st); free(completed_out); free(next); free(col); free(lg1); free(logits);
  cache_free(dec);
}

/* The logits Engine.GenerateWith samples from (inference/engine.go:131-325)
 * for one group of S rows when the token columns it feeds are given instead
 * of sampled: out[0] is the prefill's last-position logits (PrefillCED for
 * the causal encoder-decoder split, Forward otherwise) expanded to the S
 * rows, out[t] the logits after feeding column t-1, cols [ncols][S], for t =
 * 1..ncols; out is [ncols + 1][S][V].  Test infrastructure: rollouts of
 * another engine are checked by sampling each step from these logits. */
void FN(orc_decode_forced)(MODEL *m, const int32_t *prompt, int P, int S, const int32_t *cols,
                           int ncols, REAL *out) {
  const int64_t V = m->V;
  kvcache *pre = cache_new(m, 1, P);
  REAL *lg = (REAL *)malloc(sizeof(REAL) * (int64_t)P * V);
  if (m->split > 0) /* engine.go:164-173 */
    prefill_ced(m, prompt, P, pre, lg + (int64_t)(P - 1) * V);
  else
    forward_impl(m, prompt, 1, P, pre, lg, NULL);
  for (int s = 0; s < S; s++) memcpy(out + s * V, lg + (int64_t)(P - 1) * V, sizeof(REAL) * V);
  free(lg);
  kvcache *dec = cache_new(m, S, P + ncols + 1);
  prefill_from(m, dec, pre);
  cache_free(pre);
  for (int t = 0; t < ncols; t++)
    forward_impl(m, cols + (int64_t)t * S, S, 1, dec, out + (int64_t)(t + 1) * S * V, NULL);
  cache_free(dec);
}

/* cmd/chat_rl/main.go:101-183 for G effort groups (seeds given), with the
 * rewards supplied by the caller. */
double FN(orc_rl_step)(MODEL *m, const int32_t *prompts, int G, int P, int S, int max_tokens,
                        float temperature, int top_k, const uint64_t *seeds, const float *rewards,
                        int32_t *rows_out, int32_t *lens_out, float *adv_out,
                        int32_t *max_len_out, int32_t *inputs_out, int32_t *targets_out,
                        REAL *nll, REAL *grads) {
  int W = P + max_tokens, Bt = G * S;
  for (int g = 0; g < G; g++)
    FN(orc_generate_batch)(m, prompts + (int64_t)g * P, P, S, max_tokens, temperature, top_k,
                           seeds[g], rows_out + (int64_t)g * S * W, lens_out + g * S);
  /* group-mean advantages in float32 (main.go:139-155) */
  for (int g = 0; g < G; g++) {
    float mean = 0;
    for (int i = 0; i < S; i++) mean += rewards[g * S + i];
    mean /= (float)S;
    for (int i = 0; i < S; i++) adv_out[g * S + i] = rewards[g * S + i] - mean;
  }
  int maxLen = 0;
  for (int b = 0; b < Bt; b++)
    if (lens_out[b] > maxLen) maxLen = lens_out[b];
  *max_len_out = maxLen;
  int T = maxLen - 1;
  for (int b = 0; b < Bt; b++) {
    for (int t = 0; t < T; t++) {
      int32_t in = t < lens_out[b] ? rows_out[(int64_t)b * W + t] : TOK_ASSISTANT_END;
      int32_t tg = t + 1 < lens_out[b] ? rows_out[(int64_t)b * W + t + 1] : TOK_ASSISTANT_END;
      if (t < P) tg = -1;
      inputs_out[(int64_t)b * T + t] = in;
      targets_out[(int64_t)b * T + t] = tg;
    }
  }
  if (T < 1) return 0;
  return FN(orc_pg_step)(m, inputs_out, targets_out, Bt, T, adv_out, (float)maxLen, nll, grads);
}

double FN(orc_aux_loss)(const MODEL *m) { return m->aux_loss; }
