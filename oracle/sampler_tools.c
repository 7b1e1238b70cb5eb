/*
 * sampler_tools.c - Go's PCG stream, the top-k Gumbel-max sampler and the
 * calculator tool, restated in C.
 *
 * TEST INFRASTRUCTURE ONLY (see gn_oracle.h).
 *
 * The RNG is the one tensors.NewRNG builds (tensors/random.go:16-18):
 * math/rand/v2 NewPCG(seed, seed^0x9e3779b97f4a7c15) wrapped in rand.New.
 * That generator lives in Go's standard library (go.mod pins go 1.27.0), not
 * in the reference tree; its published algorithm is a 128-bit LCG
 *   state = state * 0x2360ED051FC65DA44385DF649FCCF645
 *         + 0x5851F42D4C957F2D14057B7EF767814F   (mod 2^128)
 * whose output is the DXSM permutation of the *new* state, and
 * Rand.Float32() = float32(uint32(Uint64()>>32) << 8 >> 8) / 2^24.
 *
 * The PCG transition, jump-ahead and DXSM output are pinned against numpy's
 * independent PCG64 / PCG64DXSM.  The Float32 mapping is parity unpinned:
 * it follows the published math/rand/v2 source, and neither that source nor
 * a Go toolchain is in this container to check it against.
 */
#include <ctype.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "gn_oracle.h"

typedef unsigned __int128 u128;

static const uint64_t MUL_HI = 0x2360ED051FC65DA4ull;
static const uint64_t MUL_LO = 0x4385DF649FCCF645ull;
static const uint64_t INC_HI = 6364136223846793005ull;
static const uint64_t INC_LO = 1442695040888963407ull;

static u128 mk(uint64_t hi, uint64_t lo) { return ((u128)hi << 64) | lo; }

/* tensors/random.go:16-18 */
void orc_rng_new(orc_pcg *g, uint64_t seed) {
  g->hi = seed;
  g->lo = seed ^ 0x9e3779b97f4a7c15ull;
}

static void pcg_step(orc_pcg *g) {
  u128 s = mk(g->hi, g->lo) * mk(MUL_HI, MUL_LO) + mk(INC_HI, INC_LO);
  g->hi = (uint64_t)(s >> 64);
  g->lo = (uint64_t)s;
}

/* DXSM output of the post-step state ("double xorshift multiply"). */
uint64_t orc_rng_uint64(orc_pcg *g) {
  pcg_step(g);
  uint64_t hi = g->hi, lo = g->lo;
  hi ^= hi >> 32;
  hi *= 0xda942042e4dd58b5ull;
  hi ^= hi >> 48;
  hi *= (lo | 1);
  return hi;
}

/* Rand.Float32: the low 24 bits of Uint32 = Uint64 >> 32, divided by 2^24. */
float orc_rng_float32(orc_pcg *g) {
  uint64_t x = orc_rng_uint64(g);
  uint32_t u = (uint32_t)(x >> 32);
  return (float)((u << 8) >> 8) / 16777216.0f;
}

/* Jump the LCG ahead by delta steps (delta < 2^128) with square-and-multiply
 * composition of the affine map. */
void orc_rng_advance(orc_pcg *g, uint64_t delta_hi, uint64_t delta_lo) {
  u128 n = mk(delta_hi, delta_lo);
  u128 cm = mk(MUL_HI, MUL_LO), cp = mk(INC_HI, INC_LO);
  u128 am = 1, ap = 0;
  while (n) {
    if (n & 1) {
      am *= cm;
      ap = ap * cm + cp;
    }
    cp = (cm + 1) * cp;
    cm *= cm;
    n >>= 1;
  }
  u128 s = am * mk(g->hi, g->lo) + ap;
  g->hi = (uint64_t)(s >> 64);
  g->lo = (uint64_t)s;
}

/* tensors/random.go:67-72: u <= 0 becomes 1e-12, gumbel = -float32(ln(-ln u)). */
float orc_gumbel_from_uniform(float u) {
  if (u <= 0) u = 1e-12f;
  return -(float)log(-log((double)u));
}

/* inference/sampler.go:63-77 (kthLargest): a sorted window of the rank
 * largest values seen so far; returns the rank-th largest of the multiset. */
static int cmp_float_asc(const void *a, const void *b) {
  float x = *(const float *)a, y = *(const float *)b;
  return (x < y) ? -1 : (x > y) ? 1 : 0;
}
float orc_kth_largest(const float *v, int64_t n, int64_t rank) {
  float *top = (float *)malloc(sizeof(float) * rank);
  memcpy(top, v, sizeof(float) * rank);
  qsort(top, rank, sizeof(float), cmp_float_asc);
  for (int64_t i = rank; i < n; i++) {
    if (v[i] > top[0]) {
      top[0] = v[i];
      for (int64_t j = 0; j + 1 < rank && top[j] > top[j + 1]; j++) {
        float t = top[j];
        top[j] = top[j + 1];
        top[j + 1] = t;
      }
    }
  }
  float r = top[0];
  free(top);
  (void)n;
  return r;
}

/* tensors/random.go:60-80 (SampleMultinomial) */
int64_t orc_sample_multinomial(orc_pcg *g, const float *logits, int64_t n, float temperature) {
  if (temperature <= 0) return orc_argmax(logits, n);
  int64_t best = 0;
  float best_score = -INFINITY;
  for (int64_t i = 0; i < n; i++) {
    float u = orc_rng_float32(g);
    float gum = orc_gumbel_from_uniform(u);
    volatile float scaled = logits[i] / temperature;
    float score = scaled + gum;
    if (score > best_score) {
      best_score = score;
      best = i;
    }
  }
  return best;
}

/* inference/sampler.go:16-60 (SampleNextToken, sampleRow, argMax, maskTopK) */
void orc_sample_next_token(const float *logits, int64_t rows, int64_t vocab, orc_pcg *g,
                           float temperature, int64_t top_k, int32_t *out) {
  float *masked = (float *)malloc(sizeof(float) * vocab);
  for (int64_t r = 0; r < rows; r++) {
    const float *row = logits + r * vocab;
    if (temperature <= 0) {
      out[r] = (int32_t)orc_argmax(row, vocab);
      continue;
    }
    const float *use = row;
    if (top_k > 0 && top_k < vocab) {
      float thr = orc_kth_largest(row, vocab, top_k);
      for (int64_t i = 0; i < vocab; i++) masked[i] = row[i] >= thr ? row[i] : -INFINITY;
      use = masked;
    }
    out[r] = (int32_t)orc_sample_multinomial(g, use, vocab, temperature);
  }
  free(masked);
}

/* ---------------------------------------------------------------------- */
/* Calculator (inference/tooluse.go:27-47, 93-190).                        */
/* ---------------------------------------------------------------------- */
typedef struct {
  const char *s;
  size_t n, pos;
} parser;

static void skip_space(parser *p) {
  while (p->pos < p->n && p->s[p->pos] == ' ') p->pos++;
}
static int p_expr(parser *p, double *out);
/* inference/tooluse.go:138-173 (number) */
static int p_number(parser *p, double *out) {
  size_t start = p->pos;
  int seen = 0;
  while (p->pos < p->n && p->s[p->pos] >= '0' && p->s[p->pos] <= '9') { p->pos++; seen = 1; }
  if (p->pos < p->n && p->s[p->pos] == '.') {
    p->pos++;
    while (p->pos < p->n && p->s[p->pos] >= '0' && p->s[p->pos] <= '9') { p->pos++; seen = 1; }
  }
  if (!seen) return 0;
  double value = 0, fraction = 0.1;
  int integer = 1;
  for (size_t i = start; i < p->pos; i++) {
    char c = p->s[i];
    if (c == '.') { integer = 0; fraction = 0.1; continue; }
    double d = (double)(c - '0');
    if (integer) value = value * 10 + d;
    else { value += d * fraction; fraction *= 0.1; }
  }
  *out = value;
  return 1;
}
/* inference/tooluse.go:112-136 (factor) */
static int p_factor(parser *p, double *out) {
  skip_space(p);
  if (p->pos >= p->n) return 0;
  if (p->s[p->pos] == '-') {
    p->pos++;
    double v;
    int ok = p_factor(p, &v);
    *out = -v;
    return ok;
  }
  if (p->s[p->pos] == '(') {
    p->pos++;
    double v;
    if (!p_expr(p, &v)) return 0;
    skip_space(p);
    if (p->pos >= p->n || p->s[p->pos] != ')') return 0;
    p->pos++;
    *out = v;
    return 1;
  }
  return p_number(p, out);
}
/* inference/tooluse.go:82-110 (term) */
static int p_term(parser *p, double *out) {
  double v;
  if (!p_factor(p, &v)) return 0;
  for (;;) {
    skip_space(p);
    if (p->pos >= p->n) { *out = v; return 1; }
    char op = p->s[p->pos];
    if (op != '*' && op != '/') { *out = v; return 1; }
    p->pos++;
    double r;
    if (!p_factor(p, &r)) return 0;
    if (op == '*') v *= r;
    else {
      if (r == 0) return 0;
      v /= r;
    }
  }
}
/* inference/tooluse.go:55-80 (expr) */
static int p_expr(parser *p, double *out) {
  double v;
  if (!p_term(p, &v)) return 0;
  for (;;) {
    skip_space(p);
    if (p->pos >= p->n) { *out = v; return 1; }
    char op = p->s[p->pos];
    if (op != '+' && op != '-') { *out = v; return 1; }
    p->pos++;
    double r;
    if (!p_term(p, &r)) return 0;
    if (op == '+') v += r;
    else v -= r;
  }
}

/* inference/tooluse.go:186-191 (formatNumber): integers print as int64,
 * others with the shortest decimal digits that round-trip, in %f style. */
static void format_number(double v, char *out, size_t cap) {
  if (isnan(v)) { snprintf(out, cap, "NaN"); return; }
  if (isinf(v)) { snprintf(out, cap, v > 0 ? "+Inf" : "-Inf"); return; }
  if (v >= -9.2233720368547758e18 && v < 9.2233720368547758e18 && v == (double)(int64_t)v) {
    snprintf(out, cap, "%lld", (long long)(int64_t)v);
    return;
  }
  /* shortest significant digits that round-trip */
  char buf[64];
  int prec;
  for (prec = 1; prec <= 17; prec++) {
    snprintf(buf, sizeof buf, "%.*e", prec - 1, v);
    if (strtod(buf, NULL) == v) break;
  }
  /* buf = [-]d.ddde[+-]XX ; expand to plain decimal */
  char digits[32];
  int nd = 0, neg = 0;
  const char *c = buf;
  if (*c == '-') { neg = 1; c++; }
  for (; *c && *c != 'e'; c++)
    if (isdigit((unsigned char)*c)) digits[nd++] = *c;
  int exp10 = atoi(c + 1);
  /* value = 0.d1d2... * 10^(exp10+1) */
  int point = exp10 + 1; /* digits before the decimal point */
  size_t o = 0;
  if (neg) out[o++] = '-';
  if (point <= 0) {
    out[o++] = '0';
    out[o++] = '.';
    for (int i = 0; i < -point; i++) out[o++] = '0';
    for (int i = 0; i < nd; i++) out[o++] = digits[i];
  } else {
    for (int i = 0; i < point; i++) out[o++] = i < nd ? digits[i] : '0';
    if (nd > point) {
      out[o++] = '.';
      for (int i = point; i < nd; i++) out[o++] = digits[i];
    }
  }
  out[o] = 0;
  (void)cap;
}

/* inference/tooluse.go:146-154 (unquote) */
static int unquote(const char *t, size_t n, const char **s, size_t *len) {
  if (n < 2) return 0;
  if ((t[0] == '"' && t[n - 1] == '"') || (t[0] == '\'' && t[n - 1] == '\'')) {
    *s = t + 1;
    *len = n - 2;
    return 1;
  }
  return 0;
}
static void trim(const char **s, size_t *n) {
  while (*n && isspace((unsigned char)(*s)[0])) { (*s)++; (*n)--; }
  while (*n && isspace((unsigned char)(*s)[*n - 1])) (*n)--;
}

int orc_calculator(const char *expr_in, char *out, size_t cap) {
  /* strings.ReplaceAll(expr, ",", "") */
  size_t n0 = strlen(expr_in);
  char *e = (char *)malloc(n0 + 1);
  size_t n = 0;
  for (size_t i = 0; i < n0; i++)
    if (expr_in[i] != ',') e[n++] = expr_in[i];
  e[n] = 0;
  int ok = 0;
  /* isArithmetic (inference/tooluse.go:93-102); the expression is bytes, and
   * any byte outside the set (including UTF-8 continuation bytes) fails. */
  int arith = n > 0;
  for (size_t i = 0; i < n && arith; i++) {
    char c = e[i];
    if (!((c >= '0' && c <= '9') || c == '*' || c == '+' || c == '-' || c == '/' || c == '.' ||
          c == '(' || c == ')' || c == ' '))
      arith = 0;
  }
  if (arith) {
    if (strstr(e, "**")) goto done;
    parser p = {e, n, 0};
    double v;
    if (p_expr(&p, &v)) {
      skip_space(&p);
      if (p.pos == p.n) {
        format_number(v, out, cap);
        ok = 1;
      }
    }
    goto done;
  }
  /* isCountExpression (inference/tooluse.go:104-120) */
  {
    int cnt = 1;
    for (size_t i = 0; i < n && cnt; i++) {
      char c = e[i];
      if (!((c >= 'a' && c <= 'z') || (c >= 'A' && c <= 'Z') || (c >= '0' && c <= '9') ||
            c == '\'' || c == '"' || c == '.' || c == '(' || c == ')' || c == '_' || c == ' '))
        cnt = 0;
    }
    if (!cnt) goto done;
    char *lower = strdup(e);
    for (size_t i = 0; i < n; i++) lower[i] = (char)tolower((unsigned char)lower[i]);
    static const char *forbidden[] = {"__",   "import",  "exec",    "eval",    "compile", "open",
                                      "file", "input",   "globals", "locals",  "vars",    "dir",
                                      "getattr", "setattr", "delattr", "hasattr"};
    for (size_t f = 0; f < sizeof forbidden / sizeof *forbidden; f++)
      if (strstr(lower, forbidden[f])) cnt = 0;
    free(lower);
    if (!cnt || !strstr(e, ".count(")) goto done;
    /* evalCount (inference/tooluse.go:123-144) */
    const char *dot = strstr(e, ".count(");
    const char *lit = e;
    size_t litn = (size_t)(dot - e);
    const char *arg = dot + 7;
    size_t argn = n - (size_t)(arg - e);
    trim(&lit, &litn);
    trim(&arg, &argn);
    if (argn == 0 || arg[argn - 1] != ')') goto done;
    argn--;
    trim(&arg, &argn);
    const char *ls, *ss;
    size_t ln, sn;
    if (!unquote(lit, litn, &ls, &ln)) goto done;
    if (!unquote(arg, argn, &ss, &sn)) goto done;
    long long count = 0;
    if (sn == 0) count = (long long)ln + 1; /* strings.Count with an empty separator */
    else
      for (size_t i = 0; i + sn <= ln;) {
        if (memcmp(ls + i, ss, sn) == 0) { count++; i += sn; }
        else i++;
      }
    format_number((double)count, out, cap);
    ok = 1;
  }
done:
  free(e);
  return ok;
}
