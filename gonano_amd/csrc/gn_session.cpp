// gn_session.cpp - the device-resident RL step for the dense preset.
//
//   gn_generate_batch        Engine.GenerateBatchWith for all groups at once
//                            (inference/engine.go:112-369)
//   gn_policy_gradient_step  trainer.PolicyGradientStep (trainer/rl.go:14-60)
//   gn_rl_step               cmd/chat_rl's step body (cmd/chat_rl/main.go:101-183)
//
// Weights, KV cache, activations and RNG state stay in HBM; the host runs the
// per-row state machine (forced tool tokens, completion) between decode
// steps, exchanging one token per row.
#include <algorithm>
#include <array>
#include <chrono>
#include <cmath>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include "gn_model.h"
#include "gn_tools.h"

namespace gn {

static constexpr int HD = 128;
static constexpr int SMEAR_CH = 24;
static constexpr int VE_CH = 12;

// -------------------------------------------------------------------------
// Go PCG stream bookkeeping on the host (tensors/random.go:16-18).
// -------------------------------------------------------------------------
typedef unsigned __int128 u128h;
static const u128h kPcgMul = ((u128h)0x2360ED051FC65DA4ull << 64) | 0x4385DF649FCCF645ull;
static const u128h kPcgInc = ((u128h)6364136223846793005ull << 64) | 1442695040888963407ull;
static u128h pcg_advance_host(u128h s, u128h n) {
  u128h cm = kPcgMul, cp = kPcgInc, am = 1, ap = 0;
  while (n) {
    if (n & 1) {
      am *= cm;
      ap = ap * cm + cp;
    }
    cp = (cm + 1) * cp;
    cm *= cm;
    n >>= 1;
  }
  return am * s + ap;
}
static u128h new_rng_state(uint64_t seed) {
  return ((u128h)seed << 64) | (seed ^ 0x9e3779b97f4a7c15ull);
}

// -------------------------------------------------------------------------
struct ParamEntry {
  std::string name;
  int64_t rows, cols, offset;  // offset in the sorted flat vector
  float* dev;                  // device pointer of this tensor (packed layout)
  float* grad;
};

struct Layer {
  float *wqkv, *wo, *wfc, *wproj, *wve, *ve;
  float *gqkv, *go, *gfc, *gproj, *gwve, *gve;
  int window;
  bool has_ve;
};

}  // namespace gn

struct gn_session {
  gn_config cfg{};
  int device = 0;
  int C = 0, Hq = 0, Hkv = 0, D = 0, R = 0, F = 0, L = 0, V = 0, PV = 0, S = 0;
  int QKVW = 0, KVW = 0;
  int64_t total = 0;
  hipStream_t stream = nullptr;
  std::unique_ptr<gn::DeviceArena> arena;
  float* params = nullptr;  // packed device storage
  float* grads = nullptr;
  float *wte = nullptr, *lm = nullptr, *rl = nullptr, *x0l = nullptr, *smg = nullptr,
        *sml = nullptr, *bkl = nullptr;
  float *gwte = nullptr, *glm = nullptr, *grl = nullptr, *gx0l = nullptr, *gsmg = nullptr,
        *gsml = nullptr, *gbkl = nullptr;
  std::vector<gn::Layer> layers;
  std::vector<gn::ParamEntry> table;
  float *cosT = nullptr, *sinT = nullptr;
  // timing
  bool timing = false;
  gn_timing t{};
  std::vector<std::pair<hipEvent_t, hipEvent_t>> gemm_events, attn_events;
  std::vector<double> gemm_ev_flops, attn_ev_bytes;
  std::vector<hipEvent_t> event_pool;
  size_t event_next = 0;
  // decode steps replayed from one captured HIP graph per rollout
  bool decode_graph = true;
  bool capturing = false;
  void* pinned = nullptr;  // host staging for the per-step copies
  size_t pinned_bytes = 0;
};

namespace gn {

static hipEvent_t next_event(gn_session* s) {
  if (s->event_next == s->event_pool.size()) {
    hipEvent_t e;
    GN_HIP(hipEventCreate(&e));
    s->event_pool.push_back(e);
  }
  return s->event_pool[s->event_next++];
}

// Grow-only pinned host buffer (hipHostMalloc; the stream must be idle when
// it grows).
static void* pinned(gn_session* s, size_t bytes) {
  if (bytes > s->pinned_bytes) {
    GN_HIP(hipStreamSynchronize(s->stream));
    if (s->pinned) GN_HIP(hipHostFree(s->pinned));
    s->pinned = nullptr;
    s->pinned_bytes = 0;
    GN_HIP(hipHostMalloc(&s->pinned, bytes, hipHostMallocDefault));
    s->pinned_bytes = bytes;
  }
  return s->pinned;
}

// GEMM launch with optional event timing (not while a graph is captured).
static void sgemm(gn_session* s, const GemmDesc& d) {
  if (s->timing && !s->capturing) {
    hipEvent_t a = next_event(s), b = next_event(s);
    GN_HIP(hipEventRecord(a, s->stream));
    gemm(d, s->stream, s->arena.get());
    GN_HIP(hipEventRecord(b, s->stream));
    s->gemm_events.push_back({a, b});
    s->gemm_ev_flops.push_back(2.0 * d.M * (double)d.N * d.K);
  } else {
    gemm(d, s->stream, s->arena.get());
  }
}

static void collect_timing(gn_session* s, double* gemm_ms, double* gemm_flops, int64_t* gemm_n,
                           double* attn_ms, double* attn_bytes, int64_t* attn_n) {
  for (size_t i = 0; i < s->gemm_events.size(); i++) {
    float ms = 0;
    GN_HIP(hipEventElapsedTime(&ms, s->gemm_events[i].first, s->gemm_events[i].second));
    *gemm_ms += ms;
    *gemm_flops += s->gemm_ev_flops[i];
    (*gemm_n)++;
  }
  for (size_t i = 0; i < s->attn_events.size(); i++) {
    float ms = 0;
    GN_HIP(hipEventElapsedTime(&ms, s->attn_events[i].first, s->attn_events[i].second));
    *attn_ms += ms;
    *attn_bytes += s->attn_ev_bytes[i];
    (*attn_n)++;
  }
  s->gemm_events.clear();
  s->gemm_ev_flops.clear();
  s->attn_events.clear();
  s->attn_ev_bytes.clear();
  s->event_next = 0;
}

template <typename T>
static T* A(gn_session* s, const std::string& name, size_t count) {
  return s->arena->get<T>(name, count);
}

// ---- parameter table (model/params.go:14-85) ------------------------------
static bool has_value_embedding(int l, int L) { return l % 2 == (L - 1) % 2; }

static std::vector<int32_t> window_sizes(const gn_config& c) {  // config.go:629-645
  int T = c.sequence_len;
  int shortw = ((T / 4) / 128) * 128;
  size_t n = strnlen(c.window_pattern, sizeof(c.window_pattern));
  std::vector<int32_t> w(c.n_layer);
  for (int l = 0; l < c.n_layer; l++) {
    char p = c.window_pattern[l % n];
    w[l] = (p == 'L' || p == 'l') ? T : shortw;
  }
  w[c.n_layer - 1] = T;
  return w;
}

static void build_session(gn_session* s, const gn_config& cfg) {
  s->cfg = cfg;
  GN_CHECK(cfg.n_head > 0 && cfg.n_kv_head > 0 && cfg.n_layer > 0 && cfg.n_embd > 0,
           "config: non-positive dimension");
  GN_CHECK(cfg.n_embd % cfg.n_head == 0, "config: EmbedDim not divisible by NumHead");
  GN_CHECK(cfg.n_kv_head <= cfg.n_head && cfg.n_head % cfg.n_kv_head == 0,
           "config: NumKVHead must divide NumHead");
  size_t plen = strnlen(cfg.window_pattern, sizeof(cfg.window_pattern));
  GN_CHECK(plen > 0 && plen < sizeof(cfg.window_pattern), "config: empty window pattern");
  for (size_t i = 0; i < plen; i++)
    GN_CHECK(strchr("LSls", cfg.window_pattern[i]) != nullptr, "config: invalid window pattern");
  s->C = cfg.n_embd;
  s->Hq = cfg.n_head;
  s->Hkv = cfg.n_kv_head;
  s->D = s->C / s->Hq;
  GN_CHECK(s->D == HD, "session: head dimension must be 128");
  s->R = cfg.rotary_dims <= 0 ? s->D : cfg.rotary_dims;
  GN_CHECK(s->R <= s->D && s->R % 2 == 0, "config: RotaryDims must be even and <= head dim");
  GN_CHECK(s->C <= 1024, "session: EmbedDim above 1024 is not supported");
  GN_CHECK(s->Hq / s->Hkv <= 8, "session: GQA ratio above 8 is not supported");
  GN_CHECK(s->Hq + 2 * s->Hkv <= 16, "session: at most 16 q+k+v heads");
  s->F = 4 * s->C;
  s->L = cfg.n_layer;
  s->V = cfg.vocab_size;
  GN_CHECK(s->V > 0, "config: vocab_size must be positive");
  s->PV = ((s->V + 63) / 64) * 64;
  s->S = cfg.sequence_len;
  GN_CHECK(s->S > 0, "config: sequence_len must be positive");
  s->KVW = s->Hkv * s->D;
  s->QKVW = s->Hq * s->D + 2 * s->KVW;

  // sorted-name table with packed placement
  struct Ent {
    std::string name;
    int64_t rows, cols;
    int kind;  // 0 global, 1 q, 2 k, 3 v, 4 proj, 5 vegate, 6 ve, 7 fc, 8 mproj
    int layer;
  };
  std::vector<Ent> ents;
  auto add = [&](const std::string& n, int64_t r, int64_t c, int kind, int layer) {
    ents.push_back({n, r, c, kind, layer});
  };
  add("transformer.wte.weight", s->PV, s->C, 0, -1);
  add("lm_head.weight", s->PV, s->C, 0, -1);
  for (int l = 0; l < s->L; l++) {
    std::string p = "transformer.h." + std::to_string(l) + ".";
    add(p + "attn.c_q.weight", s->Hq * s->D, s->C, 1, l);
    add(p + "attn.c_k.weight", s->KVW, s->C, 2, l);
    add(p + "attn.c_v.weight", s->KVW, s->C, 3, l);
    add(p + "attn.c_proj.weight", s->C, s->C, 4, l);
    if (has_value_embedding(l, s->L)) {
      add(p + "attn.ve_gate.weight", s->Hkv, VE_CH, 5, l);
      add("value_embeds." + std::to_string(l) + ".weight", s->PV, s->KVW, 6, l);
    }
    add(p + "mlp.c_fc.weight", s->F, s->C, 7, l);
    add(p + "mlp.c_proj.weight", s->C, s->F, 8, l);
  }
  add("resid_lambdas", s->L, 1, 0, -1);
  add("x0_lambdas", s->L, 1, 0, -1);
  add("smear_gate.weight", 1, SMEAR_CH, 0, -1);
  add("smear_lambda", 1, 1, 0, -1);
  add("backout_lambda", 1, 1, 0, -1);
  std::sort(ents.begin(), ents.end(), [](const Ent& a, const Ent& b) { return a.name < b.name; });
  int64_t total = 0;
  for (auto& e : ents) total += e.rows * e.cols;
  s->total = total;
  GN_HIP(hipMalloc(&s->params, sizeof(float) * total));
  GN_HIP(hipMalloc(&s->grads, sizeof(float) * total));
  GN_HIP(hipMemsetAsync(s->params, 0, sizeof(float) * total, s->stream));
  GN_HIP(hipMemsetAsync(s->grads, 0, sizeof(float) * total, s->stream));

  // packed placement: per layer [wqkv | wo | wfc | wproj | wve | ve], then globals
  s->layers.assign(s->L, Layer{});
  int64_t cur = 0;
  auto place = [&](int64_t n) {
    int64_t o = cur;
    cur += (n + 63) / 64 * 64;
    return o;
  };
  std::vector<int64_t> lay_qkv(s->L), lay_o(s->L), lay_fc(s->L), lay_pj(s->L), lay_vg(s->L),
      lay_ve(s->L);
  for (int l = 0; l < s->L; l++) {
    lay_qkv[l] = place((int64_t)s->QKVW * s->C);
    lay_o[l] = place((int64_t)s->C * s->C);
    lay_fc[l] = place((int64_t)s->F * s->C);
    lay_pj[l] = place((int64_t)s->C * s->F);
    bool hv = has_value_embedding(l, s->L);
    lay_vg[l] = hv ? place((int64_t)s->Hkv * VE_CH) : -1;
    lay_ve[l] = hv ? place((int64_t)s->PV * s->KVW) : -1;
  }
  int64_t off_wte = place((int64_t)s->PV * s->C), off_lm = place((int64_t)s->PV * s->C);
  int64_t off_rl = place(s->L), off_x0 = place(s->L), off_smg = place(SMEAR_CH),
          off_sml = place(1), off_bkl = place(1);
  // re-allocate with padding room
  GN_HIP(hipFree(s->params));
  GN_HIP(hipFree(s->grads));
  GN_HIP(hipMalloc(&s->params, sizeof(float) * cur));
  GN_HIP(hipMalloc(&s->grads, sizeof(float) * cur));
  GN_HIP(hipMemsetAsync(s->params, 0, sizeof(float) * cur, s->stream));
  GN_HIP(hipMemsetAsync(s->grads, 0, sizeof(float) * cur, s->stream));
  auto P = [&](int64_t o) { return s->params + o; };
  auto G = [&](int64_t o) { return s->grads + o; };
  for (int l = 0; l < s->L; l++) {
    Layer& ly = s->layers[l];
    ly.wqkv = P(lay_qkv[l]); ly.gqkv = G(lay_qkv[l]);
    ly.wo = P(lay_o[l]); ly.go = G(lay_o[l]);
    ly.wfc = P(lay_fc[l]); ly.gfc = G(lay_fc[l]);
    ly.wproj = P(lay_pj[l]); ly.gproj = G(lay_pj[l]);
    ly.has_ve = lay_vg[l] >= 0;
    ly.wve = ly.has_ve ? P(lay_vg[l]) : nullptr; ly.gwve = ly.has_ve ? G(lay_vg[l]) : nullptr;
    ly.ve = ly.has_ve ? P(lay_ve[l]) : nullptr; ly.gve = ly.has_ve ? G(lay_ve[l]) : nullptr;
  }
  s->wte = P(off_wte); s->gwte = G(off_wte);
  s->lm = P(off_lm); s->glm = G(off_lm);
  s->rl = P(off_rl); s->grl = G(off_rl);
  s->x0l = P(off_x0); s->gx0l = G(off_x0);
  s->smg = P(off_smg); s->gsmg = G(off_smg);
  s->sml = P(off_sml); s->gsml = G(off_sml);
  s->bkl = P(off_bkl); s->gbkl = G(off_bkl);
  auto w = window_sizes(cfg);
  for (int l = 0; l < s->L; l++) s->layers[l].window = w[l];

  int64_t off = 0;
  for (auto& e : ents) {
    ParamEntry pe{e.name, e.rows, e.cols, off, nullptr, nullptr};
    int64_t loc = -1;
    const int l = e.layer;
    switch (e.kind) {
      case 0:
        if (e.name == "transformer.wte.weight") loc = off_wte;
        else if (e.name == "lm_head.weight") loc = off_lm;
        else if (e.name == "resid_lambdas") loc = off_rl;
        else if (e.name == "x0_lambdas") loc = off_x0;
        else if (e.name == "smear_gate.weight") loc = off_smg;
        else if (e.name == "smear_lambda") loc = off_sml;
        else if (e.name == "backout_lambda") loc = off_bkl;
        break;
      case 1: loc = lay_qkv[l]; break;
      case 2: loc = lay_qkv[l] + (int64_t)s->Hq * s->D * s->C; break;
      case 3: loc = lay_qkv[l] + ((int64_t)s->Hq * s->D + s->KVW) * s->C; break;
      case 4: loc = lay_o[l]; break;
      case 5: loc = lay_vg[l]; break;
      case 6: loc = lay_ve[l]; break;
      case 7: loc = lay_fc[l]; break;
      case 8: loc = lay_pj[l]; break;
    }
    GN_CHECK(loc >= 0, "internal: unplaced parameter " + e.name);
    pe.dev = P(loc);
    pe.grad = G(loc);
    s->table.push_back(pe);
    off += e.rows * e.cols;
  }

  // rotary tables (model/rotary.go:16-30), SequenceLen*10 positions, computed
  // in float64 and rounded to float32
  int half = s->R / 2;
  int64_t npos = (int64_t)s->S * 10;
  std::vector<float> c((size_t)(npos * half)), sn((size_t)(npos * half));
  for (int64_t p = 0; p < npos; p++)
    for (int j = 0; j < half; j++) {
      double inv = std::pow(100000.0, -2.0 * (double)j / (double)s->R);
      double f = (double)p * inv;
      c[(size_t)(p * half + j)] = (float)std::cos(f);
      sn[(size_t)(p * half + j)] = (float)std::sin(f);
    }
  GN_HIP(hipMalloc(&s->cosT, sizeof(float) * std::max<int64_t>(npos * half, 1)));
  GN_HIP(hipMalloc(&s->sinT, sizeof(float) * std::max<int64_t>(npos * half, 1)));
  GN_HIP(hipMemcpy(s->cosT, c.data(), sizeof(float) * npos * half, hipMemcpyHostToDevice));
  GN_HIP(hipMemcpy(s->sinT, sn.data(), sizeof(float) * npos * half, hipMemcpyHostToDevice));
  GN_HIP(hipStreamSynchronize(s->stream));
}

// ---------------------------------------------------------------------------
// Full-sequence forward (training recompute, prefill, no-cache Forward)
// ---------------------------------------------------------------------------
enum SeqMode { SEQ_TRAIN, SEQ_PREFILL, SEQ_FORWARD };

struct SeqBuffers {
  int B = 0, T = 0;
  int64_t N = 0;
  int32_t* ids = nullptr;
  float *raw, *embn, *smsig, *x0;
  std::vector<float*> xin, xb, h, qrot, krot, qn, kn, v, vesig, o, lse, mid, h2, u, act;
  float *xfinal, *fpre, *fn;
  float* backout;
};

// Per-layer activation buffer: distinct per layer when training saves it,
// shared otherwise.
static float* layer_buf(gn_session* s, const char* nm, int l, bool per_layer, size_t count) {
  std::string key = std::string(nm) + (per_layer ? std::to_string(l) : std::string("*"));
  return A<float>(s, key, count);
}

static void seq_forward(gn_session* s, SeqBuffers& sb, SeqMode mode, float* kcache_pf,
                        float* vcache_pf) {
  const int C = s->C, Hq = s->Hq, Hkv = s->Hkv, F = s->F, L = s->L;
  const int B = sb.B, T = sb.T;
  const int64_t N = sb.N;
  const bool save = mode == SEQ_TRAIN;
  hipStream_t st = s->stream;
  sb.raw = save ? A<float>(s, "raw", N * C) : nullptr;
  sb.embn = A<float>(s, "embn", N * C);
  sb.smsig = A<float>(s, "smsig", std::max<int64_t>((int64_t)B * (T - 1), 1));
  sb.x0 = A<float>(s, "x0", N * C);
  launch_embed_smear(sb.ids, s->wte, s->smg, s->sml, B, T, C, sb.raw, sb.embn, sb.smsig, sb.x0, st);
  for (auto* vec : {&sb.xin, &sb.xb, &sb.h, &sb.qrot, &sb.krot, &sb.qn, &sb.kn, &sb.v, &sb.vesig,
                    &sb.o, &sb.lse, &sb.mid, &sb.h2, &sb.u, &sb.act})
    vec->assign(L, nullptr);
  float* qkv = A<float>(s, "qkv", N * s->QKVW);
  float* xcur = sb.x0;
  const int bk = L / 2;
  sb.backout = nullptr;
  for (int l = 0; l < L; l++) {
    Layer& ly = s->layers[l];
    sb.xin[l] = xcur;
    float* xb = layer_buf(s, "xb", l, save, N * C);
    float* h = layer_buf(s, "h", l, save, N * C);
    launch_resid_norm(xcur, sb.x0, s->rl, s->x0l, l, N, C, xb, h, st);
    sb.xb[l] = xb;
    sb.h[l] = h;
    sgemm(s, linear_fwd_desc(h, ly.wqkv, qkv, (int)N, C, s->QKVW));
    QkvPostArgs qa{};
    qa.qkv = qkv; qa.h = h; qa.ids = sb.ids;
    qa.ve = ly.has_ve ? ly.ve : nullptr; qa.wve = ly.wve;
    qa.cosT = s->cosT; qa.sinT = s->sinT;
    qa.C = C; qa.Hq = Hq; qa.Hkv = Hkv; qa.R = s->R; qa.T = T; qa.pos0 = 0;
    qa.qn = layer_buf(s, "qn", l, save, N * Hq * HD);
    qa.kn = layer_buf(s, "kn", l, save, N * s->KVW);
    qa.vout = layer_buf(s, "v", l, save, N * s->KVW);
    qa.qrot = save ? layer_buf(s, "qrot", l, true, N * Hq * HD) : nullptr;
    qa.krot = save ? layer_buf(s, "krot", l, true, N * s->KVW) : nullptr;
    qa.vesig = (save && ly.has_ve) ? layer_buf(s, "vesig", l, true, N * Hkv) : nullptr;
    if (mode == SEQ_PREFILL) {
      qa.kcache = kcache_pf + (int64_t)l * B * Hkv * T * HD;
      qa.vcache = vcache_pf + (int64_t)l * B * Hkv * T * HD;
      qa.maxSeq = T;
      qa.rows_per_seq = 1;
    }
    launch_qkv_post(qa, N, st);
    sb.qn[l] = qa.qn; sb.kn[l] = qa.kn; sb.v[l] = qa.vout;
    sb.qrot[l] = qa.qrot; sb.krot[l] = qa.krot; sb.vesig[l] = qa.vesig;
    FlashArgs fa{};
    fa.q = qa.qn; fa.k = qa.kn; fa.v = qa.vout;
    fa.o = layer_buf(s, "o", l, save, N * Hq * HD);
    fa.lse = save ? layer_buf(s, "lse", l, true, N * Hq) : nullptr;
    fa.B = B; fa.T = T; fa.Hq = Hq; fa.Hkv = Hkv; fa.window = ly.window;
    launch_flash_fwd(fa, st);
    sb.o[l] = fa.o; sb.lse[l] = fa.lse;
    float* mid = layer_buf(s, "mid", l, save, N * C);
    GemmDesc go = linear_fwd_desc(fa.o, ly.wo, mid, (int)N, Hq * HD, C, EPI_ADD_SRC);
    go.aux = xb; go.ldaux = C;
    sgemm(s, go);
    sb.mid[l] = mid;
    float* h2 = layer_buf(s, "h2", l, save, N * C);
    launch_norm_rows(mid, nullptr, nullptr, N, C, nullptr, h2, st);
    sb.h2[l] = h2;
    float* act = layer_buf(s, "act", l, save, N * F);
    float* u = save ? layer_buf(s, "u", l, true, N * F) : nullptr;
    GemmDesc gf = linear_fwd_desc(h2, ly.wfc, act, (int)N, C, F, EPI_RELU2_SAVE);
    gf.aux_out = u; gf.ldaux = F;
    sgemm(s, gf);
    sb.u[l] = u; sb.act[l] = act;
    // next layer input: distinct buffers when training (the backward needs
    // every layer's input), ping-pong otherwise
    float* xout = save ? A<float>(s, "xout" + std::to_string(l), N * C)
                       : A<float>(s, (l % 2) ? "xpong" : "xping", N * C);
    GemmDesc gp = linear_fwd_desc(act, ly.wproj, xout, (int)N, F, C, EPI_ADD_SRC);
    gp.aux = mid; gp.ldaux = C;
    sgemm(s, gp);
    if (l == bk) {
      sb.backout = A<float>(s, "backout", N * C);
      GN_HIP(hipMemcpyAsync(sb.backout, xout, sizeof(float) * N * C, hipMemcpyDeviceToDevice, st));
    }
    xcur = xout;
  }
  sb.xfinal = xcur;
  sb.fpre = A<float>(s, "fpre", N * C);
  sb.fn = A<float>(s, "fn", N * C);
  launch_norm_rows(xcur, sb.backout, s->bkl, N, C, sb.fpre, sb.fn, st);
}

static int32_t* upload_ids(gn_session* s, const char* name, const int32_t* ids, int64_t n,
                           int V) {
  for (int64_t i = 0; i < n; i++)
    GN_CHECK(ids[i] >= 0 && ids[i] < ((V + 63) / 64) * 64, "token id out of range");
  int32_t* d = A<int32_t>(s, name, n);
  GN_HIP(hipMemcpyAsync(d, ids, sizeof(int32_t) * n, hipMemcpyHostToDevice, s->stream));
  return d;
}

// Row chunk of the [N, V] logits that fits the logits budget.
static int64_t logits_chunk(gn_session* s, int64_t N) {
  const int64_t budget = (int64_t)4 << 30;  // 4 GiB of logits per chunk
  int64_t rows = std::max<int64_t>(1, budget / ((int64_t)s->V * 4));
  rows = std::min<int64_t>(rows, N);
  return rows;
}

// ---------------------------------------------------------------------------
// PolicyGradientStep
// ---------------------------------------------------------------------------
static void pg_step(gn_session* s, const int32_t* inputs, const int32_t* targets, int B, int T,
                    const float* adv, float norm, float* loss_out, float* nll_out) {
  GN_CHECK(B > 0 && T > 1, "policy gradient step: need batch > 0 and seq_len > 1");
  GN_CHECK(T <= s->S, "model: sequence longer than rotary cache");
  const int C = s->C, Hq = s->Hq, Hkv = s->Hkv, F = s->F, L = s->L, V = s->V;
  const int64_t N = (int64_t)B * T;
  hipStream_t st = s->stream;
  for (int64_t i = 0; i < N; i++)
    GN_CHECK(targets[i] == -1 || (targets[i] >= 0 && targets[i] < V), "target id out of range");
  hipEvent_t ev0 = nullptr, ev1 = nullptr;
  if (s->timing) {
    ev0 = next_event(s);
    ev1 = next_event(s);
    GN_HIP(hipEventRecord(ev0, st));
  }
  SeqBuffers sb;
  sb.B = B; sb.T = T; sb.N = N;
  sb.ids = upload_ids(s, "ids", inputs, N, V);
  int32_t* dtg = A<int32_t>(s, "targets", N);
  GN_HIP(hipMemcpyAsync(dtg, targets, sizeof(int32_t) * N, hipMemcpyHostToDevice, st));
  float* dadv = A<float>(s, "adv", B);
  GN_HIP(hipMemcpyAsync(dadv, adv, sizeof(float) * B, hipMemcpyHostToDevice, st));
  seq_forward(s, sb, SEQ_TRAIN, nullptr, nullptr);

  // ---- fused lm_head + softcap + PG loss + softcap backward, row chunks --
  float* nll = A<float>(s, "nll", N);
  double* loss_rows = A<double>(s, "loss_rows", N);
  float* dfn = A<float>(s, "dfn", N * C);
  const int64_t chunk = logits_chunk(s, N);
  float* Z = A<float>(s, "logits", chunk * V);
  for (int64_t r0 = 0; r0 < N; r0 += chunk) {
    const int64_t rows = std::min(chunk, N - r0);
    sgemm(s, linear_fwd_desc(sb.fn + r0 * C, s->lm, Z, (int)rows, C, V, EPI_SOFTCAP));
    launch_pg_loss_rows(Z, V, V, r0, rows, dtg, dadv, T, norm, nll, loss_rows, st);
    sgemm(s, linear_dx_desc(Z, s->lm, dfn + r0 * C, (int)rows, C, V));
    sgemm(s, linear_dw_desc(Z, sb.fn + r0 * C, s->glm, (int)rows, C, V));
  }
  double* dloss = A<double>(s, "loss", 1);
  launch_sum_f64(loss_rows, N, dloss, false, st);

  // ---- trunk backward (train_transformer.go:176-265) ---------------------
  double* part = A<double>(s, "partials", 65536);
  float* g = A<float>(s, "g", N * C);
  launch_rmsnorm_bwd(sb.fpre, dfn, nullptr, N, C, g, st);
  float* gback = nullptr;
  if (sb.backout) {
    gback = A<float>(s, "gback", N * C);
    // gback = -lambda_b * g
    GN_HIP(hipMemsetAsync(gback, 0, sizeof(float) * N * C, st));
    launch_axpy(gback, gback, g, s->bkl, 0.f, N * C, st);
    launch_dot_into_grad(g, sb.backout, nullptr, -1.f, N * C, s->gbkl, nullptr, part, st);
  }
  float* gx0 = A<float>(s, "gx0", N * C);
  GN_HIP(hipMemsetAsync(gx0, 0, sizeof(float) * N * C, st));
  float* lg = A<float>(s, "lg", N * C);
  float* gb = A<float>(s, "gb", N * C);
  float* gmid = A<float>(s, "gmid", N * C);
  float* dtmp = A<float>(s, "dtmp", N * C);
  float* du = A<float>(s, "du", N * F);
  float* dqn = A<float>(s, "dqn", N * Hq * HD);
  float* dkn = A<float>(s, "dkn", N * s->KVW);
  float* dvv = A<float>(s, "dv", N * s->KVW);
  float* delta = A<float>(s, "delta", N * Hq);
  float* dqkv = A<float>(s, "dqkv", N * s->QKVW);
  float* dpre = A<float>(s, "dpre", N * Hkv);
  const int bk = L / 2;
  for (int l = L - 1; l >= 0; l--) {
    Layer& ly = s->layers[l];
    const float* lgp = g;
    if (l == bk && gback) {
      launch_axpy(lg, g, gback, nullptr, 1.f, N * C, st);
      lgp = lg;
    }
    // MLP (train.go:505-514): du = (lg . Wproj) * 2 relu(u); dh2 = du . Wfc
    GemmDesc d1 = linear_dx_desc(lgp, ly.wproj, du, (int)N, F, C, EPI_DRELU2);
    d1.aux = sb.u[l]; d1.ldaux = F;
    sgemm(s, d1);
    sgemm(s, linear_dw_desc(lgp, sb.act[l], ly.gproj, (int)N, F, C));
    sgemm(s, linear_dx_desc(du, ly.wfc, dtmp, (int)N, C, F));
    sgemm(s, linear_dw_desc(du, sb.h2[l], ly.gfc, (int)N, C, F));
    launch_rmsnorm_bwd(sb.mid[l], dtmp, lgp, N, C, gmid, st);
    // attention (train.go:198-427)
    float* dout = dtmp;  // [N, Hq*D] (Hq*D == C)
    sgemm(s, linear_dx_desc(gmid, ly.wo, dout, (int)N, Hq * HD, C));
    sgemm(s, linear_dw_desc(gmid, sb.o[l], ly.go, (int)N, Hq * HD, C));
    FlashBwdArgs fb{};
    fb.q = sb.qn[l]; fb.k = sb.kn[l]; fb.v = sb.v[l]; fb.o = sb.o[l]; fb.dout = dout;
    fb.lse = sb.lse[l]; fb.delta = delta; fb.dq = dqn; fb.dk = dkn; fb.dv = dvv;
    fb.B = B; fb.T = T; fb.Hq = Hq; fb.Hkv = Hkv; fb.window = ly.window;
    launch_flash_bwd(fb, st);
    QkvPostBwdArgs qb{};
    qb.dqn = dqn; qb.dkn = dkn; qb.dv = dvv; qb.qrot = sb.qrot[l]; qb.krot = sb.krot[l];
    qb.vesig = ly.has_ve ? sb.vesig[l] : nullptr;
    qb.ve = ly.ve; qb.ids = sb.ids; qb.cosT = s->cosT; qb.sinT = s->sinT;
    qb.Hq = Hq; qb.Hkv = Hkv; qb.R = s->R; qb.T = T;
    qb.dqkv = dqkv; qb.dpre = dpre; qb.gve = ly.gve;
    launch_qkv_post_bwd(qb, N, st);
    float* dh = dout;  // reuse: dout no longer needed
    sgemm(s, linear_dx_desc(dqkv, ly.wqkv, dh, (int)N, C, s->QKVW));
    sgemm(s, linear_dw_desc(dqkv, sb.h[l], ly.gqkv, (int)N, C, s->QKVW));
    if (ly.has_ve) launch_ve_gate_bwd(dpre, sb.h[l], ly.wve, C, Hkv, N, ly.gwve, dh, part, st);
    launch_rmsnorm_bwd(sb.xb[l], dh, gmid, N, C, gb, st);
    // residual mixing (train_transformer.go:218-240)
    launch_dot_into_grad(gb, sb.xin[l], sb.x0, 1.f, N * C, s->grl + l, s->gx0l + l, part, st);
    launch_resid_bwd(gb, s->rl, s->x0l, l, g, gx0, N * C, st);
  }
  launch_axpy(g, g, gx0, nullptr, 1.f, N * C, st);
  // smear, embedding norm, embedding scatter (train_transformer.go:244-264)
  float* ge = A<float>(s, "ge", N * C);
  float* ggate = A<float>(s, "ggate", std::max<int64_t>((int64_t)B * (T - 1), 1));
  double* lam_rows = A<double>(s, "lam_rows", std::max<int64_t>((int64_t)B * (T - 1), 1));
  launch_smear_bwd(g, sb.embn, sb.smsig, s->sml, s->smg, B, T, C, ge, ggate, lam_rows, part,
                   s->gsmg, s->gsml, st);
  launch_rmsnorm_bwd(sb.raw, ge, nullptr, N, C, gb, st);
  launch_embed_scatter(gb, sb.ids, C, N, s->gwte, st);

  double loss = 0;
  GN_HIP(hipMemcpyAsync(&loss, dloss, sizeof(double), hipMemcpyDeviceToHost, st));
  if (nll_out) GN_HIP(hipMemcpyAsync(nll_out, nll, sizeof(float) * N, hipMemcpyDeviceToHost, st));
  if (s->timing) GN_HIP(hipEventRecord(ev1, st));
  GN_HIP(hipStreamSynchronize(st));
  if (loss_out) *loss_out = (float)loss;
  if (s->timing) {
    float ms = 0;
    GN_HIP(hipEventElapsedTime(&ms, ev0, ev1));
    s->t.train_ms = ms;
    s->t.gemm_ms = 0; s->t.gemm_flops = 0; s->t.gemm_launches = 0;
    double am = 0, ab = 0;
    int64_t an = 0;
    collect_timing(s, &s->t.gemm_ms, &s->t.gemm_flops, &s->t.gemm_launches, &am, &ab, &an);
  }
}

// ---------------------------------------------------------------------------
// Rollout (Engine.GenerateBatchWith for every group)
// ---------------------------------------------------------------------------
struct RowState {  // inference/engine.go:11-22
  std::vector<int> forced;
  size_t forced_pos = 0;
  bool in_tool = false;
  std::vector<int> tool;
  bool completed = false;
};

// One decode forward: tokens dtok at position pos -> logits.  With dpos set
// the position is read on the device (the step is captured once and
// replayed).
static void decode_step(gn_session* s, int rows, int pos, int maxSeq, int32_t* dtok, float* kc,
                        float* vc, float* logits, const int* dpos = nullptr) {
  const int C = s->C, Hq = s->Hq, Hkv = s->Hkv, F = s->F, L = s->L;
  hipStream_t st = s->stream;
  float* x = A<float>(s, "dec_x", (size_t)rows * C);
  float* x0 = A<float>(s, "dec_x0", (size_t)rows * C);
  float* h = A<float>(s, "dec_h", (size_t)rows * C);
  float* prev = A<float>(s, "dec_prev", (size_t)rows * C);
  float* qkv = A<float>(s, "dec_qkv", (size_t)rows * s->QKVW);
  float* q = A<float>(s, "dec_q", (size_t)rows * Hq * HD);
  float* o = A<float>(s, "dec_o", (size_t)rows * Hq * HD);
  float* act = A<float>(s, "dec_act", (size_t)rows * F);
  float* back = A<float>(s, "dec_back", (size_t)rows * C);
  float* part = A<float>(s, "dec_part", (size_t)rows * Hkv * ((maxSeq + 63) / 64) * (Hq / Hkv) * (HD + 2));
  launch_embed_decode(dtok, s->wte, s->smg, s->sml, rows, C, prev, x, x0, st);
  const int bk = L / 2;
  for (int l = 0; l < L; l++) {
    Layer& ly = s->layers[l];
    launch_resid_norm(x, x0, s->rl, s->x0l, l, rows, C, x, h, st);
    sgemm(s, linear_fwd_desc(h, ly.wqkv, qkv, rows, C, s->QKVW));
    QkvPostArgs qa{};
    qa.qkv = qkv; qa.h = h; qa.ids = dtok;
    qa.ve = ly.has_ve ? ly.ve : nullptr; qa.wve = ly.wve;
    qa.cosT = s->cosT; qa.sinT = s->sinT;
    qa.C = C; qa.Hq = Hq; qa.Hkv = Hkv; qa.R = s->R; qa.T = 1; qa.pos0 = pos;
    qa.pos_dev = dpos;
    qa.qn = q;
    qa.kcache = kc + (int64_t)l * rows * Hkv * maxSeq * HD;
    qa.vcache = vc + (int64_t)l * rows * Hkv * maxSeq * HD;
    qa.maxSeq = maxSeq;
    qa.rows_per_seq = 1;
    launch_qkv_post(qa, rows, st);
    DecodeAttnArgs da{};
    da.q = q; da.kc = qa.kcache; da.vc = qa.vcache; da.part = part; da.o = o;
    da.rows = rows; da.Hq = Hq; da.Hkv = Hkv; da.maxSeq = maxSeq;
    da.kstart = std::max(0, pos - ly.window);
    da.kend = pos + 1;
    da.pos_dev = dpos;
    da.window = ly.window;
    if (s->timing && !s->capturing) {
      hipEvent_t e0 = next_event(s), e1 = next_event(s);
      GN_HIP(hipEventRecord(e0, st));
      launch_decode_attention(da, st);
      GN_HIP(hipEventRecord(e1, st));
      s->attn_events.push_back({e0, e1});
      s->attn_ev_bytes.push_back(2.0 * rows * Hkv * HD * 4.0 * (da.kend - da.kstart));
    } else {
      launch_decode_attention(da, st);
    }
    GemmDesc go = linear_fwd_desc(o, ly.wo, x, rows, Hq * HD, C, EPI_ADD_SRC);
    go.aux = x; go.ldaux = C;
    sgemm(s, go);
    launch_norm_rows(x, nullptr, nullptr, rows, C, nullptr, h, st);
    GemmDesc gf = linear_fwd_desc(h, ly.wfc, act, rows, C, F, EPI_RELU2_SAVE);
    sgemm(s, gf);
    GemmDesc gp = linear_fwd_desc(act, ly.wproj, x, rows, F, C, EPI_ADD_SRC);
    gp.aux = x; gp.ldaux = C;
    sgemm(s, gp);
    if (l == bk) GN_HIP(hipMemcpyAsync(back, x, sizeof(float) * rows * C, hipMemcpyDeviceToDevice, st));
  }
  launch_norm_rows(x, back, s->bkl, rows, C, nullptr, h, st);
  sgemm(s, linear_fwd_desc(h, s->lm, logits, rows, C, s->V, EPI_SOFTCAP));
}

static void generate(gn_session* s, const int32_t* prompts, int G, int P, int S, int N,
                     float temperature, int top_k, const uint64_t* seeds, int32_t* rows_out,
                     int32_t* lens_out) {
  GN_CHECK(G > 0 && S > 0 && P > 0 && N >= 0, "generate: bad sizes");
  GN_CHECK(P + N <= s->S * 10, "generate: context exceeds the rotary table");
  GN_CHECK(P <= s->S, "model: sequence longer than rotary cache");
  const int C = s->C, Hkv = s->Hkv, L = s->L, V = s->V;
  const int rows = G * S;
  const int W = P + N;
  hipStream_t st = s->stream;
  auto t0 = std::chrono::steady_clock::now();
  hipEvent_t ev0 = nullptr, ev1 = nullptr;
  if (s->timing) {
    ev0 = next_event(s);
    ev1 = next_event(s);
    GN_HIP(hipEventRecord(ev0, st));
  }
  for (int r = 0; r < rows; r++) {
    memcpy(rows_out + (int64_t)r * W, prompts + (int64_t)(r / S) * P, sizeof(int32_t) * P);
    lens_out[r] = P;
  }
  if (N == 0) return;
  // 1) batch prefill of every prompt (engine.go:141-173)
  SeqBuffers sb;
  sb.B = G; sb.T = P; sb.N = (int64_t)G * P;
  sb.ids = upload_ids(s, "pf_ids", prompts, sb.N, V);
  float* kpf = A<float>(s, "pf_k", (size_t)L * G * Hkv * P * HD);
  float* vpf = A<float>(s, "pf_v", (size_t)L * G * Hkv * P * HD);
  seq_forward(s, sb, SEQ_PREFILL, kpf, vpf);
  // last-position logits of each prompt, expanded to its S rows (engine.go:182-191)
  float* lastfn = A<float>(s, "pf_lastfn", (size_t)rows * C);
  launch_expand_last_rows(sb.fn, lastfn, G, P, S, C, st);
  float* logits = A<float>(s, "dec_logits", (size_t)rows * V);
  sgemm(s, linear_fwd_desc(lastfn, s->lm, logits, rows, C, V, EPI_SOFTCAP));
  // 2) PrefillFrom (kvcache.go:383-448): replicate KV and the smear state
  const int maxSeq = W;
  float* kc = A<float>(s, "kv_k", (size_t)L * rows * Hkv * maxSeq * HD);
  float* vc = A<float>(s, "kv_v", (size_t)L * rows * Hkv * maxSeq * HD);
  for (int l = 0; l < L; l++) {
    launch_replicate_kv(kpf + (int64_t)l * G * Hkv * P * HD, kc + (int64_t)l * rows * Hkv * maxSeq * HD,
                        G, S, Hkv, P, P, maxSeq, st);
    launch_replicate_kv(vpf + (int64_t)l * G * Hkv * P * HD, vc + (int64_t)l * rows * Hkv * maxSeq * HD,
                        G, S, Hkv, P, P, maxSeq, st);
  }
  float* prev = A<float>(s, "dec_prev", (size_t)rows * C);
  launch_expand_last_rows(sb.embn, prev, G, P, S, C, st);

  // 3) decode loop (engine.go:238-325).  Iteration `step` runs the forward
  //    that feeds the previous column (none at step 0: the prefill logits)
  //    and samples column `step`.  After two eager iterations (which size
  //    every buffer) forward + sampler are captured once as a HIP graph and
  //    replayed; the step position, the column and the group streams'
  //    base states reach the device through small copies before each launch.
  std::vector<RowState> states(rows);
  std::vector<u128h> stream(G);
  for (int g = 0; g < G; g++) stream[g] = new_rng_state(seeds[g]);
  uint64_t* dbase = A<uint64_t>(s, "rng_base", 2 * G);
  int32_t* dtok = A<int32_t>(s, "dec_tok", rows);
  int* dpos = A<int>(s, "dec_pos", 1);
  // pinned staging: base states | column | sampled | position
  char* hp = static_cast<char*>(pinned(s, sizeof(uint64_t) * 2 * G + sizeof(int32_t) * (2 * rows + 1)));
  uint64_t* base = reinterpret_cast<uint64_t*>(hp);
  int32_t* column = reinterpret_cast<int32_t*>(base + 2 * G);
  int32_t* sampled = column + rows;
  int32_t* hpos = sampled + rows;
  std::vector<char> done(rows, 0);
  int ndone = 0;
  SamplerArgs sa{};
  sa.logits = logits; sa.ldl = V; sa.rows = rows; sa.V = V; sa.samples_per_group = S;
  sa.base_states = dbase; sa.temperature = temperature; sa.top_k = top_k; sa.out = dtok;

  struct Graph {
    hipGraph_t g = nullptr;
    hipGraphExec_t e = nullptr;
    ~Graph() {
      if (e) (void)hipGraphExecDestroy(e);
      if (g) (void)hipGraphDestroy(g);
    }
  } graph;
  // (Per-launch attention timing needs events between launches, which a
  // replayed graph does not give: timed rollouts report attention only
  // for their eager steps.)
  const bool use_graph = s->decode_graph && N >= 4;

  for (int step = 0; step < N; step++) {
    for (int g = 0; g < G; g++) {
      base[2 * g] = (uint64_t)(stream[g] >> 64);
      base[2 * g + 1] = (uint64_t)stream[g];
      stream[g] = pcg_advance_host(stream[g], (u128h)S * (u128h)V);
    }
    const int pos = P + step - 1;  // position of the previous column
    if (step > 0) {
      *hpos = pos;
      GN_HIP(hipMemcpyAsync(dtok, column, sizeof(int32_t) * rows, hipMemcpyHostToDevice, st));
    }
    GN_HIP(hipMemcpyAsync(dbase, base, sizeof(uint64_t) * 2 * G, hipMemcpyHostToDevice, st));
    const bool replay = use_graph && step >= 2;
    if (replay) {
      GN_HIP(hipMemcpyAsync(dpos, hpos, sizeof(int), hipMemcpyHostToDevice, st));
      if (!graph.e) {
        GN_HIP(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
        s->capturing = true;
        try {
          decode_step(s, rows, pos, maxSeq, dtok, kc, vc, logits, dpos);
          launch_sampler(sa, st);
        } catch (...) {
          s->capturing = false;
          hipGraph_t g = nullptr;
          (void)hipStreamEndCapture(st, &g);
          if (g) (void)hipGraphDestroy(g);
          throw;
        }
        s->capturing = false;
        GN_HIP(hipStreamEndCapture(st, &graph.g));
        GN_HIP(hipGraphInstantiate(&graph.e, graph.g, nullptr, nullptr, 0));
      }
      GN_HIP(hipGraphLaunch(graph.e, st));
    } else {
      if (step > 0) decode_step(s, rows, pos, maxSeq, dtok, kc, vc, logits);
      launch_sampler(sa, st);
    }
    GN_HIP(hipMemcpyAsync(sampled, dtok, sizeof(int32_t) * rows, hipMemcpyDeviceToHost, st));
    GN_HIP(hipStreamSynchronize(st));
    for (int r = 0; r < rows; r++) {
      RowState& rs = states[r];
      int tok;
      if (rs.forced_pos < rs.forced.size()) tok = rs.forced[rs.forced_pos++];
      else tok = sampled[r];
      column[r] = tok;
      if (tok == TOK_ASSISTANT_END || tok == TOK_BOS) rs.completed = true;
      if (tok == TOK_TOOL_START) {
        rs.in_tool = true;
        rs.tool.clear();
      } else if (tok == TOK_TOOL_END && rs.in_tool) {
        rs.in_tool = false;
        if (!rs.tool.empty()) {
          auto res = calculator(decode_tokens(rs.tool));
          if (res) {
            rs.forced.push_back(TOK_TOOL_OUTPUT_START);
            for (int id : encode_bytes(*res)) rs.forced.push_back(id);
            rs.forced.push_back(TOK_TOOL_OUTPUT_END);
          }
        }
        rs.tool.clear();
      } else if (rs.in_tool) {
        rs.tool.push_back(tok);
      }
      // GenerateBatchWith's collection (engine.go:349-366)
      if (!done[r]) {
        if (tok == TOK_ASSISTANT_END || tok == TOK_BOS) {
          done[r] = 1;
          ndone++;
        } else {
          rows_out[(int64_t)r * W + lens_out[r]++] = tok;
        }
      }
    }
    if (ndone == rows) break;
    if (step + 1 == N) break;  // the reference's final forward feeds no sample
    for (int r = 0; r < rows; r++)
      GN_CHECK(column[r] >= 0 && column[r] < s->PV, "forced token outside the embedding table");
  }
  if (s->timing) {
    GN_HIP(hipEventRecord(ev1, st));
    GN_HIP(hipStreamSynchronize(st));
    float ms = 0;
    GN_HIP(hipEventElapsedTime(&ms, ev0, ev1));
    s->t.rollout_ms = ms;
    double gm = 0, gf = 0;
    int64_t gn = 0;
    s->t.decode_attn_ms = 0; s->t.decode_attn_bytes = 0; s->t.decode_attn_launches = 0;
    collect_timing(s, &gm, &gf, &gn, &s->t.decode_attn_ms, &s->t.decode_attn_bytes,
                   &s->t.decode_attn_launches);
  }
  (void)t0;
}

}  // namespace gn

using namespace gn;

extern "C" {

int gn_session_create(const gn_config* config, int device, gn_session** out) {
  return guard([&] {
    GN_CHECK(config && out, "null argument");
    int n = 0;
    GN_HIP(hipGetDeviceCount(&n));
    GN_CHECK(device >= 0 && device < n, "device index out of range");
    GN_HIP(hipSetDevice(device));
    auto s = std::make_unique<gn_session>();
    s->device = device;
    GN_HIP(hipStreamCreateWithFlags(&s->stream, hipStreamNonBlocking));
    s->arena = std::make_unique<DeviceArena>(s->stream);
    build_session(s.get(), *config);
    *out = s.release();
  });
}

int gn_session_destroy(gn_session* s) {
  return guard([&] {
    if (!s) return;
    (void)hipSetDevice(s->device);
    (void)hipStreamSynchronize(s->stream);
    s->arena.reset();
    for (auto e : s->event_pool) (void)hipEventDestroy(e);
    if (s->pinned) (void)hipHostFree(s->pinned);
    (void)hipFree(s->params);
    (void)hipFree(s->grads);
    (void)hipFree(s->cosT);
    (void)hipFree(s->sinT);
    (void)hipStreamDestroy(s->stream);
    delete s;
  });
}

int gn_session_param_total(const gn_session* s, int64_t* total) {
  return guard([&] {
    GN_CHECK(s && total, "null argument");
    *total = s->total;
  });
}
int gn_session_param_count(const gn_session* s, int32_t* count) {
  return guard([&] {
    GN_CHECK(s && count, "null argument");
    *count = (int32_t)s->table.size();
  });
}
int gn_session_param_info(const gn_session* s, int32_t index, char* name, size_t cap,
                          int64_t* rows, int64_t* cols, int64_t* offset) {
  return guard([&] {
    GN_CHECK(s, "null session");
    GN_CHECK(index >= 0 && index < (int32_t)s->table.size(), "parameter index out of range");
    const ParamEntry& e = s->table[index];
    if (name && cap) snprintf(name, cap, "%s", e.name.c_str());
    if (rows) *rows = e.rows;
    if (cols) *cols = e.cols;
    if (offset) *offset = e.offset;
  });
}

static void copy_params(const gn_session* s, float* host, int64_t count, bool to_device,
                        bool grads) {
  GN_CHECK(count == s->total, "parameter vector length mismatch");
  GN_HIP(hipSetDevice(s->device));
  for (const ParamEntry& e : s->table) {
    float* d = grads ? e.grad : e.dev;
    size_t bytes = sizeof(float) * e.rows * e.cols;
    if (to_device) GN_HIP(hipMemcpyAsync(d, host + e.offset, bytes, hipMemcpyHostToDevice, s->stream));
    else GN_HIP(hipMemcpyAsync(host + e.offset, d, bytes, hipMemcpyDeviceToHost, s->stream));
  }
  GN_HIP(hipStreamSynchronize(s->stream));
}

int gn_session_set_params(gn_session* s, const float* params, int64_t count) {
  return guard([&] {
    GN_CHECK(s && params, "null argument");
    copy_params(s, const_cast<float*>(params), count, true, false);
  });
}
int gn_session_get_params(const gn_session* s, float* params, int64_t count) {
  return guard([&] {
    GN_CHECK(s && params, "null argument");
    copy_params(s, params, count, false, false);
  });
}
int gn_session_get_grads(const gn_session* s, float* grads, int64_t count) {
  return guard([&] {
    GN_CHECK(s && grads, "null argument");
    copy_params(s, grads, count, false, true);
  });
}
int gn_session_zero_grads(gn_session* s) {
  return guard([&] {
    GN_CHECK(s, "null session");
    GN_HIP(hipSetDevice(s->device));
    for (const ParamEntry& e : s->table)
      GN_HIP(hipMemsetAsync(e.grad, 0, sizeof(float) * e.rows * e.cols, s->stream));
    GN_HIP(hipStreamSynchronize(s->stream));
  });
}

int gn_forward(gn_session* s, const int32_t* ids, int32_t B, int32_t T, float* logits) {
  return guard([&] {
    GN_CHECK(s && ids && logits, "null argument");
    GN_CHECK(B > 0 && T > 1, "forward: need batch > 0 and seq_len > 1");
    GN_CHECK(T <= s->S, "model: sequence longer than rotary cache");
    GN_HIP(hipSetDevice(s->device));
    SeqBuffers sb;
    sb.B = B; sb.T = T; sb.N = (int64_t)B * T;
    sb.ids = upload_ids(s, "ids", ids, sb.N, s->V);
    seq_forward(s, sb, SEQ_FORWARD, nullptr, nullptr);
    const int64_t chunk = logits_chunk(s, sb.N);
    float* Z = A<float>(s, "logits", chunk * s->V);
    for (int64_t r0 = 0; r0 < sb.N; r0 += chunk) {
      int64_t rows = std::min(chunk, sb.N - r0);
      sgemm(s, linear_fwd_desc(sb.fn + r0 * s->C, s->lm, Z, (int)rows, s->C, s->V, EPI_SOFTCAP));
      GN_HIP(hipMemcpyAsync(logits + r0 * s->V, Z, sizeof(float) * rows * s->V,
                            hipMemcpyDeviceToHost, s->stream));
    }
    GN_HIP(hipStreamSynchronize(s->stream));
    s->gemm_events.clear(); s->gemm_ev_flops.clear(); s->event_next = 0;
  });
}

int gn_generate_batch(gn_session* s, const int32_t* prompts, int32_t groups, int32_t prompt_len,
                      int32_t samples, int32_t max_tokens, float temperature, int32_t top_k,
                      const uint64_t* seeds, int32_t* rows_out, int32_t* lengths_out) {
  return guard([&] {
    GN_CHECK(s && prompts && seeds && rows_out && lengths_out, "null argument");
    GN_HIP(hipSetDevice(s->device));
    generate(s, prompts, groups, prompt_len, samples, max_tokens, temperature, top_k, seeds,
             rows_out, lengths_out);
  });
}

int gn_policy_gradient_step(gn_session* s, const int32_t* inputs, const int32_t* targets,
                            int32_t batch, int32_t seq_len, const float* advantages, float norm,
                            float* loss_out, float* nll_out) {
  return guard([&] {
    GN_CHECK(s && inputs && targets && advantages, "null argument");
    GN_HIP(hipSetDevice(s->device));
    pg_step(s, inputs, targets, batch, seq_len, advantages, norm, loss_out, nll_out);
  });
}

int gn_rl_step(gn_session* s, const int32_t* prompts, int32_t G, int32_t P, int32_t S, int32_t N,
               float temperature, int32_t top_k, const uint64_t* seeds, const float* rewards,
               int32_t* rows_out, int32_t* lens_out, float* adv_out, int32_t* max_len_out,
               float* loss_out) {
  return guard([&] {
    GN_CHECK(s && prompts && seeds && rewards && rows_out && lens_out && adv_out && max_len_out,
             "null argument");
    GN_HIP(hipSetDevice(s->device));
    generate(s, prompts, G, P, S, N, temperature, top_k, seeds, rows_out, lens_out);
    const int Bt = G * S, W = P + N;
    // group-relative advantages in float32 (main.go:139-155)
    for (int g = 0; g < G; g++) {
      float mean = 0.f;
      for (int i = 0; i < S; i++) mean += rewards[g * S + i];
      mean /= (float)S;
      for (int i = 0; i < S; i++) adv_out[g * S + i] = rewards[g * S + i] - mean;
    }
    // padding with <|assistant_end|> and prompt masking (main.go:157-180)
    int maxLen = 0;
    for (int b = 0; b < Bt; b++) maxLen = std::max(maxLen, lens_out[b]);
    *max_len_out = maxLen;
    const int T = maxLen - 1;
    GN_CHECK(T > 1, "rl step: rollouts too short to train on");
    std::vector<int32_t> inputs((size_t)Bt * T), targets((size_t)Bt * T);
    for (int b = 0; b < Bt; b++)
      for (int t = 0; t < T; t++) {
        int32_t in = t < lens_out[b] ? rows_out[(int64_t)b * W + t] : TOK_ASSISTANT_END;
        int32_t tg = t + 1 < lens_out[b] ? rows_out[(int64_t)b * W + t + 1] : TOK_ASSISTANT_END;
        if (t < P) tg = -1;
        inputs[(size_t)b * T + t] = in;
        targets[(size_t)b * T + t] = tg;
      }
    pg_step(s, inputs.data(), targets.data(), Bt, T, adv_out, (float)maxLen, loss_out, nullptr);
  });
}

int gn_sample_next_token(const float* logits, int64_t rows, int64_t vocab, uint64_t* rng_state,
                         float temperature, int64_t top_k, int32_t* out) {
  return guard([&] {
    GN_CHECK(logits && rng_state && out, "null argument");
    GN_CHECK(rows >= 0 && vocab > 0 && vocab < (1ll << 31), "bad logits shape");
    if (rows == 0) return;
    int dev = 0;
    GN_HIP(hipGetDevice(&dev));
    hipStream_t st;
    GN_HIP(hipStreamCreateWithFlags(&st, hipStreamNonBlocking));
    DeviceArena ar(st);
    float* dl = ar.get<float>("l", rows * vocab);
    uint64_t* db = ar.get<uint64_t>("b", 2);
    int32_t* dout = ar.get<int32_t>("o", rows);
    GN_HIP(hipMemcpyAsync(dl, logits, sizeof(float) * rows * vocab, hipMemcpyHostToDevice, st));
    GN_HIP(hipMemcpyAsync(db, rng_state, sizeof(uint64_t) * 2, hipMemcpyHostToDevice, st));
    SamplerArgs sa{};
    sa.logits = dl; sa.ldl = vocab; sa.rows = (int)rows; sa.V = (int)vocab;
    sa.samples_per_group = (int)rows; sa.base_states = db; sa.temperature = temperature;
    sa.top_k = (int)top_k; sa.out = dout;
    launch_sampler(sa, st);
    GN_HIP(hipMemcpyAsync(out, dout, sizeof(int32_t) * rows, hipMemcpyDeviceToHost, st));
    GN_HIP(hipStreamSynchronize(st));
    ar.release();
    GN_HIP(hipStreamDestroy(st));
    if (temperature > 0) {
      u128h sv = ((u128h)rng_state[0] << 64) | rng_state[1];
      sv = pcg_advance_host(sv, (u128h)rows * (u128h)vocab);
      rng_state[0] = (uint64_t)(sv >> 64);
      rng_state[1] = (uint64_t)sv;
    }
  });
}

int gn_session_set_timing(gn_session* s, int enabled) {
  return guard([&] {
    GN_CHECK(s, "null session");
    s->timing = enabled != 0;
    s->gemm_events.clear(); s->gemm_ev_flops.clear();
    s->attn_events.clear(); s->attn_ev_bytes.clear();
    s->event_next = 0;
  });
}
int gn_session_get_timing(const gn_session* s, gn_timing* out) {
  return guard([&] {
    GN_CHECK(s && out, "null argument");
    *out = s->t;
  });
}
int gn_session_set_decode_graph(gn_session* s, int enabled) {
  return guard([&] {
    GN_CHECK(s, "null session");
    s->decode_graph = enabled != 0;
  });
}
int gn_session_synchronize(gn_session* s) {
  return guard([&] {
    GN_CHECK(s, "null session");
    GN_HIP(hipSetDevice(s->device));
    GN_HIP(hipStreamSynchronize(s->stream));
  });
}

}  // extern "C"
