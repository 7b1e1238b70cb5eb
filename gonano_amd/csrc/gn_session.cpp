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
#include <cstdlib>
#include <cstdio>
#include <cstring>
#include <filesystem>
#include <memory>
#include <string>
#include <vector>

#include "gn_model.h"
#include "gn_optimizer.h"
#include "gn_tools.h"

namespace gn {

static constexpr int HD = 128;
static constexpr int SMEAR_CH = 24;

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
void advance_rng_state(uint64_t* state, uint64_t n) {
  u128h sv = ((u128h)state[0] << 64) | state[1];
  sv = pcg_advance_host(sv, (u128h)n);
  state[0] = (uint64_t)(sv >> 64);
  state[1] = (uint64_t)sv;
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
  // latent preset.  MLA: wxa = [QueryDown; KVDown; QueryRope; KeyRope] (all
  // read h), wqu = QueryUp, wkvu = [KeyUp; ValueUp] (read the KV latent);
  // wqabs / wcomb are the absorbed decode weights derived from them.
  float *wxa, *wqu, *wkvu, *gxa, *gqu, *gkvu;
  float *wqabs, *wcomb;
  // MoE: wgu = [c_gate; c_fc] of the shared expert, router, packed experts
  float *wgu, *ggu, *wr, *rbias, *gwr;
  float *eg, *eu, *ed, *geg, *geu, *ged;
  // flash preset: the layer's channel compressor (logit weight [128, C] and
  // per-slot bias [ratio, 128]), lightning indexer (query [HI, C], key
  // [HI, 128], head weights [H]); its reuse role ('F', 'R', 'U') and the
  // group's producing layer
  float *wcl, *gcl, *cbias, *gcbias;
  float *wiq, *giq, *wik, *gik, *wih, *gih;
  char mode;
  int producer;
  bool has_idx;
};

}  // namespace gn

struct gn_session {
  gn_config cfg{};
  int device = 0;
  int C = 0, Hq = 0, Hkv = 0, D = 0, R = 0, F = 0, L = 0, V = 0, PV = 0, S = 0;
  int QKVW = 0, KVW = 0;
  // latent preset: MLA widths (xa row = 2*lat + (Hq+Hkv)*rd, kvu row =
  // Hkv*(cd+D)) and MoE shape; derived decode weights are refreshed lazily
  bool mla = false, moe = false;
  int lat = 0, rd = 0, cd = 0, XW = 0, KVUW = 0;
  int E = 0, K = 0, EH = 0;
  float clamp = 0.f, mscale = 1.f, bw = 0.f;
  bool derived_dirty = true;
  float* derived = nullptr;
  // MoE.loadCounts of every layer ([L][E], float64; moe.go:41-43): tokens
  // routed to each expert by the training forwards since the last
  // UpdateRouterBias
  double* moe_load = nullptr;
  int csa_select_mode = 0;  // CsaSelectArgs::mode
  // flash preset: compressed attention (ratio > 1) with a local window
  bool hca = false;
  int ratio = 1, swa = 0;
  // CSA: top-k, indexer heads/dim/width, hierarchical pool, groups kept per
  // row, candidate capacity, distillation weight; CED split (0: off)
  int topk = 0, ih = 1, idim = 64, HI = 64, ipool = 1, gpt = 1, ccap = 1, split = 0;
  float iweight = 1.f;
  // decode-time compressed caches of the current rollout: [L][rows][Hkv]
  // [maxBlocks][128] keys and values, [L][rows][ratio][128] logit rings
  float *hck = nullptr, *hcv = nullptr, *hring = nullptr;
  int maxBlocks = 0;
  // CSA decode: indexer keys [L][rows][maxBlocks][Hkv][HI], per-layer step
  // selections [L][rows*Hkv][K] (+ counts) and Full layers' candidate pools;
  // CED decoder layers' tail keys/values [L][rows][Hkv][ratio][128]
  float* hikc = nullptr;
  int *dsel = nullptr, *dnsel = nullptr, *dpool = nullptr, *dnpool = nullptr;
  float *htailk = nullptr, *htailv = nullptr;
  // sequences of the whole policy-gradient batch when it runs in micro-batches
  // (the balance loss averages over every sequence); 0: the batch itself
  int bal_batch = 0;
  double aux_loss = 0.0;
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
  std::vector<std::pair<hipEvent_t, hipEvent_t>> gemm_events, attn_events, loss_events;
  std::vector<double> gemm_ev_flops, attn_ev_bytes, loss_ev_bytes;
  std::vector<char> gemm_ev_wide;  // the product ran on the wide-tile engine
  std::vector<int> attn_ev_launches;
  std::vector<hipEvent_t> event_pool;
  size_t event_next = 0;
  // device-resident prefix cache (inference/cache.go CacheManager): entries
  // in LRU order, oldest first; each holds one prompt's prefill state
  struct PrefixEntry {
    std::vector<int32_t> tokens;
    // the state (gn::pc_layout) on the device; a disk-backed entry's is null
    // except while a call that hit it uses it
    float* mem = nullptr;
    int64_t bytes = 0;
    double stored_at = 0.0;
    std::string path;  // the on-disk copy (CacheOptions.DiskDir), else empty
  };
  std::vector<std::unique_ptr<PrefixEntry>> pc_entries;
  bool pc_on = false;
  int pc_max_entries = 0;   // 0: unbounded (CacheOptions.MaxEntries)
  int64_t pc_max_bytes = 0; // 0: unbounded (CacheOptions.MaxBytes)
  double pc_ttl = 0.0;      // seconds; 0: no expiry (CacheOptions.TTL)
  int pc_max_prefix = 0;    // longer entries never hit; 0: any (NewPrefixCache)
  int64_t pc_bytes = 0;
  bool pc_defer = false;    // removed entries wait in pc_retired for the stream
  std::vector<std::unique_ptr<PrefixEntry>> pc_retired;
  // device memory of removed entries kept for the next call's entries
  // (hipFree synchronizes the device): (bytes, pointer)
  std::vector<std::pair<int64_t, float*>> pc_pool;
  std::vector<int32_t> pc_hits;  // prompt tokens taken from the cache, per group of the last call
  std::string pc_dir;            // on-disk tier directory (CacheOptions.DiskDir), empty: none
  // decode steps replayed from one captured HIP graph per rollout
  bool decode_graph = true;
  // q/k/v post-processing inside the decode attention kernel (plain windows)
  bool fuse_qkv_post = true;
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
    const GemmEngine e = gemm(d, s->stream, s->arena.get());
    GN_HIP(hipEventRecord(b, s->stream));
    s->gemm_events.push_back({a, b});
    s->gemm_ev_flops.push_back(2.0 * d.M * (double)d.N * d.K * d.batch);
    s->gemm_ev_wide.push_back(e == GEMM_ENGINE_WIDE ? 1 : 0);
  } else {
    gemm(d, s->stream, s->arena.get());
  }
}

// GEMM events into gemm_* (all products) and wide_* (those on the
// wide-tile engine; nullable), attention events into attn_*.
static void collect_timing(gn_session* s, double* gemm_ms, double* gemm_flops, int64_t* gemm_n,
                           double* attn_ms, double* attn_bytes, int64_t* attn_n,
                           double* wide_ms = nullptr, double* wide_flops = nullptr,
                           int64_t* wide_n = nullptr) {
  for (size_t i = 0; i < s->gemm_events.size(); i++) {
    float ms = 0;
    GN_HIP(hipEventElapsedTime(&ms, s->gemm_events[i].first, s->gemm_events[i].second));
    *gemm_ms += ms;
    *gemm_flops += s->gemm_ev_flops[i];
    (*gemm_n)++;
    if (wide_ms && s->gemm_ev_wide[i]) {
      *wide_ms += ms;
      *wide_flops += s->gemm_ev_flops[i];
      (*wide_n)++;
    }
  }
  for (size_t i = 0; i < s->attn_events.size(); i++) {
    float ms = 0;
    GN_HIP(hipEventElapsedTime(&ms, s->attn_events[i].first, s->attn_events[i].second));
    *attn_ms += ms;
    *attn_bytes += s->attn_ev_bytes[i];
    *attn_n += s->attn_ev_launches[i];
  }
  s->gemm_events.clear();
  s->gemm_ev_flops.clear();
  s->gemm_ev_wide.clear();
  s->attn_events.clear();
  s->attn_ev_bytes.clear();
  s->attn_ev_launches.clear();
  s->event_next = 0;
}

// Decode attention is timed per call, in place in the step: the launcher
// records the event pair through the dispatch itself (hipExtLaunchKernelGGL:
// the start of the attention kernel, the end of the call's last kernel), so
// the pair measures the kernels' own duration, as a kernel trace does, and
// not the launch gaps around them.
template <class Args, class F>
static void timed_attention(gn_session* s, double bytes, Args& args, F&& launch) {
  args.t_start = next_event(s);
  args.t_stop = next_event(s);
  launch();
  s->attn_events.push_back({args.t_start, args.t_stop});
  s->attn_ev_bytes.push_back(bytes);
  s->attn_ev_launches.push_back(1);
  args.t_start = args.t_stop = nullptr;
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
  s->mla = cfg.mla_latent > 0;
  s->moe = cfg.n_experts > 0;
  if (s->mla) {  // model/config.go:262-280, 476-505
    s->lat = cfg.mla_latent;
    s->rd = cfg.mla_rope_dims;
    GN_CHECK(s->rd == 64, "session: MLA decode is built for 64 rotary dims (the default for "
                          "head dim 128)");
    GN_CHECK(s->lat % 4 == 0 && s->lat <= 256, "session: MLA latent must be a multiple of 4, <= 256");
    GN_CHECK(s->Hkv * s->rd <= 256, "session: MLA rotary keys wider than 256");
    GN_CHECK(s->Hq <= 8, "session: MLA decode supports at most 8 query heads");
    s->cd = s->D - s->rd;
    s->R = s->rd;
    s->XW = 2 * s->lat + (s->Hq + s->Hkv) * s->rd;
    s->KVUW = s->Hkv * (s->cd + s->D);
  } else {
    s->R = cfg.rotary_dims <= 0 ? s->D : cfg.rotary_dims;
  }
  GN_CHECK(s->R <= s->D && s->R % 2 == 0, "config: RotaryDims must be even and <= head dim");
  s->hca = cfg.compression_ratio > 1;  // Config.Compression() (config.go:407-414)
  const size_t plen_r = strnlen(cfg.reuse_pattern, sizeof(cfg.reuse_pattern));
  GN_CHECK(plen_r < sizeof(cfg.reuse_pattern), "config: reuse pattern not terminated");
  // config.go:465-533
  GN_CHECK(cfg.sparse_topk <= 0 || s->hca, "config: SparseTopK requires CompressionRatio > 1");
  GN_CHECK(plen_r == 0 || s->hca, "config: ReusePattern requires CompressionRatio > 1");
  for (size_t i = 0; i < plen_r; i++)
    GN_CHECK(strchr("FRUfru", cfg.reuse_pattern[i]) != nullptr, "config: invalid reuse pattern");
  GN_CHECK(plen_r == 0 || cfg.reuse_pattern[0] == 'F' || cfg.reuse_pattern[0] == 'f',
           "config: reuse pattern must start with F");
  GN_CHECK(!cfg.ced || (s->hca && cfg.swa_window > 0 && cfg.n_layer >= 2),
           "config: CED requires compression, a local window and >= 2 layers");
  if (s->hca) {
    GN_CHECK(!s->mla, "config: MLA is not supported with compression");  // config.go:483-486
    GN_CHECK(hca_ratio_supported(cfg.compression_ratio),
             "session: compression ratio must be 2..8 or 16");
    GN_CHECK(cfg.swa_window >= 0, "config: negative SWA window");
    s->ratio = cfg.compression_ratio;
    s->swa = cfg.swa_window;
    s->split = cfg.ced ? cfg.n_layer / 2 : 0;
    if (cfg.sparse_topk > 0) {  // config.go:372-402
      s->topk = cfg.sparse_topk;
      GN_CHECK(s->topk <= 64, "session: sparse top-k above 64 is not supported");
      s->idim = cfg.indexer_dim > 0 ? cfg.indexer_dim : 64;
      s->ih = cfg.indexer_heads > 0 ? cfg.indexer_heads : 1;
      s->HI = s->idim * s->ih;
      GN_CHECK(s->HI <= 256 && s->ih <= 8, "session: indexer heads * dim must be <= 256");
      s->ipool = cfg.indexer_pool > 1 ? cfg.indexer_pool : 1;
      const int budget = cfg.indexer_candidates > 0 ? cfg.indexer_candidates
                                                    : std::max(8 * s->topk, 64);
      s->gpt = std::max(1, (budget + s->ipool - 1) / s->ipool);
      s->ccap = std::max(s->gpt * s->ipool, s->topk);
      s->iweight = cfg.indexer_weight > 0 ? cfg.indexer_weight : 1.f;
    }
  }
  GN_CHECK(s->C <= 2048, "session: EmbedDim above 2048 is not supported");
  GN_CHECK(s->Hq / s->Hkv <= 8, "session: GQA ratio above 8 is not supported");
  GN_CHECK(s->Hq + 2 * s->Hkv <= 16, "session: at most 16 q+k+v heads");
  if (s->moe) {  // model/config.go:138-227
    s->E = cfg.n_experts;
    s->K = cfg.experts_per_token;
    s->EH = cfg.expert_hidden;
    GN_CHECK(s->E <= 64 && s->K >= 1 && s->K <= 8 && s->K <= s->E,
             "session: MoE needs 1 <= top-k <= min(8, experts) and at most 64 experts");
    GN_CHECK(s->EH > 0 && s->EH % 4 == 0 && cfg.shared_hidden > 0 && cfg.shared_hidden % 4 == 0,
             "session: expert widths must be positive multiples of 4");
    GN_CHECK(s->C % 4 == 0, "session: MoE needs EmbedDim % 4 == 0");
    s->F = cfg.shared_hidden;
    s->clamp = cfg.moe_clamp;
    s->mscale = cfg.moe_scale;
    s->bw = cfg.balance_weight;
  } else {
    s->F = 4 * s->C;
  }
  s->L = cfg.n_layer;
  s->V = cfg.vocab_size;
  GN_CHECK(s->V > 0, "config: vocab_size must be positive");
  s->PV = ((s->V + 63) / 64) * 64;
  s->S = cfg.sequence_len;
  GN_CHECK(s->S > 0, "config: sequence_len must be positive");
  s->KVW = s->Hkv * s->D;
  s->QKVW = s->Hq * s->D + 2 * s->KVW;

  // Packed device placement: per layer the attention block(s), c_proj, the
  // value embedding, then the feed-forward; globals last.  Tensors that feed
  // one GEMM together are adjacent (q/k/v; the four MLA projections of h;
  // KeyUp/ValueUp; c_gate/c_fc).
  int64_t cur = 0;
  auto place = [&](int64_t n) {
    int64_t o = cur;
    cur += (n + 63) / 64 * 64;
    return o;
  };
  struct Ent {
    std::string name;
    int64_t rows, cols, loc;
  };
  std::vector<Ent> ents;
  auto add = [&](const std::string& n, int64_t r, int64_t c, int64_t loc) {
    ents.push_back({n, r, c, loc});
  };
  struct Off {
    int64_t qkv = -1, o = -1, fc = -1, pj = -1, vg = -1, ve = -1;
    int64_t xa = -1, qu = -1, kvu = -1, gu = -1, r = -1, rb = -1, eg = -1, eu = -1, ed = -1;
    int64_t cl = -1, cb = -1, iq = -1, ik = -1, ih = -1;
  };
  std::vector<Off> off(s->L);
  // reuse roles (config.go:303-370): the pattern restarts at the CED split
  auto half_start = [&](int l) { return (s->split > 0 && l >= s->split) ? s->split : 0; };
  auto mode_at = [&](int l) -> char {
    if (!s->hca || plen_r == 0) return 'F';
    const char ch = cfg.reuse_pattern[(l - half_start(l)) % plen_r];
    return (ch == 'R' || ch == 'r') ? 'R' : (ch == 'U' || ch == 'u') ? 'U' : 'F';
  };
  s->layers.assign(s->L, Layer{});
  for (int l = 0; l < s->L; l++) {
    Layer& ly = s->layers[l];
    ly.mode = mode_at(l);
    ly.producer = l;
    if (ly.mode != 'F')
      for (int i = l - 1; i >= half_start(l); i--)
        if (mode_at(i) == 'F') {
          ly.producer = i;
          break;
        }
    ly.has_idx = s->topk > 0 && ly.mode != 'U';
  }
  GN_CHECK(!s->split || mode_at(s->split) == 'F', "config: CED reuse pattern must start each half with F");
  const int C = s->C, D = s->D, Hq = s->Hq, Hkv = s->Hkv, F = s->F;
  for (int l = 0; l < s->L; l++) {
    Off& o = off[l];
    const std::string p = "transformer.h." + std::to_string(l) + ".";
    if (s->mla) {  // model/params.go:19-27
      const int lat = s->lat, rd = s->rd, cd = s->cd;
      o.xa = place((int64_t)s->XW * C);
      add(p + "attn.mla_q_down.weight", lat, C, o.xa);
      add(p + "attn.mla_kv_down.weight", lat, C, o.xa + (int64_t)lat * C);
      add(p + "attn.mla_q_rope.weight", Hq * rd, C, o.xa + (int64_t)2 * lat * C);
      add(p + "attn.mla_k_rope.weight", Hkv * rd, C, o.xa + (int64_t)(2 * lat + Hq * rd) * C);
      o.qu = place((int64_t)Hq * cd * lat);
      add(p + "attn.mla_q_up.weight", Hq * cd, lat, o.qu);
      o.kvu = place((int64_t)s->KVUW * lat);
      add(p + "attn.mla_k_up.weight", Hkv * cd, lat, o.kvu);
      add(p + "attn.mla_v_up.weight", Hkv * D, lat, o.kvu + (int64_t)Hkv * cd * lat);
    } else {
      o.qkv = place((int64_t)s->QKVW * C);
      add(p + "attn.c_q.weight", Hq * D, C, o.qkv);
      add(p + "attn.c_k.weight", s->KVW, C, o.qkv + (int64_t)Hq * D * C);
      add(p + "attn.c_v.weight", s->KVW, C, o.qkv + ((int64_t)Hq * D + s->KVW) * C);
    }
    o.o = place((int64_t)C * C);
    add(p + "attn.c_proj.weight", C, C, o.o);
    if (s->hca && s->layers[l].mode == 'F') {  // model/params.go:43-51
      o.cl = place((int64_t)D * C);
      add(p + "attn.compress_logits.weight", D, C, o.cl);
      o.cb = place((int64_t)s->ratio * D);
      add(p + "attn.compress_bias", s->ratio, D, o.cb);
    }
    if (s->layers[l].has_idx) {
      o.iq = place((int64_t)s->HI * C);
      add(p + "attn.indexer_query.weight", s->HI, C, o.iq);
      o.ik = place((int64_t)s->HI * D);
      add(p + "attn.indexer_key.weight", s->HI, D, o.ik);
      o.ih = place(s->ih);
      add(p + "attn.indexer_heads", s->ih, 1, o.ih);
    }
    if (!s->mla && has_value_embedding(l, s->L)) {  // no VE under MLA (transformer.go:72-78)
      o.vg = place((int64_t)Hkv * VE_CH);
      add(p + "attn.ve_gate.weight", Hkv, VE_CH, o.vg);
      o.ve = place((int64_t)s->PV * s->KVW);
      add("value_embeds." + std::to_string(l) + ".weight", s->PV, s->KVW, o.ve);
    }
    if (s->moe) {  // model/params.go:52-63
      o.gu = place((int64_t)2 * F * C);
      add(p + "mlp.c_gate.weight", F, C, o.gu);
      o.fc = o.gu + (int64_t)F * C;
      add(p + "mlp.c_fc.weight", F, C, o.fc);
      o.pj = place((int64_t)C * F);
      add(p + "mlp.c_proj.weight", C, F, o.pj);
      const int E = s->E, EH = s->EH;
      o.r = place((int64_t)E * C);
      add(p + "moe.router.weight", E, C, o.r);
      o.rb = place(E);
      add(p + "moe.router_bias", E, 1, o.rb);
      o.eg = place((int64_t)E * EH * C);
      add(p + "moe.experts.gate.weight", (int64_t)E * EH, C, o.eg);
      o.eu = place((int64_t)E * EH * C);
      add(p + "moe.experts.up.weight", (int64_t)E * EH, C, o.eu);
      o.ed = place((int64_t)E * C * EH);
      add(p + "moe.experts.down.weight", (int64_t)E * C, EH, o.ed);
    } else {
      o.fc = place((int64_t)F * C);
      add(p + "mlp.c_fc.weight", F, C, o.fc);
      o.pj = place((int64_t)C * F);
      add(p + "mlp.c_proj.weight", C, F, o.pj);
    }
  }
  const int64_t off_wte = place((int64_t)s->PV * C), off_lm = place((int64_t)s->PV * C);
  const int64_t off_rl = place(s->L), off_x0 = place(s->L), off_smg = place(SMEAR_CH),
                off_sml = place(1), off_bkl = place(1);
  add("transformer.wte.weight", s->PV, C, off_wte);
  add("lm_head.weight", s->PV, C, off_lm);
  add("resid_lambdas", s->L, 1, off_rl);
  add("x0_lambdas", s->L, 1, off_x0);
  add("smear_gate.weight", 1, SMEAR_CH, off_smg);
  add("smear_lambda", 1, 1, off_sml);
  add("backout_lambda", 1, 1, off_bkl);
  std::sort(ents.begin(), ents.end(), [](const Ent& a, const Ent& b) { return a.name < b.name; });
  int64_t total = 0;
  for (auto& e : ents) total += e.rows * e.cols;
  s->total = total;
  GN_HIP(hipMalloc(&s->params, sizeof(float) * cur));
  GN_HIP(hipMalloc(&s->grads, sizeof(float) * cur));
  GN_HIP(hipMemsetAsync(s->params, 0, sizeof(float) * cur, s->stream));
  GN_HIP(hipMemsetAsync(s->grads, 0, sizeof(float) * cur, s->stream));
  if (s->moe) {
    GN_HIP(hipMalloc(&s->moe_load, sizeof(double) * s->L * s->E));
    GN_HIP(hipMemsetAsync(s->moe_load, 0, sizeof(double) * s->L * s->E, s->stream));
  }
  auto P = [&](int64_t o) { return o >= 0 ? s->params + o : nullptr; };
  auto G = [&](int64_t o) { return o >= 0 ? s->grads + o : nullptr; };
  for (int l = 0; l < s->L; l++) {
    Layer& ly = s->layers[l];
    const Off& o = off[l];
    ly.wqkv = P(o.qkv); ly.gqkv = G(o.qkv);
    ly.wo = P(o.o); ly.go = G(o.o);
    ly.wfc = P(o.fc); ly.gfc = G(o.fc);
    ly.wproj = P(o.pj); ly.gproj = G(o.pj);
    ly.has_ve = o.vg >= 0;
    ly.wve = P(o.vg); ly.gwve = G(o.vg);
    ly.ve = P(o.ve); ly.gve = G(o.ve);
    ly.wxa = P(o.xa); ly.gxa = G(o.xa);
    ly.wqu = P(o.qu); ly.gqu = G(o.qu);
    ly.wkvu = P(o.kvu); ly.gkvu = G(o.kvu);
    ly.wgu = P(o.gu); ly.ggu = G(o.gu);
    ly.wr = P(o.r); ly.gwr = G(o.r); ly.rbias = P(o.rb);
    ly.eg = P(o.eg); ly.geg = G(o.eg);
    ly.eu = P(o.eu); ly.geu = G(o.eu);
    ly.ed = P(o.ed); ly.ged = G(o.ed);
    ly.wcl = P(o.cl); ly.gcl = G(o.cl);
    ly.cbias = P(o.cb); ly.gcbias = G(o.cb);
    ly.wiq = P(o.iq); ly.giq = G(o.iq);
    ly.wik = P(o.ik); ly.gik = G(o.ik);
    ly.wih = P(o.ih); ly.gih = G(o.ih);
  }
  if (s->mla) {  // absorbed decode weights, per layer [Hq*lat, lat] and [C, Hq*lat]
    const int64_t per = (int64_t)Hq * s->lat * s->lat + (int64_t)C * Hq * s->lat;
    GN_HIP(hipMalloc(&s->derived, sizeof(float) * per * s->L));
    for (int l = 0; l < s->L; l++) {
      s->layers[l].wqabs = s->derived + per * l;
      s->layers[l].wcomb = s->derived + per * l + (int64_t)Hq * s->lat * s->lat;
    }
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
  int64_t offset = 0;
  for (auto& e : ents) {
    s->table.push_back(ParamEntry{e.name, e.rows, e.cols, offset, P(e.loc), G(e.loc)});
    offset += e.rows * e.cols;
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

// Routing and expert activations of one MoE layer (saved for the backward
// when training).
struct MoeBuffers {
  float *probs = nullptr, *w = nullptr, *perm_w = nullptr;
  int32_t* sel = nullptr;
  int *off = nullptr, *perm_row = nullptr, *inv = nullptr, *blockcnt = nullptr;
  float *xg = nullptr, *gug = nullptr, *hg = nullptr, *yg = nullptr;
};

struct SeqBuffers {
  int B = 0, T = 0;
  int64_t N = 0;
  int32_t* ids = nullptr;
  float *raw, *embn, *smsig, *x0;
  std::vector<float*> xin, xb, h, qrot, krot, qn, kn, v, vesig, o, lse, mid, h2, u, act;
  std::vector<float*> xa, gu;  // latent preset: MLA xa rows, shared-expert [gate | up]
  std::vector<MoeBuffers> moe;
  // flash preset: per layer the compressed keys/values and the compressor's
  // softmax weights; prefill outputs (layer-major) of the compressed caches
  // [L][B][Hkv][T / ratio][128] and of the logit rings [L][B][ratio][128]
  std::vector<float*> hkc, hvc, hprobs;
  float *pf_ck = nullptr, *pf_cv = nullptr, *pf_ring = nullptr;
  // sparse selection per layer (a Reuse layer points at the published one),
  // a Full layer's candidate pool, indexer query/key projections; CED: the
  // encoder hidden state and, per decoder Full layer, its projections of it
  std::vector<int*> sel, nsel, pool, npool;
  std::vector<float*> iq, ik, ced_k, ced_v, ced_krot;
  float* enc = nullptr;
  int qoff = 0;  // position of the first row (CED bounded replay)
  // partial forwards (CED prefill): layer range [l0, l1) (l1 < 0: all),
  // given activations and initial residual instead of the embedding, the
  // final activations out; replay: Full layers use the precomputed group
  // compressed blocks pre_kc/pre_vc (gblocks of them) instead of compressing
  int l0 = 0, l1 = -1;
  const float *x_in = nullptr, *x0_in = nullptr;
  float* x_out = nullptr;
  bool replay = false;
  std::vector<float*> pre_kc, pre_vc;
  int gblocks = 0;
  int pf_maxseq = 0;  // prefill raw caches' length (0: T)
  // continuation of cached prefixes (prefix cache hits): pre_len positions
  // of every sequence already computed.  kv_k/kv_v [L][B][pre_len+T][Hkv*128]
  // hold their token-major keys/values in the first pre_len rows of each
  // sequence; the forward writes the new rows after them and attends the
  // whole.  seed_prev [B][C] is each sequence's previous-token embedding for
  // the smear; qoff == pre_len
  int pre_len = 0;
  float *kv_k = nullptr, *kv_v = nullptr;
  const float* seed_prev = nullptr;
  // training: the tokens grouped by id, for the embedding gradients
  TokenGroups groups;
  // when set (a forward from position 0), every layer's token-major
  // keys/values are copied here: [L][B*T][Hkv*128]
  float *tm_k_out = nullptr, *tm_v_out = nullptr;
  // compressed models with a prefix cache: the compressor's logits (h . Wl^T)
  // of every Full layer -- a forward from position 0 copies them to
  // tm_clog_out [L][B*T][128]; a continuation finds the prefix's rows in
  // pre_clog [L][B][pre_len+T][128], writes the new rows after them and
  // compresses the whole sequences
  float* tm_clog_out = nullptr;
  float* pre_clog = nullptr;
  // prefill: the decode caches to fill (indexer keys [L][G*S][maxBlocks]
  // [Hkv][HI] of the complete blocks, replicated over S rows per prompt)
  float* dec_ikc = nullptr;
  int dec_S = 0, dec_maxBlocks = 0;
  float *xfinal, *fpre, *fn;
  float* backout;
};

// Per-layer activation buffer: distinct per layer when training saves it,
// shared otherwise.
static float* layer_buf(gn_session* s, const char* nm, int l, bool per_layer, size_t count) {
  std::string key = std::string(nm) + (per_layer ? std::to_string(l) : std::string("*"));
  return A<float>(s, key, count);
}

static constexpr int MOE_PAD = 128;

// MoE buffers of `rows` tokens under name prefix `pre` (per layer when
// training saves them).
static MoeBuffers moe_buffers(gn_session* s, const std::string& pre, int64_t rows) {
  const int64_t NK = rows * s->K;
  MoeBuffers m;
  m.probs = A<float>(s, pre + "probs", rows * s->E);
  m.sel = A<int32_t>(s, pre + "sel", NK);
  m.w = A<float>(s, pre + "w", NK);
  m.off = A<int>(s, pre + "off", s->E + 1);
  m.perm_row = A<int>(s, pre + "prow", NK);
  m.perm_w = A<float>(s, pre + "pw", NK);
  m.inv = A<int>(s, pre + "inv", NK);
  m.blockcnt = A<int>(s, "moe_blockcnt", ceil_div(NK, 256) * s->E);
  // rows read as the A operand of expert-grouped GEMMs carry MOE_PAD rows of
  // padding (full tiles may read past a group's end)
  m.xg = A<float>(s, pre + "xg", (NK + MOE_PAD) * s->C);
  m.gug = A<float>(s, pre + "gug", NK * 2 * s->EH);
  m.hg = A<float>(s, pre + "hg", (NK + MOE_PAD) * s->EH);
  m.yg = A<float>(s, pre + "yg", NK * s->C);
  return m;
}

// The feed-forward of a MoE block (model/block.go:40-45, mlp.go:62-76,
// moe.go:118-198): xout = mid + (shared(h2) + routed(h2)).  gu and act
// receive the shared expert's [gate | up] pre-activations and its SwiGLU.
// small: decode-size batches (a few to tens of pairs per expert) run the
// expert products as weight-streaming kernels (gate/up with the SwiGLU fused,
// no gathered rows, no pre-activations kept) when the shapes allow.
static void moe_ffn_forward(gn_session* s, const Layer& ly, const float* mid, const float* h2,
                            int64_t rows, float* gu, float* act, const MoeBuffers& m,
                            float* xout, bool small = false, double* load = nullptr) {
  const int C = s->C, F = s->F, E = s->E, EH = s->EH;
  const int64_t NK = rows * s->K;
  hipStream_t st = s->stream;
  const bool stream_experts =
      small && moe_expert_small_supported(EH, C) && moe_expert_small_supported(C, EH);
  // Decode-size batches leave the split-K sums of the shared-expert
  // products to their consumers (the SwiGLU and combine kernels) instead of
  // reduction launches (gu is then not materialized), and compute the router
  // logits in the gate kernel.  The shared expert's output sum stays pending
  // across the routed experts, in its own partial buffer.
  float* logits = A<float>(s, "moe_logits", rows * E);
  PendingSum gsum, ssum;
  // decode-size batches: the gate kernel computes the router logits itself
  if (!small) sgemm(s, linear_fwd_desc(h2, ly.wr, logits, (int)rows, C, E));
  MoeRouteArgs ra{};
  ra.logits = logits; ra.bias = ly.rbias; ra.x = h2; ra.rows = rows;
  ra.E = E; ra.K = s->K; ra.C = C;
  ra.probs = m.probs; ra.sel = m.sel; ra.w = m.w; ra.blockcnt = m.blockcnt; ra.off = m.off;
  ra.perm_row = m.perm_row; ra.perm_w = m.perm_w; ra.inv = m.inv;
  ra.xg = stream_experts ? nullptr : m.xg;
  if (small) ra.wr = ly.wr;
  launch_moe_route(ra, st);
  if (load) launch_moe_load_accum(m.off, E, load, st);  // moe.go:192-193
  GemmDesc dg = linear_fwd_desc(h2, ly.wgu, gu, (int)rows, C, 2 * F);
  if (small) dg.defer = &gsum;
  sgemm(s, dg);
  launch_swiglu_rows(gu, F, rows, s->clamp, act, st, gsum);
  float* shared = A<float>(s, "moe_shared", rows * C);
  GemmDesc ds = linear_fwd_desc(act, ly.wproj, shared, (int)rows, F, C);
  if (small) {
    ds.defer = &ssum;
    ds.defer_slot = 1;
  }
  sgemm(s, ds);
  if (stream_experts) {
    MoeExpertArgs gx{};
    gx.x = h2; gx.perm_row = m.perm_row; gx.off = m.off; gx.w0 = ly.eg; gx.w1 = ly.eu;
    gx.out = m.hg; gx.E = E; gx.N = EH; gx.K = C; gx.clamp = s->clamp; gx.pairs = NK;
    GN_CHECK(launch_moe_expert_small(gx, st), "moe: expert gate/up shape");
    MoeExpertArgs dx{};
    dx.x = m.hg; dx.off = m.off; dx.w0 = ly.ed; dx.out = m.yg; dx.E = E; dx.N = C; dx.K = EH;
    dx.pairs = NK;
    GN_CHECK(launch_moe_expert_small(dx, st), "moe: expert down shape");
  } else {
    // expert gate and up projections into [gate | up] rows, SwiGLU, down
    for (int half = 0; half < 2; half++) {
      GemmDesc d = linear_fwd_desc(m.xg, half ? ly.eu : ly.eg, m.gug + half * EH, (int)NK, C, EH);
      d.ldc = 2 * EH;
      d.group = GEMM_GROUP_ROWS; d.group_off = m.off; d.groups = E;
      d.group_stride = (int64_t)EH * C;
      d.a_pad_rows = MOE_PAD;
      sgemm(s, d);
    }
    launch_swiglu_rows(m.gug, EH, NK, s->clamp, m.hg, st);
    GemmDesc dd = linear_fwd_desc(m.hg, ly.ed, m.yg, (int)NK, EH, C);
    dd.group = GEMM_GROUP_ROWS; dd.group_off = m.off; dd.groups = E;
    dd.group_stride = (int64_t)C * EH;
    dd.a_pad_rows = MOE_PAD;
    sgemm(s, dd);
  }
  MoeCombineArgs ca{};
  ca.mid = mid; ca.shared = shared; ca.yg = m.yg; ca.perm_w = m.perm_w; ca.sel = m.sel;
  ca.inv = m.inv; ca.scale = s->mscale; ca.K = s->K; ca.C = C; ca.out = xout;
  ca.shared_sum = ssum;
  launch_moe_combine(ca, rows, st);
}

// Compressed attention of one layer over full sequences (model/train.go:
// 99-169 with compressForward / compressedAttentionForward,
// compress_attention.go:562-677): compressor logits on the matrix cores, the
// compressor, the global branch over compressed blocks and, with a window,
// the local branch, merged by log-sum-exp.  Writes sb.o[l] (and sb.lse[l],
// the merged log-sum-exp, when training).
// Sequences per chunk of the indexer's [T][blocks] score-like matrices: about
// 2^27 floats (512 MB) per matrix.
static int csa_chunk(gn_session* s, int B, int T, int blocks) {
  const int64_t per = (int64_t)s->Hkv * T * std::max(blocks, 1);
  return (int)std::max<int64_t>(1, std::min<int64_t>(B, ((int64_t)1 << 27) / per));
}
static CsaShape csa_shape(gn_session* s, int T, int blocks, int qoff, int b0) {
  CsaShape c{};
  c.T = T; c.blocks = blocks; c.Hkv = s->Hkv; c.ratio = s->ratio; c.qoff = qoff; c.b0 = b0;
  c.ldo = std::max(blocks, 1); c.H = s->ih; c.dim = s->idim;
  return c;
}

// sparseTrainingPlan's projections and selection (compress_attention.go:
// 45-131, indexer.go:378-558) of a layer with an indexer: indexer queries of
// h, keys of the group's compressed keys, chunked scores and the per-row
// selection (within the Full layer's candidate pool on a Reindex layer).
static void csa_select_layer(gn_session* s, SeqBuffers& sb, const Layer& ly, int l, bool save,
                             const float* kc, int blocks) {
  const int B = sb.B, T = sb.T, Hkv = s->Hkv, HI = s->HI;
  const int64_t N = sb.N;
  hipStream_t st = s->stream;
  float* iq = layer_buf(s, "csa_iq", l, save, N * HI);
  sgemm(s, linear_fwd_desc(sb.h[l], ly.wiq, iq, (int)N, s->C, HI));
  float* ik = layer_buf(s, "csa_ik", l, save, (size_t)B * blocks * Hkv * HI);
  sgemm(s, linear_fwd_desc(kc, ly.wik, ik, B * blocks * Hkv, HD, HI));
  int* sel = reinterpret_cast<int*>(layer_buf(s, "csa_sel", l, save, (size_t)B * Hkv * T * s->topk));
  int* nsel = reinterpret_cast<int*>(layer_buf(s, "csa_nsel", l, save, (size_t)B * Hkv * T));
  const bool produce = ly.mode == 'F' && s->ipool > 1;
  const int p = ly.producer;
  const bool within = ly.mode == 'R' && s->ipool > 1 && sb.pool[p];
  int *pool = nullptr, *npool = nullptr;
  if (produce) {
    pool = reinterpret_cast<int*>(layer_buf(s, "csa_pool", l, true, (size_t)B * Hkv * T * s->ccap));
    npool = reinterpret_cast<int*>(layer_buf(s, "csa_npool", l, true, (size_t)B * Hkv * T));
  }
  const int chunk = csa_chunk(s, B, T, blocks);
  float* scores = A<float>(s, "csa_scores", (size_t)chunk * Hkv * T * std::max(blocks, 1));
  for (int b0 = 0; b0 < B; b0 += chunk) {
    const int nb = std::min(chunk, B - b0);
    IndexerScoreArgs ia{};
    ia.shape = csa_shape(s, T, blocks, sb.qoff, b0);
    ia.iq = iq; ia.ik = ik; ia.w = ly.wih; ia.out = scores;
    launch_indexer_scores(ia, nb, st);
    CsaSelectArgs ca{};
    ca.shape = ia.shape; ca.chunk_seqs = nb; ca.scores = scores;
    ca.K = s->topk; ca.pool = s->ipool; ca.gpt = s->gpt; ca.ccap = s->ccap;
    ca.pool_in = within ? sb.pool[p] : nullptr;
    ca.npool_in = within ? sb.npool[p] : nullptr;
    ca.sel = sel; ca.nsel = nsel; ca.pool_out = pool; ca.npool_out = npool;
    ca.mode = s->csa_select_mode;
    launch_csa_select(ca, st);
  }
  sb.iq[l] = iq; sb.ik[l] = ik;
  sb.sel[l] = sel; sb.nsel[l] = nsel;
  sb.pool[l] = pool; sb.npool[l] = npool;
}

// Compressed attention of one layer over full sequences (model/train.go:
// 99-169 with compressForward, sparseTrainingPlan, compressedAttentionForward
// [Sparse], attentionForwardWindowed and mergeAttentionBranches): a Full
// layer compresses (on a CED decoder layer, its own projections of the
// encoder hidden state); every layer attends to its group's compressed
// blocks -- all blocks before its own, or the indexer's selection (a Reuse
// layer takes the latest published one) -- merged with the local window by
// log-sum-exp.  Writes sb.o[l] (and sb.lse[l], the merged log-sum-exp, when
// training).
static void hca_forward(gn_session* s, SeqBuffers& sb, const Layer& ly, int l, SeqMode mode) {
  const int C = s->C, Hq = s->Hq, Hkv = s->Hkv, B = sb.B, T = sb.T, ratio = s->ratio;
  const int64_t N = sb.N;
  const bool save = mode == SEQ_TRAIN;
  hipStream_t st = s->stream;
  const int Tall = sb.pre_len + T;  // positions per sequence (a continuation: its prefix too)
  const int blocks = sb.replay ? sb.gblocks : (int)ceil_div(Tall, ratio);
  const bool ced = s->split > 0 && l >= s->split;
  if (ly.mode == 'F' && sb.replay) {  // the global blocks were filled from the encoder
    sb.hkc[l] = sb.pre_kc[l];
    sb.hvc[l] = sb.pre_vc[l];
  } else if (ly.mode == 'F') {
    const float *hin = sb.h[l], *kin = sb.kn[l], *vin = sb.v[l];
    if (ced) {  // cedGlobalKeyValue (attention.go:156-171) of the encoder hidden state
      float* kv = A<float>(s, "ced_kv", N * 2 * s->KVW);
      GemmDesc d = linear_fwd_desc(sb.enc, ly.wqkv + (int64_t)Hq * HD * C, kv, (int)N, C, 2 * s->KVW);
      sgemm(s, d);
      QkvPostArgs qa{};
      qa.qkv = kv; qa.cosT = s->cosT; qa.sinT = s->sinT;
      qa.C = C; qa.Hq = 0; qa.Hkv = Hkv; qa.R = s->R; qa.T = T; qa.pos0 = sb.qoff;
      qa.kn = layer_buf(s, "ced_k", l, save, N * s->KVW);
      qa.vout = layer_buf(s, "ced_v", l, save, N * s->KVW);
      qa.krot = save ? layer_buf(s, "ced_krot", l, true, N * s->KVW) : nullptr;
      launch_qkv_post(qa, N, st);
      sb.ced_k[l] = qa.kn; sb.ced_v[l] = qa.vout; sb.ced_krot[l] = qa.krot;
      hin = sb.enc; kin = qa.kn; vin = qa.vout;
    }
    float* clog = A<float>(s, "hca_clog", N * HD);
    sgemm(s, linear_fwd_desc(hin, ly.wcl, clog, (int)N, C, HD));
    if (sb.tm_clog_out)
      GN_HIP(hipMemcpyAsync(sb.tm_clog_out + (int64_t)l * N * HD, clog, sizeof(float) * N * HD,
                            hipMemcpyDeviceToDevice, st));
    if (sb.pre_len > 0) {  // the new rows after each sequence's prefix; compress the whole
      float* all = sb.pre_clog + (int64_t)l * B * Tall * HD;
      GN_HIP(hipMemcpy2DAsync(all + (int64_t)sb.pre_len * HD, sizeof(float) * Tall * HD, clog,
                              sizeof(float) * T * HD, sizeof(float) * T * HD, B,
                              hipMemcpyDeviceToDevice, st));
      clog = all;
    }
    HcaCompressArgs ca{};
    ca.clog = clog; ca.bias = ly.cbias; ca.k = kin; ca.v = vin;
    ca.B = B; ca.T = Tall; ca.Hkv = Hkv; ca.ratio = ratio;
    ca.probs = layer_buf(s, "hca_probs", l, save, (size_t)B * blocks * ratio * HD);
    ca.kc = layer_buf(s, "hca_kc", l, true, (size_t)B * blocks * s->KVW);
    ca.vc = layer_buf(s, "hca_vc", l, true, (size_t)B * blocks * s->KVW);
    if (mode == SEQ_PREFILL) {
      const int64_t full = Tall / ratio;
      if (full > 0) {
        ca.ck_pf = sb.pf_ck + (int64_t)l * B * Hkv * full * HD;
        ca.cv_pf = sb.pf_cv + (int64_t)l * B * Hkv * full * HD;
      }
      ca.ring_pf = sb.pf_ring + (int64_t)l * B * ratio * HD;
    }
    launch_hca_compress(ca, st);
    sb.hkc[l] = ca.kc; sb.hvc[l] = ca.vc; sb.hprobs[l] = ca.probs;
  }
  const int p = ly.producer;
  const float *kc = sb.hkc[p], *vc = sb.hvc[p];
  if (s->topk > 0) {
    if (ly.mode == 'U') {  // the group's latest published selection
      int q = l - 1;
      while (q > p && s->layers[q].mode == 'U') q--;
      sb.sel[l] = sb.sel[q];
      sb.nsel[l] = sb.nsel[q];
    } else {
      csa_select_layer(s, sb, ly, l, save, kc, blocks);
      if (mode == SEQ_PREFILL && sb.dec_ikc && !sb.replay) {  // the decode indexer-key cache
        const int full = Tall / ratio;
        launch_replicate_rows(sb.iq[l] ? sb.ik[l] : nullptr,
                              sb.dec_ikc + (int64_t)l * B * sb.dec_S * sb.dec_maxBlocks * Hkv * s->HI,
                              B, sb.dec_S, full, Hkv * s->HI, blocks, sb.dec_maxBlocks, st);
      }
    }
  }
  float* o = layer_buf(s, "o", l, save, N * Hq * HD);
  float* lse = save ? layer_buf(s, "lse", l, true, N * Hq) : A<float>(s, "hca_lse", N * Hq);
  float* og = s->swa > 0 ? A<float>(s, "hca_og", N * Hq * HD) : o;
  float* lg = s->swa > 0 ? A<float>(s, "hca_lg", N * Hq) : lse;
  if (s->topk > 0) {
    CsaAttnArgs aa{};
    aa.q = sb.qn[l]; aa.kc = kc; aa.vc = vc; aa.sel = sb.sel[l]; aa.nsel = sb.nsel[l];
    aa.B = B; aa.T = T; aa.blocks = blocks; aa.Hq = Hq; aa.Hkv = Hkv; aa.K = s->topk;
    aa.o = og; aa.lse = lg;
    launch_csa_attn_fwd(aa, st);
  } else {
    FlashArgs fg{};
    fg.q = sb.qn[l]; fg.k = kc; fg.v = vc; fg.o = og; fg.lse = lg;
    fg.B = B; fg.T = T; fg.Tk = blocks; fg.ratio = ratio; fg.qoff = sb.qoff;
    fg.Hq = Hq; fg.Hkv = Hkv; fg.window = -1;
    launch_flash_fwd(fg, st);
  }
  if (s->swa > 0) {
    FlashArgs fl{};  // localAttentionRow over the sliding window (compress_attention.go:543-560)
    fl.q = sb.qn[l]; fl.k = sb.kn[l]; fl.v = sb.v[l];
    fl.o = A<float>(s, "hca_ol", N * Hq * HD);
    fl.lse = A<float>(s, "hca_ll", N * Hq);
    fl.B = B; fl.T = T; fl.Hq = Hq; fl.Hkv = Hkv; fl.window = s->swa;
    fl.Tk = Tall; fl.qoff = sb.pre_len;  // a continuation: the prefix's rows first
    launch_flash_fwd(fl, st);
    launch_merge_branches(og, lg, fl.o, fl.lse, o, lse, N * Hq, st);
  }
  sb.o[l] = o;
  sb.lse[l] = save ? lse : nullptr;
}

static void seq_forward(gn_session* s, SeqBuffers& sb, SeqMode mode, float* kcache_pf,
                        float* vcache_pf) {
  const int C = s->C, Hq = s->Hq, Hkv = s->Hkv, F = s->F, L = s->L;
  const int B = sb.B, T = sb.T;
  const int64_t N = sb.N;
  const bool save = mode == SEQ_TRAIN;
  hipStream_t st = s->stream;
  float* xcur;
  if (sb.x_in) {
    sb.x0 = A<float>(s, "x0", N * C);
    GN_HIP(hipMemcpyAsync(sb.x0, sb.x0_in, sizeof(float) * N * C, hipMemcpyDeviceToDevice, st));
    xcur = A<float>(s, "replay_x", N * C);
    GN_HIP(hipMemcpyAsync(xcur, sb.x_in, sizeof(float) * N * C, hipMemcpyDeviceToDevice, st));
  } else {
    sb.raw = save ? A<float>(s, "raw", N * C) : nullptr;
    sb.embn = A<float>(s, "embn", N * C);
    sb.smsig = A<float>(s, "smsig", std::max<int64_t>((int64_t)B * (T - 1), 1));
    sb.x0 = A<float>(s, "x0", N * C);
    launch_embed_smear(sb.ids, s->wte, s->smg, s->sml, B, T, C, sb.raw, sb.embn, sb.smsig, sb.x0,
                       st, sb.seed_prev,
                       sb.seed_prev ? A<float>(s, "seed_sig", std::max(B, 1)) : nullptr);
    xcur = sb.x0;
  }
  const int l_end = sb.l1 < 0 ? L : sb.l1;
  for (auto* vec : {&sb.xin, &sb.xb, &sb.h, &sb.qrot, &sb.krot, &sb.qn, &sb.kn, &sb.v, &sb.vesig,
                    &sb.o, &sb.lse, &sb.mid, &sb.h2, &sb.u, &sb.act, &sb.xa, &sb.gu, &sb.hkc,
                    &sb.hvc, &sb.hprobs, &sb.iq, &sb.ik, &sb.ced_k, &sb.ced_v, &sb.ced_krot})
    vec->assign(L, nullptr);
  for (auto* vec : {&sb.sel, &sb.nsel, &sb.pool, &sb.npool}) vec->assign(L, nullptr);
  sb.moe.assign(L, MoeBuffers{});
  float* qkv = s->mla ? nullptr : A<float>(s, "qkv", N * s->QKVW);
  const int bk = L / 2;
  sb.backout = nullptr;
  GN_CHECK(sb.pre_len == 0 || (!save && s->split == 0 && (!s->hca || sb.pre_clog) &&
                                sb.qoff == sb.pre_len && sb.kv_k && sb.kv_v && !sb.tm_k_out),
           "prefix continuation: prefill only, no encoder-decoder split");
  const int Tall = sb.pre_len + T;  // keys per sequence
  // the new rows' keys/values into the rows after each sequence's prefix
  auto append_rows = [&](float* all, const float* rows) {
    GN_HIP(hipMemcpy2DAsync(all + (int64_t)sb.pre_len * s->KVW, sizeof(float) * Tall * s->KVW, rows,
                            sizeof(float) * T * s->KVW, sizeof(float) * T * s->KVW, B,
                            hipMemcpyDeviceToDevice, st));
  };
  for (int l = sb.l0; l < l_end; l++) {
    Layer& ly = s->layers[l];
    sb.xin[l] = xcur;
    float* pre_k = sb.pre_len > 0 ? sb.kv_k + (int64_t)l * B * Tall * s->KVW : nullptr;
    float* pre_v = sb.pre_len > 0 ? sb.kv_v + (int64_t)l * B * Tall * s->KVW : nullptr;
    if (s->split > 0 && l == s->split) {  // encoderHidden (transformer.go:310-312)
      sb.enc = A<float>(s, "ced_enc", N * C);
      GN_HIP(hipMemcpyAsync(sb.enc, xcur, sizeof(float) * N * C, hipMemcpyDeviceToDevice, st));
    }
    float* xb = layer_buf(s, "xb", l, save, N * C);
    float* h = layer_buf(s, "h", l, save, N * C);
    launch_resid_norm(xcur, sb.x0, s->rl, s->x0l, l, N, C, xb, h, st);
    sb.xb[l] = xb;
    sb.h[l] = h;
    if (s->mla) {
      // mlaProjectHeads (mla.go:106-122): one GEMM for the four projections
      // of h, then QueryUp and [KeyUp; ValueUp] on the latents
      float* xa = layer_buf(s, "xa", l, save, N * s->XW);
      sgemm(s, linear_fwd_desc(h, ly.wxa, xa, (int)N, C, s->XW));
      float* qc = A<float>(s, "mla_qc", N * Hq * s->cd);
      GemmDesc dq = linear_fwd_desc(xa, ly.wqu, qc, (int)N, s->lat, Hq * s->cd);
      dq.lda = s->XW;
      sgemm(s, dq);
      float* kvu = A<float>(s, "mla_kvu", N * s->KVUW);
      GemmDesc dk = linear_fwd_desc(xa + s->lat, ly.wkvu, kvu, (int)N, s->lat, s->KVUW);
      dk.lda = s->XW;
      sgemm(s, dk);
      MlaAssembleArgs ma{};
      ma.xa = xa; ma.xw = s->XW; ma.qc = qc; ma.kvu = kvu; ma.cosT = s->cosT; ma.sinT = s->sinT;
      ma.Hq = Hq; ma.Hkv = Hkv; ma.lat = s->lat; ma.rd = s->rd; ma.T = T; ma.pos0 = sb.qoff;
      ma.q = layer_buf(s, "qn", l, save, N * Hq * HD);
      ma.k = layer_buf(s, "kn", l, save, N * s->KVW);
      ma.v = layer_buf(s, "v", l, save, N * s->KVW);
      if (mode == SEQ_PREFILL) {  // latent + rotary-key cache of the prompt
        const int pm = sb.pf_maxseq > 0 ? sb.pf_maxseq : T;
        ma.lat_cache = kcache_pf + (int64_t)l * B * pm * s->lat;
        ma.rk_cache = vcache_pf + (int64_t)l * B * pm * Hkv * s->rd;
        ma.maxSeq = pm;
      }
      launch_mla_assemble(ma, N, st);
      sb.xa[l] = xa;
      sb.qn[l] = ma.q;
      sb.kn[l] = ma.k;
      sb.v[l] = ma.v;
    } else {
    sgemm(s, linear_fwd_desc(h, ly.wqkv, qkv, (int)N, C, s->QKVW));
    QkvPostArgs qa{};
    qa.qkv = qkv; qa.h = h; qa.ids = sb.ids;
    qa.ve = ly.has_ve ? ly.ve : nullptr; qa.wve = ly.wve;
    qa.cosT = s->cosT; qa.sinT = s->sinT;
    qa.C = C; qa.Hq = Hq; qa.Hkv = Hkv; qa.R = s->R; qa.T = T; qa.pos0 = sb.qoff;
    qa.qn = layer_buf(s, "qn", l, save, N * Hq * HD);
    qa.kn = layer_buf(s, "kn", l, save, N * s->KVW);
    qa.vout = layer_buf(s, "v", l, save, N * s->KVW);
    qa.qrot = save ? layer_buf(s, "qrot", l, true, N * Hq * HD) : nullptr;
    qa.krot = save ? layer_buf(s, "krot", l, true, N * s->KVW) : nullptr;
    qa.vesig = (save && ly.has_ve) ? layer_buf(s, "vesig", l, true, N * Hkv) : nullptr;
    if (mode == SEQ_PREFILL) {
      const int pm = sb.pf_maxseq > 0 ? sb.pf_maxseq : T;
      qa.kcache = kcache_pf + (int64_t)l * B * Hkv * pm * HD;
      qa.vcache = vcache_pf + (int64_t)l * B * Hkv * pm * HD;
      qa.maxSeq = pm;
      qa.rows_per_seq = 1;
    }
    launch_qkv_post(qa, N, st);
    sb.qn[l] = qa.qn;
    sb.kn[l] = qa.kn;
    sb.v[l] = qa.vout;
    sb.qrot[l] = qa.qrot; sb.krot[l] = qa.krot; sb.vesig[l] = qa.vesig;
    }
    if (pre_k) {  // attend the cached prefixes and the new rows
      append_rows(pre_k, sb.kn[l]);
      append_rows(pre_v, sb.v[l]);
      sb.kn[l] = pre_k;
      sb.v[l] = pre_v;
    }
    if (sb.tm_k_out) {  // this layer's keys/values of every sequence
      const int64_t tm = (int64_t)B * T * s->KVW;
      GN_HIP(hipMemcpyAsync(sb.tm_k_out + l * tm, sb.kn[l], sizeof(float) * tm,
                            hipMemcpyDeviceToDevice, st));
      GN_HIP(hipMemcpyAsync(sb.tm_v_out + l * tm, sb.v[l], sizeof(float) * tm,
                            hipMemcpyDeviceToDevice, st));
    }
    if (s->hca) {
      hca_forward(s, sb, ly, l, mode);
    } else {
      FlashArgs fa{};
      fa.q = sb.qn[l]; fa.k = sb.kn[l]; fa.v = sb.v[l];
      fa.o = layer_buf(s, "o", l, save, N * Hq * HD);
      fa.lse = save ? layer_buf(s, "lse", l, true, N * Hq) : nullptr;
      fa.B = B; fa.T = T; fa.Hq = Hq; fa.Hkv = Hkv; fa.window = ly.window;
      fa.Tk = Tall; fa.qoff = sb.pre_len;  // keys of the cached prefix first
      launch_flash_fwd(fa, st);
      sb.o[l] = fa.o; sb.lse[l] = fa.lse;
    }
    float* mid = layer_buf(s, "mid", l, save, N * C);
    GemmDesc go = linear_fwd_desc(sb.o[l], ly.wo, mid, (int)N, Hq * HD, C, EPI_ADD_SRC);
    go.aux = xb; go.ldaux = C;
    sgemm(s, go);
    sb.mid[l] = mid;
    float* h2 = layer_buf(s, "h2", l, save, N * C);
    launch_norm_rows(mid, nullptr, nullptr, N, C, nullptr, h2, st);
    sb.h2[l] = h2;
    if (s->moe) {
      float* xout = save ? A<float>(s, "xout" + std::to_string(l), N * C)
                         : A<float>(s, (l % 2) ? "xpong" : "xping", N * C);
      float* gu = layer_buf(s, "gu", l, save, N * 2 * F);
      float* act = layer_buf(s, "act", l, save, N * F);
      MoeBuffers mb = moe_buffers(s, save ? "moe" + std::to_string(l) + "_" : "moe*_", N);
      // training forwards count the routed tokens (MoE.forwardTraining)
      moe_ffn_forward(s, ly, mid, h2, N, gu, act, mb, xout, false,
                      save ? s->moe_load + (int64_t)l * s->E : nullptr);
      sb.gu[l] = gu; sb.act[l] = act; sb.moe[l] = mb;
      if (l == bk) {
        sb.backout = A<float>(s, "backout", N * C);
        GN_HIP(hipMemcpyAsync(sb.backout, xout, sizeof(float) * N * C, hipMemcpyDeviceToDevice, st));
      }
      xcur = xout;
      continue;
    }
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
  if (sb.x_out) GN_HIP(hipMemcpyAsync(sb.x_out, xcur, sizeof(float) * N * C, hipMemcpyDeviceToDevice, st));
  if (l_end < L) return;  // a partial forward (CED prefill encoder)
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
  if (const char* e = getenv("GN_LOGITS_CHUNK"))  // a smaller chunk (tests: several chunks at small V)
    rows = std::min<int64_t>(rows, std::max(1, atoi(e)));
  rows = std::min<int64_t>(rows, N);
  return rows;
}

// MoE block feed-forward backward (train.go:505-514 with the SwiGLU shared
// expert, moe.go:203-267): dh2 (overwritten) is the gradient wrt the FFN
// input; parameter gradients accumulate.  dauxl, when set, accumulates the
// per-sequence balance-loss terms (moe.go:276-326).
static void moe_ffn_backward(gn_session* s, const Layer& ly, const MoeBuffers& m, const float* g,
                             const float* h2, const float* gu, const float* act, int B, int T,
                             float* dh2, double* dauxl) {
  const int C = s->C, F = s->F, E = s->E, EH = s->EH, K = s->K;
  const int64_t N = (int64_t)B * T, NK = N * K;
  hipStream_t st = s->stream;
  // shared expert
  float* dact = A<float>(s, "moe_dact", N * F);
  sgemm(s, linear_dx_desc(g, ly.wproj, dact, (int)N, F, C));
  sgemm(s, linear_dw_desc(g, act, ly.gproj, (int)N, F, C));
  float* dgu = A<float>(s, "moe_dgu", N * 2 * F);
  launch_swiglu_rows_bwd(gu, dact, F, N, s->clamp, dgu, st);
  float* dsh = A<float>(s, "moe_dsh", N * C);
  sgemm(s, linear_dx_desc(dgu, ly.wgu, dsh, (int)N, C, 2 * F));
  sgemm(s, linear_dw_desc(dgu, h2, ly.ggu, (int)N, C, 2 * F));
  // routed experts
  float* gy = A<float>(s, "moe_gy", (NK + MOE_PAD) * C);
  double* dotp = A<double>(s, "moe_dotp", NK);
  launch_moe_bwd_prep(g, m.yg, m.perm_row, m.perm_w, s->mscale, NK, C, gy, dotp, st);
  float* dhg = A<float>(s, "moe_dhg", NK * EH);
  {  // dhg = gy . Wd_e; dWd_e += gy_e^T . hg_e
    GemmDesc d = linear_dx_desc(gy, ly.ed, dhg, (int)NK, EH, C);
    d.group = GEMM_GROUP_ROWS; d.group_off = m.off; d.groups = E;
    d.group_stride = (int64_t)C * EH;
    d.a_pad_rows = MOE_PAD;
    sgemm(s, d);
    GemmDesc w = linear_dw_desc(gy, m.hg, ly.ged, (int)NK, EH, C);
    w.group = GEMM_GROUP_K; w.group_off = m.off; w.groups = E;
    w.group_stride = (int64_t)C * EH;
    sgemm(s, w);
  }
  float* dgug = A<float>(s, "moe_dgug", (NK + MOE_PAD) * 2 * EH);
  launch_swiglu_rows_bwd(m.gug, dhg, EH, NK, s->clamp, dgug, st);
  float* dxg = A<float>(s, "moe_dxg", NK * C);
  for (int half = 0; half < 2; half++) {  // dxg = dgate . Wg_e + dup . Wu_e
    GemmDesc d = linear_dx_desc(dgug + half * EH, half ? ly.eu : ly.eg, dxg, (int)NK, C, EH,
                                half ? EPI_ACCUM : EPI_STORE);
    d.lda = 2 * EH;
    d.group = GEMM_GROUP_ROWS; d.group_off = m.off; d.groups = E;
    d.group_stride = (int64_t)EH * C;
    d.a_pad_rows = MOE_PAD;
    sgemm(s, d);
    GemmDesc w = linear_dw_desc(dgug + half * EH, m.xg, half ? ly.geu : ly.geg, (int)NK, C, EH);
    w.lda = 2 * EH;
    w.group = GEMM_GROUP_K; w.group_off = m.off; w.groups = E;
    w.group_stride = (int64_t)EH * C;
    sgemm(s, w);
  }
  // router softmax backward with the balance-loss gradient
  MoeRouterBwdArgs rb{};
  if (s->bw > 0.f) {
    float* cnt = A<float>(s, "moe_balcnt", (int64_t)B * E);
    double* lseq = A<double>(s, "moe_balloss", B);
    launch_moe_balance(m.probs, m.sel, B, T, E, K, cnt, lseq, st);
    if (dauxl) launch_sum_f64(lseq, B, dauxl, true, st);
    rb.bal_cnt = cnt;
    const int Bs = s->bal_batch > 0 ? s->bal_batch : B;
    rb.bal_coef = (double)s->bw / ((double)Bs * T) * ((double)E / ((double)K * T));
  }
  float* glog = A<float>(s, "moe_glog", N * E);
  rb.probs = m.probs; rb.sel = m.sel; rb.inv = m.inv; rb.dotp = dotp; rb.rows = N;
  rb.E = E; rb.K = K; rb.T = T; rb.glog = glog;
  launch_moe_router_bwd(rb, st);
  float* drt = A<float>(s, "moe_drt", N * C);
  sgemm(s, linear_dx_desc(glog, ly.wr, drt, (int)N, C, E));
  sgemm(s, linear_dw_desc(glog, h2, ly.gwr, (int)N, C, E));
  MoeBwdCombineArgs cb{};
  cb.dshared = dsh; cb.dxg = dxg; cb.drouter = drt; cb.sel = m.sel; cb.inv = m.inv;
  cb.K = K; cb.C = C; cb.out = dh2;
  launch_moe_bwd_combine(cb, N, st);
}

// MLA attention backward after the flash kernels (train.go:414-419,
// mla.go:126-146): dh (overwritten) is the gradient wrt the attention input.
static void mla_backward(gn_session* s, const Layer& ly, const float* xa, const float* h,
                         const float* dq, const float* dk, const float* dv, int64_t N, int T,
                         float* dh) {
  const int C = s->C, lat = s->lat, XW = s->XW;
  hipStream_t st = s->stream;
  float* dxa = A<float>(s, "mla_dxa", N * XW);
  float* dqc = A<float>(s, "mla_dqc", N * s->Hq * s->cd);
  float* dkvu = A<float>(s, "mla_dkvu", N * s->KVUW);
  MlaPostBwdArgs pb{};
  pb.dq = dq; pb.dk = dk; pb.dv = dv; pb.cosT = s->cosT; pb.sinT = s->sinT;
  pb.Hq = s->Hq; pb.Hkv = s->Hkv; pb.lat = lat; pb.rd = s->rd; pb.T = T; pb.xw = XW;
  pb.dqc = dqc; pb.dxa = dxa; pb.dkvu = dkvu;
  launch_mla_post_bwd(pb, N, st);
  // query latent: dq_lat = dqc . QueryUp -> dxa[:, :lat]
  GemmDesc a1 = linear_dx_desc(dqc, ly.wqu, dxa, (int)N, lat, s->Hq * s->cd);
  a1.ldc = XW;
  sgemm(s, a1);
  GemmDesc a2 = linear_dw_desc(dqc, xa, ly.gqu, (int)N, lat, s->Hq * s->cd);
  a2.ldb = XW;
  sgemm(s, a2);
  // KV latent: dkv_lat = [dk content | dv] . [KeyUp; ValueUp] -> dxa[:, lat:2lat]
  GemmDesc a3 = linear_dx_desc(dkvu, ly.wkvu, dxa + lat, (int)N, lat, s->KVUW);
  a3.ldc = XW;
  sgemm(s, a3);
  GemmDesc a4 = linear_dw_desc(dkvu, xa + lat, ly.gkvu, (int)N, lat, s->KVUW);
  a4.ldb = XW;
  sgemm(s, a4);
  // the four projections of h
  sgemm(s, linear_dx_desc(dxa, ly.wxa, dh, (int)N, C, XW));
  sgemm(s, linear_dw_desc(dxa, h, ly.gxa, (int)N, C, XW));
}

// ---------------------------------------------------------------------------
// PolicyGradientStep
// ---------------------------------------------------------------------------
// A GEMM whose product with the attention input's gradient (dh += g . W)
// the caller adds after the q/k/v projection backward.
struct DhExtra {
  const float* g;
  const float* W;
  int K;
};

// The indexer's distillation backward of one layer (compress_attention.go:
// 133-196 with SparseIndexer.Backward, indexer.go:107-151): per chunk of
// sequences the scores are recomputed, the target is the softmax of the
// mean main-attention logit, gs = (softmax(I) - target) * weight, the
// per-head ReLU masks give the query/key gradients by GEMMs; the head
// weights' gradient is reduced in a fixed order.  Adds the key gradient's
// image into the group's compressed-key gradient gkc and returns the query
// gradient [N, HI] for the attention input.
static float* csa_distill_backward(gn_session* s, SeqBuffers& sb, const Layer& ly, int l,
                                   int blocks, const float* kc, float* gkc) {
  const int B = sb.B, T = sb.T, Hkv = s->Hkv, HI = s->HI, H = s->ih, dim = s->idim;
  const int64_t N = sb.N;
  const int rr = s->Hq / Hkv, p = ly.producer;
  const bool within = ly.mode == 'R' && s->ipool > 1 && sb.pool[p];
  hipStream_t st = s->stream;
  float* qsum = A<float>(s, "csa_qsum", N * Hkv * HD);
  launch_query_group_sum(sb.qn[l], s->Hq, Hkv, N, qsum, st);
  float* gq = A<float>(s, "csa_gq", N * HI);
  GN_HIP(hipMemsetAsync(gq, 0, sizeof(float) * N * HI, st));
  float* gk = A<float>(s, "csa_gk", (size_t)B * blocks * Hkv * HI);
  const int chunk = csa_chunk(s, B, T, blocks);
  const CsaShape s0 = csa_shape(s, T, blocks, sb.qoff, 0);
  const int64_t per = (int64_t)chunk * Hkv * T * s0.ldo;
  float* scores = A<float>(s, "csa_scores", per);
  float* tlog = A<float>(s, "csa_tlog", per);
  float* gs = A<float>(s, "csa_gs", per);
  float* masks = A<float>(s, "csa_mask", per * H);
  const int64_t nblk = indexer_mask_blocks(s0, chunk);
  float* gwb = A<float>(s, "csa_gwb", nblk * H);
  for (int b0 = 0; b0 < B; b0 += chunk) {
    const int nb = std::min(chunk, B - b0);
    const CsaShape sh = csa_shape(s, T, blocks, sb.qoff, b0);
    IndexerScoreArgs ia{};
    ia.shape = sh; ia.iq = sb.iq[l]; ia.ik = sb.ik[l]; ia.w = ly.wih; ia.out = scores;
    launch_indexer_scores(ia, nb, st);
    for (int hh = 0; hh < Hkv; hh++) {  // mean main-attention logits, batched over sequences
      const int b = b0;
      GemmDesc d;
      d.M = T; d.N = blocks; d.K = HD;
      d.A = qsum + ((int64_t)b * T * Hkv + hh) * HD; d.lda = (int64_t)Hkv * HD;
      d.B = kc + ((int64_t)b * blocks * Hkv + hh) * HD; d.ldb = (int64_t)Hkv * HD;
      d.C = tlog + (int64_t)hh * T * sh.ldo; d.ldc = sh.ldo;
      d.alpha = 1.f / (float)rr;
      d.batch = nb;
      d.batch_sa = (int64_t)T * Hkv * HD;
      d.batch_sb = (int64_t)blocks * Hkv * HD;
      d.batch_sc = (int64_t)Hkv * T * sh.ldo;
      sgemm(s, d);
    }
    CsaDistillArgs da{};
    da.shape = sh; da.scores = scores; da.tlog = tlog;
    da.pool_in = within ? sb.pool[p] : nullptr;
    da.npool_in = within ? sb.npool[p] : nullptr;
    da.ccap = s->ccap; da.weight = s->iweight; da.gs = gs;
    launch_csa_distill(da, nb, st);
    IndexerScoreArgs ma = ia;
    ma.out = nullptr; ma.gs = gs; ma.mask_out = masks; ma.mask_stride = per;
    ma.gw_blocks = gwb;
    launch_indexer_scores(ma, nb, st);
    const int64_t nbk = indexer_mask_blocks(sh, nb);
    for (int h = 0; h < H; h++) launch_sum_partials(gwb + (int64_t)h * nbk, nbk, ly.gih + h, st);
    // per sequence (batched over the chunk's nb sequences), KV head and
    // indexer head
    for (int hh = 0; hh < Hkv; hh++)
      for (int h = 0; h < H; h++) {
        const int b = b0;
        const float* mh = masks + (int64_t)h * per + (int64_t)hh * T * sh.ldo;
        const int64_t mstride = (int64_t)Hkv * T * sh.ldo;  // sequence to sequence
        GemmDesc dq;  // gq[b, t, h] += mask . ik
        dq.M = T; dq.N = dim; dq.K = blocks;
        dq.A = mh; dq.lda = sh.ldo;
        dq.B = sb.ik[l] + ((int64_t)b * blocks * Hkv + hh) * HI + h * dim;
        dq.ldb = (int64_t)Hkv * HI; dq.b_kcontig = false;
        dq.C = gq + (int64_t)b * T * HI + h * dim; dq.ldc = HI; dq.epi = EPI_ACCUM;
        dq.batch = nb;
        dq.batch_sa = mstride; dq.batch_sb = (int64_t)blocks * Hkv * HI; dq.batch_sc = (int64_t)T * HI;
        sgemm(s, dq);
        GemmDesc dk;  // gk[b, s, hh, h] = mask^T . iq
        dk.M = blocks; dk.N = dim; dk.K = T;
        dk.A = mh; dk.lda = sh.ldo; dk.a_kcontig = false;
        dk.B = sb.iq[l] + (int64_t)b * T * HI + h * dim; dk.ldb = HI; dk.b_kcontig = false;
        dk.C = gk + ((int64_t)b * blocks * Hkv + hh) * HI + h * dim; dk.ldc = (int64_t)Hkv * HI;
        dk.batch = nb;
        dk.batch_sa = mstride; dk.batch_sb = (int64_t)T * HI; dk.batch_sc = (int64_t)blocks * Hkv * HI;
        sgemm(s, dk);
      }
  }
  sgemm(s, linear_dw_desc(gq, sb.h[l], ly.giq, (int)N, s->C, HI));
  sgemm(s, linear_dw_desc(gk, kc, ly.gik, B * blocks * Hkv, HD, HI));
  sgemm(s, linear_dx_desc(gk, ly.wik, gkc, B * blocks * Hkv, HD, HI, EPI_ACCUM));
  return gq;
}

// Backward of hca_forward (model/train.go:198-303 with compressedAttention-
// Backward[Sparse], indexerDistillationGradient, attentionBackwardWindowed
// and compressBackward, compress_attention.go:376-433, 737-845, 1182-1209):
// both branches from the merged log-sum-exp and the merged row correction
// dO . O; compressed-key/value gradients accumulate in the group's buffers,
// which the Full layer -- the last of its group in the backward -- runs
// through the compressor (a CED decoder layer's into the encoder gradient
// genc).  Appends the attention input's extra gradient GEMMs to `extra`.
static void hca_backward(gn_session* s, SeqBuffers& sb, const Layer& ly, int l, const float* dout,
                         float* delta, float* dqn, float* dkn, float* dvv,
                         std::vector<DhExtra>& extra, float* genc) {
  const int C = s->C, Hq = s->Hq, Hkv = s->Hkv, B = sb.B, T = sb.T, ratio = s->ratio;
  const int64_t N = sb.N;
  hipStream_t st = s->stream;
  const int blocks = (int)ceil_div(T, ratio);
  const int p = ly.producer;
  const bool ced = s->split > 0 && l >= s->split;
  const float *kc = sb.hkc[p], *vc = sb.hvc[p];
  const size_t cw = (size_t)B * blocks * s->KVW;
  float* gkc = A<float>(s, "hca_gkc" + std::to_string(p), cw);
  float* gvc = A<float>(s, "hca_gvc" + std::to_string(p), cw);
  launch_row_dot(sb.o[l], dout, delta, N * Hq, st);
  if (s->topk > 0) {
    CsaAttnArgs aa{};
    aa.q = sb.qn[l]; aa.kc = kc; aa.vc = vc; aa.sel = sb.sel[l]; aa.nsel = sb.nsel[l];
    aa.B = B; aa.T = T; aa.blocks = blocks; aa.Hq = Hq; aa.Hkv = Hkv; aa.K = s->topk;
    aa.lse = sb.lse[l]; aa.dout = dout; aa.delta = delta; aa.dq = dqn; aa.dkc = gkc; aa.dvc = gvc;
    launch_csa_attn_bwd(aa, st);
  } else {
    float* tk = A<float>(s, "hca_dkc", cw);
    float* tv = A<float>(s, "hca_dvc", cw);
    FlashBwdArgs bg{};
    bg.q = sb.qn[l]; bg.k = kc; bg.v = vc; bg.o = sb.o[l]; bg.dout = dout;
    bg.lse = sb.lse[l]; bg.delta = delta; bg.delta_ready = true;
    bg.dq = dqn; bg.dk = tk; bg.dv = tv;
    bg.B = B; bg.T = T; bg.Tk = blocks; bg.ratio = ratio; bg.qoff = sb.qoff;
    bg.Hq = Hq; bg.Hkv = Hkv; bg.window = -1;
    launch_flash_bwd(bg, st);
    launch_axpy(gkc, gkc, tk, nullptr, 1.f, (int64_t)cw, st);
    launch_axpy(gvc, gvc, tv, nullptr, 1.f, (int64_t)cw, st);
  }
  if (s->swa > 0) {
    FlashBwdArgs bl{};
    bl.q = sb.qn[l]; bl.k = sb.kn[l]; bl.v = sb.v[l]; bl.o = sb.o[l]; bl.dout = dout;
    bl.lse = sb.lse[l]; bl.delta = delta; bl.delta_ready = true;
    bl.dq = dqn; bl.dq_accum = true; bl.dk = dkn; bl.dv = dvv;
    bl.B = B; bl.T = T; bl.Hq = Hq; bl.Hkv = Hkv; bl.window = s->swa;
    launch_flash_bwd(bl, st);
  } else {
    GN_HIP(hipMemsetAsync(dkn, 0, sizeof(float) * N * s->KVW, st));
    GN_HIP(hipMemsetAsync(dvv, 0, sizeof(float) * N * s->KVW, st));
  }
  if (ly.has_idx) {
    float* gq = csa_distill_backward(s, sb, ly, l, blocks, kc, gkc);
    extra.push_back({gq, ly.wiq, s->HI});
  }
  if (ly.mode != 'F') return;
  HcaCompressBwdArgs cb{};
  cb.probs = sb.hprobs[l]; cb.kc = kc; cb.vc = vc; cb.dkc = gkc; cb.dvc = gvc;
  cb.B = B; cb.T = T; cb.Hkv = Hkv; cb.ratio = ratio;
  cb.glog = A<float>(s, "hca_glog" + std::to_string(l % 2), N * HD);
  cb.gbias = ly.gcbias;
  cb.bias_part = A<float>(s, "hca_bpart", hca_bias_part_floats(ratio));
  if (!ced) {
    cb.k = sb.kn[l]; cb.v = sb.v[l]; cb.dk = dkn; cb.dv = dvv;
    launch_hca_compress_bwd(cb, st);
    sgemm(s, linear_dw_desc(cb.glog, sb.h[l], ly.gcl, (int)N, C, HD));
    extra.push_back({cb.glog, ly.wcl, HD});
    return;
  }
  // CED decoder: the compressor read the encoder hidden state and its own
  // projections of it (cedKey/ValueProjectionBackward, train.go:454-479)
  float* dkg = A<float>(s, "ced_dk", N * s->KVW);
  float* dvg = A<float>(s, "ced_dv", N * s->KVW);
  GN_HIP(hipMemsetAsync(dkg, 0, sizeof(float) * N * s->KVW, st));
  GN_HIP(hipMemsetAsync(dvg, 0, sizeof(float) * N * s->KVW, st));
  cb.k = sb.ced_k[l]; cb.v = sb.ced_v[l]; cb.dk = dkg; cb.dv = dvg;
  launch_hca_compress_bwd(cb, st);
  sgemm(s, linear_dw_desc(cb.glog, sb.enc, ly.gcl, (int)N, C, HD));
  sgemm(s, linear_dx_desc(cb.glog, ly.wcl, genc, (int)N, C, HD, EPI_ACCUM));
  float* dkv = A<float>(s, "ced_dkv", N * 2 * s->KVW);
  QkvPostBwdArgs qb{};
  qb.dkn = dkg; qb.dv = dvg; qb.krot = sb.ced_krot[l]; qb.cosT = s->cosT; qb.sinT = s->sinT;
  qb.Hq = 0; qb.Hkv = Hkv; qb.R = s->R; qb.T = T; qb.dqkv = dkv;
  launch_qkv_post_bwd(qb, N, st);
  const int64_t kvoff = (int64_t)Hq * HD * C;
  sgemm(s, linear_dw_desc(dkv, sb.enc, ly.gqkv + kvoff, (int)N, C, 2 * s->KVW));
  sgemm(s, linear_dx_desc(dkv, ly.wqkv + kvoff, genc, (int)N, C, 2 * s->KVW, EPI_ACCUM));
}

// On-policy distillation (trainer/distill.go:13-46) runs the policy-gradient
// step's training forward and backward with the distillation loss in place
// of the PG loss: the frozen teacher's final hidden states of the same rows
// (teacher.Forward up to its final norm) give its logits chunk by chunk.
struct DistillCtx {
  const gn_session* teacher;
  const float* tfn;  // teacher's final normalized hidden states [N, teacher C]
  double tau;
  float scale;  // 1 / (valid tokens * gradient-accumulation steps)
};

static void pg_step_chunk(gn_session* s, const int32_t* inputs, const int32_t* targets, int B,
                          int T, const float* adv, float norm, double* loss_out, float* nll_out,
                          const DistillCtx* dc = nullptr) {
  GN_CHECK(B > 0 && T > 1, "policy gradient step: need batch > 0 and seq_len > 1");
  GN_CHECK(T <= s->S, "model: sequence longer than rotary cache");
  const int C = s->C, Hq = s->Hq, Hkv = s->Hkv, F = s->F, L = s->L, V = s->V;
  const int64_t N = (int64_t)B * T;
  hipStream_t st = s->stream;
  for (int64_t i = 0; i < N; i++)
    GN_CHECK(targets[i] == -1 || (targets[i] >= 0 && targets[i] < V), "target id out of range");
  hipEvent_t ev0 = nullptr, ev1 = nullptr;
  s->loss_events.clear();
  s->loss_ev_bytes.clear();
  if (s->timing) {
    ev0 = next_event(s);
    ev1 = next_event(s);
    GN_HIP(hipEventRecord(ev0, st));
  }
  SeqBuffers sb;
  sb.B = B; sb.T = T; sb.N = N;
  sb.ids = upload_ids(s, "ids", inputs, N, V);
  // the tokens grouped by id (counting sort, token order kept within an id)
  // for the deterministic embedding-gradient scatters
  std::vector<int32_t> grp;  // perm [N] | off [U+1] | uid [U]
  {
    std::vector<int32_t> cnt((size_t)s->PV + 1, 0);
    for (int64_t i = 0; i < N; i++) cnt[(size_t)inputs[i] + 1]++;
    int U = 0;
    for (int v = 0; v < s->PV; v++) U += cnt[(size_t)v + 1] > 0;
    for (int v = 0; v < s->PV; v++) cnt[(size_t)v + 1] += cnt[v];
    grp.resize((size_t)N + 2 * (size_t)U + 1);
    int32_t *perm = grp.data(), *off = perm + N, *uid = off + U + 1;
    std::vector<int32_t> fill(cnt.begin(), cnt.end() - 1);
    for (int64_t i = 0; i < N; i++) perm[fill[inputs[i]]++] = (int32_t)i;
    int u = 0;
    for (int v = 0; v < s->PV; v++)
      if (cnt[(size_t)v + 1] > cnt[v]) {
        off[u] = cnt[v];
        uid[u++] = v;
      }
    off[U] = (int32_t)N;
    int32_t* d = A<int32_t>(s, "id_groups", grp.size());
    GN_HIP(hipMemcpyAsync(d, grp.data(), sizeof(int32_t) * grp.size(), hipMemcpyHostToDevice, st));
    sb.groups.perm = d;
    sb.groups.off = d + N;
    sb.groups.uid = d + N + U + 1;
    sb.groups.n_ids = U;
  }
  int32_t* dtg = A<int32_t>(s, "targets", N);
  GN_HIP(hipMemcpyAsync(dtg, targets, sizeof(int32_t) * N, hipMemcpyHostToDevice, st));
  float* dadv = A<float>(s, "adv", B);
  GN_HIP(hipMemcpyAsync(dadv, adv, sizeof(float) * B, hipMemcpyHostToDevice, st));
  seq_forward(s, sb, SEQ_TRAIN, nullptr, nullptr);

  // ---- fused lm_head + softcap + PG loss + softcap backward, row chunks --
  // Only rows with a target have a loss and a logits gradient: an ignored
  // row's NLL, loss term and gradient row are exactly zero (rl.go:25-56,
  // loss.go:16-46), so the lm_head forward and both of its backward
  // products run over the rows with targets alone (gathered in order), and
  // their hidden-state gradients are scattered back into a zeroed dfn.
  std::vector<int32_t> vrows;
  vrows.reserve(N);
  for (int64_t i = 0; i < N; i++)
    if (targets[i] >= 0) vrows.push_back((int32_t)i);
  const int64_t Nv = (int64_t)vrows.size();
  const bool compact = Nv < N;
  float* nll = A<float>(s, "nll", N);
  double* loss_rows = A<double>(s, "loss_rows", std::max<int64_t>(Nv, 1));
  float* dfn = A<float>(s, "dfn", N * C);
  const int32_t* rowmap = nullptr;
  const float* fnv = sb.fn;  // [Nv, C] final-norm rows with targets
  const float* tfnv = dc ? dc->tfn : nullptr;
  float* dfnv = dfn;
  if (compact) {
    GN_HIP(hipMemsetAsync(nll, 0, sizeof(float) * N, st));
    GN_HIP(hipMemsetAsync(dfn, 0, sizeof(float) * N * C, st));
    if (Nv > 0) {
      int32_t* drm = A<int32_t>(s, "loss_rowmap", Nv);
      GN_HIP(hipMemcpyAsync(drm, vrows.data(), sizeof(int32_t) * Nv, hipMemcpyHostToDevice, st));
      rowmap = drm;
      float* g1 = A<float>(s, "loss_fn_rows", Nv * C);
      launch_gather_rows(sb.fn, drm, g1, Nv, C, st);
      fnv = g1;
      if (dc) {
        const int Ct = dc->teacher->C;
        float* g2 = A<float>(s, "loss_tfn_rows", Nv * Ct);
        launch_gather_rows(dc->tfn, drm, g2, Nv, Ct, st);
        tfnv = g2;
      }
      dfnv = A<float>(s, "loss_dfn_rows", Nv * C);
    }
  }
  const int64_t chunk = logits_chunk(s, std::max<int64_t>(Nv, 1));
  float* Z = A<float>(s, "logits", chunk * V);
  float* Zt = dc ? A<float>(s, "teacher_logits", chunk * V) : nullptr;
  for (int64_t r0 = 0; r0 < Nv; r0 += chunk) {
    const int64_t rows = std::min(chunk, Nv - r0);
    // lm_head products; the loss kernels apply the softcap on load
    sgemm(s, linear_fwd_desc(fnv + r0 * C, s->lm, Z, (int)rows, C, V));
    if (dc) {
      const int Ct = dc->teacher->C;
      sgemm(s, linear_fwd_desc(tfnv + r0 * Ct, dc->teacher->lm, Zt, (int)rows, Ct, V));
      launch_distill_rows(Z, Zt, V, V, r0, rows, rowmap, dtg, dc->tau, dc->scale, loss_rows, st);
    } else {
      if (s->timing && !s->capturing) {
      hipEvent_t a = next_event(s), b = next_event(s);
      GN_HIP(hipEventRecord(a, st));
      launch_pg_loss_rows(Z, V, V, r0, rows, rowmap, dtg, dadv, T, norm, nll, loss_rows, st);
      GN_HIP(hipEventRecord(b, st));
      s->loss_events.push_back({a, b});
      s->loss_ev_bytes.push_back(2.0 * 4.0 * (double)rows * V);
    } else {
      launch_pg_loss_rows(Z, V, V, r0, rows, rowmap, dtg, dadv, T, norm, nll, loss_rows, st);
    }
    }
    sgemm(s, linear_dx_desc(Z, s->lm, dfnv + r0 * C, (int)rows, C, V));
    sgemm(s, linear_dw_desc(Z, fnv + r0 * C, s->glm, (int)rows, C, V));
  }
  if (compact && Nv > 0) launch_scatter_rows(dfnv, rowmap, dfn, Nv, C, st);
  double* dloss = A<double>(s, "loss", 1);
  if (Nv > 0) launch_sum_f64(loss_rows, Nv, dloss, false, st);
  else GN_HIP(hipMemsetAsync(dloss, 0, sizeof(double), st));

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
  float* dqkv = s->mla ? nullptr : A<float>(s, "dqkv", N * s->QKVW);
  float* dpre = s->mla ? nullptr : A<float>(s, "dpre", N * Hkv);
  double* dauxl = nullptr;
  if (s->moe && s->bw > 0.f) {
    dauxl = A<double>(s, "aux_loss", 1);
    GN_HIP(hipMemsetAsync(dauxl, 0, sizeof(double), st));
  }
  const int bk = L / 2;
  float* genc = nullptr;
  if (s->hca) {  // the groups' compressed-KV gradient accumulators
    const size_t cw = (size_t)B * ceil_div(T, s->ratio) * s->KVW;
    for (int l = 0; l < L; l++)
      if (s->layers[l].mode == 'F') {
        GN_HIP(hipMemsetAsync(A<float>(s, "hca_gkc" + std::to_string(l), cw), 0, sizeof(float) * cw, st));
        GN_HIP(hipMemsetAsync(A<float>(s, "hca_gvc" + std::to_string(l), cw), 0, sizeof(float) * cw, st));
      }
    if (s->split > 0) {
      genc = A<float>(s, "ced_genc", N * C);
      GN_HIP(hipMemsetAsync(genc, 0, sizeof(float) * N * C, st));
    }
  }
  for (int l = L - 1; l >= 0; l--) {
    Layer& ly = s->layers[l];
    const float* lgp = g;
    if (l == bk && gback) {
      launch_axpy(lg, g, gback, nullptr, 1.f, N * C, st);
      lgp = lg;
    }
    if (s->moe) {
      moe_ffn_backward(s, ly, sb.moe[l], lgp, sb.h2[l], sb.gu[l], sb.act[l], B, T, dtmp, dauxl);
    } else {
      // MLP (train.go:505-514): du = (lg . Wproj) * 2 relu(u); dh2 = du . Wfc
      GemmDesc d1 = linear_dx_desc(lgp, ly.wproj, du, (int)N, F, C, EPI_DRELU2);
      d1.aux = sb.u[l]; d1.ldaux = F;
      sgemm(s, d1);
      sgemm(s, linear_dw_desc(lgp, sb.act[l], ly.gproj, (int)N, F, C));
      sgemm(s, linear_dx_desc(du, ly.wfc, dtmp, (int)N, C, F));
      sgemm(s, linear_dw_desc(du, sb.h2[l], ly.gfc, (int)N, C, F));
    }
    launch_rmsnorm_bwd(sb.mid[l], dtmp, lgp, N, C, gmid, st);
    // attention (train.go:198-427)
    float* dout = dtmp;  // [N, Hq*D] (Hq*D == C)
    sgemm(s, linear_dx_desc(gmid, ly.wo, dout, (int)N, Hq * HD, C));
    sgemm(s, linear_dw_desc(gmid, sb.o[l], ly.go, (int)N, Hq * HD, C));
    std::vector<DhExtra> extra;
    if (s->hca) {
      hca_backward(s, sb, ly, l, dout, delta, dqn, dkn, dvv, extra, genc);
    } else {
      FlashBwdArgs fb{};
      fb.q = sb.qn[l]; fb.k = sb.kn[l]; fb.v = sb.v[l]; fb.o = sb.o[l]; fb.dout = dout;
      fb.lse = sb.lse[l]; fb.delta = delta; fb.dq = dqn; fb.dk = dkn; fb.dv = dvv;
      fb.B = B; fb.T = T; fb.Hq = Hq; fb.Hkv = Hkv; fb.window = ly.window;
      launch_flash_bwd(fb, st);
    }
    float* dh = dout;  // reuse: dout no longer needed
    if (s->mla) {
      mla_backward(s, ly, sb.xa[l], sb.h[l], dqn, dkn, dvv, N, T, dh);
    } else {
    QkvPostBwdArgs qb{};
    qb.dqn = dqn; qb.dkn = dkn; qb.dv = dvv; qb.qrot = sb.qrot[l]; qb.krot = sb.krot[l];
    qb.vesig = ly.has_ve ? sb.vesig[l] : nullptr;
    qb.ve = ly.ve; qb.ids = sb.ids; qb.cosT = s->cosT; qb.sinT = s->sinT;
    qb.Hq = Hq; qb.Hkv = Hkv; qb.R = s->R; qb.T = T;
    qb.dqkv = dqkv; qb.dpre = dpre;
    qb.gve_rows = ly.has_ve ? A<float>(s, "gve_rows", (size_t)N * Hkv * HD) : nullptr;
    launch_qkv_post_bwd(qb, N, st);
    if (ly.has_ve) launch_rows_scatter(qb.gve_rows, sb.groups, Hkv * HD, ly.gve, st);
    sgemm(s, linear_dx_desc(dqkv, ly.wqkv, dh, (int)N, C, s->QKVW));
    sgemm(s, linear_dw_desc(dqkv, sb.h[l], ly.gqkv, (int)N, C, s->QKVW));
    if (ly.has_ve) launch_ve_gate_bwd(dpre, sb.h[l], ly.wve, C, Hkv, N, ly.gwve, dh, part, st);
    for (const DhExtra& e : extra) sgemm(s, linear_dx_desc(e.g, e.W, dh, (int)N, C, e.K, EPI_ACCUM));
    }
    launch_rmsnorm_bwd(sb.xb[l], dh, gmid, N, C, gb, st);
    // residual mixing (train_transformer.go:218-240)
    launch_dot_into_grad(gb, sb.xin[l], sb.x0, 1.f, N * C, s->grl + l, s->gx0l + l, part, st);
    launch_resid_bwd(gb, s->rl, s->x0l, l, g, gx0, N * C, st);
    // CED: the decoder's global-KV gradient enters at the encoder output
    // (train_transformer.go:221-229)
    if (genc && l == s->split) launch_axpy(g, g, genc, nullptr, 1.f, N * C, st);
  }
  launch_axpy(g, g, gx0, nullptr, 1.f, N * C, st);
  // smear, embedding norm, embedding scatter (train_transformer.go:244-264)
  float* ge = A<float>(s, "ge", N * C);
  float* ggate = A<float>(s, "ggate", std::max<int64_t>((int64_t)B * (T - 1), 1));
  double* lam_rows = A<double>(s, "lam_rows", std::max<int64_t>((int64_t)B * (T - 1), 1));
  launch_smear_bwd(g, sb.embn, sb.smsig, s->sml, s->smg, B, T, C, ge, ggate, lam_rows, part,
                   s->gsmg, s->gsml, st);
  launch_rmsnorm_bwd(sb.raw, ge, nullptr, N, C, gb, st);
  launch_rows_scatter(gb, sb.groups, C, s->gwte, st);

  double loss = 0, aux = 0;
  GN_HIP(hipMemcpyAsync(&loss, dloss, sizeof(double), hipMemcpyDeviceToHost, st));
  if (dauxl) GN_HIP(hipMemcpyAsync(&aux, dauxl, sizeof(double), hipMemcpyDeviceToHost, st));
  if (nll_out) GN_HIP(hipMemcpyAsync(nll_out, nll, sizeof(float) * N, hipMemcpyDeviceToHost, st));
  if (s->timing) GN_HIP(hipEventRecord(ev1, st));
  GN_HIP(hipStreamSynchronize(st));
  if (loss_out) *loss_out = loss;
  // moe.go:313: weight * sum over sequences / sequences, summed over layers
  s->aux_loss = dauxl ? (double)s->bw * aux / (double)B : 0.0;
  if (s->timing) {
    float ms = 0;
    GN_HIP(hipEventElapsedTime(&ms, ev0, ev1));
    s->t.train_ms = ms;
    s->t.gemm_ms = 0; s->t.gemm_flops = 0; s->t.gemm_launches = 0;
    s->t.gemm_wide_ms = 0; s->t.gemm_wide_flops = 0; s->t.gemm_wide_launches = 0;
    double am = 0, ab = 0;
    int64_t an = 0;
    collect_timing(s, &s->t.gemm_ms, &s->t.gemm_flops, &s->t.gemm_launches, &am, &ab, &an,
                   &s->t.gemm_wide_ms, &s->t.gemm_wide_flops, &s->t.gemm_wide_launches);
    s->t.loss_ms = 0; s->t.loss_bytes = 0; s->t.loss_launches = 0;
    for (size_t i = 0; i < s->loss_events.size(); i++) {
      float lms = 0;
      GN_HIP(hipEventElapsedTime(&lms, s->loss_events[i].first, s->loss_events[i].second));
      s->t.loss_ms += lms;
      s->t.loss_bytes += s->loss_ev_bytes[i];
      s->t.loss_launches++;
    }
  }
  s->loss_events.clear();
  s->loss_ev_bytes.clear();
}

// Sequences per micro-batch of the policy-gradient step: the saved
// activations of one micro-batch stay within 160 GB (an estimate per token
// of every layer's saved tensors).  The loss, the NLL and the gradients are
// sums over sequences, so micro-batching changes only the float summation
// order (the balance loss keeps the whole batch's sequence count).
static int pg_micro_batch(gn_session* s, int B, int T) {
  const int64_t C = s->C;
  const int64_t per_layer = 10 * C + 3 * (int64_t)s->Hq * HD + 6 * (int64_t)s->KVW +
                            3 * (int64_t)s->F +
                            (s->moe ? (int64_t)s->K * (2 * C + 3 * (int64_t)s->EH) + 2 * s->E : 0) +
                            (s->hca ? 4 * HD : 0);
  const int64_t per_tok = s->L * per_layer + 16 * C;
  const int64_t budget = (int64_t)160 << 30;
  int64_t mb = std::max<int64_t>(1, std::min<int64_t>(B, budget / (4 * per_tok * T)));
  if (const char* e = getenv("GN_PG_MICRO_BATCH"))  // a smaller cap (tests)
    mb = std::min<int64_t>(mb, std::max(1, atoi(e)));
  return (int)mb;
}

// trainer.PolicyGradientStep (trainer/rl.go:14-60) over the batch, in
// micro-batches of sequences when it is too large for one pass.
static void pg_step(gn_session* s, const int32_t* inputs, const int32_t* targets, int B, int T,
                    const float* adv, float norm, float* loss_out, float* nll_out) {
  const int mb = pg_micro_batch(s, B, T);
  double loss = 0, aux = 0, tms = 0, gms = 0, gfl = 0, wms = 0, wfl = 0, lms = 0, lby = 0;
  int64_t gn = 0, wn = 0, ln = 0;
  s->bal_batch = B;
  try {
    for (int b0 = 0; b0 < B; b0 += mb) {
      const int nb = std::min(mb, B - b0);
      double l = 0;
      pg_step_chunk(s, inputs + (int64_t)b0 * T, targets + (int64_t)b0 * T, nb, T, adv + b0, norm,
                    &l, nll_out ? nll_out + (int64_t)b0 * T : nullptr);
      loss += l;
      aux += s->aux_loss * nb;
      tms += s->t.train_ms; gms += s->t.gemm_ms; gfl += s->t.gemm_flops; gn += s->t.gemm_launches;
      wms += s->t.gemm_wide_ms; wfl += s->t.gemm_wide_flops; wn += s->t.gemm_wide_launches;
      lms += s->t.loss_ms; lby += s->t.loss_bytes; ln += s->t.loss_launches;
    }
  } catch (...) {
    s->bal_batch = 0;
    throw;
  }
  s->bal_batch = 0;
  if (loss_out) *loss_out = (float)loss;
  s->aux_loss = aux / B;
  if (s->timing) {
    s->t.train_ms = tms; s->t.gemm_ms = gms; s->t.gemm_flops = gfl; s->t.gemm_launches = gn;
    s->t.gemm_wide_ms = wms; s->t.gemm_wide_flops = wfl; s->t.gemm_wide_launches = wn;
    s->t.loss_ms = lms; s->t.loss_bytes = lby; s->t.loss_launches = ln;
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
  bool in_thinking = false;
  int thinking_tokens = 0;
  bool completed = false;
};

// GenerateOptions with the engine's tokenizer ids and tool registry
// (inference/engine.go:25-34, 215-224): the byte-level tokenizer
// (tokenizer/special.go:19-31), thinking off and the built-in calculator.
static gn_generate_options default_generate_options() {
  gn_generate_options o{};
  o.thinking = 0;
  o.thinking_budget = 0;
  o.bos = TOK_BOS;
  o.assistant_end = TOK_ASSISTANT_END;
  o.tool_start = TOK_TOOL_START;
  o.tool_end = TOK_TOOL_END;
  o.tool_output_start = TOK_TOOL_OUTPUT_START;
  o.tool_output_end = TOK_TOOL_OUTPUT_END;
  o.think_start = TOK_THINK_START;
  o.think_end = TOK_THINK_END;
  o.tool = nullptr;
  o.tool_user = nullptr;
  return o;
}

// Registry.Execute(Tokenizer.Decode(call)) then Tokenizer.Encode of the
// result (engine.go:282-296): the caller's tool, or the built-in calculator
// over the byte-level tokenizer.  Appends <|tool_output_start|>, the result
// ids and <|tool_output_end|> to the row's forced tokens when a tool
// understands the call.
static void run_tool(const gn_generate_options& o, RowState& rs) {
  std::vector<int> result;
  if (o.tool) {
    std::vector<int32_t> call(rs.tool.begin(), rs.tool.end());
    std::vector<int32_t> out(4096);
    int32_t n = o.tool(o.tool_user, call.data(), (int32_t)call.size(), out.data(),
                       (int32_t)out.size());
    if (n < 0) return;
    GN_CHECK(n <= (int32_t)out.size(), "tool: result longer than 4096 tokens");
    result.assign(out.begin(), out.begin() + n);
  } else {
    auto res = calculator(decode_tokens(rs.tool));
    if (!res) return;
    result = encode_bytes(*res);
  }
  rs.forced.push_back(o.tool_output_start);
  rs.forced.insert(rs.forced.end(), result.begin(), result.end());
  rs.forced.push_back(o.tool_output_end);
}

// Absorbed decode weights (mla.go:233-273 folded): per query head h with KV
// head kv, W_qabs[h] = KeyUp_kv^T . QueryUp_h ([lat, lat]: the content query
// times the key up-projection, as a map of the query latent) and
// W_comb[:, h] = Wo[:, h] . ValueUp_kv ([C, lat]: the value up-projection
// followed by the output projection).
static void prepare_decode_weights(gn_session* s) {
  if (!s->mla || !s->derived_dirty) return;
  const int lat = s->lat, cd = s->cd, Hq = s->Hq, ratio = s->Hq / s->Hkv, C = s->C;
  for (int l = 0; l < s->L; l++) {
    Layer& ly = s->layers[l];
    const float* wku = ly.wkvu;
    const float* wvu = ly.wkvu + (int64_t)s->Hkv * cd * lat;
    for (int h = 0; h < Hq; h++) {
      const int kv = h / ratio;
      GemmDesc a;  // [rank][j] = sum_c KeyUp[kv*cd + c][rank] * QueryUp[h*cd + c][j]
      a.M = lat; a.N = lat; a.K = cd;
      a.A = wku + (int64_t)kv * cd * lat; a.lda = lat; a.a_kcontig = false;
      a.B = ly.wqu + (int64_t)h * cd * lat; a.ldb = lat; a.b_kcontig = false;
      a.C = ly.wqabs + (int64_t)h * lat * lat; a.ldc = lat;
      gemm(a, s->stream, s->arena.get());
      GemmDesc b;  // [c][h*lat + rank] = sum_d Wo[c][h*D + d] * ValueUp[kv*D + d][rank]
      b.M = C; b.N = lat; b.K = HD;
      b.A = ly.wo + (int64_t)h * HD; b.lda = C; b.a_kcontig = true;
      b.B = wvu + (int64_t)kv * HD * lat; b.ldb = lat; b.b_kcontig = false;
      b.C = ly.wcomb + (int64_t)h * lat; b.ldc = (int64_t)Hq * lat;
      gemm(b, s->stream, s->arena.get());
    }
  }
  s->derived_dirty = false;
}

// One absorbed-MLA decode layer (mlaForwardInference, mla.go:185-279) on
// h; the attention output projection is added into x.
// The output projection's residual add is left pending on x (*pend) for the
// MLP norm; the input projection's split-K sum is applied by the prep kernel.
static void mla_decode_layer(gn_session* s, const Layer& ly, int l, int rows, int pos, int maxSeq,
                             const float* h, float* latc, float* rkc, float* x, const int* dpos,
                             PendingSum* pend) {
  const int C = s->C, Hq = s->Hq, lat = s->lat;
  hipStream_t st = s->stream;
  float* xa = A<float>(s, "dec_xa", (size_t)rows * s->XW);
  PendingSum xsum;
  GemmDesc gx = linear_fwd_desc(h, ly.wxa, xa, rows, C, s->XW);
  gx.defer = &xsum;
  sgemm(s, gx);
  float* qabs = A<float>(s, "dec_qabs", (size_t)rows * Hq * lat);
  MlaDecodeArgs md{};
  md.xa = xa; md.xw = s->XW; md.qabs = qabs;
  md.xa_sum = xsum; md.xa_w = xa;
  md.qrope = A<float>(s, "dec_qrope", (size_t)rows * Hq * s->rd);
  md.lat_cache = latc + (int64_t)l * rows * maxSeq * lat;
  md.rk_cache = rkc + (int64_t)l * rows * maxSeq * s->Hkv * s->rd;
  md.cosT = s->cosT; md.sinT = s->sinT;
  md.out = A<float>(s, "dec_ol", (size_t)rows * Hq * lat);
  md.part_splits = mla_decode_max_splits(maxSeq, maxSeq);
  md.part = A<float>(s, "dec_mlapart", (size_t)rows * md.part_splits * Hq * (lat + 2));
  md.rows = rows; md.Hq = Hq; md.Hkv = s->Hkv; md.lat = lat; md.rd = s->rd;
  md.maxSeq = maxSeq; md.window = ly.window; md.pos = pos; md.pos_dev = dpos;
  launch_mla_decode_prep(md, st);
  GemmDesc gq = linear_fwd_desc(xa, ly.wqabs, qabs, rows, lat, Hq * lat);
  gq.lda = s->XW;
  sgemm(s, gq);
  if (s->timing && !s->capturing) {
    const int keys = pos + 1 - std::max(0, pos - ly.window);
    timed_attention(s, (double)rows * keys * (lat + s->Hkv * s->rd) * 4.0, md,
                    [&] { launch_mla_decode(md, st); });
  } else {
    launch_mla_decode(md, st);
  }
  GemmDesc go = linear_fwd_desc(md.out, ly.wcomb, x, rows, Hq * lat, C, EPI_ADD_SRC);
  go.aux = x; go.ldaux = C;
  go.defer = pend;
  sgemm(s, go);
}

// One decode forward: tokens dtok at position pos -> logits.  With dpos set
// the position is read on the device (the step is captured once and
// replayed).
// forwardCompressed / forwardCompressedSparse (compress_attention.go:895-1146)
// for one decode step of layer l: a Full layer buffers the token (on a CED
// decoder layer its projections of the encoder hidden state) and compresses
// a completed block (with its indexer key); a Reindex layer caches its own
// indexer key of the producer's new block; then the selection -- the
// indexer's top-k (within the Full layer's pool on a Reindex layer, the
// published one on a Reuse layer) -- and the attention arguments over the
// group's compressed cache merged with the local window.
static void hca_decode_layer(gn_session* s, const Layer& ly, int l, int rows, int pos, int maxSeq,
                             const float* h, const float* enc, const float* kcl, const float* vcl,
                             const int* dpos, DecodeAttnArgs& da) {
  const int C = s->C, Hkv = s->Hkv, HI = s->HI, mb = s->maxBlocks;
  hipStream_t st = s->stream;
  const int64_t cstride = (int64_t)rows * Hkv * mb * HD;
  const bool ced = s->split > 0 && l >= s->split;
  if (ly.mode == 'F') {
    const float* hin = ced ? enc : h;
    float* clog = A<float>(s, "dec_clog", (size_t)rows * HD);
    sgemm(s, linear_fwd_desc(hin, ly.wcl, clog, rows, C, HD));
    HcaDecodeArgs hd{};
    hd.clog = clog; hd.bias = ly.cbias;
    hd.ring = s->hring + (int64_t)l * rows * s->ratio * HD;
    hd.kc = kcl; hd.vc = vcl;
    if (ced) {  // the token's global key/value from the encoder hidden state
      float* kv = A<float>(s, "dec_cedkv", (size_t)rows * 2 * s->KVW);
      sgemm(s, linear_fwd_desc(enc, ly.wqkv + (int64_t)s->Hq * HD * C, kv, rows, C, 2 * s->KVW));
      QkvPostArgs qa{};
      qa.qkv = kv; qa.cosT = s->cosT; qa.sinT = s->sinT;
      qa.C = C; qa.Hq = 0; qa.Hkv = Hkv; qa.R = s->R; qa.T = 1; qa.pos0 = pos; qa.pos_dev = dpos;
      qa.kn = A<float>(s, "dec_cedk", (size_t)rows * s->KVW);
      qa.vout = A<float>(s, "dec_cedv", (size_t)rows * s->KVW);
      launch_qkv_post(qa, rows, st);
      const int64_t tw = (int64_t)rows * Hkv * s->ratio * HD;
      hd.knew = qa.kn; hd.vnew = qa.vout;
      hd.tailk = s->htailk + (int64_t)l * tw;
      hd.tailv = s->htailv + (int64_t)l * tw;
    }
    hd.ck = s->hck + (int64_t)l * cstride;
    hd.cv = s->hcv + (int64_t)l * cstride;
    hd.rows = rows; hd.Hkv = Hkv; hd.ratio = s->ratio; hd.maxSeq = maxSeq;
    hd.maxBlocks = mb; hd.pos = pos; hd.pos_dev = dpos;
    launch_hca_decode_compress(hd, st);
  }
  const int p = ly.producer;
  const int64_t ikstride = (int64_t)rows * mb * Hkv * HI;
  if (ly.has_idx)  // this layer's indexer key of the block completed now
    launch_indexer_key_step(s->hck + (int64_t)p * cstride, ly.wik, s->hikc + (int64_t)l * ikstride,
                            rows, Hkv, mb, HI, s->ratio, pos, dpos, st);
  da.ck = s->hck + (int64_t)p * cstride;
  da.cv = s->hcv + (int64_t)p * cstride;
  da.maxBlocks = mb; da.ratio = s->ratio; da.window = s->swa; da.kstart = 0;
  if (s->topk == 0) return;
  const int64_t sstride = (int64_t)rows * Hkv;
  int q = l;  // the layer whose selection this one attends
  if (ly.mode == 'U')
    for (q = l - 1; q > p && s->layers[q].mode == 'U'; q--) {
    }
  if (ly.mode != 'U') {
    float* iq = A<float>(s, "dec_iq", (size_t)rows * HI);
    sgemm(s, linear_fwd_desc(h, ly.wiq, iq, rows, C, HI));
    CsaShape sh{};
    sh.T = 1; sh.blocks = mb; sh.Hkv = Hkv; sh.ratio = s->ratio; sh.qoff = pos; sh.b0 = 0;
    sh.ldo = mb; sh.H = s->ih; sh.dim = s->idim; sh.qoff_dev = dpos;
    float* scores = A<float>(s, "dec_scores", (size_t)sstride * mb);
    IndexerScoreArgs ia{};
    ia.shape = sh; ia.iq = iq; ia.ik = s->hikc + (int64_t)l * ikstride; ia.w = ly.wih; ia.out = scores;
    launch_indexer_scores(ia, rows, st);
    CsaSelectArgs ca{};
    ca.shape = sh; ca.chunk_seqs = rows; ca.scores = scores;
    ca.K = s->topk; ca.pool = s->ipool; ca.gpt = s->gpt; ca.ccap = s->ccap;
    if (ly.mode == 'R' && s->ipool > 1) {
      ca.pool_in = s->dpool + (int64_t)p * sstride * s->ccap;
      ca.npool_in = s->dnpool + (int64_t)p * sstride;
    }
    if (ly.mode == 'F' && s->ipool > 1) {
      ca.pool_out = s->dpool + (int64_t)l * sstride * s->ccap;
      ca.npool_out = s->dnpool + (int64_t)l * sstride;
    }
    ca.sel = s->dsel + (int64_t)l * sstride * s->topk;
    ca.nsel = s->dnsel + (int64_t)l * sstride;
    ca.mode = s->csa_select_mode;
    launch_csa_select(ca, st);
  }
  da.sel = s->dsel + (int64_t)q * sstride * s->topk;
  da.nsel = s->dnsel + (int64_t)q * sstride;
  da.kcap = s->topk;
}

static void decode_step(gn_session* s, int rows, int pos, int maxSeq, int32_t* dtok, float* kc,
                        float* vc, float* logits, const int* dpos = nullptr,
                        const int32_t* ovr = nullptr) {
  const int C = s->C, Hq = s->Hq, Hkv = s->Hkv, F = s->F, L = s->L;
  hipStream_t st = s->stream;
  float* x = A<float>(s, "dec_x", (size_t)rows * C);
  float* x0 = A<float>(s, "dec_x0", (size_t)rows * C);
  float* h = A<float>(s, "dec_h", (size_t)rows * C);
  float* prev = A<float>(s, "dec_prev", (size_t)rows * C);
  float* qkv = s->mla ? nullptr : A<float>(s, "dec_qkv", (size_t)rows * s->QKVW);
  float* q = s->mla ? nullptr : A<float>(s, "dec_q", (size_t)rows * Hq * HD);
  float* o = s->mla ? nullptr : A<float>(s, "dec_o", (size_t)rows * Hq * HD);
  float* act = A<float>(s, "dec_act", (size_t)rows * F);
  float* back = A<float>(s, "dec_back", (size_t)rows * C);
  // split capacity of the attention partials: the largest split count of
  // any layer's key range (dense: the full-context layer's; compressed: the
  // blocks plus the local window)
  int part_splits = 1;
  for (const Layer& ly : s->layers) {
    DecodeAttnArgs cap{};
    cap.maxSeq = maxSeq; cap.window = std::min(ly.window, maxSeq);
    if (s->hca) {
      cap.window = s->swa; cap.ratio = s->ratio; cap.maxBlocks = s->maxBlocks;
    }
    part_splits = std::max(part_splits, decode_attention_split_cap(cap));
  }
  float* dec_enc = s->split > 0 ? A<float>(s, "dec_enc", (size_t)rows * C) : nullptr;
  float* part = s->mla ? nullptr
                       : A<float>(s, "dec_part", (size_t)rows * Hkv * part_splits *
                                                     (Hq / Hkv) * (HD + 2));
  // the embedding, smear and layer 0's residual mix + norm in one launch
  launch_embed_decode_mix(dtok, s->wte, s->smg, s->sml, s->rl, s->x0l, rows, C, prev, x, x0, h,
                          st, ovr);
  const int bk = L / 2;
  // The decode projections split K (M = rows is small); their partial sums
  // are added by the next row kernel instead of a reduction launch: qkv by
  // qkv_post, the attention output projection by the MLP norm, the MLP
  // output projection by the next layer's residual mix (or the final norm).
  PendingSum pend;  // a residual-add product pending on x
  bool back_pending = false;  // the backout copy is the next residual mix's summed x
  for (int l = 0; l < L; l++) {
    Layer& ly = s->layers[l];
    if (dec_enc && l == s->split)  // encoderHidden (transformer.go:310-312)
      GN_HIP(hipMemcpyAsync(dec_enc, x, sizeof(float) * rows * C, hipMemcpyDeviceToDevice, st));
    if (l > 0)
      launch_resid_norm(x, x0, s->rl, s->x0l, l, rows, C, x, h, st, pend,
                        back_pending ? back : nullptr);
    pend = PendingSum{};
    back_pending = false;
    if (s->mla) {
      mla_decode_layer(s, ly, l, rows, pos, maxSeq, h, kc, vc, x, dpos, &pend);
    } else {
    PendingSum qsum;
    GemmDesc gq = linear_fwd_desc(h, ly.wqkv, qkv, rows, C, s->QKVW);
    gq.defer = &qsum;
    sgemm(s, gq);
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
    qa.qkv_sum = qsum;
    // plain windows: the attention kernel does the q/k/v post-processing of
    // its own heads (one launch less per layer; GN_FUSE_QKV_POST=0 keeps
    // the separate launch, same results)
    const bool fuse = !s->hca && s->fuse_qkv_post && qsum.splits <= DECODE_POST_MAX_SPLITS;
    if (!fuse) launch_qkv_post(qa, rows, st);
    DecodeAttnArgs da{};
    da.fuse_post = fuse;
    da.post = qa;
    da.q = q; da.kc = qa.kcache; da.vc = qa.vcache; da.part = part; da.o = o;
    da.part_floats = (int64_t)rows * Hkv * part_splits * (Hq / Hkv) * (HD + 2);
    da.rows = rows; da.Hq = Hq; da.Hkv = Hkv; da.maxSeq = maxSeq;
    da.kstart = std::max(0, pos - ly.window);
    da.kend = pos + 1;
    da.pos_dev = dpos;
    da.window = ly.window;
    int64_t nkeys = da.kend - da.kstart;
    if (s->hca) {
      hca_decode_layer(s, ly, l, rows, pos, maxSeq, h, dec_enc, qa.kcache, qa.vcache, dpos, da);
      nkeys = (s->topk > 0 ? std::min(s->topk, pos / s->ratio) : pos / s->ratio) +
              (s->swa > 0 ? pos - std::max(0, pos - s->swa) + 1 : 0);
    }
    if (s->timing && !s->capturing) {
      timed_attention(s, 2.0 * rows * Hkv * HD * 4.0 * nkeys, da,
                      [&] { launch_decode_attention(da, st); });
    } else {
      launch_decode_attention(da, st);
    }
    GemmDesc go = linear_fwd_desc(o, ly.wo, x, rows, Hq * HD, C, EPI_ADD_SRC);
    go.aux = x; go.ldaux = C;
    go.defer = &pend;
    sgemm(s, go);
    }
    launch_norm_rows(x, nullptr, nullptr, rows, C, nullptr, h, st, pend);
    pend = PendingSum{};
    if (s->moe) {
      float* gu = A<float>(s, "dec_gu", (size_t)rows * 2 * F);
      MoeBuffers mb = moe_buffers(s, "dec_moe_", rows);
      moe_ffn_forward(s, ly, x, h, rows, gu, act, mb, x, true);
      if (l == bk) GN_HIP(hipMemcpyAsync(back, x, sizeof(float) * rows * C, hipMemcpyDeviceToDevice, st));
      continue;
    }
    GemmDesc gf = linear_fwd_desc(h, ly.wfc, act, rows, C, F, EPI_RELU2_SAVE);
    sgemm(s, gf);
    GemmDesc gp = linear_fwd_desc(act, ly.wproj, x, rows, F, C, EPI_ADD_SRC);
    gp.aux = x; gp.ldaux = C;
    // x is copied at the next one's start (CED encoder state): that layer
    // sums its own product.  The backout copy of x after layer bk is written
    // by the next layer's residual mix, which sums the deferred product
    // (the same float64 sum + x as the reduction), unless bk is the last layer.
    const bool own = (dec_enc && l + 1 == s->split) || (l == bk && l + 1 == L);
    if (!own) gp.defer = &pend;
    sgemm(s, gp);
    if (l == bk) {
      if (own) GN_HIP(hipMemcpyAsync(back, x, sizeof(float) * rows * C, hipMemcpyDeviceToDevice, st));
      else back_pending = true;
    }
  }
  launch_norm_rows(x, back, s->bkl, rows, C, nullptr, h, st, pend);
  // lm_head products; the sampler applies the softcap on load
  sgemm(s, linear_fwd_desc(h, s->lm, logits, rows, C, s->V));
}

// PrefillCED (model/transformer.go:363-449) of G prompts: the encoder over
// the full prompts (its caches filled as in a plain prefill); every decoder
// Full layer's compressed blocks, logit ring and tail from its projections of
// the encoder's final hidden state (Reindex layers' indexer keys of them);
// then the decoder replayed over the last min(SWA window, P) tokens from the
// encoder rows with embedAndSmear's smear (the first replayed row is not
// mixed with the previous token; a lone replayed row is mixed with its own
// embedding, the cached previous one).  Leaves the replay's final norm in
// sb.fn and its embeddings in sb.embn; returns the replay length.
static int prefill_ced(gn_session* s, SeqBuffers& sb, const int32_t* prompts, int G, int P,
                       float* kpf, float* vpf, float* pf_tailk, float* pf_tailv) {
  const int C = s->C, Hq = s->Hq, Hkv = s->Hkv, L = s->L, split = s->split, ratio = s->ratio;
  hipStream_t st = s->stream;
  const int R = std::min(s->swa, P), rstart = P - R;
  const int64_t NP = (int64_t)G * P, NR = (int64_t)G * R;
  // 1) the encoder
  float* enc = A<float>(s, "cedpf_enc", NP * C);
  sb.l0 = 0; sb.l1 = split; sb.x_out = enc;
  seq_forward(s, sb, SEQ_PREFILL, kpf, vpf);
  // 2) the decoder's global caches
  const int blocks = (int)ceil_div(P, ratio), full = P / ratio;
  std::vector<float*> pre_kc(L, nullptr), pre_vc(L, nullptr);
  float* kv = A<float>(s, "cedpf_kv", NP * 2 * s->KVW);
  float* kg = A<float>(s, "cedpf_k", NP * s->KVW);
  float* vg = A<float>(s, "cedpf_v", NP * s->KVW);
  float* clog = A<float>(s, "cedpf_clog", NP * HD);
  float* probs = A<float>(s, "cedpf_probs", (size_t)G * blocks * ratio * HD);
  float* ik = s->topk > 0 ? A<float>(s, "cedpf_ik", (size_t)G * blocks * Hkv * s->HI) : nullptr;
  for (int l = split; l < L; l++) {
    const Layer& ly = s->layers[l];
    if (ly.mode == 'F') {
      sgemm(s, linear_fwd_desc(enc, ly.wqkv + (int64_t)Hq * HD * C, kv, (int)NP, C, 2 * s->KVW));
      QkvPostArgs qa{};
      qa.qkv = kv; qa.cosT = s->cosT; qa.sinT = s->sinT;
      qa.C = C; qa.Hq = 0; qa.Hkv = Hkv; qa.R = s->R; qa.T = P; qa.pos0 = 0;
      qa.kn = kg; qa.vout = vg;
      launch_qkv_post(qa, NP, st);
      sgemm(s, linear_fwd_desc(enc, ly.wcl, clog, (int)NP, C, HD));
      HcaCompressArgs ca{};
      ca.clog = clog; ca.bias = ly.cbias; ca.k = kg; ca.v = vg;
      ca.B = G; ca.T = P; ca.Hkv = Hkv; ca.ratio = ratio; ca.probs = probs;
      pre_kc[l] = ca.kc = A<float>(s, "cedpf_kc" + std::to_string(l), (size_t)G * blocks * s->KVW);
      pre_vc[l] = ca.vc = A<float>(s, "cedpf_vc" + std::to_string(l), (size_t)G * blocks * s->KVW);
      if (full > 0) {
        ca.ck_pf = sb.pf_ck + (int64_t)l * G * Hkv * full * HD;
        ca.cv_pf = sb.pf_cv + (int64_t)l * G * Hkv * full * HD;
      }
      ca.ring_pf = sb.pf_ring + (int64_t)l * G * ratio * HD;
      ca.tailk_pf = pf_tailk + (int64_t)l * G * Hkv * ratio * HD;
      ca.tailv_pf = pf_tailv + (int64_t)l * G * Hkv * ratio * HD;
      launch_hca_compress(ca, st);
    }
    if (ly.has_idx) {  // compressTail's / cacheReusedIndexerKeys' indexer keys
      sgemm(s, linear_fwd_desc(pre_kc[ly.producer], ly.wik, ik, G * blocks * Hkv, HD, s->HI));
      launch_replicate_rows(ik, sb.dec_ikc + (int64_t)l * G * sb.dec_S * sb.dec_maxBlocks * Hkv * s->HI,
                            G, sb.dec_S, full, Hkv * s->HI, blocks, sb.dec_maxBlocks, st);
    }
  }
  // 3) bounded replay of the decoder
  SeqBuffers rb;
  rb.B = G; rb.T = R; rb.N = NR;
  std::vector<int32_t> rids((size_t)NR);
  for (int g = 0; g < G; g++)
    memcpy(rids.data() + (size_t)g * R, prompts + (size_t)g * P + rstart, sizeof(int32_t) * R);
  rb.ids = upload_ids(s, "cedpf_rids", rids.data(), NR, s->V);
  float* xr = A<float>(s, "cedpf_xr", NR * C);
  GN_HIP(hipMemcpy2DAsync(xr, sizeof(float) * R * C, enc + (int64_t)rstart * C, sizeof(float) * P * C,
                          sizeof(float) * R * C, G, hipMemcpyDeviceToDevice, st));
  // embedAndSmear of the replayed tokens (transformer.go:452-477)
  float* embn = A<float>(s, "cedpf_embn", NR * C);
  float* smsig = A<float>(s, "cedpf_smsig", std::max<int64_t>((int64_t)G * (R - 1), 1));
  float* x0 = A<float>(s, "cedpf_x0", NR * C);
  launch_embed_smear(rb.ids, s->wte, s->smg, s->sml, G, R, C, nullptr, embn, smsig, x0, st);
  if (R == 1) {  // smearDecode with the cached previous embedding: its own
    float* prev = A<float>(s, "cedpf_prev", NR * C);
    float* xd = A<float>(s, "cedpf_xd", NR * C);
    GN_HIP(hipMemcpyAsync(prev, embn, sizeof(float) * NR * C, hipMemcpyDeviceToDevice, st));
    launch_embed_decode(rb.ids, s->wte, s->smg, s->sml, G, C, prev, xd, x0, st);
  }
  rb.qoff = rstart; rb.l0 = split; rb.x_in = xr; rb.x0_in = x0;
  rb.replay = true; rb.pre_kc = pre_kc; rb.pre_vc = pre_vc; rb.gblocks = blocks;
  rb.pf_maxseq = P;
  seq_forward(s, rb, SEQ_PREFILL, kpf, vpf);
  sb.fn = rb.fn;
  sb.embn = embn;
  return R;
}

// ---------------------------------------------------------------------------
// Prefix cache (inference/cache.go CacheManager, inference/prefix.go
// PrefixCache) on the device.  An entry holds one prompt's prefill state:
// every layer's token-major keys/values [L][P][Hkv*128] (what a continued
// prefill attends to), its decode-cache rows (dense and compressed: K and V
// [L][Hkv][P][128]; latent: the latent rows [L][P][lat] and rotated keys
// [L][P][Hkv*rd]), the last token's embedding (the next token's smear input,
// KVBuffer's PrevEmbedding) and, for compressed attention, the Full layers'
// compressor logits of every position.  A compressed model's continuation
// compresses the whole sequence again from the stored logits and keys/values
// together with the new rows' (the compressor pass is small next to the
// projections), which gives the blocks, the logit ring of an incomplete last
// block and the indexer keys exactly as a prefill from position 0 does.  The reference stores the whole KVBuffer
// (its sliding-window rows too, or with CacheOptions.StripSWA without them,
// rebuilt by a bounded replay on a hit: inference/cache.go:134-140,
// 286-311); here the raw rows of every position are kept, so no replay is
// needed.  Encoder-decoder (CED) models are not cached, as in the reference
// (inference/engine.go:128-140).
//
// Byte accounting (MaxBytes): an entry counts the device bytes it holds, the
// layout above -- not the reference's KVBuffer.BytesAllocated, whose
// prefill buffer is sized to the whole SequenceLen.
// ---------------------------------------------------------------------------
struct PcLayout {
  int64_t ktm, vtm, kdc, vdc, prev, clog, total;  // float offsets
};
static PcLayout pc_layout(const gn_session* s, int P) {
  PcLayout o;
  const int64_t tm = (int64_t)s->L * P * s->KVW;
  const int64_t kdc = s->mla ? (int64_t)s->L * P * s->lat : tm;
  const int64_t vdc = s->mla ? (int64_t)s->L * P * s->Hkv * s->rd : tm;
  o.ktm = 0;
  o.vtm = tm;
  o.kdc = 2 * tm;
  o.vdc = o.kdc + kdc;
  o.prev = o.vdc + vdc;
  o.clog = o.prev + s->C;
  // compressed attention: the compressor's logits of every position
  // [L][P][128] (the Full layers' rows; the compressed blocks, the logit
  // ring and the indexer keys are recomputed from them and the keys/values)
  o.total = o.clog + (s->hca ? (int64_t)s->L * P * HD : 0);
  return o;
}
static double pc_now() {
  return std::chrono::duration<double>(std::chrono::steady_clock::now().time_since_epoch()).count();
}
// Entries leave the list through pc_remove; their device memory is released
// at once, or -- while a prefill still reads it (pc_defer) -- when that
// prefill has finished (pc_flush).
// A disk-backed entry's file goes with it (removeEntryLocked, cache.go:
// 201-214), also deferred while a prefill runs (a failed call restores it).
static void pc_remove(gn_session* s, size_t i) {
  auto& e = s->pc_entries[i];
  s->pc_bytes -= e->bytes;
  if (s->pc_defer) {
    s->pc_retired.push_back(std::move(e));
  } else {
    if (!e->path.empty()) std::remove(e->path.c_str());
    if (e->mem) (void)hipFree(e->mem);
  }
  s->pc_entries.erase(s->pc_entries.begin() + i);
}
// Removed entries' memory goes to the pool, which keeps at most `keep`
// buffers (the newest); the rest is released.  Their files are deleted.
static void pc_flush(gn_session* s, size_t keep = 0) {
  for (auto& e : s->pc_retired) {
    if (!e->path.empty()) std::remove(e->path.c_str());
    if (e->mem) s->pc_pool.push_back({e->bytes, e->mem});
  }
  s->pc_retired.clear();
  while (s->pc_pool.size() > keep) {
    (void)hipFree(s->pc_pool.front().second);
    s->pc_pool.erase(s->pc_pool.begin());
  }
}
// Memory for a new entry: a pooled buffer of the same size, else hipMalloc.
static float* pc_alloc(gn_session* s, int64_t bytes) {
  for (size_t i = s->pc_pool.size(); i-- > 0;)
    if (s->pc_pool[i].first == bytes) {
      float* p = s->pc_pool[i].second;
      s->pc_pool.erase(s->pc_pool.begin() + i);
      return p;
    }
  float* p = nullptr;
  GN_HIP(hipMalloc(&p, bytes));
  return p;
}
// On-disk tier (CacheOptions.DiskDir; saveKVFile / loadKVFile, cache.go:
// 145-150, 254-284): one file per entry, named by a hash of its tokens, with
// the tokens in the header so that a file written for another sequence (a
// hash collision, a stale file) is refused on load.  Format: "GNPC", version
// 1, token count, state bytes (little-endian int64 each after the magic),
// the tokens (int32), the state (float32, gn::pc_layout).
static constexpr char PC_MAGIC[4] = {'G', 'N', 'P', 'C'};
static std::string pc_file(const gn_session* s, const std::vector<int32_t>& toks) {
  uint64_t h = 1469598103934665603ull;  // FNV-1a over the token bytes
  for (int32_t t : toks)
    for (int b = 0; b < 4; b++) {
      h ^= (uint64_t)(((uint32_t)t >> (8 * b)) & 0xff);
      h *= 1099511628211ull;
    }
  char name[64];
  snprintf(name, sizeof name, "%016llx-%zu.kv", (unsigned long long)h, toks.size());
  return (std::filesystem::path(s->pc_dir) / name).string();
}
// Writes e's device state to its file; true on success.
static bool pc_save(gn_session* s, gn_session::PrefixEntry& e) {
  const std::string path = pc_file(s, e.tokens);
  std::vector<char> host((size_t)e.bytes);
  if (hipMemcpy(host.data(), e.mem, (size_t)e.bytes, hipMemcpyDeviceToHost) != hipSuccess)
    return false;
  FILE* f = std::fopen(path.c_str(), "wb");
  if (!f) return false;
  const int64_t head[3] = {1, (int64_t)e.tokens.size(), e.bytes};
  bool ok = std::fwrite(PC_MAGIC, 1, 4, f) == 4 && std::fwrite(head, 8, 3, f) == 3 &&
            std::fwrite(e.tokens.data(), 4, e.tokens.size(), f) == e.tokens.size() &&
            std::fwrite(host.data(), 1, host.size(), f) == host.size();
  ok = std::fclose(f) == 0 && ok;
  if (!ok) {
    std::remove(path.c_str());
    return false;
  }
  e.path = path;
  return true;
}
// Reads e's file into fresh device memory; false (and nothing allocated)
// when the file is missing, short, or written for another sequence.
static bool pc_load(gn_session* s, gn_session::PrefixEntry& e) {
  FILE* f = std::fopen(e.path.c_str(), "rb");
  if (!f) return false;
  char magic[4];
  int64_t head[3];
  std::vector<int32_t> toks;
  std::vector<char> host;
  bool ok = std::fread(magic, 1, 4, f) == 4 && std::memcmp(magic, PC_MAGIC, 4) == 0 &&
            std::fread(head, 8, 3, f) == 3 && head[0] == 1 &&
            head[1] == (int64_t)e.tokens.size() && head[2] == e.bytes;
  if (ok) {
    toks.resize(e.tokens.size());
    host.resize((size_t)e.bytes);
    ok = std::fread(toks.data(), 4, toks.size(), f) == toks.size() && toks == e.tokens &&
         std::fread(host.data(), 1, host.size(), f) == host.size();
  }
  std::fclose(f);
  if (!ok) return false;
  float* mem = pc_alloc(s, e.bytes);
  if (hipMemcpy(mem, host.data(), (size_t)e.bytes, hipMemcpyHostToDevice) != hipSuccess) {
    s->pc_pool.push_back({e.bytes, mem});
    return false;
  }
  e.mem = mem;
  return true;
}
// expireLocked (cache.go:236-252): entries stored longer ago than the TTL
static void pc_expire(gn_session* s) {
  if (s->pc_ttl <= 0) return;
  const double now = pc_now();
  for (size_t i = s->pc_entries.size(); i-- > 0;)
    if (now - s->pc_entries[i]->stored_at > s->pc_ttl) pc_remove(s, i);
}
// Lookup (cache.go:79-119, prefix.go:38-60): the longest stored strict prefix
// of the prompt (none longer than max_prefix when that is set), moved to the
// most recently used end; nullptr on a miss.
static gn_session::PrefixEntry* pc_lookup(gn_session* s, const int32_t* toks, int P) {
  pc_expire(s);
  int best = -1;
  size_t best_len = 0;
  for (size_t i = 0; i < s->pc_entries.size(); i++) {
    const auto& e = s->pc_entries[i]->tokens;
    if (e.empty() || e.size() >= (size_t)P || e.size() <= best_len) continue;
    if (s->pc_max_prefix > 0 && e.size() > (size_t)s->pc_max_prefix) continue;
    if (std::equal(e.begin(), e.end(), toks)) {
      best = (int)i;
      best_len = e.size();
    }
  }
  if (best < 0) return nullptr;
  auto e = std::move(s->pc_entries[best]);
  s->pc_entries.erase(s->pc_entries.begin() + best);
  s->pc_entries.push_back(std::move(e));
  gn_session::PrefixEntry* hit = s->pc_entries.back().get();
  // a disk-backed entry is read back for this call; one that cannot be read
  // is dropped and the lookup misses (cache.go:112-117)
  if (!hit->mem && !pc_load(s, *hit)) {
    pc_remove(s, s->pc_entries.size() - 1);
    return nullptr;
  }
  return hit;
}
// evictLocked (cache.go:216-231): least recently used entries first, until
// the entry count and then the byte total fit
static void pc_evict(gn_session* s) {
  while (s->pc_max_entries > 0 && (int)s->pc_entries.size() > s->pc_max_entries) pc_remove(s, 0);
  while (s->pc_max_bytes > 0 && s->pc_bytes > s->pc_max_bytes && !s->pc_entries.empty())
    pc_remove(s, 0);
}
// Store (cache.go:121-161): replaces an entry of the same prompt, appends the
// new one at the most recently used end, then evicts.
static void pc_insert(gn_session* s, std::unique_ptr<gn_session::PrefixEntry> e) {
  for (size_t i = 0; i < s->pc_entries.size(); i++)
    if (s->pc_entries[i]->tokens == e->tokens) {
      pc_remove(s, i);
      break;
    }
  s->pc_bytes += e->bytes;
  s->pc_entries.push_back(std::move(e));
  pc_evict(s);
}
// Every entry, and the pooled memory, released.
static void pc_clear(gn_session* s) {
  while (!s->pc_entries.empty()) pc_remove(s, s->pc_entries.size() - 1);
  if (!s->pc_defer) pc_flush(s);
}

// Strided copies gathered on the host and run as one launch per batch.  The
// host descriptor arrays stay alive until the owner has synchronized the
// stream.
struct CopyList {
  std::vector<CopyBlock> v;
  std::vector<std::vector<CopyBlock>> sent;
  void add(const float* src, float* dst, int64_t count, int outer, int64_t s_outer,
           int64_t d_outer, int inner = 1, int64_t s_inner = 0, int64_t d_inner = 0) {
    if (count > 0 && outer > 0 && inner > 0)
      v.push_back(CopyBlock{src, dst, count, s_outer, s_inner, d_outer, d_inner, outer, inner});
  }
  void run(gn_session* s, const char* name) {
    if (v.empty()) return;
    sent.push_back(std::move(v));
    v.clear();
    const auto& h = sent.back();
    CopyBlock* d = A<CopyBlock>(s, name, h.size());
    GN_HIP(hipMemcpyAsync(d, h.data(), sizeof(CopyBlock) * h.size(), hipMemcpyHostToDevice,
                          s->stream));
    for (size_t i = 0; i < h.size(); i += 65535)
      launch_copy_blocks(d + i, (int)std::min<size_t>(65535, h.size() - i), s->stream);
  }
};

// The prefill of GenerateWith with a prefix cache (engine.go:120-173), for G
// prompts as G successive calls would see the cache: prompt g looks up the
// longest stored strict prefix, then stores its own state, evicting as the
// limits require (the prompts of one call have one length, so none is a
// strict prefix of another, but an earlier prompt's store can evict the
// entry a later one would have hit).  That sequence is settled on the host
// first, with the memory of entries it removes kept until the prefill has
// run.  Then the prompts without a hit are prefilled together from position
// 0, and the hits, batched by matched length m, continue from their entries
// over the last P - m tokens (the entries' keys attended first, their
// decode-cache rows copied in, the smear seeded with their stored embedding
// -- KVBuffer.PrevEmbedding; compressed attention: the stored compressor
// logits in front of the new rows').  Fills the decode prefill caches
// kpf/vpf (the plain prefill's layout), each prompt's last-row final norm
// and embedding lastfn/lastemb [G][C] and, for compressed attention, out's
// compressed caches pf_ck/pf_cv/pf_ring (layout [L][G]...) and indexer-key
// decode cache dec_ikc (out.dec_S rows per prompt), as seq_forward fills
// them for a plain prefill.
static void prefill_cached(gn_session* s, const int32_t* prompts, int G, int P, float* kpf,
                           float* vpf, float* lastfn, float* lastemb, const SeqBuffers& out) {
  GN_CHECK(s->split == 0, "prefix cache: encoder-decoder (CED) models are not cached");
  const int L = s->L, C = s->C, Hkv = s->Hkv;
  const int64_t KVW = s->KVW;
  // floats per (layer, prompt) of the decode prefill caches
  const int64_t kg = s->mla ? (int64_t)P * s->lat : (int64_t)Hkv * P * HD;
  const int64_t vg = s->mla ? (int64_t)P * Hkv * s->rd : (int64_t)Hkv * P * HD;
  const PcLayout lay = pc_layout(s, P);
  // compressed attention: per (layer, prompt) floats of the complete blocks'
  // cache, of the logit ring, and per (layer, row) of the indexer-key cache
  const bool hca = s->hca;
  const int full = hca ? P / s->ratio : 0;
  const int64_t cg = (int64_t)Hkv * full * HD;
  const int64_t rg = hca ? (int64_t)s->ratio * HD : 0;
  const int64_t ikw = hca && out.dec_ikc ? (int64_t)out.dec_maxBlocks * Hkv * s->HI : 0;
  if (hca) GN_CHECK(out.pf_ck && out.pf_cv && out.pf_ring, "prefix cache: compressed outputs");
  struct Plan {
    gn_session::PrefixEntry* src = nullptr;  // the hit (nullptr: a miss)
    int m = 0;
    gn_session::PrefixEntry* dst = nullptr;  // this prompt's new entry
  };
  std::vector<Plan> plan(G);
  CopyList cp;
  std::vector<std::vector<int32_t>> ids_kept;  // uploaded token ids, until the stream is idle
  // the list as the call found it (least recently used first), restored if
  // the call fails
  std::vector<gn_session::PrefixEntry*> before;
  for (const auto& e : s->pc_entries) before.push_back(e.get());
  s->pc_defer = true;
  try {
    // 1) the cache sequence of G successive GenerateWith calls
    for (int g = 0; g < G; g++) {
      const int32_t* toks = prompts + (int64_t)g * P;
      if (auto* e = pc_lookup(s, toks, P)) {
        plan[g].src = e;
        plan[g].m = (int)e->tokens.size();
      }
      auto ne = std::make_unique<gn_session::PrefixEntry>();
      ne->tokens.assign(toks, toks + P);
      ne->bytes = sizeof(float) * lay.total;
      ne->mem = pc_alloc(s, ne->bytes);
      ne->stored_at = pc_now();
      plan[g].dst = ne.get();
      pc_insert(s, std::move(ne));
    }
    s->pc_hits.assign(G, 0);
    for (int g = 0; g < G; g++) s->pc_hits[g] = plan[g].m;
    // compressed attention: a batch's compressed prefill caches, in the
    // batch's own layout (set up by hca_targets, moved by collect)
    float *bck = nullptr, *bcv = nullptr, *bring = nullptr, *bik = nullptr;
    auto hca_targets = [&](SeqBuffers& sb) {
      if (!hca) return;
      const int B = sb.B;
      bck = A<float>(s, "pc_bck", (size_t)L * B * std::max<int64_t>(cg, 1));
      bcv = A<float>(s, "pc_bcv", (size_t)L * B * std::max<int64_t>(cg, 1));
      bring = A<float>(s, "pc_bring", (size_t)L * B * rg);
      sb.pf_ck = bck;
      sb.pf_cv = bcv;
      sb.pf_ring = bring;
      if (ikw > 0) {
        bik = A<float>(s, "pc_bik", (size_t)L * B * ikw);
        sb.dec_ikc = bik;
        sb.dec_S = 1;
        sb.dec_maxBlocks = out.dec_maxBlocks;
      }
    };
    // one batch of prompts (prompt g at batch row i), positions [m, P): the
    // forward's decode caches kt/vt [L][B] and its last rows into the
    // call's per-prompt outputs, the whole prompts' keys/values (compressed:
    // and compressor logits clog [L][B][P][128]) into their entries
    auto collect = [&](const std::vector<int>& gs, int m, SeqBuffers& sb, const float* kt,
                       const float* vt, const float* kall, const float* vall, const float* clog) {
      const int B = (int)gs.size(), T = P - m;
      for (int i = 0; i < B; i++) {
        const int g = gs[i];
        cp.add(kt + i * kg, kpf + g * kg, kg, L, B * kg, G * kg);
        cp.add(vt + i * vg, vpf + g * vg, vg, L, B * vg, G * vg);
        const int64_t last = ((int64_t)i * T + T - 1) * C;
        cp.add(sb.fn + last, lastfn + (int64_t)g * C, C, 1, 0, 0);
        cp.add(sb.embn + last, lastemb + (int64_t)g * C, C, 1, 0, 0);
        float* dm = plan[g].dst->mem;
        cp.add(kall + (int64_t)i * P * KVW, dm + lay.ktm, (int64_t)P * KVW, L, (int64_t)B * P * KVW,
               (int64_t)P * KVW);
        cp.add(vall + (int64_t)i * P * KVW, dm + lay.vtm, (int64_t)P * KVW, L, (int64_t)B * P * KVW,
               (int64_t)P * KVW);
        // the state stored with the prompt: its decode-cache rows and last embedding
        cp.add(kt + i * kg, dm + lay.kdc, kg, L, B * kg, kg);
        cp.add(vt + i * vg, dm + lay.vdc, vg, L, B * vg, vg);
        cp.add(sb.embn + last, dm + lay.prev, C, 1, 0, 0);
        if (hca) {
          cp.add(bck + i * cg, out.pf_ck + g * cg, cg, L, B * cg, G * cg);
          cp.add(bcv + i * cg, out.pf_cv + g * cg, cg, L, B * cg, G * cg);
          cp.add(bring + i * rg, out.pf_ring + g * rg, rg, L, B * rg, G * rg);
          // the complete blocks' indexer keys into every row of the prompt
          if (ikw > 0)
            cp.add(bik + i * ikw, out.dec_ikc + (int64_t)g * out.dec_S * ikw,
                   (int64_t)full * Hkv * s->HI, L, B * ikw, (int64_t)G * out.dec_S * ikw,
                   out.dec_S, 0, ikw);
          for (int l = 0; l < L; l++)  // the Full layers' compressor logits
            if (s->layers[l].mode == 'F')
              cp.add(clog + ((int64_t)l * B + i) * P * HD, dm + lay.clog + (int64_t)l * P * HD,
                     (int64_t)P * HD, 1, 0, 0);
        }
      }
      cp.run(s, "pc_desc_out");
    };
    // 2) prompts with no cached prefix, together from position 0
    std::vector<int> miss;
    std::vector<std::pair<int, int>> hits;  // (m, g)
    for (int g = 0; g < G; g++) {
      if (plan[g].src) hits.push_back({plan[g].m, g});
      else miss.push_back(g);
    }
    if (!miss.empty()) {
      const int B = (int)miss.size();
      ids_kept.emplace_back((size_t)B * P);
      std::vector<int32_t>& ids = ids_kept.back();
      for (int i = 0; i < B; i++)
        memcpy(ids.data() + (size_t)i * P, prompts + (int64_t)miss[i] * P, sizeof(int32_t) * P);
      SeqBuffers sb;
      sb.B = B; sb.T = P; sb.N = (int64_t)B * P;
      sb.ids = upload_ids(s, "pc_ids", ids.data(), sb.N, s->V);
      sb.tm_k_out = A<float>(s, "pc_kall", (size_t)L * sb.N * KVW);
      sb.tm_v_out = A<float>(s, "pc_vall", (size_t)L * sb.N * KVW);
      if (hca) sb.tm_clog_out = A<float>(s, "pc_clog", (size_t)L * sb.N * HD);
      hca_targets(sb);
      float* kt = A<float>(s, "pc_kt", (size_t)L * B * kg);
      float* vt = A<float>(s, "pc_vt", (size_t)L * B * vg);
      seq_forward(s, sb, SEQ_PREFILL, kt, vt);
      collect(miss, 0, sb, kt, vt, sb.tm_k_out, sb.tm_v_out, sb.tm_clog_out);
    }
    // 3) hits, one batch per matched length (one prompt length per call, so
    //    equal m means equal continuation length)
    std::sort(hits.begin(), hits.end());
    for (size_t h0 = 0; h0 < hits.size();) {
      size_t h1 = h0;
      while (h1 < hits.size() && hits[h1].first == hits[h0].first) h1++;
      const int m = hits[h0].first, T = P - m, B = (int)(h1 - h0);
      std::vector<int> gs;
      for (size_t h = h0; h < h1; h++) gs.push_back(hits[h].second);
      const PcLayout el = pc_layout(s, m);
      float* kall = A<float>(s, "pc_kall", (size_t)L * B * P * KVW);
      float* vall = A<float>(s, "pc_vall", (size_t)L * B * P * KVW);
      float* kt = A<float>(s, "pc_kt", (size_t)L * B * kg);
      float* vt = A<float>(s, "pc_vt", (size_t)L * B * vg);
      float* prev = A<float>(s, "pc_prev", (size_t)B * C);
      float* clog = hca ? A<float>(s, "pc_clog", (size_t)L * B * P * HD) : nullptr;
      ids_kept.emplace_back((size_t)B * T);
      std::vector<int32_t>& ids = ids_kept.back();
      for (int i = 0; i < B; i++) {
        const float* em = plan[gs[i]].src->mem;
        memcpy(ids.data() + (size_t)i * T, prompts + (int64_t)gs[i] * P + m, sizeof(int32_t) * T);
        // the entry's keys/values: rows [0, m) of sequence i of every layer
        cp.add(em + el.ktm, kall + (int64_t)i * P * KVW, (int64_t)m * KVW, L, (int64_t)m * KVW,
               (int64_t)B * P * KVW);
        cp.add(em + el.vtm, vall + (int64_t)i * P * KVW, (int64_t)m * KVW, L, (int64_t)m * KVW,
               (int64_t)B * P * KVW);
        if (s->mla) {  // latent rows and rotated keys of positions [0, m)
          cp.add(em + el.kdc, kt + i * kg, (int64_t)m * s->lat, L, (int64_t)m * s->lat, B * kg);
          cp.add(em + el.vdc, vt + i * vg, (int64_t)m * Hkv * s->rd, L, (int64_t)m * Hkv * s->rd,
                 B * vg);
        } else {  // K and V rows [0, m) of every (layer, KV head)
          cp.add(em + el.kdc, kt + i * kg, (int64_t)m * HD, L, (int64_t)Hkv * m * HD, B * kg, Hkv,
                 (int64_t)m * HD, (int64_t)P * HD);
          cp.add(em + el.vdc, vt + i * vg, (int64_t)m * HD, L, (int64_t)Hkv * m * HD, B * vg, Hkv,
                 (int64_t)m * HD, (int64_t)P * HD);
        }
        cp.add(em + el.prev, prev + (int64_t)i * C, C, 1, 0, 0);
        if (hca)  // the Full layers' compressor logits of positions [0, m)
          for (int l = 0; l < L; l++)
            if (s->layers[l].mode == 'F')
              cp.add(em + el.clog + (int64_t)l * m * HD, clog + ((int64_t)l * B + i) * P * HD,
                     (int64_t)m * HD, 1, 0, 0);
      }
      cp.run(s, "pc_desc_in");
      SeqBuffers sb;
      sb.B = B; sb.T = T; sb.N = (int64_t)B * T;
      sb.ids = upload_ids(s, "pc_ids", ids.data(), sb.N, s->V);
      sb.qoff = m;
      sb.pf_maxseq = P;
      sb.pre_len = m;
      sb.kv_k = kall;
      sb.kv_v = vall;
      sb.pre_clog = clog;
      sb.seed_prev = prev;
      hca_targets(sb);
      seq_forward(s, sb, SEQ_PREFILL, kt, vt);
      collect(gs, m, sb, kt, vt, kall, vall, clog);
      h0 = h1;
    }
    GN_HIP(hipStreamSynchronize(s->stream));
  } catch (...) {
    // The cache as the call found it: its entries in their order (those the
    // call evicted or expired come back from pc_retired, untouched: retired
    // memory is not reused before the flush); the call's own entries, which
    // may be incomplete, are dropped and released after the stream has
    // drained.
    std::vector<std::unique_ptr<gn_session::PrefixEntry>> all;
    for (auto& e : s->pc_entries) all.push_back(std::move(e));
    for (auto& e : s->pc_retired) all.push_back(std::move(e));
    s->pc_entries.clear();
    s->pc_retired.clear();
    s->pc_bytes = 0;
    for (auto* want : before)
      for (auto& e : all)
        if (e.get() == want) {
          s->pc_bytes += e->bytes;
          s->pc_entries.push_back(std::move(e));
          break;
        }
    for (auto& e : all)
      if (e) s->pc_retired.push_back(std::move(e));
    (void)hipStreamSynchronize(s->stream);
    for (auto& e : s->pc_entries)  // read-back state of disk-backed entries
      if (!e->path.empty() && e->mem) {
        s->pc_pool.push_back({e->bytes, e->mem});
        e->mem = nullptr;
      }
    s->pc_defer = false;
    pc_flush(s);
    throw;
  }
  s->pc_defer = false;
  pc_flush(s, (size_t)G);  // removed entries' files deleted (before a same-prompt entry's is written)
  // disk tier: the new entries are written out (an entry whose file cannot be
  // written stays in device memory, as Store keeps it in memory), and every
  // disk-backed entry's device state is released
  if (!s->pc_dir.empty())
    for (auto& e : s->pc_entries)
      if (e->path.empty() && e->mem) pc_save(s, *e);
  for (auto& e : s->pc_entries)
    if (!e->path.empty() && e->mem) {
      s->pc_pool.push_back({e->bytes, e->mem});
      e->mem = nullptr;
    }
  pc_flush(s, (size_t)G);  // the next call of this size reuses them
}

static void generate(gn_session* s, const int32_t* prompts, int G, int P, int S, int N,
                     float temperature, int top_k, const uint64_t* seeds, int32_t* rows_out,
                     int32_t* lens_out, const gn_generate_options& opt, int32_t* masks_out) {
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
    if (masks_out) memset(masks_out + (int64_t)r * W, 0, sizeof(int32_t) * W);
  }
  s->pc_hits.assign(G, 0);
  // with a prefix cache the prompts are prefilled (and stored) even when no
  // token is asked for, as GenerateWith does
  if (N == 0 && !s->pc_on) return;
  // 1) batch prefill of every prompt (engine.go:141-173)
  SeqBuffers sb;
  sb.B = G; sb.T = P; sb.N = (int64_t)G * P;
  sb.ids = upload_ids(s, "pf_ids", prompts, sb.N, V);
  prepare_decode_weights(s);
  // dense: K and V [L][G][Hkv][P][D]; MLA: latent [L][G][P][lat] and rotary
  // keys [L][G][P][Hkv*rd]
  const size_t kw = s->mla ? (size_t)s->lat : (size_t)Hkv * HD;
  const size_t vw = s->mla ? (size_t)Hkv * s->rd : (size_t)Hkv * HD;
  float* kpf = A<float>(s, "pf_k", (size_t)L * G * P * kw);
  float* vpf = A<float>(s, "pf_v", (size_t)L * G * P * vw);
  const int maxSeq = W;
  const int pfull = s->hca ? P / s->ratio : 0;  // complete blocks of the prompt
  float *pf_tailk = nullptr, *pf_tailv = nullptr;
  if (s->hca) {  // decode caches (kvcache.go:142-220, 276-378)
    s->maxBlocks = maxSeq / s->ratio + 1;
    const size_t cbytes = (size_t)L * rows * Hkv * s->maxBlocks * HD;
    s->hck = A<float>(s, "kv_hck", cbytes);
    s->hcv = A<float>(s, "kv_hcv", cbytes);
    s->hring = A<float>(s, "kv_ring", (size_t)L * rows * s->ratio * HD);
    if (s->topk > 0) {
      s->hikc = A<float>(s, "kv_ikc", (size_t)L * rows * s->maxBlocks * Hkv * s->HI);
      s->dsel = A<int>(s, "dec_sel", (size_t)L * rows * Hkv * s->topk);
      s->dnsel = A<int>(s, "dec_nsel", (size_t)L * rows * Hkv);
      s->dpool = A<int>(s, "dec_pool", (size_t)L * rows * Hkv * s->ccap);
      s->dnpool = A<int>(s, "dec_npool", (size_t)L * rows * Hkv);
      sb.dec_ikc = s->hikc;
      sb.dec_S = S;
      sb.dec_maxBlocks = s->maxBlocks;
    }
    if (s->split > 0) {
      const size_t tw = (size_t)L * rows * Hkv * s->ratio * HD;
      s->htailk = A<float>(s, "kv_tailk", tw);
      s->htailv = A<float>(s, "kv_tailv", tw);
      pf_tailk = A<float>(s, "pf_tailk", (size_t)L * G * Hkv * s->ratio * HD);
      pf_tailv = A<float>(s, "pf_tailv", (size_t)L * G * Hkv * s->ratio * HD);
    }
    sb.pf_ck = A<float>(s, "pf_hck", (size_t)L * G * Hkv * std::max(pfull, 1) * HD);
    sb.pf_cv = A<float>(s, "pf_hcv", (size_t)L * G * Hkv * std::max(pfull, 1) * HD);
    sb.pf_ring = A<float>(s, "pf_ring", (size_t)L * G * s->ratio * HD);
  }
  int Tlast = P;
  const bool pcache = s->pc_on;
  float* lastfn = A<float>(s, "pf_lastfn", (size_t)rows * C);
  float *gfn = nullptr, *gemb = nullptr;  // per group (prefix cache)
  if (pcache) {
    gfn = A<float>(s, "pc_gfn", (size_t)G * C);
    gemb = A<float>(s, "pc_gemb", (size_t)G * C);
    prefill_cached(s, prompts, G, P, kpf, vpf, gfn, gemb, sb);
    if (N == 0) return;
    launch_expand_last_rows(gfn, lastfn, G, 1, S, C, st);
  } else {
    if (s->split > 0) Tlast = prefill_ced(s, sb, prompts, G, P, kpf, vpf, pf_tailk, pf_tailv);
    else seq_forward(s, sb, SEQ_PREFILL, kpf, vpf);
    // last-position logits of each prompt, expanded to its S rows (engine.go:182-191)
    launch_expand_last_rows(sb.fn, lastfn, G, Tlast, S, C, st);
  }
  float* logits = A<float>(s, "dec_logits", (size_t)rows * V);
  // lm_head products; the sampler applies the softcap on load
  sgemm(s, linear_fwd_desc(lastfn, s->lm, logits, rows, C, V));
  // 2) PrefillFrom (kvcache.go:383-448): replicate KV and the smear state
  float* kc = A<float>(s, "kv_k", (size_t)L * rows * maxSeq * kw);
  float* vc = A<float>(s, "kv_v", (size_t)L * rows * maxSeq * vw);
  if (s->hca) {
    for (int l = 0; l < L; l++) {
      if (pf_tailk) {
        const int64_t tw = (int64_t)Hkv * s->ratio * HD;
        launch_replicate_rows(pf_tailk + (int64_t)l * G * tw, s->htailk + (int64_t)l * rows * tw, G,
                              S, 1, (int)tw, 1, 1, st);
        launch_replicate_rows(pf_tailv + (int64_t)l * G * tw, s->htailv + (int64_t)l * rows * tw, G,
                              S, 1, (int)tw, 1, 1, st);
      }
      const int64_t dst = (int64_t)l * rows * Hkv * s->maxBlocks * HD;
      const int64_t src = (int64_t)l * G * Hkv * pfull * HD;
      launch_replicate_kv(sb.pf_ck + src, s->hck + dst, G, S, Hkv, pfull, pfull, s->maxBlocks, st);
      launch_replicate_kv(sb.pf_cv + src, s->hcv + dst, G, S, Hkv, pfull, pfull, s->maxBlocks, st);
      launch_replicate_rows(sb.pf_ring + (int64_t)l * G * s->ratio * HD,
                            s->hring + (int64_t)l * rows * s->ratio * HD, G, S, s->ratio, HD,
                            s->ratio, s->ratio, st);
    }
  }
  for (int l = 0; l < L; l++) {
    if (s->mla) {
      launch_replicate_rows(kpf + (int64_t)l * G * P * kw, kc + (int64_t)l * rows * maxSeq * kw, G,
                            S, P, (int)kw, P, maxSeq, st);
      launch_replicate_rows(vpf + (int64_t)l * G * P * vw, vc + (int64_t)l * rows * maxSeq * vw, G,
                            S, P, (int)vw, P, maxSeq, st);
      continue;
    }
    launch_replicate_kv(kpf + (int64_t)l * G * Hkv * P * HD, kc + (int64_t)l * rows * Hkv * maxSeq * HD,
                        G, S, Hkv, P, P, maxSeq, st);
    launch_replicate_kv(vpf + (int64_t)l * G * Hkv * P * HD, vc + (int64_t)l * rows * Hkv * maxSeq * HD,
                        G, S, Hkv, P, P, maxSeq, st);
  }
  float* prev = A<float>(s, "dec_prev", (size_t)rows * C);
  if (pcache) launch_expand_last_rows(gemb, prev, G, 1, S, C, st);
  else launch_expand_last_rows(sb.embn, prev, G, Tlast, S, C, st);

  // 3) decode loop (engine.go:238-325).  Step `step` runs the forward that
  //    feeds column step - 1 (none at step 0: the prefill logits) and
  //    samples column `step`.  After two eager steps (which size every
  //    buffer) forward + sampler are captured once as a HIP graph and
  //    replayed.  The sampler writes its ids into the buffer the next
  //    forward reads, so the steps are pipelined: step `step` is launched
  //    before the host runs the row state machine on column step - 1, and
  //    the device is never idle waiting for the host.  That is exact because
  //    whether a row's next column is forced depends only on the state
  //    after the column before it: the forced tokens of column step - 1
  //    (known once column step - 2 is processed) reach the forward as an
  //    override (a token >= 0 replaces the sampled id; the embedding kernel
  //    writes it back), and a step launched past the end (every row done
  //    after its previous column) is discarded.  Per step the base states of
  //    the group streams, the override and the position reach the device in
  //    one copy from a pinned block (two blocks, alternating, so a copy
  //    still queued is never overwritten), the sampled ids come back in one
  //    copy (two buffers, alternating).
  std::vector<RowState> states(rows);
  // a prompt that ends inside a reasoning trace starts every row of its group
  // there, so the budget counts from the first generated token (engine.go:226-236)
  const bool think = opt.thinking != 0 || opt.thinking_budget > 0;
  if (think)
    for (int r = 0; r < rows; r++)
      states[r].in_thinking = prompts[(int64_t)(r / S) * P + P - 1] == opt.think_start;
  std::vector<u128h> stream(G);
  for (int g = 0; g < G; g++) stream[g] = new_rng_state(seeds[g]);
  // device inputs of a step: base states [2G] u64 | override [rows] i32 | position
  const size_t in_bytes = sizeof(uint64_t) * 2 * G + sizeof(int32_t) * (rows + 1);
  char* din = A<char>(s, "dec_in", in_bytes);
  uint64_t* dbase = reinterpret_cast<uint64_t*>(din);
  int32_t* dovr = reinterpret_cast<int32_t*>(dbase + 2 * G);
  int* dpos = dovr + rows;
  int32_t* dtok = A<int32_t>(s, "dec_tok", rows);
  // pinned staging: two input blocks, then two sampled-id buffers
  const size_t in_pad = (in_bytes + 255) / 256 * 256;
  char* hp = static_cast<char*>(pinned(s, 2 * in_pad + 2 * sizeof(int32_t) * rows));
  int32_t* hsampled[2] = {reinterpret_cast<int32_t*>(hp + 2 * in_pad),
                          reinterpret_cast<int32_t*>(hp + 2 * in_pad) + rows};
  hipEvent_t evs[2] = {next_event(s), next_event(s)};
  std::vector<int32_t> column(rows);
  std::vector<char> done(rows, 0);
  int ndone = 0;
  SamplerArgs sa{};
  sa.logits = logits; sa.ldl = V; sa.rows = rows; sa.V = V; sa.samples_per_group = S;
  sa.base_states = dbase; sa.temperature = temperature; sa.top_k = top_k; sa.out = dtok;
  sa.softcap = 1;  // the decode logits buffer holds lm_head products

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

  // Launches step `step`: its inputs (the override of the column it feeds
  // comes from the rows' forced tokens), forward + sampler, the ids back.
  auto launch = [&](int step) {
    char* hin = hp + (step & 1) * in_pad;
    uint64_t* base = reinterpret_cast<uint64_t*>(hin);
    int32_t* ovr = reinterpret_cast<int32_t*>(base + 2 * G);
    for (int g = 0; g < G; g++) {
      base[2 * g] = (uint64_t)(stream[g] >> 64);
      base[2 * g + 1] = (uint64_t)stream[g];
      stream[g] = pcg_advance_host(stream[g], (u128h)S * (u128h)V);
    }
    for (int r = 0; r < rows; r++) {
      const RowState& rs = states[r];
      ovr[r] = -1;
      if (rs.forced_pos < rs.forced.size()) {
        ovr[r] = rs.forced[rs.forced_pos];
        GN_CHECK(ovr[r] >= 0 && ovr[r] < s->PV, "forced token outside the embedding table");
      }
    }
    const int pos = P + step - 1;  // position of the column fed
    ovr[rows] = pos;
    GN_HIP(hipMemcpyAsync(din, hin, in_bytes, hipMemcpyHostToDevice, st));
    if (use_graph && step >= 2) {
      if (!graph.e) {
        GN_HIP(hipStreamSynchronize(st));  // the capture starts on an idle stream
        GN_HIP(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
        s->capturing = true;
        try {
          decode_step(s, rows, pos, maxSeq, dtok, kc, vc, logits, dpos, dovr);
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
      if (step > 0) decode_step(s, rows, pos, maxSeq, dtok, kc, vc, logits, nullptr, dovr);
      launch_sampler(sa, st);
    }
    GN_HIP(hipMemcpyAsync(hsampled[step & 1], dtok, sizeof(int32_t) * rows,
                          hipMemcpyDeviceToHost, st));
    GN_HIP(hipEventRecord(evs[step & 1], st));
  };
  // The row state machine on column `step` (engine.go:258-314); true when
  // generation ends with it.
  auto process = [&](int step) -> bool {
    GN_HIP(hipEventSynchronize(evs[step & 1]));
    const int32_t* sampled = hsampled[step & 1];
    for (int r = 0; r < rows; r++) {
      RowState& rs = states[r];
      int tok;
      const bool forced = rs.forced_pos < rs.forced.size();
      if (forced) tok = rs.forced[rs.forced_pos++];
      else tok = sampled[r];
      column[r] = tok;
      if (tok == opt.assistant_end || tok == opt.bos) rs.completed = true;
      if (tok == opt.tool_start) {
        rs.in_tool = true;
        rs.tool.clear();
      } else if (tok == opt.tool_end && rs.in_tool) {
        rs.in_tool = false;
        if (!rs.tool.empty()) run_tool(opt, rs);
        rs.tool.clear();
      } else if (rs.in_tool) {
        rs.tool.push_back(tok);
      }
      if (think) {  // thinking-trace tracking and the budget (engine.go:298-313)
        if (tok == opt.think_start) {
          rs.in_thinking = true;
          rs.thinking_tokens = 0;
        } else if (tok == opt.think_end && rs.in_thinking) {
          rs.in_thinking = false;
        } else if (rs.in_thinking) {
          rs.thinking_tokens++;
          if (opt.thinking_budget > 0 && rs.thinking_tokens >= opt.thinking_budget)
            rs.forced.push_back(opt.think_end);
        }
      }
      // GenerateBatchWith's collection (engine.go:349-366): 1 for sampled,
      // 0 for forced tokens
      if (!done[r]) {
        if (tok == opt.assistant_end || tok == opt.bos) {
          done[r] = 1;
          ndone++;
        } else {
          if (masks_out) masks_out[(int64_t)r * W + lens_out[r]] = forced ? 0 : 1;
          rows_out[(int64_t)r * W + lens_out[r]++] = tok;
        }
      }
    }
    // the reference's final forward feeds no sample
    return ndone == rows || step + 1 == N;
  };
  if (N > 0) {
    launch(0);
    bool end = false;
    for (int step = 1; step < N && !end; step++) {
      launch(step);
      end = process(step - 1);
    }
    if (!end) process(N - 1);
  }
  // nothing may still write the pinned staging (a step launched past the end)
  GN_HIP(hipStreamSynchronize(st));
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
    gn_session* s = new gn_session();
    s->device = device;
    try {
      GN_HIP(hipStreamCreateWithFlags(&s->stream, hipStreamNonBlocking));
      s->arena = std::make_unique<DeviceArena>(s->stream);
      build_session(s, *config);
      const char* fp = std::getenv("GN_FUSE_QKV_POST");
      s->fuse_qkv_post = !fp || std::strcmp(fp, "0") != 0;
      // GN_CSA_SELECT=wave / block forces one selection kernel (tests)
      if (const char* cs = std::getenv("GN_CSA_SELECT"))
        s->csa_select_mode = !std::strcmp(cs, "wave") ? 1 : !std::strcmp(cs, "block") ? 2 : 0;
    } catch (...) {  // a rejected config or a failed allocation frees what was made
      if (s->stream) (void)gn_session_destroy(s);
      else delete s;
      throw;
    }
    *out = s;
  });
}

int gn_session_destroy(gn_session* s) {
  return guard([&] {
    if (!s) return;
    (void)hipSetDevice(s->device);
    (void)hipStreamSynchronize(s->stream);
    s->pc_defer = false;
    pc_clear(s);
    s->arena.reset();
    for (auto e : s->event_pool) (void)hipEventDestroy(e);
    if (s->pinned) (void)hipHostFree(s->pinned);
    (void)hipFree(s->params);
    (void)hipFree(s->grads);
    (void)hipFree(s->cosT);
    (void)hipFree(s->sinT);
    if (s->derived) (void)hipFree(s->derived);
    if (s->moe_load) (void)hipFree(s->moe_load);
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
    s->derived_dirty = true;
    pc_clear(s);  // stored prefills belong to the old parameters
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

int gn_session_update_router_bias(gn_session* s, float speed) {
  return guard([&] {
    GN_CHECK(s, "null session");
    if (!s->moe) return;  // Transformer.UpdateRouterBias: no MoE, nothing to do
    GN_HIP(hipSetDevice(s->device));
    for (int l = 0; l < s->L; l++)
      launch_moe_bias_update(s->moe_load + (int64_t)l * s->E, s->layers[l].rbias, s->E, speed,
                             s->stream);
    GN_HIP(hipStreamSynchronize(s->stream));
    s->derived_dirty = true;
    pc_clear(s);  // stored prefills were routed with the old bias
  });
}
int gn_session_moe_loads(const gn_session* s, double* loads, int64_t count) {
  return guard([&] {
    GN_CHECK(s && loads, "null argument");
    GN_CHECK(count == (s->moe ? (int64_t)s->L * s->E : 0), "moe loads: count must be layers x experts");
    if (!s->moe) return;
    GN_HIP(hipSetDevice(s->device));
    GN_HIP(hipMemcpyAsync(loads, s->moe_load, sizeof(double) * count, hipMemcpyDeviceToHost,
                          s->stream));
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
    s->gemm_events.clear(); s->gemm_ev_flops.clear(); s->gemm_ev_wide.clear(); s->event_next = 0;
  });
}

int gn_generate_options_default(gn_generate_options* out) {
  return guard([&] {
    GN_CHECK(out, "null argument");
    *out = default_generate_options();
  });
}

int gn_generate_batch(gn_session* s, const int32_t* prompts, int32_t groups, int32_t prompt_len,
                      int32_t samples, int32_t max_tokens, float temperature, int32_t top_k,
                      const uint64_t* seeds, int32_t* rows_out, int32_t* lengths_out) {
  return gn_generate_batch_with(s, prompts, groups, prompt_len, samples, max_tokens, temperature,
                                top_k, seeds, nullptr, rows_out, lengths_out, nullptr);
}

int gn_generate_batch_with(gn_session* s, const int32_t* prompts, int32_t groups,
                           int32_t prompt_len, int32_t samples, int32_t max_tokens,
                           float temperature, int32_t top_k, const uint64_t* seeds,
                           const gn_generate_options* options, int32_t* rows_out,
                           int32_t* lengths_out, int32_t* masks_out) {
  return guard([&] {
    GN_CHECK(s && prompts && seeds && rows_out && lengths_out, "null argument");
    GN_HIP(hipSetDevice(s->device));
    const gn_generate_options o = options ? *options : default_generate_options();
    generate(s, prompts, groups, prompt_len, samples, max_tokens, temperature, top_k, seeds,
             rows_out, lengths_out, o, masks_out);
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

int gn_distill_step(gn_session* s, gn_session* teacher, const int32_t* inputs,
                    const int32_t* mask, int32_t batch, int32_t seq_len, float temperature,
                    int32_t grad_accum_steps, float* loss_out) {
  return guard([&] {
    GN_CHECK(s && teacher && inputs && loss_out, "null argument");
    GN_CHECK(s != teacher, "distillation: the teacher must be another session");
    GN_CHECK(s->device == teacher->device, "distillation: teacher and student on one device");
    GN_CHECK(s->V == teacher->V, "distillation: teacher and student vocabularies differ");
    GN_CHECK(batch > 0 && seq_len > 1, "distillation: need batch > 0 and seq_len > 1");
    GN_CHECK(seq_len <= teacher->S, "model: sequence longer than the teacher's rotary cache");
    GN_HIP(hipSetDevice(s->device));
    const int B = batch, T = seq_len;
    const int64_t NT = (int64_t)B * T;
    // the valid positions fix the scale of every row (distill.go:33-36)
    int64_t valid = 0;
    std::vector<int32_t> slot((size_t)NT);
    for (int64_t i = 0; i < NT; i++) {
      const bool on = !mask || mask[i] != 0;
      slot[i] = on ? 0 : -1;
      valid += on;
    }
    const int64_t vt = valid == 0 ? 1 : valid;
    GN_CHECK(grad_accum_steps >= 1, "distillation: gradient-accumulation steps must be >= 1");
    // the balance loss's gradient would need the 1/steps scale of
    // SetAuxiliaryGradientScale (distill.go:21), which this step does not apply
    GN_CHECK(grad_accum_steps == 1 || !(s->moe && s->bw > 0.f),
             "distillation: a MoE student with a balance loss takes one accumulation step");
    DistillCtx dc;
    dc.teacher = teacher;
    dc.tau = temperature <= 0.f ? 1.0 : (double)temperature;  // distillationTemperature
    dc.scale = 1.0f / ((float)vt * (float)grad_accum_steps);
    const std::vector<float> zero_adv((size_t)B, 0.f);
    const int mb = pg_micro_batch(s, B, T);
    double sum = 0;
    s->bal_batch = B;
    try {
      for (int b0 = 0; b0 < B; b0 += mb) {
        const int nb = std::min(mb, B - b0);
        // teacher.Forward of these sequences up to its final norm, on its stream
        SeqBuffers tb;
        tb.B = nb; tb.T = T; tb.N = (int64_t)nb * T;
        tb.ids = upload_ids(teacher, "ids", inputs + (int64_t)b0 * T, tb.N, teacher->V);
        seq_forward(teacher, tb, SEQ_FORWARD, nullptr, nullptr);
        GN_HIP(hipStreamSynchronize(teacher->stream));
        dc.tfn = tb.fn;
        double l = 0;
        pg_step_chunk(s, inputs + (int64_t)b0 * T, slot.data() + (int64_t)b0 * T, nb, T,
                      zero_adv.data() + b0, 1.f, &l, nullptr, &dc);
        sum += l;
      }
    } catch (...) {
      s->bal_batch = 0;
      throw;
    }
    s->bal_batch = 0;
    *loss_out = (float)(sum / (double)vt);
  });
}

int gn_rl_step(gn_session* s, const int32_t* prompts, int32_t G, int32_t P, int32_t S, int32_t N,
               float temperature, int32_t top_k, const uint64_t* seeds, const float* rewards,
               int32_t* rows_out, int32_t* lens_out, float* adv_out, int32_t* max_len_out,
               float* loss_out) {
  return gn_rl_step_with(s, prompts, G, P, S, N, temperature, top_k, seeds, nullptr, rewards,
                         rows_out, lens_out, adv_out, max_len_out, loss_out);
}

int gn_rl_step_with(gn_session* s, const int32_t* prompts, int32_t G, int32_t P, int32_t S,
                    int32_t N, float temperature, int32_t top_k, const uint64_t* seeds,
                    const gn_generate_options* options, const float* rewards, int32_t* rows_out,
                    int32_t* lens_out, float* adv_out, int32_t* max_len_out, float* loss_out) {
  return guard([&] {
    GN_CHECK(s && prompts && seeds && rewards && rows_out && lens_out && adv_out && max_len_out,
             "null argument");
    GN_HIP(hipSetDevice(s->device));
    const gn_generate_options o = options ? *options : default_generate_options();
    generate(s, prompts, G, P, S, N, temperature, top_k, seeds, rows_out, lens_out, o, nullptr);
    const int32_t pad = o.assistant_end;
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
        int32_t in = t < lens_out[b] ? rows_out[(int64_t)b * W + t] : pad;
        int32_t tg = t + 1 < lens_out[b] ? rows_out[(int64_t)b * W + t + 1] : pad;
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
    if (temperature > 0) advance_rng_state(rng_state, (uint64_t)rows * (uint64_t)vocab);
  });
}

int gn_softcap_order_check(uint64_t* violations) {
  return guard([&] {
    GN_CHECK(violations, "null argument");
    *violations = count_softcap_order_violations();
  });
}

int gn_session_set_timing(gn_session* s, int enabled) {
  return guard([&] {
    GN_CHECK(s, "null session");
    s->timing = enabled != 0;
    s->gemm_events.clear(); s->gemm_ev_flops.clear(); s->gemm_ev_wide.clear();
    s->attn_events.clear(); s->attn_ev_bytes.clear(); s->attn_ev_launches.clear();
    s->loss_events.clear(); s->loss_ev_bytes.clear();
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
int gn_session_aux_loss(const gn_session* s, double* out) {
  return guard([&] {
    GN_CHECK(s && out, "null argument");
    *out = s->aux_loss;
  });
}
int gn_session_synchronize(gn_session* s) {
  return guard([&] {
    GN_CHECK(s, "null session");
    GN_HIP(hipSetDevice(s->device));
    GN_HIP(hipStreamSynchronize(s->stream));
  });
}

// ---- prefix cache (inference/cache.go, inference/prefix.go) -----------------
int gn_session_set_prefix_cache(gn_session* s, const gn_prefix_cache_options* o) {
  return guard([&] {
    GN_CHECK(s, "null session");
    GN_HIP(hipSetDevice(s->device));
    if (!o) {
      pc_clear(s);
      s->pc_on = false;
      return;
    }
    if (s->split > 0)  // as the reference (inference/engine.go:128-140, 175-182)
      throw Error(GN_ERR_UNSUPPORTED,
                  "prefix cache: encoder-decoder (CED) models are not cached");
    GN_CHECK(o->max_entries >= 0 && o->max_bytes >= 0 && o->max_prefix >= 0 &&
                 o->ttl_seconds >= 0.0,
             "prefix cache: negative limit");
    s->pc_on = true;
    s->pc_max_entries = o->max_entries;
    s->pc_max_bytes = o->max_bytes;
    s->pc_max_prefix = o->max_prefix;
    s->pc_ttl = o->ttl_seconds;
    // NewCacheManager (cache.go:64-77): the directory is created if missing;
    // if that fails the cache keeps to device memory
    s->pc_dir.clear();
    if (o->disk_dir && o->disk_dir[0]) {
      std::error_code ec;
      std::filesystem::create_directories(o->disk_dir, ec);
      if (!ec && std::filesystem::is_directory(o->disk_dir, ec)) s->pc_dir = o->disk_dir;
    }
    pc_evict(s);
  });
}
int gn_session_prefix_cache_invalidate(gn_session* s) {
  return guard([&] {
    GN_CHECK(s, "null session");
    GN_HIP(hipSetDevice(s->device));
    pc_clear(s);
  });
}
int gn_session_prefix_cache_len(gn_session* s, int32_t* entries, int64_t* bytes) {
  return guard([&] {
    GN_CHECK(s && entries, "null argument");
    pc_expire(s);
    *entries = (int32_t)s->pc_entries.size();
    if (bytes) *bytes = s->pc_bytes;
  });
}
int gn_session_prefix_cache_hits(const gn_session* s, int32_t* hits, int32_t groups) {
  return guard([&] {
    GN_CHECK(s && hits, "null argument");
    GN_CHECK(groups == (int32_t)s->pc_hits.size(), "prefix cache: groups differ from the last call");
    std::copy(s->pc_hits.begin(), s->pc_hits.end(), hits);
  });
}

// ---- optimizer ---------------------------------------------------------------
struct gn_optimizer {
  gn_session* s = nullptr;
  std::vector<OptTensor> ts;
  float* state = nullptr;  // device, every entry's region in table order
  int64_t state_floats = 0;
};

int gn_optimizer_create(gn_session* s, const gn_opt_param* table, int32_t count,
                        gn_optimizer** out) {
  return guard([&] {
    GN_CHECK(s && table && out && count > 0, "optimizer: null argument or empty table");
    *out = nullptr;
    GN_HIP(hipSetDevice(s->device));
    auto o = std::make_unique<gn_optimizer>();
    o->s = s;
    for (int32_t i = 0; i < count; i++) {
      const gn_opt_param& h = table[i];
      GN_CHECK(h.kind == GN_OPT_ADAMW || h.kind == GN_OPT_MUON || h.kind == GN_OPT_SINKHORN,
               "optimizer: unknown parameter kind");
      GN_CHECK(h.rows > 0 && h.cols > 0 && h.offset >= 0, "optimizer: bad tensor shape");
      GN_CHECK(h.kind != GN_OPT_MUON || (h.ns_steps >= 0 && h.ns_steps <= 5),
               "optimizer: Muon takes at most 5 Polar Express steps");
      GN_CHECK(h.kind != GN_OPT_SINKHORN || h.sinkhorn_steps >= 1,
               "optimizer: Sinkhorn needs at least one normalization step");
      const int64_t n = (int64_t)h.rows * h.cols;
      const ParamEntry* owner = nullptr;
      for (const ParamEntry& e : s->table)
        if (h.offset >= e.offset && h.offset + n <= e.offset + e.rows * e.cols) owner = &e;
      GN_CHECK(owner != nullptr, "optimizer: entry is not inside one parameter tensor");
      OptTensor t;
      t.p = owner->dev + (h.offset - owner->offset);
      t.g = owner->grad + (h.offset - owner->offset);
      t.rows = h.rows;
      t.cols = h.cols;
      t.h = h;
      o->ts.push_back(t);
      o->state_floats += opt_state_floats(h);
    }
    GN_HIP(hipMalloc(&o->state, sizeof(float) * o->state_floats));
    GN_HIP(hipMemsetAsync(o->state, 0, sizeof(float) * o->state_floats, s->stream));
    float* st = o->state;
    for (OptTensor& t : o->ts) {
      t.st = st;
      st += opt_state_floats(t.h);
    }
    GN_HIP(hipStreamSynchronize(s->stream));
    *out = o.release();
  });
}
int gn_optimizer_step(gn_optimizer* o) {
  return guard([&] {
    GN_CHECK(o && o->s, "null optimizer");
    gn_session* s = o->s;
    GN_HIP(hipSetDevice(s->device));
    optimizer_step(o->ts, s->stream, s->arena.get());
    GN_HIP(hipStreamSynchronize(s->stream));
    s->derived_dirty = true;  // absorbed decode weights follow the parameters
    pc_clear(s);              // and stored prefills are stale
  });
}
int gn_optimizer_set_hyper(gn_optimizer* o, const float* lr, const float* momentum,
                           const float* weight_decay, int32_t count) {
  return guard([&] {
    GN_CHECK(o, "null optimizer");
    GN_CHECK(count == (int32_t)o->ts.size(), "optimizer: one value per table entry");
    for (int32_t i = 0; i < count; i++) {
      gn_opt_param& h = o->ts[i].h;
      if (lr) h.lr = lr[i];
      if (momentum) h.momentum = momentum[i];
      if (weight_decay) h.weight_decay = weight_decay[i];
    }
  });
}
int gn_optimizer_state_size(const gn_optimizer* o, int64_t* count) {
  return guard([&] {
    GN_CHECK(o && count, "null argument");
    *count = o->state_floats;
  });
}
int gn_optimizer_get_state(const gn_optimizer* o, float* state, int64_t count) {
  return guard([&] {
    GN_CHECK(o && state, "null argument");
    GN_CHECK(count == o->state_floats, "optimizer state length mismatch");
    GN_HIP(hipSetDevice(o->s->device));
    GN_HIP(hipMemcpyAsync(state, o->state, sizeof(float) * count, hipMemcpyDeviceToHost,
                          o->s->stream));
    GN_HIP(hipStreamSynchronize(o->s->stream));
  });
}
int gn_optimizer_destroy(gn_optimizer* o) {
  return guard([&] {
    if (!o) return;
    if (o->state) {
      GN_HIP(hipSetDevice(o->s->device));
      GN_HIP(hipStreamSynchronize(o->s->stream));
      GN_HIP(hipFree(o->state));
    }
    delete o;
  });
}

}  // extern "C"
