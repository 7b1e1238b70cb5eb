// Copied into gonano's tree as kernels/hip; built with the rest of the
// package (backend.go carries the #cgo flags and the call helper).

package hip

/*
#include <stdlib.h>
#include "gonano_hip.h"
*/
import "C"

import (
	"unsafe"

	"github.com/cookiengineer/gonano/inference"
	"github.com/cookiengineer/gonano/model"
)

// Session keeps a model's parameters, gradients, KV caches and activations
// in device memory and runs the RL step there (include/gonano_hip.h,
// gn_session_*).
type Session struct{ h *C.gn_session; total int }

func NewSession(cfg model.Config, device int) *Session {
	var c C.gn_config
	c.sequence_len = C.int32_t(cfg.SequenceLen)
	c.vocab_size = C.int32_t(cfg.VocabSize)
	c.n_layer = C.int32_t(cfg.NumLayer)
	c.n_head = C.int32_t(cfg.NumHead)
	c.n_kv_head = C.int32_t(cfg.NumKVHead)
	c.n_embd = C.int32_t(cfg.EmbedDim)
	c.rotary_dims = C.int32_t(cfg.RotaryDimension())
	for i, b := range []byte(cfg.WindowPattern) {
		c.window_pattern[i] = C.char(b)
	}
	if cfg.MLAEnabled() { // latent preset: absorbed MLA (model/config.go:250-280)
		c.mla_latent = C.int32_t(cfg.MLARank())
		c.mla_rope_dims = C.int32_t(cfg.MLARotaryDimension())
	}
	if cfg.MoEEnabled() { // DeepSeekMoE, resolved values (model/config.go:138-227)
		c.n_experts = C.int32_t(cfg.NumExperts)
		c.experts_per_token = C.int32_t(cfg.MoEActiveExperts())
		c.expert_hidden = C.int32_t(cfg.MoEExpertHidden())
		c.shared_hidden = C.int32_t(cfg.MoESharedHidden())
		c.moe_clamp = C.float(cfg.MoEEffectiveClamp())
		c.moe_scale = C.float(cfg.MoEEffectiveScale())
		c.balance_weight = C.float(cfg.MoEBalanceLossWeight())
	}
	if cfg.Compression() > 1 { // flash preset, resolved values (model/config.go:282-420)
		// Config.indexerDefaults (model/config.go:394-404) is unexported; the
		// binding applies the same defaults, as engine.go's indexerKeyWidth does
		dim, heads := cfg.IndexerDim, cfg.IndexerHeads
		if dim <= 0 {
			dim = 64
		}
		if heads <= 0 {
			heads = 1
		}
		c.compression_ratio = C.int32_t(cfg.Compression())
		c.swa_window = C.int32_t(cfg.SWAWindowSize())
		c.sparse_topk = C.int32_t(cfg.SparseTopK)
		c.indexer_dim = C.int32_t(dim)
		c.indexer_heads = C.int32_t(heads)
		c.indexer_pool = C.int32_t(cfg.IndexerPool)
		c.indexer_candidates = C.int32_t(cfg.IndexerCandidateBudget())
		c.indexer_weight = C.float(cfg.IndexerWeight())
		for i, b := range []byte(cfg.ReusePattern) {
			c.reuse_pattern[i] = C.char(b)
		}
		if cfg.CEDEnabled() {
			c.ced = 1
		}
	}
	s := &Session{}
	call(func() C.int { return C.gn_session_create(&c, C.int(device), &s.h) })
	var t C.int64_t
	call(func() C.int { return C.gn_session_param_total(s.h, &t) })
	s.total = int(t)
	return s
}

// LoadParameters copies the tensors of Transformer.Parameters(), which come
// in ParameterNames order (model/params.go:77-113), into the session;
// gradients come back in the same order.
func (s *Session) LoadParameters(m *model.Transformer) {
	flat := make([]float32, 0, s.total)
	for _, p := range m.Parameters() {
		flat = append(flat, p.Data...)
	}
	call(func() C.int { return C.gn_session_set_params(s.h, f32(flat), C.int64_t(len(flat))) })
}

// RLStep = chat_rl's step body (main.go:101-183) + trainer.PolicyGradientStep
// (trainer/rl.go:14-60) without the optimizer: rollouts, advantages, padding,
// recompute, PG loss and gradients (accumulated on the device).
func (s *Session) RLStep(prompts [][]int32, samples, maxTokens int, temperature float32,
	topK int, seeds []uint64, rewards []float32) (loss float32, rows [][]int32, adv []float32) {
	G, P := len(prompts), len(prompts[0])
	flat := make([]int32, 0, G*P)
	for _, p := range prompts {
		flat = append(flat, p...)
	}
	W := P + maxTokens
	out := make([]int32, G*samples*W)
	lens := make([]int32, G*samples)
	adv = make([]float32, G*samples)
	var maxLen C.int32_t
	var l C.float
	call(func() C.int { return C.gn_rl_step(s.h, i32(flat), C.int32_t(G), C.int32_t(P), C.int32_t(samples),
		C.int32_t(maxTokens), C.float(temperature), C.int32_t(topK),
		(*C.uint64_t)(unsafe.Pointer(&seeds[0])), f32(rewards), i32(out), i32(lens), f32(adv),
		&maxLen, &l) })
	rows = make([][]int32, G*samples)
	for b := range rows {
		rows[b] = out[b*W : b*W+int(lens[b])]
	}
	return float32(l), rows, adv
}

func (s *Session) Gradients(dst []float32) { call(func() C.int { return C.gn_session_get_grads(s.h, f32(dst), C.int64_t(len(dst))) }) }

// AuxiliaryLoss = Transformer.AuxiliaryLoss (model/transformer.go:108-116):
// the MoE balance loss of the last step, for logging; its gradient is
// already in Gradients.
func (s *Session) AuxiliaryLoss() float64 {
	var v C.double
	call(func() C.int { return C.gn_session_aux_loss(s.h, &v) })
	return float64(v)
}
func (s *Session) ZeroGrad()               { call(func() C.int { return C.gn_session_zero_grads(s.h) }) }
func (s *Session) Close()                  { C.gn_session_destroy(s.h) }

// UpdateRouterBias mirrors Transformer.UpdateRouterBias.
func (s *Session) UpdateRouterBias(cfg model.Config) {
	call(func() C.int { return C.gn_session_update_router_bias(s.h, C.float(cfg.MoERouterBiasUpdate())) })
}

func (s *Session) DistillStep(teacher *Session, inputs, mask []int32, batch, seqLen int,
	temperature float32, gradAccumSteps int) float32 {
	var l C.float
	var m *C.int32_t
	if mask != nil {
		m = i32(mask)
	}
	call(func() C.int { return C.gn_distill_step(s.h, teacher.h, i32(inputs), m, C.int32_t(batch),
		C.int32_t(seqLen), C.float(temperature), C.int32_t(gradAccumSteps), &l) })
	return float32(l)
}

// Engine.Cache = inference.NewCacheManager(opts), or, with maxEntries 1 and
// maxPrefix, Engine.Prefix = inference.NewPrefixCache(maxPrefix)
func (s *Session) SetPrefixCache(opts inference.CacheOptions, maxPrefix int) {
	o := C.gn_prefix_cache_options{
		max_entries: C.int32_t(opts.MaxEntries),
		max_prefix:  C.int32_t(maxPrefix),
		max_bytes:   C.int64_t(opts.MaxBytes),
		ttl_seconds: C.double(opts.TTL.Seconds()),
	}
	if opts.DiskDir != "" {
		dir := C.CString(opts.DiskDir)
		defer C.free(unsafe.Pointer(dir))
		o.disk_dir = dir
	}
	call(func() C.int { return C.gn_session_set_prefix_cache(s.h, &o) })
}
func (s *Session) DisablePrefixCache()  { call(func() C.int { return C.gn_session_set_prefix_cache(s.h, nil) }) }
func (s *Session) InvalidatePrefixCache() { call(func() C.int { return C.gn_session_prefix_cache_invalidate(s.h) }) }
func (s *Session) PrefixCacheLen() int {
	var n C.int32_t
	call(func() C.int { return C.gn_session_prefix_cache_len(s.h, &n, nil) })
	return int(n)
}
