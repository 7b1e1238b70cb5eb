// Package hip is a kernels.Backend backed by hand-written HIP kernels for
// AMD MI355X (gfx950), through libgnhip.so.
package hip

/*
#cgo CFLAGS: -I${SRCDIR}/../../third_party/gonano_hip/include
#cgo LDFLAGS: -L${SRCDIR}/../../third_party/gonano_hip/lib -lgnhip -Wl,-rpath,${SRCDIR}/../../third_party/gonano_hip/lib
#include <stdlib.h>
#include "gonano_hip.h"
*/
import "C"

import (
	"fmt"
	"runtime"
	"unsafe"

	"github.com/cookiengineer/gonano/kernels"
)

type Backend struct{}

var _ kernels.Backend = (*Backend)(nil)

// New returns the HIP backend; it panics when no device is visible.
func New() *Backend {
	if C.gn_device_count() < 1 {
		panic("kernels/hip: no HIP device")
	}
	return &Backend{}
}

// call runs one C-ABI call and reads its error message on the same OS
// thread: gn_last_error (like gn_set_device) is per thread, and a goroutine
// may move to another thread between two cgo calls unless it is locked.
func call(f func() C.int) {
	runtime.LockOSThread()
	defer runtime.UnlockOSThread()
	if status := f(); status != 0 {
		panic(fmt.Sprintf("kernels/hip: %s", C.GoString(C.gn_last_error())))
	}
}

func f32(s []float32) *C.float {
	if len(s) == 0 {
		return nil
	}
	return (*C.float)(unsafe.Pointer(&s[0]))
}
func i32(s []int32) *C.int32_t {
	if len(s) == 0 {
		return nil
	}
	return (*C.int32_t)(unsafe.Pointer(&s[0]))
}
func n(s []float32) C.int64_t { return C.int64_t(len(s)) }

// Elementwise (kernels/backend.go:21-67)
func (Backend) Add(d, l, r []float32)      { call(func() C.int { return C.gn_add(f32(d), f32(l), f32(r), n(d)) }) }
func (Backend) Subtract(d, l, r []float32) { call(func() C.int { return C.gn_subtract(f32(d), f32(l), f32(r), n(d)) }) }
func (Backend) Multiply(d, l, r []float32) { call(func() C.int { return C.gn_multiply(f32(d), f32(l), f32(r), n(d)) }) }
func (Backend) Divide(d, l, r []float32)   { call(func() C.int { return C.gn_divide(f32(d), f32(l), f32(r), n(d)) }) }
func (Backend) Scale(d, s []float32, f float32) {
	call(func() C.int { return C.gn_scale(f32(d), f32(s), C.float(f), n(d)) })
}
func (Backend) AddScaled(d, b, s []float32, f float32) {
	call(func() C.int { return C.gn_add_scaled(f32(d), f32(b), f32(s), C.float(f), n(d)) })
}
func (Backend) Negate(d, s []float32)      { call(func() C.int { return C.gn_negate(f32(d), f32(s), n(d)) }) }
func (Backend) Abs(d, s []float32)         { call(func() C.int { return C.gn_abs(f32(d), f32(s), n(d)) }) }
func (Backend) Square(d, s []float32)      { call(func() C.int { return C.gn_square(f32(d), f32(s), n(d)) }) }
func (Backend) ReluSquared(d, s []float32) { call(func() C.int { return C.gn_relu_squared(f32(d), f32(s), n(d)) }) }
func (Backend) SwiGLU(d, g, u []float32, clamp float32) {
	call(func() C.int { return C.gn_swiglu(f32(d), f32(g), f32(u), C.float(clamp), n(d)) })
}
func (Backend) SwiGLUBackward(gg, ug, g, u, og []float32, clamp float32) {
	call(func() C.int { return C.gn_swiglu_backward(f32(gg), f32(ug), f32(g), f32(u), f32(og), C.float(clamp), n(g)) })
}
func (Backend) Exp(d, s []float32)     { call(func() C.int { return C.gn_exp(f32(d), f32(s), n(d)) }) }
func (Backend) Sigmoid(d, s []float32) { call(func() C.int { return C.gn_sigmoid(f32(d), f32(s), n(d)) }) }
func (Backend) Tanh(d, s []float32)    { call(func() C.int { return C.gn_tanh(f32(d), f32(s), n(d)) }) }
func (Backend) Rsqrt(d, s []float32)   { call(func() C.int { return C.gn_rsqrt(f32(d), f32(s), n(d)) }) }

// Reductions (:70-78)
func (Backend) Sum(v []float32) float32 {
	var r C.float
	call(func() C.int { return C.gn_sum(f32(v), n(v), &r) })
	return float32(r)
}
func (Backend) Max(v []float32) float32 {
	var r C.float
	call(func() C.int { return C.gn_max(f32(v), n(v), &r) })
	return float32(r)
}
func (Backend) ArgMax(v []float32) int {
	var r C.int64_t
	call(func() C.int { return C.gn_argmax(f32(v), n(v), &r) })
	return int(r)
}

// LinearAlgebra (:82-93)
func (Backend) MatMul(d, l, r []float32, rows, cols, inner int) {
	call(func() C.int { return C.gn_matmul(f32(d), f32(l), f32(r), C.int64_t(rows), C.int64_t(cols), C.int64_t(inner)) })
}
func (Backend) MatMulTransposed(d, l, r []float32, rows, cols, inner int) {
	call(func() C.int { return C.gn_matmul_transposed(f32(d), f32(l), f32(r), C.int64_t(rows), C.int64_t(cols), C.int64_t(inner)) })
}
func (Backend) DotProduct(l, r []float32) float32 {
	var out C.float
	call(func() C.int { return C.gn_dot_product(f32(l), n(l), f32(r), n(r), &out) })
	return float32(out)
}

// Indexer (:103-115)
func (Backend) IndexerScores(d, q, k, w []float32, rows, blocks, heads, dim int) {
	call(func() C.int { return C.gn_indexer_scores(f32(d), f32(q), f32(k), f32(w), C.int64_t(rows), C.int64_t(blocks),
		C.int64_t(heads), C.int64_t(dim)) })
}
func (Backend) IndexerBlockMax(d, s []float32, rows, blocks, group int) {
	call(func() C.int { return C.gn_indexer_block_max(f32(d), f32(s), C.int64_t(rows), C.int64_t(blocks), C.int64_t(group)) })
}

// MoE (:119-140)
func (Backend) TopKIndices(d []int32, s []float32, rows, count, k int) {
	call(func() C.int { return C.gn_topk_indices(i32(d), f32(s), C.int64_t(rows), C.int64_t(count), C.int64_t(k)) })
}
func (Backend) MoEGateTopK(logits, bias, probs []float32, sel []int32, w []float32, rows, experts, k int) {
	call(func() C.int { return C.gn_moe_gate_topk(f32(logits), f32(bias), f32(probs), i32(sel), f32(w), C.int64_t(rows),
		C.int64_t(experts), C.int64_t(k)) })
}
func (Backend) GroupedMatMulTransposed(d, in, w []float32, counts []int32, experts, cols, inner int) {
	call(func() C.int { return C.gn_grouped_matmul_transposed(f32(d), f32(in), f32(w), i32(counts), C.int64_t(experts),
		C.int64_t(cols), C.int64_t(inner)) })
}

// Rows (:145-153)
func (Backend) SoftmaxLastDim(d, s []float32, rows, cols int) {
	call(func() C.int { return C.gn_softmax_last_dim(f32(d), f32(s), C.int64_t(rows), C.int64_t(cols)) })
}
func (Backend) RMSNormLastDim(d, s []float32, rows, cols int, eps float32) {
	call(func() C.int { return C.gn_rmsnorm_last_dim(f32(d), f32(s), C.int64_t(rows), C.int64_t(cols), C.float(eps)) })
}

// Attention (:267-283)
func (Backend) AttentionForward(p kernels.AttentionForwardParameters, r kernels.AttentionForwardResult) {
	call(func() C.int { return C.gn_attention_forward(f32(p.Query), f32(p.Key), f32(p.Value), i32(p.SegmentIDs),
		C.int64_t(len(p.SegmentIDs)), C.int64_t(p.QueryLength), C.int64_t(p.KeyLength),
		C.int64_t(p.HeadDim), C.int64_t(p.PositionOffset), C.int64_t(p.Window),
		f32(r.Output), f32(r.LogSumExp)) })
}
func (Backend) AttentionBackward(p kernels.AttentionBackwardParameters, r kernels.AttentionBackwardResult) {
	call(func() C.int { return C.gn_attention_backward(f32(p.Query), f32(p.Key), f32(p.Value), f32(p.Output),
		f32(p.OutputGradient), f32(p.LogSumExp), f32(p.RowCorrection), i32(p.SegmentIDs),
		C.int64_t(len(p.SegmentIDs)), C.int64_t(p.QueryLength), C.int64_t(p.KeyLength),
		C.int64_t(p.HeadDim), C.int64_t(p.PositionOffset), C.int64_t(p.Window),
		f32(r.QueryGradient), f32(r.KeyGradient), f32(r.ValueGradient)) })
}
func (Backend) AttentionForwardSplit(p kernels.AttentionSplitParameters, r kernels.AttentionSplitResult) {
	call(func() C.int { return C.gn_attention_forward_split(f32(p.Query), f32(p.Key), f32(p.Value), i32(p.SegmentIDs),
		C.int64_t(len(p.SegmentIDs)), C.int64_t(p.QueryLength), C.int64_t(p.KeyLength),
		C.int64_t(p.HeadDim), C.int64_t(p.PositionOffset), C.int64_t(p.Window),
		C.int64_t(p.KeyStart), C.int64_t(p.KeyEnd), f32(r.Accumulator), f32(r.Maximum), f32(r.Sum)) })
}

// AttentionCombine passes three arrays of pointers to Go memory: they live in
// C memory and the slices they point at are pinned for the call (Go >= 1.21).
func (Backend) AttentionCombine(p kernels.AttentionCombineParameters, r kernels.AttentionForwardResult) {
	parts := len(p.Partials)
	size := C.size_t(parts) * C.size_t(unsafe.Sizeof(uintptr(0)))
	acc := (*[1 << 20]*C.float)(C.malloc(size))[:parts:parts]
	mx := (*[1 << 20]*C.float)(C.malloc(size))[:parts:parts]
	sm := (*[1 << 20]*C.float)(C.malloc(size))[:parts:parts]
	defer C.free(unsafe.Pointer(&acc[0]))
	defer C.free(unsafe.Pointer(&mx[0]))
	defer C.free(unsafe.Pointer(&sm[0]))
	var pin runtime.Pinner
	defer pin.Unpin()
	for i, part := range p.Partials {
		pin.Pin(&part.Accumulator[0])
		pin.Pin(&part.Maximum[0])
		pin.Pin(&part.Sum[0])
		acc[i], mx[i], sm[i] = f32(part.Accumulator), f32(part.Maximum), f32(part.Sum)
	}
	call(func() C.int { return C.gn_attention_combine(&acc[0], &mx[0], &sm[0], C.int64_t(parts),
		C.int64_t(p.QueryLength), C.int64_t(p.HeadDim), f32(r.Output), f32(r.LogSumExp)) })
}
