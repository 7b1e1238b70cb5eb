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

	"github.com/cookiengineer/gonano/model"
	"github.com/cookiengineer/gonano/optimizer"
	"github.com/cookiengineer/gonano/tensors"
)

type DeviceOptimizer struct {
	h *C.gn_optimizer
	n int // table entries
}

// NewDeviceOptimizer mirrors optimizer.NewMuonAdamW(groups)
// (optimizer/optimizer.go:81-110) for parameters living in s.
func NewDeviceOptimizer(s *Session, m *model.Transformer, groups []optimizer.ParamGroup) *DeviceOptimizer {
	// flat offset of every parameter's backing array, in ParameterNames order
	base := map[*float32]int64{}
	var off int64
	for _, p := range m.Parameters() {
		base[&p.Data[0]] = off
		off += int64(len(p.Data))
	}
	offsetOf := func(t *tensors.Tensor) int64 { // views point inside a parent
		for _, p := range m.Parameters() {
			start := uintptr(unsafe.Pointer(&p.Data[0]))
			at := uintptr(unsafe.Pointer(&t.Data[0]))
			if at >= start && at < start+uintptr(4*len(p.Data)) {
				return base[&p.Data[0]] + int64((at-start)/4)
			}
		}
		panic("optimizer tensor outside the model's parameters")
	}
	var table []C.gn_opt_param
	for _, g := range groups {
		for _, t := range g.Params {
			e := C.gn_opt_param{offset: C.int64_t(offsetOf(t)), kind: C.int32_t(g.Kind),
				lr: C.float(g.LR), beta1: C.float(g.Beta1), beta2: C.float(g.Beta2),
				eps: C.float(g.Eps), weight_decay: C.float(g.WeightDecay),
				momentum: C.float(g.Momentum), ns_steps: C.int32_t(g.NSSteps),
				muon_beta2: C.float(g.MuonBeta2), gamma: C.float(g.Gamma),
				sinkhorn_steps: C.int32_t(g.SinkhornSteps), tau: C.float(g.SinkhornTau),
				sinkhorn_eps: C.float(g.SinkhornEps)}
			e.rows, e.cols = 1, C.int32_t(t.Numel()) // AdamW: any shape, elementwise
			if len(t.Shape) == 2 {
				e.rows, e.cols = C.int32_t(t.Shape[0]), C.int32_t(t.Shape[1])
			}
			table = append(table, e)
		}
	}
	o := &DeviceOptimizer{n: len(table)}
	call(func() C.int { return C.gn_optimizer_create(s.h, &table[0], C.int32_t(len(table)), &o.h) })
	return o
}
func (o *DeviceOptimizer) Step()  { call(func() C.int { return C.gn_optimizer_step(o.h) }) } // MuonAdamW.Step
func (o *DeviceOptimizer) Close() { C.gn_optimizer_destroy(o.h) }      // before the session

// SetSchedules: one value per table entry, in table order (the entry's
// group's LR / Momentum / WeightDecay); nil leaves a field unchanged.
func (o *DeviceOptimizer) SetSchedules(lr, momentum, weightDecay []float32) {
	p := func(v []float32) *C.float {
		if v == nil {
			return nil
		}
		return (*C.float)(&v[0])
	}
	call(func() C.int { return C.gn_optimizer_set_hyper(o.h, p(lr), p(momentum), p(weightDecay), C.int32_t(o.n)) })
}
