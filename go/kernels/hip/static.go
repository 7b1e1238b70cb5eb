// Copied into gonano's tree as kernels/hip; built with the rest of the
// package (backend.go carries the #cgo flags and the call helper).

package hip

/*
#include <stdlib.h>
#include "gonano_hip.h"
*/
import "C"

import (
	"runtime"
	"sync"
)

// staticSampler serializes gn_sample_next_token_static: its device scratch
// array is shared by every call on a GPU (the library also holds a
// per-device lock through each call).
var staticSampler sync.Mutex

// SampleNextTokenStatic is SampleNextToken without device allocation; calls
// on one GPU must not overlap.
func SampleNextTokenStatic(logits []float32, rows, vocab int, state *[2]uint64,
	temperature float32, topK int) []int32 {
	out := make([]int32, rows)
	staticSampler.Lock()
	defer staticSampler.Unlock()
	runtime.LockOSThread()
	defer runtime.UnlockOSThread()
	if st := C.gn_sample_next_token_static((*C.float)(&logits[0]), C.int64_t(rows),
		C.int64_t(vocab), (*C.uint64_t)(&state[0]), C.float(temperature), C.int64_t(topK),
		(*C.int32_t)(&out[0])); st != 0 {
		panic(C.GoString(C.gn_last_error()))
	}
	return out
}
