// Copied into gonano's tree as kernels/hip.  This file exports
// gonanoHipTool to C, so its preamble holds declarations only.

package hip

/*
#include <stdint.h>
#include "gonano_hip.h"
int32_t gonanoHipTool(void* user, int32_t* call, int32_t n, int32_t* out, int32_t capacity);
*/
import "C"

import (
	"runtime/cgo"
	"unsafe"

	"github.com/cookiengineer/gonano/inference"
)

// gonanoHipTool is the gn_tool_fn the library calls for a row that closed a
// tool call: the engine's tool registry runs the decoded call
// (inference/engine.go:282-296) and the result goes back as token ids.
//export gonanoHipTool
func gonanoHipTool(user unsafe.Pointer, call *C.int32_t, n C.int32_t, out *C.int32_t,
	capacity C.int32_t) C.int32_t {
	e := cgo.Handle(uintptr(user)).Value().(*inference.Engine)
	ids := make([]int, int(n))
	for i, v := range unsafe.Slice(call, int(n)) {
		ids[i] = int(v)
	}
	result, ok := e.Tools.Execute(e.Tokenizer.Decode(ids))
	if !ok {
		return -1
	}
	enc := e.Tokenizer.Encode(result)
	if len(enc) > int(capacity) {
		return capacity + 1 // rejected by the library as too long
	}
	dst := unsafe.Slice(out, int(capacity))
	for i, v := range enc {
		dst[i] = C.int32_t(v)
	}
	return C.int32_t(len(enc))
}

// Options builds gn_generate_options from an Engine (its tokenizer and tools)
// and GenerateOptions (inference/engine.go:25-34); free the handle after use.
func Options(e *inference.Engine, o inference.GenerateOptions) (C.gn_generate_options, cgo.Handle) {
	var c C.gn_generate_options
	tk := e.Tokenizer
	if o.Thinking {
		c.thinking = 1
	}
	c.thinking_budget = C.int32_t(o.ThinkingBudget)
	c.bos = C.int32_t(tk.BOSTokenID())
	c.assistant_end = C.int32_t(tk.EncodeSpecial("<|assistant_end|>"))
	c.tool_start = C.int32_t(tk.EncodeSpecial("<|tool_start|>"))
	c.tool_end = C.int32_t(tk.EncodeSpecial("<|tool_end|>"))
	c.tool_output_start = C.int32_t(tk.EncodeSpecial("<|tool_output_start|>"))
	c.tool_output_end = C.int32_t(tk.EncodeSpecial("<|tool_output_end|>"))
	c.think_start = C.int32_t(tk.EncodeSpecial("<|think_start|>"))
	c.think_end = C.int32_t(tk.EncodeSpecial("<|think_end|>"))
	h := cgo.NewHandle(e)
	c.tool = (*[0]byte)(C.gonanoHipTool)
	c.tool_user = unsafe.Pointer(uintptr(h))
	return c, h
}
