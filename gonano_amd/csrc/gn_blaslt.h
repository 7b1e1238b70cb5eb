// gn_blaslt.h - plain fp32 products through hipBLASLt.
//
// A session's GEMMs whose epilogue is a plain store, an accumulate or a
// residual add (C = alpha*A.B^T [+ Cin]) and that are large enough go to
// hipBLASLt, which reaches 0.8-0.97 of the fp32 MFMA peak on the
// session's training and lm_head shapes.  Products with a fused epilogue
// (ReLU^2 and its gradient, softcap, deferred split-K sums), the
// expert-grouped MoE products and small ones stay on gemm_kernel.
//
// Algorithm choice is deterministic: the first result of hipBLASLt's
// heuristic for the problem, cached per problem (results do not depend on
// timing noise).  Every such algorithm was checked to be bitwise
// deterministic run to run and to capture into a HIP graph as kernel nodes
// only (no memset or copy nodes).
#pragma once

#include "gn_kernels.h"

namespace gn {

struct BlasLt;
// One handle and workspace per session (device current at creation).
BlasLt* blaslt_create();
void blaslt_destroy(BlasLt* b);
// Runs d on hipBLASLt if it is a plain product hipBLASLt takes; returns
// false (nothing launched) otherwise, for the caller's own kernel.  Never
// chooses an algorithm for a new problem while `st` is being captured.
bool blaslt_gemm(BlasLt* b, const GemmDesc& d, hipStream_t st);

}  // namespace gn
