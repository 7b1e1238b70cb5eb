// gn_prims.h - launchers of the kernels.Backend primitive kernels.
#pragma once

#include "gn_common.h"

namespace gn {

enum EwOp {
  EW_ADD, EW_SUB, EW_MUL, EW_DIV, EW_SCALE, EW_ADD_SCALED, EW_NEG, EW_ABS, EW_SQUARE, EW_RELU2,
  EW_EXP, EW_SIGMOID, EW_TANH, EW_RSQRT, EW_SWIGLU
};
enum RedOp { RED_SUM, RED_MAX, RED_ARGMAX, RED_DOT };

void launch_elementwise(float* d, const float* l, const float* r, int64_t n, int op, float f,
                        hipStream_t st);
void launch_swiglu_backward(float* dg, float* du, const float* g, const float* u, const float* d,
                            float clamp, int64_t n, hipStream_t st);
void launch_reduce(const float* v, int64_t n, int op, float* out_f, int64_t* out_i,
                   const float* w, hipStream_t st);
void launch_softmax_rows(float* d, const float* s, int64_t rows, int64_t cols, hipStream_t st);
void launch_rmsnorm_rows_prim(float* d, const float* s, int64_t rows, int64_t cols, float eps,
                              hipStream_t st);
void launch_indexer_scores(float* d, const float* q, const float* k, const float* w, int64_t rows,
                           int64_t blocks, int64_t heads, int64_t dim, hipStream_t st);
void launch_indexer_block_max(float* d, const float* s, int64_t rows, int64_t blocks,
                              int64_t group, hipStream_t st);
void launch_topk_rows(int32_t* out, const float* scores, const float* bias, int64_t rows,
                      int64_t count, int64_t k, uint8_t* taken, hipStream_t st);
void launch_gather_weights(float* w, const float* probs, const int32_t* sel, int64_t rows,
                           int64_t experts, int64_t k, hipStream_t st);
void launch_attn_row_fwd(float* S, int64_t ncols, int64_t kstart, int64_t qlen, int64_t offset,
                         int64_t window, const int32_t* seg, int64_t nseg, int mode, float* lse,
                         float* mx, float* sum, hipStream_t st);
void launch_attn_row_bwd(float* S, float* dP, int64_t qlen, int64_t klen, int64_t offset,
                         int64_t window, const int32_t* seg, int64_t nseg, const float* lse,
                         const float* corr, hipStream_t st);
void launch_attn_combine(const float* const* accs, const float* const* mxs,
                         const float* const* sums, int64_t parts, int64_t qlen, int64_t dim,
                         float* out, float* lse, hipStream_t st);

}  // namespace gn
