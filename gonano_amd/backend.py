"""HipBackend: gonano's kernels.Backend (kernels/backend.go:21-297) over the
HIP C ABI, with the interface's method names and argument meaning so code
and tests written against the reference read the same.

Slices are numpy float32/int32 arrays; destinations are written in place and
may alias sources.  A failing call raises HipError (the reference panics).
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass
from typing import Optional, Sequence

import numpy as np

from ._lib import call, lib


def _f(a):
    if not (isinstance(a, np.ndarray) and a.dtype == np.float32 and a.flags.c_contiguous):
        raise TypeError("expected a C-contiguous float32 array")
    return a


def _ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


@dataclass
class AttentionForwardParameters:  # kernels/backend.go:167-177
    Query: np.ndarray
    Key: np.ndarray
    Value: np.ndarray
    QueryLength: int
    KeyLength: int
    HeadDim: int
    PositionOffset: int = 0
    Window: int = -1
    SegmentIDs: Optional[np.ndarray] = None


@dataclass
class AttentionForwardResult:  # kernels/backend.go:183-186
    Output: np.ndarray
    LogSumExp: Optional[np.ndarray] = None


@dataclass
class AttentionBackwardParameters:  # kernels/backend.go:201-215
    Query: np.ndarray
    Key: np.ndarray
    Value: np.ndarray
    Output: np.ndarray
    OutputGradient: np.ndarray
    LogSumExp: np.ndarray
    QueryLength: int
    KeyLength: int
    HeadDim: int
    PositionOffset: int = 0
    Window: int = -1
    RowCorrection: Optional[np.ndarray] = None
    SegmentIDs: Optional[np.ndarray] = None


@dataclass
class AttentionBackwardResult:  # kernels/backend.go:221-225
    QueryGradient: np.ndarray
    KeyGradient: np.ndarray
    ValueGradient: np.ndarray


@dataclass
class AttentionSplitParameters:  # kernels/backend.go:233-245
    Query: np.ndarray
    Key: np.ndarray
    Value: np.ndarray
    QueryLength: int
    KeyLength: int
    HeadDim: int
    PositionOffset: int
    Window: int
    KeyStart: int
    KeyEnd: int
    SegmentIDs: Optional[np.ndarray] = None


@dataclass
class AttentionSplitResult:  # kernels/backend.go:251-255
    Accumulator: np.ndarray
    Maximum: np.ndarray
    Sum: np.ndarray


@dataclass
class AttentionCombineParameters:  # kernels/backend.go:259-263
    Partials: Sequence[AttentionSplitResult]
    QueryLength: int
    HeadDim: int


def _seg(s):
    if s is None:
        return None, 0
    s = np.ascontiguousarray(s, np.int32)
    return s, s.size


class HipBackend:
    """kernels.Backend on an MI355X."""

    def __init__(self, device: int = 0):
        lib()
        call("gn_set_device", device)

    # -- Elementwise (kernels/backend.go:21-67) ----------------------------
    def Add(self, d, l, r): call("gn_add", _f(d), _f(l), _f(r), l.size)
    def Subtract(self, d, l, r): call("gn_subtract", _f(d), _f(l), _f(r), l.size)
    def Multiply(self, d, l, r): call("gn_multiply", _f(d), _f(l), _f(r), l.size)
    def Divide(self, d, l, r): call("gn_divide", _f(d), _f(l), _f(r), l.size)
    def Scale(self, d, s, factor): call("gn_scale", _f(d), _f(s), float(factor), s.size)
    def AddScaled(self, d, base, scaled, factor):
        call("gn_add_scaled", _f(d), _f(base), _f(scaled), float(factor), base.size)
    def Negate(self, d, s): call("gn_negate", _f(d), _f(s), s.size)
    def Abs(self, d, s): call("gn_abs", _f(d), _f(s), s.size)
    def Square(self, d, s): call("gn_square", _f(d), _f(s), s.size)
    def ReluSquared(self, d, s): call("gn_relu_squared", _f(d), _f(s), s.size)
    def SwiGLU(self, d, gate, up, clamp): call("gn_swiglu", _f(d), _f(gate), _f(up), float(clamp), gate.size)
    def SwiGLUBackward(self, dgate, dup, gate, up, dout, clamp):
        call("gn_swiglu_backward", _f(dgate), _f(dup), _f(gate), _f(up), _f(dout), float(clamp), gate.size)
    def Exp(self, d, s): call("gn_exp", _f(d), _f(s), s.size)
    def Sigmoid(self, d, s): call("gn_sigmoid", _f(d), _f(s), s.size)
    def Tanh(self, d, s): call("gn_tanh", _f(d), _f(s), s.size)
    def Rsqrt(self, d, s): call("gn_rsqrt", _f(d), _f(s), s.size)

    # -- Reductions (kernels/backend.go:70-78) -----------------------------
    def Sum(self, v) -> float:
        out = C.c_float()
        call("gn_sum", _f(v), v.size, C.byref(out))
        return out.value

    def Max(self, v) -> float:
        out = C.c_float()
        call("gn_max", _f(v), v.size, C.byref(out))
        return out.value

    def ArgMax(self, v) -> int:
        out = C.c_int64()
        call("gn_argmax", _f(v), v.size, C.byref(out))
        return out.value

    # -- LinearAlgebra (kernels/backend.go:82-93) --------------------------
    def MatMul(self, d, l, r, rowCount, columnCount, innerCount):
        call("gn_matmul", _f(d), _f(l), _f(r), rowCount, columnCount, innerCount)

    def MatMulTransposed(self, d, l, r, rowCount, columnCount, innerCount):
        call("gn_matmul_transposed", _f(d), _f(l), _f(r), rowCount, columnCount, innerCount)

    def DotProduct(self, l, r) -> float:
        out = C.c_float()
        call("gn_dot_product", _f(l), l.size, _f(r), r.size, C.byref(out))
        return out.value

    # -- Indexer (kernels/backend.go:103-116) ------------------------------
    def IndexerScores(self, d, q, k, w, rowCount, blockCount, headCount, dim):
        call("gn_indexer_scores", _f(d), _f(q), _f(k), _f(w), rowCount, blockCount, headCount, dim)

    def IndexerBlockMax(self, d, scores, rowCount, blockCount, groupSize):
        call("gn_indexer_block_max", _f(d), _f(scores), rowCount, blockCount, groupSize)

    # -- MoE (kernels/backend.go:119-141) ----------------------------------
    def TopKIndices(self, d, scores, rowCount, count, k):
        call("gn_topk_indices", d, _f(scores), rowCount, count, k)

    def MoEGateTopK(self, logits, bias, probs, selected, selectedWeights, rowCount, expertCount, k):
        call("gn_moe_gate_topk", _f(logits), _f(bias), _f(probs), selected, _f(selectedWeights),
             rowCount, expertCount, k)

    def GroupedMatMulTransposed(self, d, inp, w, tokenCounts, expertCount, columnCount, innerCount):
        call("gn_grouped_matmul_transposed", _f(d), _f(inp), _f(w),
             np.ascontiguousarray(tokenCounts, np.int32), expertCount, columnCount, innerCount)

    # -- Rows (kernels/backend.go:145-153) ---------------------------------
    def SoftmaxLastDim(self, d, s, rowCount, columnCount):
        call("gn_softmax_last_dim", _f(d), _f(s), rowCount, columnCount)

    def RMSNormLastDim(self, d, s, rowCount, columnCount, epsilon):
        call("gn_rmsnorm_last_dim", _f(d), _f(s), rowCount, columnCount, float(epsilon))

    # -- Attention (kernels/backend.go:267-283) ----------------------------
    def AttentionForward(self, p: AttentionForwardParameters, r: AttentionForwardResult):
        seg, n = _seg(p.SegmentIDs)
        call("gn_attention_forward", _f(p.Query), _f(p.Key), _f(p.Value), _ptr(seg), n,
             p.QueryLength, p.KeyLength, p.HeadDim, p.PositionOffset, p.Window, _f(r.Output),
             _ptr(r.LogSumExp))

    def AttentionBackward(self, p: AttentionBackwardParameters, r: AttentionBackwardResult):
        seg, n = _seg(p.SegmentIDs)
        call("gn_attention_backward", _f(p.Query), _f(p.Key), _f(p.Value), _f(p.Output),
             _f(p.OutputGradient), _f(p.LogSumExp), _ptr(p.RowCorrection), _ptr(seg), n,
             p.QueryLength, p.KeyLength, p.HeadDim, p.PositionOffset, p.Window,
             _f(r.QueryGradient), _f(r.KeyGradient), _f(r.ValueGradient))

    def AttentionForwardSplit(self, p: AttentionSplitParameters, r: AttentionSplitResult):
        seg, n = _seg(p.SegmentIDs)
        call("gn_attention_forward_split", _f(p.Query), _f(p.Key), _f(p.Value), _ptr(seg), n,
             p.QueryLength, p.KeyLength, p.HeadDim, p.PositionOffset, p.Window, p.KeyStart,
             p.KeyEnd, _f(r.Accumulator), _f(r.Maximum), _f(r.Sum))

    def AttentionCombine(self, p: AttentionCombineParameters, r: AttentionForwardResult):
        k = len(p.Partials)
        accs = (C.c_void_p * max(k, 1))(*[_ptr(_f(x.Accumulator)) for x in p.Partials])
        mxs = (C.c_void_p * max(k, 1))(*[_ptr(_f(x.Maximum)) for x in p.Partials])
        sums = (C.c_void_p * max(k, 1))(*[_ptr(_f(x.Sum)) for x in p.Partials])
        call("gn_attention_combine", accs, mxs, sums, k, p.QueryLength, p.HeadDim, _f(r.Output),
             _ptr(r.LogSumExp))


def sample_next_token(logits: np.ndarray, rng_state: np.ndarray, temperature: float,
                      top_k: int) -> np.ndarray:
    """inference.SampleNextToken (inference/sampler.go:16-24) on the GPU.
    rng_state is the uint64 pair {hi, lo} of the group's tensors.RNG stream
    and is advanced in place past the rows*vocab draws."""
    logits = _f(np.ascontiguousarray(logits, np.float32))
    rows, vocab = logits.shape
    out = np.zeros(rows, np.int32)
    call("gn_sample_next_token", logits, rows, vocab, rng_state, float(temperature), top_k, out)
    return out


def softcap_order_violations() -> int:
    """Neighbouring floats (all 2^32 bit patterns but NaNs, in increasing
    order) whose device softcap decreases: 0 when it is non-decreasing, which
    the decode sampler's selection on raw lm_head products relies on."""
    out = np.zeros(1, np.uint64)
    call("gn_softcap_order_check", out)
    return int(out[0])


def sample_next_token_static(logits: np.ndarray, rng_state: np.ndarray, temperature: float,
                             top_k: int) -> np.ndarray:
    """sample_next_token through the allocation-free entry point (the
    library's fixed device staging array: rows <= 65536, rows * vocab <=
    16 Mi floats; the library serializes calls on one device)."""
    logits = _f(np.ascontiguousarray(logits, np.float32))
    rows, vocab = logits.shape
    out = np.zeros(rows, np.int32)
    call("gn_sample_next_token_static", logits, rows, vocab, rng_state, float(temperature), top_k,
         out)
    return out
