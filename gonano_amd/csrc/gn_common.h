// gn_common.h - shared host/device helpers for libgnhip.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <stdexcept>
#include <string>

#include "../../include/gonano_hip.h"

namespace gn {

// A failed HIP call or a rejected argument throws; every extern "C" entry
// point catches, records the message for gn_last_error() and returns a
// gn_status code (the Go wrapper turns it into a panic, matching the
// reference's panic-on-misuse convention).
struct Error : std::runtime_error {
  int code;
  Error(int c, const std::string& m) : std::runtime_error(m), code(c) {}
};

void set_last_error(const std::string& msg);

#define GN_HIP(expr)                                                                   \
  do {                                                                                 \
    hipError_t _e = (expr);                                                            \
    if (_e != hipSuccess)                                                              \
      throw ::gn::Error(_e == hipErrorOutOfMemory ? GN_ERR_OOM : GN_ERR_HIP,           \
                        std::string(#expr) + ": " + hipGetErrorString(_e));            \
  } while (0)

#define GN_CHECK(cond, msg)                                                            \
  do {                                                                                 \
    if (!(cond)) throw ::gn::Error(GN_ERR_INVALID, std::string(msg));                  \
  } while (0)

// Runs body, mapping exceptions to status codes.  A failed runtime call
// (an allocation beyond the device memory, say) stays recorded as the
// thread's last HIP error; it is cleared here, so the next call's launch
// checks do not report it again.
template <class F>
int guard(F&& body) {
  try {
    body();
    return GN_OK;
  } catch (const Error& e) {
    set_last_error(e.what());
    if (e.code == GN_ERR_HIP || e.code == GN_ERR_OOM) (void)hipGetLastError();
    return e.code;
  } catch (const std::bad_alloc&) {
    set_last_error("host allocation failed");
    return GN_ERR_OOM;
  } catch (const std::exception& e) {
    set_last_error(e.what());
    return GN_ERR_INTERNAL;
  }
}

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// ---------------------------------------------------------------------------
// Device helpers
// ---------------------------------------------------------------------------
__device__ __forceinline__ float warp_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ float warp_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ double warp_sum_d(double v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Block-wide reductions for blockDim.x a multiple of 64 (<= 1024). `scratch`
// must hold blockDim.x/64 values; the result is broadcast to every thread.
template <typename T>
__device__ __forceinline__ T block_sum(T v, T* scratch) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6, nw = blockDim.x >> 6;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  __syncthreads();
  if (lane == 0) scratch[wid] = v;
  __syncthreads();
  T t = 0;
  for (int i = 0; i < nw; i++) t += scratch[i];
  return t;
}
__device__ __forceinline__ float block_max(float v, float* scratch) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6, nw = blockDim.x >> 6;
  v = warp_max(v);
  __syncthreads();
  if (lane == 0) scratch[wid] = v;
  __syncthreads();
  float t = scratch[0];
  for (int i = 1; i < nw; i++) t = fmaxf(t, scratch[i]);
  return t;
}

// Cross-lane sums inside groups of 8 / 16 lanes with DPP (no LDS traffic,
// unlike __shfl_xor, which lowers to ds_bpermute): quad_perm [1,0,3,2] and
// [2,3,0,1] give each quad its sum, row_half_mirror adds the other quad of
// the 8-lane half-row, row_mirror the other half of the 16-lane row.  Every
// lane ends with the same value (each step adds two equal partial sums in
// either order).
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}
__device__ __forceinline__ float sum8_dpp(float v) {
  v += dpp_f32<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp_f32<0x4E>(v);   // quad_perm [2,3,0,1]
  return v + dpp_f32<0x141>(v);  // row_half_mirror
}
__device__ __forceinline__ float sum16_dpp(float v) {
  v = sum8_dpp(v);
  return v + dpp_f32<0x140>(v);  // row_mirror
}
__device__ __forceinline__ float max16_dpp(float v) {
  v = fmaxf(v, dpp_f32<0xB1>(v));
  v = fmaxf(v, dpp_f32<0x4E>(v));
  v = fmaxf(v, dpp_f32<0x141>(v));
  return fmaxf(v, dpp_f32<0x140>(v));
}

// Softcap (model/transformer.go:11, tensors/math.go:38-45):
// 15 * tanh(y * float32(1/15)).
__device__ __forceinline__ float softcap15(float y) {
  const float inv = 1.0f / 15.0f;
  return tanhf(y * inv) * 15.0f;
}

}  // namespace gn
