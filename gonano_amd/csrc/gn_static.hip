// gn_static.hip - gn_sample_next_token_static: inference.SampleNextToken on
// host logits without any device allocation.
//
// gn_sample_next_token stages the logits, the RNG state and the sampled ids
// through a device arena (hipMalloc) on a stream it creates per call.  This
// variant stages them through one fixed array of device memory that lives in
// the library's code object, so it allocates nothing: for callers that
// cannot call hipMalloc (tight serving loops, harnesses that forbid it).
//
// Layout of the array (kStaticBytes):
//   [0, 256)                 the RNG base state {hi, lo} of the call
//   [256, 256 + kIdBytes)    the sampled ids, rows int32
//   [256 + kIdBytes, end)    the logits, rows * vocab float32
// Every call on a device reuses that device's copy and leaves the last
// call's contents in it; calls on one device take that device's lock for
// their whole duration (copies, sampler, stream synchronization), so they
// never overlap on the array.
#include <mutex>
#include <vector>

#include "gn_model.h"

namespace gn {

static constexpr size_t kStateBytes = 256;
static constexpr int64_t kMaxRows = 65536;
static constexpr size_t kIdBytes = (size_t)kMaxRows * sizeof(int32_t);
static constexpr int64_t kMaxLogits = (int64_t)16 << 20;  // floats: 64 MiB
static constexpr size_t kStaticBytes = kStateBytes + kIdBytes + (size_t)kMaxLogits * sizeof(float);

static __device__ __align__(256) unsigned char scratch[kStaticBytes];

// The array's device address, per device.  In host code `scratch` names a
// host-side stand-in, never device memory: kernels and copies only ever
// receive the address hipGetSymbolAddress returns for the current device.
static std::mutex g_scratch_mu;
static std::vector<void*> g_scratch_ptr;
// One lock per device, held through a whole call.
static constexpr int kMaxDevices = 64;
static std::mutex g_call_mu[kMaxDevices];

static unsigned char* scratch_on(int device) {
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if ((int)g_scratch_ptr.size() <= device) g_scratch_ptr.resize(device + 1, nullptr);
  if (!g_scratch_ptr[device]) {
    void* p = nullptr;
    GN_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    GN_CHECK(p != nullptr, "sampler scratch: no device address");
    g_scratch_ptr[device] = p;
  }
  return static_cast<unsigned char*>(g_scratch_ptr[device]);
}

}  // namespace gn

using namespace gn;

extern "C" {

int gn_sample_next_token_static(const float* logits, int64_t rows, int64_t vocab,
                                uint64_t* rng_state, float temperature, int64_t top_k,
                                int32_t* out) {
  return guard([&] {
    GN_CHECK(logits && rng_state && out, "null argument");
    GN_CHECK(rows >= 0 && vocab > 0 && vocab < (1ll << 31), "bad logits shape");
    GN_CHECK(rows <= kMaxRows, "sample_next_token_static: more than 65536 rows");
    GN_CHECK(rows * vocab <= kMaxLogits,
             "sample_next_token_static: rows * vocab exceeds the 16 Mi-float static buffer");
    if (rows == 0) return;
    int dev = 0;
    GN_HIP(hipGetDevice(&dev));
    GN_CHECK(dev >= 0 && dev < kMaxDevices, "sample_next_token_static: device index above 63");
    std::lock_guard<std::mutex> call_lock(g_call_mu[dev]);
    unsigned char* base = scratch_on(dev);
    uint64_t* dstate = reinterpret_cast<uint64_t*>(base);
    int32_t* dout = reinterpret_cast<int32_t*>(base + kStateBytes);
    float* dl = reinterpret_cast<float*>(base + kStateBytes + kIdBytes);
    hipStream_t st = hipStreamPerThread;
    GN_HIP(hipMemcpyAsync(dl, logits, sizeof(float) * rows * vocab, hipMemcpyHostToDevice, st));
    GN_HIP(hipMemcpyAsync(dstate, rng_state, sizeof(uint64_t) * 2, hipMemcpyHostToDevice, st));
    SamplerArgs sa{};
    sa.logits = dl; sa.ldl = vocab; sa.rows = (int)rows; sa.V = (int)vocab;
    sa.samples_per_group = (int)rows; sa.base_states = dstate; sa.temperature = temperature;
    sa.top_k = (int)top_k; sa.out = dout;
    launch_sampler(sa, st);
    GN_HIP(hipMemcpyAsync(out, dout, sizeof(int32_t) * rows, hipMemcpyDeviceToHost, st));
    GN_HIP(hipStreamSynchronize(st));
    if (temperature > 0) advance_rng_state(rng_state, (uint64_t)rows * (uint64_t)vocab);
  });
}

}  // extern "C"
