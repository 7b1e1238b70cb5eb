// gn_optimizer.h - MuonAdamW on the device (optimizer/optimizer.go).
#pragma once

#include <vector>

#include "gn_kernels.h"
#include "gonano_hip.h"

namespace gn {

// One optimized tensor (or tensor view) of the session: device parameter
// and gradient pointers, its shape, its group's hyperparameters and its
// state region (layout: opt_state_floats).
struct OptTensor {
  float* p = nullptr;
  const float* g = nullptr;
  int64_t rows = 0, cols = 0;
  gn_opt_param h{};
  float* st = nullptr;
  int step = 0;  // AdamW step count (optimizer.go:55-59)
};

// AdamW: expAvg[n], expAvgSq[n]; Muon: momentum[n], secondMom[max(rows,
// cols)]; Sinkhorn: momentum[n].
int64_t opt_state_floats(const gn_opt_param& h);

// MuonAdamW.Step (optimizer.go:118-137) over `ts` in order, on stream st.
void optimizer_step(std::vector<OptTensor>& ts, hipStream_t st, DeviceArena* ws);

}  // namespace gn
