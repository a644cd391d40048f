// Entry of the streamed bf16 rollout kernel (C = 64, hidden = 256), defined in nca_stream.hip.
#pragma once

#include <hip/hip_runtime.h>

#include "nca_rollout.h"

namespace nca {

// Launches the streamed kernel when the call fits it (grid width <= 15, no noise, no single-step
// fp32 mask, LDS plan within lds_limit bytes) and sets *used; otherwise leaves *used false.
hipError_t launch_stream64(const RolloutParams &p, hipStream_t st, unsigned lds_limit, bool *used);

}  // namespace nca
