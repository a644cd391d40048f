// Entry of the halo-tiled per-step kernel, defined in nca_tiled.hip.
#pragma once

#include <hip/hip_runtime.h>

#include "nca_rollout.h"

namespace nca {

// One step of every row: p.x_in -> p.x_out (distinct buffers). `step` is the step's index in the
// call (Philox counter p.step0 + step, injected-mask slice), `first` applies the clamp. Sets
// *ok false (and launches nothing) when the cell shape has no tiled kernel or no window fits.
hipError_t tiled_step(int C, int HD, bool bf16, const RolloutParams &p, int step, int first, hipStream_t st,
                      bool *ok);

}  // namespace nca
