// Entry of the halo-tiled per-step kernel, defined in nca_tiled.hip.
#pragma once

#include <hip/hip_runtime.h>

#include "nca_rollout.h"

namespace nca {

// One step of every row: p.x_in -> p.x_out (distinct buffers). `step` is the step's index in the
// call (Philox counter p.step0 + step, injected-mask slice), `first` applies the clamp;
// in_nchw / out_nchw select the caller's (rows, C, H, W) layout for x_in / x_out instead of the
// cell-major (rows, H, W, C) layout of the steps in between. bf16 cells with C = 16 run on the
// wave-per-tile kernel (step_stream16) unless `windows` asks for the halo-window kernel, as do
// noise and confidence-gated firing. Sets *ok false (and launches nothing) when the cell shape
// has no per-step kernel or no window fits.
hipError_t tiled_step(int C, int HD, bool bf16, const RolloutParams &p, int step, int first, int in_nchw,
                      int out_nchw, hipStream_t st, bool windows, bool *ok);

// Temporal blocking (rollout_window16): bf16 cells with C = 16 and 128 hidden units, uniform
// firing (Philox or injected u8 masks), no noise. window16_plan gives the windows per board
// along an axis of length L for T steps per launch (0: no window of at most kWinMax cells fits).
int window16_windows(int L, int T, bool wrap);
// Steps step .. step + T - 1 of the call in one launch: p.x_in -> p.x_out (distinct buffers).
hipError_t window16_steps(const RolloutParams &p, int step, int T, int first, int in_nchw, int out_nchw,
                          hipStream_t st);

}  // namespace nca
