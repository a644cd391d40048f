// The library's error channel (thread-local message read by nca_last_error), shared by the
// translation units of libnca_hip.so.
#pragma once

#include <hip/hip_runtime.h>

#include "nca_hip.h"

namespace nca {

int set_error(int code, const char *msg);           // stores msg, returns code
void clear_error();                                  // empties the message (start of an entry point)
int hip_status(hipError_t e, const char *what);      // NCA_OK, or NCA_ERR_HIP with the HIP message

// n_steps fused steps on the streamed C = 32 kernel that also write the state after every step
// (step s to x_rec + s rec_stride); *used = false (nothing launched) when that kernel does not
// take the call. The arguments are nca_rollout's, already checked by the caller. With xch_bytes
// >= recorded_xch_bytes(...) of device memory at xch, boards run in pieces of rows on several
// workgroups when the device has the CUs for them (*pieces, when given, is set to their number
// per board, 1 for whole boards; with pieces the launch clears the status word at xch itself).
// x_rec0, when given, receives a copy of x_in from the same launch (when *used).
int rollout_recorded(const nca_cell_desc *cell, const void *packed, int64_t rows, int H, int W, const float *x_in,
                     const uint8_t *given, const float *clamp, float *x_out, const nca_fire_desc *fire, int n_steps,
                     float *x_rec, int64_t rec_stride, hipStream_t st, bool *used, void *xch = nullptr,
                     size_t xch_bytes = 0, int *pieces = nullptr, float *x_rec0 = nullptr);

// Device memory rollout_recorded can use to run boards in pieces (0: it runs whole boards).
size_t recorded_xch_bytes(const nca_cell_desc *cell, int64_t rows, int H, int W);

}  // namespace nca
