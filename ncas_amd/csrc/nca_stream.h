// Entries of the streamed bf16 rollout kernels (C = 64 and C = 32, hidden = 256), defined in
// nca_stream.hip and nca_stream32.hip.
#pragma once

#include <hip/hip_runtime.h>

#include "nca_rollout.h"

namespace nca {

// Launches the streamed kernel when the call fits it (grid width <= 15, no noise, no single-step
// fp32 mask, LDS plan within lds_limit bytes) and sets *used; otherwise leaves *used false.
hipError_t launch_stream64(const RolloutParams &p, hipStream_t st, unsigned lds_limit, bool *used);

// Whether a grid fits the streamed C = 32, hidden = 256 kernel (one board per workgroup).
bool stream32_fits(int H, int W, int padding, int c_out, int n_out, unsigned lds_limit);

// Launches the streamed C = 32 kernel when the call fits it (stream32_fits, no noise, no
// single-step fp32 mask, gated firing with the output slice in one channel quad) and sets *used;
// otherwise leaves *used false. pieces > 1 (recording calls without per-board outputs): that many
// workgroups per board, exchanging boundary rows through xch (stream32_xch_bytes, cleared by the
// call).
hipError_t launch_stream32(const RolloutParams &p, hipStream_t st, unsigned lds_limit, bool *used, int pieces = 1,
                           uint64_t *xch = nullptr);

// Workgroups per board for a recording call on a device of `cus` CUs (1: whole boards), and the
// exchange bytes that takes: a status block of kXchStatusBytes (its first word is set to 1 when
// a piece's wait for its neighbour ran out) and the exchange slots.
int stream32_pieces(int64_t rows, int H, int W, int c_out, int n_out, unsigned lds_limit, int cus);
size_t stream32_xch_bytes(int64_t rows, int P, int W);
constexpr size_t kXchStatusBytes = 256;

// re-reads of an exchange word before a piece gives up on its neighbour (about a second)
constexpr int kHaloSpin = 1 << 20;

// Zero n 8-byte words on the stream (a kernel, so the call can sit in a captured graph).
hipError_t clear_words(uint64_t *x, int64_t n, hipStream_t st);

// Test settings of the pieces' bounded waits and of their planning (nca_set_piece_debug):
// spin_limit > 0 replaces the wait's limit of re-reads; force_timeout makes every wait look for a
// tag that never comes (so it runs out after spin_limit re-reads); plan_cus > 0 plans pieces as
// for a device of that many CUs (a launch too large to be resident is then refused and the
// boards run whole). All zero in use. back_path (nca_set_bptt_backward_path): 0 automatic, 1 the
// backward as three launches per step, 2 the one-launch backward on whole boards.
struct PieceDebug {
    int spin_limit = 0, force_timeout = 0, plan_cus = 0, back_path = 0;
};
extern PieceDebug g_piece_debug;

}  // namespace nca
