// The streamed bf16 rollout kernel's translation unit (built with MFMA results in VGPRs) and its
// launch planning.
#include <hip/hip_runtime.h>

#include <string.h>

#include "nca_stream.h"
#include "nca_rollout_stream.h"

namespace nca {

// Streamed bf16 kernel for C = 64, hidden = 256: R rows per workgroup with (R-1) H W >= 79, so a
// board's next step starts five tiles after its previous one; needs W + 1 <= 16 (single
// perception buffer), at most 64 halo cells (two 16-byte halo chunks per thread), the plan within
// the LDS and 16-bit halo offsets.
hipError_t launch_stream64(const RolloutParams &p, hipStream_t st, unsigned lds_limit, bool *used) {
    *used = false;
    if (p.W + 1 > 16 || 2 * (p.W + 2) + 2 * p.H > 64 || p.noise || p.fire_f32) return hipSuccess;
    const int hw = p.H * p.W, nq4 = (hw + 3) / 4;
    const bool batched = !p.adaptive && !p.fire_u8;
    const int R = 1 + (St64::GAP + hw - 1) / hw;
    int nb = batched ? 256 / (R * nq4) : 1;
    nb = nb < 1 ? 1 : (nb > 16 ? 16 : nb);
    const StPlan L = st_plan(R, p.H, p.W, p.c_out, p.n_out, nb);
    if (L.total > lds_limit || L.PB >= 65536) return hipSuccess;
    if ((int64_t)p.n_steps * L.RH + 64 > 0x7fffffff) return hipSuccess;
    StParams sp;
    memset(&sp, 0, sizeof(sp));
    sp.a = p;
    sp.R = R;
    sp.RP = L.RP;
    sp.PB = L.PB;
    sp.NB = L.NB;
    sp.RH = L.RH;
    sp.RING = L.RING;
    sp.T = (int)(((int64_t)p.n_steps * L.RH + 15) / 16);
    sp.l_P = L.P;
    sp.l_M = L.M;
    sp.l_Z = L.Z;
    sp.l_H = L.H;
    sp.l_cinfo = L.cinfo;
    sp.l_ring = L.ring;
    sp.l_fired = L.fired;
    sp.l_head = L.head;
    sp.l_hcp = L.hcp;
    sp.l_evp = L.evp;
    sp.off_w1q = p.off_w1q;
    sp.off_w2h = p.off_w2h;
    auto kfn = rollout_stream64;
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(kfn),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)L.total);
    if (e != hipSuccess) return e;
    const int64_t grid = (p.rows + R - 1) / R;
    if (grid <= 0) return hipSuccess;
    hipLaunchKernelGGL(kfn, dim3((unsigned)grid), dim3(512), L.total, st, sp);
    *used = true;
    return hipGetLastError();
}

}  // namespace nca
