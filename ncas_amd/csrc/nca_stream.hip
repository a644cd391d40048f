// The streamed bf16 rollout kernel's translation unit (built with MFMA results in VGPRs) and its
// launch planning.
#include <hip/hip_runtime.h>

#include <string.h>

#include "nca_stream.h"
#include "nca_rollout_stream.h"

namespace nca {

// Streamed bf16 kernel for C = 64, hidden = 256: two row groups per workgroup; needs W + 1 <= 16
// (single perception buffer) and a board small enough for 16-bit halo offsets.
hipError_t launch_stream64(const RolloutParams &p, hipStream_t st, unsigned lds_limit, bool *used) {
    *used = false;
    if (p.W + 1 > 16 || p.noise || p.fire_f32) return hipSuccess;
    const int hw = p.H * p.W, nq4 = (hw + 3) / 4;
    const bool batched = !p.adaptive && !p.fire_u8;
    int rg = (int)((p.rows + 511) / 512);
    if (rg > 8) rg = 8;
    if (rg < 1) rg = 1;
    StPlan L{};
    for (; rg >= 1; --rg) {
        int nb = batched ? 256 / (rg * nq4) : 1;
        nb = nb < 1 ? 1 : (nb > 16 ? 16 : nb);
        L = st_plan(rg, p.H, p.W, p.c_out, p.n_out, nb);
        if (L.total <= lds_limit && L.PB < 65536) break;
    }
    if (rg < 1) return hipSuccess;
    StParams sp;
    memset(&sp, 0, sizeof(sp));
    sp.a = p;
    sp.rg = rg;
    sp.G = L.G;
    sp.RP = L.RP;
    sp.PB = L.PB;
    sp.NB = L.NB;
    sp.l_P = L.P;
    sp.l_Ptrash = L.Ptrash;
    sp.l_M = L.M;
    sp.l_Z = L.Z;
    sp.l_D = L.D;
    sp.l_cinfo = L.cinfo;
    sp.l_fire = L.fire;
    sp.l_fired = L.fired;
    sp.l_head = L.head;
    sp.l_hcp = L.hcp;
    sp.off_w1q = p.off_w1q;
    sp.off_w2k = p.off_w2k;
    auto kfn = rollout_stream64;
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(kfn),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)L.total);
    if (e != hipSuccess) return e;
    const int64_t grid = (p.rows + 2 * rg - 1) / (2 * rg);
    hipLaunchKernelGGL(kfn, dim3((unsigned)grid), dim3(256), L.total, st, sp);
    *used = true;
    return hipGetLastError();
}

}  // namespace nca
