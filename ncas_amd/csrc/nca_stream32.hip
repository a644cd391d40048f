// The streamed bf16 rollout kernel for C = 32, hidden = 256 (built with MFMA results in VGPRs)
// and its launch planning.
#include <hip/hip_runtime.h>

#include <math.h>
#include <string.h>

#include "nca_stream.h"
#include "nca_rollout_stream32.h"

namespace nca {

// The gated-firing threshold on s = sum of exponentials (s >= 1) for a 2-output mlp head: the
// readout's confidence min(max(1/s, 0), 1) (IEEE single-precision division, round to nearest)
// exceeds tau exactly when s < the returned value, the smallest single-precision s >= 1 whose
// confidence is <= tau (1/s does not increase with s).
static float conf_threshold(float tau) {
    if (!(tau < 1.0f)) return 0.0f;  // conf <= 1: never above tau
    if (tau < 0.0f) return INFINITY;
    auto conf_le = [&](uint32_t bits) {
        float sv;
        memcpy(&sv, &bits, 4);
        volatile float num = 1.0f;
        float c = num / sv;
        if (c > 1.0f) c = 1.0f;
        return c <= tau;
    };
    uint32_t lo = 0x3f800000u, hi = 0x7f800000u;  // 1.0 .. +inf (conf(+inf) = 0 <= tau)
    if (conf_le(lo)) return 1.0f;
    while (hi - lo > 1) {
        const uint32_t mid = lo + (hi - lo) / 2;
        if (conf_le(mid))
            hi = mid;
        else
            lo = mid;
    }
    float r;
    memcpy(&r, &hi, 4);
    return r;
}

// The gated decision of a 2-output mlp head, 1 + readout_expf(d) < conf_s for the logit gap
// d = min - max <= 0, as d <= the returned limit: readout_expf is non-decreasing on [-87, 0]
// (checked for every float of that range) and constant below it, so the decision holds on a
// down-set of gaps, whose largest member a bisection over the magnitudes 0 .. 87 finds with the
// same readout_expf. NaN: never (conf_s <= 1); +inf: always.
static float conf_gap_limit(float conf_s) {
    auto hi = [&](uint32_t mbits) {
        float m;
        memcpy(&m, &mbits, 4);
        volatile float one = 1.0f;
        return one + readout_expf(-m) < conf_s;
    };
    if (!(conf_s > 1.0f)) return __builtin_nanf("");
    if (hi(0u)) return INFINITY;
    uint32_t lo = 0u, top = 0x42ae0000u;  // 87.0f: hi(top) since 1 + readout_expf(-87) rounds to 1
    while (top - lo > 1) {
        const uint32_t mid = lo + (top - lo) / 2;
        if (hi(mid))
            top = mid;
        else
            lo = mid;
    }
    float m;
    memcpy(&m, &top, 4);
    return -m;
}

// One board per workgroup: needs W <= 31 (in-place update distance), H W >= W + 81 (taps loaded an
// interval ahead hold the step's state), H W <= 1024 (a step's draw is one group of 4 cells per
// channel-wave thread), wall or zero padding (the border cells are constants),
// for gated firing the output slice inside one channel quad and at most 4 outputs, and the plan
// within the LDS.
bool stream32_fits(int H, int W, int padding, int c_out, int n_out, unsigned lds_limit) {
    if (W > 31 || H < 1 || W < 1 || H * W < W + 81 || H * W > 1024 || padding == 2) return false;
    const St32Plan L = st32_plan(H, W, c_out, n_out);
    return L.total <= lds_limit && L.NM < 65536;
}

// Pieces per board for the recording kernel (1: whole boards). P in {3, 2} when the rows' P
// workgroups all fit the device at once (rows P <= cus, one workgroup per CU), every piece has
// (Hs - 1) W >= 240 (a halo refresh fits between the taps that read the old and the new row) and
// the piece's plan fits the LDS.
int stream32_pieces(int64_t rows, int H, int W, int c_out, int n_out, unsigned lds_limit, int cus) {
    if (g_piece_debug.plan_cus > 0) cus = g_piece_debug.plan_cus;
    for (int P = 3; P >= 2; --P) {
        const int Hp = (H + P - 1) / P, last = H - (P - 1) * Hp;
        if (last < 1 || rows * P > cus) continue;
        const int Hm = last < Hp ? last : Hp;
        if ((Hm - 1) * W < 240) continue;
        if (st32_plan(Hp, W, c_out, n_out, true).total > lds_limit) continue;
        return P;
    }
    return 1;
}

size_t stream32_xch_bytes(int64_t rows, int P, int W) {
    return P > 1 ? kXchStatusBytes + (size_t)rows * P * 2 * 4 * W * St32::C * sizeof(uint64_t) : 0;
}

// n 8-byte words at x cleared with 16-byte stores where x is 16-byte aligned (a leading odd word
// and a trailing one with 8-byte stores)
__global__ void xch_clear(uint64_t *x, int64_t n) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x, stride = (int64_t)gridDim.x * blockDim.x;
    const int64_t head = (reinterpret_cast<uintptr_t>(x) & 15u) ? 1 : 0;
    if (t == 0 && head && n > 0) x[0] = 0;
    const int64_t np = (n - head) / 2;
    uint4 *xp = reinterpret_cast<uint4 *>(x + head);
    for (int64_t e = t; e < np; e += stride) xp[e] = make_uint4(0u, 0u, 0u, 0u);
    if (t == 0 && head + 2 * np < n) x[n - 1] = 0;
}

hipError_t clear_words(uint64_t *x, int64_t n, hipStream_t st) {
    if (n <= 0) return hipSuccess;
    const int64_t b = (n / 2 + 255) / 256;
    hipLaunchKernelGGL(xch_clear, dim3((unsigned)(b < 1024 ? (b > 0 ? b : 1) : 1024)), dim3(256), 0, st, x, n);
    return hipGetLastError();
}

PieceDebug g_piece_debug;

// pieces > 1 (recording only): P workgroups per board exchanging their boundary rows through xch,
// stream32_xch_bytes of device memory that this call clears before the launch, then the repair
// launch (whole boards, run only if a piece's wait ran out)
hipError_t launch_stream32(const RolloutParams &p, hipStream_t st, unsigned lds_limit, bool *used, int pieces,
                           uint64_t *xch) {
    *used = false;
    if (p.noise || p.fire_f32) return hipSuccess;
    if (!stream32_fits(p.H, p.W, p.padding, p.c_out, p.n_out, lds_limit)) return hipSuccess;
    if (p.adaptive && ((p.out_off & 3) != 0 || p.c_out > 4 || p.n_out > 4)) return hipSuccess;
    const int hw = p.H * p.W;
    if ((int64_t)p.n_steps * hw + 64 > 0x7fffffff) return hipSuccess;
    if (p.rows > 0x7fffffff) return hipSuccess;
    if (p.x_rec && p.adaptive) return hipSuccess;  // recording is for uniform firing
    const int P = (pieces > 1 && p.x_rec && !p.adaptive && !p.conf_out && !p.fired_out && xch) ? pieces : 1;
    auto kfn = p.adaptive ? rollout_stream32<true, false>
                          : (p.x_rec ? rollout_stream32<false, true> : rollout_stream32<false, false>);
    // the attribute is the limit for every launch of the function (whole boards and pieces take
    // different sizes), so calls from several host threads cannot undercut one another's
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(kfn),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds_limit);
    if (e != hipSuccess) return e;
    if (p.rows <= 0) return hipSuccess;
    uint32_t *status = P > 1 ? reinterpret_cast<uint32_t *>(xch) : nullptr;
    // one launch of np workgroups per board (1: whole boards); run_if: the repair launch
    auto launch = [&](int np, const uint32_t *run_if) -> hipError_t {
        const int Hp = (p.H + np - 1) / np;
        const St32Plan L = st32_plan(np > 1 ? Hp : p.H, p.W, p.c_out, p.n_out, np > 1);
        St32Params sp;
        memset(&sp, 0, sizeof(sp));
        sp.a = p;
        sp.P = np;
        sp.Hp = np > 1 ? Hp : 0;
        sp.xch = np > 1 ? xch + kXchStatusBytes / sizeof(uint64_t) : nullptr;
        sp.halo_status = np > 1 ? status : nullptr;
        sp.spin_limit = g_piece_debug.spin_limit > 0 ? g_piece_debug.spin_limit : kHaloSpin;
        sp.tag_skew = g_piece_debug.force_timeout ? (1 << 30) : 0;
        sp.run_if = run_if;
        sp.l_gidx = L.gidx;
        sp.NM = L.NM;
        sp.RING = L.RING;
        sp.T = (int)(((int64_t)p.n_steps * hw + 15) / 16);
        sp.l_M = L.M;
        sp.l_Z = L.Z;
        sp.l_D = L.D;
        sp.l_cinfo = L.cinfo;
        sp.l_ring = L.ring;
        sp.l_given = L.given;
        sp.l_head = L.head;
        sp.l_evp = L.evp;
        sp.l_flags = L.flags;
        sp.off_w1q = p.off_w1q;
        sp.off_w2k = p.off_w2k;
        sp.fast_conf = p.adaptive && p.head_kind == 0 && p.n_out == 2;
        sp.conf_s = conf_threshold(p.tau);
        sp.conf_d = conf_gap_limit(sp.conf_s);
        // pieces: more than half the LDS, so no two workgroups share a CU (each piece runs
        // alongside its neighbours)
        const unsigned lds = np > 1 && L.total <= lds_limit / 2 ? lds_limit / 2 + 16u : L.total;
        hipLaunchKernelGGL(kfn, dim3((unsigned)(p.rows * np)), dim3(512), lds, st, sp);
        return hipGetLastError();
    };
    if (P > 1) {
        const int64_t n = (int64_t)(stream32_xch_bytes(p.rows, P, p.W) / sizeof(uint64_t));
        hipLaunchKernelGGL(xch_clear, dim3(256), dim3(256), 0, st, xch, n);
        if ((e = hipGetLastError()) != hipSuccess) return e;
        // The pieces of a board wait on one another, and nothing makes the runtime keep them
        // resident together (a cooperative launch would, but on this runtime it held the host
        // back for the rest of the training iteration: 3.5 - 5.3 ms per 64-board 30x30 iteration
        // against 3.4 ms, and 3.6 - 3.8 ms from a stream of its own). A wait that runs out sets
        // the status word instead, and the repair launch then recomputes every board whole,
        // overwriting the pieces' states, so the states are right in every case; when no wait ran
        // out its workgroups return at once (a few microseconds).
        if ((e = launch(P, nullptr)) != hipSuccess) return e;
        if ((e = launch(1, status)) != hipSuccess) return e;
        *used = true;
        return hipSuccess;
    }
    if ((e = launch(1, nullptr)) != hipSuccess) return e;
    *used = true;
    return hipSuccess;
}

}  // namespace nca
