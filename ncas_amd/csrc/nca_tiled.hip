// The halo-tiled per-step kernel's translation unit: window planning and launch of one step.
#include <hip/hip_runtime.h>

#include <string.h>

#include "nca_step16.h"
#include "nca_tiled_launch.h"
#include "nca_tiled.h"
#include "nca_window16.h"

namespace nca {

namespace {

constexpr unsigned kTiledLds = 160u * 1024u;

int cu_count() {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 256;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n < 1) return 256;
    return n;
}

// Window TW = min(W, 32) (a 128-byte row segment of one channel), TH the largest height up to
// 1024 / TW cells whose LDS plan fits.
template <int C, int HD, bool BF16>
bool choose_window(int H, int W, int c_out, int n_out, int *TH, int *TW, TiledPlan *L) {
    const int tw = W < 32 ? W : 32;
    int th = 1024 / tw;
    if (th > H) th = H;
    if (th < 1) th = 1;
    for (; th >= 1; --th) {
        *L = tiled_plan<C, HD, BF16>(th, tw, c_out, n_out);
        if (L->total <= kTiledLds) {
            *TH = th;
            *TW = tw;
            return true;
        }
    }
    return false;
}

template <int C, int HD, bool BF16, bool NOISE>
hipError_t launch(const RolloutParams &p, int step, int first, int in_nchw, int out_nchw, hipStream_t st,
                  bool *ok) {
    TiledParams tp;
    memset(&tp, 0, sizeof(tp));
    TiledPlan L;
    *ok = choose_window<C, HD, BF16>(p.H, p.W, p.c_out, p.n_out, &tp.TH, &tp.TW, &L);
    if (!*ok) return hipSuccess;
    tp.a = p;
    tp.step = step;
    tp.first = first;
    tp.in_nchw = in_nchw;
    tp.out_nchw = out_nchw;
    tp.tiles_y = (p.H + tp.TH - 1) / tp.TH;
    tp.tiles_x = (p.W + tp.TW - 1) / tp.TW;
    tp.n_windows = p.rows * tp.tiles_y * tp.tiles_x;
    tp.l_P = L.P;
    tp.l_M = L.M;
    tp.l_Z = L.Z;
    tp.l_H = L.H;
    tp.l_given = L.given;
    tp.l_fire = L.fire;
    tp.l_cinfo = L.cinfo;
    tp.l_head = L.head;
    tp.l_fired = L.fired;
    auto kfn = step_tiled<C, HD, BF16, NOISE>;
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(kfn),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)L.total);
    if (e != hipSuccess) return e;
    static const int n_cu = cu_count();
    const int64_t grid = tp.n_windows < n_cu ? tp.n_windows : n_cu;
    if (grid < 1) return hipSuccess;
    hipLaunchKernelGGL(kfn, dim3((unsigned)grid), dim3(256), L.total, st, tp);
    return hipGetLastError();
}

template <int C, int HD>
hipError_t launch_cell(bool bf16, const RolloutParams &p, int step, int first, int in_nchw, int out_nchw,
                       hipStream_t st, bool *ok) {
    if (bf16)
        return p.noise ? launch<C, HD, true, true>(p, step, first, in_nchw, out_nchw, st, ok)
                       : launch<C, HD, true, false>(p, step, first, in_nchw, out_nchw, st, ok);
    return p.noise ? launch<C, HD, false, true>(p, step, first, in_nchw, out_nchw, st, ok)
                   : launch<C, HD, false, false>(p, step, first, in_nchw, out_nchw, st, ok);
}

template <bool IN_NCHW, bool OUT_NCHW>
hipError_t launch_stream16(const RolloutParams &p, int step, int first, hipStream_t st) {
    Step16Params sp;
    memset(&sp, 0, sizeof(sp));
    sp.a = p;
    sp.step = step;
    sp.first = first;
    sp.tiles_per_row = (p.H * p.W + 15) / 16;
    sp.n_tiles = p.rows * (int64_t)sp.tiles_per_row;
    static const int n_cu = cu_count();
    sp.tiles_per_wg = (sp.n_tiles + n_cu - 1) / n_cu;
    const int64_t grid = (sp.n_tiles + sp.tiles_per_wg - 1) / sp.tiles_per_wg;
    if (grid < 1) return hipSuccess;
    if (first)
        hipLaunchKernelGGL((step_stream16<IN_NCHW, OUT_NCHW, true>), dim3((unsigned)grid), dim3(512), 0, st, sp);
    else
        hipLaunchKernelGGL((step_stream16<IN_NCHW, OUT_NCHW, false>), dim3((unsigned)grid), dim3(512), 0, st, sp);
    return hipGetLastError();
}

}  // namespace

int window16_windows(int L, int T, bool wrap) {
    if (T < 1 || T > kWinMaxT || 2 * T >= kWinMax) return 0;
    for (int n = 1; n <= L; ++n) {
        int widest = 0;
        for (int i = 0; i < n; ++i) {
            const WinAxis a = win_axis(i, n, L, T, wrap);
            const int wdt = a.h0 + (a.hi - a.lo) + a.h1;
            widest = wdt > widest ? wdt : widest;
        }
        if (widest <= kWinMax) return n;
    }
    return 0;
}

hipError_t window16_steps(const RolloutParams &p, int step, int T, int first, int in_nchw, int out_nchw,
                          hipStream_t st) {
    Win16Params wp;
    memset(&wp, 0, sizeof(wp));
    wp.a = p;
    wp.step = step;
    wp.T = T;
    wp.first = first;
    wp.in_nchw = in_nchw;
    wp.out_nchw = out_nchw;
    const bool wrap = p.padding == 2;
    wp.nwy = window16_windows(p.H, T, wrap);
    wp.nwx = window16_windows(p.W, T, wrap);
    if (wp.nwy < 1 || wp.nwx < 1) return hipErrorInvalidValue;
    wp.n_windows = p.rows * (int64_t)wp.nwy * wp.nwx;
    if (wp.n_windows < 1) return hipSuccess;
    if (wp.n_windows > 0x7fffffff) return hipErrorInvalidValue;
    auto kfn = first ? rollout_window16<true> : rollout_window16<false>;
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(kfn), hipFuncAttributeMaxDynamicSharedMemorySize,
                                       (int)kWinLds);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(kfn, dim3((unsigned)wp.n_windows), dim3(512), kWinLds, st, wp);
    return hipGetLastError();
}

hipError_t tiled_step(int C, int HD, bool bf16, const RolloutParams &p, int step, int first, int in_nchw,
                      int out_nchw, hipStream_t st, bool windows, bool *ok) {
    *ok = false;
    // the wave-per-tile kernel addresses the cell-major state with 31-bit byte offsets (its
    // stores put cells past a row's end at offset 2^31, beyond the buffer): larger batches run on
    // the halo-window kernel
    const bool offsets32 = p.rows * (int64_t)p.H * p.W * 16 * (int64_t)sizeof(float) < ((int64_t)1 << 31);
    if (C == 16 && HD == 128 && bf16 && !windows && !p.noise && !p.adaptive && offsets32) {
        *ok = true;
        if (in_nchw)
            return out_nchw ? launch_stream16<true, true>(p, step, first, st) : launch_stream16<true, false>(p, step, first, st);
        return out_nchw ? launch_stream16<false, true>(p, step, first, st) : launch_stream16<false, false>(p, step, first, st);
    }
    if (C == 16 && HD == 128) return launch_cell<16, 128>(bf16, p, step, first, in_nchw, out_nchw, st, ok);
    if (C == 32 && HD == 256) return launch_cell<32, 256>(bf16, p, step, first, in_nchw, out_nchw, st, ok);
    if (C == 64 && HD == 256) return launch_cell<64, 256>(bf16, p, step, first, in_nchw, out_nchw, st, ok);
    return hipSuccess;
}

}  // namespace nca
