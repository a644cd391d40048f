// C ABI of libnca_hip.so (declared in include/nca_hip.h): argument checks, weight packing,
// launch planning and the small kernels (fire mask, readout, conf@K selection).
#include <hip/hip_runtime.h>

#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <mutex>

#include "nca_hip.h"
#include "nca_device.h"
#include "nca_layout.h"
#include "nca_rollout.h"
#include "nca_stream.h"
#include "nca_tiled_launch.h"
#include "nca_status.h"
#include "nca_window16.h"

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

int hip_check(hipError_t e, const char *what) {
    if (e != hipSuccess) return fail(NCA_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
    return NCA_OK;
}

inline hipStream_t as_stream(void *s) { return reinterpret_cast<hipStream_t>(s); }

}  // namespace

namespace nca {

int set_error(int code, const char *msg) { return fail(code, "%s", msg); }
void clear_error() { g_err[0] = 0; }
int hip_status(hipError_t e, const char *what) { return hip_check(e, what); }

}  // namespace nca

namespace {

constexpr unsigned kLdsBytes = 160u * 1024u;  // gfx950 LDS per workgroup

// Kernel selection (nca_set_kernel_path): 0 automatic, 1 generic resident kernel for bf16,
// 2 the per-step kernels for every grid (no temporal blocking), 3 the halo-window per-step kernel
// for every grid, 4 the temporally blocked kernel wherever it applies, also on grids the
// resident kernels take. Per thread, so that a thread choosing a path never changes another
// thread's calls; so is the temporally blocked kernel's step count (nca_set_window_steps).
thread_local int g_path = 0;
thread_local int g_window_steps = 0;
// The automatic choice is one step per launch: on the 201x201 mazes the temporally blocked
// kernel (2 to 4 steps per launch) measured 63 to 79 us per step against 46 to 50 us for the
// wave-per-tile kernel, whose state stays in the Infinity Cache between steps.
constexpr int kDefaultWindowSteps = 1;

bool shape_supported(int C, int hidden) {
    return (C == 16 && hidden == 128) || (C == 32 && hidden == 256) || (C == 64 && hidden == 256);
}

int check_cell(const nca_cell_desc *d) {
    if (!d) return fail(NCA_ERR_INVALID, "cell descriptor is NULL");
    if (d->heads != 4)
        return fail(NCA_ERR_UNSUPPORTED, "heads=%d: only 4 perception kernels are implemented", d->heads);
    if (!shape_supported(d->channels, d->hidden))
        return fail(NCA_ERR_UNSUPPORTED,
                    "cell C=%d hidden=%d is not built (built: 16/128, 32/256, 64/256)", d->channels,
                    d->hidden);
    if (d->c_in < 0 || d->in_offset < 0 || d->in_offset + d->c_in > d->channels)
        return fail(NCA_ERR_INVALID, "input slice [%d, %d) exceeds the state", d->in_offset,
                    d->in_offset + d->c_in);
    if (d->c_out < 1 || d->out_offset < 0 || d->out_offset + d->c_out > d->channels)
        return fail(NCA_ERR_INVALID, "output slice [%d, %d) exceeds the state", d->out_offset,
                    d->out_offset + d->c_out);
    if (d->n_out < 1 || d->n_out > 16) return fail(NCA_ERR_UNSUPPORTED, "n_out=%d (1..16)", d->n_out);
    if (d->padding < NCA_PAD_ZERO || d->padding > NCA_PAD_WRAP)
        return fail(NCA_ERR_INVALID, "padding=%d", d->padding);
    if (d->head_kind != NCA_HEAD_MLP && d->head_kind != NCA_HEAD_L2)
        return fail(NCA_ERR_INVALID, "head_kind=%d", d->head_kind);
    if (d->precision != NCA_FP32 && d->precision != NCA_BF16)
        return fail(NCA_ERR_INVALID, "precision=%d", d->precision);
    return NCA_OK;
}

nca::PackedLayout layout_of(const nca_cell_desc *d) {
    return nca::packed_layout(d->channels, d->heads, d->hidden, d->c_out, d->n_out,
                              d->precision == NCA_BF16);
}

// ------------------------------------------------------------------------------------------
// Weight packing
__device__ __forceinline__ void pack_small(const float *src, int n, float *dst, int round_bf16, int b, int nb) {
    for (int i = b * blockDim.x + threadIdx.x; i < n; i += nb * blockDim.x) {
        const float v = src ? src[i] : 0.0f;
        dst[i] = round_bf16 ? nca::round_bf16(v) : v;
    }
}

// A fragments of an (M x K) row-major matrix (M, K multiples of 16 and of the k-tile). qC > 0
// (bf16 only) reorders the k axis quad-major: fragment column k = 16 iq + 4 head + ch reads
// matrix column head * qC + 4 iq + ch.
__device__ __forceinline__ void pack_frags(const float *src, int M, int K, int bf16, int qC, void *dst, int b, int nb) {
    const int total = M * K;
    const int ktile = bf16 ? 32 : 4;
    const int nkt = K / ktile;
    for (int e = b * blockDim.x + threadIdx.x; e < total; e += nb * blockDim.x) {
        int m, k;
        if (bf16) {
            const int s = e & 7, lane = (e >> 3) & 63, blk = e >> 9;
            const int kt = blk % nkt, mt = blk / nkt;
            m = mt * 16 + (lane & 15);
            k = kt * 32 + 8 * (lane >> 4) + s;
            if (qC > 0) k = ((k >> 2) & 3) * qC + 4 * (k >> 4) + (k & 3);
            reinterpret_cast<__bf16 *>(dst)[e] = (__bf16)src[(size_t)m * K + k];
        } else {
            const int lane = e & 63, blk = e >> 6;
            const int kt = blk % nkt, mt = blk / nkt;
            m = mt * 16 + (lane & 15);
            k = kt * 4 + (lane >> 4);
            reinterpret_cast<float *>(dst)[e] = src[(size_t)m * K + k];
        }
    }
}

// fc2 fragments of the streamed kernel (see nca_layout.h), bf16: the k axis follows the order in
// which fc1's accumulators are stored, p = 64 w + 16 g + 4 mt + v -> hidden 64 w + 16 mt + 4 g + v.
__device__ __forceinline__ void pack_w2h(const float *w2, int C, int HD, __bf16 *dst, int b, int nb) {
    const int nkt = HD / 32;
    const int total = C * HD;
    for (int e = b * blockDim.x + threadIdx.x; e < total; e += nb * blockDim.x) {
        const int s = e & 7, lane = (e >> 3) & 63, blk = e >> 9;
        const int kt = blk % nkt, m = blk / nkt;
        const int ch = 16 * m + (lane & 15);
        const int p = 32 * kt + 8 * (lane >> 4) + s;
        const int hid = (p & ~63) + 16 * ((p >> 2) & 3) + 4 * ((p >> 4) & 3) + (p & 3);
        dst[e] = (__bf16)w2[(size_t)ch * HD + hid];
    }
}

// fc2 fragments per hidden quarter (see nca_layout.h), bf16: the k axis of quarter q follows the
// order of fc1's accumulators in the wave that owns it, slot s of lane group g of k-tile k ->
// hidden q HD/4 + 16 (2 k + s / 4) + 4 g + s % 4.
__device__ __forceinline__ void pack_w2k(const float *w2, int C, int HD, __bf16 *dst, int b, int nb) {
    const int hpw = HD / 4, kt2n = hpw / 32, mt2n = C / 16;
    const int total = C * HD;
    for (int e = b * blockDim.x + threadIdx.x; e < total; e += nb * blockDim.x) {
        const int s = e & 7, lane = (e >> 3) & 63, blk = e >> 9;
        const int kt = blk % kt2n, m2 = (blk / kt2n) % mt2n, q = blk / (kt2n * mt2n);
        const int ch = 16 * m2 + (lane & 15);
        const int hid = q * hpw + 16 * (2 * kt + s / 4) + 4 * (lane >> 4) + (s % 4);
        dst[e] = (__bf16)w2[(size_t)ch * HD + hid];
    }
}

// The whole packing in one launch: workgroups [64 k, 64 k + 64) build fragment layout k (W1, W2,
// and for bf16 cells W2 for the hidden-major fc2, W1 quad-major, W2 k-major), the last one the
// small vectors (kernels, b1, b2, head, padding value).
struct PackArgs {
    const float *kernels, *w1, *b1, *w2, *b2, *head_w, *head_b, *pad_vec;
    int nk, HD, C, F, nhw, nhb, bf;
    unsigned char *pk;
    nca::PackedLayout L;
};

__global__ void pack_all(PackArgs a) {
    constexpr int kPB = 64;
    const int b = blockIdx.x, part = b / kPB, pb = b - part * kPB;
    const int nfrag = a.bf ? 5 : 2;
    unsigned char *pk = a.pk;
    if (part >= nfrag) {
        pack_small(a.kernels, a.nk, reinterpret_cast<float *>(pk + a.L.kern), a.bf, 0, 1);
        pack_small(a.b1, a.HD, reinterpret_cast<float *>(pk + a.L.b1), a.bf, 0, 1);
        pack_small(a.b2, a.C, reinterpret_cast<float *>(pk + a.L.b2), a.bf, 0, 1);
        pack_small(a.head_w, a.nhw, reinterpret_cast<float *>(pk + a.L.headw), 0, 0, 1);
        pack_small(a.head_b, a.nhb, reinterpret_cast<float *>(pk + a.L.headb), 0, 0, 1);
        pack_small(a.pad_vec, a.C, reinterpret_cast<float *>(pk + a.L.padv), 0, 0, 1);
    } else if (part == 0) {
        pack_frags(a.w1, a.HD, a.F, a.bf, 0, (void *)(pk + a.L.w1), pb, kPB);
    } else if (part == 1) {
        pack_frags(a.w2, a.C, a.HD, a.bf, 0, (void *)(pk + a.L.w2), pb, kPB);
    } else if (part == 2) {
        pack_w2h(a.w2, a.C, a.HD, reinterpret_cast<__bf16 *>(pk + a.L.w2h), pb, kPB);
    } else if (part == 3) {
        pack_frags(a.w1, a.HD, a.F, 1, a.C, (void *)(pk + a.L.w1q), pb, kPB);
    } else {
        pack_w2k(a.w2, a.C, a.HD, reinterpret_cast<__bf16 *>(pk + a.L.w2k), pb, kPB);
    }
}

// ------------------------------------------------------------------------------------------
// Fire mask of one step
__global__ void fire_mask_kernel(int64_t rows, int hw, uint64_t seed, int64_t row0, uint32_t step,
                                 float p, float p_low, float tau, int adaptive, int given_conf,
                                 const float *conf, const uint8_t *given, uint8_t *out) {
    const int nq = (hw + 3) >> 2;
    const int64_t total = rows * nq;
    for (int64_t it = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; it < total;
         it += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = it / nq;
        const int qq = (int)(it - r * nq);
        float u[4];
        nca::cell_uniforms4(seed, (uint32_t)(row0 + r), step, (uint32_t)qq, u);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int q = 4 * qq + e;
            if (q >= hw) break;
            const int64_t cell = r * hw + q;
            float pc = p;
            if (adaptive) {
                const bool confident = conf[cell] > tau || (given_conf && given && given[cell]);
                if (confident) pc = p_low;
            }
            out[cell] = u[e] < pc ? 1 : 0;
        }
    }
}

// ------------------------------------------------------------------------------------------
// Readout: one workgroup per row, cells in chunks of the workgroup size; the board sum runs in
// cell order on one lane so that its rounding matches the sequential definition.
__global__ void readout_kernel(const float *x, int C, int hw, int out_off, int c_out, int n_out,
                               int head_kind, const float *headw, const float *headb,
                               float *conf_cell, float *conf_board, int32_t *argmax) {
    __shared__ float chunk[256];
    const int64_t r = blockIdx.x;
    const float *xr = x + (r * C + out_off) * (int64_t)hw;
    float sum = 0.0f;
    for (int base = 0; base < hw; base += 256) {
        const int q = base + threadIdx.x;
        if (q < hw) {
            int am;
            const float cf = nca::cell_readout(xr + q, hw, c_out, n_out, head_kind, headw, headb, &am);
            if (conf_cell) conf_cell[r * hw + q] = cf;
            if (argmax) argmax[r * hw + q] = am;
            chunk[threadIdx.x] = cf;
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            const int n = hw - base < 256 ? hw - base : 256;
            for (int i = 0; i < n; ++i) sum = __fadd_rn(sum, chunk[i]);
        }
        __syncthreads();
    }
    if (threadIdx.x == 0 && conf_board) conf_board[r] = __fdiv_rn(sum, (float)hw);
}

// ------------------------------------------------------------------------------------------
// conf@K: one wavefront per board; (value, index) pairs reduced across lanes with the
// first-maximum rule (ties -> lower index; NaN counts as the largest, like np.argmax).
__device__ __forceinline__ bool better(float v, int i, float bv, int bi) {
    const bool vn = v != v, bn = bv != bv;
    if (vn != bn) return vn;
    if (!vn && v != bv) return v > bv;
    return i < bi;
}

__global__ void conf_select_kernel(const float *conf, const uint8_t *alive, int N, int K, int k,
                                   int32_t *best) {
    const int wave = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const int lane = threadIdx.x & 63;
    if (wave >= N) return;
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int t = lane; t < k; t += 64) {
        float v = conf[(int64_t)wave * K + t];
        if (alive && !alive[(int64_t)wave * K + t]) v = -INFINITY;
        if (bi == 0x7fffffff || better(v, t, bv, bi)) {
            bv = v;
            bi = t;
        }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const float ov = __shfl_xor(bv, off, 64);
        const int oi = __shfl_xor(bi, off, 64);
        if (oi != 0x7fffffff && (bi == 0x7fffffff || better(ov, oi, bv, bi))) {
            bv = ov;
            bi = oi;
        }
    }
    if (lane == 0) best[wave] = bi == 0x7fffffff ? 0 : bi;
}

// ------------------------------------------------------------------------------------------
// Rollout launch
__global__ void fill_i32(int32_t *p, int64_t n, int32_t v) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        p[i] = v;
}

// Rows per workgroup and LDS plan of the resident kernel; false when one row does not fit.
template <int C, int HD, bool BF16>
bool resident_plan(int64_t rows, int H, int W, int c_in, int c_out, int n_out, int *R_out, nca::LdsPlan *L) {
    int R = (int)((rows + 255) / 256);
    if (R < 1) R = 1;
    if (R > 16) R = 16;
    for (; R >= 1; --R) {
        *L = nca::lds_plan<C, HD, BF16>(R, H, W, c_in, c_out, n_out);
        if (L->total <= kLdsBytes) {
            *R_out = R;
            return true;
        }
    }
    return false;
}

template <int C, int HD>
bool resident_fits(bool bf, int64_t rows, int H, int W, int c_in, int c_out, int n_out) {
    int R;
    nca::LdsPlan L;
    return bf ? resident_plan<C, HD, true>(rows, H, W, c_in, c_out, n_out, &R, &L)
              : resident_plan<C, HD, false>(rows, H, W, c_in, c_out, n_out, &R, &L);
}

// Does the call run on the LDS-resident kernels (true) or the halo-tiled per-step kernel?
bool takes_resident(const nca_cell_desc *d, int64_t rows, int H, int W) {
    if (g_path >= 2) return false;
    const bool bf = d->precision == NCA_BF16;
    const int C = d->channels, HD = d->hidden;
    if (C == 16 && HD == 128) return resident_fits<16, 128>(bf, rows, H, W, d->c_in, d->c_out, d->n_out);
    if (C == 32 && HD == 256) return resident_fits<32, 256>(bf, rows, H, W, d->c_in, d->c_out, d->n_out);
    if (C == 64 && HD == 256) return resident_fits<64, 256>(bf, rows, H, W, d->c_in, d->c_out, d->n_out);
    return false;
}

template <int C, int HD, bool BF16, bool NOISE>
int launch_rollout(nca::RolloutParams p, hipStream_t st) {
    int R = 0;
    nca::LdsPlan L{};
    if (!resident_plan<C, HD, BF16>(p.rows, p.H, p.W, p.c_in, p.c_out, p.n_out, &R, &L))
        return fail(NCA_ERR_UNSUPPORTED,
                    "a %dx%d grid with C=%d does not fit the LDS-resident rollout kernel", p.H, p.W, C);
    p.rows_per_wg = R;
    p.l_P = L.P;
    p.l_M = L.M;
    p.l_Z = L.Z;
    p.l_H = L.H;
    p.l_clamp = L.clamp;
    p.l_given = L.given;
    p.l_fire = L.fire;
    p.l_conf = L.conf;
    p.l_fired = L.fired;
    p.l_head = L.head;
    p.l_cinfo = L.cinfo;
    auto kfn = nca::rollout_resident<C, HD, BF16, NOISE>;
    int rc = hip_check(hipFuncSetAttribute(reinterpret_cast<const void *>(kfn),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)L.total),
                       "hipFuncSetAttribute");
    if (rc) return rc;
    const int64_t grid = (p.rows + R - 1) / R;
    hipLaunchKernelGGL(kfn, dim3((unsigned)grid), dim3(256), L.total, st, p);
    return hip_check(hipGetLastError(), "rollout launch");
}

size_t state_bytes(const nca_cell_desc *d, int64_t rows, int H, int W) {
    return (size_t)rows * d->channels * (size_t)H * W * sizeof(float);
}

bool overlaps(const void *a, size_t na, const void *b, size_t nb) {
    const char *pa = static_cast<const char *>(a), *pb = static_cast<const char *>(b);
    return pa < pb + nb && pb < pa + na;
}

// Steps per launch on the per-step path: T > 1 when the call runs on the temporally blocked
// kernel (bf16 cells with C = 16, uniform firing without a float mask, no noise, two or more
// steps, a window fits), else 1.
int steps_per_launch(const nca_cell_desc *d, int H, int W, int n, bool noise, bool adaptive, bool fire_f32) {
    if (g_path == 2 || g_path == 3) return 1;
    if (d->channels != 16 || d->hidden != 128 || d->precision != NCA_BF16) return 1;
    if (noise || adaptive || fire_f32 || n < 2) return 1;
    int T = g_window_steps > 0 ? g_window_steps : g_path == 4 ? 2 : kDefaultWindowSteps;
    const bool wrap = d->padding == NCA_PAD_WRAP;
    while (T > 1 && (nca::window16_windows(H, T, wrap) < 1 || nca::window16_windows(W, T, wrap) < 1)) --T;
    if (T < 2) return 1;
    return T;
}

// Workspace bytes the per-step path asks for (run_tiled): two state buffers for three or more
// launches, one for two launches or an in-place single launch, none otherwise.
size_t per_step_need(const nca_cell_desc *d, int64_t rows, int H, int W, int n, bool alias, int spl) {
    const size_t sb = state_bytes(d, rows, H, W);
    const int launches = spl > 1 ? (n + spl - 1) / spl : n;
    return launches >= 3 ? 2 * sb : (launches == 2 || (launches == 1 && alias)) ? sb : 0;
}

// The per-step path: launches of one step each (the wave-per-tile or halo-window kernel) or of
// T steps each (the temporally blocked kernel). The first launch reads the caller's NCHW x_in
// and the last writes NCHW x_out; the launches in between alternate between the two halves A, B
// of the workspace in cell-major order. A single launch in place goes through A.
int run_tiled(const nca_cell_desc *d, const nca::RolloutParams &p, hipStream_t st, void *ws, size_t ws_bytes) {
    const size_t sb = state_bytes(d, p.rows, p.H, p.W);
    const int n = p.n_steps;
    const bool alias = p.x_in == p.x_out;
    if (!alias && overlaps(p.x_in, sb, p.x_out, sb))
        return fail(NCA_ERR_INVALID, "x_in and x_out overlap without being the same buffer");
    const int spl = steps_per_launch(d, p.H, p.W, n, p.noise != nullptr, p.adaptive != 0, p.fire_f32 != nullptr);
    const size_t need = per_step_need(d, p.rows, p.H, p.W, n, alias, spl);
    if (need) {
        if (!ws || ws_bytes < need)
            return fail(NCA_ERR_UNSUPPORTED,
                        "a %d-step rollout of a %dx%d grid with C=%d runs step by step and needs a "
                        "workspace of %zu bytes (nca_rollout_workspace_bytes, nca_rollout_ws)",
                        n, p.H, p.W, d->channels, need);
        if (overlaps(ws, need, p.x_in, sb) || overlaps(ws, need, p.x_out, sb))
            return fail(NCA_ERR_INVALID, "the workspace overlaps x_in or x_out");
    }
    if (p.fired_out) {
        hipLaunchKernelGGL(fill_i32, dim3((unsigned)((p.rows + 255) / 256 < 4096 ? (p.rows + 255) / 256 : 4096)),
                           dim3(256), 0, st, p.fired_out, p.rows, 0);
        int rc = hip_check(hipGetLastError(), "fill launch");
        if (rc) return rc;
    }
    float *A = static_cast<float *>(ws);
    float *B = A ? A + sb / sizeof(float) : nullptr;
    if (n == 0) {
        if (!alias) {
            int rc = hip_check(hipMemcpyAsync(p.x_out, p.x_in, sb, hipMemcpyDeviceToDevice, st), "state copy");
            if (rc) return rc;
        }
    } else {
        const float *src = p.x_in;
        const int launches = spl > 1 ? (n + spl - 1) / spl : n;
        for (int l = 0, s = 0; l < launches; ++l) {
            const int k = spl > 1 ? (n - s < spl ? n - s : spl) : 1;  // steps of this launch
            const bool last = l == launches - 1;
            float *dst = last ? (alias && launches == 1 ? A : p.x_out) : ((l & 1) ? B : A);
            nca::RolloutParams q = p;
            q.x_in = src;
            q.x_out = dst;
            q.noise = s == 0 ? p.noise : nullptr;
            if (spl > 1) {
                int rc = hip_check(nca::window16_steps(q, s, k, s == 0, s == 0, last, st), "windowed launch");
                if (rc) return rc;
            } else {
                bool ok = false;
                int rc = hip_check(nca::tiled_step(d->channels, d->hidden, d->precision == NCA_BF16, q, s, s == 0,
                                                   s == 0, last, st, g_path == 3, &ok),
                                   "tiled step launch");
                if (rc) return rc;
                if (!ok)
                    return fail(NCA_ERR_UNSUPPORTED, "no window of a %dx%d grid with C=%d fits the LDS", p.H, p.W,
                                d->channels);
            }
            src = dst;
            s += k;
        }
        if (src != p.x_out) {
            int rc = hip_check(hipMemcpyAsync(p.x_out, src, sb, hipMemcpyDeviceToDevice, st), "state copy");
            if (rc) return rc;
        }
    }
    if (p.conf_out) {
        if (p.rows > 0x7fffffff) return fail(NCA_ERR_UNSUPPORTED, "rows=%lld", (long long)p.rows);
        const float *hw = reinterpret_cast<const float *>(p.packed + p.off_headw);
        const float *hb = reinterpret_cast<const float *>(p.packed + p.off_headb);
        hipLaunchKernelGGL(readout_kernel, dim3((unsigned)p.rows), dim3(256), 0, st, p.x_out, d->channels, p.H * p.W,
                           d->out_offset, d->c_out, d->n_out, d->head_kind, hw, hb, (float *)nullptr, p.conf_out,
                           (int32_t *)nullptr);
        return hip_check(hipGetLastError(), "readout launch");
    }
    return NCA_OK;
}

// bf16 cells with C = 32, hidden 256 on boards up to 31 wide (30x30 hard mazes, also the small
// boards the generic resident kernel takes) run on the streamed C = 32 kernel: one launch for
// the rollout, no workspace. A cell whose output slice spans two channel quads or whose head has
// more than 4 outputs does not (gated firing reads the slice from one quad, the head from registers).
bool takes_stream32(const nca_cell_desc *d, int64_t rows, int H, int W) {
    (void)rows;
    if (g_path != 0 || d->precision != NCA_BF16 || d->channels != 32 || d->hidden != 256) return false;
    if ((d->out_offset & 3) != 0 || d->c_out > 4 || d->n_out > 4) return false;
    return nca::stream32_fits(H, W, d->padding, d->c_out, d->n_out, kLdsBytes);
}

template <int C, int HD>
int launch_cell(const nca_cell_desc *d, const nca::RolloutParams &p, hipStream_t st, void *ws, size_t ws_bytes) {
    const bool bf = d->precision == NCA_BF16;
    if (C == 32 && HD == 256 && takes_stream32(d, p.rows, p.H, p.W)) {
        bool used = false;
        const int rc = hip_check(nca::launch_stream32(p, st, kLdsBytes, &used), "streamed rollout launch");
        if (rc || used) return rc;
    }
    if (!takes_resident(d, p.rows, p.H, p.W)) return run_tiled(d, p, st, ws, ws_bytes);
    if (bf && C == 64 && HD == 256 && g_path == 0) {
        bool used = false;
        const int rc = hip_check(nca::launch_stream64(p, st, kLdsBytes, &used), "streamed rollout launch");
        if (rc || used) return rc;
    }
    if (p.noise)
        return bf ? launch_rollout<C, HD, true, true>(p, st) : launch_rollout<C, HD, false, true>(p, st);
    return bf ? launch_rollout<C, HD, true, false>(p, st) : launch_rollout<C, HD, false, false>(p, st);
}

int dispatch_rollout(const nca_cell_desc *d, const nca::RolloutParams &p, hipStream_t st, void *ws = nullptr,
                     size_t ws_bytes = 0) {
    if (d->channels == 16 && d->hidden == 128) return launch_cell<16, 128>(d, p, st, ws, ws_bytes);
    if (d->channels == 32 && d->hidden == 256) return launch_cell<32, 256>(d, p, st, ws, ws_bytes);
    if (d->channels == 64 && d->hidden == 256) return launch_cell<64, 256>(d, p, st, ws, ws_bytes);
    return fail(NCA_ERR_UNSUPPORTED, "cell C=%d hidden=%d", d->channels, d->hidden);
}

nca::RolloutParams base_params(const nca_cell_desc *d, const void *packed, int64_t rows, int H,
                               int W) {
    nca::RolloutParams p;
    memset(&p, 0, sizeof(p));
    const nca::PackedLayout L = layout_of(d);
    p.packed = static_cast<const unsigned char *>(packed);
    p.rows = rows;
    p.H = H;
    p.W = W;
    p.c_in = d->c_in;
    p.in_off = d->in_offset;
    p.c_out = d->c_out;
    p.out_off = d->out_offset;
    p.n_out = d->n_out;
    p.head_kind = d->head_kind;
    p.padding = d->padding;
    p.off_kern = (unsigned)L.kern;
    p.off_b1 = (unsigned)L.b1;
    p.off_b2 = (unsigned)L.b2;
    p.off_headw = (unsigned)L.headw;
    p.off_headb = (unsigned)L.headb;
    p.off_padv = (unsigned)L.padv;
    p.off_w1 = (unsigned)L.w1;
    p.off_w2 = (unsigned)L.w2;
    p.off_w2h = (unsigned)L.w2h;
    p.off_w1q = (unsigned)L.w1q;
    p.off_w2k = (unsigned)L.w2k;
    return p;
}

int check_grid(int64_t rows, int H, int W) {
    if (rows < 0 || H < 1 || W < 1) return fail(NCA_ERR_INVALID, "rows=%lld H=%d W=%d", (long long)rows, H, W);
    if ((int64_t)H * W > (1 << 24)) return fail(NCA_ERR_UNSUPPORTED, "grid %dx%d too large", H, W);
    return NCA_OK;
}

}  // namespace

namespace nca {

// CUs of the current device (cached per device)
int device_cus();

namespace {

int recorded_pieces(const nca_cell_desc *cell, int64_t rows, int H, int W);

}  // namespace

int device_cus() {
    static int cus[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
    if (cus[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n < 1) return 0;
        cus[dev] = n;
    }
    return cus[dev];
}

namespace {

int recorded_pieces(const nca_cell_desc *cell, int64_t rows, int H, int W) {
    return nca::stream32_pieces(rows, H, W, cell->c_out, cell->n_out, kLdsBytes, device_cus());
}

}  // namespace

size_t recorded_xch_bytes(const nca_cell_desc *cell, int64_t rows, int H, int W) {
    if (check_cell(cell) || check_grid(rows, H, W) || !takes_stream32(cell, rows, H, W)) {
        g_err[0] = 0;
        return 0;
    }
    return nca::stream32_xch_bytes(rows, recorded_pieces(cell, rows, H, W), W);
}

int rollout_recorded(const nca_cell_desc *cell, const void *packed, int64_t rows, int H, int W, const float *x_in,
                     const uint8_t *given, const float *clamp, float *x_out, const nca_fire_desc *fire, int n_steps,
                     float *x_rec, int64_t rec_stride, hipStream_t st, bool *used, void *xch, size_t xch_bytes,
                     int *pieces, float *x_rec0) {
    *used = false;
    if (pieces) *pieces = 1;
    // anything the checks of nca_rollout_ws would refuse is left to the caller's fallback
    if (check_cell(cell) || check_grid(rows, H, W)) {
        g_err[0] = 0;
        return NCA_OK;
    }
    if (!packed || !x_in || !given || (!clamp && cell->c_in > 0) || !x_out || !x_rec) return NCA_OK;
    if (fire->adaptive || rows < 1 || n_steps < 1 || !takes_stream32(cell, rows, H, W)) return NCA_OK;
    nca::RolloutParams p = base_params(cell, packed, rows, H, W);
    p.x_in = x_in;
    p.x_out = x_out;
    p.given = given;
    p.clamp = clamp;
    p.fire_u8 = fire->fire_in;
    p.step_seeds = fire->step_seeds;
    p.seed = fire->seed;
    p.row0 = fire->row0;
    p.step0 = fire->step0;
    p.n_steps = n_steps;
    p.p = fire->p_fire;
    p.p_low = fire->p_low;
    p.tau = fire->tau;
    p.x_rec = x_rec;
    p.rec_stride = rec_stride;
    p.x_rec0 = x_rec0;
    int P = xch ? recorded_pieces(cell, rows, H, W) : 1;
    if (P > 1 && xch_bytes < nca::stream32_xch_bytes(rows, P, W)) P = 1;
    const int rc = hip_check(nca::launch_stream32(p, st, kLdsBytes, used, P, static_cast<uint64_t *>(xch)),
                             "streamed rollout launch");
    if (pieces && *used) *pieces = P;
    return rc;
}

}  // namespace nca

// ------------------------------------------------------------------------------------------
// The allocation-free entry point's scratch: the per-step path's state buffers in a device
// array of the library's code object, so that every GPU the library runs on holds its own copy
// until the process ends. Host code never passes `scratch` itself to a kernel (on the host it is
// only a stand-in for the symbol): it looks up each device's address once, on that device's
// first call, and passes that.
static __device__ __align__(256) unsigned char scratch[NCA_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices] = {};

// The current device's address of `scratch`.
int scratch_address(void **out) {
    int dev = 0;
    int rc = hip_check(hipGetDevice(&dev), "hipGetDevice");
    if (rc) return rc;
    if (dev < 0 || dev >= kMaxDevices) return fail(NCA_ERR_UNSUPPORTED, "device %d (0..%d)", dev, kMaxDevices - 1);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        rc = hip_check(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
        if (rc) return rc;
        if (!p) return fail(NCA_ERR_HIP, "hipGetSymbolAddress(scratch) returned NULL");
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return NCA_OK;
}

}  // namespace

extern "C" {

const char *nca_last_error(void) { return g_err; }

int nca_version(void) { return 100; }

int nca_set_kernel_path(int path) {
    if (path < 0 || path > 4)
        return fail(NCA_ERR_INVALID, "path=%d (0 auto, 1 generic, 2 per-step, 3 halo-window, 4 temporal blocking)",
                    path);
    g_path = path;
    return NCA_OK;
}

int nca_set_piece_debug(int32_t spin_limit, int32_t force_timeout, int32_t plan_cus) {
    if (spin_limit < 0 || plan_cus < 0) return fail(NCA_ERR_INVALID, "spin_limit >= 0, plan_cus >= 0");
    nca::g_piece_debug.spin_limit = spin_limit;
    nca::g_piece_debug.force_timeout = force_timeout ? 1 : 0;
    nca::g_piece_debug.plan_cus = plan_cus;
    return NCA_OK;
}

int nca_set_bptt_backward_path(int32_t path) {
    if (path < 0 || path > 2) return fail(NCA_ERR_INVALID, "path=%d (0 automatic, 1 per-step launches, 2 whole boards)", path);
    nca::g_piece_debug.back_path = path;
    return NCA_OK;
}

int32_t nca_bptt_forward_pieces(const nca_cell_desc *cell, int64_t rows, int32_t height, int32_t width,
                                int32_t cus) {
    g_err[0] = 0;
    if (check_cell(cell) || check_grid(rows, height, width)) return 0;
    if (!takes_stream32(cell, rows, height, width)) return 1;
    return nca::stream32_pieces(rows, height, width, cell->c_out, cell->n_out, kLdsBytes,
                                cus > 0 ? cus : nca::device_cus());
}

int nca_set_window_steps(int steps) {
    if (steps < 0 || steps > nca::kWinMaxT) return fail(NCA_ERR_INVALID, "steps=%d (0 automatic, 1..%d)", steps, nca::kWinMaxT);
    g_window_steps = steps;
    return NCA_OK;
}

size_t nca_rollout_workspace_bytes(const nca_cell_desc *cell, int64_t rows, int32_t height, int32_t width) {
    if (check_cell(cell) || check_grid(rows, height, width)) return 0;
    if (takes_resident(cell, rows, height, width) || takes_stream32(cell, rows, height, width)) return 0;
    return 2 * state_bytes(cell, rows, height, width);
}

size_t nca_packed_weights_bytes(const nca_cell_desc *cell) {
    if (check_cell(cell)) return 0;
    return layout_of(cell).total;
}

int nca_pack_weights(const nca_cell_desc *cell, const nca_cell_weights *w, void *packed, void *stream) {
    g_err[0] = 0;
    int rc = check_cell(cell);
    if (rc) return rc;
    if (!w || !w->kernels || !w->w1 || !w->b1 || !w->w2 || !w->b2 || !w->head_w || !packed)
        return fail(NCA_ERR_INVALID, "NULL weight pointer");
    if (cell->head_kind == NCA_HEAD_MLP && !w->head_b) return fail(NCA_ERR_INVALID, "mlp head needs head_b");
    if (cell->padding == NCA_PAD_WALL && !w->pad_vec) return fail(NCA_ERR_INVALID, "wall padding needs pad_vec");
    const nca::PackedLayout L = layout_of(cell);
    const bool bf = cell->precision == NCA_BF16;
    hipStream_t st = as_stream(stream);
    unsigned char *pk = static_cast<unsigned char *>(packed);
    const int C = cell->channels, HD = cell->hidden, F = cell->heads * C;
    PackArgs pa;
    memset(&pa, 0, sizeof(pa));
    pa.kernels = w->kernels;
    pa.w1 = w->w1;
    pa.b1 = w->b1;
    pa.w2 = w->w2;
    pa.b2 = w->b2;
    pa.head_w = w->head_w;
    pa.head_b = w->head_b;
    pa.pad_vec = w->pad_vec;
    pa.nk = cell->heads * 9;
    pa.HD = HD;
    pa.C = C;
    pa.F = F;
    pa.nhw = cell->n_out * cell->c_out;
    pa.nhb = cell->n_out;
    pa.bf = bf ? 1 : 0;
    pa.pk = pk;
    pa.L = L;
    hipLaunchKernelGGL(pack_all, dim3((bf ? 5 : 2) * 64 + 1), dim3(256), 0, st, pa);
    return hip_check(hipGetLastError(), "pack launch");
}

int nca_rollout_ws(const nca_cell_desc *cell, const void *packed, int64_t rows, int32_t height,
                   int32_t width, const float *x_in, const uint8_t *given, const float *clamp,
                   float *x_out, const nca_fire_desc *fire, int32_t n_steps, const float *noise,
                   float *conf_out, int32_t *fired_out, void *workspace, size_t workspace_bytes,
                   void *stream) {
    g_err[0] = 0;
    int rc = check_cell(cell);
    if (rc) return rc;
    if ((rc = check_grid(rows, height, width))) return rc;
    if (rows == 0) return NCA_OK;
    if (!packed || !x_in || !given || (!clamp && cell->c_in > 0) || !x_out || !fire)
        return fail(NCA_ERR_INVALID, "NULL pointer argument");
    if (n_steps < 0) return fail(NCA_ERR_INVALID, "n_steps=%d", n_steps);
    if (noise && n_steps != 1) return fail(NCA_ERR_INVALID, "noise needs n_steps == 1");
    if (fire->adaptive && fire->fire_in) return fail(NCA_ERR_INVALID, "adaptive firing with injected masks");
    nca::RolloutParams p = base_params(cell, packed, rows, height, width);
    p.x_in = x_in;
    p.x_out = x_out;
    p.given = given;
    p.clamp = clamp;
    p.fire_u8 = fire->fire_in;
    p.noise = noise;
    p.step_seeds = fire->step_seeds;
    p.conf_out = conf_out;
    p.fired_out = fired_out;
    p.seed = fire->seed;
    p.row0 = fire->row0;
    p.step0 = fire->step0;
    p.n_steps = n_steps;
    p.p = fire->p_fire;
    p.p_low = fire->p_low;
    p.tau = fire->tau;
    p.adaptive = fire->adaptive;
    p.given_confident = fire->given_confident;
    return dispatch_rollout(cell, p, as_stream(stream), workspace, workspace_bytes);
}

int nca_rollout_noalloc(const nca_cell_desc *cell, const void *packed, int64_t rows, int32_t height,
                        int32_t width, const float *x_in, const uint8_t *given, const float *clamp,
                        float *x_out, const nca_fire_desc *fire, int32_t n_steps, const float *noise,
                        float *conf_out, int32_t *fired_out, void *stream) {
    g_err[0] = 0;
    int rc = check_cell(cell);
    if (rc) return rc;
    if ((rc = check_grid(rows, height, width))) return rc;
    if (n_steps < 0) return fail(NCA_ERR_INVALID, "n_steps=%d", n_steps);
    // the per-step path's workspace must fit the scratch (the other paths need none)
    if (nca_rollout_workspace_bytes(cell, rows, height, width) > 0) {
        const int spl = steps_per_launch(cell, height, width, n_steps, noise != nullptr, fire && fire->adaptive,
                                         false);
        const size_t need = per_step_need(cell, rows, height, width, n_steps, x_in == x_out, spl);
        if (need > NCA_NOALLOC_SCRATCH_BYTES)
            return fail(NCA_ERR_UNSUPPORTED,
                        "this call needs %zu bytes of workspace, above the %zu-byte scratch of "
                        "nca_rollout_noalloc (use nca_rollout_ws)",
                        need, (size_t)NCA_NOALLOC_SCRATCH_BYTES);
    }
    void *ws = nullptr;
    if ((rc = scratch_address(&ws))) return rc;
    return nca_rollout_ws(cell, packed, rows, height, width, x_in, given, clamp, x_out, fire, n_steps, noise,
                          conf_out, fired_out, ws, NCA_NOALLOC_SCRATCH_BYTES, stream);
}

int nca_rollout(const nca_cell_desc *cell, const void *packed, int64_t rows, int32_t height,
                int32_t width, const float *x_in, const uint8_t *given, const float *clamp,
                float *x_out, const nca_fire_desc *fire, int32_t n_steps, const float *noise,
                float *conf_out, int32_t *fired_out, void *stream) {
    return nca_rollout_ws(cell, packed, rows, height, width, x_in, given, clamp, x_out, fire, n_steps, noise,
                          conf_out, fired_out, nullptr, 0, stream);
}

int nca_step(const nca_cell_desc *cell, const void *packed, int64_t rows, int32_t height,
             int32_t width, const float *x, const uint8_t *given, const float *clamp,
             const float *fire, const float *noise, float *x_out, void *stream) {
    g_err[0] = 0;
    int rc = check_cell(cell);
    if (rc) return rc;
    if ((rc = check_grid(rows, height, width))) return rc;
    if (rows == 0) return NCA_OK;
    if (!packed || !x || !given || (!clamp && cell->c_in > 0) || !fire || !x_out)
        return fail(NCA_ERR_INVALID, "NULL pointer argument");
    nca::RolloutParams p = base_params(cell, packed, rows, height, width);
    p.x_in = x;
    p.x_out = x_out;
    p.given = given;
    p.clamp = clamp;
    p.fire_f32 = fire;
    p.noise = noise;
    p.n_steps = 1;
    return dispatch_rollout(cell, p, as_stream(stream));
}

int nca_fire_mask(int64_t rows, int32_t height, int32_t width, const nca_fire_desc *fire,
                  int64_t step, const float *conf_cell, const uint8_t *given, uint8_t *out,
                  void *stream) {
    g_err[0] = 0;
    int rc = check_grid(rows, height, width);
    if (rc) return rc;
    if (!fire || !out) return fail(NCA_ERR_INVALID, "NULL pointer argument");
    if (fire->adaptive && !conf_cell) return fail(NCA_ERR_INVALID, "adaptive firing needs conf_cell");
    if (rows == 0) return NCA_OK;
    const int hw = height * width;
    const int64_t items = rows * ((hw + 3) / 4);
    const int blocks = (int)((items + 255) / 256 < 65536 ? (items + 255) / 256 : 65536);
    hipLaunchKernelGGL(fire_mask_kernel, dim3(blocks), dim3(256), 0, as_stream(stream), rows, hw,
                       fire->seed, fire->row0, (uint32_t)step, fire->p_fire, fire->p_low, fire->tau,
                       fire->adaptive, fire->given_confident, conf_cell, given, out);
    return hip_check(hipGetLastError(), "fire mask launch");
}

int nca_readout(const nca_cell_desc *cell, const void *packed, int64_t rows, int32_t height,
                int32_t width, const float *x, float *conf_cell, float *conf_board,
                int32_t *argmax, void *stream) {
    g_err[0] = 0;
    int rc = check_cell(cell);
    if (rc) return rc;
    if ((rc = check_grid(rows, height, width))) return rc;
    if (!packed || !x) return fail(NCA_ERR_INVALID, "NULL pointer argument");
    if (rows == 0) return NCA_OK;
    if (rows > 0x7fffffff) return fail(NCA_ERR_UNSUPPORTED, "rows=%lld", (long long)rows);
    const nca::PackedLayout L = layout_of(cell);
    const unsigned char *pk = static_cast<const unsigned char *>(packed);
    hipLaunchKernelGGL(readout_kernel, dim3((unsigned)rows), dim3(256), 0, as_stream(stream), x,
                       cell->channels, height * width, cell->out_offset, cell->c_out, cell->n_out,
                       cell->head_kind, reinterpret_cast<const float *>(pk + L.headw),
                       reinterpret_cast<const float *>(pk + L.headb), conf_cell, conf_board, argmax);
    return hip_check(hipGetLastError(), "readout launch");
}

int nca_conf_select(const float *conf, const uint8_t *alive, int32_t n_boards, int32_t k_trials,
                    int32_t k, int32_t *best, void *stream) {
    g_err[0] = 0;
    if (!conf || !best) return fail(NCA_ERR_INVALID, "NULL pointer argument");
    if (n_boards < 0 || k_trials < 1 || k < 1)
        return fail(NCA_ERR_INVALID, "N=%d K=%d k=%d", n_boards, k_trials, k);
    if (n_boards == 0) return NCA_OK;
    if (k > k_trials) k = k_trials;
    const int64_t threads = (int64_t)n_boards * 64;
    hipLaunchKernelGGL(conf_select_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0,
                       as_stream(stream), conf, alive, n_boards, k_trials, k, best);
    return hip_check(hipGetLastError(), "conf select launch");
}

}  // extern "C"
