// BPTT of an NCA chunk on gfx950 (nca_bptt_forward / nca_bptt_backward, include/nca_hip.h).
//
// Forward: the chunk's steps run on the rollout kernels one step per call, and every state of
// the chunk is kept (n + 1 states); nothing else is stored. Backward: the steps are walked in
// reverse; each step recomputes its perception z and hidden activation h from the saved state
// (the forward's rounding points for bf16 cells) instead of reading stored activations:
//
//   front      per cell: the loss gradient of the step's output state (cross-entropy of the
//              mlp head's logits, reference src/nca/train.py:183-207, weighted as in
//              src/nca/engine/step.py:243-245 and normalised as in engine.py:490), plus the
//              gradient arriving from the next step; the clamp's backward zeroes the input
//              slice of given cells (ops.py:276-294): g_u; the fire mask gives g_dx = g_u * fire;
//              partial sums of db2, the head's gradients and the loss
//   stencil_z  z = perception of the saved state (feature-major, F x cells)
//   MLP        h = relu(W1 z + b1); g_a = (W2^T g_dx) * [h > 0]; g_z = W1^T g_a: bf16 cells with
//              32 channels and 256 hidden units in one fused kernel (mlp_back32, which also sums
//              dW1, dW2 and db1, and stores g_z as bf16), other cells on fp32 MFMA GEMMs
//   stencil_back  g_x = g_u + the transposed stencil of g_z (padding-aware: wall / zero halos
//              take no gradient, wrap halos give it to the wrapped cell), the next step's
//              gradient, and partial sums of the kernel-weight gradient
//   partials   dW1 = g_a z^T, dW2 = g_dx h^T (split-K GEMMs), db1 (row sums of g_a), unless fused
//
// Every partial sum belongs to one of 256 fixed cell ranges (slots); each step adds its sums
// into the slots, and one kernel adds the slots up in slot order after the last step, so the
// gradients are deterministic (the same bits on every run). fp32 cells: the exact fp32
// gradients of the forward as computed. bf16 cells: the rounding points are straight-through
// (derivative 1), the backward uses the forward's bf16-rounded weights and inputs, and the
// gradients of dx, of fc1's output and of z are rounded to bf16 where the reference's bf16
// backward rounds them (they are gradients of bf16 tensors; src/nca/engine/triton_mlp.py:46-78),
// which makes every MLP product of the backward a product of bf16 values.
#include <hip/hip_runtime.h>

#include <math.h>
#include <stdio.h>
#include <string.h>

#include "nca_hip.h"
#include "nca_bptt_mlp.h"
#include "nca_device.h"
#include "nca_layout.h"
#include "nca_status.h"
#include "nca_stream.h"

namespace {

constexpr int kSplit = 256;  // cell ranges of the split-K weight-gradient sums
constexpr int kThreads = 256;
constexpr int kPlaneMax = 2048;  // cells of a board whose planes the LDS stencil kernels stage

struct Dims {
    int C, F, HD, c_in, in_off, c_out, out_off, n_out, padding, bf16;
    int gz16;  // g_z is stored as bf16 (by the fused MLP backward), else fp32
    int H, W, HW;
    int64_t rows, M;  // M = rows * HW cells
};

// Offsets (floats) of every gradient in one flat parameter vector: kernels, w1, b1, w2, b2,
// head_w, head_b.
struct ParamLayout {
    int64_t K, W1, B1, W2, B2, HW, HB, P;
};

ParamLayout param_layout(const Dims &d) {
    ParamLayout L;
    int64_t o = 0;
    L.K = o;
    o += 4 * 9;
    L.W1 = o;
    o += (int64_t)d.HD * d.F;
    L.B1 = o;
    o += d.HD;
    L.W2 = o;
    o += (int64_t)d.C * d.HD;
    L.B2 = o;
    o += d.C;
    L.HW = o;
    o += (int64_t)d.n_out * d.c_out;
    L.HB = o;
    o += d.n_out;
    L.P = o;
    return L;
}

// The fused MLP backward (mlp_back32) takes bf16 cells of 32 channels, 128 features and 256 hidden
// units; it addresses z and g_z with 32-bit byte offsets.
bool fused_mlp(const Dims &d) { return d.bf16 && d.C == 32 && d.F == 128 && d.HD == 256 && d.M * d.F * 4 < ((int64_t)1 << 32); }
// Boards small enough to stage (row, channel) planes in LDS.
bool planes_fit(const Dims &d) { return d.HW <= kPlaneMax && d.rows * d.C <= 0x7fffffff; }

// Workspace (floats, 64-float aligned pieces, after the status block). part holds kSplit slots of P partial sums
// each (slot s: the cells of range s), added to by every step of the chunk and reduced once at
// the end; lossacc holds the loss's kSplit slots. The GEMM path's h and g_a (Hb, Ga) are not
// needed by the fused kernel.
struct WsLayout {
    int64_t Z, Hb, Ga, Gz, Gdx, Gu, Gx0, Gx1, part, acc, lossacc, dk, denom, img, total;
};

WsLayout ws_layout(const Dims &d, int n) {
    (void)n;
    const ParamLayout P = param_layout(d);
    const bool fused = fused_mlp(d);
    auto al = [](int64_t v) { return (v + 63) & ~(int64_t)63; };
    WsLayout L;
    // the first kXchStatusBytes hold the status words of the forward's and the one-launch
    // backward's pieces; nothing else writes them
    int64_t o = (int64_t)(nca::kXchStatusBytes / sizeof(float));
    L.Z = o;
    o = al(o + (int64_t)d.F * d.M);
    L.Hb = o;
    o = al(o + (fused ? 0 : (int64_t)d.HD * d.M));
    L.Ga = o;
    o = al(o + (fused ? 0 : (int64_t)d.HD * d.M));
    L.Gz = o;
    o = al(o + (int64_t)d.F * d.M);
    L.Gdx = o;
    o = al(o + (int64_t)d.C * d.M);
    L.Gu = o;
    o = al(o + (int64_t)d.C * d.M);
    L.Gx0 = o;
    o = al(o + (int64_t)d.C * d.M);
    L.Gx1 = o;
    o = al(o + (int64_t)d.C * d.M);
    L.part = o;
    o = al(o + (int64_t)kSplit * P.P);
    L.acc = o;
    o = al(o + P.P);
    L.lossacc = o;
    o = al(o + kSplit);
    L.dk = o;  // kernel-weight slots of the plane kernels, one per (row, channel)
    o = al(o + (d.HW <= kPlaneMax ? d.rows * d.C * 36 : 0));
    L.denom = o;
    o = al(o + 1);
    L.img = o;  // weight image of the fused MLP backward
    o = al(o + nca::Mb32::IMG_BYTES / 4);
    L.total = o;
    return L;
}

// The neighbour of cell (i, j) at (i + dy, j + dx), |dy|, |dx| <= 1: its cell index, or -1 for a
// constant halo cell (wall / zero padding); wrap padding wraps around (reference
// src/nca/model.py:140-152). Selects only: the kernels load at every tap without a branch, so the
// loads of a thread are all in flight together.
__device__ __forceinline__ int neighbour(int i, int j, int dy, int dx, int H, int W, int padding) {
    int a = i + dy, b = j + dx;
    const bool in = a >= 0 && a < H && b >= 0 && b < W;
    const bool wrap = padding == 2;
    a = a < 0 ? H - 1 : (a >= H ? 0 : a);
    b = b < 0 ? W - 1 : (b >= W ? 0 : b);
    return (in || wrap) ? a * W + b : -1;
}

// Element i of g_z: fp32, or bf16 where the fused MLP backward wrote it (gz16).
__device__ __forceinline__ float gz_at(const float *Gz, int gz16, int64_t i) {
    return gz16 ? __uint_as_float((uint32_t)reinterpret_cast<const uint16_t *>(Gz)[i] << 16) : Gz[i];
}

// Block-wide sum of one float per thread in a fixed tree order (deterministic).
__device__ float block_sum(float v, float *red) {
    const int t = threadIdx.x;
    red[t] = v;
    __syncthreads();
    for (int s = kThreads / 2; s > 0; s >>= 1) {
        if (t < s) red[t] = __fadd_rn(red[t], red[t + s]);
        __syncthreads();
    }
    const float r = red[0];
    __syncthreads();
    return r;
}

// the value of the lane that DPP control CTRL selects (no LDS traffic)
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float x) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), CTRL, 0xf, 0xf, false));
}

// Block-wide sums of N floats per thread over a block of WAVES waves: each wave folds its lanes
// in a fixed order of symmetric pairings (both partners of an exchange add the same two values,
// so every lane ends with the same bits), then thread i < N adds the waves' totals in wave order.
// Returns the block total of v[i] in thread i (0 in threads >= N); red holds WAVES * N floats.
template <int N, int WAVES>
__device__ float block_sums(const float (&v)[N], float *red) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int i = 0; i < N; ++i) {
        float x = v[i];
        // lanes paired with lane ^ 1, ^ 2 (quad_perm), 7 - i and 15 - i within the row (half mirror,
        // mirror: by then the 4 lanes of a quad, and the 8 of a half row, hold the same value),
        // then ^ 16 and ^ 32: partners add the same two values, so every lane ends with the same bits
        x = __fadd_rn(x, dpp_f32<0xb1>(x));   // quad_perm [1, 0, 3, 2]
        x = __fadd_rn(x, dpp_f32<0x4e>(x));   // quad_perm [2, 3, 0, 1]
        x = __fadd_rn(x, dpp_f32<0x141>(x));  // row_half_mirror
        x = __fadd_rn(x, dpp_f32<0x140>(x));  // row_mirror
        x = __fadd_rn(x, __shfl_xor(x, 16));
        x = __fadd_rn(x, __shfl_xor(x, 32));
        if (lane == 0) red[wave * N + i] = x;
    }
    __syncthreads();
    float r = 0.0f;
    if (threadIdx.x < N) {
        r = red[threadIdx.x];
#pragma unroll
        for (int w = 1; w < WAVES; ++w) r = __fadd_rn(r, red[w * N + threadIdx.x]);
    }
    __syncthreads();
    return r;
}

// two ranges cleared in one launch: n floats at p and m 8-byte words at q
__global__ void zero_f32_words(float *p, int64_t n, uint64_t *q, int64_t m) {
    const int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x, stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = t; i < n; i += stride) p[i] = 0.0f;
    for (int64_t i = t; i < m; i += stride) q[i] = 0;
}

// the one-launch backward's set-up: blocks below kMb32PrepBlocks build mlp_back32_prep's weight
// image, the others clear m 8-byte words at q (the status word and exchange slots of its pieces)
// and the n1 and n2 floats at p1 and p2 (the partial-sum and loss slots no workgroup writes)
constexpr int kPrepClearBlocks = 238;
__global__ void __launch_bounds__(512) prep_clear_kernel(const float *w1, const float *w2, unsigned char *img,
                                                         uint64_t *q, int64_t m, float *p1, int64_t n1, float *p2,
                                                         int64_t n2) {
    if ((int)blockIdx.x < nca::kMb32PrepBlocks) {
        nca::mb32_prep_fragment(blockIdx.x, w1, w2, img);
        return;
    }
    const int64_t t = (blockIdx.x - nca::kMb32PrepBlocks) * (int64_t)blockDim.x + threadIdx.x;
    const int64_t stride = (int64_t)(gridDim.x - nca::kMb32PrepBlocks) * blockDim.x;
    // the words with 16-byte stores from the first 16-byte boundary (a leading and a trailing
    // odd word with 8-byte ones)
    const int64_t head = (reinterpret_cast<uintptr_t>(q) & 15u) ? 1 : 0;
    const int64_t np = m > head ? (m - head) / 2 : 0;
    if (t == 0 && head && m > 0) q[0] = 0;
    if (t == 0 && m > head + 2 * np) q[m - 1] = 0;
    uint4 *qp = reinterpret_cast<uint4 *>(q + head);
    for (int64_t i = t; i < np; i += stride) qp[i] = make_uint4(0u, 0u, 0u, 0u);
    for (int64_t i = t; i < n1; i += stride) p1[i] = 0.0f;
    for (int64_t i = t; i < n2; i += stride) p2[i] = 0.0f;
}

__global__ void zero_f32(float *p, int64_t n) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        p[i] = 0.0f;
}

// denom = max(sum of the loss mask, 1) in a fixed order (train.py:204-205).
__global__ void mask_sum(const float *mask, int64_t n, float *out) {
    __shared__ float red[kThreads];
    float s = 0.0f;
    for (int64_t i = threadIdx.x; i < n; i += kThreads) s = __fadd_rn(s, mask[i]);
    s = block_sum(s, red);
    if (threadIdx.x == 0) *out = s < 1.0f ? 1.0f : s;
}

struct FrontArgs {
    Dims d;
    const float *x1;        // the step's output state (rows, C, H, W)
    const float *gin;       // gradient w.r.t. x1 from the later steps, or null
    const uint8_t *given;   // (rows, HW)
    const int32_t *targets;  // (rows, HW)
    const float *mask;      // (rows, HW) or null
    const float *denom;     // device scalar: max(sum(mask), 1), used with mask
    float wscale;           // w_t / sum(w) (/ M without a mask); 0: the step has no loss term
    const float *head_w, *head_b;
    // fire mask of the step
    const uint8_t *fire_u8;  // (rows, HW) slice of the injected masks, or null
    const float *fire_f32;   // (rows, HW) fire values of a single step's VJP (any real value), or null
    const uint64_t *key_ptr;  // per-step Philox key (device), or null: key
    uint64_t key;
    int64_t row0;
    uint32_t step;
    float p;
    float *Gu, *Gdx;
    float *part, *lossacc;  // partial-sum slots (db2, dhead) and the loss's slots
    int64_t P, offB2, offHW, offHB;
};

// The output channels of a cell (x1c: channel 0 of the cell in the step's output state), loaded
// without a branch: xo[c] for c < c_out (<= NO), 0 beyond.
template <int NO>
__device__ __forceinline__ void load_out(const Dims &d, const float *x1c, float xo[NO]) {
    float v[NO];
#pragma unroll
    for (int c = 0; c < NO; ++c) v[c] = x1c[(int64_t)(d.out_off + (c < d.c_out ? c : 0)) * d.HW];
#pragma unroll
    for (int c = 0; c < NO; ++c) xo[c] = c < d.c_out ? v[c] : 0.0f;
}

// The cross-entropy gradient of the mlp head's logits at a cell with output channels xo, target
// tgt and loss-mask value mk (gl[v] = d loss / d logit v, times the step's scale; 0 for
// v >= n_out, and everywhere on a step without a loss term) and the cell's loss term (reference
// src/nca/train.py:183-207). n_out, c_out <= NO.
template <int NO>
__device__ __forceinline__ float head_grad_core(const Dims &d, float wscale, bool masked, const float *denom,
                                                const float *hw, const float *hb, const float xo[NO], int tgt, float mk,
                                                float gl[NO]) {
#pragma unroll
    for (int v = 0; v < NO; ++v) gl[v] = 0.0f;
    if (wscale == 0.0f) return 0.0f;
    const float scale = masked ? wscale * mk / *denom : wscale;
    float l[NO];
    float mx = -INFINITY;
#pragma unroll
    for (int v = 0; v < NO; ++v) {
        l[v] = 0.0f;
        if (v < d.n_out) {
            float acc = hb[v];
#pragma unroll
            for (int c = 0; c < NO; ++c)
                if (c < d.c_out) acc = __builtin_fmaf(hw[v * d.c_out + c], xo[c], acc);
            l[v] = acc;
            mx = fmaxf(mx, acc);
        }
    }
    float s = 0.0f, lt = mx, e[NO];
#pragma unroll
    for (int v = 0; v < NO; ++v)
        if (v < d.n_out) {
            e[v] = expf(l[v] - mx);
            s += e[v];
            if (v == tgt) lt = l[v];
        }
#pragma unroll
    for (int v = 0; v < NO; ++v)
        if (v < d.n_out) gl[v] = (e[v] / s - (v == tgt ? 1.0f : 0.0f)) * scale;
    return (mx + logf(s) - lt) * scale;
}
template <int NO>
__device__ __forceinline__ float head_grad(const FrontArgs &a, const float *hw, const float *hb, const float xo[NO], int tgt,
                                           float mk, float gl[NO]) {
    return head_grad_core<NO>(a.d, a.wscale, a.mask != nullptr, a.denom, hw, hb, xo, tgt, mk, gl);
}

constexpr int kFrontCh = 8;  // channels per front block (the channel count is a multiple of 8)

// Per cell of range blockIdx.x, channels [8 blockIdx.y, 8 blockIdx.y + 8): the loss gradient of
// the step's output state plus the gradient from the later steps; the clamp's backward zeroes
// the input slice of given cells (reference src/nca/engine/ops.py:276-294): g_u; the fire mask
// gives g_dx = g_u * fire. The block adds its sums of g_dx (db2) into its slot; the blocks of
// channel group 0 also add the loss and the head's weight / bias gradients. Every load of a cell
// is issued before its arithmetic. n_out, c_out <= NO.
// The front of cell range s, channel group cg (one workgroup): red and hwL in LDS.
template <int NO>
__device__ void front_body(const FrontArgs &a, int s, int cg, float *red, float *hwL) {
    const Dims &d = a.d;
    for (int i = threadIdx.x; i < d.n_out * d.c_out; i += kThreads) hwL[i] = a.head_w[i];
    for (int i = threadIdx.x; i < d.n_out; i += kThreads) hwL[NO * NO + i] = a.head_b[i];
    __syncthreads();
    const int c0 = kFrontCh * cg;
    const int per = (int)((d.M + kSplit - 1) / kSplit), m0 = s * per;
    const int m1 = m0 + per < (int)d.M ? m0 + per : (int)d.M;
    const bool head = cg == 0;
    // small heads (n_out, c_out <= 4): the head's gradient sums kept in registers, hs[v NO + c] of
    // g_l[v] x1[out_off + c] and hs[NO NO + v] of g_l[v]
    constexpr bool kRegHead = NO <= 4;
    constexpr int NP = NO * NO + NO;
    float hs[kRegHead ? NP : 1];
#pragma unroll
    for (int p = 0; p < (kRegHead ? NP : 1); ++p) hs[p] = 0.0f;
    float db2[kFrontCh];
#pragma unroll
    for (int j = 0; j < kFrontCh; ++j) db2[j] = 0.0f;
    float lossv = 0.0f;
    for (int m = m0 + threadIdx.x; m < m1; m += kThreads) {
        const int row = m / d.HW, q = m - row * d.HW;
        const int64_t cb = (int64_t)row * d.C * d.HW + q;  // channel 0 of the cell
        float gi[kFrontCh], xo[NO];
#pragma unroll
        for (int j = 0; j < kFrontCh; ++j) gi[j] = a.gin ? a.gin[cb + (int64_t)(c0 + j) * d.HW] : 0.0f;
        load_out<NO>(d, a.x1 + cb, xo);
        const bool gv = a.given[m] != 0;
        const int tgt = a.targets ? a.targets[m] : 0;  // no targets: a step without a loss term
        const float mk = a.mask ? a.mask[m] : 0.0f;
        float f;
        if (a.fire_f32) {
            f = a.fire_f32[m];
        } else if (a.fire_u8) {
            f = a.fire_u8[m] ? 1.0f : 0.0f;
        } else {
            float u[4];
            nca::cell_uniforms4(a.key_ptr ? *a.key_ptr : a.key, (uint32_t)(a.row0 + row), a.step, (uint32_t)(q >> 2), u);
            const int e4 = q & 3;
            const float uq = e4 == 0 ? u[0] : e4 == 1 ? u[1] : e4 == 2 ? u[2] : u[3];
            f = uq < a.p ? 1.0f : 0.0f;
        }
        float gl[NO];
        const float lc = head_grad<NO>(a, hwL, hwL + NO * NO, xo, tgt, mk, gl);
        if (head) lossv = __fadd_rn(lossv, lc);
        if (kRegHead && head) {
#pragma unroll
            for (int v = 0; v < NO; ++v) {
#pragma unroll
                for (int c = 0; c < NO; ++c) hs[v * NO + c] = __builtin_fmaf(gl[v], xo[c], hs[v * NO + c]);
                hs[NO * NO + v] = __fadd_rn(hs[NO * NO + v], gl[v]);
            }
        }
#pragma unroll
        for (int j = 0; j < kFrontCh; ++j) {
            const int c = c0 + j;
            float g = gi[j];
            const int co = c - d.out_off;
            if (co >= 0 && co < d.c_out) {
#pragma unroll
                for (int v = 0; v < NO; ++v)
                    if (v < d.n_out) g = __builtin_fmaf(hwL[v * d.c_out + co], gl[v], g);
            }
            if (gv && c >= d.in_off && c < d.in_off + d.c_in) g = 0.0f;
            a.Gu[cb + (int64_t)c * d.HW] = g;
            // bf16 cells: dx is a bf16 tensor, so its gradient is bf16 (the reference's bf16
            // backward; triton_mlp.py:46-78 receives it as bf16)
            const float gd = d.bf16 ? nca::round_bf16(g * f) : g * f;
            a.Gdx[(int64_t)c * d.M + m] = gd;
            db2[j] = __fadd_rn(db2[j], gd);
        }
    }
    if (kRegHead && head) {  // one reduction: db2, the loss and the head's sums
        constexpr int NV = kFrontCh + 1 + (kRegHead ? NP : 0);
        float vals[NV];
#pragma unroll
        for (int j = 0; j < kFrontCh; ++j) vals[j] = db2[j];
        vals[kFrontCh] = lossv;
#pragma unroll
        for (int p = 0; p < NV - kFrontCh - 1; ++p) vals[kFrontCh + 1 + p] = hs[p];
        const float r = block_sums<NV, kThreads / 64>(vals, red);
        const int t = threadIdx.x;
        float *ps = a.part + s * a.P;
        if (t < kFrontCh) {
            ps[a.offB2 + c0 + t] = __fadd_rn(ps[a.offB2 + c0 + t], r);
        } else if (t == kFrontCh) {
            if (a.wscale != 0.0f) a.lossacc[s] = __fadd_rn(a.lossacc[s], r);
        } else if (t < NV && a.wscale != 0.0f) {
            const int p = t - kFrontCh - 1;
            int o = -1;
            if (p < NO * NO) {
                const int v = p / NO, c = p - v * NO;
                if (v < a.d.n_out && c < a.d.c_out) o = (int)a.offHW + v * a.d.c_out + c;
            } else if (p - NO * NO < a.d.n_out) {
                o = (int)a.offHB + p - NO * NO;
            }
            if (o >= 0) ps[o] = __fadd_rn(ps[o], r);
        }
        return;
    }
    const float r = block_sums<kFrontCh, kThreads / 64>(db2, red);
    if (threadIdx.x < kFrontCh) {
        float *pp = a.part + s * a.P + a.offB2 + c0 + threadIdx.x;
        *pp = __fadd_rn(*pp, r);
    }
    if (!head || a.wscale == 0.0f) return;  // uniform across the block
    {
        const float lv[1] = {lossv};
        const float rl = block_sums<1, kThreads / 64>(lv, red);
        if (threadIdx.x == 0) a.lossacc[s] = __fadd_rn(a.lossacc[s], rl);
    }
    // dhead: pair p < n_out c_out is (v, c): sum g_l[v] x1[out_off + c]; pair n_out c_out + v is
    // the bias: sum g_l[v]; 16 pairs at a time
    const int npw = d.n_out * d.c_out, np = npw + d.n_out;
    for (int p0 = 0; p0 < np; p0 += 16) {
        float acc[16];
#pragma unroll
        for (int k = 0; k < 16; ++k) acc[k] = 0.0f;
        for (int m = m0 + threadIdx.x; m < m1; m += kThreads) {
            const int row = m / d.HW, q = m - row * d.HW;
            float xo[NO], gl[NO];
            load_out<NO>(d, a.x1 + (int64_t)row * d.C * d.HW + q, xo);
            head_grad<NO>(a, hwL, hwL + NO * NO, xo, a.targets[m], a.mask ? a.mask[m] : 0.0f, gl);
#pragma unroll
            for (int k = 0; k < 16; ++k) {
                const int p = p0 + k;
                if (p >= np) break;
                const int v = p < npw ? p / d.c_out : p - npw, c = p < npw ? p - v * d.c_out : -1;
                float g = 0.0f, xc = 0.0f;
#pragma unroll
                for (int w = 0; w < NO; ++w) {
                    g = w == v ? gl[w] : g;
                    xc = w == c ? xo[w] : xc;
                }
                acc[k] = c < 0 ? __fadd_rn(acc[k], g) : __builtin_fmaf(g, xc, acc[k]);
            }
        }
        const float rh = block_sums<16, kThreads / 64>(acc, red);
        const int p = p0 + threadIdx.x;
        if (threadIdx.x < 16 && p < np) {
            const int v = p < npw ? p / d.c_out : p - npw;
            float *pp = a.part + s * a.P + (p < npw ? a.offHW + p : a.offHB + v);
            *pp = __fadd_rn(*pp, rh);
        }
    }
}

template <int NO>
__global__ void __launch_bounds__(kThreads) front_kernel(FrontArgs a) {
    __shared__ float red[(kThreads / 64) * 32];
    // the head's weights and bias in LDS: read in the loop next to the gradient stores, from global
    // memory each read would wait behind them
    __shared__ float hwL[NO * NO + NO];
    front_body<NO>(a, blockIdx.x, blockIdx.y, red, hwL);
}

// The perception input of tap (dy, dx) of cell (i, j) of row xr: the state (or the halo value
// hv), rounded to bf16 for bf16 cells like the forward's perception buffer. A halo tap loads
// the row's first cell and discards it.
__device__ __forceinline__ float tap_value(const float *xr, const Dims &d, int i, int j, int dy, int dx, float hv) {
    const int nq = neighbour(i, j, dy, dx, d.H, d.W, d.padding);
    const float x = xr[nq < 0 ? 0 : nq];
    const float v = nq >= 0 ? x : hv;
    return d.bf16 ? nca::round_bf16(v) : v;
}

// z element i: fp32, or bf16 for the fused MLP backward (Z16)
template <bool Z16>
__device__ __forceinline__ void z_store(float *Z, int64_t i, float v) {
    if (Z16)
        reinterpret_cast<__bf16 *>(Z)[i] = (__bf16)v;  // v is a bf16 value
    else
        Z[i] = v;
}

// z (F x M, feature-major) of the state x (rows, C, H, W): thread (row, channel, cell) with
// channel and cell from blockIdx.x, rows strided over blockIdx.y.
template <bool Z16>
__global__ void __launch_bounds__(kThreads) stencil_z_kernel(Dims d, const float *__restrict__ x,
                                                             const float *__restrict__ kern,
                                                             const float *__restrict__ padv, float *__restrict__ Z) {
    const int e = blockIdx.x * kThreads + threadIdx.x;
    if (e >= d.C * d.HW) return;
    const int c = e / d.HW, q = e - c * d.HW, i = q / d.W, j = q - i * d.W;
    const float hv = d.padding == 1 ? padv[c] : 0.0f;
    for (int64_t row = blockIdx.y; row < d.rows; row += gridDim.y) {
        const float *xr = x + (row * d.C + c) * (int64_t)d.HW;
        float xv[9];
#pragma unroll
        for (int t = 0; t < 9; ++t) xv[t] = tap_value(xr, d, i, j, t / 3 - 1, t % 3 - 1, hv);
        const int64_t m = row * d.HW + q;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            float acc = 0.0f;
#pragma unroll
            for (int t = 0; t < 9; ++t) acc = __builtin_fmaf(kern[k * 9 + t], xv[t], acc);
            z_store<Z16>(Z, (int64_t)(k * d.C + c) * d.M + m, d.bf16 ? nca::round_bf16(acc) : acc);
        }
    }
}

constexpr int kBackThreads = 1024;

// g_x = g_u + the transposed stencil of g_z, one thread per (row, channel, cell) in NCHW order
// (padding-aware: wall / zero halos take no gradient, wrap halos give it to the wrapped cell),
// and the kernel-weight gradient: sum over (c, m) of g_z[k C + c][m] * xp[c][m + tap] for every
// (k, tap). Block s takes the elements of NCHW range s and adds its 36 sums into slot s.
__global__ void __launch_bounds__(kBackThreads) stencil_back_kernel(
    Dims d, const float *__restrict__ x, const float *__restrict__ Gu, const float *__restrict__ Gz,
    const float *__restrict__ kern, const float *__restrict__ padv, float *__restrict__ gx,
    float *__restrict__ part, int64_t P, int64_t offK) {
    __shared__ float red[(kBackThreads / 64) * 36];
    const int64_t total = d.rows * d.C * (int64_t)d.HW;
    const int64_t per = (total + kSplit - 1) / kSplit, e0 = blockIdx.x * per;
    const int64_t e1 = e0 + per < total ? e0 + per : total;
    const int64_t ks = (int64_t)d.C * d.M;  // stride of k in g_z
    float acc[36];
#pragma unroll
    for (int v = 0; v < 36; ++v) acc[v] = 0.0f;
    int64_t e = e0 + threadIdx.x;
    if (e < e1) {
        int pl = (int)(e / d.HW), q = (int)(e - (int64_t)pl * d.HW);  // plane row * C + c, cell
        for (; e < e1; e += kBackThreads) {
            const int row = pl / d.C, c = pl - row * d.C, i = q / d.W, j = q - i * d.W;
            const float *xr = x + (int64_t)pl * d.HW;
            const int64_t gzo = (int64_t)c * d.M + (int64_t)row * d.HW;
            const float hv = d.padding == 1 ? padv[c] : 0.0f;
            float xv[9];
#pragma unroll
            for (int t = 0; t < 9; ++t) xv[t] = tap_value(xr, d, i, j, t / 3 - 1, t % 3 - 1, hv);
            float g = Gu[e];
#pragma unroll
            for (int t = 0; t < 9; ++t) {
                // cell q' whose tap t reads this cell: q = q' + (dy, dx); none for a halo
                const int qs = neighbour(i, j, -(t / 3 - 1), -(t % 3 - 1), d.H, d.W, d.padding);
                const int qc = qs < 0 ? 0 : qs;
                float gv[4];
#pragma unroll
                for (int k = 0; k < 4; ++k) gv[k] = gz_at(Gz, d.gz16, gzo + k * ks + qc);
#pragma unroll
                for (int k = 0; k < 4; ++k) g = qs >= 0 ? __builtin_fmaf(kern[k * 9 + t], gv[k], g) : g;
            }
            gx[e] = g;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const float gzv = gz_at(Gz, d.gz16, gzo + k * ks + q);
#pragma unroll
                for (int t = 0; t < 9; ++t) acc[k * 9 + t] = __builtin_fmaf(gzv, xv[t], acc[k * 9 + t]);
            }
            q += kBackThreads;
            if (q >= d.HW) {
                const int w = q / d.HW;
                pl += w;
                q -= w * d.HW;
            }
        }
    }
    const float r = block_sums<36, kBackThreads / 64>(acc, red);
    if (threadIdx.x < 36) {
        float *pp = part + blockIdx.x * P + offK + threadIdx.x;
        *pp = __fadd_rn(*pp, r);
    }
}

// The 3x3 taps of cell (i, j) from a plane staged in LDS (halo value hv), rounded to bf16 for
// bf16 cells.
__device__ __forceinline__ void plane_taps(const float *xs, const Dims &d, int i, int j, float hv, float xv[9]) {
#pragma unroll
    for (int t = 0; t < 9; ++t) {
        const int nq = neighbour(i, j, t / 3 - 1, t % 3 - 1, d.H, d.W, d.padding);
        const float v = nq >= 0 ? xs[nq < 0 ? 0 : nq] : hv;
        xv[t] = d.bf16 ? nca::round_bf16(v) : v;
    }
}

// stencil_z for boards of at most kPlaneMax cells: workgroup p stages plane p = (row, channel)
// of x in LDS and writes that channel's 4 features of the row's cells.
template <bool Z16>
__device__ void z_plane_body(const Dims &d, const float *__restrict__ x, const float *__restrict__ kern,
                             const float *__restrict__ padv, float *__restrict__ Z, int pl, float *xs) {
    const int row = pl / d.C, c = pl - row * d.C;
    const float *xr = x + (int64_t)pl * d.HW;
    const int H = d.H, W = d.W, W2 = W + 2, N2 = (H + 2) * W2;
    const float hv = d.padding == 1 ? padv[c] : 0.0f;
    const bool wrap = d.padding == 2;
    // the plane with a one-cell border (the padding value, or the wrapped cells) in LDS,
    // (H + 2) x (W + 2), each value rounded to bf16 once for bf16 cells; 8 cells per thread at a
    // time, every load issued before the LDS writes
    for (int e0 = 0; e0 < N2; e0 += 8 * kThreads) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int e = e0 + u * kThreads + threadIdx.x;
            const int bi = e / W2 - 1, bj = e - (bi + 1) * W2 - 1;
            const bool in = bi >= 0 && bi < H && bj >= 0 && bj < W;
            const int ai = bi < 0 ? H - 1 : (bi >= H ? 0 : bi), aj = bj < 0 ? W - 1 : (bj >= W ? 0 : bj);
            const bool take = e < N2 && (in || wrap);
            const float xv = xr[take ? ai * W + aj : 0];
            v[u] = take ? xv : hv;
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int e = e0 + u * kThreads + threadIdx.x;
            if (e < N2) xs[e] = d.bf16 ? nca::round_bf16(v[u]) : v[u];
        }
    }
    __syncthreads();
    // the 4 features of cell (i, j) from its 3x3 window, taps in the forward's order
    auto cell = [&](int i, int j, const float (&w0)[3], const float (&w1)[3], const float (&w2)[3]) {
        const float xv[9] = {w0[0], w0[1], w0[2], w1[0], w1[1], w1[2], w2[0], w2[1], w2[2]};
        const int64_t m = row * d.HW + i * W + j;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            float acc = 0.0f;
#pragma unroll
            for (int t = 0; t < 9; ++t) acc = __builtin_fmaf(kern[k * 9 + t], xv[t], acc);
            z_store<Z16>(Z, (int64_t)(k * d.C + c) * d.M + m, d.bf16 ? nca::round_bf16(acc) : acc);
        }
    };
    if (W <= kThreads) {
        // thread (band, column j) walks down rows [band R, band R + R) of column j with the window
        // in registers, reading one new row of 3 values per cell
        const int bands = kThreads / W, j = threadIdx.x % W, band = threadIdx.x / W;
        if (band >= bands) return;
        const int R = (H + bands - 1) / bands, i0 = band * R, i1 = i0 + R < H ? i0 + R : H;
        if (i0 >= i1) return;
        float w0[3], w1[3], w2[3];
#pragma unroll
        for (int k = 0; k < 3; ++k) {
            w0[k] = xs[i0 * W2 + j + k];  // bordered row i0 - 1 + 1
            w1[k] = xs[(i0 + 1) * W2 + j + k];
        }
        for (int i = i0; i < i1; ++i) {
#pragma unroll
            for (int k = 0; k < 3; ++k) w2[k] = xs[(i + 2) * W2 + j + k];
            cell(i, j, w0, w1, w2);
#pragma unroll
            for (int k = 0; k < 3; ++k) {
                w0[k] = w1[k];
                w1[k] = w2[k];
            }
        }
    } else {
        for (int q = threadIdx.x; q < d.HW; q += kThreads) {
            const int i = q / W, j = q - i * W;
            float w0[3], w1[3], w2[3];
#pragma unroll
            for (int k = 0; k < 3; ++k) {
                w0[k] = xs[i * W2 + j + k];
                w1[k] = xs[(i + 1) * W2 + j + k];
                w2[k] = xs[(i + 2) * W2 + j + k];
            }
            cell(i, j, w0, w1, w2);
        }
    }
}

template <bool Z16>
__global__ void __launch_bounds__(kThreads) stencil_z_plane(Dims d, const float *__restrict__ x,
                                                            const float *__restrict__ kern,
                                                            const float *__restrict__ padv, float *__restrict__ Z) {
    extern __shared__ float xs[];  // (H + 2) (W + 2) floats
    z_plane_body<Z16>(d, x, kern, padv, Z, blockIdx.x, xs);
}

// The front (kSplit x C / 8 workgroups) and the bf16 z (rows x C workgroups) of one step in one
// launch: they are independent, and each alone leaves most of the GPU idle.
template <int NO>
__global__ void __launch_bounds__(kThreads) front_z_kernel(FrontArgs a, const float *__restrict__ x,
                                                           const float *__restrict__ kern,
                                                           const float *__restrict__ padv, float *__restrict__ Z) {
    extern __shared__ float xs[];  // (H + 2) (W + 2) floats (z workgroups)
    __shared__ float red[(kThreads / 64) * 32];
    __shared__ float hwL[NO * NO + NO];
    const int nf = kSplit * (a.d.C / kFrontCh);
    if ((int)blockIdx.x < nf)
        front_body<NO>(a, (int)blockIdx.x % kSplit, (int)blockIdx.x / kSplit, red, hwL);
    else
        z_plane_body<true>(a.d, x, kern, padv, Z, (int)blockIdx.x - nf, xs);
}

// stencil_back for boards of at most kPlaneMax cells: workgroup p stages plane p = (row,
// channel) of x and the channel's 4 planes of g_z in LDS; g_x of the plane's cells, and the
// plane's kernel-weight sums added into its own slot dk[p][36].
__global__ void __launch_bounds__(kThreads) stencil_back_plane(Dims d, const float *__restrict__ x,
                                                               const float *__restrict__ Gu,
                                                               const float *__restrict__ Gz,
                                                               const float *__restrict__ kern,
                                                               const float *__restrict__ padv,
                                                               float *__restrict__ gx, float *__restrict__ dk) {
    extern __shared__ float xs[];  // x plane, then the 4 g_z planes: 5 HW floats
    __shared__ float red[(kThreads / 64) * 36];
    float *gs = xs + d.HW;
    const int pl = blockIdx.x, row = pl / d.C, c = pl - row * d.C;
    const float *xr = x + (int64_t)pl * d.HW;
    const int64_t ks = (int64_t)d.C * d.M;
    const int64_t gzo = (int64_t)c * d.M + (int64_t)row * d.HW;
    // staged 4 cells per thread at a time, every load issued before the LDS writes
    for (int q0 = 0; q0 < d.HW; q0 += 4 * kThreads) {
        float v[4][5];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int q = q0 + u * kThreads + threadIdx.x, qc = q < d.HW ? q : 0;
            v[u][0] = xr[qc];
#pragma unroll
            for (int k = 0; k < 4; ++k) v[u][1 + k] = gz_at(Gz, d.gz16, gzo + k * ks + qc);
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int q = q0 + u * kThreads + threadIdx.x;
            if (q < d.HW) {
                xs[q] = v[u][0];
#pragma unroll
                for (int k = 0; k < 4; ++k) gs[k * d.HW + q] = v[u][1 + k];
            }
        }
    }
    __syncthreads();
    const float hv = d.padding == 1 ? padv[c] : 0.0f;
    float acc[36];
#pragma unroll
    for (int v = 0; v < 36; ++v) acc[v] = 0.0f;
    for (int q = threadIdx.x; q < d.HW; q += kThreads) {
        const int i = q / d.W, j = q - i * d.W;
        float xv[9];
        plane_taps(xs, d, i, j, hv, xv);
        const int64_t e = (int64_t)pl * d.HW + q;
        float g = Gu[e];
#pragma unroll
        for (int t = 0; t < 9; ++t) {
            // cell q' whose tap t reads this cell: q = q' + (dy, dx); none for a halo
            const int qs = neighbour(i, j, -(t / 3 - 1), -(t % 3 - 1), d.H, d.W, d.padding);
            const int qc = qs < 0 ? 0 : qs;
#pragma unroll
            for (int k = 0; k < 4; ++k) g = qs >= 0 ? __builtin_fmaf(kern[k * 9 + t], gs[k * d.HW + qc], g) : g;
        }
        gx[e] = g;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const float gzv = gs[k * d.HW + q];
#pragma unroll
            for (int t = 0; t < 9; ++t) acc[k * 9 + t] = __builtin_fmaf(gzv, xv[t], acc[k * 9 + t]);
        }
    }
    const float r = block_sums<36, kThreads / 64>(acc, red);
    if (threadIdx.x < 36) {
        float *pp = dk + (int64_t)pl * 36 + threadIdx.x;
        *pp = __fadd_rn(*pp, r);
    }
}

constexpr int kStripPlanes = 4;  // (row, channel) planes per workgroup of stencil_back_strip

// stencil_back for boards at most 256 wide and of at most kPlaneMax cells: workgroup b takes
// planes [4b, 4b + 4) one after the other, each staged in LDS (x, g_u and the channel's 4 planes
// of g_z; the next plane's loads are in flight while this one computes from LDS). Thread (band,
// column j) walks down rows [band R, band R + R) of column j with the 3x3 neighbourhood of x and
// g_z in registers, loading one new row of 3 columns per cell (15 LDS reads instead of 45). Per
// cell the sums run in the order of stencil_back_kernel; the kernel-weight sums of the
// workgroup's planes go to slot b. GZ16: g_z is bf16.
template <bool GZ16>
__global__ void __launch_bounds__(kThreads) stencil_back_strip(Dims d, const float *__restrict__ x,
                                                               const float *__restrict__ Gu,
                                                               const float *__restrict__ Gz,
                                                               const float *__restrict__ kern,
                                                               const float *__restrict__ padv,
                                                               float *__restrict__ gx, float *__restrict__ dk) {
    extern __shared__ float xs[];  // x plane, the 4 g_z planes, g_u: 6 HW floats
    __shared__ float red[(kThreads / 64) * 36];
    float *gs = xs + d.HW, *us = xs + 5 * d.HW;
    const int H = d.H, W = d.W, HW = d.HW;
    const bool wrap = d.padding == 2;
    const int bands = kThreads / W, j = threadIdx.x % W, band = threadIdx.x / W;
    const int R = (H + bands - 1) / bands, i0 = band * R, i1 = i0 + R < H ? i0 + R : H;
    const bool active = band < bands;
    // the 3 columns of the window: cell column index (wrapped) and whether it is a halo column
    const int jc[3] = {j > 0 ? j - 1 : W - 1, j, j < W - 1 ? j + 1 : 0};
    const bool jh[3] = {j == 0 && !wrap, false, j == W - 1 && !wrap};
    const int64_t ks = (int64_t)d.C * d.M;
    float acc[36];
#pragma unroll
    for (int v = 0; v < 36; ++v) acc[v] = 0.0f;
    // the kernel weights in VGPRs (held in scalar registers they spill and reload in the row loop)
    float kr[36];
#pragma unroll
    for (int v = 0; v < 36; ++v) {
        kr[v] = kern[v];
        asm volatile("" : "+v"(kr[v]));
    }
    // this workgroup's slot of kernel-weight sums (its own, so read here, long before it is added to)
    const float dk_old = threadIdx.x < 36 ? dk[(int64_t)blockIdx.x * 36 + threadIdx.x] : 0.0f;
    const int p0 = blockIdx.x * kStripPlanes;
    const int p1 = p0 + kStripPlanes < d.rows * d.C ? p0 + kStripPlanes : (int)(d.rows * d.C);
    // a plane's 6 arrays, 8 cells per thread (HW <= kPlaneMax = 8 kThreads), in registers
    float pv[8][6];
    auto gload = [&](int pl) {
        const int row = pl / d.C, c = pl - row * d.C;
        const float *xr = x + (int64_t)pl * HW, *ur = Gu + (int64_t)pl * HW;
        const int64_t gzo = (int64_t)c * d.M + (int64_t)row * HW;
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int q = u * kThreads + threadIdx.x, qc = q < HW ? q : 0;
            if (u * kThreads < HW) {  // uniform
                pv[u][0] = xr[qc];
#pragma unroll
                for (int k = 0; k < 4; ++k) pv[u][1 + k] = gz_at(Gz, GZ16, gzo + k * ks + qc);
                pv[u][5] = ur[qc];
            }
        }
    };
    if (p0 < p1) gload(p0);
    for (int pl = p0; pl < p1; ++pl) {
        const int c = pl % d.C;
        __syncthreads();  // the previous plane's reads are done
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int q = u * kThreads + threadIdx.x;
            if (u * kThreads < HW && q < HW) {
                xs[q] = pv[u][0];
#pragma unroll
                for (int k = 0; k < 4; ++k) gs[k * HW + q] = pv[u][1 + k];
                us[q] = pv[u][5];
            }
        }
        __syncthreads();
        if (pl + 1 < p1) gload(pl + 1);  // in flight while this plane computes from LDS
        if (!active || i0 >= i1) continue;
        const float hv = d.padding == 1 ? padv[c] : 0.0f;
        // window row a of cell row i is grid row i + a - 1: x taps (halo value, bf16-rounded)
        // and g_z (zero at halo cells: no transposed contribution, so the taps need no branch).
        // The three window rows live in a ring of register slots (row i - 1, i, i + 1 in slots
        // S0, S1, S2, rotating by one per row), so sliding the window copies nothing.
        float xw[3][3], gw[3][4][3];
        auto load_row = [&](int a, int ii) __attribute__((always_inline)) {
            const bool rh = (ii < 0 || ii >= H) && !wrap;
            const int ir = ii < 0 ? H - 1 : (ii >= H ? 0 : ii);
#pragma unroll
            for (int b = 0; b < 3; ++b) {
                // every q is a cell of the plane (wrapped), so the loads need no branch
                const bool h = rh || jh[b];
                const int q = ir * W + jc[b];
                const float xl = xs[q];
                const float xv = h ? hv : xl;
                xw[a][b] = d.bf16 ? nca::round_bf16(xv) : xv;
                const unsigned keep = h ? 0u : 0xffffffffu;
#pragma unroll
                for (int k = 0; k < 4; ++k) gw[a][k][b] = __uint_as_float(__float_as_uint(gs[k * HW + q]) & keep);
            }
        };
        auto cell = [&](int i, auto s0_c, auto s1_c, auto s2_c) __attribute__((always_inline)) {
            constexpr int S0 = decltype(s0_c)::value, S1 = decltype(s1_c)::value, S2 = decltype(s2_c)::value;
            constexpr int SL[3] = {S0, S1, S2};
            load_row(S2, i + 1);
            const int64_t e = (int64_t)pl * HW + i * W + j;
            float g = us[i * W + j];
#pragma unroll
            for (int t = 0; t < 9; ++t) {
                // tap t = (dy, dx) reads x at (i + dy, j + dx); the cell whose tap t reads this
                // cell is (i - dy, j - dx): window position (1 - dy, 1 - dx)
                const int a = 2 - t / 3, b = 2 - t % 3;
#pragma unroll
                for (int k = 0; k < 4; ++k) g = __builtin_fmaf(kr[k * 9 + t], gw[SL[a]][k][b], g);
            }
            gx[e] = g;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const float gzv = gw[S1][k][1];
#pragma unroll
                for (int t = 0; t < 9; ++t) acc[k * 9 + t] = __builtin_fmaf(gzv, xw[SL[t / 3]][t % 3], acc[k * 9 + t]);
            }
        };
        using I0 = std::integral_constant<int, 0>;
        using I1 = std::integral_constant<int, 1>;
        using I2 = std::integral_constant<int, 2>;
        load_row(0, i0 - 1);
        load_row(1, i0);
        for (int i = i0; i < i1; i += 3) {
            cell(i, I0{}, I1{}, I2{});
            if (i + 1 < i1) cell(i + 1, I1{}, I2{}, I0{});
            if (i + 2 < i1) cell(i + 2, I2{}, I0{}, I1{});
        }
    }
    const float r = block_sums<36, kThreads / 64>(acc, red);
    if (threadIdx.x < 36) dk[(int64_t)blockIdx.x * 36 + threadIdx.x] = __fadd_rn(dk_old, r);
}

// acc[v] += the sum of the planes' kernel-weight slots: block v, each thread a fixed strided
// subset of the planes, then a fixed tree.
__global__ void __launch_bounds__(kThreads) reduce_dk(const float *dk, int64_t planes, float *acc) {
    __shared__ float red[kThreads];
    const int v = blockIdx.x;
    float s = 0.0f;
    for (int64_t p = threadIdx.x; p < planes; p += kThreads) s = __fadd_rn(s, dk[p * 36 + v]);
    s = block_sum(s, red);
    if (threadIdx.x == 0) acc[v] = __fadd_rn(acc[v], s);
}

// Row sums of a feature-major matrix G (R x M) over the kSplit cell ranges, added into the
// slots: wave w of block (b, s) takes row 4 b + w over range s.
__global__ void __launch_bounds__(kThreads) rowsum_kernel(const float *__restrict__ G, int64_t M, int R,
                                                          float *__restrict__ part, int64_t P, int64_t off) {
    const int lane = threadIdx.x & 63, r = blockIdx.x * 4 + (threadIdx.x >> 6), s = blockIdx.y;
    if (r >= R) return;  // uniform across the wave
    const int64_t per = (M + kSplit - 1) / kSplit, m0 = s * per, m1 = m0 + per < M ? m0 + per : M;
    const float *g = G + (int64_t)r * M;
    float acc = 0.0f;
    for (int64_t mb = m0; mb < m1; mb += 256) {
        float v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int64_t m = mb + 64 * u + lane;
            v[u] = m < m1 ? g[m] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) acc = __fadd_rn(acc, v[u]);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) acc = __fadd_rn(acc, __shfl_xor(acc, o));
    if (lane == 0) {
        float *pp = part + s * P + off + r;
        *pp = __fadd_rn(*pp, acc);
    }
}

// acc[i] = the sum of the kSplit slots in slot order.
__global__ void reduce_acc_kernel(const float *part, int64_t P, float *acc) {
    // slot order; 64 slots' loads issued before their additions (4 round trips for 256 slots)
    constexpr int kB = 64;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < P; i += (int64_t)gridDim.x * blockDim.x) {
        float s = 0.0f;
        for (int k0 = 0; k0 < kSplit; k0 += kB) {
            float v[kB];
#pragma unroll
            for (int k = 0; k < kB; ++k) v[k] = k0 + k < kSplit ? part[(int64_t)(k0 + k) * P + i] : 0.0f;
#pragma unroll
            for (int k = 0; k < kB; ++k)
                if (k0 + k < kSplit) s = __fadd_rn(s, v[k]);
        }
        acc[i] = s;
    }
}

// The loss of the chunk: the sum of the kSplit loss slots in a fixed tree; one block.
__global__ void loss_kernel(const float *lossacc, float *out) {
    __shared__ float red[kThreads];
    const float s = block_sum(threadIdx.x < kSplit ? lossacc[threadIdx.x] : 0.0f, red);
    if (threadIdx.x == 0) *out = s;
}

__global__ void copy_kernel(const float *src, float *dst, int64_t n) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        dst[i] = src[i];
}

// The summed parameter gradients (contiguous in acc) out to the caller's tensors, one launch:
// segment k is n[k] floats from acc + off[k] to dst[k] (null: skipped).
struct GradOut {
    float *dst[7];
    int64_t off[7], n[7];
    int accumulate;  // add into dst rather than write it
};

__device__ __forceinline__ void grad_put(const GradOut &g, int k, int64_t i, float v) {
    float *p = g.dst[k] + i;
    *p = g.accumulate ? __fadd_rn(*p, v) : v;
}

__global__ void grads_out_kernel(const float *acc, GradOut g) {
    const int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x, stride = (int64_t)gridDim.x * blockDim.x;
#pragma unroll
    for (int k = 0; k < 7; ++k)
        if (g.dst[k])
            for (int64_t i = t; i < g.n[k]; i += stride) grad_put(g, k, i, acc[g.off[k] + i]);
}

// The end of a backward in one launch: the slots summed in slot order (reduce_acc_kernel's sums),
// each parameter's gradient put straight into the caller's tensor (grads_out_kernel's), and the
// last block's loss (loss_kernel's), when nothing is added to acc between them.
__global__ void finish_kernel(const float *part, int64_t P, float *acc, GradOut g, const float *lossacc, float *loss_out) {
    if (blockIdx.x == gridDim.x - 1) {
        if (loss_out) {
            __shared__ float red[kThreads];
            const float s = block_sum(threadIdx.x < kSplit ? lossacc[threadIdx.x] : 0.0f, red);
            if (threadIdx.x == 0) *loss_out = s;
        }
        return;
    }
    constexpr int kB = 64;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < P; i += (int64_t)(gridDim.x - 1) * blockDim.x) {
        float s = 0.0f;
        for (int k0 = 0; k0 < kSplit; k0 += kB) {
            float v[kB];
#pragma unroll
            for (int k = 0; k < kB; ++k) v[k] = k0 + k < kSplit ? part[(int64_t)(k0 + k) * P + i] : 0.0f;
#pragma unroll
            for (int k = 0; k < kB; ++k)
                if (k0 + k < kSplit) s = __fadd_rn(s, v[k]);
        }
        acc[i] = s;
#pragma unroll
        for (int k = 0; k < 7; ++k)
            if (g.dst[k] && i >= g.off[k] && i < g.off[k] + g.n[k]) grad_put(g, k, i - g.off[k], s);
    }
}

// ------------------------------------------------------------------------------------------
// fp32 GEMM on v_mfma_f32_16x16x4_f32: C (M x N) = A (M x K) B (K x N) with strided operands
// (A(m, k) = A[m sam + k sak], B(k, n) = B[k sbk + n sbn], one of each pair of strides being 1),
// 64 x 64 block tiles, 16-deep k slices through LDS, each of the 4 waves a 32 x 32 quadrant.
// Split-K: block z sums k in [z kps, (z + 1) kps) and writes (or adds) its partial at
// C + z * csplit.
// Epilogues: 0 store (+ row bias), 1 fc1: bias, bf16 rounding for bf16 cells, ReLU,
// 2 mask: times [mask(m, n) > 0].
struct GemmArgs {
    const float *A;
    int64_t sam, sak;
    const float *B;
    int64_t sbk, sbn;
    float *Cm;
    int64_t ldc, csplit;
    int64_t M, N, K, kps;
    const float *bias;  // per row m
    const float *mask;
    int64_t ldmask;
    int epi, round_in, round_out;  // round_in: round A to bf16 on load (the forward's bf16 weights);
                                   // round_out: round the product to bf16 (before mask / ReLU)
    int accum;                     // add the result to C instead of storing it
};

constexpr int GBM = 64, GBN = 64, GBK = 16;

__global__ void __launch_bounds__(256) gemm_f32_kernel(GemmArgs g) {
    __shared__ float As[GBK][GBM + 4];
    __shared__ float Bs[GBK][GBN + 4];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int64_t m0 = (int64_t)blockIdx.y * GBM, n0 = (int64_t)blockIdx.x * GBN;
    const int64_t kb = (int64_t)blockIdx.z * g.kps, ke = kb + g.kps < g.K ? kb + g.kps : g.K;
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    f32x4 acc[2][2];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b) acc[a][b] = f32x4{0.f, 0.f, 0.f, 0.f};
    const bool a_kfast = g.sak == 1, b_nfast = g.sbn == 1;
    for (int64_t k0 = kb; k0 < ke; k0 += GBK) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int e = tid + 256 * r;
            const int am = a_kfast ? e >> 4 : e & 63, ak = a_kfast ? e & 15 : e >> 6;
            const int64_t gm = m0 + am, gk = k0 + ak;
            float v = 0.0f;
            if (gm < g.M && gk < ke) v = g.A[gm * g.sam + gk * g.sak];
            As[ak][am] = g.round_in ? nca::round_bf16(v) : v;
            const int bn = b_nfast ? e & 63 : e >> 4, bk = b_nfast ? e >> 6 : e & 15;
            const int64_t gn = n0 + bn, gk2 = k0 + bk;
            Bs[bk][bn] = (gn < g.N && gk2 < ke) ? g.B[gk2 * g.sbk + gn * g.sbn] : 0.0f;
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < GBK; kk += 4) {
            float af[2], bfv[2];
#pragma unroll
            for (int a = 0; a < 2; ++a) af[a] = As[kk + (lane >> 4)][wm * 32 + a * 16 + (lane & 15)];
#pragma unroll
            for (int b = 0; b < 2; ++b) bfv[b] = Bs[kk + (lane >> 4)][wn * 32 + b * 16 + (lane & 15)];
#pragma unroll
            for (int a = 0; a < 2; ++a)
#pragma unroll
                for (int b = 0; b < 2; ++b)
                    acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[a], bfv[b], acc[a][b], 0, 0, 0);
        }
        __syncthreads();
    }
    float *Cz = g.Cm + (int64_t)blockIdx.z * g.csplit;
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int64_t gm = m0 + wm * 32 + a * 16 + 4 * (lane >> 4) + v;
                const int64_t gn = n0 + wn * 32 + b * 16 + (lane & 15);
                if (gm >= g.M || gn >= g.N) continue;
                float r = acc[a][b][v];
                if (g.bias) r = __fadd_rn(r, g.bias[gm]);
                if (g.epi == 1) {
                    if (g.round_out) r = nca::round_bf16(r);
                    r = r > 0.0f ? r : 0.0f;
                } else {
                    if (g.round_out) r = nca::round_bf16(r);
                    if (g.epi == 2) r = g.mask[gm * g.ldmask + gn] > 0.0f ? r : 0.0f;
                }
                if (g.accum) r = __fadd_rn(Cz[gm * g.ldc + gn], r);
                Cz[gm * g.ldc + gn] = r;
            }
}

int gemm(const GemmArgs &g, int splits, hipStream_t st) {
    const int64_t gx = (g.N + GBN - 1) / GBN, gy = (g.M + GBM - 1) / GBM;
    if (gx > 0x7fffffff || gy > 65535) return nca::set_error(NCA_ERR_UNSUPPORTED, "GEMM grid too large");
    hipLaunchKernelGGL(gemm_f32_kernel, dim3((unsigned)gx, (unsigned)gy, (unsigned)splits), dim3(256), 0, st, g);
    return nca::hip_status(hipGetLastError(), "gemm launch");
}

// loss_head: the call computes the chunk loss, which is the cross-entropy of an mlp head (a single
// step's VJP has no loss term and takes any head).
int check_dims(const nca_cell_desc *cell, int64_t rows, int32_t H, int32_t W, int32_t n, Dims *d,
               bool loss_head = true) {
    if (!cell) return nca::set_error(NCA_ERR_INVALID, "cell descriptor is NULL");
    if (cell->heads != 4) return nca::set_error(NCA_ERR_UNSUPPORTED, "BPTT needs 4 perception kernels");
    if (loss_head && cell->head_kind != NCA_HEAD_MLP)
        return nca::set_error(NCA_ERR_UNSUPPORTED, "the BPTT loss is the cross-entropy of an mlp head");
    if (cell->n_out < 1 || cell->n_out > 16) return nca::set_error(NCA_ERR_UNSUPPORTED, "n_out must be 1..16");
    if (rows < 0 || H < 1 || W < 1 || n < 0) return nca::set_error(NCA_ERR_INVALID, "bad rows / grid / n_chunk");
    d->C = cell->channels;
    d->F = 4 * cell->channels;
    d->HD = cell->hidden;
    d->c_in = cell->c_in;
    d->in_off = cell->in_offset;
    d->c_out = cell->c_out;
    d->out_off = cell->out_offset;
    d->n_out = cell->n_out;
    d->padding = cell->padding;
    d->bf16 = cell->precision == NCA_BF16;
    d->gz16 = 0;
    d->H = H;
    d->W = W;
    if ((int64_t)H * W * d->C > 0x7fffffff) return nca::set_error(NCA_ERR_UNSUPPORTED, "BPTT grid too large");
    if (d->C % 8 != 0 || cell->c_out > 16) return nca::set_error(NCA_ERR_UNSUPPORTED, "BPTT needs channels % 8 == 0, c_out <= 16");
    d->HW = H * W;
    d->rows = rows;
    d->M = rows * (int64_t)H * W;
    // cell indices and (row, channel) planes are 32-bit in the kernels
    if (d->M >= ((int64_t)1 << 30) || rows * d->C >= ((int64_t)1 << 30) ||
        d->M * (int64_t)(d->F > d->HD ? d->F : d->HD) > ((int64_t)1 << 40))
        return nca::set_error(NCA_ERR_UNSUPPORTED, "BPTT batch too large");
    return NCA_OK;
}

unsigned grid_for(int64_t n) {
    const int64_t b = (n + kThreads - 1) / kThreads;
    return (unsigned)(b < 1 ? 1 : b);
}

}  // namespace

#include "nca_bptt_fused.h"

namespace nca {
int device_cus();
}

extern "C" {

size_t nca_bptt_workspace_bytes(const nca_cell_desc *cell, int64_t rows, int32_t height, int32_t width,
                                int32_t n_chunk) {
    Dims d;
    if (nca_packed_weights_bytes(cell) == 0 || check_dims(cell, rows, height, width, n_chunk, &d)) return 0;
    const size_t bwd = (size_t)ws_layout(d, n_chunk).total * sizeof(float);
    // the forward's row exchange when its boards run in pieces (nca_bptt_forward_ws)
    const size_t xch = nca::recorded_xch_bytes(cell, rows, height, width);
    return bwd > xch ? bwd : xch;
}

int nca_bptt_forward(const nca_cell_desc *cell, const void *packed, int64_t rows, int32_t height, int32_t width,
                     const float *x0, const uint8_t *given, const float *clamp, const nca_fire_desc *fire,
                     int32_t n_chunk, float *states, void *stream) {
    return nca_bptt_forward_ws(cell, packed, rows, height, width, x0, given, clamp, fire, n_chunk, states, nullptr, 0,
                               stream);
}

int nca_bptt_forward_ws(const nca_cell_desc *cell, const void *packed, int64_t rows, int32_t height, int32_t width,
                        const float *x0, const uint8_t *given, const float *clamp, const nca_fire_desc *fire,
                        int32_t n_chunk, float *states, void *workspace, size_t workspace_bytes, void *stream) {
    nca::clear_error();
    Dims d;
    int rc = check_dims(cell, rows, height, width, n_chunk, &d);
    if (rc) return rc;
    if (!fire || !states || !x0) return nca::set_error(NCA_ERR_INVALID, "NULL pointer argument");
    if (fire->adaptive) return nca::set_error(NCA_ERR_UNSUPPORTED, "BPTT chunks fire uniformly (no confidence gating)");
    const int64_t sn = d.rows * d.C * (int64_t)d.HW;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    if (rows == 0) return NCA_OK;
    // the whole chunk in one launch of the streamed kernel where it takes the cell and grid (which
    // also copies x0 into states[0]); else a copy and one launch per step
    bool used = false;
    int pieces = 1;
    if ((rc = nca::rollout_recorded(cell, packed, rows, height, width, x0, given, clamp, states + n_chunk * sn, fire,
                                    n_chunk, states + sn, sn, st, &used, workspace, workspace_bytes, &pieces,
                                    states != x0 ? states : nullptr)))
        return rc;
    if (!used && states != x0 &&
        (rc = nca::hip_status(hipMemcpyAsync(states, x0, sn * sizeof(float), hipMemcpyDeviceToDevice, st), "state copy")))
        return rc;
    // the workspace's first word reports whether a wait of the boards' pieces ran out: zero unless
    // this call sets it (the launch of pieces clears it itself)
    if (pieces == 1 && workspace && workspace_bytes >= nca::kXchStatusBytes &&
        (rc = nca::hip_status(nca::clear_words(static_cast<uint64_t *>(workspace), nca::kXchStatusBytes / 8, st),
                              "status clear")))
        return rc;
    if (used) return NCA_OK;
    for (int t = 0; t < n_chunk; ++t) {
        nca_fire_desc f = *fire;
        f.step0 = fire->step0 + t;
        if (fire->step_seeds) f.step_seeds = fire->step_seeds + t;
        if (fire->fire_in) f.fire_in = fire->fire_in + (int64_t)t * d.rows * d.HW;
        rc = nca_rollout_ws(cell, packed, rows, height, width, states + t * sn, given, clamp, states + (t + 1) * sn, &f,
                            1, nullptr, nullptr, nullptr, nullptr, 0, stream);
        if (rc) return rc;
    }
    return NCA_OK;
}

}  // extern "C"

namespace {

// The one-launch backward of a chunk (nca_bptt_fused.h) where it takes the call: pieces > 1 per
// board when the boards' pieces fit the device at once (rows * pieces workgroups on as many CUs,
// at most kSplit slots), each piece's plan fits the LDS and the exchange slots fit the
// workspace's z region; else whole boards (pieces = 1, at most kSplit boards); pieces = 0: the
// three launches per step. The whole-board plan must fit either way (it is the pieces' repair).
struct FusedChoice {
    int pieces = 0, Hp = 0;
    FusedPlan plan, whole;
    size_t xch_bytes = 0;  // pieces: the status block and the exchange slots
};

FusedChoice fused_choice(const Dims &d, int n, bool fire_f32, const WsLayout &L) {
    FusedChoice c;
    constexpr unsigned kLds = 160u * 1024u;
    const int path = nca::g_piece_debug.back_path;
    if (path == 1 || !fused_mlp(d) || fire_f32 || n < 1 || n > kFusedMaxChunk || d.M <= 0) return c;
    if (d.n_out > 4 || d.c_out > 4 || d.rows > kSplit) return c;
    c.whole = fused_plan(false, d.H, d.W);
    if (c.whole.total > kLds) return c;
    if (path != 2 && d.W <= 32) {
        int cus = nca::g_piece_debug.plan_cus > 0 ? nca::g_piece_debug.plan_cus : nca::device_cus();
        if (cus > kSplit) cus = kSplit;
        for (int P = 4; P >= 2; --P) {
            const int Hp = (d.H + P - 1) / P;
            if ((P - 1) * Hp >= d.H || d.rows * P > cus) continue;
            const FusedPlan pl = fused_plan(true, Hp, d.W);
            const size_t xb = nca::kXchStatusBytes + (size_t)d.rows * P * 4 * 64 * d.W * sizeof(uint64_t);
            if (pl.total > kLds || xb > (size_t)(L.Gz - L.Z) * sizeof(float)) continue;
            c.pieces = P;
            c.Hp = Hp;
            c.plan = pl;
            c.xch_bytes = xb;
            return c;
        }
    }
    c.pieces = 1;
    c.Hp = d.H;
    c.plan = c.whole;
    return c;
}

// The backward of n_chunk steps (nca_bptt_backward). Step t reads its input state at
// states + t * stride and its output at states + (t + 1) * stride; stride 0 (the single-step VJP,
// which has no loss term) reads `states` for both. fire_f32, when given, is the (rows, H, W) fire
// value of a one-step call instead of the fire descriptor's masks. grads->head_w / head_b may be
// NULL when no step has a loss term.
int backward_impl(const Dims &d, const void *packed, const nca_cell_weights *w,
                  const float *states, int64_t stride, const uint8_t *given, const nca_fire_desc *fire,
                  const float *fire_f32, int32_t n_chunk, const nca_bptt_loss *loss, const float *grad_final,
                  nca_cell_grads *grads, float *grad_x0, float *loss_out, void *workspace, size_t workspace_bytes,
                  hipStream_t st) {
    int rc = NCA_OK;
    const WsLayout L = ws_layout(d, n_chunk);
    if (!workspace || workspace_bytes < (size_t)L.total * sizeof(float)) {
        char msg[160];
        snprintf(msg, sizeof(msg),
                 "the backward needs a workspace of %zu bytes (nca_bptt_workspace_bytes, "
                 "nca_step_backward_workspace_bytes)",
                 (size_t)L.total * sizeof(float));
        return nca::set_error(NCA_ERR_INVALID, msg);
    }
    float wsum = 0.0f;
    for (int t = 0; t < n_chunk; ++t) wsum += loss->step_weights[t];
    const float wden = wsum < 1.0f ? 1.0f : wsum;  // weights.sum().clamp_min(1), engine.py:490
    const ParamLayout P = param_layout(d);
    const nca::PackedLayout PL = nca::packed_layout(d.C, 4, d.HD, d.c_out, d.n_out, d.bf16);
    const unsigned char *pb = static_cast<const unsigned char *>(packed);
    const float *kern = reinterpret_cast<const float *>(pb + PL.kern);
    const float *b1 = reinterpret_cast<const float *>(pb + PL.b1);
    const float *headw = reinterpret_cast<const float *>(pb + PL.headw);
    const float *headb = reinterpret_cast<const float *>(pb + PL.headb);
    const float *padv = reinterpret_cast<const float *>(pb + PL.padv);
    float *ws = static_cast<float *>(workspace);
    float *Z = ws + L.Z, *Hb = ws + L.Hb, *Ga = ws + L.Ga, *Gz = ws + L.Gz, *Gdx = ws + L.Gdx;
    float *Gu = ws + L.Gu, *Gx[2] = {ws + L.Gx0, ws + L.Gx1}, *part = ws + L.part, *acc = ws + L.acc;
    float *lossacc = ws + L.lossacc, *denom = ws + L.denom;
    const int64_t sn = d.rows * d.C * (int64_t)d.HW;

    // the partial-sum slots and the loss slots are contiguous; with the one-launch backward on
    // pieces of boards, its status word and exchange slots are cleared by the same launch
    const FusedChoice fc = fused_choice(d, n_chunk, fire_f32 != nullptr, L);
    uint64_t *const wsw = static_cast<uint64_t *>(workspace);
    const int64_t xch_words = fc.pieces > 1 ? (int64_t)(fc.xch_bytes / sizeof(uint64_t)) - 1 : 0;
    const bool fused = fused_mlp(d);
    if (fc.pieces > 0) {
        // the one-launch backward writes every value of its workgroups' slots (and the finish
        // launch writes acc): only the slots beyond them, the exchange words and the status word
        // need clearing, in the launch that builds the weight image
        const int64_t written = d.rows * (int64_t)fc.pieces;
        hipLaunchKernelGGL(prep_clear_kernel, dim3(nca::kMb32PrepBlocks + kPrepClearBlocks), dim3(512), 0, st, w->w1,
                           w->w2, reinterpret_cast<unsigned char *>(ws + L.img), wsw + 1, xch_words,
                           part + written * P.P, (kSplit - written) * P.P, lossacc + written, kSplit - written);
    } else {
        hipLaunchKernelGGL(zero_f32_words, dim3(2048), dim3(256), 0, st, part, L.denom - L.part, wsw + 1, xch_words);
    }
    auto mlp_kfn = (d.M & 3) == 0 ? nca::mlp_back32<true> : nca::mlp_back32<false>;
    if (fused && (rc = nca::hip_status(hipFuncSetAttribute(reinterpret_cast<const void *>(mlp_kfn),
                                                           hipFuncAttributeMaxDynamicSharedMemorySize,
                                                           (int)nca::Mb32::TOTAL),
                                       "mlp_back32 attribute")))
        return rc;
    // the stencil kernels read g_z as bf16 where the fused kernel writes it
    Dims ds = d;
    ds.gz16 = fused ? 1 : 0;
    // boards small enough to stage (row, channel) planes in LDS
    const bool planes_ok = planes_fit(d);
    // ... and walked by columns for boards at most 256 wide (kernel-weight slot per 4 planes)
    const bool strips_ok = planes_ok && d.W <= kThreads;
    // the z workgroups' bordered plane
    const size_t zlds = (size_t)(d.H + 2) * (d.W + 2) * sizeof(float);
    const int64_t strip_blocks = (d.rows * d.C + kStripPlanes - 1) / kStripPlanes;
    // cells per workgroup of the fused kernel: whole 32-cell tiles
    const int per32 = (int)((((d.M + kSplit - 1) / kSplit) + 31) / 32 * 32);
    if (fused && fc.pieces == 0)
        hipLaunchKernelGGL(nca::mlp_back32_prep, dim3(nca::kMb32PrepBlocks), dim3(512), 0, st, w->w1, w->w2,
                           reinterpret_cast<unsigned char *>(ws + L.img));
    if (loss->loss_mask && d.M > 0) hipLaunchKernelGGL(mask_sum, dim3(1), dim3(kThreads), 0, st, loss->loss_mask, d.M, denom);
    if ((rc = nca::hip_status(hipGetLastError(), "bptt setup"))) return rc;
    if (fc.pieces > 0) {
        FusedArgs A;
        memset(&A, 0, sizeof(A));
        A.fa.d = d;
        A.fa.given = given;
        A.fa.targets = loss->targets;
        A.fa.mask = loss->loss_mask;
        A.fa.denom = denom;
        A.fa.head_w = headw;
        A.fa.head_b = headb;
        A.fa.fire_u8 = fire->fire_in;
        A.fa.key_ptr = fire->step_seeds;
        A.fa.key = fire->seed;
        A.fa.row0 = fire->row0;
        A.fa.step = (uint32_t)fire->step0;
        A.fa.p = fire->p_fire;
        A.states = states;
        A.stride = stride;
        A.n = n_chunk;
        for (int t = 0; t < n_chunk; ++t) {
            const float wt = loss->step_weights[t] / wden;
            A.wscale[t] = loss->loss_mask ? wt : wt / (float)d.M;
        }
        A.grad_final = grad_final;
        A.grad_x0 = grad_x0;
        A.img = reinterpret_cast<const unsigned char *>(ws + L.img);
        A.b1 = b1;
        A.kern = kern;
        A.padv = padv;
        A.part = part;
        A.lossacc = lossacc;
        A.P = P.P;
        A.offK = P.K;
        A.offW1 = P.W1;
        A.offB1 = P.B1;
        A.offW2 = P.W2;
        A.offB2 = P.B2;
        A.offHW = P.HW;
        A.offHB = P.HB;
        A.gz_g = reinterpret_cast<uint16_t *>(ws + L.Gz);
        A.gx_g = ws + L.Gx0;
        A.spin_limit = nca::g_piece_debug.spin_limit > 0 ? nca::g_piece_debug.spin_limit : nca::kHaloSpin;
        A.tag_skew = nca::g_piece_debug.force_timeout ? (1 << 30) : 0;
        auto set_plan = [&](FusedArgs &a, const FusedPlan &pl) {
            a.l_GZ = pl.GZ;
            a.l_GX = pl.GX;
            a.l_XS = pl.XS;
            a.l_MLP = pl.MLP;
            a.l_FI = pl.FI;
            a.l_RED = pl.RED;
            a.l_ACC = pl.ACC;
            a.l_HWL = pl.HWL;
            a.l_FB = pl.FB;
        };
        auto kp = bptt_back_fused<true>;
        auto kw = bptt_back_fused<false>;
        if ((rc = nca::hip_status(hipFuncSetAttribute(reinterpret_cast<const void *>(kw),
                                                      hipFuncAttributeMaxDynamicSharedMemorySize, (int)fc.whole.total),
                                  "fused backward attribute")))
            return rc;
        FusedArgs Aw = A;  // whole boards
        Aw.pieces = 1;
        Aw.Hp = d.H;
        set_plan(Aw, fc.whole);
        if (fc.pieces > 1) {
            // the status word (bytes 8 .. 11 of the workspace; bytes 0 .. 3 hold the forward's) and
            // the exchange slots after the status block, cleared with the slots above
            A.status = reinterpret_cast<uint32_t *>(workspace) + 2;
            A.xch = wsw + nca::kXchStatusBytes / sizeof(uint64_t);
            A.pieces = fc.pieces;
            A.Hp = fc.Hp;
            A.gz_rows = fc.Hp + 2;
            set_plan(A, fc.plan);
            if ((rc = nca::hip_status(hipFuncSetAttribute(reinterpret_cast<const void *>(kp),
                                                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)fc.plan.total),
                                      "fused backward attribute")))
                return rc;
            hipLaunchKernelGGL(kp, dim3((unsigned)(d.rows * fc.pieces)), dim3(kFusedThreads), fc.plan.total, st, A);
            if ((rc = nca::hip_status(hipGetLastError(), "fused backward (pieces)"))) return rc;
            // the repair: whole boards, only if a piece's wait ran out
            Aw.run_if = A.status;
            Aw.zero_slots = (int)(d.rows * fc.pieces);
        }
        hipLaunchKernelGGL(kw, dim3((unsigned)d.rows), dim3(kFusedThreads), fc.whole.total, st, Aw);
        if ((rc = nca::hip_status(hipGetLastError(), "fused backward (whole boards)"))) return rc;
    }
    const float *gin = grad_final;
    for (int t = n_chunk - 1; t >= 0 && d.M > 0 && fc.pieces == 0; --t) {
        const float *xt = states + t * stride, *x1 = states + (t + 1) * stride;
        float *gx = (t == 0 && grad_x0) ? grad_x0 : Gx[t & 1];
        // front: loss gradient, clamp and fire
        FrontArgs fa;
        memset(&fa, 0, sizeof(fa));
        fa.d = d;
        fa.x1 = x1;
        fa.gin = gin;
        fa.given = given;
        fa.targets = loss->targets;
        fa.mask = loss->loss_mask;
        fa.denom = denom;
        const float wt = loss->step_weights[t] / wden;
        fa.wscale = loss->loss_mask ? wt : wt / (float)d.M;
        fa.head_w = headw;
        fa.head_b = headb;
        fa.fire_u8 = fire->fire_in ? fire->fire_in + (int64_t)t * d.rows * d.HW : nullptr;
        fa.fire_f32 = fire_f32;
        fa.key_ptr = fire->step_seeds ? fire->step_seeds + t : nullptr;
        fa.key = fire->seed;
        fa.row0 = fire->row0;
        fa.step = (uint32_t)(fire->step0 + t);
        fa.p = fire->p_fire;
        fa.Gu = Gu;
        fa.Gdx = Gdx;
        fa.part = part;
        fa.lossacc = lossacc;
        fa.P = P.P;
        fa.offB2 = P.B2;
        fa.offHW = P.HW;
        fa.offHB = P.HB;
        const int no = d.n_out > d.c_out ? d.n_out : d.c_out;
        // recompute z (and, in the MLP stage, h) from the saved state
        if (fused && planes_ok) {  // front and z in one launch
            auto fz = no <= 4 ? front_z_kernel<4> : no <= 8 ? front_z_kernel<8> : front_z_kernel<16>;
            hipLaunchKernelGGL(fz, dim3((unsigned)(kSplit * (d.C / kFrontCh) + d.rows * d.C)), dim3(kThreads),
                               zlds, st, fa, xt, kern, padv, Z);
        } else if (planes_ok) {
            auto front = no <= 4 ? front_kernel<4> : no <= 8 ? front_kernel<8> : front_kernel<16>;
            hipLaunchKernelGGL(front, dim3(kSplit, d.C / kFrontCh), dim3(kThreads), 0, st, fa);
            auto zfn = fused ? stencil_z_plane<true> : stencil_z_plane<false>;
            hipLaunchKernelGGL(zfn, dim3((unsigned)(d.rows * d.C)), dim3(kThreads), zlds, st, d, xt, kern,
                               padv, Z);
        } else {
            auto front = no <= 4 ? front_kernel<4> : no <= 8 ? front_kernel<8> : front_kernel<16>;
            hipLaunchKernelGGL(front, dim3(kSplit, d.C / kFrontCh), dim3(kThreads), 0, st, fa);
            const dim3 zgrid(grid_for((int64_t)d.C * d.HW), (unsigned)(d.rows < 65535 ? d.rows : 65535));
            hipLaunchKernelGGL(fused ? stencil_z_kernel<true> : stencil_z_kernel<false>, zgrid, dim3(kThreads), 0, st, d,
                               xt, kern, padv, Z);
        }
        if ((rc = nca::hip_status(hipGetLastError(), "bptt front / stencil"))) return rc;
        GemmArgs g;
        if (fused) {
            nca::MlpBackArgs ma;
            ma.Z = reinterpret_cast<const uint16_t *>(Z);
            ma.Gdx = Gdx;
            ma.img = reinterpret_cast<const unsigned char *>(ws + L.img);
            ma.b1 = b1;
            ma.Gz = reinterpret_cast<uint16_t *>(Gz);
            ma.part = part;
            ma.P = P.P;
            ma.offW1 = P.W1;
            ma.offB1 = P.B1;
            ma.offW2 = P.W2;
            ma.M = d.M;
            ma.per = per32;
            hipLaunchKernelGGL(mlp_kfn, dim3(kSplit), dim3(512), nca::Mb32::TOTAL, st, ma);
            if ((rc = nca::hip_status(hipGetLastError(), "mlp_back32"))) return rc;
        } else {
            memset(&g, 0, sizeof(g));
            // h = relu(W1 z + b1): (HD x F) (F x M)
            g.A = w->w1; g.sam = d.F; g.sak = 1;
            g.B = Z; g.sbk = d.M; g.sbn = 1;
            g.Cm = Hb; g.ldc = d.M; g.M = d.HD; g.N = d.M; g.K = d.F; g.kps = d.F;
            g.bias = b1; g.epi = 1; g.round_in = d.bf16; g.round_out = d.bf16;
            if ((rc = gemm(g, 1, st))) return rc;
            // g_a = (W2^T g_dx) * [h > 0]: (HD x C) (C x M)
            memset(&g, 0, sizeof(g));
            g.A = w->w2; g.sam = 1; g.sak = d.HD;
            g.B = Gdx; g.sbk = d.M; g.sbn = 1;
            g.Cm = Ga; g.ldc = d.M; g.M = d.HD; g.N = d.M; g.K = d.C; g.kps = d.C;
            g.mask = Hb; g.ldmask = d.M; g.epi = 2; g.round_in = d.bf16; g.round_out = d.bf16;
            if ((rc = gemm(g, 1, st))) return rc;
            // g_z = W1^T g_a: (F x HD) (HD x M)
            memset(&g, 0, sizeof(g));
            g.A = w->w1; g.sam = 1; g.sak = d.F;
            g.B = Ga; g.sbk = d.M; g.sbn = 1;
            g.Cm = Gz; g.ldc = d.M; g.M = d.F; g.N = d.M; g.K = d.HD; g.kps = d.HD;
            g.round_in = d.bf16; g.round_out = d.bf16;
            if ((rc = gemm(g, 1, st))) return rc;
        }
        // gradient of the step's input state and the kernel-weight partials
        auto strip_fn = fused ? stencil_back_strip<true> : stencil_back_strip<false>;
        if (strips_ok)
            hipLaunchKernelGGL(strip_fn, dim3((unsigned)strip_blocks), dim3(kThreads), 6 * d.HW * sizeof(float), st, ds,
                               xt, Gu, Gz, kern, padv, gx, ws + L.dk);
        else if (planes_ok)
            hipLaunchKernelGGL(stencil_back_plane, dim3((unsigned)(d.rows * d.C)), dim3(kThreads),
                               5 * d.HW * sizeof(float), st, ds, xt, Gu, Gz, kern, padv, gx, ws + L.dk);
        else
            hipLaunchKernelGGL(stencil_back_kernel, dim3(kSplit), dim3(kBackThreads), 0, st, ds, xt, Gu, Gz, kern, padv,
                               gx, part, P.P, P.K);
        if (!fused) {
            // weight-gradient partials over kSplit cell ranges
            const int64_t kps = (((d.M + kSplit - 1) / kSplit) + GBK - 1) / GBK * GBK;
            memset(&g, 0, sizeof(g));
            g.A = Ga; g.sam = d.M; g.sak = 1;  // dW1 = g_a z^T: (HD x M) (M x F)
            g.B = Z; g.sbk = 1; g.sbn = d.M;
            g.Cm = part + P.W1; g.ldc = d.F; g.csplit = P.P; g.M = d.HD; g.N = d.F; g.K = d.M; g.kps = kps;
            g.accum = 1;
            if ((rc = gemm(g, kSplit, st))) return rc;
            memset(&g, 0, sizeof(g));
            g.A = Gdx; g.sam = d.M; g.sak = 1;  // dW2 = g_dx h^T: (C x M) (M x HD)
            g.B = Hb; g.sbk = 1; g.sbn = d.M;
            g.Cm = part + P.W2; g.ldc = d.HD; g.csplit = P.P; g.M = d.C; g.N = d.HD; g.K = d.M; g.kps = kps;
            g.accum = 1;
            if ((rc = gemm(g, kSplit, st))) return rc;
            hipLaunchKernelGGL(rowsum_kernel, dim3((d.HD + 3) / 4, kSplit), dim3(kThreads), 0, st, Ga, d.M, d.HD, part,
                               P.P, P.B1);
        }
        if ((rc = nca::hip_status(hipGetLastError(), "bptt step kernels"))) return rc;
        gin = gx;
    }
    if (grad_x0) {
        if (n_chunk == 0 || d.M == 0) {
            if (grad_final) hipLaunchKernelGGL(copy_kernel, dim3(256), dim3(256), 0, st, grad_final, grad_x0, sn);
            else hipLaunchKernelGGL(zero_f32, dim3(256), dim3(256), 0, st, grad_x0, sn);
        }
    }
    // the gradients in the reference's parameter layouts (written, or added to the caller's)
    GradOut go;
    float *gdst[7] = {grads->kernels, grads->w1, grads->b1, grads->w2, grads->b2, grads->head_w, grads->head_b};
    const int64_t goff[7] = {P.K, P.W1, P.B1, P.W2, P.B2, P.HW, P.HB};
    const int64_t gn[7] = {36, (int64_t)d.HD * d.F, d.HD, (int64_t)d.C * d.HD, d.C, (int64_t)d.n_out * d.c_out, d.n_out};
    for (int k = 0; k < 7; ++k) {
        go.dst[k] = gdst[k];
        go.off[k] = goff[k];
        go.n[k] = gn[k];
    }
    go.accumulate = grads->accumulate != 0;
    const bool has_loss = n_chunk > 0 && d.M > 0;
    if (planes_ok && fc.pieces == 0) {
        // the slots summed in slot order, the strips' kernel-weight sums added, then the gradients
        hipLaunchKernelGGL(reduce_acc_kernel, dim3((unsigned)((P.P + 255) / 256)), dim3(256), 0, st, part, P.P, acc);
        hipLaunchKernelGGL(reduce_dk, dim3(36), dim3(kThreads), 0, st, ws + L.dk, strips_ok ? strip_blocks : d.rows * d.C,
                           acc + P.K);
        hipLaunchKernelGGL(grads_out_kernel, dim3(128), dim3(256), 0, st, acc, go);
        if (loss_out && has_loss) hipLaunchKernelGGL(loss_kernel, dim3(1), dim3(kThreads), 0, st, lossacc, loss_out);
    } else {
        hipLaunchKernelGGL(finish_kernel, dim3((unsigned)((P.P + kThreads - 1) / kThreads) + 1u), dim3(kThreads), 0, st,
                           part, P.P, acc, go, lossacc, has_loss ? loss_out : nullptr);
    }
    if (loss_out && !has_loss) hipLaunchKernelGGL(zero_f32, dim3(1), dim3(64), 0, st, loss_out, (int64_t)1);
    return nca::hip_status(hipGetLastError(), "bptt finish");
}

}  // namespace

extern "C" {

int nca_bptt_backward(const nca_cell_desc *cell, const void *packed, const nca_cell_weights *w, int64_t rows,
                      int32_t height, int32_t width, const float *states, const uint8_t *given,
                      const nca_fire_desc *fire, int32_t n_chunk, const nca_bptt_loss *loss,
                      const float *grad_final, nca_cell_grads *grads, float *grad_x0, float *loss_out,
                      void *workspace, size_t workspace_bytes, void *stream) {
    nca::clear_error();
    Dims d;
    int rc = check_dims(cell, rows, height, width, n_chunk, &d);
    if (rc) return rc;
    const size_t pk = nca_packed_weights_bytes(cell);
    if (pk == 0) return NCA_ERR_UNSUPPORTED;  // message set by the packing check
    if (!packed || !w || !w->w1 || !w->w2 || !states || !given || !fire || !loss || !grads)
        return nca::set_error(NCA_ERR_INVALID, "NULL pointer argument");
    if (!grads->kernels || !grads->w1 || !grads->b1 || !grads->w2 || !grads->b2 || !grads->head_w || !grads->head_b)
        return nca::set_error(NCA_ERR_INVALID, "NULL gradient pointer");
    if (fire->adaptive) return nca::set_error(NCA_ERR_UNSUPPORTED, "BPTT chunks fire uniformly (no confidence gating)");
    if (n_chunk > 0 && (!loss->step_weights || !loss->targets))
        return nca::set_error(NCA_ERR_INVALID, "the loss needs step_weights and targets");
    const int64_t sn = d.rows * d.C * (int64_t)d.HW;
    return backward_impl(d, packed, w, states, sn, given, fire, nullptr, n_chunk, loss, grad_final, grads,
                         grad_x0, loss_out, workspace, workspace_bytes, reinterpret_cast<hipStream_t>(stream));
}

size_t nca_step_backward_workspace_bytes(const nca_cell_desc *cell, int64_t rows, int32_t height, int32_t width) {
    Dims d;
    if (nca_packed_weights_bytes(cell) == 0 || check_dims(cell, rows, height, width, 1, &d, false)) return 0;
    return (size_t)ws_layout(d, 1).total * sizeof(float);
}

int nca_step_backward(const nca_cell_desc *cell, const void *packed, const nca_cell_weights *w, int64_t rows,
                      int32_t height, int32_t width, const float *x, const uint8_t *given, const float *fire,
                      const float *grad_out, nca_cell_grads *grads, float *grad_x, void *workspace,
                      size_t workspace_bytes, void *stream) {
    nca::clear_error();
    Dims d;
    int rc = check_dims(cell, rows, height, width, 1, &d, false);
    if (rc) return rc;
    if (nca_packed_weights_bytes(cell) == 0) return NCA_ERR_UNSUPPORTED;  // message set by the packing check
    if (!packed || !w || !w->w1 || !w->w2 || !x || !given || !fire || !grad_out || !grads)
        return nca::set_error(NCA_ERR_INVALID, "NULL pointer argument");
    if (!grads->kernels || !grads->w1 || !grads->b1 || !grads->w2 || !grads->b2)
        return nca::set_error(NCA_ERR_INVALID, "NULL gradient pointer");
    // one step with no loss term: the cotangent of the step's output is all that flows back
    nca_fire_desc fd;
    memset(&fd, 0, sizeof(fd));
    const float zero_weight = 0.0f;
    nca_bptt_loss none;
    none.targets = nullptr;
    none.loss_mask = nullptr;
    none.step_weights = &zero_weight;
    nca_cell_grads g = *grads;
    g.head_w = nullptr;
    g.head_b = nullptr;
    return backward_impl(d, packed, w, x, 0, given, &fd, fire, 1, &none, grad_out, &g, grad_x, nullptr,
                         workspace, workspace_bytes, reinterpret_cast<hipStream_t>(stream));
}

}  // extern "C"
