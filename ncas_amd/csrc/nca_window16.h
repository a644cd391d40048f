// Temporally blocked multi-step kernel for bf16 cells with C = 16 channels and 128 hidden units
// on grids whose rows do not fit one workgroup's LDS (the 201x201 mazes): T steps per launch,
// one workgroup per window of a board, everything between the window's load and its store in
// LDS (gfx950).
//
// A window is a core rectangle of the board plus a halo of T cells on every side that does not
// lie on the board's edge (wall / zero padding; with wrap padding every side has a halo, loaded
// at wrapped coordinates). Step s (0-based) of the launch computes the window shrunk by s + 1
// cells on its halo sides: a cell's new state needs its 3x3 neighbourhood, so the exact region
// loses one ring per step and after T steps is the core, which is written out. The cells outside
// the computed region, and a one-cell border ring around the window, are never read by a cell
// inside it (the border holds the padding value on board-edge sides). The core of every window
// is the board split into nwy x nwx near-equal rectangles, so every cell is written once.
//
// LDS: the fp32 state M (four planes of 16 B per cell, one per channel quad, each plane 256-byte
// aligned, so that a tile's 16 cells fill the 16 slots of a bank row; read and written only by the
// cell's own lanes, updated in place), the bf16 perception copy P twice (P_cur read by the
// stencils of a step, P_next written by its updates; 32 B per cell, window plus border), the
// given flags, and per wave one 4096-byte staging block for z (16 rows of 128 B) and then h (16
// rows of 256 B), whose 16-byte chunks are permuted per row (row_swz8, row_swz16) so that the
// MFMA operand reads are conflict-free. b1 lives in registers.
//
// Each cell of a step is computed exactly like the per-step kernel (step_stream16): lane
// (r = lane & 15, g = lane >> 4) of a 16-cell tile (a row segment of the computed region) owns
// cell r and channel quad g; the 3x3 stencil on v_dot2_f32_bf16 over the same tap pairs, z
// through the wave's staging block to fc1 (16 v_mfma_f32_16x16x32_bf16, W1 in registers, b1 as
// initial accumulators), ReLU'd bf16 h to fc2 (4 MFMAs) in natural hidden order, the update
// u = x + f * bf16(dx) with the input slice of given cells kept, and Philox fire bits keyed on
// (seed; row, step, cell quad) drawn four tiles at a time. So the results equal the per-step
// path's bit for bit. One workgroup barrier per step.
#pragma once

#include "nca_stream_util.h"

namespace nca {

constexpr int kWinMax = 30;                   // window edge in cells, halo included
constexpr int kWinStride = kWinMax + 2;       // P row stride in cells: window plus border ring
constexpr int kWinMaxT = 8;                   // steps per launch (the halo width)
constexpr unsigned kWinPBytes = kWinStride * kWinStride * 32;  // one bf16 perception copy
constexpr unsigned kWinMPlane = (kWinMax * kWinMax * 16 + 255) & ~255u;  // one channel quad of the state
constexpr unsigned kWinMBytes = 4 * kWinMPlane;                           // fp32 state
constexpr unsigned kWinGBytes = (kWinMax * kWinMax + 15) & ~15u;
constexpr unsigned kWinStage = 16 * 256;      // per wave: z (16 x 128 B), then h (16 x 256 B)
constexpr int kWinWaves = 8;
constexpr unsigned kWinLds = 2 * kWinPBytes + kWinMBytes + kWinGBytes + kWinWaves * kWinStage;
// staging offsets: chunk c of z row r, of h row r
__device__ __forceinline__ unsigned win_zoff(unsigned r, unsigned c) { return r * 128u + 16u * (c ^ row_swz8(r)); }
__device__ __forceinline__ unsigned win_hoff(unsigned r, unsigned c) { return r * 256u + 16u * (c ^ row_swz16(r)); }

struct Win16Params {
    RolloutParams a;        // x_in -> x_out of the launch
    int step;               // index in the call of the launch's first step (Philox counter, mask slice)
    int T;                  // steps of this launch, 1 .. kWinMaxT
    int first;              // the launch holds the call's first step: the clamp tensor's values
    int in_nchw, out_nchw;  // x_in / x_out in the caller's (rows, C, H, W) layout, else cell-major
    int nwy, nwx;           // windows per board along H and W
    int64_t n_windows;      // rows * nwy * nwx
};

// The core [lo, hi) of window i of n along an axis of length L (near-equal splits), its halos and
// whether each side is interior (not on the board's edge).
struct WinAxis {
    int lo, hi, h0, h1, in0, in1;
};
__host__ __device__ inline WinAxis win_axis(int i, int n, int L, int T, bool wrap) {
    WinAxis a;
    a.lo = (int)(((int64_t)i * L) / n);
    a.hi = (int)(((int64_t)(i + 1) * L) / n);
    if (wrap) {
        a.h0 = a.h1 = T;
        a.in0 = a.in1 = 1;
    } else {
        a.h0 = a.lo < T ? a.lo : T;
        a.h1 = L - a.hi < T ? L - a.hi : T;
        a.in0 = a.lo - a.h0 > 0;
        a.in1 = a.hi + a.h1 < L;
    }
    return a;
}

template <bool FIRST>
__global__ void __launch_bounds__(512, 1) rollout_window16(Win16Params wp) {
    constexpr int C = 16;
    const RolloutParams &a = wp.a;
    extern __shared__ __attribute__((aligned(16))) unsigned char win_lds[];
    unsigned char *const P0 = win_lds, *const P1 = win_lds + kWinPBytes;
    unsigned char *M = win_lds + 2 * kWinPBytes;
    unsigned char *G = M + kWinMBytes;
    unsigned char *stage = G + kWinGBytes;
    const int tid = threadIdx.x, lane = tid & 63, r = lane & 15, g = lane >> 4;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int H = a.H, W = a.W, HWn = H * W;
    const bool wrap = a.padding == 2;

    // ---- which window
    const int64_t b = blockIdx.x;
    const int per_row = wp.nwy * wp.nwx;
    const int64_t row = b / per_row;
    const int wi_ = (int)(b - row * per_row);
    const WinAxis ay = win_axis(wi_ / wp.nwx, wp.nwy, H, wp.T, wrap);
    const WinAxis ax = win_axis(wi_ % wp.nwx, wp.nwx, W, wp.T, wrap);
    const int WH = ay.h0 + (ay.hi - ay.lo) + ay.h1, WW = ax.h0 + (ax.hi - ax.lo) + ax.h1;
    const int by0 = ay.lo - ay.h0, bx0 = ax.lo - ax.h0;  // board coordinates of window cell (0, 0)

    // ---- constants (as step_stream16)
    // the stencil's B operands on v_mfma_f32_4x4x4_16b_bf16, as in step_stream16: kernel j = lane & 3,
    // one tap pair per MFMA (zeros in the other k slots), which sums as the v_dot2 chain does
    const float *kern = reinterpret_cast<const float *>(a.packed + a.off_kern);
    s16x4 kb[5];
    {
        const int j = r & 3;
        uint32_t kp[5];
#pragma unroll
        for (int p2 = 0; p2 < 4; ++p2) kp[p2] = pack_bf16x2(kern[j * 9 + 2 * p2], kern[j * 9 + 2 * p2 + 1]);
        kp[4] = pack_bf16x2(kern[j * 9 + 8], 0.0f);
#pragma unroll
        for (int p2 = 0; p2 < 5; ++p2)
            kb[p2] = __builtin_bit_cast(s16x4, (p2 & 1) ? make_uint2(0u, kp[p2]) : make_uint2(kp[p2], 0u));
    }
    bf16x8 w1f[8][2];
#pragma unroll
    for (int mt = 0; mt < 8; ++mt)
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
            w1f[mt][kt] = reinterpret_cast<const bf16x8 *>(a.packed + a.off_w1)[((size_t)mt * 2 + kt) * 64 + lane];
    bf16x8 w2f[4];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) w2f[kt] = reinterpret_cast<const bf16x8 *>(a.packed + a.off_w2)[(size_t)kt * 64 + lane];
    const float *b1 = reinterpret_cast<const float *>(a.packed + a.off_b1);
    const float *b2 = reinterpret_cast<const float *>(a.packed + a.off_b2);
    float4 b1v[8];  // fc1's initial accumulators: hidden units 16 mt + 4g .. +3
#pragma unroll
    for (int mt = 0; mt < 8; ++mt) b1v[mt] = *reinterpret_cast<const float4 *>(b1 + 16 * mt + 4 * g);
    float b2v[4];
    bool insl[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        b2v[v] = b2[4 * g + v];
        insl[v] = 4 * g + v >= a.in_off && 4 * g + v < a.in_off + a.c_in;
    }

    // ---- load the window: M (fp32), P_cur (bf16), given flags; the border ring of both P copies
    // holds the padding value on board-edge sides (wall: pad_vec, zero: 0) and 0 elsewhere
    {
        // a thread's loads all go out before its LDS stores: one store after each load would
        // wait for every load in turn (a quarter of a 2-step window's time)
        constexpr int kPer = (kWinMax * kWinMax * 4 + 511) / 512;
        const int n = WH * WW * 4;
        float4 lv[kPer];
        unsigned char lg[kPer];
#pragma unroll
        for (int k = 0; k < kPer; ++k) {
            const int e = tid + 512 * k;
            lv[k] = float4{0.f, 0.f, 0.f, 0.f};
            lg[k] = 0;
            if (e < n) {
                const int c = e >> 2, q = e & 3;
                const int wy = c / WW, wx = c - wy * WW;
                int bi = by0 + wy, bj = bx0 + wx;
                if (wrap) {
                    bi = ((bi % H) + H) % H;
                    bj = ((bj % W) + W) % W;
                }
                const int cell = bi * W + bj;
                if (wp.in_nchw) {
                    const float *xr = a.x_in + (row * C + 4 * q) * (int64_t)HWn + cell;
                    lv[k] = float4{xr[0], xr[HWn], xr[2 * (int64_t)HWn], xr[3 * (int64_t)HWn]};
                } else {
                    lv[k] = *reinterpret_cast<const float4 *>(a.x_in + (row * HWn + cell) * C + 4 * q);
                }
                if (q == 0) lg[k] = a.given[row * HWn + cell];
            }
        }
#pragma unroll
        for (int k = 0; k < kPer; ++k) {
            const int e = tid + 512 * k;
            if (e < n) {
                const int c = e >> 2, q = e & 3;
                const int wy = c / WW, wx = c - wy * WW;
                const float4 v = lv[k];
                lds_st128f(M, (unsigned)q * kWinMPlane + (unsigned)c * 16u, v);
                lds_st64(P0, (unsigned)(((wy + 1) * kWinStride + wx + 1) * 32 + 8 * q),
                         uint2{pack_bf16x2(v.x, v.y), pack_bf16x2(v.z, v.w)});
                if (q == 0) G[c] = lg[k];
            }
        }
        const int nb = 2 * (WW + 2) + 2 * WH;  // border cells
        for (int e = tid; e < nb * 4; e += 512) {
            const int k = e >> 2, q = e & 3;
            int py, px;  // border cell in P coordinates (window cell + 1)
            bool edge;   // on a board-edge side
            if (k < WW + 2) {
                py = 0;
                px = k;
                edge = !ay.in0;
            } else if (k < 2 * (WW + 2)) {
                py = WH + 1;
                px = k - (WW + 2);
                edge = !ay.in1;
            } else {
                const int k2 = k - 2 * (WW + 2);
                py = 1 + (k2 >> 1);
                px = (k2 & 1) ? WW + 1 : 0;
                edge = (k2 & 1) ? !ax.in1 : !ax.in0;
            }
            // a corner belongs to two sides: it is a padding cell when either side is the edge
            if (py == 0 || py == WH + 1) edge = edge || (px == 0 ? !ax.in0 : px == WW + 1 ? !ax.in1 : false);
            float4 pv = float4{};
            if (edge && a.padding == 1) {
                const float4 *pvq = reinterpret_cast<const float4 *>(a.packed + a.off_padv);
                pv = pvq[q];
            }
            const uint2 pb = uint2{pack_bf16x2(pv.x, pv.y), pack_bf16x2(pv.z, pv.w)};
            const unsigned off = (unsigned)((py * kWinStride + px) * 32 + 8 * q);
            lds_st64(P0, off, pb);
            lds_st64(P1, off, pb);
        }
    }
    const uint64_t key0 = a.seed;
    __syncthreads();

    unsigned char *zw = stage + w * kWinStage;  // z, then h, of the wave's tile
    int fired_run = 0;
    const bool philox = !a.fire_u8;
    for (int s = 0; s < wp.T; ++s) {
        const unsigned char *Pc = (s & 1) ? P1 : P0;
        unsigned char *Pn = (s & 1) ? P0 : P1;
        const int gs = wp.step + s;  // step index within the call
        const uint64_t key = a.step_seeds ? a.step_seeds[gs] : key0;
        const int r_lo = ay.in0 ? s + 1 : 0, r_hi = WH - (ay.in1 ? s + 1 : 0);
        const int c_lo = ax.in0 ? s + 1 : 0, c_hi = WW - (ax.in1 ? s + 1 : 0);
        const int ntx = (c_hi - c_lo + 15) >> 4;
        const int ntiles = (r_hi - r_lo) * ntx;
        uint64_t fmask = 0;
        int kgrp = 0;
        for (int t = w; t < ntiles; t += kWinWaves) {
            const int ty = t / ntx, tx = t - ty * ntx;
            const int wy = r_lo + ty, wx0 = c_lo + 16 * tx;
            const int wx = wx0 + r;
            const bool valid = wx < c_hi;
            const int wxc = valid ? wx : c_hi - 1;
            // Philox bits of this tile and the wave's next three: lane (r, g) draws cell r of the
            // tile g turns ahead
            if (philox && kgrp == 0) {
                const int t2 = t + kWinWaves * g;
                const int ty2 = t2 / ntx, tx2 = t2 - ty2 * ntx;
                int wy2 = r_lo + ty2, wx2 = c_lo + 16 * tx2 + r;
                wy2 = wy2 < r_hi ? wy2 : r_hi - 1;
                wx2 = wx2 < c_hi ? wx2 : c_hi - 1;
                int bi = by0 + wy2, bj = bx0 + wx2;
                if (wrap) {
                    bi = ((bi % H) + H) % H;
                    bj = ((bj % W) + W) % W;
                }
                const int cell = bi * W + bj;
                float u4[4];
                cell_uniforms4(key, (uint32_t)(a.row0 + row), (uint32_t)(a.step0 + gs), (uint32_t)(cell >> 2), u4);
                const int e4 = cell & 3;
                const float uq = e4 == 0 ? u4[0] : e4 == 1 ? u4[1] : e4 == 2 ? u4[2] : u4[3];
                fmask = __ballot(uq < a.p);
            }
            const int pidx = (wy + 1) * kWinStride + wxc + 1;
            // 1. taps: quad g of the 9 neighbours, bf16
            uint32_t tb[9][2];
#pragma unroll
            for (int tt = 0; tt < 9; ++tt) {
                const int dy = tt / 3, dx = tt % 3;
                const uint2 v = lds_ld64(Pc, (unsigned)((pidx + (dy - 1) * kWinStride + (dx - 1)) * 32 + 8 * g));
                tb[tt][0] = v.x;
                tb[tt][1] = v.y;
            }
            // 2. perception (five 4x4x4 MFMAs per channel over the tap pairs) -> z in the staging
            // block; lane (r, g) receives kernel j = r & 3 of cells 4 (r >> 2) + i, channel 4 g + c
            {
                typedef uint32_t w16_u32x2 __attribute__((ext_vector_type(2)));
                w16_u32x2 ta[4], tbp[4], tc[4];
#pragma unroll
                for (int q = 0; q < 2; ++q) {  // taps 4q .. 4q + 3 -> ta (q = 0) or tbp (q = 1)
                    const uint32_t *x0 = tb[4 * q], *x1 = tb[4 * q + 1], *x2 = tb[4 * q + 2], *x3 = tb[4 * q + 3];
                    w16_u32x2 *dst = q ? tbp : ta;
                    dst[0] = w16_u32x2{__builtin_amdgcn_perm(x1[0], x0[0], 0x05040100u),
                                       __builtin_amdgcn_perm(x3[0], x2[0], 0x05040100u)};
                    dst[1] = w16_u32x2{__builtin_amdgcn_perm(x1[0], x0[0], 0x07060302u),
                                       __builtin_amdgcn_perm(x3[0], x2[0], 0x07060302u)};
                    dst[2] = w16_u32x2{__builtin_amdgcn_perm(x1[1], x0[1], 0x05040100u),
                                       __builtin_amdgcn_perm(x3[1], x2[1], 0x05040100u)};
                    dst[3] = w16_u32x2{__builtin_amdgcn_perm(x1[1], x0[1], 0x07060302u),
                                       __builtin_amdgcn_perm(x3[1], x2[1], 0x07060302u)};
                }
                tc[0] = w16_u32x2{tb[8][0] & 0xffffu, 0u};
                tc[1] = w16_u32x2{tb[8][0] >> 16, 0u};
                tc[2] = w16_u32x2{tb[8][1] & 0xffffu, 0u};
                tc[3] = w16_u32x2{tb[8][1] >> 16, 0u};
                typedef float w16_zf32x4 __attribute__((ext_vector_type(4)));
                w16_zf32x4 zc[4];
#pragma unroll
                for (int c = 0; c < 4; ++c) zc[c] = w16_zf32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int p2 = 0; p2 < 5; ++p2)
#pragma unroll
                    for (int c = 0; c < 4; ++c) {
                        const w16_u32x2 av = p2 < 2 ? ta[c] : p2 < 4 ? tbp[c] : tc[c];
                        zc[c] = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(__builtin_bit_cast(s16x4, av), kb[p2], zc[c], 0,
                                                                       0, 0);
                    }
                const int j = r & 3, c0 = 4 * (r >> 2);
#pragma unroll
                for (int i = 0; i < 4; ++i)  // features 16 j + 4g .. +3 of cell c0 + i: chunk 2j + g / 2, half g & 1
                    *reinterpret_cast<uint2 *>(zw + win_zoff(c0 + i, 2 * j + (g >> 1)) + 8 * (g & 1)) =
                        uint2{pack_bf16x2(zc[0][i], zc[1][i]), pack_bf16x2(zc[2][i], zc[3][i])};
            }
            // 3. fc1
            __builtin_amdgcn_wave_barrier();
            const bf16x8 zf0 = *reinterpret_cast<const bf16x8 *>(zw + win_zoff(r, g));
            const bf16x8 zf1 = *reinterpret_cast<const bf16x8 *>(zw + win_zoff(r, 4 + g));
            typedef float w16_f32x4 __attribute__((ext_vector_type(4)));
            w16_f32x4 h[8];
#pragma unroll
            for (int mt = 0; mt < 8; ++mt) {
                h[mt] = w16_f32x4{b1v[mt].x, b1v[mt].y, b1v[mt].z, b1v[mt].w};
                h[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(w1f[mt][0], zf0, h[mt], 0, 0, 0);
                h[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(w1f[mt][1], zf1, h[mt], 0, 0, 0);
            }
            // 4. fc2 on the ReLU'd bf16 activations (the staging block now holds h: the z reads
            // above fed the MFMAs whose results these writes store)
#pragma unroll
            for (int mt = 0; mt < 8; ++mt)  // hidden 16 mt + 4g .. +3: chunk 2 mt + g / 2, half g & 1
                *reinterpret_cast<uint2 *>(zw + win_hoff(r, 2 * mt + (g >> 1)) + 8 * (g & 1)) =
                    uint2{relu_bf16x2(cvt_pk_bf16(h[mt][0], h[mt][1])), relu_bf16x2(cvt_pk_bf16(h[mt][2], h[mt][3]))};
            __builtin_amdgcn_wave_barrier();
            w16_f32x4 dx = w16_f32x4{b2v[0], b2v[1], b2v[2], b2v[3]};
#pragma unroll
            for (int kt = 0; kt < 4; ++kt) {
                const bf16x8 hf = *reinterpret_cast<const bf16x8 *>(zw + win_hoff(r, 4 * kt + g));
                dx = __builtin_amdgcn_mfma_f32_16x16x32_bf16(w2f[kt], hf, dx, 0, 0, 0);
            }
            // 5. update of the cell's quad
            int bi = by0 + wy, bj = bx0 + wxc;
            if (wrap) {
                bi = ((bi % H) + H) % H;
                bj = ((bj % W) + W) % W;
            }
            const int cell = bi * W + bj;
            float f;
            if (a.fire_u8) {
                f = a.fire_u8[((int64_t)gs * a.rows + row) * HWn + cell] ? 1.0f : 0.0f;
            } else {
                f = ((fmask >> (16 * kgrp + r)) & 1ull) ? 1.0f : 0.0f;
            }
            const int mc = wy * WW + wxc;
            const bool gv = G[mc] != 0;
            const unsigned moff = (unsigned)g * kWinMPlane + (unsigned)mc * 16u;
            const float4 xq = lds_ld128f(M, moff);
            float xo[4] = {xq.x, xq.y, xq.z, xq.w};
            if (FIRST && s == 0 && gv) {
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int ci = insl[v] ? 4 * g + v - a.in_off : 0;
                    if (insl[v] && a.c_in > 0) xo[v] = a.clamp[(row * a.c_in + ci) * (int64_t)HWn + cell];
                }
            }
            float u[4];
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const float uv = __fadd_rn(xo[v], __fmul_rn(f, round_bf16(dx[v])));
                u[v] = (gv && insl[v]) ? xo[v] : uv;
            }
            if (valid) {
                lds_st128f(M, moff, make_float4(u[0], u[1], u[2], u[3]));
                lds_st64(Pn, (unsigned)(pidx * 32 + 8 * g), uint2{pack_bf16x2(u[0], u[1]), pack_bf16x2(u[2], u[3])});
            }
            // fired cells of the core, once per cell (quad 0)
            const bool core = wy >= ay.h0 && wy < WH - ay.h1 && wx >= ax.h0 && wx < WW - ax.h1;
            fired_run += (valid && core && g == 0 && f != 0.0f) ? 1 : 0;
            kgrp = (kgrp + 1) & 3;
        }
        __syncthreads();
    }

    // ---- the core to x_out
    {
        const int CHn = ay.hi - ay.lo, CWn = ax.hi - ax.lo;
        const int n = CHn * CWn * 4;
        for (int e = tid; e < n; e += 512) {
            const int c = e >> 2, q = e & 3;
            const int cy = c / CWn, cx = c - cy * CWn;
            const int mc = (cy + ay.h0) * WW + cx + ax.h0;
            const float4 v = lds_ld128f(M, (unsigned)q * kWinMPlane + (unsigned)mc * 16u);
            const int cell = (ay.lo + cy) * W + ax.lo + cx;
            if (wp.out_nchw) {
                float *xr = a.x_out + (row * C + 4 * q) * (int64_t)HWn + cell;
                xr[0] = v.x;
                xr[HWn] = v.y;
                xr[2 * (int64_t)HWn] = v.z;
                xr[3 * (int64_t)HWn] = v.w;
            } else {
                *reinterpret_cast<float4 *>(a.x_out + (row * HWn + cell) * C + 4 * q) = v;
            }
        }
    }
    if (a.fired_out) {
        int sum = fired_run;
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) sum += __shfl_xor(sum, o);
        if (lane == 0 && sum) atomicAdd(a.fired_out + row, sum);
    }
}

}  // namespace nca
