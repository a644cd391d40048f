// The halo-tiled per-step kernel (gfx950): one NCA step over grids of any size.
//
// Used where a row's state does not fit one workgroup's LDS for a whole rollout (201x201
// mazes with C=16; 30x30 boards with C=32 x many rows), and for single steps on such grids.
// One launch advances every row one step, reading the state from x_in and writing x_out
// (fp32 NCHW, the reference layout); a rollout ping-pongs two state buffers across launches.
//
// Each workgroup (4 waves) is persistent over windows: a window is a TH x TW block of cells of
// one row (TW <= 32). For each window it
//   1. loads the window plus a 1-cell halo from x_in into the perception buffer P (bf16 for bf16
//      cells, fp32 otherwise): halo cells inside the grid come from the neighbouring windows'
//      cells, halo cells outside it follow the padding rule (wall: pad_vec, zero: 0, wrap:
//      the wrapped cell) - reference src/nca/model.py:140-152. Lanes 0-31 of each half-wave
//      read 32 consecutive cells of one (channel, grid row) line, so every load is one
//      128-byte segment. The interior also goes to the fp32 state M;
//   2. draws the fire mask of its cells (Philox keyed on (seed; row, step, cell quad), the same
//      counters as the resident kernels; adaptive firing reads the pre-step confidence from M),
//      or reads the injected mask;
//   3. on the first step of a call, sets the input slice of given cells to the clamp values
//      (model.py:430-438) in M; perception still reads the unclamped state in P;
//   4. runs the tile pipeline over super-tiles of CPI = 1024 / C cells (4, 2 or 1 tiles of 16
//      cells for C = 16, 32, 64), one workgroup barrier per super-tile: stencil of super-tile
//      t+1 (one (cell, channel quad) item per thread), fc1 of super-tile t (wave w: hidden units
//      [w HD/4, (w+1) HD/4) of every 16-cell tile), fc2 + residual update of super-tile t-1
//      (wave w: one (16-channel m-tile, 16-cell tile) pair - there are exactly four). W1/W2
//      fragments stay in registers. The update writes M only, so P stays the step's input;
//   5. writes M to x_out.
// Between the steps of a call the state lives in the caller's workspace in cell-major order
// (rows, H, W, C), so that the later steps load and store whole 16-byte channel quads of
// contiguous cells; only the first step reads the caller's NCHW state (a 128-byte line segment
// of one channel per 32 lanes) and only the last writes it. Every window reads only x_in and
// writes only x_out, so windows need no synchronisation with each other; the launch boundary
// is the step boundary.
#pragma once

#include "nca_rollout.h"

namespace nca {

struct TiledParams {
    RolloutParams a;   // x_in -> x_out of this step (n_steps, rows_per_wg unused)
    int step;          // step index within the call: Philox counter step0 + step, mask slice
    int first;         // first step of the call: apply the clamp
    int in_nchw;       // x_in is the caller's (rows, C, H, W) state, else cell-major (rows, H, W, C)
    int out_nchw;      // x_out is the caller's (rows, C, H, W) state, else cell-major
    int TH, TW;        // window interior (cells), TW <= 32
    int tiles_y, tiles_x;
    int64_t n_windows;  // rows * tiles_y * tiles_x
    unsigned l_P, l_M, l_Z, l_H, l_given, l_fire, l_cinfo, l_head, l_fired;
};

template <int C, int HD, bool BF16>
struct TShape {
    static constexpr int TPI = 64 / C;         // 16-cell tiles per super-tile
    static constexpr int CPI = 16 * TPI;       // cells per super-tile (and per interval)
    static constexpr int CPI_LOG = C == 16 ? 6 : C == 32 ? 5 : 4;
    static constexpr int F = 4 * C;            // features (4 perception kernels)
    static constexpr int KT = BF16 ? 32 : 4;   // MFMA k per instruction
    static constexpr int HPW = HD / 4;         // fc1 hidden units per wave
    static constexpr int MT1 = HPW / 16;       // fc1 m-tiles per wave
    static constexpr int KT1 = F / KT;         // fc1 k-tiles
    static constexpr int MT2 = C / 16;         // fc2 m-tiles
    static constexpr int KT2 = HD / KT;        // fc2 k-tiles
    static constexpr int ES = BF16 ? 2 : 4;    // bytes per element of P, Z, H
    static constexpr int CP = C + 4;           // P cell stride (elements)
    static constexpr int MP = C + 4;           // M cell stride (floats)
    static constexpr int ZS = F + (BF16 ? 8 : 4);
    static constexpr int HS = HD + (BF16 ? 8 : 4);
    static constexpr int ZBUF = CPI * ZS;      // elements per Z buffer
    static constexpr int HBUF = CPI * HS;      // elements per H buffer
    static_assert(C == 16 || C == 32 || C == 64, "C must be 16, 32 or 64");
    static_assert(MT2 * TPI == 4, "one fc2 (m-tile, tile) pair per wave");
    static_assert(CPI * (C / 4) == 256, "one stencil item per thread");
    static_assert(HD % 64 == 0, "hidden must be a multiple of 64");
};

struct TiledPlan {
    unsigned P, M, Z, H, given, fire, cinfo, head, fired, total;
};

template <int C, int HD, bool BF16>
inline TiledPlan tiled_plan(int TH, int TW, int c_out, int n_out) {
    using T = TShape<C, HD, BF16>;
    auto al = [](unsigned v) { return (v + 15u) & ~15u; };
    const unsigned cells = (unsigned)TH * TW, pcells = (unsigned)(TH + 2) * (TW + 2);
    TiledPlan p;
    unsigned o = 0;
    p.P = o;
    o = al(o + pcells * T::CP * T::ES);
    p.M = o;
    o = al(o + cells * T::MP * 4u);
    p.Z = o;
    o = al(o + 2u * T::ZBUF * T::ES);
    p.H = o;
    o = al(o + 2u * T::HBUF * T::ES);
    p.given = o;
    o = al(o + cells);
    p.fire = o;
    o = al(o + cells * 4u);
    p.cinfo = o;
    o = al(o + cells * 4u);
    p.head = o;
    o = al(o + (unsigned)(n_out * c_out + n_out) * 4u);
    p.fired = o;
    o = al(o + 4u);
    p.total = o;
    return p;
}

template <int C, int HD, bool BF16, bool NOISE>
__global__ void __launch_bounds__(256, 1) step_tiled(TiledParams tp) {
    using T = TShape<C, HD, BF16>;
    using FR = Frag<BF16>;
    using fr_t = typename FR::type;
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    const RolloutParams &a = tp.a;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, l16 = lane & 15;
    const int lj = tid & 31, lg = tid >> 5;  // line lane (column), line group (8 groups)
    const int H = a.H, W = a.W, HWn = H * W;
    const int TH = tp.TH, TW = tp.TW, PW = TW + 2;
    const int c_in = a.c_in, in_off = a.in_off;
    constexpr int Q = C / 4, QLOG = C == 16 ? 2 : C == 32 ? 3 : 4;  // channel quads per cell

    unsigned char *Pb = smem + tp.l_P;
    float *M = reinterpret_cast<float *>(smem + tp.l_M);
    unsigned char *Zb = smem + tp.l_Z;
    unsigned char *Hb = smem + tp.l_H;
    uint8_t *givenL = smem + tp.l_given;
    float *fireL = reinterpret_cast<float *>(smem + tp.l_fire);
    int *cinfo = reinterpret_cast<int *>(smem + tp.l_cinfo);
    float *headL = reinterpret_cast<float *>(smem + tp.l_head);
    int *firedL = reinterpret_cast<int *>(smem + tp.l_fired);

    // ---- stencil kernels (uniform) and tap offsets in P elements (window row pitch PW cells)
    const float *kern = reinterpret_cast<const float *>(a.packed + a.off_kern);
    float kw[4][9];
    uint32_t kp[4][5];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
#pragma unroll
        for (int t = 0; t < 9; ++t) kw[k][t] = kern[k * 9 + t];
#pragma unroll
        for (int pr = 0; pr < 4; ++pr) kp[k][pr] = pack_bf16x2(kw[k][2 * pr], kw[k][2 * pr + 1]);
        kp[k][4] = pack_bf16x2(kw[k][8], 0.0f);
    }
    int toff[9];
#pragma unroll
    for (int t = 0; t < 9; ++t) toff[t] = ((t / 3 - 1) * PW + (t % 3 - 1)) * T::CP;

    // ---- MLP fragments and biases in registers
    const float *b1 = reinterpret_cast<const float *>(a.packed + a.off_b1);
    const float *b2 = reinterpret_cast<const float *>(a.packed + a.off_b2);
    fr_t w1f[T::MT1][T::KT1];
    f32x4 b1v[T::MT1];
#pragma unroll
    for (int mt = 0; mt < T::MT1; ++mt) {
#pragma unroll
        for (int kt = 0; kt < T::KT1; ++kt) {
            const size_t idx = ((size_t)(wave * T::MT1 + mt) * T::KT1 + kt) * 64 + lane;
            w1f[mt][kt] = reinterpret_cast<const fr_t *>(a.packed + a.off_w1)[idx];
        }
#pragma unroll
        for (int v = 0; v < 4; ++v) b1v[mt][v] = b1[wave * T::HPW + 16 * mt + 4 * g + v];
    }
    const int mt2 = wave % T::MT2, tt2 = wave / T::MT2;  // this wave's fc2 pair
    fr_t w2f[T::KT2];
    f32x4 b2v;
    bool insl[4];
    // fp32 cells with C = 16 and 128 hidden units sum fc2 as the resident kernel does: four partial
    // sums over hidden units [32 p, 32 p + 32) (the first from b2), each an MFMA chain over k-tiles
    // (mt, v) = hidden units 32 p + 16 mt + 4 k + v, k = 0..3, added in order p = 0..3
    constexpr bool KS = !BF16 && C == 16 && HD == 128;
#pragma unroll
    for (int kt = 0; kt < T::KT2; ++kt)
        w2f[kt] = reinterpret_cast<const fr_t *>(a.packed + a.off_w2)[KS ? (size_t)(8 * (kt >> 3) + 4 * ((kt >> 2) & 1) + g) * 64 + 16 * (kt & 3) + l16
                                                                          : ((size_t)mt2 * T::KT2 + kt) * 64 + lane];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        const int c = 16 * mt2 + 4 * g + v;
        b2v[v] = b2[c];
        insl[v] = c >= in_off && c < in_off + c_in;
    }
    {
        const float *hw = reinterpret_cast<const float *>(a.packed + a.off_headw);
        const float *hb = reinterpret_cast<const float *>(a.packed + a.off_headb);
        const int nw = a.n_out * a.c_out;
        for (int e = tid; e < nw + a.n_out; e += 256) headL[e] = e < nw ? hw[e] : hb[e - nw];
    }
    const float *padv = reinterpret_cast<const float *>(a.packed + a.off_padv);
    const uint64_t key = a.step_seeds ? a.step_seeds[tp.step] : a.seed;

    // ---- pipeline stages over super-tiles of CPI cells
    int ncell = 0;
    const int st_n = tid & (T::CPI - 1), st_qd = tid >> T::CPI_LOG;

    auto stencil_pc = [&](int t) {
        const int gq = t * T::CPI + st_n;
        return cinfo[gq < ncell ? gq : ncell - 1];
    };
    // stencil of one super-tile: this thread's cell centre pc, channel quad st_qd -> Z[zb]
    auto stencil = [&](int pc, int zb) {
        const int base = pc + 4 * st_qd;
        float acc[4][4];
        if constexpr (BF16) {
            uint2 nb[9];
#pragma unroll
            for (int t9 = 0; t9 < 9; ++t9) nb[t9] = *reinterpret_cast<const uint2 *>(Pb + 2 * (base + toff[t9]));
            uint32_t pr[5][4];  // [tap pair][channel]
#pragma unroll
            for (int p2 = 0; p2 < 4; ++p2) {
                const uint2 x0 = nb[2 * p2], x1 = nb[2 * p2 + 1];
                pr[p2][0] = __builtin_amdgcn_perm(x1.x, x0.x, 0x05040100u);
                pr[p2][1] = __builtin_amdgcn_perm(x1.x, x0.x, 0x07060302u);
                pr[p2][2] = __builtin_amdgcn_perm(x1.y, x0.y, 0x05040100u);
                pr[p2][3] = __builtin_amdgcn_perm(x1.y, x0.y, 0x07060302u);
            }
            pr[4][0] = nb[8].x & 0xffffu;
            pr[4][1] = nb[8].x >> 16;
            pr[4][2] = nb[8].y & 0xffffu;
            pr[4][3] = nb[8].y >> 16;
#pragma unroll
            for (int k = 0; k < 4; ++k)
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    float s = dot2_bf16_zero(pr[0][c], kp[k][0]);
#pragma unroll
                    for (int p2 = 1; p2 < 5; ++p2)
                        s = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(pr[p2][c]), as_bf16x2(kp[k][p2]), s, false);
                    acc[k][c] = s;
                }
        } else {
#pragma unroll
            for (int k = 0; k < 4; ++k)
#pragma unroll
                for (int c = 0; c < 4; ++c) acc[k][c] = 0.0f;
#pragma unroll
            for (int t9 = 0; t9 < 9; ++t9) {
                float v[4];
                lds_load4<false>(Pb, base + toff[t9], v);
#pragma unroll
                for (int k = 0; k < 4; ++k)
#pragma unroll
                    for (int c = 0; c < 4; ++c) acc[k][c] = __builtin_fmaf(kw[k][t9], v[c], acc[k][c]);
            }
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) lds_store4<BF16>(Zb, zb * T::ZBUF + st_n * T::ZS + k * C + 4 * st_qd, acc[k]);
    };
    // fc1 of the super-tile in Z[zb] -> H[hb]: every 16-cell tile, this wave's hidden units
    auto fc1 = [&](int zb, int hb) {
#pragma unroll
        for (int tt = 0; tt < T::TPI; ++tt) {
            const int zrow = zb * T::ZBUF + (tt * 16 + l16) * T::ZS + (BF16 ? 8 * g : g);
            fr_t zf[T::KT1];
#pragma unroll
            for (int kt = 0; kt < T::KT1; ++kt) zf[kt] = FR::load_lds(Zb, zrow + kt * T::KT);
            f32x4 acc[T::MT1];
#pragma unroll
            for (int mt = 0; mt < T::MT1; ++mt) acc[mt] = b1v[mt];
#pragma unroll
            for (int kt = 0; kt < T::KT1; ++kt)
#pragma unroll
                for (int mt = 0; mt < T::MT1; ++mt) acc[mt] = FR::mfma(w1f[mt][kt], zf[kt], acc[mt]);
#pragma unroll
            for (int mt = 0; mt < T::MT1; ++mt) {
                float h[4];
#pragma unroll
                for (int v = 0; v < 4; ++v) h[v] = acc[mt][v] > 0.0f ? acc[mt][v] : 0.0f;
                lds_store4<BF16>(Hb, hb * T::HBUF + (tt * 16 + l16) * T::HS + wave * T::HPW + 16 * mt + 4 * g, h);
            }
        }
    };
    // fc2 + residual update of this wave's (m-tile, tile) pair of super-tile t (H[hb]) into M.
    // Input-slice channels of given cells keep their value in M (the clamp values after the
    // first step's clamp pass).
    auto fc2_update = [&](int t, int hb, int64_t row, int i0, int j0, int tw) {
        const int gq = t * T::CPI + tt2 * 16 + l16;
        const int gc = gq < ncell ? gq : ncell - 1;
        const float f = fireL[gc];
        const bool gv = givenL[gc] != 0;
        const int c0 = 16 * mt2 + 4 * g;
        const float4 m4 = *reinterpret_cast<const float4 *>(M + gc * T::MP + c0);
        const float xo[4] = {m4.x, m4.y, m4.z, m4.w};
        const int hrow = hb * T::HBUF + (tt2 * 16 + l16) * T::HS + (BF16 ? 8 * g : g);
        fr_t hf[T::KT2];
        f32x4 acc2 = b2v;
        if constexpr (KS) {
            // k-tile 8 p + 4 mt + v: hidden unit 32 p + 16 mt + 4 g + v of the lane's cell
            const int hrow_k = hb * T::HBUF + (tt2 * 16 + l16) * T::HS + 4 * g;
#pragma unroll
            for (int kt = 0; kt < T::KT2; ++kt) hf[kt] = FR::load_lds(Hb, hrow_k + 32 * (kt >> 3) + 16 * ((kt >> 2) & 1) + (kt & 3));
            f32x4 part[4];
#pragma unroll
            for (int p4 = 0; p4 < 4; ++p4) {
                part[p4] = p4 == 0 ? b2v : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int k8 = 0; k8 < 8; ++k8) part[p4] = FR::mfma(w2f[8 * p4 + k8], hf[8 * p4 + k8], part[p4]);
            }
#pragma unroll
            for (int v = 0; v < 4; ++v)
                acc2[v] = __fadd_rn(__fadd_rn(__fadd_rn(part[0][v], part[1][v]), part[2][v]), part[3][v]);
        } else {
#pragma unroll
            for (int kt = 0; kt < T::KT2; ++kt) hf[kt] = FR::load_lds(Hb, hrow + kt * T::KT);
#pragma unroll
            for (int kt = 0; kt < T::KT2; ++kt) acc2 = FR::mfma(w2f[kt], hf[kt], acc2);
        }
        float u[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const float dxv = BF16 ? round_bf16(acc2[v]) : acc2[v];
            float uv = __fadd_rn(xo[v], __fmul_rn(f, dxv));
            if constexpr (NOISE) {
                const int i = gc / tw, j = gc - i * tw;
                uv = __fadd_rn(uv, a.noise[((row * C + c0 + v) * H + i0 + i) * (int64_t)W + j0 + j]);
            }
            u[v] = (gv && insl[v]) ? xo[v] : uv;
        }
        if (gq < ncell) *reinterpret_cast<float4 *>(M + gc * T::MP + c0) = make_float4(u[0], u[1], u[2], u[3]);
    };
    auto put_p = [&](int ii, int jj, int c, float v) {
        const int pe = (ii * PW + jj) * T::CP + c;
        if constexpr (BF16)
            reinterpret_cast<__bf16 *>(Pb)[pe] = (__bf16)v;
        else
            reinterpret_cast<float *>(Pb)[pe] = v;
    };

    const int64_t per_row = (int64_t)tp.tiles_y * tp.tiles_x;
    for (int64_t win = blockIdx.x; win < tp.n_windows; win += gridDim.x) {
        const int64_t row = win / per_row;
        const int wr = (int)(win - row * per_row), ty = wr / tp.tiles_x, tx = wr - ty * tp.tiles_x;
        const int i0 = ty * TH, j0 = tx * TW;
        const int th = H - i0 < TH ? H - i0 : TH, tw = W - j0 < TW ? W - j0 : TW;
        ncell = th * tw;
        const int ntile = (ncell + T::CPI - 1) / T::CPI;
        const float *xr = a.x_in + row * C * (int64_t)HWn;
        // value of channel c at grid cell (gi, gj), which may lie outside the grid (padding rule)
        auto fetch = [&](int c, int gi, int gj) -> float {
            const bool inside = gi >= 0 && gi < H && gj >= 0 && gj < W;
            if (inside || a.padding == 2) {
                if (!inside) {
                    gi = (gi + H) % H;
                    gj = (gj + W) % W;
                }
                return xr[(int64_t)c * HWn + gi * W + gj];
            }
            return a.padding == 1 ? padv[c] : 0.0f;
        };

        // 1. window + halo -> P, interior -> M
        const int ph = th + 2, pw = tw + 2;
        if (tp.in_nchw) {
            // the caller's NCHW state (first step of a call). Interior columns: lane lj of line
            // group lg takes lines L = lg + 8 m of the C x (th + 2) (channel, window row) lines,
            // 32 lines per batch with every load of a batch issued before the first LDS store;
            // then the two halo columns.
            const int nlines = C * ph;
            if (lj < tw) {
                int c = 0, ii = lg;
                while (ii >= ph) {
                    ii -= ph;
                    ++c;
                }
                for (int L0 = lg; L0 < nlines; L0 += 8 * 32) {
                    float v[32];
                    int cs = c, is = ii;
#pragma unroll
                    for (int m = 0; m < 32; ++m) {
                        v[m] = (L0 + 8 * m < nlines) ? fetch(cs, i0 + is - 1, j0 + lj) : 0.0f;
                        is += 8;
                        while (is >= ph) {
                            is -= ph;
                            ++cs;
                        }
                    }
#pragma unroll
                    for (int m = 0; m < 32; ++m) {
                        if (L0 + 8 * m < nlines) {
                            put_p(ii, lj + 1, c, v[m]);
                            if (ii >= 1 && ii <= th) M[((ii - 1) * tw + lj) * T::MP + c] = v[m];
                        }
                        ii += 8;
                        while (ii >= ph) {
                            ii -= ph;
                            ++c;
                        }
                    }
                }
            }
            for (int e = tid; e < 2 * ph * C; e += 256) {
                const int side = e & 1, rest = e >> 1, c = rest / ph, ii = rest - c * ph;
                const int jj = side ? tw + 1 : 0;
                put_p(ii, jj, c, fetch(c, i0 + ii - 1, j0 + jj - 1));
            }
        } else {
            // cell-major state (steps after the first): items (window row, cell, channel quad)
            // of the window + halo, consecutive threads on consecutive 16-byte quads, 8 loads in
            // flight per thread
            const int ipr = pw * Q;  // items per window row
            const int nitems = ph * ipr;
            const float *xc = a.x_in + row * (int64_t)HWn * C;
            int ii = 0, rem = tid;
            while (rem >= ipr) {
                rem -= ipr;
                ++ii;
            }
            for (int e0 = tid; e0 < nitems; e0 += 256 * 8) {
                float4 v[8];
                int iis[8], rms[8];
#pragma unroll
                for (int m = 0; m < 8; ++m) {
                    iis[m] = ii;
                    rms[m] = rem;
                    v[m] = make_float4(0.f, 0.f, 0.f, 0.f);
                    if (e0 + 256 * m < nitems) {
                        const int jj = rem >> QLOG, q = rem & (Q - 1);
                        int gi = i0 + ii - 1, gj = j0 + jj - 1;
                        const bool inside = gi >= 0 && gi < H && gj >= 0 && gj < W;
                        if (inside || a.padding == 2) {
                            if (!inside) {
                                gi = (gi + H) % H;
                                gj = (gj + W) % W;
                            }
                            v[m] = *reinterpret_cast<const float4 *>(xc + ((int64_t)gi * W + gj) * C + 4 * q);
                        } else if (a.padding == 1) {
                            v[m] = *reinterpret_cast<const float4 *>(padv + 4 * q);
                        }
                    }
                    rem += 256;
                    while (rem >= ipr) {
                        rem -= ipr;
                        ++ii;
                    }
                }
#pragma unroll
                for (int m = 0; m < 8; ++m) {
                    if (e0 + 256 * m < nitems) {
                        const int jj = rms[m] >> QLOG, q = rms[m] & (Q - 1), iv = iis[m];
                        const float vv[4] = {v[m].x, v[m].y, v[m].z, v[m].w};
                        lds_store4<BF16>(Pb, (iv * PW + jj) * T::CP + 4 * q, vv);
                        if (iv >= 1 && iv <= th && jj >= 1 && jj <= tw)
                            *reinterpret_cast<float4 *>(M + ((iv - 1) * tw + jj - 1) * T::MP + 4 * q) = v[m];
                    }
                }
            }
        }
        if (lj < tw)
            for (int i = lg; i < th; i += 8) {
                const int k = i * tw + lj;
                givenL[k] = a.given[row * HWn + (i0 + i) * W + j0 + lj];
                cinfo[k] = ((i + 1) * PW + lj + 1) * T::CP;
            }
        if (tid == 0) *firedL = 0;
        __syncthreads();

        // 2. fire mask of the window's cells (pre-step state, before the clamp)
        if (lj < tw)
            for (int i = lg; i < th; i += 8) {
                const int k = i * tw + lj, q = (i0 + i) * W + j0 + lj;
                float f;
                if (a.fire_f32) {
                    f = a.fire_f32[row * HWn + q];
                } else if (a.fire_u8) {
                    f = a.fire_u8[((int64_t)tp.step * a.rows + row) * HWn + q] ? 1.0f : 0.0f;
                } else {
                    float u[4];
                    cell_uniforms4(key, (uint32_t)(a.row0 + row), (uint32_t)(a.step0 + tp.step), (uint32_t)(q >> 2), u);
                    const int e4 = q & 3;
                    const float uq = e4 == 0 ? u[0] : e4 == 1 ? u[1] : e4 == 2 ? u[2] : u[3];
                    float pc = a.p;
                    if (a.adaptive) {
                        int am;
                        const float cf = cell_readout(M + k * T::MP + a.out_off, 1, a.c_out, a.n_out, a.head_kind,
                                                      headL, headL + a.n_out * a.c_out, &am);
                        if (cf > a.tau || (a.given_confident && givenL[k])) pc = a.p_low;
                    }
                    f = uq < pc ? 1.0f : 0.0f;
                }
                fireL[k] = f;
                if (f != 0.0f) atomicAdd(firedL, 1);
            }
        __syncthreads();
        // 3. the first step's clamp of the given cells' input slice (M only)
        if (tp.first && c_in > 0) {
            if (lj < tw)
                for (int ci = 0; ci < c_in; ++ci)
                    for (int i = lg; i < th; i += 8) {
                        const int k = i * tw + lj;
                        if (givenL[k])
                            M[k * T::MP + in_off + ci] = a.clamp[((row * c_in + ci) * H + i0 + i) * (int64_t)W + j0 + lj];
                    }
            __syncthreads();
        }

        // 4. super-tile pipeline
        stencil(stencil_pc(0), 0);
        __syncthreads();
        fc1(0, 0);
        if (ntile > 1) stencil(stencil_pc(1), 1);
        __syncthreads();
        for (int t = 1; t + 1 < ntile; ++t) {
            fc2_update(t - 1, (t - 1) & 1, row, i0, j0, tw);
            fc1(t & 1, t & 1);
            stencil(stencil_pc(t + 1), (t + 1) & 1);
            __syncthreads();
        }
        if (ntile > 1) {
            fc2_update(ntile - 2, (ntile - 2) & 1, row, i0, j0, tw);
            fc1((ntile - 1) & 1, (ntile - 1) & 1);
            __syncthreads();
        }
        fc2_update(ntile - 1, (ntile - 1) & 1, row, i0, j0, tw);
        __syncthreads();

        // 5. write back: the caller's NCHW layout on the last step of a call (128-byte line
        // segments), else cell-major 16-byte quads; fired count
        if (tp.out_nchw) {
            float *xo = a.x_out + row * C * (int64_t)HWn;
            if (lj < tw) {
                const int nl = C * th;
                int c = 0, i = lg;
                while (i >= th) {
                    i -= th;
                    ++c;
                }
                for (int L = lg; L < nl; L += 8) {
                    xo[(int64_t)c * HWn + (i0 + i) * W + j0 + lj] = M[(i * tw + lj) * T::MP + c];
                    i += 8;
                    while (i >= th) {
                        i -= th;
                        ++c;
                    }
                }
            }
        } else {
            float *xc = a.x_out + row * (int64_t)HWn * C;
            const int ipr = tw * Q, nitems = th * ipr;
            int i = 0, rem = tid;
            while (rem >= ipr) {
                rem -= ipr;
                ++i;
            }
            for (int e = tid; e < nitems; e += 256) {
                const int j = rem >> QLOG, q = rem & (Q - 1);
                *reinterpret_cast<float4 *>(xc + ((int64_t)(i0 + i) * W + j0 + j) * C + 4 * q) =
                    *reinterpret_cast<const float4 *>(M + (i * tw + j) * T::MP + 4 * q);
                rem += 256;
                while (rem >= ipr) {
                    rem -= ipr;
                    ++i;
                }
            }
        }
        if (tid == 0 && a.fired_out && *firedL) atomicAdd(a.fired_out + row, *firedL);
        __syncthreads();  // LDS is reused by the next window
    }
}

}  // namespace nca
