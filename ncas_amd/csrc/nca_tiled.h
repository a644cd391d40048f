// The halo-tiled per-step kernel (gfx950): one NCA step over grids of any size.
//
// Used where a row's state does not fit one workgroup's LDS for a whole rollout (201x201
// mazes with C=16; 30x30 boards with C=32 x many rows), and for single steps on such grids.
// One launch advances every row one step, reading the state from x_in and writing x_out
// (fp32 NCHW, the reference layout); a rollout ping-pongs two state buffers across launches.
//
// Each workgroup (4 waves) is persistent over windows: a window is a TH x TW block of cells of
// one row. For each window it
//   1. loads the window plus a 1-cell halo from x_in into the perception buffer P (bf16 for bf16
//      cells, fp32 otherwise): halo cells inside the grid come from the neighbouring windows'
//      cells, halo cells outside it follow the padding rule (wall: pad_vec, zero: 0, wrap:
//      the wrapped cell) - reference src/nca/model.py:140-152;
//      the interior also goes to the fp32 state M;
//   2. draws the fire mask of its cells (Philox keyed on (seed; row, step, cell quad), the same
//      counters as the resident kernels; adaptive firing reads the pre-step confidence from M),
//      or reads the injected mask;
//   3. on the first step of a call, sets the input slice of given cells to the clamp values
//      (model.py:430-438) in M; perception still reads the unclamped state in P;
//   4. runs the 16-cell tile pipeline - stencil of tile t+1, fc1 of tile t, fc2 + residual
//      update of tile t-1 in one barrier interval - with W1/W2 fragments resident in registers;
//      the update writes M only, so P stays the step's input for every later stencil;
//   5. writes M to x_out.
// Since every window reads only x_in and writes only x_out, windows need no synchronisation
// with each other; the launch boundary is the step boundary.
#pragma once

#include "nca_rollout.h"

namespace nca {

struct TiledParams {
    RolloutParams a;   // x_in -> x_out of this step (n_steps, rows_per_wg unused)
    int step;          // step index within the call: Philox counter step0 + step, mask slice
    int first;         // first step of the call: apply the clamp
    int TH, TW;        // window interior (cells)
    int tiles_y, tiles_x;
    int64_t n_windows;  // rows * tiles_y * tiles_x
    unsigned l_P, l_M, l_Z, l_H, l_given, l_fire, l_cinfo, l_head, l_fired;
};

struct TiledPlan {
    unsigned P, M, Z, H, given, fire, cinfo, head, fired, total;
};

template <int C, int HD, bool BF16>
inline TiledPlan tiled_plan(int TH, int TW, int c_out, int n_out) {
    using S = Shape<C, HD, BF16>;
    auto al = [](unsigned v) { return (v + 15u) & ~15u; };
    const unsigned cells = (unsigned)TH * TW, pcells = (unsigned)(TH + 2) * (TW + 2);
    TiledPlan p;
    unsigned o = 0;
    p.P = o;
    o = al(o + pcells * S::CP * S::ES);
    p.M = o;
    o = al(o + cells * S::MP * 4u);
    p.Z = o;
    o = al(o + 2u * S::ZBUF * S::ES);
    p.H = o;
    o = al(o + 2u * S::HBUF * S::ES);
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
    using S = Shape<C, HD, BF16>;
    using FR = Frag<BF16>;
    using fr_t = typename FR::type;
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    const RolloutParams &a = tp.a;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, l16 = lane & 15;
    const int H = a.H, W = a.W, HWn = H * W;
    const int TH = tp.TH, TW = tp.TW, PW = TW + 2;
    const int c_in = a.c_in, in_off = a.in_off;

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
    for (int t = 0; t < 9; ++t) toff[t] = ((t / 3 - 1) * PW + (t % 3 - 1)) * S::CP;

    // ---- MLP fragments and biases in registers: wave w owns hidden units [w HD/4, (w+1) HD/4)
    // for fc1 and fc2 m-tiles w, w + 4, ...
    const float *b1 = reinterpret_cast<const float *>(a.packed + a.off_b1);
    const float *b2 = reinterpret_cast<const float *>(a.packed + a.off_b2);
    fr_t w1f[S::MT1][S::KT1];
    f32x4 b1v[S::MT1];
#pragma unroll
    for (int mt = 0; mt < S::MT1; ++mt) {
#pragma unroll
        for (int kt = 0; kt < S::KT1; ++kt) {
            const size_t idx = ((size_t)(wave * S::MT1 + mt) * S::KT1 + kt) * 64 + lane;
            w1f[mt][kt] = reinterpret_cast<const fr_t *>(a.packed + a.off_w1)[idx];
        }
#pragma unroll
        for (int v = 0; v < 4; ++v) b1v[mt][v] = b1[wave * S::HPW + 16 * mt + 4 * g + v];
    }
    fr_t w2f[S::MT2W][S::KT2];
    f32x4 b2v[S::MT2W];
    bool inslice[S::MT2W][4];
#pragma unroll
    for (int j = 0; j < S::MT2W; ++j) {
        const int mt2 = wave + S::NW * j;
#pragma unroll
        for (int kt = 0; kt < S::KT2; ++kt) {
            const size_t idx = ((size_t)(mt2 < S::MT2 ? mt2 : 0) * S::KT2 + kt) * 64 + lane;
            w2f[j][kt] = reinterpret_cast<const fr_t *>(a.packed + a.off_w2)[idx];
        }
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int c = 16 * mt2 + 4 * g + v;
            b2v[j][v] = mt2 < S::MT2 ? b2[c] : 0.0f;
            inslice[j][v] = c >= in_off && c < in_off + c_in;
        }
    }
    {
        const float *hw = reinterpret_cast<const float *>(a.packed + a.off_headw);
        const float *hb = reinterpret_cast<const float *>(a.packed + a.off_headb);
        const int nw = a.n_out * a.c_out;
        for (int e = tid; e < nw + a.n_out; e += S::NT) headL[e] = e < nw ? hw[e] : hb[e - nw];
    }
    const float *padv = reinterpret_cast<const float *>(a.packed + a.off_padv);
    const uint64_t key = a.step_seeds ? a.step_seeds[tp.step] : a.seed;

    // ---- per-window state of the pipeline stages
    int ncell = 0, ntile = 0;
    const int st_n = tid & 15, st_qd = tid >> 4;

    auto stencil_pc = [&](int t) {
        const int gq = t * 16 + st_n;
        return cinfo[gq < ncell ? gq : ncell - 1];
    };
    // stencil of one tile: this lane's cell centre pc, channel quad st_qd -> Z buffer zb
    auto stencil = [&](int pc, int zb) {
        if constexpr (S::NSI < S::NT) {
            if (tid >= S::NSI) return;  // whole waves (NSI is a multiple of 64)
        }
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
                    float s = 0.0f;
#pragma unroll
                    for (int p2 = 0; p2 < 5; ++p2)
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
        for (int k = 0; k < 4; ++k) lds_store4<BF16>(Zb, zb * S::ZBUF + st_n * S::ZS + k * C + 4 * st_qd, acc[k]);
    };
    // fc1 of the tile in Z buffer zb -> H buffer hb (bias, ReLU; bf16-rounded for bf16 cells)
    auto fc1 = [&](int zb, int hb) {
        fr_t zf[S::KT1];
#pragma unroll
        for (int kt = 0; kt < S::KT1; ++kt)
            zf[kt] = FR::load_lds(Zb, zb * S::ZBUF + l16 * S::ZS + kt * S::KT + (BF16 ? 8 * g : g));
        f32x4 acc[S::MT1];
#pragma unroll
        for (int mt = 0; mt < S::MT1; ++mt) acc[mt] = b1v[mt];
#pragma unroll
        for (int kt = 0; kt < S::KT1; ++kt)
#pragma unroll
            for (int mt = 0; mt < S::MT1; ++mt) acc[mt] = FR::mfma(w1f[mt][kt], zf[kt], acc[mt]);
#pragma unroll
        for (int mt = 0; mt < S::MT1; ++mt) {
            float h[4];
#pragma unroll
            for (int v = 0; v < 4; ++v) h[v] = acc[mt][v] > 0.0f ? acc[mt][v] : 0.0f;
            lds_store4<BF16>(Hb, hb * S::HBUF + l16 * S::HS + wave * S::HPW + 16 * mt + 4 * g, h);
        }
    };
    // fc2 + residual update of tile t (H buffer hb) into M. Input-slice channels of given cells
    // keep their value in M (the clamp values after the first step's clamp pass).
    auto fc2_update = [&](int t, int hb, int64_t row, int i0, int j0, int tw) {
        const int gq = t * 16 + l16;
        const int gc = gq < ncell ? gq : ncell - 1;
        const float f = fireL[gc];
        const bool gv = givenL[gc] != 0;
#pragma unroll
        for (int jj = 0; jj < S::MT2W; ++jj) {
            const int mt2 = wave + S::NW * jj;
            if (S::MT2 % S::NW != 0 && mt2 >= S::MT2) continue;  // uniform per wave
            const int c0 = 16 * mt2 + 4 * g;
            const float4 m4 = *reinterpret_cast<const float4 *>(M + gc * S::MP + c0);
            const float xo[4] = {m4.x, m4.y, m4.z, m4.w};
            fr_t hf[S::KT2];
#pragma unroll
            for (int kt = 0; kt < S::KT2; ++kt)
                hf[kt] = FR::load_lds(Hb, hb * S::HBUF + l16 * S::HS + kt * S::KT + (BF16 ? 8 * g : g));
            f32x4 acc2 = b2v[jj];
#pragma unroll
            for (int kt = 0; kt < S::KT2; ++kt) acc2 = FR::mfma(w2f[jj][kt], hf[kt], acc2);
            float u[4];
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const float dxv = BF16 ? round_bf16(acc2[v]) : acc2[v];
                float uv = __fadd_rn(xo[v], __fmul_rn(f, dxv));
                if constexpr (NOISE) {
                    const int i = gc / tw, j = gc - i * tw;
                    uv = __fadd_rn(uv, a.noise[((row * C + c0 + v) * H + i0 + i) * (int64_t)W + j0 + j]);
                }
                u[v] = (gv && inslice[jj][v]) ? xo[v] : uv;
            }
            if (gq < ncell) *reinterpret_cast<float4 *>(M + gc * S::MP + c0) = make_float4(u[0], u[1], u[2], u[3]);
        }
    };

    const int64_t per_row = (int64_t)tp.tiles_y * tp.tiles_x;
    for (int64_t win = blockIdx.x; win < tp.n_windows; win += gridDim.x) {
        const int64_t row = win / per_row;
        const int wr = (int)(win - row * per_row), ty = wr / tp.tiles_x, tx = wr - ty * tp.tiles_x;
        const int i0 = ty * TH, j0 = tx * TW;
        const int th = H - i0 < TH ? H - i0 : TH, tw = W - j0 < TW ? W - j0 : TW;
        ncell = th * tw;
        ntile = (ncell + 15) >> 4;

        // 1. window + halo -> P (and the interior -> M)
        const int pw = tw + 2, npc = (th + 2) * pw;
        const float *xr = a.x_in + row * C * (int64_t)HWn;
        for (int e = tid; e < C * npc; e += S::NT) {
            const int c = e / npc, r2 = e - c * npc, ii = r2 / pw, jj = r2 - ii * pw;
            int gi = i0 + ii - 1, gj = j0 + jj - 1;
            const bool inside = gi >= 0 && gi < H && gj >= 0 && gj < W;
            float v;
            if (inside || a.padding == 2) {
                if (!inside) {
                    gi = (gi + H) % H;
                    gj = (gj + W) % W;
                }
                v = xr[(int64_t)c * HWn + gi * W + gj];
            } else {
                v = a.padding == 1 ? padv[c] : 0.0f;
            }
            const int pe = (ii * PW + jj) * S::CP + c;
            if constexpr (BF16)
                reinterpret_cast<__bf16 *>(Pb)[pe] = (__bf16)v;
            else
                reinterpret_cast<float *>(Pb)[pe] = v;
            if (ii >= 1 && ii <= th && jj >= 1 && jj <= tw) M[((ii - 1) * tw + jj - 1) * S::MP + c] = v;
        }
        for (int k = tid; k < ncell; k += S::NT) {
            const int i = k / tw, j = k - i * tw;
            givenL[k] = a.given[row * HWn + (i0 + i) * W + j0 + j];
            cinfo[k] = ((i + 1) * PW + j + 1) * S::CP;
        }
        if (tid == 0) *firedL = 0;
        __syncthreads();

        // 2. fire mask of the window's cells (pre-step state, before the clamp)
        for (int k = tid; k < ncell; k += S::NT) {
            const int i = k / tw, j = k - i * tw, q = (i0 + i) * W + j0 + j;
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
                    const float cf = cell_readout(M + k * S::MP + a.out_off, 1, a.c_out, a.n_out, a.head_kind, headL,
                                                  headL + a.n_out * a.c_out, &am);
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
            for (int e = tid; e < ncell * c_in; e += S::NT) {
                const int ci = e / ncell, k = e - ci * ncell;
                if (!givenL[k]) continue;
                const int i = k / tw, j = k - i * tw;
                M[k * S::MP + in_off + ci] = a.clamp[((row * c_in + ci) * H + i0 + i) * (int64_t)W + j0 + j];
            }
            __syncthreads();
        }

        // 4. tile pipeline
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

        // 5. write back; fired count
        float *xo = a.x_out + row * C * (int64_t)HWn;
        for (int e = tid; e < C * ncell; e += S::NT) {
            const int c = e / ncell, k = e - c * ncell, i = k / tw, j = k - i * tw;
            xo[(int64_t)c * HWn + (i0 + i) * W + j0 + j] = M[k * S::MP + c];
        }
        if (tid == 0 && a.fired_out && *firedL) atomicAdd(a.fired_out + row, *firedL);
        __syncthreads();  // LDS is reused by the next window
    }
}

}  // namespace nca
