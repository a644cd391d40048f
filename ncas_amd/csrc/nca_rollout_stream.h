// Streamed LDS-resident rollout kernel for bf16 cells (gfx950): the fast path of the bf16
// rollout on grids up to 15 cells wide.
//
// One workgroup of 4 waves (one per SIMD, up to 512 registers per lane) owns 2*rg rows for the
// whole call, split into two row groups. The tiles of group 0 step p, group 1 step p, group 0
// step p+1, ... form one continuous stream. Interval i of the stream (one workgroup barrier)
// holds three stages of three different tiles, all issued by every wave:
//
//   stencil  tile i:    the 3x3 perception as v_mfma_f32_4x4x4_16b_bf16: each block of 4 lanes
//                       multiplies 4 cells' tap vectors (bf16 pairs from v_perm) by the 4 kernels'
//                       taps, giving z of 4 heads for 4 cells per instruction; 12 instructions per
//                       lane cover its cell x 4 channels x 9 taps. z (bf16) -> Z[i&1] (LDS).
//   MLP      tile i-1:  fc1 on v_mfma_f32_16x16x32_bf16 with W1 resident in registers (wave w owns
//                       hidden units [w*HD/4, (w+1)*HD/4)), B operand from Z; bias + ReLU + bf16
//                       in registers; fc2 over the wave's own hidden units with the fc1
//                       accumulators as B operand directly (W2 fragments packed in that k order);
//                       the 4 per-wave partial sums of dx go to D[(i-1)&1] (LDS, fp32).
//   update   tile i-2:  dx = bf16(b2 + sum of the 4 partials); x += fire * dx into the fp32 state
//                       M and the bf16 perception buffer P; clamped channels of given cells frozen.
//
// While one group's tiles run, the other group's end-of-step work - the first step's clamp, the
// wrap halo refresh, the next step's fire mask - takes the intervals 1-3 after its last update, so
// the pipeline never drains between steps.
//
// P is single-buffered: the update of tile i-2 runs with the stencil of tile i, whose 3x3
// neighbourhoods reach W+1 <= 16 cells back, i.e. never into tile i-2; wrap halos are refreshed
// only after the group's step.
#pragma once

#include <type_traits>

#include "nca_rollout.h"

namespace nca {

typedef short s16x4 __attribute__((ext_vector_type(4)));

template <int C, int HD>
struct StShape {
    static constexpr int F = 4 * C;
    static constexpr int HPW = HD / 4;        // hidden units per wave
    static constexpr int MT1 = HPW / 16;      // fc1 m-tiles per wave
    static constexpr int KT1 = F / 32;        // fc1 k-tiles
    static constexpr int MT2 = C / 16;        // fc2 m-tiles (all channels)
    static constexpr int KT2 = MT1 / 2;       // fc2 k-tiles over the wave's own hidden units
    static constexpr int CP = C + 4;          // P channel stride (bf16 elements)
    static constexpr int MP = C + 4;          // M channel stride (floats)
    static constexpr int ZS = F + 8;          // Z row stride (bf16 elements)
    static constexpr int DS = C + 4;          // partial row stride (floats)
    static constexpr int ZBUF = 16 * ZS;      // bf16 elements per Z buffer
    static constexpr int DBUF = 4 * 16 * DS;  // floats per partial buffer (4 waves)
    static constexpr int NQ = C / 4;          // channel quads
    static constexpr int QW = NQ / 4;         // waves with stencil / update items (C/16)
    static_assert(MT1 % 2 == 0, "fc2 k-tiles need an even number of fc1 m-tiles");
    static_assert(NQ % 4 == 0, "channels must be a multiple of 16");
};

struct StPlan {
    unsigned P, M, Z, D, given, fire, fired, head, cinfo, conf, trash, total;
};

template <int C, int HD>
inline StPlan st_plan(int rg, int H, int W, int c_out, int n_out) {
    using S = StShape<C, HD>;
    const unsigned R = 2u * rg, hw = (unsigned)H * W, hwp = (unsigned)(H + 2) * (W + 2);
    auto al = [](unsigned v) { return (v + 15u) & ~15u; };
    StPlan p;
    unsigned o = 0;
    p.P = o;
    o = al(o + R * hwp * S::CP * 2u);
    p.M = o;
    o = al(o + R * hw * S::MP * 4u);
    p.Z = o;
    o = al(o + 2u * S::ZBUF * 2u);
    p.D = o;
    o = al(o + 2u * S::DBUF * 4u);
    p.given = o;
    o = al(o + R * hw);
    p.fire = o;
    o = al(o + R * hw * 4u);
    p.fired = o;
    o = al(o + R * 4u);
    p.head = o;
    o = al(o + (unsigned)(n_out * c_out + n_out) * 4u);
    p.cinfo = o;
    o = al(o + R * hw * 4u);
    p.conf = o;
    o = al(o + R * hw * 4u);
    p.trash = o;  // stores of padding lanes in the branch-free interval: 16 cells of M and of P
    o = al(o + 16u * S::MP * 4u + 16u * S::CP * 2u);
    p.total = o;
    return p;
}

struct StParams {
    RolloutParams a;
    int rg;  // rows per group
    unsigned l_P, l_M, l_Z, l_D, l_given, l_fire, l_fired, l_head, l_cinfo, l_conf, l_trash;
    unsigned off_w2k;
};

template <int C, int HD>
__global__ void __launch_bounds__(256, 1) rollout_stream(StParams sp) {
    using S = StShape<C, HD>;
    const RolloutParams &a = sp.a;
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, l16 = lane & 15;
    const int H = a.H, W = a.W, HWn = H * W, Wp = W + 2, HWp = (H + 2) * Wp;
    const int rg = sp.rg;
    const int64_t rbase = (int64_t)blockIdx.x * 2 * rg;
    const int Rw = (int)((a.rows - rbase) < 2 * rg ? (a.rows - rbase) : 2 * rg);
    const int rows0 = Rw < rg ? Rw : rg, rows1 = Rw - rows0;
    const int ncg0 = rows0 * HWn, ncg1 = rows1 * HWn;
    // stream tiles per group: at least 4 (room for the other group's end-of-step work)
    const int tgr0 = (ncg0 + 15) >> 4, tgr1 = (ncg1 + 15) >> 4;
    const int tg0 = tgr0 > 4 ? tgr0 : 4, tg1 = tgr1 > 4 ? tgr1 : 4;
    const int cb1 = rg * HWn;
    auto ncg = [&](int grp) { return grp ? ncg1 : ncg0; };
    auto tg = [&](int grp) { return grp ? tg1 : tg0; };
    auto cbase = [&](int grp) { return grp ? cb1 : 0; };

    __bf16 *P = reinterpret_cast<__bf16 *>(smem + sp.l_P);
    unsigned char *Pb = smem + sp.l_P;
    float *M = reinterpret_cast<float *>(smem + sp.l_M);
    unsigned char *Zb = smem + sp.l_Z;
    float *Dp = reinterpret_cast<float *>(smem + sp.l_D);
    uint8_t *givenL = smem + sp.l_given;
    float *fireL = reinterpret_cast<float *>(smem + sp.l_fire);
    int *firedL = reinterpret_cast<int *>(smem + sp.l_fired);
    float *headL = reinterpret_cast<float *>(smem + sp.l_head);
    int *cinfo = reinterpret_cast<int *>(smem + sp.l_cinfo);
    float *confL = reinterpret_cast<float *>(smem + sp.l_conf);
    const int c_in = a.c_in, in_off = a.in_off;

    // ---- registers: MLP fragments and biases
    bf16x8 w1f[S::MT1][S::KT1];
    bf16x8 w2f[S::MT2][S::KT2];
    f32x4 b1v[S::MT1];
    {
        const bf16x8 *w1 = reinterpret_cast<const bf16x8 *>(a.packed + a.off_w1);
        const bf16x8 *w2 = reinterpret_cast<const bf16x8 *>(a.packed + sp.off_w2k);
        const float *b1 = reinterpret_cast<const float *>(a.packed + a.off_b1);
#pragma unroll
        for (int mt = 0; mt < S::MT1; ++mt) {
#pragma unroll
            for (int kt = 0; kt < S::KT1; ++kt) w1f[mt][kt] = w1[((size_t)(wave * S::MT1 + mt) * S::KT1 + kt) * 64 + lane];
#pragma unroll
            for (int v = 0; v < 4; ++v) b1v[mt][v] = b1[wave * S::HPW + 16 * mt + 4 * g + v];
        }
#pragma unroll
        for (int m2 = 0; m2 < S::MT2; ++m2)
#pragma unroll
            for (int kt = 0; kt < S::KT2; ++kt) w2f[m2][kt] = w2[((size_t)(wave * S::MT2 + m2) * S::KT2 + kt) * 64 + lane];
        // keep the MFMA weight fragments in AGPRs: the MFMAs read their A operand from there, so
        // the VGPRs stay free for the per-tile working set
#pragma unroll
        for (int mt = 0; mt < S::MT1; ++mt)
#pragma unroll
            for (int kt = 0; kt < S::KT1; ++kt) asm volatile("" : "+a"(w1f[mt][kt]));
#pragma unroll
        for (int m2 = 0; m2 < S::MT2; ++m2)
#pragma unroll
            for (int kt = 0; kt < S::KT2; ++kt) asm volatile("" : "+a"(w2f[m2][kt]));
    }
    // stencil / update items: lane -> (cell l16 of the tile, channel quad wave*4 + g)
    const bool item = wave < S::QW;
    const int iq = wave * 4 + g;                 // channel quad of the lane's items
    // 4x4x4 MFMA B operand: lane's column j = lane % 4 is kernel j; taps 0-3, 4-7, 8
    s16x4 kb[3];
    float b2q[4];
    bool insl[4];
    int toff[9];
    {
        const float *kern = reinterpret_cast<const float *>(a.packed + a.off_kern);
        const float *b2 = reinterpret_cast<const float *>(a.packed + a.off_b2);
        const int j = lane & 3;
#pragma unroll
        for (int grp3 = 0; grp3 < 3; ++grp3)
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int t = 4 * grp3 + k;
                kb[grp3][k] = __builtin_bit_cast(short, (__bf16)(t < 9 ? kern[j * 9 + t] : 0.0f));
            }
        const int qq = item ? iq : 0;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int c = 4 * qq + v;
            b2q[v] = b2[c];
            insl[v] = c >= in_off && c < in_off + c_in;
        }
#pragma unroll
        for (int t = 0; t < 9; ++t) toff[t] = ((t / 3 - 1) * Wp + (t % 3 - 1)) * S::CP;
    }

    // ---- load rows
    auto pcen = [&](int r, int q) {
        const int i = q / W, j = q - i * W;
        return (r * HWp + (i + 1) * Wp + (j + 1)) * S::CP;
    };
    for (int e = tid; e < Rw * C * HWn; e += 256) {
        const int r = e / (C * HWn), rem = e - r * C * HWn, c = rem / HWn, q = rem - c * HWn;
        const float v = a.x_in[rbase * C * HWn + e];
        M[(r * HWn + q) * S::MP + c] = v;
        P[pcen(r, q) + c] = (__bf16)v;
    }
    for (int e = tid; e < Rw * HWn; e += 256) {
        givenL[e] = a.given[rbase * HWn + e];
        const int r = e / HWn;
        cinfo[e] = pcen(r, e - r * HWn);
    }
    for (int e = tid; e < 2 * rg; e += 256) firedL[e] = 0;
    {
        const float *hw = reinterpret_cast<const float *>(a.packed + a.off_headw);
        const float *hb = reinterpret_cast<const float *>(a.packed + a.off_headb);
        const int nw = a.n_out * a.c_out;
        for (int e = tid; e < nw + a.n_out; e += 256) headL[e] = e < nw ? hw[e] : hb[e - nw];
    }
    const int nhalo = 2 * Wp + 2 * H;
    auto halo_cell = [&](int h, int &ip, int &jp) __attribute__((always_inline)) {
        if (h < Wp) {
            ip = 0;
            jp = h;
        } else if (h < 2 * Wp) {
            ip = H + 1;
            jp = h - Wp;
        } else if (h < 2 * Wp + H) {
            ip = h - 2 * Wp + 1;
            jp = 0;
        } else {
            ip = h - 2 * Wp - H + 1;
            jp = W + 1;
        }
    };
    if (a.padding != 2) {
        const float *padv = reinterpret_cast<const float *>(a.packed + a.off_padv);
        for (int e = tid; e < Rw * nhalo * C; e += 256) {
            const int c = e % C, rest = e / C, h = rest % nhalo, r = rest / nhalo;
            int ip, jp;
            halo_cell(h, ip, jp);
            P[(r * HWp + ip * Wp + jp) * S::CP + c] = (__bf16)(a.padding == 1 ? padv[c] : 0.0f);
        }
    }
    auto wrap_halo = [&](int grp) __attribute__((always_inline)) {
        const int r0 = grp * rg, nr = grp ? rows1 : rows0;
        for (int e = tid; e < nr * nhalo * S::NQ; e += 256) {
            const int qd = e % S::NQ, rest = e / S::NQ, h = rest % nhalo, r = r0 + rest / nhalo;
            int ip, jp;
            halo_cell(h, ip, jp);
            const int si = (ip - 1 + H) % H, sj = (jp - 1 + W) % W;
            *reinterpret_cast<uint2 *>(Pb + 2 * ((r * HWp + ip * Wp + jp) * S::CP + 4 * qd)) =
                *reinterpret_cast<const uint2 *>(Pb + 2 * ((r * HWp + (si + 1) * Wp + sj + 1) * S::CP + 4 * qd));
        }
    };
    auto clamp_pass = [&](int grp) __attribute__((always_inline)) {
        const int c0 = cbase(grp), n = ncg(grp);
        for (int e = tid; e < n * c_in; e += 256) {
            const int cell = c0 + e / c_in, ci = e % c_in;
            if (!givenL[cell]) continue;
            const int r = cell / HWn, q = cell - r * HWn;
            const float v = a.clamp[((rbase + r) * c_in + ci) * HWn + q];
            M[cell * S::MP + in_off + ci] = v;
            P[cinfo[cell] + in_off + ci] = (__bf16)v;
        }
    };
    const int nq4 = (HWn + 3) >> 2;
    auto draw_fire = [&](int grp, int s) __attribute__((always_inline)) {
        const int r0 = grp * rg, nr = grp ? rows1 : rows0;
        for (int it = tid; it < nr * nq4; it += 256) {
            const int r = r0 + it / nq4, qq = it % nq4;
            float u[4] = {0.f, 0.f, 0.f, 0.f};
            if (!a.fire_u8) {
                const uint64_t key = a.step_seeds ? a.step_seeds[s] : a.seed;
                cell_uniforms4(key, (uint32_t)(a.row0 + rbase + r), (uint32_t)(a.step0 + s), (uint32_t)qq, u);
            }
            int cnt = 0;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int q = 4 * qq + e;
                if (q >= HWn) break;
                const int cell = r * HWn + q;
                float f;
                if (a.fire_u8) {
                    f = a.fire_u8[((int64_t)s * a.rows + rbase + r) * HWn + q] ? 1.0f : 0.0f;
                } else {
                    float pc = a.p;
                    if (a.adaptive) {
                        int am;
                        const float cf = cell_readout(M + cell * S::MP + a.out_off, 1, a.c_out, a.n_out, a.head_kind,
                                                      headL, headL + a.n_out * a.c_out, &am);
                        if (cf > a.tau || (a.given_confident && givenL[cell])) pc = a.p_low;
                    }
                    f = u[e] < pc ? 1.0f : 0.0f;
                }
                fireL[cell] = f;
                cnt += f != 0.0f;
            }
            if (cnt) atomicAdd(&firedL[r], cnt);
        }
    };
    __syncthreads();
    if (a.padding == 2) {
        wrap_halo(0);
        wrap_halo(1);
    }
    if (a.n_steps > 0) {
        draw_fire(0, 0);
        draw_fire(1, 0);
    }
    __syncthreads();

    // ---- the tile stream
    const int T = a.n_steps * (tg0 + tg1);
    struct Pos {
        int grp, j, s;
    };
    auto advance = [&](Pos &p) __attribute__((always_inline)) {
        if (++p.j == tg(p.grp)) {
            p.j = 0;
            p.grp ^= 1;
            if (p.grp == 0) ++p.s;
        }
    };
    Pos ps = {0, 0, 0}, pu = {0, 0, 0};
    int m_grp = 0, m_s = 0, m_phase = 0;

    float *Mtrash = reinterpret_cast<float *>(smem + sp.l_trash);
    const int ptrash = (int)((sp.l_trash + 16u * S::MP * 4u - sp.l_P) / 2u);  // P element offset

    // one interval of the stream. FULL: every stage has a tile (no uniform branches; padding
    // lanes store to the trash rows); PAR: i & 1 when FULL (constant buffer offsets).
    auto interval = [&](int i, auto full_c, auto par_c) __attribute__((always_inline)) {
        constexpr bool FULL = decltype(full_c)::value;
        constexpr int PAR = decltype(par_c)::value;
        const int zs = FULL ? PAR : (i & 1), zf_b = FULL ? 1 - PAR : ((i - 1) & 1);
        const int nv_s = FULL ? min(16, ncg(ps.grp) - 16 * ps.j) : (i < T ? min(16, ncg(ps.grp) - 16 * ps.j) : 0);
        const int nv_u = FULL ? min(16, ncg(pu.grp) - 16 * pu.j) : (i >= 2 ? min(16, ncg(pu.grp) - 16 * pu.j) : 0);
        const bool do_st = FULL || (item && nv_s > 0);
        const bool do_fc = FULL || (i >= 1 && i <= T);
        const bool do_up = FULL || (item && nv_u > 0);

        // ---- LDS loads of the interval
        uint2 nb[9];
        if (do_st) {
            const int cell = cbase(ps.grp) + 16 * ps.j + (l16 < nv_s ? l16 : nv_s - 1);
            const int base = cinfo[cell] + 4 * iq;
#pragma unroll
            for (int t9 = 0; t9 < 9; ++t9) nb[t9] = *reinterpret_cast<const uint2 *>(Pb + 2 * (base + toff[t9]));
        }
        bf16x8 zf[S::KT1];
        if (do_fc) {
#pragma unroll
            for (int kt = 0; kt < S::KT1; ++kt)
                zf[kt] = *reinterpret_cast<const bf16x8 *>(Zb + 2 * (zf_b * S::ZBUF + l16 * S::ZS + kt * 32 + 8 * g));
        }
        float4 pv[4], m4;
        float f = 0.0f;
        bool gv = false;
        int ucell = 0, upc = 0;
        if (do_up) {
            ucell = cbase(pu.grp) + 16 * pu.j + (l16 < nv_u ? l16 : nv_u - 1);
            const float *dp = Dp + (FULL ? PAR : ((i - 2) & 1)) * S::DBUF + l16 * S::DS + 4 * iq;
#pragma unroll
            for (int w4 = 0; w4 < 4; ++w4) pv[w4] = *reinterpret_cast<const float4 *>(dp + w4 * 16 * S::DS);
            m4 = *reinterpret_cast<const float4 *>(M + ucell * S::MP + 4 * iq);
            f = fireL[ucell];
            gv = givenL[ucell] != 0;
            upc = cinfo[ucell];
        }
        // ---- stencil of tile i on the 4x4x4 MFMA
        if (do_st) {
            f32x4 zc[4];
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const int sel = (c & 1) ? 0x07060302 : 0x05040100;
                const uint32_t p01 = __builtin_amdgcn_perm(c < 2 ? nb[1].x : nb[1].y, c < 2 ? nb[0].x : nb[0].y, sel);
                const uint32_t p23 = __builtin_amdgcn_perm(c < 2 ? nb[3].x : nb[3].y, c < 2 ? nb[2].x : nb[2].y, sel);
                const uint32_t p45 = __builtin_amdgcn_perm(c < 2 ? nb[5].x : nb[5].y, c < 2 ? nb[4].x : nb[4].y, sel);
                const uint32_t p67 = __builtin_amdgcn_perm(c < 2 ? nb[7].x : nb[7].y, c < 2 ? nb[6].x : nb[6].y, sel);
                const uint32_t w8 = c < 2 ? nb[8].x : nb[8].y;
                const uint32_t p8 = (c & 1) ? (w8 >> 16) : (w8 & 0xffffu);
                const s16x4 a0 = __builtin_bit_cast(s16x4, make_uint2(p01, p23));
                const s16x4 a1 = __builtin_bit_cast(s16x4, make_uint2(p45, p67));
                const s16x4 a2 = __builtin_bit_cast(s16x4, make_uint2(p8, 0u));
                f32x4 d = {0.f, 0.f, 0.f, 0.f};
                d = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(a0, kb[0], d, 0, 0, 0);
                d = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(a1, kb[1], d, 0, 0, 0);
                d = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(a2, kb[2], d, 0, 0, 0);
                zc[c] = d;
            }
            const int j = lane & 3, cb = 4 * ((lane >> 2) & 3);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                uint2 o;
                o.x = pack_bf16x2(zc[0][r], zc[1][r]);
                o.y = pack_bf16x2(zc[2][r], zc[3][r]);
                *reinterpret_cast<uint2 *>(Zb + 2 * (zs * S::ZBUF + (cb + r) * S::ZS + j * C + 4 * iq)) = o;
            }
        }
        // ---- MLP of tile i-1
        if (do_fc) {
            f32x4 acc[S::MT1];
#pragma unroll
            for (int mt = 0; mt < S::MT1; ++mt) acc[mt] = b1v[mt];
#pragma unroll
            for (int kt = 0; kt < S::KT1; ++kt)
#pragma unroll
                for (int mt = 0; mt < S::MT1; ++mt)
                    acc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(w1f[mt][kt], zf[kt], acc[mt], 0, 0, 0);
            bf16x8 hf[S::KT2];
#pragma unroll
            for (int kt = 0; kt < S::KT2; ++kt)
#pragma unroll
                for (int s2 = 0; s2 < 8; ++s2) {
                    const float hv = acc[2 * kt + s2 / 4][s2 % 4];
                    hf[kt][s2] = (__bf16)(hv > 0.0f ? hv : 0.0f);
                }
            float *dpw = Dp + (FULL ? 1 - PAR : ((i - 1) & 1)) * S::DBUF + (wave * 16 + l16) * S::DS;
#pragma unroll
            for (int m2 = 0; m2 < S::MT2; ++m2) {
                f32x4 acc2 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int kt = 0; kt < S::KT2; ++kt)
                    acc2 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(w2f[m2][kt], hf[kt], acc2, 0, 0, 0);
                *reinterpret_cast<float4 *>(dpw + 16 * m2 + 4 * g) = make_float4(acc2[0], acc2[1], acc2[2], acc2[3]);
            }
        }
        // ---- update of tile i-2
        if (do_up) {
            float dsum[4] = {b2q[0], b2q[1], b2q[2], b2q[3]};
#pragma unroll
            for (int w4 = 0; w4 < 4; ++w4) {
                dsum[0] += pv[w4].x;
                dsum[1] += pv[w4].y;
                dsum[2] += pv[w4].z;
                dsum[3] += pv[w4].w;
            }
            const float xo[4] = {m4.x, m4.y, m4.z, m4.w};
            float u[4];
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const float uv = __fadd_rn(xo[v], __fmul_rn(f, round_bf16(dsum[v])));
                u[v] = (gv && insl[v]) ? xo[v] : uv;
            }
            const bool valid = l16 < nv_u;
            float *mdst = valid ? M + ucell * S::MP + 4 * iq : Mtrash + l16 * S::MP + 4 * iq;
            const int pdst = valid ? upc + 4 * iq : ptrash + l16 * S::CP + 4 * iq;
            *reinterpret_cast<float4 *>(mdst) = make_float4(u[0], u[1], u[2], u[3]);
            lds_store4<true>(Pb, pdst, u);
        }
        // ---- end-of-step work of the group whose last tile was updated 1-3 intervals ago
        if (m_phase == 1 && m_s == 0 && c_in > 0) clamp_pass(m_grp);
        if (m_phase == 2 && a.padding == 2) wrap_halo(m_grp);
        if (m_phase == 3 && m_s + 1 < a.n_steps) draw_fire(m_grp, m_s + 1);
        // bookkeeping (wave-uniform)
        m_phase = m_phase > 0 && m_phase < 3 ? m_phase + 1 : 0;
        if (i >= 2 && i - 2 < T) {
            if (pu.j == tg(pu.grp) - 1) {
                m_grp = pu.grp;
                m_s = pu.s;
                m_phase = 1;
            }
            advance(pu);
        }
        if (i < T) advance(ps);
        __syncthreads();
    };
    using F_ = std::integral_constant<bool, false>;
    using T_ = std::integral_constant<bool, true>;
    using P0 = std::integral_constant<int, 0>;
    using P1 = std::integral_constant<int, 1>;
    // the branch-free body needs every lane to own stencil / update items and real tiles only
    const bool fast = S::QW == 4 && tgr0 >= 4 && tgr1 >= 4;
    int i = 0;
    if (fast) {
        for (; i < 2 && i < T + 2; ++i) interval(i, F_{}, P0{});
        for (; i + 1 < T; i += 2) {
            interval(i, T_{}, P0{});
            interval(i + 1, T_{}, P1{});
        }
    }
    for (; i < T + 2; ++i) interval(i, F_{}, P0{});
    if (m_phase == 1 && m_s == 0 && c_in > 0) clamp_pass(m_grp);
    __syncthreads();

    // ---- write back
    for (int e = tid; e < Rw * C * HWn; e += 256) {
        const int r = e / (C * HWn), rem = e - r * C * HWn, c = rem / HWn, q = rem - c * HWn;
        a.x_out[rbase * C * HWn + e] = M[(r * HWn + q) * S::MP + c];
    }
    if (a.conf_out) {
        for (int cell = tid; cell < Rw * HWn; cell += 256) {
            int am;
            confL[cell] = cell_readout(M + cell * S::MP + a.out_off, 1, a.c_out, a.n_out, a.head_kind, headL,
                                       headL + a.n_out * a.c_out, &am);
        }
        __syncthreads();
        for (int r = tid; r < Rw; r += 256) {
            float sum = 0.0f;
            for (int q = 0; q < HWn; ++q) sum = __fadd_rn(sum, confL[r * HWn + q]);
            a.conf_out[rbase + r] = __fdiv_rn(sum, (float)HWn);
        }
    }
    if (a.fired_out)
        for (int r = tid; r < Rw; r += 256) a.fired_out[rbase + r] = firedL[r];
}

}  // namespace nca
