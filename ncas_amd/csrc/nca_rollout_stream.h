// Streamed LDS-resident rollout kernel for bf16 cells with C = 64 channels and 256 hidden units
// (gfx950): the fast path of the bf16 rollout on grids up to 15 cells wide.
//
// One workgroup of 4 waves (one per SIMD) owns 2*rg rows (rollouts) for the whole call, split
// into two row groups. The 16-cell tiles of group 0 step s, group 1 step s, group 0 step s+1, ...
// form one stream. Interval i of the stream (one workgroup barrier) runs three stages of three
// different tiles, all issued by every wave:
//
//   stencil tile i     the 3x3 perception on v_mfma_f32_4x4x4_16b_bf16. Lane (cell n, channel
//                      quad iq) reads the 9 taps of its 4 channels (bf16) from the perception
//                      buffer P; each 4-lane block multiplies 4 cells' tap vectors by the 4
//                      kernels, giving z of 4 heads for 4 cells per instruction (12 per lane).
//                      z (bf16) -> feature tile Z[i & 1].
//   MLP tile i-1       fc1 on v_mfma_f32_16x16x32_bf16 with W1 resident in AGPRs (wave w owns
//                      hidden units [64w, 64w+64)), B operand read from Z; bias + ReLU + bf16
//                      in registers; fc2 over the wave's own hidden units with the fc1
//                      accumulators as B operand (W2 fragments packed in that k order). The four
//                      waves' partial sums of dx go to D[(i-1) & 1].
//   update tile i-2    dx = bf16(b2 + sum of the 4 partials); x += fire * dx into the fp32 state
//                      M and the bf16 perception buffer P; the clamped input channels of given
//                      cells are frozen.
//
// P is single-buffered: the update of tile i-2 runs in the same interval as the stencil of tile
// i, whose neighbourhoods reach W+1 <= 16 cells back, so never into tile i-2. A group's
// end-of-step work runs in the intervals 2 and 3 of the other group's tiles:
//   * the first step's clamp (phase 1);
//   * the wrap-halo refresh and the fire masks of the next steps (phase 2).
// So the pipeline never drains between steps.
//
// LDS layouts are chosen for gfx950's banks (reads: 64 banks, ds_read_b64 in groups of 32
// lanes, ds_read_b128 in two 8-lane groups; writes: 32 banks, 16 lanes per cycle for b64 and 8
// for b128) so that the hot accesses are conflict-free:
//   * P: cell stride 144 B, padded row pitch RP = 144 (W + 2) + 224, so that the byte address
//     of cell q is 144 q + const mod 256 and a tile's 16 cells x 2 quads hit 32 distinct bank
//     pairs for every tap;
//   * M and D: 288 B per cell row, 16-byte chunk c of cell n stored at chunk c ^ ((n >> 2) & 1);
//   * Z: 576 B per cell row, features in quad-major order (16 iq + 4 head + ch), chunk c of row
//     r stored at chunk c ^ (2 ((r >> 2) & 3)).
// Fire masks of non-adaptive rollouts are drawn for up to 16 steps at a time (one Philox
// evaluation per 4 cells, as in the standalone mask kernel) into a byte ring in LDS.
#pragma once

#include <type_traits>

#include "nca_rollout.h"

namespace nca {

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef short s16x2 __attribute__((ext_vector_type(2)));

struct St64 {
    static constexpr int C = 64, HD = 256, F = 256;
    static constexpr int MT1 = 4, KT1 = 8, MT2 = 4, KT2 = 2;
    static constexpr int CS = 144;   // P bytes per cell (64 bf16 + 8 pad)
    static constexpr int MS = 288;   // M bytes per cell (64 fp32 + 8 pad)
    static constexpr int ZS = 576;   // Z bytes per cell row (256 bf16 + 32 pad)
    static constexpr int DS = 288;   // D bytes per cell row (64 fp32 + 8 pad)
    static constexpr int ZBUF = 16 * ZS;
    static constexpr int DBUF = 64 * DS;
    static constexpr int RPAD = 224;  // (-2 * CS) mod 256
};

struct StPlan {
    unsigned P, Ptrash, M, Z, D, cinfo, fire, fired, head, hcp, total;
    int RP, PB, G, NB;
};

inline unsigned st_al16(unsigned v) { return (v + 15u) & ~15u; }

// rg rows per group, NB fire-mask slots. G (cells per group, a multiple of 32 and >= 64) gives an
// even number (>= 4) of tiles per group step.
inline StPlan st_plan(int rg, int H, int W, int c_out, int n_out, int NB) {
    using S = St64;
    StPlan p;
    const int HWn = H * W;
    p.RP = (W + 2) * S::CS + S::RPAD;
    const int pb0 = (H + 2) * p.RP;
    p.PB = pb0 + (((S::CS * HWn - pb0) % 256) + 256) % 256;
    const int g = (rg * HWn + 31) & ~31;
    p.G = g < 64 ? 64 : g;
    p.NB = NB;
    unsigned o = 0;
    p.P = o;
    o = st_al16(o + 2u * rg * (unsigned)p.PB);
    p.Ptrash = o;
    o = st_al16(o + 16u * S::CS);
    p.M = o;
    o = st_al16(o + 2u * p.G * S::MS);
    p.Z = o;
    o += 2u * S::ZBUF;
    p.D = o;
    o += 2u * S::DBUF;
    p.cinfo = o;
    o = st_al16(o + 2u * p.G * 8u);
    p.fire = o;
    o = st_al16(o + (unsigned)NB * 2u * p.G);
    p.fired = o;
    o = st_al16(o + 2u * rg * 4u);
    p.head = o;
    o = st_al16(o + (unsigned)(n_out * c_out + n_out) * 4u);
    p.hcp = o;
    o = st_al16(o + (unsigned)(2 * (W + 2) + 2 * H) * 4u);
    p.total = o;
    return p;
}

struct StParams {
    RolloutParams a;
    int rg, G, RP, PB, NB;
    unsigned l_P, l_Ptrash, l_M, l_Z, l_D, l_cinfo, l_fire, l_fired, l_head, l_hcp;
    unsigned off_w1q, off_w2k;
};

__device__ __forceinline__ uint2 lds_ld64(const unsigned char *s, unsigned off) {
    return *reinterpret_cast<const uint2 *>(s + off);
}
__device__ __forceinline__ float4 lds_ld128f(const unsigned char *s, unsigned off) {
    return *reinterpret_cast<const float4 *>(s + off);
}
__device__ __forceinline__ void lds_st64(unsigned char *s, unsigned off, uint2 v) {
    *reinterpret_cast<uint2 *>(s + off) = v;
}
__device__ __forceinline__ void lds_st128f(unsigned char *s, unsigned off, float4 v) {
    *reinterpret_cast<float4 *>(s + off) = v;
}
// ReLU of two packed bf16 values: a negative bf16 is a negative int16.
__device__ __forceinline__ uint32_t relu_bf16x2(uint32_t v) {
    const s16x2 x = __builtin_bit_cast(s16x2, v);
    const s16x2 z = {0, 0};
    return __builtin_bit_cast(uint32_t, __builtin_elementwise_max(x, z));
}
__device__ __forceinline__ short bf16_bits(float v) { return __builtin_bit_cast(short, (__bf16)v); }

__global__ void __launch_bounds__(256, 1) rollout_stream64(StParams sp) {
    using S = St64;
    const RolloutParams &a = sp.a;
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, n = lane & 15;  // n: cell of the tile (MFMA column), g: lane group
    const int iq = 4 * wave + g;             // channel quad of the lane's stencil / update items
    const int H = a.H, W = a.W, HWn = H * W;
    const int rg = sp.rg, G = sp.G, RP = sp.RP, PB = sp.PB, NB = sp.NB;
    const int tg = G >> 4;
    const int64_t rbase = (int64_t)blockIdx.x * 2 * rg;
    const int Rw = (int)((a.rows - rbase) < 2 * rg ? (a.rows - rbase) : 2 * rg);
    const int rows0 = Rw < rg ? Rw : rg, rows1 = Rw - rows0;

    int *firedL = reinterpret_cast<int *>(smem + sp.l_fired);
    float *headL = reinterpret_cast<float *>(smem + sp.l_head);
    unsigned *hcp = reinterpret_cast<unsigned *>(smem + sp.l_hcp);
    uint2 *cinfo = reinterpret_cast<uint2 *>(smem + sp.l_cinfo);
    unsigned char *fireB = smem + sp.l_fire;

    // byte offset of (workgroup cell c, channel ch) in M; of the centre of cell q of board rw in P
    auto m_off = [&](int c, int ch) -> unsigned {
        return sp.l_M + (unsigned)c * S::MS + 16u * (unsigned)((ch >> 2) ^ ((c >> 2) & 1)) + 4u * (ch & 3);
    };
    auto p_cell = [&](int rw, int q) -> unsigned {
        const int i = q / W, j = q - i * W;
        return sp.l_P + (unsigned)(rw * PB + (i + 1) * RP + (j + 1) * S::CS);
    };
    auto m_at = [&](int c, int ch) -> float & { return *reinterpret_cast<float *>(smem + m_off(c, ch)); };
    auto wg_cell = [&](int rw, int q) { return (rw >= rg ? G + (rw - rg) * HWn : rw * HWn) + q; };

    // ---- registers: MLP weight fragments (AGPRs) and biases
    bf16x8 w1f[S::MT1][S::KT1];
    bf16x8 w2f[S::MT2][S::KT2];
    f32x4 b1v[S::MT1];
    {
        const bf16x8 *w1 = reinterpret_cast<const bf16x8 *>(a.packed + sp.off_w1q);
        const bf16x8 *w2 = reinterpret_cast<const bf16x8 *>(a.packed + sp.off_w2k);
        const float *b1 = reinterpret_cast<const float *>(a.packed + a.off_b1);
#pragma unroll
        for (int mt = 0; mt < S::MT1; ++mt) {
#pragma unroll
            for (int kt = 0; kt < S::KT1; ++kt) w1f[mt][kt] = w1[((wave * S::MT1 + mt) * S::KT1 + kt) * 64 + lane];
#pragma unroll
            for (int v = 0; v < 4; ++v) b1v[mt][v] = b1[wave * 64 + 16 * mt + 4 * g + v];
        }
#pragma unroll
        for (int m2 = 0; m2 < S::MT2; ++m2)
#pragma unroll
            for (int kt = 0; kt < S::KT2; ++kt) w2f[m2][kt] = w2[((wave * S::MT2 + m2) * S::KT2 + kt) * 64 + lane];
#pragma unroll
        for (int mt = 0; mt < S::MT1; ++mt)
#pragma unroll
            for (int kt = 0; kt < S::KT1; ++kt) asm volatile("" : "+a"(w1f[mt][kt]));
#pragma unroll
        for (int m2 = 0; m2 < S::MT2; ++m2)
#pragma unroll
            for (int kt = 0; kt < S::KT2; ++kt) asm volatile("" : "+a"(w2f[m2][kt]));
    }
    // stencil B operands: column j = lane % 4 is kernel j; taps 0-3, 4-7; tap 8 placed at the
    // k slot of channel c (the A operand of tap 8 is the 4 channels' tap-8 values as loaded)
    s16x4 kb0, kb1, kb2[4];
    {
        const float *kern = reinterpret_cast<const float *>(a.packed + a.off_kern);
        const int j = lane & 3;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            kb0[k] = bf16_bits(kern[j * 9 + k]);
            kb1[k] = bf16_bits(kern[j * 9 + 4 + k]);
        }
        const short k8 = bf16_bits(kern[j * 9 + 8]);
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int k = 0; k < 4; ++k) kb2[c][k] = k == c ? k8 : (short)0;
    }
    float b2q[4];
    bool insl[4];
    {
        const float *b2 = reinterpret_cast<const float *>(a.packed + a.off_b2);
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int c = 4 * iq + v;
            b2q[v] = b2[c];
            insl[v] = c >= a.in_off && c < a.in_off + a.c_in;
        }
    }
    // lane-constant LDS offsets
    const int hsw = (n >> 2) & 1;
    const unsigned kM = (unsigned)n * S::MS + 16u * (unsigned)(iq ^ hsw);                       // + l_M + cb MS
    const unsigned kDr = sp.l_D + (unsigned)n * S::DS + 16u * (unsigned)(iq ^ hsw);              // + w4 16 DS
    const unsigned kDw = sp.l_D + (unsigned)(wave * 16 + n) * S::DS + 16u * (unsigned)(g ^ hsw);  // + 64 m2
    const int sig = 2 * ((n >> 2) & 3);
    const unsigned kZ0 = sp.l_Z + (unsigned)n * S::ZS + 16u * (unsigned)(g ^ (sig & 3));
    const unsigned kZe = kZ0 + 64u * (unsigned)(sig >> 2), kZo = kZ0 - 64u * (unsigned)(sig >> 2);
    unsigned kZw;
    {
        const int j = lane & 3, b = lane >> 2;
        kZw = sp.l_Z + (unsigned)(4 * (b & 3)) * S::ZS + 16u * (unsigned)((2 * iq + (j >> 1)) ^ (2 * (b & 3))) +
              8u * (unsigned)(j & 1);
    }
    const unsigned kPs = 8u * iq - (unsigned)(RP + S::CS);  // + centre: top-left tap
    const unsigned RP2 = 2u * RP;

    // ---- load rows and tables
    for (int e = tid; e < Rw * S::C * HWn; e += 256) {
        const int rw = e / (S::C * HWn), rem = e - rw * S::C * HWn, ch = rem / HWn, q = rem - ch * HWn;
        const float v = a.x_in[rbase * S::C * HWn + e];
        m_at(wg_cell(rw, q), ch) = v;
        *reinterpret_cast<__bf16 *>(smem + p_cell(rw, q) + 2 * ch) = (__bf16)v;
    }
    for (int c = tid; c < 2 * G; c += 256) {
        const int grp = c >= G, qg = c - grp * G, nr = grp ? rows1 : rows0;
        uint2 ci;
        if (qg < nr * HWn) {
            const int r = qg / HWn, q = qg - r * HWn, rw = grp * rg + r;
            ci.x = p_cell(rw, q);
            ci.y = ci.x | (a.given[(rbase + rw) * HWn + q] ? 0x80000000u : 0u);
        } else {
            // padding cell: the stencil reads a real cell, update stores go to the trash cells
            ci.x = nr > 0 ? p_cell(grp * rg + nr - 1, HWn - 1) : p_cell(0, 0);
            ci.y = sp.l_Ptrash + (unsigned)(c & 15) * S::CS;
        }
        cinfo[c] = ci;
    }
    for (int e = tid; e < 2 * rg; e += 256) firedL[e] = 0;
    {
        const float *hw = reinterpret_cast<const float *>(a.packed + a.off_headw);
        const float *hb = reinterpret_cast<const float *>(a.packed + a.off_headb);
        const int nw = a.n_out * a.c_out;
        for (int e = tid; e < nw + a.n_out; e += 256) headL[e] = e < nw ? hw[e] : hb[e - nw];
    }
    const int Wp = W + 2, nhalo = 2 * Wp + 2 * H;
    for (int h = tid; h < nhalo; h += 256) {
        int ip, jp;
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
        const int si = (ip - 1 + H) % H, sj = (jp - 1 + W) % W;
        const unsigned dst = (unsigned)(ip * RP + jp * S::CS), src = (unsigned)((si + 1) * RP + (sj + 1) * S::CS);
        hcp[h] = dst | (src << 16);
    }
    __syncthreads();
    if (a.padding != 2) {
        const float *padv = reinterpret_cast<const float *>(a.packed + a.off_padv);
        for (int r = 0; r < Rw; ++r)
            for (int e = tid; e < nhalo * S::C; e += 256) {
                const int h = e >> 6, ch = e & 63;
                const unsigned dst = hcp[h] & 0xffffu;
                *reinterpret_cast<__bf16 *>(smem + sp.l_P + (unsigned)(r * PB) + dst + 2 * ch) =
                    (__bf16)(a.padding == 1 ? padv[ch] : 0.0f);
            }
    }
    // wrap halo of one group's boards: 16-byte chunks of 8 channels
    auto wrap_halo = [&](int grp) __attribute__((always_inline)) {
        const int nr = grp ? rows1 : rows0;
        for (int r = 0; r < nr; ++r) {
            const unsigned base = sp.l_P + (unsigned)((grp * rg + r) * PB);
            for (int e = tid; e < nhalo * 8; e += 256) {
                const unsigned hc = hcp[e >> 3], o = 16u * (unsigned)(e & 7);
                const float4 v = lds_ld128f(smem, base + (hc >> 16) + o);
                lds_st128f(smem, base + (hc & 0xffffu) + o, v);
            }
        }
    };
    // first step's clamp of the given cells of one group (model.py:430-438)
    auto clamp_pass = [&](int grp) __attribute__((always_inline)) {
        const int nr = grp ? rows1 : rows0, c_in = a.c_in;
        for (int e = tid; e < nr * HWn * c_in; e += 256) {
            const int cell = e / c_in, ci = e - cell * c_in;
            const int r = cell / HWn, q = cell - r * HWn, rw = grp * rg + r;
            if (!a.given[(rbase + rw) * HWn + q]) continue;
            const float v = a.clamp[((rbase + rw) * c_in + ci) * HWn + q];
            m_at(grp * G + cell, a.in_off + ci) = v;
            *reinterpret_cast<__bf16 *>(smem + p_cell(rw, q) + 2 * (a.in_off + ci)) = (__bf16)v;
        }
    };
    // fire masks: batched Philox draws for steps s0 .. s0 + NB - 1 (non-adaptive, no injected
    // masks), or one step (adaptive confidence gating or injected masks)
    const int nq4 = (HWn + 3) >> 2;
    const bool batched = !a.adaptive && !a.fire_u8;
    auto draw_batch = [&](int grp, int s0) __attribute__((always_inline)) {
        const int nr = grp ? rows1 : rows0;
        const int per_row = NB * nq4;
        for (int it = tid; it < nr * per_row; it += 256) {
            const int r = it / per_row, rem = it - r * per_row, sl = rem / nq4, qq = rem - sl * nq4;
            const int s = s0 + sl;
            if (s >= a.n_steps) continue;
            const int rw = grp * rg + r;
            const uint64_t key = a.step_seeds ? a.step_seeds[s] : a.seed;
            float u[4];
            cell_uniforms4(key, (uint32_t)(a.row0 + rbase + rw), (uint32_t)(a.step0 + s), (uint32_t)qq, u);
            unsigned char *fb = fireB + (unsigned)(sl * 2 * G + grp * G + r * HWn);
            int cnt = 0;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int q = 4 * qq + e;
                if (q < HWn) {
                    const int f = u[e] < a.p;
                    fb[q] = (unsigned char)f;
                    cnt += f;
                }
            }
            if (cnt) atomicAdd(&firedL[rw], cnt);
        }
    };
    auto draw_step = [&](int grp, int s) __attribute__((always_inline)) {
        const int nr = grp ? rows1 : rows0;
        for (int it = tid; it < nr * nq4; it += 256) {
            const int r = it / nq4, qq = it - r * nq4, rw = grp * rg + r;
            float u[4] = {0.f, 0.f, 0.f, 0.f};
            if (!a.fire_u8) {
                const uint64_t key = a.step_seeds ? a.step_seeds[s] : a.seed;
                cell_uniforms4(key, (uint32_t)(a.row0 + rbase + rw), (uint32_t)(a.step0 + s), (uint32_t)qq, u);
            }
            int cnt = 0;
            for (int e = 0; e < 4; ++e) {
                const int q = 4 * qq + e;
                if (q >= HWn) break;
                const int c = grp * G + r * HWn + q;
                int f;
                if (a.fire_u8) {
                    f = a.fire_u8[((int64_t)s * a.rows + rbase + rw) * HWn + q] != 0;
                } else {
                    float pc = a.p;
                    if (a.adaptive) {
                        int am;
                        const float cf = cell_readout_fn([&](int v) { return m_at(c, a.out_off + v); }, a.c_out,
                                                         a.n_out, a.head_kind, headL, headL + a.n_out * a.c_out, &am);
                        if (cf > a.tau || (a.given_confident && a.given[(rbase + rw) * HWn + q])) pc = a.p_low;
                    }
                    f = u[e] < pc;
                }
                fireB[c] = (unsigned char)f;
                cnt += f;
            }
            if (cnt) atomicAdd(&firedL[rw], cnt);
        }
    };
    __syncthreads();
    if (a.padding == 2) {
        wrap_halo(0);
        wrap_halo(1);
    }
    if (a.n_steps > 0) {
        if (batched) {
            draw_batch(0, 0);
            draw_batch(1, 0);
        } else {
            draw_step(0, 0);
            draw_step(1, 0);
        }
    }
    __syncthreads();

    // ---- the tile stream. Interval i: stencil of tile i, MLP of tile i-1, update of tile i-2;
    // tile k belongs to run k / tg (group run & 1, step run >> 1), position k % tg in the run.
    const int T = a.n_steps * 2 * tg;
    int js = 0, runs = 0;  // stencil tile position
    int ju = 0, runu = 0;  // update tile position
    int slot_u = 0;        // fire slot of the update tile's step
    uint2 cis = cinfo[n], ciu = cis;
    auto adv = [&](int &j, int &run) __attribute__((always_inline)) {
        if (++j == tg) {
            j = 0;
            ++run;
        }
    };

    auto interval = [&](auto st_c, auto fc_c, auto up_c, auto par_c) __attribute__((always_inline)) {
        constexpr bool DST = decltype(st_c)::value, DFC = decltype(fc_c)::value, DUP = decltype(up_c)::value;
        constexpr unsigned PAR = decltype(par_c)::value;
        // next tiles' table entries (prefetched; the tables never change)
        int js_n = js, runs_n = runs, ju_n = ju, runu_n = runu;
        if (DST) adv(js_n, runs_n);
        if (DUP) adv(ju_n, runu_n);
        const int cbu = (runu & 1) * G + 16 * ju;
        uint2 cis_n = cis, ciu_n = ciu;
        if (DST) cis_n = cinfo[(runs_n & 1) * G + 16 * js_n + n];
        if (DUP || DFC) ciu_n = cinfo[(runu_n & 1) * G + 16 * ju_n + n];
        // ---- LDS loads of the interval
        uint2 nb[9];
        if (DST) {
            const unsigned r0 = cis.x + kPs, r1 = r0 + (unsigned)RP, r2 = r0 + RP2;
            nb[0] = lds_ld64(smem, r0);
            nb[1] = lds_ld64(smem, r0 + S::CS);
            nb[2] = lds_ld64(smem, r0 + 2 * S::CS);
            nb[3] = lds_ld64(smem, r1);
            nb[4] = lds_ld64(smem, r1 + S::CS);
            nb[5] = lds_ld64(smem, r1 + 2 * S::CS);
            nb[6] = lds_ld64(smem, r2);
            nb[7] = lds_ld64(smem, r2 + S::CS);
            nb[8] = lds_ld64(smem, r2 + 2 * S::CS);
        }
        bf16x8 zf[S::KT1];
        if (DFC) {
#pragma unroll
            for (int kt = 0; kt < S::KT1; ++kt)
                zf[kt] = *reinterpret_cast<const bf16x8 *>(smem + ((kt & 1) ? kZo : kZe) + (PAR ^ 1u) * S::ZBUF +
                                                           64u * kt);
        }
        float4 pv[4], m4;
        float fu = 0.0f;
        unsigned madr = 0, padr = 0;
        bool gv = false;
        if (DUP) {
#pragma unroll
            for (int w4 = 0; w4 < 4; ++w4) pv[w4] = lds_ld128f(smem, kDr + PAR * S::DBUF + (unsigned)w4 * 16u * S::DS);
            madr = sp.l_M + (unsigned)cbu * S::MS + kM;
            m4 = lds_ld128f(smem, madr);
            fu = (float)fireB[(unsigned)(slot_u * 2 * G + cbu + n)];
            gv = (int)ciu.y < 0;
            padr = (ciu.y & 0x7fffffffu) + 8u * iq;
        }
        // ---- stencil of tile i
        if (DST) {
            f32x4 zc[4];
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const uint32_t sel = (c & 1) ? 0x07060302u : 0x05040100u;
                const uint32_t p01 = __builtin_amdgcn_perm(c < 2 ? nb[1].x : nb[1].y, c < 2 ? nb[0].x : nb[0].y, sel);
                const uint32_t p23 = __builtin_amdgcn_perm(c < 2 ? nb[3].x : nb[3].y, c < 2 ? nb[2].x : nb[2].y, sel);
                const uint32_t p45 = __builtin_amdgcn_perm(c < 2 ? nb[5].x : nb[5].y, c < 2 ? nb[4].x : nb[4].y, sel);
                const uint32_t p67 = __builtin_amdgcn_perm(c < 2 ? nb[7].x : nb[7].y, c < 2 ? nb[6].x : nb[6].y, sel);
                const s16x4 a0 = __builtin_bit_cast(s16x4, make_uint2(p01, p23));
                const s16x4 a1 = __builtin_bit_cast(s16x4, make_uint2(p45, p67));
                const s16x4 a2 = __builtin_bit_cast(s16x4, nb[8]);
                f32x4 d = {0.f, 0.f, 0.f, 0.f};
                d = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(a0, kb0, d, 0, 0, 0);
                d = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(a1, kb1, d, 0, 0, 0);
                d = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(a2, kb2[c], d, 0, 0, 0);
                zc[c] = d;
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                uint2 o;
                o.x = pack_bf16x2(zc[0][r], zc[1][r]);
                o.y = pack_bf16x2(zc[2][r], zc[3][r]);
                lds_st64(smem, kZw + PAR * S::ZBUF + (unsigned)r * S::ZS, o);
            }
        }
        // ---- MLP of tile i-1
        if (DFC) {
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
            for (int kt = 0; kt < S::KT2; ++kt) {
                uint4 hv;
                hv.x = relu_bf16x2(pack_bf16x2(acc[2 * kt][0], acc[2 * kt][1]));
                hv.y = relu_bf16x2(pack_bf16x2(acc[2 * kt][2], acc[2 * kt][3]));
                hv.z = relu_bf16x2(pack_bf16x2(acc[2 * kt + 1][0], acc[2 * kt + 1][1]));
                hv.w = relu_bf16x2(pack_bf16x2(acc[2 * kt + 1][2], acc[2 * kt + 1][3]));
                hf[kt] = __builtin_bit_cast(bf16x8, hv);
            }
#pragma unroll
            for (int m2 = 0; m2 < S::MT2; ++m2) {
                f32x4 acc2 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int kt = 0; kt < S::KT2; ++kt)
                    acc2 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(w2f[m2][kt], hf[kt], acc2, 0, 0, 0);
                lds_st128f(smem, kDw + (PAR ^ 1u) * S::DBUF + 64u * m2, make_float4(acc2[0], acc2[1], acc2[2], acc2[3]));
            }
        }
        // ---- update of tile i-2
        if (DUP) {
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
                const float uv = __builtin_fmaf(fu, round_bf16(dsum[v]), xo[v]);  // fu in {0, 1}: exact
                u[v] = (gv && insl[v]) ? xo[v] : uv;
            }
            lds_st128f(smem, madr, make_float4(u[0], u[1], u[2], u[3]));
            lds_st64(smem, padr, make_uint2(pack_bf16x2(u[0], u[1]), pack_bf16x2(u[2], u[3])));
        }
        // advance: a new even run is the next step, whose fire slot follows
        js = js_n;
        runs = runs_n;
        cis = cis_n;
        if (DUP) {
            if (runu_n != runu && (runu_n & 1) == 0) slot_u = slot_u + 1 == NB ? 0 : slot_u + 1;
            ju = ju_n;
            runu = runu_n;
        }
        ciu = ciu_n;
    };
    // end-of-step work of the group of run `run`, whose last update was two intervals ago
    // (phase 1: first-step clamp) or three (phase 2: wrap halo, next fire masks)
    auto eos1 = [&](int run) __attribute__((always_inline)) {
        if ((run >> 1) == 0 && a.c_in > 0) clamp_pass(run & 1);
    };
    auto eos2 = [&](int run) __attribute__((always_inline)) {
        const int grp = run & 1, s = run >> 1;
        if (a.padding == 2) wrap_halo(grp);
        if (s + 1 < a.n_steps) {
            if (batched) {
                if ((s + 1) % NB == 0) draw_batch(grp, s + 1);
            } else {
                draw_step(grp, s + 1);
            }
        }
    };
    using F_ = std::integral_constant<bool, false>;
    using T_ = std::integral_constant<bool, true>;
    using P0 = std::integral_constant<unsigned, 0>;
    using P1 = std::integral_constant<unsigned, 1>;
    if (T > 0) {
        interval(T_{}, F_{}, F_{}, P0{});
        __syncthreads();
        interval(T_{}, T_{}, F_{}, P1{});
        __syncthreads();
        // steady state: intervals i, i+1 (i even). Interval i is at position jm of its run;
        // jm == 2 -> phase 1 (at i) and phase 2 (at i+1) of the previous run
        int jm = 2, erun = -1;
        for (int i = 2; i < T; i += 2) {
            interval(T_{}, T_{}, T_{}, P0{});
            if (jm == 2 && erun >= 0) eos1(erun);
            __syncthreads();
            interval(T_{}, T_{}, T_{}, P1{});
            if (jm == 2 && erun >= 0) eos2(erun);
            __syncthreads();
            jm += 2;
            if (jm == tg) {
                jm = 0;
                ++erun;
            }
        }
        interval(F_{}, T_{}, T_{}, P0{});
        __syncthreads();
        interval(F_{}, F_{}, T_{}, P1{});
        __syncthreads();
        eos1(2 * a.n_steps - 1);  // the last run's first-step clamp (one-step calls)
        __syncthreads();
    }

    // ---- write back
    for (int e = tid; e < Rw * S::C * HWn; e += 256) {
        const int rw = e / (S::C * HWn), rem = e - rw * S::C * HWn, ch = rem / HWn, q = rem - ch * HWn;
        a.x_out[rbase * S::C * HWn + e] = m_at(wg_cell(rw, q), ch);
    }
    if (a.conf_out) {
        float *confL = reinterpret_cast<float *>(smem + sp.l_D);  // D is free now
        for (int cell = tid; cell < Rw * HWn; cell += 256) {
            const int rw = cell / HWn, c = wg_cell(rw, cell - rw * HWn);
            int am;
            confL[cell] = cell_readout_fn([&](int v) { return m_at(c, a.out_off + v); }, a.c_out, a.n_out,
                                          a.head_kind, headL, headL + a.n_out * a.c_out, &am);
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
