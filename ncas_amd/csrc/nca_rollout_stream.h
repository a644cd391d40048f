// Streamed LDS-resident rollout kernel for bf16 cells with C = 64 channels and 256 hidden units
// (gfx950): the fast path of the bf16 rollout on small grids (up to about 10x10).
//
// A workgroup owns R rows (boards) for the whole call. The cells of its boards, board after board
// and step after step, form one stream: stream position p = (s R + r) HW + q is cell q of board r
// at step s. The stream is cut into 16-cell tiles (tile t = positions 16t .. 16t+15; a tile may
// span two boards or two steps, so no cell is padding).
//
// The workgroup has 8 waves, two per SIMD, specialised so that one wave's MFMAs overlap the other
// wave's VALU and LDS work on the same SIMD:
//   hidden wave w (0-3)    owns hidden units [64w, 64w+64) with its W1 fragments in AGPRs: fc1
//                          h = W1 z + b1 on v_mfma_f32_16x16x32_bf16 (B operand from Z), then
//                          bf16 rounding + ReLU (autocast rounds fc1's output before the ReLU)
//                          into H.
//   stencil wave (4, 5)    channels [32(w-4), 32(w-4)+32): the 3x3 perception on
//                          v_mfma_f32_4x4x4_16b_bf16. Lane (cell n, channel octet) reads the 9
//                          taps of its 8 channels from the perception buffer P, one 16-byte load
//                          each; each 4-lane block multiplies 4 cells' tap vectors by the 4
//                          kernels -> Z.
//   update wave (6, 7)     channels [32(w-6), 32(w-6)+32): fc2 dx = W2 h + b2 for two 16-channel
//                          m-tiles (W2 fragments in AGPRs, one read of H as the B operand of
//                          both), whose accumulator layout puts channels 4 iq .. 4 iq+3 of cell n
//                          in lane (n, g): the update x += fire * bf16(dx) into the fp32 state M
//                          and the bf16 buffer P happens in those registers; the clamped input
//                          channels of given cells keep their value.
// The four channel waves also share the end-of-step work (wrap halo refresh, fire masks).
//
// Interval i (one workgroup barrier) runs: stencil of tile i (-> Z[i & 1]); fc1 + epilogue of
// tile i-2 (-> H[i & 1]) from Z operands the hidden wave loaded into registers in interval i-1,
// while it loads those of tile i-1 from Z[(i-1) & 1]; fc2 + update of tile i-3 (from
// H[(i-1) & 1]). A hidden wave thus opens every interval with 32 MFMAs whose operands are
// already in registers.
//
// P is single-buffered: the update of tile i-3 runs in the same interval as the stencil of tile
// i, whose neighbourhoods reach W+1 <= 16 positions back, never into tile i-3. A board's next
// step starts (R-1) HW + 1 >= 80 positions after its previous step ended, so its first stencil
// comes at least five tiles after the tile holding its last cell: that tile's update (three
// intervals later) and, for wrap padding, the halo refresh of the interval after it are done
// before the board's next stencil reads P. Adaptive (confidence-gated) and injected fire masks
// of the board's next step are produced in that same interval. Uniform Philox masks are drawn
// for NB steps of all boards at a time into one half of a two-half byte ring, while the other
// half is being read.
//
// Clamp (model.py:430-438): the first step's perception reads the caller's state, and the
// step's output holds the clamp values in the input slice of given cells. The load therefore
// writes the caller's state into P and the clamped state into M; the update keeps those
// channels of given cells at their M value, which is bitwise the reference's clamp at every step.
//
// LDS layouts (gfx950: 64 banks of 4 bytes; measured with 8 waves streaming one access pattern,
// ds_read_b128 takes 4 cycles per instruction when conflict-free, ds_write_b128 13, ds_write_b64 6):
//   * P: cell stride 144 B, padded row pitch RP = 144 (W + 2) + 224 and board pitch PB = 144 HW
//     mod 256, so the byte address of stream cell p is 144 p + const mod 256 within a step: the 16
//     cells of a tile land on 16 distinct 16-byte bank groups. The stencil's tap loads still take
//     8 cycles, not 4: the four 16-lane groups of one load read octets 16 B apart in the same
//     cells, which gfx950 serves in two passes (the same loads with the groups 4 KB apart take
//     one; removing the extra pass would save about 1 % of the launch);
//   * M: 288 B per cell (64 fp32 + 32 B) (the update's b128 accesses: 4.4 cycles per read, 16
//     per write);
//   * Z: 576 B per tile row, features in quad-major order (16 iq + 4 head + ch), chunk c of row
//     r stored at chunk c ^ (2 ((r >> 2) & 3)) (conflict-free reads and writes);
//   * H: 544 B per tile row, 16-byte chunk c of row n stored at chunk c ^ ((n >> 2) & 1); the 16
//     hidden values of fc1 lane (n, g) of hidden wave w are contiguous at physical position
//     64 w + 16 g + 4 mt + v (logical hidden unit 64 w + 16 mt + 4 g + v); the fc2 fragments are
//     packed in that order (conflict-free reads and writes).
// Per 16-cell interval the LDS serves about 70 KB of reads and 22 KB of writes, about 670 cycles of
// its time, beside 768 MFMA cycles on each of SIMDs 2-3; the hidden waves' own Z loads and H stores
// are on the interval's critical path (without them the launch would take about a fifth less).
#pragma once

#include <type_traits>

#include "nca_stream_util.h"

namespace nca {

struct St64 {
    static constexpr int C = 64, HD = 256, F = 256;
    static constexpr int MT1 = 4, KT1 = 8, KT2 = 8;
    static constexpr int CS = 144;   // P bytes per cell (64 bf16 + 8 pad)
    static constexpr int MS = 288;   // M bytes per cell (64 fp32 + 8 pad)
    static constexpr int ZS = 576;   // Z bytes per tile row (256 bf16 + 32 pad)
    static constexpr int HS = 544;   // H bytes per tile row (256 bf16 + 16 pad)
    static constexpr int ZBUF = 16 * ZS;
    static constexpr int HBUF = 16 * HS;
    static constexpr int RPAD = 224;  // (-2 * CS) mod 256
    static constexpr int GAP = 79;    // (R-1) HW must reach this
};

struct StPlan {
    unsigned P, M, Z, H, cinfo, ring, fired, head, hcp, evp, total;
    int R, RP, PB, NB, RH, RING;
};


// R rows per workgroup, NB steps per fire-mask batch (1 for per-step masks).
inline StPlan st_plan(int R, int H, int W, int c_out, int n_out, int NB) {
    using S = St64;
    StPlan p;
    const int HWn = H * W;
    p.R = R;
    p.RH = R * HWn;
    p.NB = NB;
    p.RING = 2 * NB * p.RH;
    p.RP = (W + 2) * S::CS + S::RPAD;
    const int pb0 = (H + 2) * p.RP;
    p.PB = pb0 + (((S::CS * HWn - pb0) % 256) + 256) % 256;
    unsigned o = 0;
    p.P = o;
    o = st_al16(o + (unsigned)R * (unsigned)p.PB);
    p.M = o;
    o = st_al16(o + (unsigned)p.RH * S::MS);
    p.Z = o;
    o += 2u * S::ZBUF;
    p.H = o;
    o += 2u * S::HBUF;
    p.cinfo = o;
    o = st_al16(o + (unsigned)(p.RH + 16) * 8u);
    p.ring = o;
    o = st_al16(o + (unsigned)p.RING + 16u);
    p.fired = o;
    o = st_al16(o + (unsigned)R * 4u);
    p.head = o;
    o = st_al16(o + (unsigned)(n_out * c_out + n_out) * 4u);
    p.hcp = o;
    o = st_al16(o + (unsigned)(2 * (W + 2) + 2 * H) * 4u);
    p.evp = o;  // a copy of the call's parameters for the end-of-step work
    o = st_al16(o + (unsigned)sizeof(RolloutParams));
    p.total = o;
    return p;
}

struct StParams {
    RolloutParams a;
    int R, RP, PB, NB, RH, RING, T;
    unsigned l_P, l_M, l_Z, l_H, l_cinfo, l_ring, l_fired, l_head, l_hcp, l_evp;
    unsigned off_w1q, off_w2h;
};

__global__ void __launch_bounds__(512, 1) rollout_stream64(StParams sp) {
    using S = St64;
    constexpr int NT = 512;
    const RolloutParams &a = sp.a;
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, n = lane & 15;  // n: cell of the tile (MFMA column), g: lane group
    const bool hidden_wave = wave < 4;
    const int ws = wave & 3;                 // hidden slice or channel set of the wave
    const int tb = tid - 256;                // thread index among the channel waves
    const int H = a.H, W = a.W, HWn = H * W;
    const int R = sp.R, RH = sp.RH, RP = sp.RP, PB = sp.PB, NB = sp.NB, RING = sp.RING;
    const int64_t rbase = (int64_t)blockIdx.x * R;
    const int Rw = (int)((a.rows - rbase) < R ? (a.rows - rbase) : R);

    int *firedL = reinterpret_cast<int *>(smem + sp.l_fired);
    float *headL = reinterpret_cast<float *>(smem + sp.l_head);
    unsigned *hcp = reinterpret_cast<unsigned *>(smem + sp.l_hcp);
    uint2 *cinfo = reinterpret_cast<uint2 *>(smem + sp.l_cinfo);
    unsigned char *ring = smem + sp.l_ring;

    // byte offset of the centre of cell q of board r in P; of cell q of board r in M
    auto p_cell = [&](int r, int q) -> unsigned {
        const int i = q / W, j = q - i * W;
        return sp.l_P + (unsigned)(r * PB + (i + 1) * RP + (j + 1) * S::CS);
    };
    auto m_cell = [&](int r, int q) -> unsigned { return sp.l_M + (unsigned)(r * HWn + q) * S::MS; };
    auto m_at = [&](int r, int q, int ch) -> float & {
        return *reinterpret_cast<float *>(smem + m_cell(r, q) + 4u * (unsigned)ch);
    };

    // ---- load rows (phantom rows of a ragged last workgroup hold zeros and never fire)
    for (int e = tid; e < R * S::C * HWn; e += NT) {
        const int r = e / (S::C * HWn), rem = e - r * S::C * HWn, ch = rem / HWn, q = rem - ch * HWn;
        const float v = r < Rw ? a.x_in[rbase * S::C * HWn + e] : 0.0f;
        m_at(r, q, ch) = v;
        *reinterpret_cast<__bf16 *>(smem + p_cell(r, q) + 2 * ch) = (__bf16)v;
    }
    for (int c = tid; c < RH + 16; c += NT) {
        const int cc = c < RH ? c : c - RH, r = cc / HWn, q = cc - r * HWn;
        uint2 ci;
        ci.x = p_cell(r, q);
        ci.y = m_cell(r, q) | (r < Rw && a.given[(rbase + r) * HWn + q] ? 0x80000000u : 0u);
        cinfo[c] = ci;
    }
    for (int e = tid; e < R; e += NT) firedL[e] = 0;
    for (int e = tid; e < (int)(sizeof(RolloutParams) / 4); e += NT)
        reinterpret_cast<unsigned *>(smem + sp.l_evp)[e] = reinterpret_cast<const unsigned *>(&a)[e];
    {
        const float *hw = reinterpret_cast<const float *>(a.packed + a.off_headw);
        const float *hb = reinterpret_cast<const float *>(a.packed + a.off_headb);
        const int nw = a.n_out * a.c_out;
        for (int e = tid; e < nw + a.n_out; e += NT) headL[e] = e < nw ? hw[e] : hb[e - nw];
    }
    const int Wp = W + 2, nhalo = 2 * Wp + 2 * H;
    for (int h = tid; h < nhalo; h += NT) {
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
        for (int r = 0; r < R; ++r)
            for (int e = tid; e < nhalo * S::C; e += NT) {
                const int h = e >> 6, ch = e & 63;
                const unsigned dst = hcp[h] & 0xffffu;
                *reinterpret_cast<__bf16 *>(smem + sp.l_P + (unsigned)(r * PB) + dst + 2 * ch) =
                    (__bf16)(a.padding == 1 ? padv[ch] : 0.0f);
            }
    } else {
        for (int r = 0; r < R; ++r) {
            const unsigned base = sp.l_P + (unsigned)(r * PB);
            for (int e = tid; e < nhalo * 8; e += NT) {
                const unsigned hc = hcp[e >> 3], o = 16u * (unsigned)(e & 7);
                const float4 v = lds_ld128f(smem, base + (hc >> 16) + o);
                lds_st128f(smem, base + (hc & 0xffffu) + o, v);
            }
        }
    }
    // ---- end-of-step work, done by the channel waves (thread tb of 256)
    // fire byte of stream position (s, r, q): ring slot ((s mod 2NB) RH + r HW + q); slots below
    // 16 are mirrored after the ring so that a tile reads 16 consecutive bytes
    auto ring_put = [&](int s, int r, int q, int f) __attribute__((always_inline)) {
        const int o = (s % (2 * NB)) * RH + r * HWn + q;
        ring[o] = (unsigned char)f;
        if (o < 16) ring[RING + o] = (unsigned char)f;
    };
    // uniform Philox masks of all boards for the steps of batch b (non-adaptive, no injected
    // masks), one Philox evaluation per 4 cells
    const int nq4 = (HWn + 3) >> 2;
    const bool batched = !a.adaptive && !a.fire_u8;
    // fired cells are counted only for a caller that asks for them
    const bool count_fired = a.fired_out != nullptr;
    // a batch has at most 256 items when NB > 1 (one per channel-wave thread): this thread's
    // first item (board, step of the batch, group of 4 cells), found once
    const int per_row = NB * nq4;
    const int dr0 = tb >= 0 ? tb / per_row : 0, drem0 = tb - dr0 * per_row;
    const int dsl0 = drem0 / nq4, dqq0 = drem0 - dsl0 * nq4;
    auto draw_batch = [&](const RolloutParams &pa, int b) __attribute__((always_inline)) {
        for (int it = tb; it < R * per_row; it += 256) {
            int r = dr0, sl = dsl0, qq = dqq0;
            if (it != tb) {
                r = it / per_row;
                const int rem = it - r * per_row;
                sl = rem / nq4;
                qq = rem - sl * nq4;
            }
            const int s = b * NB + sl;
            if (s >= pa.n_steps) continue;
            float u[4] = {1.0f, 1.0f, 1.0f, 1.0f};
            if (r < Rw) {
                const uint64_t key = pa.step_seeds ? pa.step_seeds[s] : pa.seed;
                cell_uniforms4(key, (uint32_t)(pa.row0 + rbase + r), (uint32_t)(pa.step0 + s), (uint32_t)qq, u);
            }
            int cnt = 0;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int q = 4 * qq + e;
                if (q < HWn) {
                    const int f = r < Rw && u[e] < pa.p;
                    ring_put(s, r, q, f);
                    cnt += f;
                }
            }
            if (count_fired && cnt) atomicAdd(&firedL[r], cnt);
        }
    };
    // masks of board r for step s: adaptive gating reads the board's current state (the state
    // before step s), injected masks are copied
    auto draw_step = [&](const RolloutParams &pa, int r, int s) __attribute__((always_inline)) {
        for (int it = tb; it < nq4; it += 256) {
            const int qq = it;
            float u[4] = {1.0f, 1.0f, 1.0f, 1.0f};
            if (r < Rw && !pa.fire_u8) {
                const uint64_t key = pa.step_seeds ? pa.step_seeds[s] : pa.seed;
                cell_uniforms4(key, (uint32_t)(pa.row0 + rbase + r), (uint32_t)(pa.step0 + s), (uint32_t)qq, u);
            }
            int cnt = 0;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int q = 4 * qq + e;
                if (q >= HWn) continue;
                int f = 0;
                if (r < Rw) {
                    if (pa.fire_u8) {
                        f = pa.fire_u8[((int64_t)s * pa.rows + rbase + r) * HWn + q] != 0;
                    } else {
                        float pc = pa.p;
                        if (pa.adaptive) {
                            int am;
                            const float cf = cell_readout_fn([&](int v) { return m_at(r, q, pa.out_off + v); }, pa.c_out,
                                                             pa.n_out, pa.head_kind, headL, headL + pa.n_out * pa.c_out,
                                                             &am);
                            if (cf > pa.tau || (pa.given_confident && pa.given[(rbase + r) * HWn + q])) pc = pa.p_low;
                        }
                        f = u[e] < pc;
                    }
                }
                ring_put(s, r, q, f);
                cnt += f;
            }
            if (count_fired && cnt) atomicAdd(&firedL[r], cnt);
        }
    };
    __syncthreads();
    if (!hidden_wave && a.n_steps > 0) {
        if (batched) {
            draw_batch(a, 0);
            draw_batch(a, 1);
        } else {
            for (int r = 0; r < R; ++r) draw_step(a, r, 0);
        }
    }
    __syncthreads();
    // the step's clamp lands in M (P keeps the caller's state for the first perception)
    if (a.n_steps > 0 && a.c_in > 0) {
        for (int e = tid; e < Rw * HWn * a.c_in; e += NT) {
            const int cell = e / a.c_in, ci = e - cell * a.c_in;
            const int r = cell / HWn, q = cell - r * HWn;
            if (!a.given[(rbase + r) * HWn + q]) continue;
            m_at(r, q, a.in_off + ci) = a.clamp[((rbase + r) * a.c_in + ci) * HWn + q];
        }
    }
    __syncthreads();

    using F_ = std::integral_constant<bool, false>;
    using T_ = std::integral_constant<bool, true>;
    using P0 = std::integral_constant<unsigned, 0>;
    using P1 = std::integral_constant<unsigned, 1>;
    const int T = sp.T;
    const int total = a.n_steps * RH;
    // Both wave kinds run the same interval sequence (prologue 0-2, steady state, drain T..T+2)
    // with one workgroup barrier per interval.
    if (T > 0 && hidden_wave) {
        // ================= hidden waves: fc1 + epilogue
        bf16x8 w1f[S::MT1][S::KT1];
        f32x4 b1v[S::MT1];
        {
            const bf16x8 *w1 = reinterpret_cast<const bf16x8 *>(a.packed + sp.off_w1q);
            const float *b1 = reinterpret_cast<const float *>(a.packed + a.off_b1);
#pragma unroll
            for (int mt = 0; mt < S::MT1; ++mt) {
#pragma unroll
                for (int kt = 0; kt < S::KT1; ++kt) w1f[mt][kt] = w1[((ws * S::MT1 + mt) * S::KT1 + kt) * 64 + lane];
#pragma unroll
                for (int v = 0; v < 4; ++v) b1v[mt][v] = b1[ws * 64 + 16 * mt + 4 * g + v];
            }
#pragma unroll
            for (int mt = 0; mt < S::MT1; ++mt)
#pragma unroll
                for (int kt = 0; kt < S::KT1; ++kt) asm volatile("" : "+a"(w1f[mt][kt]));
        }
        const int sig = 2 * ((n >> 2) & 3);
        const unsigned kZ0 = sp.l_Z + (unsigned)n * S::ZS + 16u * (unsigned)(g ^ (sig & 3));
        const unsigned kZe = kZ0 + 64u * (unsigned)(sig >> 2), kZo = kZ0 - 64u * (unsigned)(sig >> 2);
        // H row n: 16-byte chunk c stored at chunk c ^ hx, hx = (n >> 2) & 1
        const unsigned hx = (unsigned)((n >> 2) & 1);
        const unsigned kHw0 = sp.l_H + (unsigned)n * S::HS + 128u * (unsigned)ws + 32u * (unsigned)g + 16u * hx;
        const unsigned kHw1 = kHw0 + 16u - 32u * hx;
        bf16x8 zqb[2][S::KT1];
#pragma unroll
        for (int q = 0; q < 2; ++q)
#pragma unroll
            for (int k = 0; k < S::KT1; ++k)
#pragma unroll
                for (int e = 0; e < 8; ++e) zqb[q][k][e] = (__bf16)0.0f;
        // fcb: fc1 of tile i-2 (32 MFMAs from registers, m-tile by m-tile) and its epilogue ->
        // H[i & 1], each half stored as soon as its two m-tiles are done; fca: the Z operands of
        // tile i-1 into zqb[i & 1] (fc1 of tile i-2 reads zqb[(i-1) & 1]). The eight Z loads are
        // spread over m-tiles 1 and 2, one after every second MFMA, rather than issued as a burst:
        // the LDS is then still serving the channel waves' loads that open the interval, and a
        // load the wave cannot issue holds back its next MFMA (about 1 % of the launch).
        auto hinterval = [&](auto fca_c, auto fcb_c, auto par_c) __attribute__((always_inline)) {
            constexpr bool FCA = decltype(fca_c)::value, FCB = decltype(fcb_c)::value;
            constexpr unsigned PAR = decltype(par_c)::value;
            auto loadz1 = [&](int kt) __attribute__((always_inline)) {
                zqb[PAR][kt] = *reinterpret_cast<const bf16x8 *>(smem + ((kt & 1) ? kZo : kZe) + (PAR ^ 1u) * S::ZBUF +
                                                               64u * kt);
            };
            if (FCB) {
                f32x4 acc[S::MT1];
#pragma unroll
                for (int mt = 0; mt < S::MT1; ++mt) {
                    acc[mt] = b1v[mt];
#pragma unroll
                    for (int kt = 0; kt < S::KT1; ++kt) {
                        acc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(w1f[mt][kt], zqb[PAR ^ 1u][kt], acc[mt], 0, 0, 0);
                        if (FCA && (mt == 1 || mt == 2) && (kt & 1)) {
                            __builtin_amdgcn_sched_barrier(0);
                            loadz1((mt - 1) * 4 + (kt >> 1));
                            __builtin_amdgcn_sched_barrier(0);
                        }
                    }
                    if (mt & 1) {
                        uint4 hv;
                        hv.x = relu_bf16x2(cvt_pk_bf16(acc[mt - 1][0], acc[mt - 1][1]));
                        hv.y = relu_bf16x2(cvt_pk_bf16(acc[mt - 1][2], acc[mt - 1][3]));
                        hv.z = relu_bf16x2(cvt_pk_bf16(acc[mt][0], acc[mt][1]));
                        hv.w = relu_bf16x2(cvt_pk_bf16(acc[mt][2], acc[mt][3]));
                        lds_st128(smem, (mt == 1 ? kHw0 : kHw1) + PAR * S::HBUF, hv);
                    }
                }
            } else if (FCA) {
#pragma unroll
                for (int kt = 0; kt < S::KT1; ++kt) loadz1(kt);
            }
        };
        int i = 0;
        hinterval(F_{}, F_{}, P0{});
        __syncthreads();
        hinterval(T_{}, F_{}, P1{});
        __syncthreads();
        hinterval(T_{}, T_{}, P0{});
        __syncthreads();
        for (i = 3; i + 1 < T; i += 2) {
            hinterval(T_{}, T_{}, P1{});
            __syncthreads();
            hinterval(T_{}, T_{}, P0{});
            __syncthreads();
        }
        if (i < T) {
            hinterval(T_{}, T_{}, P1{});
            __syncthreads();
            ++i;
        }
        // drain: intervals T, T+1 (T+2 has no hidden work) with compile-time parities
        if (i & 1) {
            hinterval(T_{}, T_{}, P1{});
            __syncthreads();
            hinterval(F_{}, T_{}, P0{});
            __syncthreads();
        } else {
            hinterval(T_{}, T_{}, P0{});
            __syncthreads();
            hinterval(F_{}, T_{}, P1{});
            __syncthreads();
        }
        __syncthreads();
    } else if (T > 0) {
        // ================= channel waves: stencil (waves 4, 5) or fc2 + update (waves 6, 7) of
        // channels [32 cw, 32 cw + 32), and the end-of-step work (all four)
        // the channel waves hold the interval's longest dependency chains: their instructions win
        // the SIMD's issue arbitration over the hidden waves' MFMAs
        __builtin_amdgcn_s_setprio(3);
        const bool stencil_wave = wave < 6;
        const int cw = wave & 1;
        const unsigned kCi = sp.l_cinfo + 8u * (unsigned)n;
        const unsigned kRg = sp.l_ring + (unsigned)n;
        // the thread's (at most two, nhalo <= 64) 16-byte wrap-halo chunks: board-relative source
        // offset in the high half, destination in the low half, 0 when there is none (offset 0 is
        // a corner halo cell, never a source)
        auto halo_item = [&](int e) -> unsigned {
            if (e >= nhalo * 8) return 0u;
            const unsigned hc = hcp[e >> 3], o = 16u * (unsigned)(e & 7);
            return (((hc >> 16) + o) << 16) | ((hc & 0xffffu) + o);
        };
        const unsigned hsd0 = a.padding == 2 ? halo_item(tb) : 0u, hsd1 = a.padding == 2 ? halo_item(tb + 256) : 0u;
        // wrap halo of board r after one of its steps: both chunks loaded, then stored
        auto wrap_halo = [&](int r) __attribute__((always_inline)) {
            const unsigned base = sp.l_P + (unsigned)(r * PB);
            float4 v0, v1;
            if (hsd0) v0 = lds_ld128f(smem, base + (hsd0 >> 16));
            if (hsd1) v1 = lds_ld128f(smem, base + (hsd1 >> 16));
            if (hsd0) lds_st128f(smem, base + (hsd0 & 0xffffu), v0);
            if (hsd1) lds_st128f(smem, base + (hsd1 & 0xffffu), v1);
        };

        int i = 0;
        // unit (board ur, step us) ends at stream position uend; batch nb is drawn when the update
        // stage has passed position dpos = (nb - 1) NB RH
        const bool unit_events = a.padding == 2 || !batched;
        int ur = 0, us = 0, uend = HWn - 1;
        int ev_unit = unit_events ? (uend >> 4) + 4 : 0x7fffffff;
        int nb = 2, dpos = NB * RH;
        int ev_batch = (batched && 2 * NB < a.n_steps) ? (dpos >> 4) + 4 : 0x7fffffff;

        // the end-of-step work reads the call's parameters from the LDS copy, so that they do not
        // occupy scalar registers through the loop
        const bool wrap = a.padding == 2;
        auto events = [&]() __attribute__((always_inline)) {
            const RolloutParams &ea = *reinterpret_cast<const RolloutParams *>(smem + sp.l_evp);
            while (i == ev_unit) {
                if (wrap) wrap_halo(ur);
                if (!batched && us + 1 < ea.n_steps) draw_step(ea, ur, us + 1);
                if (++ur == R) {
                    ur = 0;
                    ++us;
                }
                uend += HWn;
                ev_unit = (uend >> 4) + 4;
            }
            if (i == ev_batch) {
                draw_batch(ea, nb);
                ++nb;
                dpos += NB * RH;
                ev_batch = nb * NB < ea.n_steps ? (dpos >> 4) + 4 : 0x7fffffff;
            }
        };
        if (stencil_wave) {
            // stencil B operands: column j = lane % 4 is kernel j; taps 0-3, 4-7; tap 8 placed at
            // the k slot of channel c % 4 (the A operand of tap 8 is 4 channels' tap-8 values)
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
            // lane (cell n, channel octet oc = 4 cw + g): taps of channels 8 oc .. 8 oc + 7, one
            // 16-byte load each. Output lane (block b, kernel j) holds rows r (cells 4 (b & 3) + r)
            // of octet 4 cw + b / 4: Z quads 2 oc and 2 oc + 1.
            const int oc = 4 * cw + g;
            unsigned kZw0, kZw1;
            {
                const int j = lane & 3, b = lane >> 2, ob = 4 * cw + (b >> 2), sw = 2 * (b & 3);
                const unsigned base = sp.l_Z + (unsigned)(4 * (b & 3)) * S::ZS + 8u * (unsigned)(j & 1);
                kZw0 = base + 16u * (unsigned)((2 * (2 * ob) + (j >> 1)) ^ sw);
                kZw1 = base + 16u * (unsigned)((2 * (2 * ob + 1) + (j >> 1)) ^ sw);
            }
            // + centre: the top-left tap, the left taps of the middle and bottom rows
            const unsigned kPs = 16u * (unsigned)oc - (unsigned)(RP + S::CS), kPs1 = kPs + (unsigned)RP,
                           kPs2 = kPs1 + (unsigned)RP;
            int cbS = 0;  // cinfo index of the stencil tile's first cell: (16 i) mod RH
            unsigned cis = cinfo[n].x, cis_n = 0;
            auto sinterval = [&](auto par_c) __attribute__((always_inline)) {
                constexpr unsigned PAR = decltype(par_c)::value;
                uint4 t[9];
                {
                    const unsigned r0 = cis + kPs, r1 = cis + kPs1, r2 = cis + kPs2;
                    t[0] = *reinterpret_cast<const uint4 *>(smem + r0);
                    t[3] = *reinterpret_cast<const uint4 *>(smem + r1);
                    t[6] = *reinterpret_cast<const uint4 *>(smem + r2);
                    t[1] = *reinterpret_cast<const uint4 *>(smem + r0 + S::CS);
                    t[4] = *reinterpret_cast<const uint4 *>(smem + r1 + S::CS);
                    t[7] = *reinterpret_cast<const uint4 *>(smem + r2 + S::CS);
                    t[2] = *reinterpret_cast<const uint4 *>(smem + r0 + 2 * S::CS);
                    t[5] = *reinterpret_cast<const uint4 *>(smem + r1 + 2 * S::CS);
                    t[8] = *reinterpret_cast<const uint4 *>(smem + r2 + 2 * S::CS);
                    int cs = cbS + 16;
                    if (cs >= RH) cs -= RH;
                    cis_n = lds_ld64(smem, kCi + 8u * (unsigned)cs).x;
                }
                auto word = [&](const uint4 &v, int c) -> uint32_t {
                    const int w = c >> 1;
                    return w == 0 ? v.x : w == 1 ? v.y : w == 2 ? v.z : v.w;
                };
                // channels 4 h .. 4 h + 3 of the octet: A operands (channel c, taps 0-3 / 4-7 as
                // packed bf16 pairs), 3 MFMAs each, then the quad's Z stores
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    f32x4 zc[4];
#pragma unroll
                    for (int cc = 0; cc < 4; ++cc) {
                        const int c = 4 * h + cc;
                        const uint32_t sel = (c & 1) ? 0x07060302u : 0x05040100u;
                        const s16x4 sa0 = __builtin_bit_cast(
                            s16x4, make_uint2(__builtin_amdgcn_perm(word(t[1], c), word(t[0], c), sel),
                                              __builtin_amdgcn_perm(word(t[3], c), word(t[2], c), sel)));
                        const s16x4 sa1 = __builtin_bit_cast(
                            s16x4, make_uint2(__builtin_amdgcn_perm(word(t[5], c), word(t[4], c), sel),
                                              __builtin_amdgcn_perm(word(t[7], c), word(t[6], c), sel)));
                        const s16x4 a2 = __builtin_bit_cast(s16x4, h ? make_uint2(t[8].z, t[8].w) : make_uint2(t[8].x, t[8].y));
                        f32x4 d = {0.f, 0.f, 0.f, 0.f};
                        d = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(sa0, kb0, d, 0, 0, 0);
                        d = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(sa1, kb1, d, 0, 0, 0);
                        d = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(a2, kb2[cc], d, 0, 0, 0);
                        zc[cc] = d;
                    }
                    const unsigned kz = (h ? kZw1 : kZw0) + PAR * S::ZBUF;
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        uint2 o;
                        o.x = cvt_pk_bf16(zc[0][r], zc[1][r]);
                        o.y = cvt_pk_bf16(zc[2][r], zc[3][r]);
                        lds_st64(smem, kz + (unsigned)r * S::ZS, o);
                    }
                }
            };
            auto advance = [&]() __attribute__((always_inline)) {
                ++i;
                cbS += 16;
                if (cbS >= RH) cbS -= RH;
                cis = cis_n;
            };
            while (i + 1 < T) {
                sinterval(P0{});
                events();
                advance();
                __syncthreads();
                sinterval(P1{});
                events();
                advance();
                __syncthreads();
            }
            if (i < T) {
                sinterval(P0{});
                events();
                advance();
                __syncthreads();
            }
            // drain: intervals T .. T+2 have no stencil work
            for (int k = 0; k < 3; ++k) {
                events();
                ++i;
                __syncthreads();
            }
        } else {
            // fc2 of m-tiles 2 cw and 2 cw + 1 (W2 fragments in AGPRs) and the update of their
            // channels: lane (cell n, g) holds quads iq0 = 8 cw + g and iq1 = iq0 + 4
            const int iq0 = 8 * cw + g, iq1 = iq0 + 4;
            bf16x8 w2f[2][S::KT2];
            f32x4 b2v[2];
            {
                const bf16x8 *w2 = reinterpret_cast<const bf16x8 *>(a.packed + sp.off_w2h);
                const float *b2 = reinterpret_cast<const float *>(a.packed + a.off_b2);
#pragma unroll
                for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
                    for (int kt = 0; kt < S::KT2; ++kt) w2f[mt][kt] = w2[((2 * cw + mt) * S::KT2 + kt) * 64 + lane];
#pragma unroll
                    for (int v = 0; v < 4; ++v) b2v[mt][v] = b2[4 * (mt ? iq1 : iq0) + v];
                }
#pragma unroll
                for (int mt = 0; mt < 2; ++mt)
#pragma unroll
                    for (int kt = 0; kt < S::KT2; ++kt) asm volatile("" : "+a"(w2f[mt][kt]));
            }
            // all ones where the lane's channel 4 iq + v lies in the clamped input slice
            unsigned imv[2][4];
#pragma unroll
            for (int mt = 0; mt < 2; ++mt)
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int c = 4 * (mt ? iq1 : iq0) + v;
                    imv[mt][v] = (c >= a.in_off && c < a.in_off + a.c_in) ? 0xffffffffu : 0u;
                    asm volatile("" : "+v"(imv[mt][v]));  // kept a plain VGPR mask
                }
            const unsigned hx = (unsigned)((n >> 2) & 1);
            const unsigned kHr = sp.l_H + (unsigned)n * S::HS + 16u * ((unsigned)g ^ hx);
            int cbU = RH - 48;    // cinfo index of the update tile's first cell: (16 (i-3)) mod RH
            int rbU = RING - 48;  // its ring slot: (16 (i-3)) mod RING
            uint2 ciu = make_uint2(0u, 0u), ciu_n = ciu;
            auto uinterval = [&](auto up_c, auto last_c) __attribute__((always_inline)) {
                constexpr bool DUP = decltype(up_c)::value, LAST = decltype(last_c)::value;
                const unsigned PAR = (unsigned)(i & 1);
                bf16x8 hb[S::KT2];
                float4 m4[2];
                unsigned madr = 0, padr = 0, gvm = 0;
                float fu = 0.0f;
                if (DUP) {
#pragma unroll
                    for (int kt = 0; kt < S::KT2; ++kt)
                        hb[kt] = *reinterpret_cast<const bf16x8 *>(smem + kHr + (PAR ^ 1u) * S::HBUF + 64u * kt);
                    madr = (ciu.y & 0x7fffffffu) + 16u * (unsigned)iq0;
                    m4[0] = lds_ld128f(smem, madr);
                    m4[1] = lds_ld128f(smem, madr + 64u);
                    fu = (float)smem[kRg + (unsigned)rbU];
                    gvm = (unsigned)((int)ciu.y >> 31);  // all ones for a given cell
                    padr = ciu.x + 8u * (unsigned)iq0;
                }
                {  // next interval's table entry (the tables never change)
                    int cu = cbU + 16;
                    if (cu >= RH) cu -= RH;
                    ciu_n = lds_ld64(smem, kCi + 8u * (unsigned)cu);
                }
                if (!DUP) return;
                f32x4 acc[2] = {b2v[0], b2v[1]};
#pragma unroll
                for (int kt = 0; kt < S::KT2; ++kt)
#pragma unroll
                    for (int mt = 0; mt < 2; ++mt)
                        acc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(w2f[mt][kt], hb[kt], acc[mt], 0, 0, 0);
                bool ok = true;
                if (LAST) ok = 16 * (i - 3) + n < total;
#pragma unroll
                for (int mt = 0; mt < 2; ++mt) {
                    const uint32_t d01 = cvt_pk_bf16(acc[mt][0], acc[mt][1]), d23 = cvt_pk_bf16(acc[mt][2], acc[mt][3]);
                    const float dx[4] = {bf16_lo(d01), bf16_hi(d01), bf16_lo(d23), bf16_hi(d23)};
                    const float xo[4] = {m4[mt].x, m4[mt].y, m4[mt].z, m4[mt].w};
                    float u[4];
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        const float uv = __builtin_fmaf(fu, dx[v], xo[v]);  // fu in {0, 1}: exact
                        const unsigned km = imv[mt][v] & gvm;                 // clamped: keep x
                        u[v] = __uint_as_float((km & __float_as_uint(xo[v])) | (~km & __float_as_uint(uv)));
                    }
                    if (ok) {
                        lds_st128f(smem, madr + 64u * mt, make_float4(u[0], u[1], u[2], u[3]));
                        lds_st64(smem, padr + 32u * mt, make_uint2(cvt_pk_bf16(u[0], u[1]), cvt_pk_bf16(u[2], u[3])));
                    }
                }
            };
            auto advance = [&]() __attribute__((always_inline)) {
                ++i;
                cbU += 16;
                if (cbU >= RH) cbU -= RH;
                rbU += 16;
                if (rbU >= RING) rbU -= RING;
                ciu = ciu_n;
            };
            while (i < 3) {
                uinterval(F_{}, F_{});
                events();
                advance();
                __syncthreads();
            }
            while (i < T + 2) {
                uinterval(T_{}, F_{});
                events();
                advance();
                __syncthreads();
            }
            uinterval(T_{}, T_{});
            events();
            advance();
            __syncthreads();
        }
    }

    // ---- write back
    for (int e = tid; e < Rw * S::C * HWn; e += NT) {
        const int r = e / (S::C * HWn), rem = e - r * S::C * HWn, ch = rem / HWn, q = rem - ch * HWn;
        a.x_out[rbase * S::C * HWn + e] = m_at(r, q, ch);
    }
    if (a.conf_out) {
        float *confL = reinterpret_cast<float *>(smem + sp.l_Z);  // Z is free now
        for (int cell = tid; cell < Rw * HWn; cell += NT) {
            const int r = cell / HWn, q = cell - r * HWn;
            int am;
            confL[cell] = cell_readout_fn([&](int v) { return m_at(r, q, a.out_off + v); }, a.c_out, a.n_out,
                                          a.head_kind, headL, headL + a.n_out * a.c_out, &am);
        }
        __syncthreads();
        for (int r = tid; r < Rw; r += NT) {
            float sum = 0.0f;
            for (int q = 0; q < HWn; ++q) sum = __fadd_rn(sum, confL[r * HWn + q]);
            a.conf_out[rbase + r] = __fdiv_rn(sum, (float)HWn);
        }
    }
    if (a.fired_out)
        for (int r = tid; r < Rw; r += NT) a.fired_out[rbase + r] = firedL[r];
}

}  // namespace nca
