// Streamed LDS-resident rollout kernel for bf16 cells with C = 32 channels and 256 hidden units
// (gfx950): the rollout of boards up to 31 cells wide whose fp32 state fits the LDS (30x30: one
// board per workgroup, 127 KB of state), D steps in one launch.
//
// One workgroup owns one row (board) for the whole call. Its cells, step after step, form one
// stream: position p = s HW + q is cell q at step s. The stream is cut into 16-cell tiles (a tile
// may span two steps, so no cell is padding).
//
// The state lives only in fp32, in M: the stencil reads its taps as fp32 and rounds them to bf16
// in registers (the rounding autocast applies before the convolution), which also puts them in
// the MFMA operand order. M holds the board inside a one-cell border of constant cells (the wall
// value or zero), rows W+1 cells apart, so the right border cell of a row is the left border cell
// of the next: cell (i, j) is M cell (i+1)(W+1) + j + 1, 128 bytes each.
//
// The workgroup has 8 waves, two per SIMD:
//   hidden wave w (0-3)    hidden units [64w, 64w+64), W1 fragments in AGPRs: fc1 of a tile (16
//                          v_mfma_f32_16x16x32_bf16 from Z operands loaded in the previous
//                          interval), bf16 rounding + ReLU in registers, then fc2 over its 64
//                          hidden units for all 32 channels (4 MFMAs whose B operand is the
//                          epilogue's registers) -> fp32 partial sums in D.
//   stencil wave (4, 5)    cells 8(w-4) .. 8(w-4)+7 of a tile, all 8 channel quads: lane (cell,
//                          quad) loads the 9 taps of its 4 channels (a 16-lane group reads two
//                          whole cells, free of bank conflicts) and runs the 3x3 perception on
//                          v_mfma_f32_4x4x4_16b_bf16 -> Z.
//   update wave (6, 7)     cells 8(w-6) .. 8(w-6)+7 of a tile, all quads: dx = bf16(b2 + the four
//                          partial sums in a fixed order), x += fire dx into M; the clamped input
//                          channels of given cells keep their value. With confidence-gated firing
//                          each of the cell's 8 lanes reads the output quad of its state at the
//                          start of the step (M before the update) and makes the same decision.
// Interval i (one workgroup barrier): stencil of tile i -> Z[i & 1]; fc1 + fc2 partials of tile
// i-2 -> D[i & 1], while the Z operands of tile i-1 load from Z[(i-1) & 1] into registers for the
// next interval; update of tile i-3 from D[(i-1) & 1]. The stencil waves likewise load the next
// tile's taps while they work on this one.
//
// M is updated in place. The stencil waves load the taps of tile i+1 in interval i: positions
// 16(i+1) - (W+1) .. 16(i+1) + 15 + (W+1) of its step, while the update of tile i-3 in the same
// interval writes positions 16i - 48 .. 16i - 33: disjoint for W <= 31. Those taps hold the step's
// state once the previous step's updates of the same cells are done, up to position
// 16(i+1) + 16 + W - HW in tile i-4 or earlier: HW >= W + 81.
//
// Fire masks: a four-step byte ring in stream order (4 HW bytes and a 16-byte mirror of its
// start, so that a tile's 16 bytes are contiguous): bit 0 fire, bit 1 (u < p_low) for gated
// firing, bit 7 the cell's given flag. The channel waves draw the Philox uniforms of a whole step
// two steps ahead (one evaluation per 4 cells); with gating the update chooses between the two
// threshold bits. The decision needs only conf > tau: for a 2-output mlp head that is s < conf_s
// on the sum of exponentials s, with conf_s found on the host with the readout's own division,
// and since s = 1 + readout_expf(gap) grows with the gap between the two logits, a comparison of
// the gap with a limit found on the host (no exponential, no division).
//
// Clamp (model.py:430-438): the first step's perception reads the caller's state and every step's
// output holds the clamp values in the input slice of given cells. M starts as the caller's state;
// the update keeps those channels of given cells at their M value, which after the first step is
// the clamp value. When the caller's state already holds the clamp values there (the usual case),
// the first step needs nothing else; otherwise its updates take the values from the clamp tensor.
//
// LDS layouts (conflict-free for the access patterns here on gfx950's 64 banks):
//   * M: 128 B per cell; 16-lane groups read or write two cells x 8 quads;
//   * Z: 256 B per tile row (features in quad-major order 16 quad + 4 kernel + ch), 16-byte chunk c
//     of row r stored at chunk c ^ zsw(r);
//   * D: per partial 16 rows of 128 B (32 fp32), chunk c of row r stored at c ^ (r >> 1 & 7).
// gfx950 serves a ds_read_b128 in four cycles of 16 lanes: lanes 0-3 and 12-15 of a 16-lane group
// with lanes 4-11 of the next group (groups 0/1 and 2/3), then the remaining 16; the 16 lanes of a
// cycle must read distinct 16-byte slots of the 256-byte bank row (measured: a two-way conflict in
// those sets doubles the instruction's 4 cycles). zsw maps rows 0-3, 12-15 to 0-7 and rows 4-11 to
// 8-15 and keeps bit 0 of the chunk free, so the hidden waves' operand loads (group g reads chunk
// 4 kt + g of rows 0-15) fill each cycle's 16 slots; the stencil's stores of 8 rows x 4 chunks still
// meet every slot twice.
#pragma once

#include "nca_stream_util.h"

namespace nca {

struct St32 {
    static constexpr int C = 32, HD = 256, F = 128;
    static constexpr int MT1 = 4, KT1 = 4;  // fc1 per hidden wave: 64 hidden x 128 features
    static constexpr int MT2 = 2, KT2 = 2;  // fc2 per hidden wave: 32 channels x its 64 hidden
    static constexpr int MS = 128;          // M bytes per cell
    static constexpr int ZS = 256;          // Z bytes per tile row
    static constexpr int ZBUF = 16 * ZS;
    static constexpr int DS = 128;          // D bytes per row of one partial
    static constexpr int DPART = 16 * DS;
    static constexpr int DBUF = 4 * DPART;
    static constexpr int NSLOT = 4;  // fire ring steps
};

// (kHaloSpin, nca_stream.h: re-reads of an exchange word before a piece gives up on its
// neighbour; after that its halo rows are NaN and it waits no more)

struct St32Plan {
    unsigned M, Z, D, cinfo, ring, given, head, evp, flags, gidx, total;
    int NM, RING;
};

// H: the rows one workgroup runs (a board's, or a piece's); pieces: with the board-cell table
inline St32Plan st32_plan(int H, int W, int c_out, int n_out, bool pieces = false) {
    using S = St32;
    St32Plan p;
    const int HWn = H * W;
    p.NM = (H + 1) * (W + 1) + W + 2;
    p.RING = S::NSLOT * HWn;
    unsigned o = 0;
    p.M = o;
    o = st_al16(o + (unsigned)p.NM * S::MS);
    p.Z = o;
    o += 2u * S::ZBUF;
    p.D = o;
    o += 2u * S::DBUF;
    p.cinfo = o;  // u16 M cell index of board cell q, q < HW + 16 (the last 16 repeat the first)
    o = st_al16(o + (unsigned)(HWn + 16) * 2u);
    p.ring = o;
    o = st_al16(o + (unsigned)p.RING + 16u);
    p.given = o;
    o = st_al16(o + (unsigned)((HWn + 31) / 32) * 4u);
    p.head = o;
    o = st_al16(o + (unsigned)(n_out * c_out + n_out) * 4u);
    p.evp = o;  // a copy of the call's parameters for the per-step draws
    o = st_al16(o + (unsigned)sizeof(RolloutParams));
    p.flags = o;  // [0] fired count, [1] first-step clamp needed, [2..5] two per-step keys
    o = st_al16(o + 24u);
    p.gidx = o;  // pieces: u16 board cell of stream position q, q < HW
    if (pieces) o = st_al16(o + (unsigned)HWn * 2u);
    p.total = o;
    return p;
}

struct St32Params {
    RolloutParams a;
    int NM, RING, T;
    // gated firing with an mlp head of 2 outputs: conf = 1/s > tau exactly when s < conf_s (s the
    // sum of exponentials, conf_s computed on the host with IEEE division), and s = 1 +
    // readout_expf(d) for the gap d = min - max of the two logits, which is non-decreasing in d, so
    // exactly when d <= conf_d (found on the host through the same readout_expf); fast_conf
    // selects it
    float conf_s;
    float conf_d;
    int fast_conf;
    unsigned l_M, l_Z, l_D, l_cinfo, l_ring, l_given, l_head, l_evp, l_flags, l_gidx;
    unsigned off_w1q, off_w2k;
    // board pieces (recording kernel only): P workgroups per board, piece p runs board rows
    // [p Hp, p Hp + Hp) (the last piece may have fewer); xch: the exchange slots, (rows, P, 2, 4,
    // W, 32) words of (step tag << 32 | fp32 bits), all zero at the launch
    int P, Hp;
    uint64_t *xch;
    // a piece whose wait for a neighbour's row runs out sets *halo_status to 1 (the host clears
    // it); a wait re-reads at most spin_limit times; tag_skew (0 in use) makes every wait look
    // for a tag that never comes, so the host can force the bounded waits to run out
    uint32_t *halo_status;
    int spin_limit, tag_skew;
    // the repair launch after a launch in pieces: whole boards, run only when *run_if != 0 (a
    // piece's wait ran out), otherwise every workgroup returns at once
    const uint32_t *run_if;
};

// zsw: the Z row swizzle (a permutation of 0..15)
__device__ __forceinline__ unsigned zsw(unsigned r) { return row_swz16(r); }

// GATED: confidence-gated firing (a.adaptive), compiled out of the plain kernel
// REC: also write the state after every step to a.x_rec (the BPTT chunk's forward).
template <bool GATED, bool REC>
__global__ void __launch_bounds__(512, 1) rollout_stream32(St32Params sp) {
    using S = St32;
    constexpr int NT = 512;
    const RolloutParams &a = sp.a;
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];

    if (REC && sp.run_if && __hip_atomic_load(sp.run_if, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0u) return;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // the workgroup runs rows [r0, r0 + Hs) of board `row`: all of it, or piece `piece` of P. An
    // even piece streams its rows top to bottom, an odd one bottom to top, so two neighbours
    // meet at rows both stream first or both stream last; M keeps the board's orientation.
    const int P = REC ? sp.P : 1;
    const int64_t row = P > 1 ? (int64_t)(blockIdx.x / (unsigned)P) : (int64_t)blockIdx.x;
    const int piece = P > 1 ? (int)(blockIdx.x - (unsigned)row * (unsigned)P) : 0;
    const int W = a.W, Ht = a.H, HWt = Ht * W;
    const int r0 = piece * sp.Hp;
    const int Hs = P > 1 ? (Ht - r0 < sp.Hp ? Ht - r0 : sp.Hp) : Ht;
    const bool down = (piece & 1) == 0;
    const int HWn = Hs * W, RING = S::NSLOT * HWn;
    const int tb = tid - 256;  // thread index among the channel waves

    float *headL = reinterpret_cast<float *>(smem + sp.l_head);
    int *flagsL = reinterpret_cast<int *>(smem + sp.l_flags);
    unsigned short *cinfo = reinterpret_cast<unsigned short *>(smem + sp.l_cinfo);
    unsigned *givenL = reinterpret_cast<unsigned *>(smem + sp.l_given);
    unsigned char *ring = smem + sp.l_ring;

    // M cell and board cell of stream position q (row q / W of the workgroup's stream)
    auto m_index = [&](int q) -> int {
        const int k = q / W, j = q - k * W;
        return ((down ? k : Hs - 1 - k) + 1) * (W + 1) + j + 1;
    };
    auto g_index = [&](int q) -> int {
        const int k = q / W, j = q - k * W;
        return (r0 + (down ? k : Hs - 1 - k)) * W + j;
    };
    auto m_at = [&](int q, int ch) -> float & {
        return *reinterpret_cast<float *>(smem + sp.l_M + (unsigned)m_index(q) * S::MS + 4u * (unsigned)ch);
    };

    // ---- set-up: border cells, the caller's state, tables
    {
        const float *padv = reinterpret_cast<const float *>(a.packed + a.off_padv);
        float *M = reinterpret_cast<float *>(smem + sp.l_M);
        for (int e = tid; e < sp.NM * S::C; e += NT) M[e] = a.padding == 1 ? padv[e & (S::C - 1)] : 0.0f;
    }
    if (tid == 0) {
        flagsL[0] = 0;
        flagsL[1] = 0;
    }
    for (int e = tid; e < (HWn + 31) / 32; e += NT) givenL[e] = 0u;
    __syncthreads();
    {
        // batches of 8 loads per thread issued before their stores (a store after each load would
        // wait for every load in turn: 56 round trips per thread for a 30x30 board)
        constexpr int kB = 8;
        const float *xr = a.x_in + row * S::C * HWt;
        // board rows rlo .. rhi: the workgroup's and, for a piece, the halo rows inside the board
        const int rlo = r0 > 0 ? r0 - 1 : 0, rhi = r0 + Hs < Ht ? r0 + Hs : Ht - 1;
        const int NR = (rhi - rlo + 1) * W;
        const int N = S::C * NR;
        float *M = reinterpret_cast<float *>(smem + sp.l_M);
        for (int e0 = tid; e0 < N; e0 += NT * kB) {
            float v[kB];
#pragma unroll
            for (int k = 0; k < kB; ++k) {
                const int e = e0 + NT * k, ec = e < N ? e : N - 1;
                const int ch = ec / NR, c = ec - ch * NR;
                v[k] = xr[ch * HWt + rlo * W + c];
            }
#pragma unroll
            for (int k = 0; k < kB; ++k) {
                const int e = e0 + NT * k;
                if (e < N) {
                    const int ch = e / NR, c = e - ch * NR, rr = c / W, j = c - rr * W;
                    M[((rlo + rr - r0 + 1) * (W + 1) + j + 1) * S::C + ch] = v[k];
                    // the copy of the caller's state (the chunk's first record): the workgroup's
                    // own rows only
                    if (REC && a.x_rec0 && rlo + rr >= r0 && rlo + rr < r0 + Hs)
                        a.x_rec0[row * S::C * HWt + ch * HWt + rlo * W + c] = v[k];
                }
            }
        }
        // whether the caller's state already holds the clamp values in the input slice of given
        // cells (the usual case; otherwise the first step's updates take them from the clamp)
        const int N2 = a.c_in * HWn;
        int need = 0;
        for (int e0 = tid; e0 < N2; e0 += NT * kB) {
            unsigned xv[kB], cv[kB];
            unsigned char gv[kB];
#pragma unroll
            for (int k = 0; k < kB; ++k) {
                const int e = e0 + NT * k, ec = e < N2 ? e : N2 - 1;
                const int ci = ec / HWn, q = g_index(ec - ci * HWn);
                xv[k] = __float_as_uint(xr[(a.in_off + ci) * HWt + q]);
                cv[k] = __float_as_uint(a.clamp[(row * a.c_in + ci) * HWt + q]);
                gv[k] = a.given[row * HWt + q];
            }
#pragma unroll
            for (int k = 0; k < kB; ++k)
                if (e0 + NT * k < N2 && gv[k] && xv[k] != cv[k]) need = 1;
        }
        if (need) flagsL[1] = 1;
    }
    for (int c = tid; c < HWn + 16; c += NT) cinfo[c] = (unsigned short)m_index(c < HWn ? c : c - HWn);
    unsigned short *gidxL = reinterpret_cast<unsigned short *>(smem + sp.l_gidx);
    if (P > 1)
        for (int c = tid; c < HWn; c += NT) gidxL[c] = (unsigned short)g_index(c);
    for (int q = tid; q < HWn; q += NT)
        if (a.given[row * HWt + g_index(q)]) atomicOr(&givenL[q >> 5], 1u << (q & 31));
    for (int e = tid; e < (int)(sizeof(RolloutParams) / 4); e += NT)
        reinterpret_cast<unsigned *>(smem + sp.l_evp)[e] = reinterpret_cast<const unsigned *>(&a)[e];
    {
        const float *hw = reinterpret_cast<const float *>(a.packed + a.off_headw);
        const float *hb = reinterpret_cast<const float *>(a.packed + a.off_headb);
        const int nw = a.n_out * a.c_out;
        for (int e = tid; e < nw + a.n_out; e += NT) headL[e] = e < nw ? hw[e] : hb[e - nw];
    }
    __syncthreads();

    // ---- fire masks of step s for all cells (channel waves, thread tb of 256): the fire bit, or
    // for gated firing both threshold bits (the update decides between them)
    auto ring_put = [&](int s, int q, unsigned v) __attribute__((always_inline)) {
        const int o = (s % S::NSLOT) * HWn + q;
        ring[o] = (unsigned char)v;
        if (o < 16) ring[RING + o] = (unsigned char)v;
    };
    // the Philox draws go by the board's groups of 4 cells: those holding the workgroup's cells,
    // at most 256 (H W <= 1024, checked by the host), one per channel-wave thread, the update
    // waves' threads first (the stencil waves set the interval's pace). A thread's group, the
    // stream positions of its cells in the workgroup (or -1) and their given bits (bit 16) are
    // found once here, so a step's draw is one Philox evaluation and four ring stores.
    const int qlo = r0 * W, qhi = qlo + HWn;
    const int it0 = qlo >> 2, it1 = (qhi + 3) >> 2;
    const int dit = it0 + (255 - tb);  // this thread's group (channel waves; none if >= it1)
    int dq[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int qt = 4 * dit + e;  // board cell
        int v = -1;
        if (wave >= 4 && dit < it1 && qt >= qlo && qt < qhi) {
            const int tl = qt / W - r0, j = qt - (qt / W) * W;
            const int q = (down ? tl : Hs - 1 - tl) * W + j;  // its stream position
            v = q | (int)(((givenL[q >> 5] >> (q & 31)) & 1u) << 16);
        }
        dq[e] = v;
    }
    const bool count_fired = a.fired_out != nullptr && !a.adaptive;
    // per-step keys for the draws of steps 2, 3, ..: slot s & 1, written 4 intervals after the
    // previous draw by one stencil lane (so no draw waits for a global load)
    uint64_t *keyL = reinterpret_cast<uint64_t *>(flagsL + 2);
    auto draw = [&](const RolloutParams &pa, int s, uint64_t key) __attribute__((always_inline)) {
        unsigned fired = 0;
        if (dit < it1) {
            float u[4] = {1.0f, 1.0f, 1.0f, 1.0f};
            if (!pa.fire_u8)
                cell_uniforms4(key, (uint32_t)(pa.row0 + row), (uint32_t)(pa.step0 + s), (uint32_t)dit, u);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                if (dq[e] < 0) continue;
                const int q = dq[e] & 0xffff;
                unsigned b;
                if (pa.fire_u8) {
                    b = pa.fire_u8[((int64_t)s * pa.rows + row) * HWt + 4 * dit + e] != 0;
                } else {
                    const unsigned b0 = u[e] < pa.p, b1 = u[e] < pa.p_low;
                    b = pa.adaptive ? (b0 | (b1 << 1)) : b0;
                }
                ring_put(s, q, b | ((unsigned)(dq[e] >> 16) << 7));
                fired += b & 1u;
            }
        }
        if (count_fired) {
            // the wave's fired cells from the bits of the lanes' counts (0 .. 4)
            const int tot = __popcll(__ballot(fired & 1u)) + 2 * __popcll(__ballot(fired & 2u)) +
                            4 * __popcll(__ballot(fired & 4u));
            if (lane == 0 && tot) atomicAdd(&flagsL[0], tot);
        }
    };
    if (wave >= 4 && a.n_steps > 0) {
        draw(a, 0, a.step_seeds ? a.step_seeds[0] : a.seed);
        if (a.n_steps > 1) draw(a, 1, a.step_seeds ? a.step_seeds[1] : a.seed);
    }
    if (tid == 256 && a.step_seeds && a.n_steps > 2) keyL[0] = a.step_seeds[2];
    __syncthreads();

    using F_ = std::integral_constant<bool, false>;
    using T_ = std::integral_constant<bool, true>;
    using P0 = std::integral_constant<unsigned, 0>;
    using P1 = std::integral_constant<unsigned, 1>;
    const int T = P > 1 ? (int)(((int64_t)a.n_steps * HWn + 15) >> 4) : sp.T;
    const int total = a.n_steps * HWn;
    // a piece's neighbours: on the side of its first stream row (the row above for an even
    // piece, below for an odd one) and on the side of its last
    const bool has_first = P > 1 && (down ? piece > 0 : piece < P - 1);
    const bool has_last = P > 1 && (down ? piece < P - 1 : piece > 0);
    const int g = lane >> 4, n = lane & 15;
    const int ws = wave & 3;

    if (T > 0 && wave < 4) {
        // ================= hidden waves: fc1, epilogue, fc2 partial sums
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
                for (int kt = 0; kt < S::KT1; ++kt) w1f[mt][kt] = w1[((ws * S::MT1 + mt) * S::KT1 + kt) * 64 + lane];
#pragma unroll
                for (int v = 0; v < 4; ++v) b1v[mt][v] = b1[ws * 64 + 16 * mt + 4 * g + v];
            }
#pragma unroll
            for (int m2 = 0; m2 < S::MT2; ++m2)
#pragma unroll
                for (int kt = 0; kt < S::KT2; ++kt) w2f[m2][kt] = w2[((ws * S::MT2 + m2) * S::KT2 + kt) * 64 + lane];
#pragma unroll
            for (int mt = 0; mt < S::MT1; ++mt)
#pragma unroll
                for (int kt = 0; kt < S::KT1; ++kt) asm volatile("" : "+a"(w1f[mt][kt]));
#pragma unroll
            for (int m2 = 0; m2 < S::MT2; ++m2)
#pragma unroll
                for (int kt = 0; kt < S::KT2; ++kt) asm volatile("" : "+a"(w2f[m2][kt]));
        }
        // B operand of k-tile kt: features 32 kt + 8 g .. +7 of cell n = chunk 4 kt + g of Z row n
        unsigned kZ[S::KT1];
#pragma unroll
        for (int kt = 0; kt < S::KT1; ++kt)
            kZ[kt] = sp.l_Z + (unsigned)n * S::ZS + 16u * ((unsigned)(4 * kt + g) ^ zsw((unsigned)n));
        // partial sums of channels 16 m2 + 4 g .. +3 of cell n: chunk 4 m2 + g of this wave's D row n
        unsigned kD[S::MT2];
#pragma unroll
        for (int m2 = 0; m2 < S::MT2; ++m2)
            kD[m2] = sp.l_D + (unsigned)ws * S::DPART + (unsigned)n * S::DS +
                     16u * ((unsigned)(4 * m2 + g) ^ ((unsigned)(n >> 1) & 7u));
        // Z operands: tile i-1's are loaded at the start of interval i into zqb[i & 1] (they are
        // in flight during fc1 of tile i-2, which reads zqb[(i-1) & 1])
        bf16x8 zqb[2][S::KT1];
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int k = 0; k < S::KT1; ++k)
#pragma unroll
                for (int e = 0; e < 8; ++e) zqb[b][k][e] = (__bf16)0.0f;
        // fcb: fc1 of tile i-2, its epilogue in registers, fc2 over the wave's 64 hidden units
        // with those registers as B operand (the W2 fragments are packed in that k order) ->
        // D[i & 1]; fca: the Z operands of tile i-1
        auto hinterval = [&](auto fca_c, auto fcb_c, auto par_c) __attribute__((always_inline)) {
            constexpr bool FCA = decltype(fca_c)::value, FCB = decltype(fcb_c)::value;
            constexpr unsigned PAR = decltype(par_c)::value;
            auto load_z = [&]() __attribute__((always_inline)) {
                if (FCA) {
#pragma unroll
                    for (int kt = 0; kt < S::KT1; ++kt)
                        zqb[PAR][kt] = *reinterpret_cast<const bf16x8 *>(smem + kZ[kt] + (PAR ^ 1u) * S::ZBUF);
                }
            };
            load_z();
            if (FCB) {
                f32x4 acc[S::MT1];
#pragma unroll
                for (int mt = 0; mt < S::MT1; ++mt) {
                    acc[mt] = b1v[mt];
#pragma unroll
                    for (int kt = 0; kt < S::KT1; ++kt)
                        acc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(w1f[mt][kt], zqb[PAR ^ 1u][kt], acc[mt], 0,
                                                                          0, 0);
                }
                bf16x8 hf[S::KT2];
#pragma unroll
                for (int kt = 0; kt < S::KT2; ++kt) {
                    uint4 hv;
                    hv.x = relu_bf16x2(cvt_pk_bf16(acc[2 * kt][0], acc[2 * kt][1]));
                    hv.y = relu_bf16x2(cvt_pk_bf16(acc[2 * kt][2], acc[2 * kt][3]));
                    hv.z = relu_bf16x2(cvt_pk_bf16(acc[2 * kt + 1][0], acc[2 * kt + 1][1]));
                    hv.w = relu_bf16x2(cvt_pk_bf16(acc[2 * kt + 1][2], acc[2 * kt + 1][3]));
                    hf[kt] = __builtin_bit_cast(bf16x8, hv);
                }
#pragma unroll
                for (int m2 = 0; m2 < S::MT2; ++m2) {
                    f32x4 acc2 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int kt = 0; kt < S::KT2; ++kt)
                        acc2 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(w2f[m2][kt], hf[kt], acc2, 0, 0, 0);
                    lds_st128f(smem, kD[m2] + PAR * S::DBUF, make_float4(acc2[0], acc2[1], acc2[2], acc2[3]));
                }
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
        // drain: intervals T, T+1 (T+2 has no hidden work)
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
        // ================= channel waves: stencil (waves 4, 5) or update (waves 6, 7), and the
        // per-step draws
        __builtin_amdgcn_s_setprio(3);  // issue priority over the hidden waves' MFMAs
        const bool stencil_wave = wave < 6;
        const int cw = wave & 1;
        const int cl = 8 * cw + (lane >> 3);  // cell of the tile
        const int q8 = lane & 7;              // channel quad
        int i = 0;
        // the per-step draws: when the update stage enters step sd, step sd + 2 is drawn (its
        // ring slot was last read by the updates of step sd - 2)
        int sd = 0, ev_draw = 3;
        int kput = -1;  // stencil lane 0 of wave 4: the interval that stores knext into keyL
        uint64_t knext = 0;
        auto events = [&]() __attribute__((always_inline)) {
            if (i == ev_draw) {
                const RolloutParams &ea = *reinterpret_cast<const RolloutParams *>(smem + sp.l_evp);
                if (sd + 2 < ea.n_steps) draw(ea, sd + 2, ea.step_seeds ? keyL[sd & 1] : ea.seed);
                if (tb == 0 && ea.step_seeds && sd + 3 < ea.n_steps) {
                    knext = ea.step_seeds[sd + 3];  // the next draw's key, (sd + 3) & 1 = (sd + 1) & 1
                    kput = i + 4;
                }
                ++sd;
                ev_draw = ((sd * HWn) >> 4) + 3;
            }
            if (i == kput) {
                keyL[sd & 1] = knext;
                kput = -1;
            }
        };
        // gated firing: the update lanes decide a cell's mask for the step from its state at the
        // step's start (the output quad of M before the update, read by all 8 lanes of the cell:
        // 8 cycles, cheaper than one lane's decision handed on by a ballot); the head (at most 4
        // outputs over at most 4 channels) is held in registers
        const int oqi = a.out_off >> 2;
        const bool oq = GATED && q8 == oqi;
        float hw4[4][4], hb4[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            hb4[v] = v < a.n_out ? headL[a.n_out * a.c_out + v] : 0.0f;
#pragma unroll
            for (int c = 0; c < 4; ++c) hw4[v][c] = (v < a.n_out && c < a.c_out) ? headL[v * a.c_out + c] : 0.0f;
        }
        const float tau = a.tau, conf_d = sp.conf_d;
        const bool gconf = a.given_confident != 0, fast = sp.fast_conf != 0;
        // the fire bit from a cell's drawn byte and its state's out-slice channels xo
        auto gated_fire = [&](const float xo[4], unsigned byte) -> bool {
            bool hi;
            if (fast) {
                // two logits in cell_readout_fn's order; s = exp(l0 - m) + exp(l1 - m) where the
                // larger term is exactly 1, so s < conf_s is a test on the gap alone
                float l0 = hb4[0], l1 = hb4[1];
#pragma unroll
                for (int c = 0; c < 4; ++c)
                    if (c < a.c_out) {
                        l0 = __builtin_fmaf(hw4[0][c], xo[c], l0);
                        l1 = __builtin_fmaf(hw4[1][c], xo[c], l1);
                    }
                const float best = l1 > l0 ? l1 : l0;
                hi = (l1 > l0 ? l0 : l1) - best <= conf_d;
            } else {
                hi = cell_readout4(xo, a.c_out, a.n_out, a.head_kind, hw4, hb4) > tau;
            }
            const bool lo = hi || (gconf && (byte & 0x80u));
            return ((lo ? byte >> 1 : byte) & 1u) != 0;
        };
        int fired_dec = 0;  // this lane's fired decisions (gated firing), added up at the end
        if (stencil_wave) {
            // B operands: column j = lane % 4 is kernel j; taps 0-3, 4-7; tap 8 at the k slot of
            // channel c (the A operand of tap 8 is the 4 channels' tap-8 values)
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
            // output lane (block b, kernel j) holds rows r = quads 4 (b & 1) + r of cell 8 cw + b / 2
            unsigned kZw[4];
            {
                const unsigned b = (unsigned)lane >> 2, j = (unsigned)lane & 3u, r0 = 8u * cw + (b >> 1);
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const unsigned chunk = 2u * (4u * (b & 1u) + (unsigned)r) + (j >> 1);
                    kZw[r] = sp.l_Z + r0 * S::ZS + 16u * (chunk ^ zsw(r0)) + 8u * (j & 1u);
                }
            }
            const unsigned RPb = (unsigned)(W + 1) * S::MS;
            // top-left tap of M cell x: x - (W + 2)
            const unsigned kT = sp.l_M + 16u * (unsigned)q8 - (unsigned)(W + 2) * S::MS;
            int cbS = 0;  // board cell of tile i's first position: (16 i) mod HW
            // the taps of tile i are in tb[i & 1], loaded at the start of interval i-1 (tile 0's
            // before interval 0); xs1: M cell of the lane's cell in tile i+1
            float4 tb[2][9];
            auto load_taps = [&](float4(&t)[9], unsigned x) __attribute__((always_inline)) {
                const unsigned r0 = kT + x * S::MS, r1 = r0 + RPb, r2 = r1 + RPb;
                t[0] = lds_ld128f(smem, r0);
                t[1] = lds_ld128f(smem, r0 + S::MS);
                t[2] = lds_ld128f(smem, r0 + 2 * S::MS);
                t[3] = lds_ld128f(smem, r1);
                t[4] = lds_ld128f(smem, r1 + S::MS);
                t[5] = lds_ld128f(smem, r1 + 2 * S::MS);
                t[6] = lds_ld128f(smem, r2);
                t[7] = lds_ld128f(smem, r2 + S::MS);
                t[8] = lds_ld128f(smem, r2 + 2 * S::MS);
            };
            load_taps(tb[0], cinfo[cl]);
            unsigned xs1 = cinfo[16 + cl], xs2 = 0;  // HW >= 32
            auto sinterval = [&](auto par_c) __attribute__((always_inline)) {
                constexpr unsigned PAR = decltype(par_c)::value;
                // the next tile's taps (read after this interval's barrier-separated updates; the
                // last interval's read tile T, whose cells exist but are unused)
                load_taps(tb[PAR ^ 1u], xs1);
                {
                    int c2 = cbS + 32;
                    if (c2 >= HWn) c2 -= HWn;
                    xs2 = cinfo[c2 + cl];
                }
                const float4(&t)[9] = tb[PAR];
                // bf16 taps in operand order: channel c, taps 0-3 / 4-7; tap 8 of the 4 channels
                s16x4 sa0[4], sa1[4];
                auto ch = [&](const float4 &v, int c) -> float { return c == 0 ? v.x : c == 1 ? v.y : c == 2 ? v.z : v.w; };
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    sa0[c] = __builtin_bit_cast(s16x4, make_uint2(cvt_pk_bf16(ch(t[0], c), ch(t[1], c)),
                                                                  cvt_pk_bf16(ch(t[2], c), ch(t[3], c))));
                    sa1[c] = __builtin_bit_cast(s16x4, make_uint2(cvt_pk_bf16(ch(t[4], c), ch(t[5], c)),
                                                                  cvt_pk_bf16(ch(t[6], c), ch(t[7], c))));
                }
                const s16x4 a2 =
                    __builtin_bit_cast(s16x4, make_uint2(cvt_pk_bf16(t[8].x, t[8].y), cvt_pk_bf16(t[8].z, t[8].w)));
                f32x4 zc[4];
#pragma unroll
                for (int c0 = 0; c0 < 4; c0 += 2) {
                    f32x4 d0 = {0.f, 0.f, 0.f, 0.f}, d1 = d0;
                    d0 = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(sa0[c0], kb0, d0, 0, 0, 0);
                    d1 = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(sa0[c0 + 1], kb0, d1, 0, 0, 0);
                    d0 = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(sa1[c0], kb1, d0, 0, 0, 0);
                    d1 = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(sa1[c0 + 1], kb1, d1, 0, 0, 0);
                    d0 = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(a2, kb2[c0], d0, 0, 0, 0);
                    d1 = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(a2, kb2[c0 + 1], d1, 0, 0, 0);
                    zc[c0] = d0;
                    zc[c0 + 1] = d1;
                }
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    uint2 o;
                    o.x = cvt_pk_bf16(zc[0][r], zc[1][r]);
                    o.y = cvt_pk_bf16(zc[2][r], zc[3][r]);
                    lds_st64(smem, kZw[r] + PAR * S::ZBUF, o);
                }
            };
            auto advance = [&]() __attribute__((always_inline)) {
                ++i;
                cbS += 16;
                if (cbS >= HWn) cbS -= HWn;
                xs1 = xs2;
            };
            // pieces: M's halo rows hold the neighbours' rows of the state the stencil reads.
            // Refresh k (k = 0 .. n_steps - 1) brings the last side's row of state k and the first
            // side's row of state k + 1; its loads are issued in interval hB = (((k HW) >> 4) + 9)
            // rounded down to even, checked and stored in interval hB + 4. The last side's old
            // row (state k - 1) was
            // last read by taps loaded before interval (k HW) >> 4 and the new one is first read
            // by the taps of step k's last row, loaded from interval ((k HW + (Hs - 1) W) >> 4) - 1
            // >= hB + 5 ((Hs - 1) W >= 240, checked by the host); the first side's old row (state
            // k) by step k's first row, loaded before interval ((k HW) >> 4) + 2, the new one from
            // interval (((k + 1) HW) >> 4) - 1 >= hB + 5. A neighbour writes its last row of state
            // k in its step k - 1 and its first row of state k + 1 early in step k, intervals
            // before hB when the two run in step. A word whose tag is not yet that state's is
            // read again; after sp.spin_limit reads (kHaloSpin, about a second, in use) the halo
            // takes NaN (which reaches every result), *sp.halo_status is set, no later refresh
            // of the thread waits, and the kernel still ends; the host's repair launch then
            // recomputes the boards whole (a wait runs out only when the pieces of a board are
            // not resident together).
            const int th = tid - 256;  // 0 .. 127 over the stencil waves
            const int NE = W * S::C;
            const int nf = down ? piece - 1 : piece + 1, nl = down ? piece + 1 : piece - 1;
            const int mrow_f = down ? 0 : Hs + 1, mrow_l = down ? Hs + 1 : 0;
            int hk = 0, hB = 8;  // refresh hk's block starts at interval hB (even)
            bool hfail = false;  // a wait ran out: no later wait (the results are NaN already)
            auto xslot = [&](int side, int nb, int st) -> const uint64_t * {
                return sp.xch + (((row * P + nb) * 2 + side) * 4 + (st & 3)) * (int64_t)NE;
            };
            // the 8 words of a thread are loaded together, unconditionally (a lane past the row
            // reads its last word and ignores it): a conditional load gets a wait of its own
            auto halo_load = [&](uint64_t(&hw)[8], int side, int nb, int st) __attribute__((always_inline)) {
                const uint64_t *src = xslot(side, nb, st);
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    const int e = th + 128 * k;
                    hw[k] = __hip_atomic_load(src + (e < NE ? e : NE - 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
            };
            auto halo_store = [&](uint64_t(&hw)[8], int side, int nb, int st, int mrow) __attribute__((always_inline)) {
                float *Mh = reinterpret_cast<float *>(smem + sp.l_M + (unsigned)(mrow * (W + 1) + 1) * S::MS);
                // while a word is not yet tagged st, the thread's words are read again together
                // (one round trip a try)
                const uint32_t want = (uint32_t)(st + sp.tag_skew);
                auto stale = [&](int k) { return th + 128 * k < NE && (uint32_t)(hw[k] >> 32) != want; };
                for (int n = 0; !hfail; ++n) {
                    bool any = false;
#pragma unroll
                    for (int k = 0; k < 8; ++k) any |= stale(k);
                    if (!any) break;
                    if (n >= sp.spin_limit) {
                        hfail = true;
                        __hip_atomic_fetch_or(sp.halo_status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        break;
                    }
                    __builtin_amdgcn_s_sleep(2);
                    halo_load(hw, side, nb, st);  // a word already tagged st keeps its value
                }
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    const int e = th + 128 * k;
                    if (e < NE) {
                        const uint64_t wd = hw[k];
                        Mh[e] = (uint32_t)(wd >> 32) == (uint32_t)st ? __uint_as_float((uint32_t)wd) : __builtin_nanf("");
                    }
                }
            };
            // a refresh runs as a block of six intervals from hB: the loads in the first, the
            // check and the stores in the fifth, so its words are not live in the other intervals
            auto halo_block = [&]() __attribute__((always_inline)) {
                const bool hl = has_last && hk >= 1, hf = has_first && hk + 1 < a.n_steps;
                uint64_t hwl[8], hwf[8];
                sinterval(P0{});
                events();
                if (hl) halo_load(hwl, 1, nl, hk);
                if (hf) halo_load(hwf, 0, nf, hk + 1);
                advance();
                __syncthreads();
                sinterval(P1{});
                events();
                advance();
                __syncthreads();
                sinterval(P0{});
                events();
                advance();
                __syncthreads();
                sinterval(P1{});
                events();
                advance();
                __syncthreads();
                sinterval(P0{});
                events();
                if (hl) halo_store(hwl, 1, nl, hk, mrow_l);
                if (hf) halo_store(hwf, 0, nf, hk + 1, mrow_f);
                advance();
                __syncthreads();
                sinterval(P1{});
                events();
                advance();
                __syncthreads();
                ++hk;
                hB = ((((hk * HWn) >> 4) + 9) & ~1);
            };
            i = 0;
            while (i + 1 < T) {
                if (P > 1 && i == hB && hk < a.n_steps) {  // i is even here
                    halo_block();
                    continue;
                }
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
            f32x4 b2v;
            {
                const float *b2 = reinterpret_cast<const float *>(a.packed + a.off_b2);
#pragma unroll
                for (int v = 0; v < 4; ++v) b2v[v] = b2[4 * q8 + v];
                // complete before the loop: a load still pending where the loop starts makes every
                // interval wait for all vector memory operations (the state stores included)
                asm volatile("" ::"v"(b2v));
            }
            // all ones where the lane's channel 4 q8 + v lies in the clamped input slice
            unsigned imv[4];
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int c = 4 * q8 + v;
                imv[v] = (c >= a.in_off && c < a.in_off + a.c_in) ? 0xffffffffu : 0u;
                asm volatile("" : "+v"(imv[v]));
            }
            const bool need0 = flagsL[1] != 0;
            const unsigned kDr = sp.l_D + (unsigned)cl * S::DS + 16u * ((unsigned)q8 ^ ((unsigned)(cl >> 1) & 7u));
            const unsigned kM = sp.l_M + 16u * (unsigned)q8;
            int cbU = HWn - 48;   // board cell of the update tile's first position: 16 (i-3) mod HW
            int rbU = RING - 48;  // its ring slot: 16 (i-3) mod RING
            int usU = -1;         // its step
            unsigned xu = 0, xu_n = 0;
            auto uinterval = [&](auto up_c, auto last_c) __attribute__((always_inline)) {
                constexpr bool DUP = decltype(up_c)::value, LAST = decltype(last_c)::value;
                const unsigned PAR = (unsigned)(i & 1);
                {
                    int cu = cbU + 16;
                    if (cu >= HWn) cu -= HWn;
                    xu_n = cinfo[cu + cl];
                }
                if (!DUP) return;
                // the state loads first: with gated firing the decision is made while the partial
                // sums are in flight
                const unsigned madr = kM + xu * S::MS;
                const float4 m4 = lds_ld128f(smem, madr);
                const unsigned fb = ring[rbU + cl];
                float4 mo4;
                if (GATED) mo4 = lds_ld128f(smem, madr + 16u * (unsigned)(oqi - q8));  // the output quad
                float4 pd[4];
#pragma unroll
                for (int p = 0; p < 4; ++p) pd[p] = lds_ld128f(smem, kDr + (PAR ^ 1u) * S::DBUF + (unsigned)p * S::DPART);
                // the cell's step, stream position and board cell
                const bool nxt = cbU + cl >= HWn;
                const int sc = usU + (nxt ? 1 : 0);
                const int qc = cbU + cl - (nxt ? HWn : 0);
                const int qg = P > 1 ? (int)gidxL[qc] : qc;
                unsigned fbit = fb & 1u;
                if (GATED) {
                    // the output-quad lane's decision (its m4 is the output quad) to all 8 lanes
                    const float xq[4] = {mo4.x, mo4.y, mo4.z, mo4.w};
                    const unsigned f = gated_fire(xq, fb) ? 1u : 0u;
                    fbit = f;
                    if (oq && (!LAST || 16 * (i - 3) + cl < total)) fired_dec += (int)f;
                }
                float ds[4];
#pragma unroll
                for (int v = 0; v < 4; ++v) ds[v] = (((b2v[v] + pd[0][v]) + pd[1][v]) + pd[2][v]) + pd[3][v];
                const uint32_t d01 = cvt_pk_bf16(ds[0], ds[1]), d23 = cvt_pk_bf16(ds[2], ds[3]);
                const float dx[4] = {bf16_lo(d01), bf16_hi(d01), bf16_lo(d23), bf16_hi(d23)};
                float xo[4] = {m4.x, m4.y, m4.z, m4.w};
                const float fu = (float)fbit;
                const unsigned gvm = (fb & 0x80u) ? 0xffffffffu : 0u;
                float xk[4] = {xo[0], xo[1], xo[2], xo[3]};
                if (need0 && usU <= 0) {
                    // first step, caller's state not clamped: the kept channels take the clamp values
                    if (sc == 0 && gvm) {
#pragma unroll
                        for (int v = 0; v < 4; ++v)
                            if (imv[v])
                                xk[v] = a.clamp[(row * a.c_in + (4 * q8 + v - a.in_off)) * HWt + qg];
                        // the loads complete here, in this rare branch: a wait where the paths
                        // meet would also wait for every interval's state stores
#pragma unroll
                        for (int v = 0; v < 4; ++v) asm volatile("" ::"v"(xk[v]));
                    }
                }
                float u[4];
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const float uv = __builtin_fmaf(fu, dx[v], xo[v]);  // fu in {0, 1}: exact
                    const unsigned km = imv[v] & gvm;                     // clamped: keep x
                    u[v] = __uint_as_float((km & __float_as_uint(xk[v])) | (~km & __float_as_uint(uv)));
                }
                bool ok = true;
                if (LAST) ok = 16 * (i - 3) + cl < total;
                if (ok) {
                    lds_st128f(smem, madr, make_float4(u[0], u[1], u[2], u[3]));
                    if (REC) {  // every step's state, for the BPTT chunk
                        float *xr = a.x_rec + (int64_t)sc * a.rec_stride + ((int64_t)row * S::C + 4 * q8) * HWt + qg;
#pragma unroll
                        for (int v = 0; v < 4; ++v) xr[(int64_t)v * HWt] = u[v];
                        if (P > 1) {
                            // a piece's first and last stream rows go to the exchange slots of
                            // state sc + 1, tagged with it (single-copy atomic 8-byte words, so a
                            // reader sees a value with its own step's tag)
                            int side = -1, j = 0;
                            if (qc < W && has_first) {
                                side = 0;
                                j = qc;
                            } else if (qc >= HWn - W && has_last) {
                                side = 1;
                                j = qc - (HWn - W);
                            }
                            if (side >= 0) {
                                uint64_t *xo = sp.xch + ((((row * P + piece) * 2 + side) * 4 + ((sc + 1) & 3)) * W + j) * 32 + 4 * q8;
                                const uint64_t tag = (uint64_t)(uint32_t)(sc + 1) << 32;
#pragma unroll
                                for (int v = 0; v < 4; ++v)
                                    __hip_atomic_store(xo + v, tag | __float_as_uint(u[v]), __ATOMIC_RELAXED,
                                                       __HIP_MEMORY_SCOPE_AGENT);
                            }
                        }
                    }
                }
            };
            auto advance = [&]() __attribute__((always_inline)) {
                ++i;
                cbU += 16;
                if (cbU >= HWn) {
                    cbU -= HWn;
                    ++usU;
                }
                rbU += 16;
                if (rbU >= RING) rbU -= RING;
                xu = xu_n;
            };
            i = 0;
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
            if (GATED) {
#pragma unroll
                for (int o = 32; o >= 1; o >>= 1) fired_dec += __shfl_xor(fired_dec, o);
                if (lane == 0 && fired_dec) atomicAdd(&flagsL[0], fired_dec);
            }
        }
    }
    __syncthreads();

    // ---- write back (LDS reads in batches of 8 ahead of their stores)
    {
        constexpr int kB = 8;
        float *xr = a.x_out + row * S::C * HWt;
        const int N = S::C * HWn;
        for (int e0 = tid; e0 < N; e0 += NT * kB) {
            float v[kB];
            int o[kB];
#pragma unroll
            for (int k = 0; k < kB; ++k) {
                const int e = e0 + NT * k, ec = e < N ? e : N - 1;
                const int ch = ec / HWn, q = ec - ch * HWn;
                v[k] = m_at(q, ch);
                o[k] = P > 1 ? ch * HWt + g_index(q) : ec;
            }
#pragma unroll
            for (int k = 0; k < kB; ++k)
                if (e0 + NT * k < N) xr[o[k]] = v[k];
        }
    }
    if (a.conf_out) {
        float *confL = reinterpret_cast<float *>(smem + sp.l_Z);  // Z and D are free now
        for (int q = tid; q < HWn; q += NT) {
            int am;
            confL[q] = cell_readout_fn([&](int v) { return m_at(q, a.out_off + v); }, a.c_out, a.n_out, a.head_kind,
                                       headL, headL + a.n_out * a.c_out, &am);
        }
        __syncthreads();
        if (tid == 0) {
            float sum = 0.0f;
            for (int q = 0; q < HWn; ++q) sum = __fadd_rn(sum, confL[q]);
            a.conf_out[row] = __fdiv_rn(sum, (float)HWn);
        }
    }
    if (a.fired_out && tid == 0) a.fired_out[row] = flagsL[0];
}

}  // namespace nca
