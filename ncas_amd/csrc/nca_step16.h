// Per-step kernel for bf16 cells with C = 16 channels and 128 hidden units on grids of any size
// (gfx950): one NCA step of every row, x_in -> x_out, each wave on its own 16-cell tiles.
//
// A tile is 16 consecutive cells q0 .. q0 + 15 of one row in raster order. Lane (r = lane & 15,
// g = lane >> 4) owns cell q0 + r, channel quad g, for the whole tile:
//   1. its 9 taps: the 16-byte quad g of the 3x3 neighbours (cell-major state), or the padding
//      value for a neighbour outside the grid (wall: pad_vec, zero: 0, wrap: the wrapped cell;
//      reference src/nca/model.py:140-152), with the cell's given flag, injected mask and clamp
//      values, all loaded for the next tile while this one computes (vmcnt counts in order, so a
//      tile's own loads must all be older than the next tile's);
//   2. the 3x3 perception of its 4 channels on v_mfma_f32_4x4x4_16b_bf16 over tap pairs (the taps
//      rounded to bf16 like the forward's perception buffer; one pair per MFMA, which sums
//      exactly as the other kernels' v_dot2 chains do) -> z, through a wave-private LDS block to
//      the fc1 operand layout;
//   3. fc1 on v_mfma_f32_16x16x32_bf16 (W1 fragments in registers, b1 from LDS as the initial
//      accumulators), ReLU and bf16 rounding, through the wave's LDS block to fc2's operand
//      layout (hidden units in natural order, so every sum runs in the same order as in the
//      halo-window and resident kernels and the results are theirs bit for bit);
//   4. fc2: D[channel 4g + i][cell r] = the lane's own quad, so the residual update, the fire
//      mask (Philox keyed on (seed; row, step, cell quad) like every kernel, or an injected
//      mask) and the clamp (the input slice of given cells keeps its value; the first step of a
//      call takes the clamp tensor's) need no other lane.
// No workgroup barrier: a workgroup's waves share only the b1 vector in LDS. Workgroup b takes a
// contiguous range of tiles (so most neighbour rows are in its XCD's L2); its waves interleave.
// The first step of a call may read the caller's NCHW state and the last may write it
// (IN_NCHW / OUT_NCHW); the steps between use the cell-major state (rows, H, W, C).
#pragma once

#include "nca_stream_util.h"

namespace nca {

struct Step16Params {
    RolloutParams a;  // x_in -> x_out of this step
    int step;         // step index within the call (Philox counter step0 + step, mask slice)
    int first;        // first step of a call: the clamp tensor's values for the clamped channels
    int64_t n_tiles;  // rows * tiles_per_row
    int tiles_per_row;
    int64_t tiles_per_wg;
};

typedef float s16_f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// FIRST equals sp.first: the clamp values are loaded (and the loop carries them) on a call's
// first step only
template <bool IN_NCHW, bool OUT_NCHW, bool FIRST>
__global__ void __launch_bounds__(512, 1) step_stream16(Step16Params sp) {
    constexpr int C = 16, HD = 128;
    const RolloutParams &a = sp.a;
    __shared__ float b1L[HD];
    // per wave: z (16 cells x 64 bf16, 144-byte rows) and h (16 cells x 128 bf16, 272-byte rows)
    __shared__ __attribute__((aligned(16))) unsigned char zL[8][16 * 144 + 16 * 272];
    const int tid = threadIdx.x, lane = tid & 63, r = lane & 15, g = lane >> 4;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int H = a.H, W = a.W, HWn = H * W;

    // ---- constants: stencil B operands, W1 / W2 fragments, biases
    // The stencil runs on v_mfma_f32_4x4x4_16b_bf16: block b = lane / 4 multiplies 4 cells' tap
    // pairs (A rows) by the 4 kernels (B columns, kernel j = lane & 3). Each MFMA adds one tap pair
    // to the accumulator: the B operand holds kernel j's pair in k slots 0-1 or 2-3 and zeros in
    // the others, so the A operand can be two adjacent packed pairs of the lane's channel as they
    // are. One pair of products plus the accumulator rounds exactly like v_dot2_f32_bf16 (checked
    // bit for bit on 16.8M operand sets, the zeros in either half, unit and tiny magnitudes), so
    // the five MFMAs per channel give the v_dot2 chain's sums of the other kernels bit for bit.
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
    bf16x8 w1f[8][2];  // [m-tile][k-tile]: W1[16 mt + r][32 kt + 8g + j]
#pragma unroll
    for (int mt = 0; mt < 8; ++mt)
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
            w1f[mt][kt] = reinterpret_cast<const bf16x8 *>(a.packed + a.off_w1)[((size_t)mt * 2 + kt) * 64 + lane];
    bf16x8 w2f[4];  // [k-tile]: W2[r][32 kt + 8g + j]
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) w2f[kt] = reinterpret_cast<const bf16x8 *>(a.packed + a.off_w2)[(size_t)kt * 64 + lane];
    const float *b1 = reinterpret_cast<const float *>(a.packed + a.off_b1);
    const float *b2 = reinterpret_cast<const float *>(a.packed + a.off_b2);
    if (tid < HD) b1L[tid] = b1[tid];
    float b2v[4];
    bool insl[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        b2v[v] = b2[4 * g + v];
        insl[v] = 4 * g + v >= a.in_off && 4 * g + v < a.in_off + a.c_in;
    }
    const float4 pq = a.padding == 1 ? reinterpret_cast<const float4 *>(a.packed + a.off_padv)[g]
                                     : float4{0.f, 0.f, 0.f, 0.f};
    const uint64_t key = a.step_seeds ? a.step_seeds[sp.step] : a.seed;
    __syncthreads();

    // ---- this wave's tiles: t = t0 + w, t0 + w + 8, ... within the workgroup's range
    const int64_t t_begin = (int64_t)blockIdx.x * sp.tiles_per_wg;
    int64_t t_end = t_begin + sp.tiles_per_wg;
    if (t_end > sp.n_tiles) t_end = sp.n_tiles;
    unsigned char *zw = zL[w];
    unsigned char *hw = zL[w] + 16 * 144;
    // the cell-major output state (below 2^31 bytes, checked by the host); the third dword is
    // gfx9's format word
    const __amdgpu_buffer_rsrc_t out_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        a.x_out, (short)0, OUT_NCHW ? 0 : (int)(a.rows * HWn * C * (int64_t)sizeof(float)), 0x00020000);

    // everything tile t loads: taps (float4 per tap), given flag, injected mask, clamp values
    struct TileIn {
        float4 tp[9];  // raw loads; halo taps are replaced by the padding value when packed
        float fin;     // the injected float mask's value
        float cv[4];
        int gv, fu8;  // raw bytes (converting them here would wait for their loads)
        int padm;     // bit tt: tap tt is a constant halo cell (wall / zero padding)
    };
    const bool wrap = a.padding == 2;
    // the tile at (row, tile tir of the row): cells q0 = 16 tir .. q0 + 15
    auto load_tile = [&](int64_t row, int tir, TileIn &in) {
        const int q0 = 16 * tir, q = q0 + r;
        const int i0 = q0 / W, j0 = q0 - i0 * W;  // uniform
        int i, j;
        if (q >= HWn) {
            i = H - 1;
            j = W - 1;
        } else if (W >= 16) {  // at most one row boundary within the tile
            const int jj = j0 + r;
            const bool nx = jj >= W;
            i = i0 + (nx ? 1 : 0);
            j = jj - (nx ? W : 0);
        } else {
            i = q / W;
            j = q - i * W;
        }
        const int qc = i * W + j;
        // neighbour offsets in cells by row (dy) and column (dx), wrapped at the grid's edge (for
        // wall / zero padding the wrapped cell is loaded and replaced), and the halo flags
        const int ro[3] = {i > 0 ? -W : (H - 1) * W, 0, i < H - 1 ? W : -(H - 1) * W};
        const int co[3] = {j > 0 ? -1 : W - 1, 0, j < W - 1 ? 1 : -(W - 1)};
        // halo taps: the top row of taps (bits 0-2), the bottom (6-8), the left column (0, 3, 6),
        // the right (2, 5, 8)
        in.padm = wrap ? 0
                       : ((i == 0 ? 0x007 : 0) | (i == H - 1 ? 0x1c0 : 0) | (j == 0 ? 0x049 : 0) |
                          (j == W - 1 ? 0x124 : 0));
#pragma unroll
        for (int tt = 0; tt < 9; ++tt) {
            const int dy = tt / 3, dx = tt % 3;
            if (IN_NCHW) {
                const float *xr = a.x_in + (row * C + 4 * g) * (int64_t)HWn + qc + ro[dy] + co[dx];
                in.tp[tt] = float4{xr[0], xr[HWn], xr[2 * HWn], xr[3 * HWn]};
            } else {
                // byte offset from the state's base, below 2^32 (checked by the host)
                const uint32_t off = ((uint32_t)(row * HWn) + (uint32_t)(qc + ro[dy] + co[dx])) * (uint32_t)(4 * C) +
                                     16u * (uint32_t)g;
                in.tp[tt] = *reinterpret_cast<const float4 *>(reinterpret_cast<const unsigned char *>(a.x_in) + off);
            }
        }
        in.gv = a.given[row * HWn + qc];
        // the injected masks are loaded without a branch (a mask that is absent loads some other
        // element of the row instead, unused): a memory access under a branch leaves the compiler
        // unsure how many are in flight, and it then waits for all of them, the tile's store
        // included, before the next tile
        const float *fsrc = a.fire_f32 ? a.fire_f32 + (row * HWn + qc) : a.x_in + (row * HWn + qc);
        const unsigned char *usrc =
            a.fire_u8 ? a.fire_u8 + (((int64_t)sp.step * a.rows + row) * HWn + qc) : a.given + (row * HWn + qc);
        in.fin = *fsrc;
        in.fu8 = *usrc;
        if (FIRST) {
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int ci = insl[v] ? 4 * g + v - a.in_off : 0;
                in.cv[v] = a.c_in > 0 ? a.clamp[(row * a.c_in + ci) * (int64_t)HWn + qc] : 0.0f;
            }
        }
    };

    int64_t cur_row = -1;
    int fired_run = 0;  // fired cells of cur_row counted by this wave, not yet added
    auto flush_fired = [&]() {
        int s = fired_run;
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) s += __shfl_xor(s, o);
        if (lane == 0 && s && a.fired_out) atomicAdd(a.fired_out + cur_row, s);
        fired_run = 0;
    };

    // what the compute of a tile keeps of its loads: the taps as bf16 pairs of one channel (taps
    // 2p and 2p + 1, tap 8 with a zero; halo taps replaced by the padding value), the cell's fp32
    // quad, flags and mask / clamp values
    // the stencil's A operands of channel c: taps 0-3 and 4-7 as two bf16 pairs each, tap 8 with
    // a zero (pairs (t0, t1), (t2, t3) / (t4, t5), (t6, t7) / (t8, 0), 0)
    struct TileCur {
        u32x2 ta[4], tb[4], tc[4];
        float xo[4], fin, cv[4];
        int gv, fu8;
    };
    auto unpack = [&](const TileIn &in, TileCur &cu) __attribute__((always_inline)) {
        auto pack = [&](const float4 *tp) __attribute__((always_inline)) {
            const float *f[9];
#pragma unroll
            for (int tt = 0; tt < 9; ++tt) f[tt] = reinterpret_cast<const float *>(&tp[tt]);
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                cu.ta[c] = u32x2{pack_bf16x2(f[0][c], f[1][c]), pack_bf16x2(f[2][c], f[3][c])};
                cu.tb[c] = u32x2{pack_bf16x2(f[4][c], f[5][c]), pack_bf16x2(f[6][c], f[7][c])};
                cu.tc[c] = u32x2{pack_bf16x2(f[8][c], 0.0f), 0u};
            }
        };
        pack(in.tp);
        // tiles with a cell on the grid's edge pack again with the padding value in place of the
        // halo taps (a branch uniform over the wave; most tiles have none)
        if (__builtin_amdgcn_ballot_w64(in.padm != 0)) {
            float4 tp[9];
#pragma unroll
            for (int tt = 0; tt < 9; ++tt) tp[tt] = ((in.padm >> tt) & 1) ? pq : in.tp[tt];
            pack(tp);
        }
        cu.xo[0] = in.tp[4].x;
        cu.xo[1] = in.tp[4].y;
        cu.xo[2] = in.tp[4].z;
        cu.xo[3] = in.tp[4].w;
        cu.fin = in.fin;
        cu.gv = in.gv;
        cu.fu8 = in.fu8;
#pragma unroll
        for (int v = 0; v < 4; ++v) cu.cv[v] = in.cv[v];
    };
    // Philox fire bits of 16 tiles at a time: lane L evaluates cell quad L & 3 of the wave's tile
    // L >> 2 tiles ahead (tiles start at multiples of 16 cells; all four of an evaluation's
    // uniforms are used), and ballot e gives bit 4 k + j = cell 4 j + e of tile k
    uint64_t fb[4] = {0, 0, 0, 0};
    int kgrp = 0;
    const int tpr = sp.tiles_per_row;
    const int fbit = 4 * (r & 3) + (r >> 2);  // cell r's bit in a tile's 16-bit mask
    auto draw16 = [&](int64_t row, int tir) {
        int ti = tir + 8 * (lane >> 2);
        int64_t rw = row;
        while (ti >= tpr) {
            ti -= tpr;
            ++rw;
        }
        float u4[4];
        cell_uniforms4(key, (uint32_t)(a.row0 + rw), (uint32_t)(a.step0 + sp.step), (uint32_t)(4 * ti + (lane & 3)),
                       u4);
#pragma unroll
        for (int e = 0; e < 4; ++e) fb[e] = __ballot(u4[e] < a.p);
    };
    // one tile: the cells' new states to x_out
    auto process = [&](const TileCur &cur, int64_t row, int tir) __attribute__((always_inline)) {
        const int q = 16 * tir + r;
        const bool valid = q < HWn;

        // 2. perception: per channel of the lane's quad, five MFMAs over the tap pairs; lane
        // (r, g) receives z of kernel j = r & 3 for cells 4 (r >> 2) + i, channel 4 g + c
        {
            s16_f32x4 zc[4];
#pragma unroll
            for (int c = 0; c < 4; ++c) zc[c] = s16_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int p2 = 0; p2 < 5; ++p2)
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const u32x2 av = p2 < 2 ? cur.ta[c] : p2 < 4 ? cur.tb[c] : cur.tc[c];
                    zc[c] = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(__builtin_bit_cast(s16x4, av), kb[p2], zc[c], 0, 0,
                                                                   0);
                }
            const int j = r & 3, c0 = 4 * (r >> 2);
#pragma unroll
            for (int i = 0; i < 4; ++i)  // feature j C + 4g + c of cell c0 + i
                *reinterpret_cast<uint2 *>(zw + (c0 + i) * 144 + 2 * (j * C + 4 * g)) =
                    uint2{pack_bf16x2(zc[0][i], zc[1][i]), pack_bf16x2(zc[2][i], zc[3][i])};
        }
        // 3. fc1 (the LDS block is this wave's own: its writes above precede these reads, a
        // wave's LDS operations complete in order)
        __builtin_amdgcn_wave_barrier();
        const bf16x8 zf0 = *reinterpret_cast<const bf16x8 *>(zw + r * 144 + 16 * g);
        const bf16x8 zf1 = *reinterpret_cast<const bf16x8 *>(zw + r * 144 + 64 + 16 * g);
        s16_f32x4 h[8];
#pragma unroll
        for (int mt = 0; mt < 8; ++mt) {
            const float4 bq = *reinterpret_cast<const float4 *>(b1L + 16 * mt + 4 * g);
            h[mt] = s16_f32x4{bq.x, bq.y, bq.z, bq.w};
            h[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(w1f[mt][0], zf0, h[mt], 0, 0, 0);
            h[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(w1f[mt][1], zf1, h[mt], 0, 0, 0);
        }
        // 4. fc2 on the ReLU'd bf16 activations (hidden 16 mt + 4g + i of cell r to the wave's
        // LDS block, read back as 8 consecutive hidden units), then the update of this lane's quad
#pragma unroll
        for (int mt = 0; mt < 8; ++mt)  // bf16 rounding, then ReLU on the packed pairs
            *reinterpret_cast<uint2 *>(hw + r * 272 + 2 * (16 * mt + 4 * g)) =
                uint2{relu_bf16x2(cvt_pk_bf16(h[mt][0], h[mt][1])), relu_bf16x2(cvt_pk_bf16(h[mt][2], h[mt][3]))};
        __builtin_amdgcn_wave_barrier();
        s16_f32x4 dx = s16_f32x4{b2v[0], b2v[1], b2v[2], b2v[3]};
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) {
            const bf16x8 hf = *reinterpret_cast<const bf16x8 *>(hw + r * 272 + 2 * (32 * kt + 8 * g));
            dx = __builtin_amdgcn_mfma_f32_16x16x32_bf16(w2f[kt], hf, dx, 0, 0, 0);
        }
        float f;
        if (a.fire_f32) {
            f = cur.fin;
        } else if (a.fire_u8) {
            f = cur.fu8 ? 1.0f : 0.0f;
        } else {
            // tile kgrp's 16 bits, cell 4 j + e at bit 4 e + j (the same for every lane)
            uint32_t m16 = 0;
#pragma unroll
            for (int e = 0; e < 4; ++e) m16 |= (uint32_t)((fb[e] >> (4 * kgrp)) & 0xfull) << (4 * e);
            f = ((m16 >> fbit) & 1u) ? 1.0f : 0.0f;
        }
        const bool gv = cur.gv != 0;
        float xo[4] = {cur.xo[0], cur.xo[1], cur.xo[2], cur.xo[3]};
        if (FIRST && gv) {
#pragma unroll
            for (int v = 0; v < 4; ++v)
                if (insl[v]) xo[v] = cur.cv[v];
        }
        float u[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const float uv = __fadd_rn(xo[v], __fmul_rn(f, round_bf16(dx[v])));
            u[v] = (gv && insl[v]) ? xo[v] : uv;
        }
        if (OUT_NCHW) {
            if (valid) {
                float *xr = a.x_out + (row * C + 4 * g) * (int64_t)HWn + q;
#pragma unroll
                for (int v = 0; v < 4; ++v) xr[(int64_t)v * HWn] = u[v];
            }
        } else {
            // cells past the row's end store at an offset beyond the buffer, which the hardware
            // drops, so the store needs no branch
            const uint32_t off = valid ? ((uint32_t)(row * HWn + q) * (uint32_t)C + 4u * (uint32_t)g) * 4u : 0x80000000u;
            __builtin_amdgcn_raw_buffer_store_b128(u32x4{__float_as_uint(u[0]), __float_as_uint(u[1]),
                                                         __float_as_uint(u[2]), __float_as_uint(u[3])},
                                                   out_rsrc, off, 0, 0);
        }
        // fired cells, counted once per cell (quad 0) and added per row (the row's flush is at
        // the top of the tile, before its loads)
        if (a.fired_out) fired_run += (valid && g == 0 && f != 0.0f) ? 1 : 0;
    };

    // the wave's tiles t = t_begin + w + 8k, at (row, tile of the row) tracked without division;
    // two load buffers alternate so that the next tile's loads are in flight during this one
    int64_t t = t_begin + w;
    int64_t row = t / tpr;
    int tir = (int)(t - row * tpr);
    auto advance = [&](int64_t &rw, int &ti) {
        ti += 8;
        while (ti >= tpr) {
            ti -= tpr;
            ++rw;
        }
    };
    TileIn nx;
    if (t < t_end) load_tile(row, tir, nx);
    const bool philox = !a.fire_f32 && !a.fire_u8;
    // vmcnt(0) (expcnt and lgkmcnt left open): the weights' loads are done before the loop, so the
    // waits the compiler places at their uses in the loop body do not hold back the prefetch
    __builtin_amdgcn_s_waitcnt(0x0f70);
    for (; t < t_end; t += 8) {
        TileCur cu;
        unpack(nx, cu);  // this tile's loads, consumed before the buffer takes the next tile's
        // the unpacked values are materialised here, before the next tile's loads are issued:
        // left to sink to their uses (past the Philox branch) they keep the buffer's old values
        // alive across its new loads, and the compiler then carries the buffer in two register
        // sets copied at the end of every iteration (38 moves per tile)
#pragma unroll
        for (int c = 0; c < 4; ++c) asm volatile("" : "+v"(cu.ta[c]), "+v"(cu.tb[c]), "+v"(cu.tc[c]));
        asm volatile("" : "+v"(cu.xo[0]), "+v"(cu.xo[1]), "+v"(cu.xo[2]), "+v"(cu.xo[3]));
        asm volatile("" : "+v"(cu.fin), "+v"(cu.gv), "+v"(cu.fu8));
        if (FIRST) asm volatile("" : "+v"(cu.cv[0]), "+v"(cu.cv[1]), "+v"(cu.cv[2]), "+v"(cu.cv[3]));
        asm volatile("" ::: "memory");
        if (a.fired_out && row != cur_row) {
            if (cur_row >= 0) flush_fired();
            cur_row = row;
        }
        int64_t rn = row;
        int tn = tir;
        advance(rn, tn);
        // the last tile reloads itself (unused) rather than branching around the loads: a branch
        // join makes the compiler wait for them before the tile's compute
        const bool more = t + 8 < t_end;
        load_tile(more ? rn : row, more ? tn : tir, nx);
        if (philox && kgrp == 0) draw16(row, tir);
        process(cu, row, tir);
        kgrp = (kgrp + 1) & 15;
        row = rn;
        tir = tn;
    }
    if (a.fired_out && cur_row >= 0) flush_fired();
}

}  // namespace nca
