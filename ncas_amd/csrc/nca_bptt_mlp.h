// Fused MLP backward of one BPTT step for bf16 cells with C = 32 channels, F = 128 features and
// 256 hidden units (gfx950): for a tile of 32 cells,
//
//   h    = relu(bf16(W1 z + b1))            recomputed (the forward's rounding points)
//   g_a  = bf16(W2^T g_dx) * [h > 0]
//   g_z  = bf16(W1^T g_a)                    -> HBM as bf16, for the transposed stencil
//   dW1 += g_a z^T,  dW2 += g_dx h^T,  db1 += sum over cells of g_a   (registers)
//
// with every product on v_mfma_f32_16x16x32_bf16. The gradients take the reference's bf16
// backward rounding points: g_dx arrives as bf16 values (the gradient of the bf16 tensor dx), the
// gradient of fc1's output and the gradient of z are rounded to bf16 (reference
// src/nca/engine/triton_mlp.py:46-78: gh = bf16(G W2) masked by h > 0, gx = bf16(gh W1)). W1, W2
// (rounded from the fp32 master weights), z, h, g_dx and g_a are then all bf16 values, so every
// product is exact and accumulates in fp32; the weight gradients stay fp32 sums over the
// cells (the reference rounds each step's weight gradient to bf16 as well; these are exact
// sums in another order).
//
// One workgroup per cell range (its slot of the partial sums), 8 waves; wave w owns hidden units
// [32w, 32w + 32) for fc1, g_a and the weight gradients, whose accumulators stay in registers for
// the whole range and are added into the slot at the end. MFMA operand layouts (16x16x32): lane
// (r = lane & 15, g = lane >> 4) holds A[r][8g + j] / B[8g + j][r], j < 8, and D[4g + i][r],
// i < 4. fc1 and g_a are computed in both orientations ([hidden][cell] and [cell][hidden]) so
// that each later product finds its operand in registers: D[cell 4g + i][hidden r] of two cell
// tiles is an operand whose k runs over 8 cells in the order perm(g, j) = j < 4 ? 4g + j :
// 16 + 4g + j - 4; the LDS operands of those products use the same cell order. g_z sums over all
// hidden units, so g_a goes through LDS and wave w computes g_z for features [16w, 16w + 16) of
// the tile's 32 cells, with its W1^T fragments (8 KB) held in registers.
//
// Per tile: the tile's z and g_dx (prefetched into registers during the previous tile) are stored
// to LDS; barrier; fc1, g_a, g_a to LDS, dW2 and dW1; barrier; g_z.
//
// LDS: every buffer is k-major with the cells of a row contiguous, in rows of 64 bytes (32 bf16)
// whose 16-byte chunk c sits at chunk c ^ ((row >> 1) & 3):
//   ZB   z [feature 128][cell 32 in perm order]
//   GB   g_dx [channel 32][cell 32 in perm order]
//   GL   g_a [hidden 256][cell 32]
//   B1   b1 fp32
// An operand whose k runs along the rows (z and g_dx for fc1 and g_a, with k over features and
// channels; g_a for g_z, with k over hidden units) is read with ds_read_b64_tr_b16, which within
// each 16-lane group gives lane i element i & 3 of the 8-byte loads of lanes 4m + (i >> 2),
// m < 4: lane 4m + s loads cells 4s .. 4s+3 of k-row m, so lane i receives cell i of k-rows
// 0..3; two such loads make an 8-element operand. The tile's stores are then whole 16-byte chunks
// (z and g_dx as loaded, 8 cells of one row) and 8-byte pieces (g_a, 4 cells of one hidden unit),
// where a [cell][k] layout took a 2-byte store per element. The row swizzle makes the 16-byte
// operand reads (lane (r, g): chunk g of row r) conflict-free for gfx950's ds_read_b128, which
// serves lanes 0-3 and 12-15 of one 16-lane group with lanes 4-11 of the next in one cycle, and
// the transposed reads of g_a take the 2.6 cycles of a plain ds_read_b64; those of z and g_dx take
// 4 (measured with a probe replaying each access pattern from 8 waves). Every address in the
// tile loop is a per-lane base plus a constant.
#pragma once

#include "nca_stream_util.h"

namespace nca {

struct MlpBackArgs {
    const uint16_t *Z;  // z (F x M) as bf16
    const float *Gdx;  // g_dx (C x M), bf16 values
    const unsigned char *img;  // the weight image written by mlp_back32_prep
    const float *b1;   // HD
    uint16_t *Gz;      // g_z (F x M) as bf16
    float *part;       // partial-sum slots, P floats each; workgroup s adds into slot s
    int64_t P, offW1, offB1, offW2, M;
    int per;  // cells per workgroup, a multiple of 32
};

struct Mb32 {
    static constexpr unsigned RS = 64;  // bytes per LDS row: 32 bf16
    static constexpr unsigned ZB = 0, GB = ZB + 128 * RS, GL = GB + 32 * RS, B1 = GL + 256 * RS, TOTAL = B1 + 1024;
    // weight image: per (wave, lane) the W1 fragments [ht][kb], the W2 fragments [ht] and the
    // W1^T fragments [kb], 16 bytes each
    static constexpr unsigned IMG_W1F = 0, IMG_W2F = IMG_W1F + 512 * 8 * 16, IMG_W1TF = IMG_W2F + 512 * 2 * 16,
                              IMG_BYTES = IMG_W1TF + 512 * 8 * 16;
};

typedef float mb_f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ mb_f32x4 mb_mfma(const bf16x8 &a, const bf16x8 &b, const mb_f32x4 &c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ bf16x8 mb_ld(const unsigned char *s, unsigned off) {
    return *reinterpret_cast<const bf16x8 *>(s + off);
}
__device__ __forceinline__ bf16x8 mb_pack8(const float v[8]) {
    const uint4 u = {cvt_pk_bf16(v[0], v[1]), cvt_pk_bf16(v[2], v[3]), cvt_pk_bf16(v[4], v[5]),
                     cvt_pk_bf16(v[6], v[7])};
    return __builtin_bit_cast(bf16x8, u);
}
__device__ __forceinline__ int mb_perm(int g, int j) { return j < 4 ? 4 * g + j : 16 + 4 * g + j - 4; }
// byte offset of 16-byte chunk c of LDS row `row`
__device__ __forceinline__ unsigned mb_off(unsigned row, unsigned c) { return row * Mb32::RS + 16u * (c ^ ((row >> 1) & 3u)); }
// ds_read_b64_tr_b16 at byte offset off of the LDS
__device__ __forceinline__ s16x4 mb_ldtr(const unsigned char *s, unsigned off) {
    typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (lds_s16x4 *)((__attribute__((address_space(3))) const unsigned char *)s + off));
}
// the 8-element operand of two transposed loads (k-rows 0-3, then 4-7)
__device__ __forceinline__ bf16x8 mb_cat(s16x4 lo, s16x4 hi) {
    const uint2 a = __builtin_bit_cast(uint2, lo), b = __builtin_bit_cast(uint2, hi);
    return __builtin_bit_cast(bf16x8, make_uint4(a.x, a.y, b.x, b.y));
}

// The weight image of mlp_back32 from the fp32 master weights (rounded to bf16): the register
// fragments of every (wave, lane): W1 for fc1, W2 for g_a, and W1^T for g_z (the A operand of
// feature tile w, hidden block kb in perm order). 18 workgroups of 512 threads, one per fragment
// of a lane (W1 [ht][kb]: 0-7, W2 [ht]: 8-9, W1^T [kb]: 10-17), so that a thread's chain is one
// fragment's 8 loads.
constexpr int kMb32PrepBlocks = 18;

__device__ __forceinline__ void mb32_prep_fragment(int f, const float *w1, const float *w2, unsigned char *img) {
    typedef Mb32 S;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, r = lane & 15, g = lane >> 4;
    float v[8];
    if (f < 8) {
        const int ht = f >> 2, kb = f & 3, hid = 32 * w + 16 * ht + r;
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = w1[hid * 128 + 32 * kb + 8 * g + j];
        *reinterpret_cast<bf16x8 *>(img + S::IMG_W1F + (tid * 8 + 4 * ht + kb) * 16) = mb_pack8(v);
    } else if (f < 10) {
        const int ht = f - 8, hid = 32 * w + 16 * ht + r;
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = w2[(8 * g + j) * 256 + hid];
        *reinterpret_cast<bf16x8 *>(img + S::IMG_W2F + (tid * 2 + ht) * 16) = mb_pack8(v);
    } else {
        const int kb = f - 10;
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = w1[(32 * kb + mb_perm(g, j)) * 128 + 16 * w + r];
        *reinterpret_cast<bf16x8 *>(img + S::IMG_W1TF + (tid * 8 + kb) * 16) = mb_pack8(v);
    }
}

__global__ void __launch_bounds__(512) mlp_back32_prep(const float *w1, const float *w2, unsigned char *img) {
    mb32_prep_fragment(blockIdx.x, w1, w2, img);
}

// VEC: M is a multiple of 4, so the cell quads of a tile are 16-byte aligned.
template <bool VEC>
__global__ void __launch_bounds__(512, 1) mlp_back32(MlpBackArgs a) {
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    typedef Mb32 S;
    const int tid = threadIdx.x, lane = tid & 63, r = lane & 15, g = lane >> 4;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int64_t M = a.M;
    const int64_t mb0 = (int64_t)blockIdx.x * a.per;
    if (mb0 >= M) return;  // uniform: an empty range adds nothing to its slot
    const int64_t mb1 = mb0 + a.per < M ? mb0 + a.per : M;

    // ---- set-up: b1 into LDS, W1 / W2 / W1^T fragments into registers
    if (tid < 256) reinterpret_cast<float *>(smem + S::B1)[tid] = a.b1[tid];
    bf16x8 w1f[2][4];   // [ht][kb]: W1[32w + 16ht + r][32kb + 8g + j]
    bf16x8 w2f[2];      // [ht]: W2[8g + j][32w + 16ht + r]
    bf16x8 w1t[8];      // [kb]: W1[32kb + perm(g, j)][16w + r]
#pragma unroll
    for (int ht = 0; ht < 2; ++ht) {
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
            w1f[ht][kb] = *reinterpret_cast<const bf16x8 *>(a.img + S::IMG_W1F + (tid * 8 + 4 * ht + kb) * 16);
        w2f[ht] = *reinterpret_cast<const bf16x8 *>(a.img + S::IMG_W2F + (tid * 2 + ht) * 16);
    }
#pragma unroll
    for (int kb = 0; kb < 8; ++kb) w1t[kb] = *reinterpret_cast<const bf16x8 *>(a.img + S::IMG_W1TF + (tid * 8 + kb) * 16);
    // the weight fragments live in AGPRs (MFMA reads its A / B operands from them), leaving the
    // VGPRs to the accumulators and the tile's operands
#pragma unroll
    for (int ht = 0; ht < 2; ++ht) {
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) asm volatile("" : "+a"(w1f[ht][kb]));
        asm volatile("" : "+a"(w2f[ht]));
    }
#pragma unroll
    for (int kb = 0; kb < 8; ++kb) asm volatile("" : "+a"(w1t[kb]));
    mb_f32x4 dw1[2][8], dw2[2][2];  // dw1[ht][ft]: D[hid 32w+16ht+4g+i][f 16ft+r]; dw2[ct][ht]: D[ch 16ct+4g+i][hid 32w+16ht+r]
#pragma unroll
    for (int x = 0; x < 2; ++x) {
#pragma unroll
        for (int y = 0; y < 8; ++y) dw1[x][y] = mb_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int y = 0; y < 2; ++y) dw2[x][y] = mb_f32x4{0.f, 0.f, 0.f, 0.f};
    }
    float db1[2] = {0.f, 0.f};  // hidden 32w + 16ht + r, this lane's cells

    // ---- the tile's loads (prefetched one tile ahead): thread (row tid >> 2, q = tid & 3) loads
    // cells perm(q, 0..7) of z row tid >> 2 and, in waves 0 and 1, of g_dx row tid >> 2 (byte
    // offsets below 2^32, checked by the host). Cells past the range read cell mb0 and are zeroed
    // when the tile is stored, so the loads need no branch and nothing uses them before then
    // (either would make the compiler wait for them).
    const int lrow = tid >> 2, q = tid & 3;
    const unsigned char *zb = reinterpret_cast<const unsigned char *>(a.Z);
    const unsigned char *gb = reinterpret_cast<const unsigned char *>(a.Gdx);
    const uint32_t rowb = (uint32_t)lrow * (uint32_t)M * 4u, rowz = (uint32_t)lrow * (uint32_t)M * 2u;
    // z arrives as raw bf16 words, kept unconverted until the tile is stored: any use at the load
    // would make the compiler wait for it there. VEC: pzv[h] = cells perm(q, 4h .. 4h+3);
    // otherwise pzs[j] = cell perm(q, j) in the low 16 bits
    uint2 pzv[2];
    uint32_t pzs[8];
    float pg[8];
    auto load8 = [&](const unsigned char *base, int64_t m0, float v[8]) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int64_t m = m0 + 16 * h + 4 * q;
            if (VEC) {
                const bool ok = m < mb1;  // the whole quad (mb1 is a multiple of 4)
                const uint32_t off = rowb + (uint32_t)(ok ? m : mb0) * 4u;
                const float4 x = *reinterpret_cast<const float4 *>(base + off);
                v[4 * h] = x.x;
                v[4 * h + 1] = x.y;
                v[4 * h + 2] = x.z;
                v[4 * h + 3] = x.w;
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const bool ok = m + e < mb1;
                    v[4 * h + e] = *reinterpret_cast<const float *>(base + rowb + (uint32_t)(ok ? m + e : mb0) * 4u);
                }
            }
        }
    };
    auto load8z = [&](int64_t m0) {  // z: bf16
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int64_t m = m0 + 16 * h + 4 * q;
            if (VEC) {
                const bool ok = m < mb1;
                pzv[h] = *reinterpret_cast<const uint2 *>(zb + rowz + (uint32_t)(ok ? m : mb0) * 2u);
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const bool ok = m + e < mb1;
                    pzs[4 * h + e] = *reinterpret_cast<const uint16_t *>(zb + rowz + (uint32_t)(ok ? m + e : mb0) * 2u);
                }
            }
        }
    };
    auto zero_past = [&](int64_t m0, float v[8]) {  // cells past the range
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = m0 + mb_perm(q, j) < mb1 ? v[j] : 0.0f;
    };
    auto load_tile = [&](int64_t m0) {
        load8z(m0);
        if (w < 2) load8(gb, m0, pg);
    };
    const unsigned o_st = mb_off((unsigned)lrow, (unsigned)q);
    auto store_tile = [&](int64_t m0) {  // ZB (GB) row lrow chunk q: cells perm(q, 0..7)
        uint32_t zw[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            uint32_t v = VEC ? ((e & 1) ? pzv[e >> 1].y : pzv[e >> 1].x) : (pzs[2 * e] | (pzs[2 * e + 1] << 16));
            if (m0 + mb_perm(q, 2 * e) >= mb1) v &= 0xffff0000u;  // cells past the range
            if (m0 + mb_perm(q, 2 * e + 1) >= mb1) v &= 0x0000ffffu;
            zw[e] = v;
        }
        *reinterpret_cast<uint4 *>(smem + S::ZB + o_st) = make_uint4(zw[0], zw[1], zw[2], zw[3]);
        if (w < 2) {
            zero_past(m0, pg);
            *reinterpret_cast<bf16x8 *>(smem + S::GB + o_st) = mb_pack8(pg);
        }
    };
    // per-lane LDS offsets of the tile loop. Transposed operand loads: lane 4m + s of the group
    // loads cells 4s .. 4s+3 of k-row 8g + m (fc1, g_a; +4 for k-rows 4-7), in perm order chunk s,
    // half ct; for g_z cells 16ct + 4s .. +3 (chunk 2ct + s / 2, half s & 1) of hidden row
    // 4g + m (+16 for k-rows 4-7) of each 32-block
    const unsigned tm = (unsigned)r >> 2, ts = (unsigned)r & 3u;
    const unsigned o_tr0 = mb_off(8u * g + tm, ts), o_tr1 = mb_off(8u * g + 4u + tm, ts);
    unsigned o_gl[2][2];  // [ct][k-rows 0-3 / 4-7]
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
        o_gl[ct][0] = mb_off(4u * g + tm, 2u * ct + (ts >> 1)) + 8u * (ts & 1u);
        o_gl[ct][1] = mb_off(4u * g + 16u + tm, 2u * ct + (ts >> 1)) + 8u * (ts & 1u);
    }
    // 16-byte operand loads: chunk g of row r (+16 rows per tile or feature block)
    const unsigned o_rg = mb_off((unsigned)r, (unsigned)g);

    // g_z's buffer (below 2^31 bytes, checked by the host); the third dword is gfx9's format word
    const __amdgpu_buffer_rsrc_t gz_rsrc =
        __builtin_amdgcn_make_buffer_rsrc(a.Gz, (short)0, (int)(M * 128 * 2), 0x00020000);
    const int ntile = (int)((mb1 - mb0 + 31) / 32);
    load_tile(mb0);
    // the first tile's loads complete here, so that the loop's wait for each prefetch counts the
    // previous tile's stores issued after it (else the first iteration's state, with no stores
    // behind the loads, makes every iteration wait for them as well)
    if (VEC) asm volatile("" : : "v"(pzv[0]), "v"(pzv[1]));
    else asm volatile("" : : "v"(pzs[0]), "v"(pzs[7]));
    if (w < 2) asm volatile("" : : "v"(pg[0]), "v"(pg[7]));
    for (int t = 0; t < ntile; ++t) {
        const int64_t m0 = mb0 + 32 * (int64_t)t;
        store_tile(m0);
        if (t + 1 < ntile) load_tile(m0 + 32);
        __syncthreads();

        // ---- fc1: hT[ct][ht] = D[cell 16ct+4g+i][hid 32w+16ht+r]
        mb_f32x4 hT[2][2];
#pragma unroll
        for (int x = 0; x < 2; ++x)
#pragma unroll
            for (int y = 0; y < 2; ++y) hT[x][y] = mb_f32x4{0.f, 0.f, 0.f, 0.f};
        // operands of fc1 read up front; those of g_a while fc1 finishes
        bf16x8 zf[4][2], gf[2];
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
            for (int ct = 0; ct < 2; ++ct) {
                const unsigned zo = S::ZB + 32u * S::RS * kb + 8u * ct;  // k-rows 32 kb + 8g + m
                zf[kb][ct] = mb_cat(mb_ldtr(smem, zo + o_tr0), mb_ldtr(smem, zo + o_tr1));
            }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
            for (int ht = 0; ht < 2; ++ht) {
                hT[0][ht] = mb_mfma(zf[kb][0], w1f[ht][kb], hT[0][ht]);
                hT[1][ht] = mb_mfma(zf[kb][1], w1f[ht][kb], hT[1][ht]);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int ct = 0; ct < 2; ++ct)
            gf[ct] = mb_cat(mb_ldtr(smem, S::GB + 8u * ct + o_tr0), mb_ldtr(smem, S::GB + 8u * ct + o_tr1));
        __builtin_amdgcn_sched_barrier(0);
        {
            const float *b1L = reinterpret_cast<const float *>(smem + S::B1);
#pragma unroll
            for (int ht = 0; ht < 2; ++ht) {
                const float bt = b1L[32 * w + 16 * ht + r];
#pragma unroll
                for (int ct = 0; ct < 2; ++ct)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const float vt = round_bf16(__fadd_rn(hT[ct][ht][i], bt));
                        hT[ct][ht][i] = vt > 0.0f ? vt : 0.0f;
                    }
            }
        }

        // ---- g_a = bf16(W2^T g_dx) * [h > 0]: gaT[ct][ht] like hT
        mb_f32x4 gaT[2][2];
#pragma unroll
        for (int ct = 0; ct < 2; ++ct)
#pragma unroll
            for (int ht = 0; ht < 2; ++ht) gaT[ct][ht] = mb_mfma(gf[ct], w2f[ht], mb_f32x4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
        for (int x = 0; x < 2; ++x)
#pragma unroll
            for (int y = 0; y < 2; ++y)
#pragma unroll
                for (int i = 0; i < 4; ++i) gaT[x][y][i] = hT[x][y][i] > 0.0f ? round_bf16(gaT[x][y][i]) : 0.0f;
        // db1: this lane's hidden unit 32w + 16ht + r over cells 16ct + 4g + i
#pragma unroll
        for (int ht = 0; ht < 2; ++ht)
#pragma unroll
            for (int ct = 0; ct < 2; ++ct)
#pragma unroll
                for (int i = 0; i < 4; ++i) db1[ht] = __fadd_rn(db1[ht], gaT[ct][ht][i]);
        // g_a, k over cells in perm order: ap[ht] element j = g_a[hid 32w + 16ht + r][cell perm(g, j)]
        bf16x8 ap[2];
#pragma unroll
        for (int ht = 0; ht < 2; ++ht) {
            const float v[8] = {gaT[0][ht][0], gaT[0][ht][1], gaT[0][ht][2], gaT[0][ht][3],
                                gaT[1][ht][0], gaT[1][ht][1], gaT[1][ht][2], gaT[1][ht][3]};
            ap[ht] = mb_pack8(v);
        }
        // ... and into GL for g_z: hidden row 32w + 16ht + r, cells 16ct + 4g .. +3 (chunk
        // 2ct + g / 2, half g & 1): the ct halves of ap
#pragma unroll
        for (int ht = 0; ht < 2; ++ht) {
            const uint4 u = __builtin_bit_cast(uint4, ap[ht]);
            const unsigned row = 32u * (unsigned)w + 16u * ht + (unsigned)r;
#pragma unroll
            for (int ct = 0; ct < 2; ++ct)
                *reinterpret_cast<uint2 *>(smem + S::GL + mb_off(row, 2u * ct + ((unsigned)g >> 1)) + 8u * (g & 1)) =
                    ct ? make_uint2(u.z, u.w) : make_uint2(u.x, u.y);
        }

        // ---- dW2 += g_dx h^T: A = g_dx [channel][cells perm], B = h^T
        {
            bf16x8 hb[2];
#pragma unroll
            for (int ht = 0; ht < 2; ++ht) {
                const float v[8] = {hT[0][ht][0], hT[0][ht][1], hT[0][ht][2], hT[0][ht][3],
                                    hT[1][ht][0], hT[1][ht][1], hT[1][ht][2], hT[1][ht][3]};
                hb[ht] = mb_pack8(v);
            }
#pragma unroll
            for (int ct = 0; ct < 2; ++ct) {
                const bf16x8 gbv = mb_ld(smem, S::GB + 16u * S::RS * ct + o_rg);
#pragma unroll
                for (int ht = 0; ht < 2; ++ht) dw2[ct][ht] = mb_mfma(gbv, hb[ht], dw2[ct][ht]);
            }
        }
        // ---- dW1 += g_a z^T: A = g_a (hidden x cells perm), B = z [cells perm][feature]
#pragma unroll
        for (int ft = 0; ft < 8; ft += 2) {
            const bf16x8 zb0 = mb_ld(smem, S::ZB + 16u * S::RS * ft + o_rg);  // feature 16 ft + r
            const bf16x8 zb1 = mb_ld(smem, S::ZB + 16u * S::RS * (ft + 1) + o_rg);
#pragma unroll
            for (int ht = 0; ht < 2; ++ht) {
                dw1[ht][ft] = mb_mfma(ap[ht], zb0, dw1[ht][ft]);
                dw1[ht][ft + 1] = mb_mfma(ap[ht], zb1, dw1[ht][ft + 1]);
            }
        }
        __syncthreads();

        // ---- g_z = bf16(W1^T g_a): features 16w + 4g + i of cells 16ct + r, even and odd hidden
        //      blocks in separate chains
        {
            mb_f32x4 gz[2][2];
#pragma unroll
            for (int x = 0; x < 2; ++x)
#pragma unroll
                for (int y = 0; y < 2; ++y) gz[x][y] = mb_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kb = 0; kb < 8; ++kb) {
                // k = 8g + j over hidden units 32 kb + perm(g, j): rows 32 kb + 4g + m, then +16
                const unsigned bo = S::GL + 32u * S::RS * kb;
                const bf16x8 B0 = mb_cat(mb_ldtr(smem, bo + o_gl[0][0]), mb_ldtr(smem, bo + o_gl[0][1]));
                const bf16x8 B1 = mb_cat(mb_ldtr(smem, bo + o_gl[1][0]), mb_ldtr(smem, bo + o_gl[1][1]));
                gz[0][kb & 1] = mb_mfma(w1t[kb], B0, gz[0][kb & 1]);
                gz[1][kb & 1] = mb_mfma(w1t[kb], B1, gz[1][kb & 1]);
            }
            // raw buffer stores: a lane past the range gets an offset beyond the buffer, whose
            // store the hardware drops, so the stores need no branch (a branch around them
            // leaves their number unknown to the next tile's wait for its prefetched loads)
#pragma unroll
            for (int ct = 0; ct < 2; ++ct) {
                const int64_t m = m0 + 16 * ct + r;
                const uint32_t o0 = ((uint32_t)(16 * w + 4 * g) * (uint32_t)M + (uint32_t)m) * 2u;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint32_t off = m < mb1 ? o0 + (uint32_t)i * (uint32_t)M * 2u : 0x80000000u;
                    const __bf16 v = (__bf16)__fadd_rn(gz[ct][0][i], gz[ct][1][i]);
                    __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(unsigned short, v), gz_rsrc, off, 0, 0);
                }
            }
        }
    }

    // ---- this range's partial sums into slot blockIdx.x
    float *ps = a.part + (int64_t)blockIdx.x * a.P;
#pragma unroll
    for (int ht = 0; ht < 2; ++ht)
#pragma unroll
        for (int ft = 0; ft < 8; ++ft)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                float *p = ps + a.offW1 + (32 * w + 16 * ht + 4 * g + i) * 128 + 16 * ft + r;
                *p = __fadd_rn(*p, dw1[ht][ft][i]);
            }
#pragma unroll
    for (int ct = 0; ct < 2; ++ct)
#pragma unroll
        for (int ht = 0; ht < 2; ++ht)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                float *p = ps + a.offW2 + (16 * ct + 4 * g + i) * 256 + 32 * w + 16 * ht + r;
                *p = __fadd_rn(*p, dw2[ct][ht][i]);
            }
#pragma unroll
    for (int ht = 0; ht < 2; ++ht) {
        float v = db1[ht];
        v = __fadd_rn(v, __shfl_xor(v, 16));
        v = __fadd_rn(v, __shfl_xor(v, 32));
        if (g == 0) {
            float *p = ps + a.offB1 + 32 * w + 16 * ht + r;
            *p = __fadd_rn(*p, v);
        }
    }
}

}  // namespace nca
