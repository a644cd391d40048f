// The whole backward of a BPTT chunk in one launch, for bf16 cells with 32 channels, 128
// features and 256 hidden units (gfx950); included by nca_bptt.hip (it uses that file's Dims,
// FrontArgs, head_grad_core, load_out and block_sums).
//
// A workgroup owns a block of board rows for every step of the chunk: a piece of Hp rows of one
// board (pieces > 1), or a whole board (the repair launch, and calls with too many boards for
// pieces). Walking the steps in reverse, each step runs, for the workgroup's cells:
//
//   stage    x_t of its rows and one halo row on each side into XS (bf16, padding applied)
//   tiles    per 32 cells: the front (loss gradient of the step's output, the gradient from the
//            later step, the clamp's and the fire mask's backward: g_u into GX, bf16 g_dx into
//            the MLP's operand buffer) and z (the perception of XS) side by side, then the MLP
//            backward of mlp_back32 (h recomputed; g_a; g_z; dW1, dW2, db1 summed in registers),
//            with g_z stored into GZ
//   exchange pieces: the first and last rows of g_z go to the neighbouring pieces through tagged
//            words in global memory, and their rows come back into GZ's halo rows
//   back     g_x = g_u + the transposed stencil of g_z (into GX, the next step's incoming
//            gradient) and the kernel-weight sums
//
// so g_z, g_u / g_x and the weight-gradient sums never leave the CU between steps: one launch
// replaces three per step, and the weight-gradient partial sums are written once per chunk
// instead of being read, added to and written back every step (the multi-launch path's
// mlp_back32 moves 160 KB per workgroup per step for that).
//
// Per step and cell the arithmetic is that of the multi-launch path (front_body, z_plane_body,
// mlp_back32, stencil_back_strip) in the same per-element order; the sums over cells run in
// another fixed order (per workgroup: tiles, then the workgroup's slot), so the gradients are
// deterministic and agree with that path to fp32 rounding.
//
// Pieces wait for their neighbours' rows of every step: word e of a row is (tag << 32 | two bf16
// of g_z) with tag = step + 1, stored and loaded as single-copy atomic 8-byte words at agent
// scope, in one of two slots by step parity (a piece runs at most one step ahead of a
// neighbour). A word whose tag is not yet the step's is re-read; after spin_limit re-reads the
// piece sets *status, waits no more, and its results are wrong: the host queues the repair
// launch (whole boards, g_z and g_x in global memory, no waits) behind the pieces' launch, which
// runs only if *status is set and then rewrites every output. A wait runs out only when the
// pieces of a board are not resident together.
#pragma once

namespace {

constexpr int kFusedThreads = 256;  // 4 waves, one per SIMD (each with the whole register file)
constexpr int kFusedMaxChunk = 64;  // steps of a chunk (the per-step loss weights travel as arguments)

struct FusedArgs {
    FrontArgs fa;  // d, given, targets, mask, denom, head_w, head_b; fire: fire_u8 = the chunk's masks
                   // (n, rows, HW) or null, key_ptr = the per-step keys or null, key, row0, step =
                   // the chunk's first step, p
    const float *states;  // n + 1 states (rows, C, H, W), stride floats apart
    int64_t stride;
    int n;
    float wscale[kFusedMaxChunk];  // per step: w_t / sum(w) (/ M without a loss mask); 0: no loss term
    const float *grad_final;       // (rows, C, H, W) or null
    float *grad_x0;                // (rows, C, H, W) or null
    const unsigned char *img;      // mlp_back32_prep's weight image
    const float *b1, *kern, *padv;
    float *part, *lossacc;  // slot blockIdx.x of each (the slots were zeroed by the host)
    int64_t P, offK, offW1, offB1, offW2, offB2, offHW, offHB;
    int pieces, Hp;         // pieces per board and rows per piece; pieces = 1: whole boards
    uint16_t *gz_g;         // whole boards: g_z, (rows, 4, H, W, 32) bf16
    float *gx_g;            // whole boards: g_u / g_x, (rows, HW, 32) fp32
    uint64_t *xch;          // pieces: (rows, pieces, 2 sides, 2 slots, 64 W) words, zero at launch
    uint32_t *status;       // pieces: set to 1 when a wait runs out
    int spin_limit, tag_skew;
    const uint32_t *run_if;  // whole boards: run only if *run_if != 0 (the repair launch)
    int zero_slots;          // the repair: slots [gridDim.x, zero_slots) are zeroed
    unsigned l_GZ, l_GX, l_XS, l_MLP, l_FI, l_RED, l_ACC, l_HWL, l_FB;
    int gz_rows;  // rows of a g_z plane in LDS (Hp + 2)
};

// LDS plan: GZ g_z [k 4][row Hw + 2][col W][c 32] bf16 and GX [cell][c 32] fp32 (pieces only),
// XS x_t [row Hw + 2][col W + 2][c 32] bf16, the MLP buffers of mlp_back32, the per-cell
// head terms FI [3 tiles][32][12], the reduction scratch, the chunk's small sums (dk 36, db2 32, head and
// loss 21), the head's weights (floats 0-19 of HWL; 24-31 zero; 32-67 the perception kernels; 68-99
// the wall value) and FB, the step's fire bits of the workgroup's cells (a byte each).
struct FusedPlan {
    unsigned GZ, GX, XS, MLP, FI, RED, ACC, HWL, FB, total;
};

inline FusedPlan fused_plan(bool pieces, int Hw, int W) {
    FusedPlan p;
    unsigned o = 0;
    p.GZ = o;
    if (pieces) o += 4u * (unsigned)(Hw + 2) * (unsigned)W * 64u;
    p.GX = o;
    if (pieces) o += (unsigned)(Hw * W) * 128u;
    p.XS = o;
    o += (unsigned)(Hw + 2) * (unsigned)(W + 2) * 64u;
    p.MLP = o;
    o += nca::Mb32::TOTAL;
    p.FI = o;
    o += 3u * 32u * 12u * 4u;
    p.RED = o;
    o += 4u * 40u * 4u;
    p.ACC = o;
    o += 96u * 4u;
    p.HWL = o;
    o += 100u * 4u;
    p.FB = o;
    o += 2u * (((unsigned)(Hw * W) + 15u) & ~15u);
    p.total = o;
    return p;
}

// The MLP of mlp_back32: with NH = 8 / waves, wave w takes the hidden blocks of mlp_back32's waves
// NH w .. NH w + NH - 1 (virtual waves vw = NH w + hb), one after the other for the products whose
// operands differ, all from one load where they share one.
template <bool PIECES>
__global__ void __launch_bounds__(kFusedThreads, 1) bptt_back_fused(FusedArgs A) {
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    typedef nca::Mb32 S;
    using nca::mb_cat;
    using nca::mb_ld;
    using nca::mb_ldtr;
    using nca::mb_mfma;
    using nca::mb_off;
    using nca::mb_f32x4;
    constexpr int NWV = kFusedThreads / 64, NH = 8 / NWV;
    constexpr int FT = kFusedThreads / 2;  // front threads (then z threads)
    constexpr int FCH = 32 * 32 / FT;      // channels per front thread (cells per z thread)
    if (!PIECES && A.run_if && __hip_atomic_load(A.run_if, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0u) return;
    const Dims &d = A.fa.d;
    // the thread's indices are made opaque at every step (below), so that the compiler keeps the
    // addresses derived from them inside the step loop rather than hoisting hundreds of them out
    // of it (which spills them)
    int tid = threadIdx.x, lane = tid & 63, r = lane & 15, g = lane >> 4;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int H = d.H, W = d.W, HW = d.HW, W2 = W + 2;
    const int P = PIECES ? A.pieces : 1;
    const int board = (int)blockIdx.x / P, piece = (int)blockIdx.x - board * P;
    const int r0 = PIECES ? piece * A.Hp : 0;
    const int r1 = PIECES ? (r0 + A.Hp < H ? r0 + A.Hp : H) : H;
    const int Hw = r1 - r0, nw = Hw * W;
    const bool wrap = d.padding == 2;
    unsigned char *ms = smem + A.l_MLP;
    float *fiL = reinterpret_cast<float *>(smem + A.l_FI);
    float *redL = reinterpret_cast<float *>(smem + A.l_RED);
    float *dkacc = reinterpret_cast<float *>(smem + A.l_ACC), *hacc = dkacc + 68;
    // hacc: the loss (0), the head weights' gradient (1 + 4 v + c), its bias's (17 + v)
    float *hwL = reinterpret_cast<float *>(smem + A.l_HWL);
    unsigned char *fbL = smem + A.l_FB;  // the step's fire bits of the workgroup's cells
    const int64_t xb = (int64_t)board * 32 * HW;  // channel 0 of the board in a state
    const int64_t mb = (int64_t)board * HW;       // the board's first cell

    // ---- set-up: b1, the head's weights, zero sums; the W1 / W2 / W1^T fragments of both
    // virtual waves into AGPRs
    for (int e = tid; e < 256; e += kFusedThreads) reinterpret_cast<float *>(ms + S::B1)[e] = A.b1[e];
    if (tid < d.n_out * d.c_out) hwL[tid] = A.fa.head_w[tid];
    if (tid < d.n_out) hwL[16 + tid] = A.fa.head_b[tid];
    if (tid < 8) hwL[24 + tid] = 0.0f;  // zeros read by the transposed stencil's taps outside the board
    if (tid < 36) hwL[32 + tid] = A.kern[tid];  // the perception kernels, read from LDS in the loops
    if (tid < 32) hwL[68 + tid] = A.padv[tid];  // the wall value of each channel
    if (tid < 96) dkacc[tid] = 0.0f;
    nca::bf16x8 w1f[NH][2][4], w2f[NH][2], w1t[NH][8];
#pragma unroll
    for (int hb = 0; hb < NH; ++hb) {
        const int t8 = (NH * w + hb) * 64 + lane;  // mlp_back32's thread of the fragment
#pragma unroll
        for (int ht = 0; ht < 2; ++ht) {
#pragma unroll
            for (int kb = 0; kb < 4; ++kb)
                w1f[hb][ht][kb] = *reinterpret_cast<const nca::bf16x8 *>(A.img + S::IMG_W1F + (t8 * 8 + 4 * ht + kb) * 16);
            w2f[hb][ht] = *reinterpret_cast<const nca::bf16x8 *>(A.img + S::IMG_W2F + (t8 * 2 + ht) * 16);
        }
#pragma unroll
        for (int kb = 0; kb < 8; ++kb)
            w1t[hb][kb] = *reinterpret_cast<const nca::bf16x8 *>(A.img + S::IMG_W1TF + (t8 * 8 + kb) * 16);
    }
#pragma unroll
    for (int hb = 0; hb < NH; ++hb) {
#pragma unroll
        for (int ht = 0; ht < 2; ++ht) {
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) asm volatile("" : "+a"(w1f[hb][ht][kb]));
            asm volatile("" : "+a"(w2f[hb][ht]));
        }
#pragma unroll
        for (int kb = 0; kb < 8; ++kb) asm volatile("" : "+a"(w1t[hb][kb]));
    }
    // dw1[hb][ht][ft]: D[hid 32vw+16ht+4g+i][f 16ft+r]; dw2[hb][ct][ht]: D[ch 16ct+4g+i][hid 32vw+16ht+r]
    mb_f32x4 dw1[NH][2][8], dw2[NH][2][2];
#pragma unroll
    for (int hb = 0; hb < NH; ++hb)
#pragma unroll
        for (int x = 0; x < 2; ++x) {
#pragma unroll
            for (int y = 0; y < 8; ++y) dw1[hb][x][y] = mb_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int y = 0; y < 2; ++y) dw2[hb][x][y] = mb_f32x4{0.f, 0.f, 0.f, 0.f};
        }
    float db1[NH][2] = {};  // hidden 32 vw + 16 ht + r, this lane's cells
    // dW2 and the kernel-weight sums live in AGPRs between their updates, leaving the VGPRs
    // to dW1 and the phases' operands
    auto pin_dw2 = [&]() {
#pragma unroll
        for (int hb = 0; hb < NH; ++hb)
#pragma unroll
            for (int ct = 0; ct < 2; ++ct)
#pragma unroll
                for (int ht = 0; ht < 2; ++ht) asm volatile("" : "+a"(dw2[hb][ct][ht]));
    };
    mb_f32x4 dkw = {0.f, 0.f, 0.f, 0.f};         // this wave's kernel-weight sums (lanes 0 .. 8)
    // wave 0: db2 of channels 16 ct + 4 g + i in column r of the product with a matrix of ones
    mb_f32x4 db2m[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
    // the z waves' stencil B operands: column k = lane % 4 is kernel k, taps 0-3 / 4-7; tap 8 in
    // the k slot of the channel's place in its quad (the forward's operands)
    nca::s16x4 kzb0, kzb1, kzb2[4];
    {
        const int k = lane & 3;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            kzb0[e] = nca::bf16_bits(A.kern[k * 9 + e]);
            kzb1[e] = nca::bf16_bits(A.kern[k * 9 + 4 + e]);
        }
        const short k8 = nca::bf16_bits(A.kern[k * 9 + 8]);
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int e = 0; e < 4; ++e) kzb2[c][e] = e == c ? k8 : (short)0;
    }
    const nca::bf16x8 ones8 = __builtin_bit_cast(nca::bf16x8, make_uint4(0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u));

    // MLP operand offsets (mlp_back32's)
    const unsigned tm = (unsigned)r >> 2, ts = (unsigned)r & 3u;
    const unsigned o_tr0 = mb_off(8u * g + tm, ts), o_tr1 = mb_off(8u * g + 4u + tm, ts);
    unsigned o_gl[2][2];
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
        o_gl[ct][0] = mb_off(4u * g + tm, 2u * ct + (ts >> 1)) + 8u * (ts & 1u);
        o_gl[ct][1] = mb_off(4u * g + 16u + tm, 2u * ct + (ts >> 1)) + 8u * (ts & 1u);
    }
    const unsigned o_rg = mb_off((unsigned)r, (unsigned)g);

    // g_z of plane k, workgroup row pr (-1 .. Hw), column col, channels c ..: LDS byte offset
    // (pieces) or global element (whole boards; board row pr, wrapped by the caller)
    auto gz_lds = [&](int k, int pr, int col, int c) -> unsigned {
        return A.l_GZ + (unsigned)((((k * A.gz_rows) + pr + 1) * W + col) * 64 + 2 * c);
    };
    auto gz_glb = [&](int k, int br, int col, int c) -> uint16_t * {
        return A.gz_g + ((((int64_t)board * 4 + k) * H + br) * W + col) * 32 + c;
    };
    // g_u / g_x of workgroup cell mt, channels 4 cq .. 4 cq + 3
    auto gx_ld = [&](int mt, int cq) -> float4 {
        if (PIECES) return nca::lds_ld128f(smem, A.l_GX + (unsigned)(mt * 128 + cq * 16));
        return *reinterpret_cast<const float4 *>(A.gx_g + (mb + mt) * 32 + 4 * cq);
    };
    auto gx_st = [&](int mt, int cq, float4 v) {
        if (PIECES)
            nca::lds_st128f(smem, A.l_GX + (unsigned)(mt * 128 + cq * 16), v);
        else
            *reinterpret_cast<float4 *>(A.gx_g + (mb + mt) * 32 + 4 * cq) = v;
    };

    bool hfail = false;  // pieces: a wait ran out (no later wait)

    // XS staging: thread item (row, channel octet, column), columns fastest; the loads of up to
    // XSU items a thread are issued together into xsv, then converted and stored
    constexpr int XSU = 6;
    const int xs_items = (Hw + 2) * 4 * W2;
    float xsv[XSU][8];
    auto xs_load = [&](int ts, int e0) {
        const float *xs_src = A.states + (int64_t)ts * A.stride + xb;
#pragma unroll
        for (int uu = 0; uu < XSU; ++uu) {
            const int e = e0 + uu * kFusedThreads, ec = e < xs_items ? e : 0;
            const int pc = ec % W2, rest = ec / W2, o = rest & 3, pr = rest >> 2;
            const int br = r0 - 1 + pr, bc = pc - 1;
            const bool in = br >= 0 && br < H && bc >= 0 && bc < W;
            const int ar = br < 0 ? br + H : (br >= H ? br - H : br);
            const int ac = bc < 0 ? bc + W : (bc >= W ? bc - W : bc);
            const bool take = in || wrap;
            const int q = take ? ar * W + ac : 0;
            // raw loads (the padding value replaces those of cells outside the board in xs_store)
#pragma unroll
            for (int u = 0; u < 8; ++u) xsv[uu][u] = xs_src[(int64_t)(8 * o + u) * HW + q];
        }
    };
    auto xs_store = [&](int e0) {
#pragma unroll
        for (int uu = 0; uu < XSU; ++uu) {
            const int e = e0 + uu * kFusedThreads;
            if (e < xs_items) {
                const int pc = e % W2, rest = e / W2, o = rest & 3, pr = rest >> 2;
                const int br = r0 - 1 + pr, bc = pc - 1;
                if (!wrap && !(br >= 0 && br < H && bc >= 0 && bc < W)) {
#pragma unroll
                    for (int u = 0; u < 8; ++u) xsv[uu][u] = d.padding == 1 ? hwL[68 + 8 * o + u] : 0.0f;
                }
                const uint4 pk = {nca::cvt_pk_bf16(xsv[uu][0], xsv[uu][1]), nca::cvt_pk_bf16(xsv[uu][2], xsv[uu][3]),
                                  nca::cvt_pk_bf16(xsv[uu][4], xsv[uu][5]), nca::cvt_pk_bf16(xsv[uu][6], xsv[uu][7])};
                nca::lds_st128(smem, A.l_XS + (unsigned)((pr * W2 + pc) * 64 + o * 16), pk);
            }
        }
    };

    // g_x = g_u + the transposed stencil of g_z for the workgroup rows [ra, rb): thread item
    // (cell, channel quad), the quads of a cell on consecutive threads; an item's 36 loads are
    // issued before its arithmetic
    auto gx_rows = [&](int ra, int rb) {
        // the kernels' LDS offset, opaque here: the compiler would otherwise keep the 36 weights
        // in registers through the whole step loop (they never change), crowding the staging
        unsigned kofs = A.l_HWL + 128u;
        asm volatile("" : "+s"(kofs));
        float kwv[36];  // loaded once per call
#pragma unroll
        for (int e = 0; e < 9; ++e) {
            const float4 v = nca::lds_ld128f(smem, kofs + 16u * (unsigned)e);
            kwv[4 * e] = v.x;
            kwv[4 * e + 1] = v.y;
            kwv[4 * e + 2] = v.z;
            kwv[4 * e + 3] = v.w;
        }
        for (int it = ra * W * 8 + tid; it < rb * W * 8; it += kFusedThreads) {
            const int mt = it >> 3, cq = it & 7, c0 = 4 * cq;
            const int pr = mt / W, col = mt - pr * W, bi = r0 + pr;
            const float4 gu = gx_ld(mt, cq);
            uint2 zv[9][4];
#pragma unroll
            for (int tp = 0; tp < 9; ++tp) {
                // tap tp = (dy, dx) of cell (bi - dy, col - dx) reads this cell; outside the board
                // (wall or zero padding) it reads zeros (pieces: 8 zero bytes in LDS)
                const int dy = tp / 3 - 1, dx = tp % 3 - 1;
                int sc = col - dx;
                const int sb = bi - dy;
                const bool ok = wrap | (((unsigned)sc < (unsigned)W) & ((unsigned)sb < (unsigned)H));  // no branches
                sc = sc < 0 ? sc + W : (sc >= W ? sc - W : sc);
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    if (PIECES) {
                        unsigned ad = ok ? gz_lds(k, pr - dy, sc, c0) : A.l_HWL + 96u;
                        asm("" : "+v"(ad));  // a select of the address, not a branch around the load
                        zv[tp][k] = nca::lds_ld64(smem, ad);
                    } else {
                        const int sr = sb < 0 ? sb + H : (sb >= H ? sb - H : sb);
                        const uint2 z = *reinterpret_cast<const uint2 *>(gz_glb(k, sr, sc, c0));
                        zv[tp][k] = ok ? z : make_uint2(0u, 0u);
                    }
                }
            }
            float gq[4] = {gu.x, gu.y, gu.z, gu.w};
#pragma unroll
            for (int tp = 0; tp < 9; ++tp) {
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const float kw = kwv[k * 9 + tp];
                    const uint2 z = zv[tp][k];
                    gq[0] = __builtin_fmaf(kw, nca::bf16_lo(z.x), gq[0]);
                    gq[1] = __builtin_fmaf(kw, nca::bf16_hi(z.x), gq[1]);
                    gq[2] = __builtin_fmaf(kw, nca::bf16_lo(z.y), gq[2]);
                    gq[3] = __builtin_fmaf(kw, nca::bf16_hi(z.y), gq[3]);
                }
            }
            gx_st(mt, cq, make_float4(gq[0], gq[1], gq[2], gq[3]));
        }
    };
    __syncthreads();

    // The head terms of the chunk's tile G (tiles numbered across the chunk's steps, tile tt of
    // the si-th step processed is G = si ntile + tt) go to FI buffer G % 3, a row of 12 floats per
    // cell: gl = d loss / d logits (0-3), the output channels xo (4-7) and the loss term (8), zero
    // for cells past the workgroup's, and 1 (9). The first z wave computes them two tiles at a time ahead
    // of the front (lanes 0-31: cells of tile G + 1, lanes 32-63: of tile G + 2, in the tiles
    // G = 0, 2, 4, ...); the front reads gl, the second z wave sums the loss and the head's
    // gradient products gl[v] xo[c]. The inputs are loaded first (head_load, raw: nothing selects
    // on a load when it is issued, so the compiler waits for them only at their use in
    // head_terms; an absent tensor loads another element of the step's state instead, which the
    // use ignores).
    const int ntile = (nw + 31) / 32;
    struct HeadIn {
        float xo[4], mk;
        int tgt;
    };
    auto head_load = [&](int ts, int tt) {
        HeadIn hi;
        const int j = (tid - FT) & 31, mt = 32 * tt + j;
        const int q = r0 * W + (mt < nw ? mt : 0);
        const int64_t m = mb + q;
        const float *xs1 = A.states + (int64_t)(ts + 1) * A.stride + xb;
#pragma unroll
        for (int c = 0; c < 4; ++c) hi.xo[c] = xs1[(int64_t)(d.out_off + (c < d.c_out ? c : 0)) * HW + q];
        hi.tgt = *(A.fa.targets ? A.fa.targets + m : reinterpret_cast<const int32_t *>(xs1 + q));
        hi.mk = *(A.fa.mask ? A.fa.mask + m : xs1 + q);
        return hi;
    };
    auto head_terms = [&](const HeadIn &hi, int ts, int tt, int fb) {
        const int j = (tid - FT) & 31;
        const bool ok = 32 * tt + j < nw;
        float xo[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) xo[c] = c < d.c_out ? hi.xo[c] : 0.0f;
        const int tgt = A.fa.targets ? hi.tgt : 0;  // no targets: a step without a loss term
        const float mk = A.fa.mask ? hi.mk : 0.0f;
        float gl[4];
        const float lc =
            head_grad_core<4>(d, A.wscale[ts], A.fa.mask != nullptr, A.fa.denom, hwL, hwL + 16, xo, tgt, mk, gl);
        float *fi = fiL + fb * 384 + j * 12;
        const float4 z4 = make_float4(0.f, 0.f, 0.f, 0.f);
        *reinterpret_cast<float4 *>(fi) = ok ? make_float4(gl[0], gl[1], gl[2], gl[3]) : z4;
        *reinterpret_cast<float4 *>(fi + 4) = ok ? make_float4(xo[0], xo[1], xo[2], xo[3]) : z4;
        fi[8] = ok ? lc : 0.0f;
        fi[9] = 1.0f;  // the factor of the sums that are not products
    };
    // the Philox fire bits of step ts for the workgroup's cells into FB buffer ts & 1, one
    // evaluation per 4 cells of the board (the uniforms of cells 4 g4 .. 4 g4 + 3); threads
    // [t0, t0 + nt)
    const unsigned fbs = ((unsigned)nw + 15u) & ~15u;
    auto fire_bits = [&](int ts, int t0, int nt) {
        const int qa = r0 * W, qe = qa + nw;
        const uint64_t key = A.fa.key_ptr ? A.fa.key_ptr[ts] : A.fa.key;
        unsigned char *fo = fbL + (unsigned)(ts & 1) * fbs;
        for (int g4 = (qa >> 2) + tid - t0; g4 < (qe + 3) >> 2; g4 += nt) {
            float u[4];
            nca::cell_uniforms4(key, (uint32_t)(A.fa.row0 + board), A.fa.step + (uint32_t)ts, (uint32_t)g4, u);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int q = 4 * g4 + e;
                if (q >= qa && q < qe) fo[q - qa] = u[e] < A.fa.p ? 1 : 0;
            }
        }
    };
    int G = 0;  // the chunk's tile in progress
    for (int t = A.n - 1; t >= 0; --t) {
        asm volatile("" : "+v"(tid));
        lane = tid & 63;
        r = lane & 15;
        g = lane >> 4;
        // ---- x_t of rows r0 - 1 .. r1 and columns -1 .. W into XS; on the chunk's last step the
        // head terms of its tile 0 and its fire bits (later steps get theirs during the step after)
        if (t == A.n - 1) {
            if (tid >= FT && tid < FT + 32) head_terms(head_load(t, 0), t, 0, 0);
            if (!A.fa.fire_u8) fire_bits(t, 0, kFusedThreads);
        }
        for (int e0 = tid; e0 < xs_items; e0 += XSU * kFusedThreads) {
            xs_load(t, e0);
            xs_store(e0);
        }
        __syncthreads();

        // ---- the workgroup's cells in tiles of 32. The front's per-cell inputs from global memory
        // (given, injected fire) are loaded one tile ahead, so their latency passes during the
        // previous tile's MLP
        struct FrontIn {
            uint32_t gv, fb;
        };
        FrontIn fin;
        auto front_load = [&](int tl, FrontIn &fi) {
            const int j = tid & 31;
            const int mt = 32 * tl + j, mtc = mt < nw ? mt : 0;
            const int64_t m = mb + r0 * W + mtc;
            fi.gv = A.fa.given[m];
            fi.fb = A.fa.fire_u8 ? A.fa.fire_u8[(int64_t)t * d.rows * HW + m] : 0u;
        };
        if (tid < FT) front_load(0, fin);
        for (int tl = 0; tl < ntile; ++tl) {
            asm volatile("" : "+v"(tid));
            lane = tid & 63;
            r = lane & 15;
            g = lane >> 4;
            if (tid < FT) {
                // front: thread (cell j of the tile, channel group oc of FCH channels)
                const int j = tid & 31, oc = tid >> 5;
                const int mt = 32 * tl + j;
                const bool ok = mt < nw;
                const int mtc = ok ? mt : 0;
                const int q = r0 * W + mtc;
                float gi[FCH];
                if (t == A.n - 1) {
#pragma unroll
                    for (int u = 0; u < FCH; ++u)
                        gi[u] = A.grad_final ? A.grad_final[xb + (int64_t)(FCH * oc + u) * HW + q] : 0.0f;
                } else {
#pragma unroll
                    for (int h = 0; h < FCH / 4; ++h) {
                        const float4 v = gx_ld(mtc, FCH / 4 * oc + h);
                        gi[4 * h] = v.x;
                        gi[4 * h + 1] = v.y;
                        gi[4 * h + 2] = v.z;
                        gi[4 * h + 3] = v.w;
                    }
                }
                const bool gv = fin.gv != 0;
                const uint32_t fbyte = fin.fb;
                if (tl + 1 < ntile) front_load(tl + 1, fin);
                const float f = (A.fa.fire_u8 ? fbyte : (uint32_t)fbL[(unsigned)(t & 1) * fbs + mtc]) ? 1.0f : 0.0f;
                // d loss / d logits of the cell, from the head terms of this tile
                const float4 glv = *reinterpret_cast<const float4 *>(fiL + (G % 3) * 384 + j * 12);
                const float gl[4] = {glv.x, glv.y, glv.z, glv.w};
                const unsigned pg = (unsigned)((j & 15) >> 2), pj = (unsigned)((j & 3) + 4 * (j >> 4));
#pragma unroll
                for (int h = 0; h < FCH / 4; ++h) {
                    float gu[4];
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        const int c = FCH * oc + 4 * h + u;
                        float gg = gi[4 * h + u];
                        const int co = c - d.out_off;
                        if (co >= 0 && co < d.c_out) {
#pragma unroll
                            for (int v = 0; v < 4; ++v)
                                if (v < d.n_out) gg = __builtin_fmaf(hwL[v * d.c_out + co], gl[v], gg);
                        }
                        if (gv && c >= d.in_off && c < d.in_off + d.c_in) gg = 0.0f;
                        gu[u] = gg;
                        // g_dx (bf16: the gradient of the bf16 tensor dx) into row c of the MLP
                        // operand, cell j at its place in the perm order
                        const float gd = ok ? nca::round_bf16(gg * f) : 0.0f;
                        *reinterpret_cast<__bf16 *>(ms + S::GB + mb_off((unsigned)c, pg) + 2u * pj) = (__bf16)gd;
                    }
                    if (ok) gx_st(mt, FCH / 4 * oc + h, make_float4(gu[0], gu[1], gu[2], gu[3]));
                }
            } else {
                // z of the tile as the forward computes it, on v_mfma_f32_4x4x4_16b_bf16: block
                // bz = (cell group m, channel octet o) of the two z waves; its row i is cell 4 m + i,
                // whose lane loads the 9 taps of the octet; per channel c the taps 0-3, 4-7 (bf16
                // pairs) and tap 8 (with its quad, kernel weight in slot c % 4) take one MFMA
                // each. Output lane (block, kernel k) holds z of the group's 4 cells.
                const int u = tid - FT;
                // the first z wave, in the tiles G = 0, 2, 4, ...: the head terms of tiles G + 1
                // (lanes 0-31) and G + 2 (lanes 32-63), inputs loaded now and used after the z work
                const int hG = G + 1 + (u >> 5), hsi = hG / ntile;
                const int hts = A.n - 1 - hsi, htt = hG - hsi * ntile;
                const bool head_now = u < 64 && (G & 1) == 0 && hts >= 0;
                HeadIn hin;
                if (head_now) hin = head_load(hts, htt);
                if (u >= 64 && tl == 0 && t > 0 && !A.fa.fire_u8)
                    fire_bits(t - 1, FT + 64, 64);  // the second z wave: the next step's fire bits
                const int bz = u >> 2, m = bz & 7, o = bz >> 3;
                const int jc = 32 * tl + 4 * m + (u & 3), mc = jc < nw ? jc : 0;
                const int pr = mc / W, col = mc - pr * W;
                uint4 tq[9];
#pragma unroll
                for (int tp = 0; tp < 9; ++tp)
                    tq[tp] = *reinterpret_cast<const uint4 *>(
                        smem + A.l_XS + (unsigned)(((pr + tp / 3) * W2 + col + tp % 3) * 64 + 16 * o));
                auto word = [&](const uint4 &v, int c) -> uint32_t {
                    const int wd = c >> 1;
                    return wd == 0 ? v.x : wd == 1 ? v.y : wd == 2 ? v.z : v.w;
                };
                const int kz = u & 3;
                const unsigned zrow0 = (unsigned)(32 * kz + 8 * o);
                const unsigned zcol = 8u * (unsigned)(m >> 2);
                const int jv = 32 * tl + 4 * m;  // the group's first tile cell
#pragma unroll
                for (int c = 0; c < 8; ++c) {
                    const uint32_t sel = (c & 1) ? 0x07060302u : 0x05040100u;
                    const nca::s16x4 sa0 = __builtin_bit_cast(
                        nca::s16x4, make_uint2(__builtin_amdgcn_perm(word(tq[1], c), word(tq[0], c), sel),
                                               __builtin_amdgcn_perm(word(tq[3], c), word(tq[2], c), sel)));
                    const nca::s16x4 sa1 = __builtin_bit_cast(
                        nca::s16x4, make_uint2(__builtin_amdgcn_perm(word(tq[5], c), word(tq[4], c), sel),
                                               __builtin_amdgcn_perm(word(tq[7], c), word(tq[6], c), sel)));
                    const nca::s16x4 a2 =
                        __builtin_bit_cast(nca::s16x4, c < 4 ? make_uint2(tq[8].x, tq[8].y) : make_uint2(tq[8].z, tq[8].w));
                    nca::f32x4 dz = {0.f, 0.f, 0.f, 0.f};
                    dz = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(sa0, kzb0, dz, 0, 0, 0);
                    dz = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(sa1, kzb1, dz, 0, 0, 0);
                    dz = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(a2, kzb2[c & 3], dz, 0, 0, 0);
#pragma unroll
                    for (int i = 0; i < 4; ++i) dz[i] = jv + i < nw ? dz[i] : 0.0f;
                    nca::lds_st64(smem, A.l_MLP + S::ZB + mb_off(zrow0 + (unsigned)c, (unsigned)(m & 3)) + zcol,
                                  make_uint2(nca::cvt_pk_bf16(dz[0], dz[1]), nca::cvt_pk_bf16(dz[2], dz[3])));
                }
                if (head_now) head_terms(hin, hts, htt, hG % 3);
                // this tile's loss and head terms (FI buffer G % 3), summed by the second z wave
                // and added to the chunk's sums in tile order: term uu is the loss (0), a product
                // gl[v] xo[c] (1 + 4 v + c) or gl[v] (17 + v) (a product with the row's 1); lane
                // 3 uu + sg sums the cells 11 sg .. 11 sg + 10 of the tile, lane 3 uu adds the three
                // partial sums in order
                if (u >= 64) {
                    const int u3 = u - 64, uu = u3 / 3, sg = u3 - 3 * uu;
                    const int ea = uu == 0 ? 8 : (uu <= 16 ? (uu - 1) >> 2 : uu - 17);
                    const int eb = uu >= 1 && uu <= 16 ? 4 + ((uu - 1) & 3) : 9;
                    const float *fp = fiL + (G % 3) * 384 + 11 * sg * 12;
                    const int nseg = sg < 2 ? 11 : 10;
                    float sacc = 0.0f;
#pragma unroll
                    for (int jj = 0; jj < 11; ++jj)
                        if (jj < nseg) sacc = __fadd_rn(sacc, __fmul_rn(fp[jj * 12 + ea], fp[jj * 12 + eb]));
                    const float p1 = __shfl(sacc, (lane + 1) & 63), p2 = __shfl(sacc, (lane + 2) & 63);
                    if (sg == 0 && uu < 21) hacc[uu] = __fadd_rn(hacc[uu], __fadd_rn(__fadd_rn(sacc, p1), p2));
                }
            }
            __syncthreads();

            // ---- MLP backward of the tile (mlp_back32's tile body, two virtual waves)
            nca::bf16x8 zf[4][2], gf[2];
#pragma unroll
            for (int kb = 0; kb < 4; ++kb)
#pragma unroll
                for (int ct = 0; ct < 2; ++ct) {
                    const unsigned zo = S::ZB + 32u * S::RS * kb + 8u * ct;
                    zf[kb][ct] = mb_cat(mb_ldtr(ms, zo + o_tr0), mb_ldtr(ms, zo + o_tr1));
                }
#pragma unroll
            for (int ct = 0; ct < 2; ++ct)
                gf[ct] = mb_cat(mb_ldtr(ms, S::GB + 8u * ct + o_tr0), mb_ldtr(ms, S::GB + 8u * ct + o_tr1));
            const float *b1L = reinterpret_cast<const float *>(ms + S::B1);
#pragma unroll
            for (int hb = 0; hb < NH; ++hb) {
                const int vw = NH * w + hb;
                // fc1: hT[ct][ht] = D[cell 16ct+4g+i][hid 32vw+16ht+r]
                mb_f32x4 hT[2][2];
#pragma unroll
                for (int x = 0; x < 2; ++x)
#pragma unroll
                    for (int y = 0; y < 2; ++y) hT[x][y] = mb_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
                    for (int ht = 0; ht < 2; ++ht) {
                        hT[0][ht] = mb_mfma(zf[kb][0], w1f[hb][ht][kb], hT[0][ht]);
                        hT[1][ht] = mb_mfma(zf[kb][1], w1f[hb][ht][kb], hT[1][ht]);
                    }
                }
#pragma unroll
                for (int ht = 0; ht < 2; ++ht) {
                    const float bt = b1L[32 * vw + 16 * ht + r];
#pragma unroll
                    for (int ct = 0; ct < 2; ++ct)
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            const float vt = nca::round_bf16(__fadd_rn(hT[ct][ht][i], bt));
                            hT[ct][ht][i] = vt > 0.0f ? vt : 0.0f;
                        }
                }
                // g_a = bf16(W2^T g_dx) * [h > 0]
                mb_f32x4 gaT[2][2];
#pragma unroll
                for (int ct = 0; ct < 2; ++ct)
#pragma unroll
                    for (int ht = 0; ht < 2; ++ht) gaT[ct][ht] = mb_mfma(gf[ct], w2f[hb][ht], mb_f32x4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
                for (int x = 0; x < 2; ++x)
#pragma unroll
                    for (int y = 0; y < 2; ++y)
#pragma unroll
                        for (int i = 0; i < 4; ++i)
                            gaT[x][y][i] = hT[x][y][i] > 0.0f ? nca::round_bf16(gaT[x][y][i]) : 0.0f;
#pragma unroll
                for (int ht = 0; ht < 2; ++ht)
#pragma unroll
                    for (int ct = 0; ct < 2; ++ct)
#pragma unroll
                        for (int i = 0; i < 4; ++i) db1[hb][ht] = __fadd_rn(db1[hb][ht], gaT[ct][ht][i]);
                nca::bf16x8 ap[2];
#pragma unroll
                for (int ht = 0; ht < 2; ++ht) {
                    const float v[8] = {gaT[0][ht][0], gaT[0][ht][1], gaT[0][ht][2], gaT[0][ht][3],
                                        gaT[1][ht][0], gaT[1][ht][1], gaT[1][ht][2], gaT[1][ht][3]};
                    ap[ht] = nca::mb_pack8(v);
                }
#pragma unroll
                for (int ht = 0; ht < 2; ++ht) {
                    const uint4 uu = __builtin_bit_cast(uint4, ap[ht]);
                    const unsigned row = 32u * (unsigned)vw + 16u * ht + (unsigned)r;
#pragma unroll
                    for (int ct = 0; ct < 2; ++ct)
                        *reinterpret_cast<uint2 *>(ms + S::GL + mb_off(row, 2u * ct + ((unsigned)g >> 1)) + 8u * (g & 1)) =
                            ct ? make_uint2(uu.z, uu.w) : make_uint2(uu.x, uu.y);
                }
                // dW2 += g_dx h^T
                {
                    nca::bf16x8 hbv[2];
#pragma unroll
                    for (int ht = 0; ht < 2; ++ht) {
                        const float v[8] = {hT[0][ht][0], hT[0][ht][1], hT[0][ht][2], hT[0][ht][3],
                                            hT[1][ht][0], hT[1][ht][1], hT[1][ht][2], hT[1][ht][3]};
                        hbv[ht] = nca::mb_pack8(v);
                    }
#pragma unroll
                    for (int ct = 0; ct < 2; ++ct) {
                        const nca::bf16x8 gbv = mb_ld(ms, S::GB + 16u * S::RS * ct + o_rg);
#pragma unroll
                        for (int ht = 0; ht < 2; ++ht) dw2[hb][ct][ht] = mb_mfma(gbv, hbv[ht], dw2[hb][ct][ht]);
                        // db2 = g_dx times a column of ones (exact products): wave 0, once a tile
                        if (hb == 0 && w == 0) db2m[ct] = mb_mfma(gbv, ones8, db2m[ct]);
                    }
                }
                pin_dw2();
                asm volatile("" : "+a"(db2m[0]), "+a"(db2m[1]));
                // dW1 += g_a z^T
#pragma unroll
                for (int ft = 0; ft < 8; ft += 2) {
                    const nca::bf16x8 zb0 = mb_ld(ms, S::ZB + 16u * S::RS * ft + o_rg);
                    const nca::bf16x8 zb1 = mb_ld(ms, S::ZB + 16u * S::RS * (ft + 1) + o_rg);
#pragma unroll
                    for (int ht = 0; ht < 2; ++ht) {
                        dw1[hb][ht][ft] = mb_mfma(ap[ht], zb0, dw1[hb][ht][ft]);
                        dw1[hb][ht][ft + 1] = mb_mfma(ap[ht], zb1, dw1[hb][ht][ft + 1]);
                    }
                }
            }
            __syncthreads();
            // ---- g_z = bf16(W1^T g_a): features 16 vw + 4g + i of cells 16ct + r; the g_a
            // operands of a hidden block serve both virtual waves
            {
                mb_f32x4 gz[NH][2][2];  // [hb][ct][kb & 1]
#pragma unroll
                for (int hb = 0; hb < NH; ++hb)
#pragma unroll
                    for (int x = 0; x < 2; ++x)
#pragma unroll
                        for (int y = 0; y < 2; ++y) gz[hb][x][y] = mb_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int kb = 0; kb < 8; ++kb) {
                    const unsigned bo = S::GL + 32u * S::RS * kb;
                    const nca::bf16x8 B0 = mb_cat(mb_ldtr(ms, bo + o_gl[0][0]), mb_ldtr(ms, bo + o_gl[0][1]));
                    const nca::bf16x8 B1 = mb_cat(mb_ldtr(ms, bo + o_gl[1][0]), mb_ldtr(ms, bo + o_gl[1][1]));
#pragma unroll
                    for (int hb = 0; hb < NH; ++hb) {
                        gz[hb][0][kb & 1] = mb_mfma(w1t[hb][kb], B0, gz[hb][0][kb & 1]);
                        gz[hb][1][kb & 1] = mb_mfma(w1t[hb][kb], B1, gz[hb][1][kb & 1]);
                    }
                }
                // features 16 vw + 4 g + i: plane vw / 2, channels 16 (vw & 1) + 4 g + i
#pragma unroll
                for (int hb = 0; hb < NH; ++hb) {
                    const int vw = NH * w + hb, kp = vw >> 1, c0 = 16 * (vw & 1) + 4 * g;
#pragma unroll
                    for (int ct = 0; ct < 2; ++ct) {
                        const int mt = 32 * tl + 16 * ct + r;
                        if (mt < nw) {
                            const int pr = mt / W, col = mt - pr * W;
                            const uint2 v = make_uint2(
                                nca::cvt_pk_bf16(__fadd_rn(gz[hb][ct][0][0], gz[hb][ct][1][0]),
                                                 __fadd_rn(gz[hb][ct][0][1], gz[hb][ct][1][1])),
                                nca::cvt_pk_bf16(__fadd_rn(gz[hb][ct][0][2], gz[hb][ct][1][2]),
                                                 __fadd_rn(gz[hb][ct][0][3], gz[hb][ct][1][3])));
                            if (PIECES)
                                nca::lds_st64(smem, gz_lds(kp, pr, col, c0), v);
                            else
                                *reinterpret_cast<uint2 *>(gz_glb(kp, pr, col, c0)) = v;
                        }
                    }
                }
            }
            ++G;
        }
        __syncthreads();  // g_z of every cell of the workgroup is stored

        // ---- the kernel-weight sums dk[k][tap] += sum over channels of g_z[k][c] x_tap[c]: one
        // v_mfma_f32_16x16x32_bf16 per cell (A rows k < 4 of g_z, k over the 32 channels; B
        // columns tap < 9 of XS; products of bf16 values, exact), cells strided over the waves;
        // lane (tap n, group 0) holds dk[i][n] in element i
        auto dk_operands = [&](int mt, nca::bf16x8 &za, nca::bf16x8 &xbv) {
            const int pr = mt / W, col = mt - pr * W;
            if (r < 4) {
                if (PIECES)
                    za = mb_ld(smem, gz_lds(r, pr, col, 8 * g));
                else
                    za = *reinterpret_cast<const nca::bf16x8 *>(gz_glb(r, pr, col, 8 * g));
            } else {
                za = __builtin_bit_cast(nca::bf16x8, make_uint4(0u, 0u, 0u, 0u));
            }
            if (r < 9)
                xbv = mb_ld(smem, A.l_XS + (unsigned)(((pr + r / 3) * W2 + col + r % 3) * 64 + 16 * g));
            else
                xbv = __builtin_bit_cast(nca::bf16x8, make_uint4(0u, 0u, 0u, 0u));
        };
        auto dk_sums = [&]() {
            for (int mt = w; mt < nw; mt += 4 * NWV) {  // four cells at a time (their loads together)
                nca::bf16x8 za[4], xq[4];
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    if (mt + k * NWV < nw) dk_operands(mt + k * NWV, za[k], xq[k]);
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    if (mt + k * NWV < nw) dkw = mb_mfma(za[k], xq[k], dkw);
            }
        };
        if (PIECES) {
            // ---- exchange: side 0 is the piece's first row, side 1 its last; the piece above
            // sends its last row (into row -1), the piece below its first (into row Hw)
            const bool up = piece > 0 || wrap, down = piece < P - 1 || wrap;
            const int nup = piece > 0 ? piece - 1 : P - 1, ndn = piece < P - 1 ? piece + 1 : 0;
            const int NE = 64 * W;  // words of a row: 4 planes x W cells x 16 channel pairs
            const uint32_t tag = (uint32_t)(t + 1);
            auto slot = [&](int pc, int side) -> uint64_t * {
                return A.xch + ((((int64_t)board * P + pc) * 2 + side) * 2 + (t & 1)) * NE;
            };
            auto word_at = [&](int ee, int pr) -> unsigned {  // LDS offset of word ee of workgroup row pr
                const int k = ee / (16 * W), rem = ee - k * 16 * W, col = rem >> 4, cp = rem & 15;
                return gz_lds(k, pr, col, 2 * cp);
            };
            for (int e = tid; e < 2 * NE; e += kFusedThreads) {
                const int side = e >= NE ? 1 : 0, ee = e - side * NE;
                if (side ? !down : !up) continue;
                const uint32_t v = *reinterpret_cast<const uint32_t *>(smem + word_at(ee, side ? Hw - 1 : 0));
                __hip_atomic_store(slot(piece, side) + ee, ((uint64_t)tag << 32) | v, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
            }
            // the interior rows' g_x and the kernel-weight sums need no neighbour's row: they run
            // while their rows arrive
            if (Hw > 2) gx_rows(1, Hw - 1);
            dk_sums();
            // receive: at most 4096 words (2 NE, W <= 32, checked by the host), in passes of 8 a
            // thread; the words of a pass are loaded together, and all of them again
            // while one is stale
            const uint64_t *src_up = slot(nup, 1), *src_dn = slot(ndn, 0);
            const uint32_t want = tag + (uint32_t)A.tag_skew;
            auto need = [&](int e) { return e < 2 * NE && (e >= NE ? down : up); };
#pragma unroll
            for (int pass = 0; pass < (2 * 64 * 32 + 8 * kFusedThreads - 1) / (8 * kFusedThreads); ++pass) {
                uint64_t hw[8];
                auto load_words = [&]() {
#pragma unroll
                    for (int kk = 0; kk < 8; ++kk) {
                        const int e = tid + kFusedThreads * (8 * pass + kk);
                        const uint64_t *sp = e >= NE ? src_dn + (e - NE) : src_up + e;
                        hw[kk] = need(e) ? __hip_atomic_load(sp, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0;
                    }
                };
                load_words();
                for (int nspin = 0; !hfail; ++nspin) {
                    bool any = false;
#pragma unroll
                    for (int kk = 0; kk < 8; ++kk)
                        any |= need(tid + kFusedThreads * (8 * pass + kk)) && (uint32_t)(hw[kk] >> 32) != want;
                    if (!any) break;
                    if (nspin >= A.spin_limit) {
                        hfail = true;
                        __hip_atomic_fetch_or(A.status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        break;
                    }
                    __builtin_amdgcn_s_sleep(2);
                    load_words();
                }
#pragma unroll
                for (int kk = 0; kk < 8; ++kk) {
                    const int e = tid + kFusedThreads * (8 * pass + kk);
                    if (need(e)) {
                        const int side = e >= NE ? 1 : 0, ee = e - side * NE;
                        *reinterpret_cast<uint32_t *>(smem + word_at(ee, side ? Hw : -1)) = (uint32_t)hw[kk];
                    }
                }
            }
            __syncthreads();
            gx_rows(0, 1);
            if (Hw > 1) gx_rows(Hw - 1, Hw);
        } else {
            gx_rows(0, Hw);
            dk_sums();
        }
        asm volatile("" : "+a"(dkw));
        __syncthreads();
    }

    // ---- the kernel-weight sums of the waves, added in wave order
    if (g == 0 && r < 9) {
#pragma unroll
        for (int i = 0; i < 4; ++i) redL[w * 36 + i * 9 + r] = dkw[i];
    }
    __syncthreads();
    if (tid < 36) {
        float v = redL[tid];
        for (int ww = 1; ww < NWV; ++ww) v = __fadd_rn(v, redL[ww * 36 + tid]);
        dkacc[tid] = v;
    }
    __syncthreads();

    // ---- the gradient of the chunk's first state
    if (A.grad_x0) {
        for (int e = tid; e < 32 * nw; e += kFusedThreads) {
            const int c = e / nw, mt = e - c * nw;
            float v;
            if (PIECES)
                v = reinterpret_cast<const float *>(smem + A.l_GX)[mt * 32 + c];
            else
                v = A.gx_g[(mb + mt) * 32 + c];
            A.grad_x0[xb + (int64_t)c * HW + r0 * W + mt] = v;
        }
    }
    // ---- the chunk's sums into slot blockIdx.x
    float *ps = A.part + (int64_t)blockIdx.x * A.P;
#pragma unroll
    for (int hb = 0; hb < NH; ++hb) {
        const int vw = NH * w + hb;
#pragma unroll
        for (int ht = 0; ht < 2; ++ht)
#pragma unroll
            for (int ft = 0; ft < 8; ++ft)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    ps[A.offW1 + (32 * vw + 16 * ht + 4 * g + i) * 128 + 16 * ft + r] = dw1[hb][ht][ft][i];
#pragma unroll
        for (int ct = 0; ct < 2; ++ct)
#pragma unroll
            for (int ht = 0; ht < 2; ++ht)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    ps[A.offW2 + (16 * ct + 4 * g + i) * 256 + 32 * vw + 16 * ht + r] = dw2[hb][ct][ht][i];
#pragma unroll
        for (int ht = 0; ht < 2; ++ht) {
            float v = db1[hb][ht];
            v = __fadd_rn(v, __shfl_xor(v, 16));
            v = __fadd_rn(v, __shfl_xor(v, 32));
            if (g == 0) ps[A.offB1 + 32 * vw + 16 * ht + r] = v;
        }
    }
    if (tid < 36) ps[A.offK + tid] = dkacc[tid];
    if (w == 0 && r == 0) {
#pragma unroll
        for (int ct = 0; ct < 2; ++ct)
#pragma unroll
            for (int i = 0; i < 4; ++i) ps[A.offB2 + 16 * ct + 4 * g + i] = db2m[ct][i];
    }
    if (tid < d.n_out * d.c_out) ps[A.offHW + tid] = hacc[1 + (tid / d.c_out) * 4 + tid % d.c_out];
    if (tid < d.n_out) ps[A.offHB + tid] = hacc[17 + tid];
    if (tid == 0) A.lossacc[blockIdx.x] = hacc[0];
    // the repair: the slots of the pieces' launch beyond this launch's
    for (int s = (int)gridDim.x + (int)blockIdx.x; s < A.zero_slots; s += (int)gridDim.x) {
        float *pz = A.part + (int64_t)s * A.P;
        for (int64_t e = tid; e < A.P; e += kFusedThreads) pz[e] = 0.0f;
        if (tid == 0) A.lossacc[s] = 0.0f;
    }
}

}  // namespace
