// The LDS-resident multi-step rollout kernel (gfx950).
//
// One workgroup of 4 waves owns `rows_per_wg` rows (rollouts) for the whole call: their states
// are loaded from HBM once, advanced `n_steps` steps inside LDS and written back once. One step
// of the reference cell (src/nca/model.py:503-559) is computed over tiles of 16 cells:
//
//   stencil  all lanes: z[cell][k*C + c] = sum_taps kern[k][tap] * P[nbr(cell, tap)][c] from
//            the perception buffer P (LDS, 1-cell halo) into Z (LDS). bf16 cells use
//            v_dot2_f32_bf16 on tap pairs; fp32 cells use fp32 FMAs.
//   fc1      wave w owns hidden units [w*HD/4, (w+1)*HD/4): h^T = W1 z^T on MFMA with its W1
//            fragments resident in registers (A operand) and z^T read from Z (B operand); bias
//            (accumulator init) and ReLU fused, h written to H (LDS).
//   fc2      wave w owns output channels [16w, 16w+16) (C/16 m-tiles spread over the waves):
//            dx^T = W2 h^T with register-resident W2 fragments.
//   update   in the fc2 accumulator layout (lane: 4 consecutive channels of one cell):
//            u = x + fire * dx (+ noise); input-slice channels of given cells are frozen at
//            their clamp value; written to the fp32 state and the other perception buffer.
//
// fp32 cells with C = 16 (one fc2 m-tile) split the work otherwise: each wave runs fc2 over its
// own hidden units from its fc1 registers, the update adds the four partial sums, and the
// stencil's kernel k runs on wave k (see KSPLIT below).
//
// Software pipeline: Z and H are double-buffered so that one barrier interval holds fc2 and the
// update of tile t-1, fc1 of tile t and the stencil of tile t+1 - MFMA and VALU work of the same
// wave that the hardware overlaps - with a single workgroup barrier per tile.
//
// The fire mask of a step is drawn once for all cells (Philox, or read from injected masks);
// adaptive firing reads the pre-step confidence first. With wrap padding the halo of the new
// perception buffer is refreshed after each step; wall / zero halos are constant. The board
// confidence of the final state is computed in-kernel.
//
// Clamp: the first step of a launch resets the input slice of given cells to the clamp values
// (model.py:430-438); the state then holds exactly those values, so later steps keep them by
// not updating those channels, which is bitwise the same as clamping again.
//
// Precision: BF16 reproduces bf16 autocast (perception input, z, h, dx rounded to bf16, fp32
// accumulation, fp32 state in a separate buffer M); fp32 keeps everything fp32 and uses
// v_mfma_f32_16x16x4_f32 (the perception buffer is then the state itself).
#pragma once

#include "nca_device.h"
#include "nca_layout.h"

namespace nca {

struct RolloutParams {
    const float *x_in;
    float *x_out;
    const uint8_t *given;
    const float *clamp;
    const unsigned char *packed;
    const uint8_t *fire_u8;      // injected masks (n_steps, rows, HW), or null
    const float *fire_f32;       // injected mask of a single step (rows, HW), or null
    const float *noise;          // (rows, C, HW), single step only, or null
    const uint64_t *step_seeds;  // (n_steps) or null
    float *conf_out;
    int32_t *fired_out;
    float *x_rec;        // or null: the state after step s of the call goes to x_rec + s rec_stride
    int64_t rec_stride;  // (the streamed C = 32 kernel only)
    float *x_rec0;       // or null: the call's input state copied there (the same kernel, with x_rec)
    int64_t rows;
    int H, W;
    int c_in, in_off, c_out, out_off, n_out, head_kind, padding;
    uint64_t seed;
    int64_t row0, step0;
    int n_steps;
    float p, p_low, tau;
    int adaptive, given_confident;
    int rows_per_wg;
    unsigned off_kern, off_b1, off_b2, off_headw, off_headb, off_padv, off_w1, off_w2, off_w2h, off_w1q, off_w2k;
    unsigned l_P, l_M, l_Z, l_H, l_clamp, l_given, l_fire, l_conf, l_fired, l_head, l_cinfo;
};

template <int C, int HD, bool BF16>
struct Shape {
    static constexpr int NH = 4;            // perception kernels
    static constexpr int F = NH * C;        // features
    static constexpr int NW = 4;            // waves per workgroup
    static constexpr int NT = NW * 64;      // threads
    static constexpr int KT = BF16 ? 32 : 4;  // MFMA k per instruction
    static constexpr int HPW = HD / NW;     // hidden units per wave
    static constexpr int MT1 = HPW / 16;    // fc1 m-tiles per wave
    static constexpr int KT1 = F / KT;      // fc1 k-tiles
    static constexpr int MT2 = C / 16;      // fc2 m-tiles (all waves)
    static constexpr int MT2W = (MT2 + NW - 1) / NW;  // fc2 m-tiles per wave (max)
    static constexpr int KT2 = HD / KT;     // fc2 k-tiles
    static constexpr int ES = BF16 ? 2 : 4;  // bytes per element of P, Z, H
    static constexpr int CP = C + 4;        // P channel stride (elements)
    static constexpr int MP = C + 4;        // M channel stride (floats)
    static constexpr int ZS = F + (BF16 ? 8 : 4);   // Z row stride (elements)
    static constexpr int HS = HD + (BF16 ? 8 : 4);  // H row stride (elements)
    static constexpr int ZBUF = 16 * ZS;    // elements per Z buffer
    static constexpr int HBUF = 16 * HS;    // elements per H buffer
    static constexpr int NSI = 16 * (C / 4);  // stencil items per tile (16 cells x C/4 quads)
    static_assert(HD % 64 == 0, "hidden must be a multiple of 64");
    static_assert(C % 16 == 0 && C <= 64, "channels must be 16, 32, 48 or 64");
    static_assert(NSI <= NT, "stencil items exceed the workgroup");
};

// LDS plan for R rows of an H x W grid.
struct LdsPlan {
    unsigned P, M, Z, H, clamp, given, fire, conf, fired, head, cinfo, total;
};

template <int C, int HD, bool BF16>
inline LdsPlan lds_plan(int R, int H, int W, int c_in, int c_out, int n_out) {
    using S = Shape<C, HD, BF16>;
    const unsigned hw = (unsigned)H * W, hwp = (unsigned)(H + 2) * (W + 2);
    auto al = [](unsigned v) { return (v + 15u) & ~15u; };
    LdsPlan p;
    unsigned o = 0;
    p.P = o;
    o = al(o + 2u * R * hwp * S::CP * S::ES);
    p.M = o;
    o = al(o + (BF16 ? (unsigned)R * hw * S::MP * 4u : 0u));
    p.Z = o;
    o = al(o + 2u * S::ZBUF * S::ES);
    p.H = o;
    o = al(o + 2u * S::HBUF * S::ES);
    p.clamp = o;
    o = al(o + (unsigned)R * hw * c_in * 4u);
    p.given = o;
    o = al(o + (unsigned)R * hw);
    p.fire = o;
    o = al(o + (unsigned)R * hw * 4u);
    p.conf = o;
    o = al(o + (unsigned)R * hw * 4u);
    p.fired = o;
    o = al(o + (unsigned)R * 4u);
    p.head = o;
    o = al(o + (unsigned)(n_out * c_out + n_out) * 4u);
    p.cinfo = o;
    o = al(o + (unsigned)R * hw * 4u);
    p.total = o;
    return p;
}

template <bool BF16>
__device__ __forceinline__ void lds_load4(const unsigned char *base, int elem, float v[4]) {
    if constexpr (BF16) {
        const uint2 u = *reinterpret_cast<const uint2 *>(base + 2 * elem);
        v[0] = bf16_lo(u.x);
        v[1] = bf16_hi(u.x);
        v[2] = bf16_lo(u.y);
        v[3] = bf16_hi(u.y);
    } else {
        const float4 u = *reinterpret_cast<const float4 *>(base + 4 * elem);
        v[0] = u.x;
        v[1] = u.y;
        v[2] = u.z;
        v[3] = u.w;
    }
}

template <bool BF16>
__device__ __forceinline__ void lds_store4(unsigned char *base, int elem, const float v[4]) {
    if constexpr (BF16) {
        uint2 u;
        u.x = pack_bf16x2(v[0], v[1]);
        u.y = pack_bf16x2(v[2], v[3]);
        *reinterpret_cast<uint2 *>(base + 2 * elem) = u;
    } else {
        *reinterpret_cast<float4 *>(base + 4 * elem) = make_float4(v[0], v[1], v[2], v[3]);
    }
}

template <bool BF16>
struct Frag;
template <>
struct Frag<true> {
    typedef bf16x8 type;
    static __device__ __forceinline__ type load_lds(const unsigned char *base, int elem) {
        return *reinterpret_cast<const bf16x8 *>(base + 2 * elem);
    }
    static __device__ __forceinline__ f32x4 mfma(type a, type b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
    }
};
template <>
struct Frag<false> {
    typedef float type;
    static __device__ __forceinline__ type load_lds(const unsigned char *base, int elem) {
        return *reinterpret_cast<const float *>(base + 4 * elem);
    }
    static __device__ __forceinline__ f32x4 mfma(type a, type b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
    }
};

__device__ __forceinline__ bf16x2 as_bf16x2(uint32_t u) { return __builtin_bit_cast(bf16x2, u); }

template <int C, int HD, bool BF16, bool NOISE>
__global__ void __launch_bounds__(256, 1) rollout_resident(RolloutParams a) {
    using S = Shape<C, HD, BF16>;
    using FR = Frag<BF16>;
    using fr_t = typename FR::type;
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, l16 = lane & 15;
    const int H = a.H, W = a.W, HWn = H * W, Wp = W + 2, HWp = (H + 2) * Wp;
    const int Rcap = a.rows_per_wg;
    const int64_t rbase = (int64_t)blockIdx.x * Rcap;
    const int Rw = (int)((a.rows - rbase) < Rcap ? (a.rows - rbase) : Rcap);
    const int ncell = Rw * HWn;
    const int ntile = (ncell + 15) >> 4;
    const int PBUF = Rcap * HWp * S::CP;  // elements per perception buffer

    unsigned char *Pb = smem + a.l_P;
    float *M = reinterpret_cast<float *>(smem + a.l_M);
    unsigned char *Zb = smem + a.l_Z;
    unsigned char *Hb = smem + a.l_H;
    float *clampL = reinterpret_cast<float *>(smem + a.l_clamp);
    uint8_t *givenL = smem + a.l_given;
    float *fireL = reinterpret_cast<float *>(smem + a.l_fire);
    float *confL = reinterpret_cast<float *>(smem + a.l_conf);
    int *firedL = reinterpret_cast<int *>(smem + a.l_fired);
    float *headL = reinterpret_cast<float *>(smem + a.l_head);
    int *cinfo = reinterpret_cast<int *>(smem + a.l_cinfo);  // P centre element of cell g
    const int c_in = a.c_in, in_off = a.in_off;

    // ---- stencil kernels: bf16 tap pairs (bf16 cells) or floats (fp32 cells), uniform
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
    int toff[9];  // tap offsets in P elements, tap = (dy + 1) * 3 + (dx + 1)
#pragma unroll
    for (int t = 0; t < 9; ++t) toff[t] = ((t / 3 - 1) * Wp + (t % 3 - 1)) * S::CP;

    // ---- MFMA fragments and biases in registers
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

    // ---- load rows: state, clamp, given, head weights, cell table; halos
    auto pcen = [&](int r, int q) {  // P centre element (buffer 0) of cell q of row r
        const int i = q / W, j = q - i * W;
        return (r * HWp + (i + 1) * Wp + (j + 1)) * S::CP;
    };
    for (int e = tid; e < Rw * C * HWn; e += S::NT) {
        const int r = e / (C * HWn), rem = e - r * C * HWn, c = rem / HWn, q = rem - c * HWn;
        const float v = a.x_in[rbase * C * HWn + e];
        const int pe = pcen(r, q) + c;
        if constexpr (BF16) {
            M[(r * HWn + q) * S::MP + c] = v;
            reinterpret_cast<__bf16 *>(Pb)[pe] = (__bf16)v;
        } else {
            reinterpret_cast<float *>(Pb)[pe] = v;
        }
    }
    for (int e = tid; e < Rw * c_in * HWn; e += S::NT) {
        const int r = e / (c_in * HWn), rem = e - r * c_in * HWn, ci = rem / HWn, q = rem - ci * HWn;
        clampL[(r * HWn + q) * c_in + ci] = a.clamp[rbase * c_in * HWn + e];
    }
    for (int e = tid; e < ncell; e += S::NT) {
        givenL[e] = a.given[rbase * HWn + e];
        const int r = e / HWn;
        cinfo[e] = pcen(r, e - r * HWn);
    }
    for (int e = tid; e < Rcap; e += S::NT) firedL[e] = 0;
    {
        const float *hw = reinterpret_cast<const float *>(a.packed + a.off_headw);
        const float *hb = reinterpret_cast<const float *>(a.packed + a.off_headb);
        const int nw = a.n_out * a.c_out;
        for (int e = tid; e < nw + a.n_out; e += S::NT) headL[e] = e < nw ? hw[e] : hb[e - nw];
    }
    const int nhalo = 2 * Wp + 2 * H;
    auto halo_cell = [&](int h, int &ip, int &jp) {
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
    if (a.padding != 2) {  // wall / zero: constant halo in both buffers
        const float *padv = reinterpret_cast<const float *>(a.packed + a.off_padv);
        for (int e = tid; e < 2 * Rw * nhalo * C; e += S::NT) {
            const int c = e % C, rest = e / C, h = rest % nhalo, rb = rest / nhalo;
            const int r = rb % Rw, buf = rb / Rw;
            int ip, jp;
            halo_cell(h, ip, jp);
            const float v = a.padding == 1 ? padv[c] : 0.0f;
            const int pe = buf * PBUF + (r * HWp + ip * Wp + jp) * S::CP + c;
            if constexpr (BF16)
                reinterpret_cast<__bf16 *>(Pb)[pe] = (__bf16)v;
            else
                reinterpret_cast<float *>(Pb)[pe] = v;
        }
    }
    __syncthreads();
    auto wrap_halo = [&](int buf) {
        for (int e = tid; e < Rw * nhalo * (C / 4); e += S::NT) {
            const int qd = e % (C / 4), rest = e / (C / 4), h = rest % nhalo, r = rest / nhalo;
            int ip, jp;
            halo_cell(h, ip, jp);
            const int si = (ip - 1 + H) % H, sj = (jp - 1 + W) % W;
            float v[4];
            lds_load4<BF16>(Pb, buf * PBUF + (r * HWp + (si + 1) * Wp + sj + 1) * S::CP + 4 * qd, v);
            lds_store4<BF16>(Pb, buf * PBUF + (r * HWp + ip * Wp + jp) * S::CP + 4 * qd, v);
        }
    };
    if (a.padding == 2) {
        wrap_halo(0);
        __syncthreads();
    }

    // fp32 state of a cell (for readout): M in bf16 mode, the perception buffer in fp32 mode
    auto state_ptr = [&](int buf, int cell) -> const float * {
        if constexpr (BF16) {
            return M + cell * S::MP;
        } else {
            return reinterpret_cast<const float *>(Pb) + buf * PBUF + cinfo[cell];
        }
    };

    // ---- pipeline stages ------------------------------------------------------------------
    const int st_n = tid & 15, st_qd = tid >> 4;

    // centre offset of this lane's stencil cell in tile t (padding cells read a valid cell;
    // their features are never used)
    auto stencil_pc = [&](int t) {
        const int gq = t * 16 + st_n;
        return cinfo[gq < ncell ? gq : ncell - 1];
    };
    // stencil of a tile (this lane's cell centre pc) from perception buffer `cur` into Z buffer zb
    auto stencil = [&](int pc, int zb, int cur) {
        if constexpr (S::NSI < S::NT) {
            if (tid >= S::NSI) return;  // whole waves (NSI is a multiple of 64)
        }
        const int base = cur * PBUF + pc + 4 * st_qd;
        float acc[4][4];
        if constexpr (BF16) {
            uint2 nb[9];
#pragma unroll
            for (int t9 = 0; t9 < 9; ++t9) nb[t9] = *reinterpret_cast<const uint2 *>(Pb + 2 * (base + toff[t9]));
            uint32_t pr[5][4];  // [tap pair][channel]: (bf16 of tap 2p, bf16 of tap 2p+1)
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
        for (int k = 0; k < 4; ++k) lds_store4<BF16>(Zb, zb * S::ZBUF + st_n * S::ZS + k * C + 4 * st_qd, acc[k]);
    };

    // fc1 of the tile in Z buffer zb -> H buffer hb
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

    // ---- fp32 cells with C = 16 and 128 hidden units (one fc2 m-tile): the work of a tile split
    // evenly over the four waves. fc2 is split by hidden unit: wave w's fc1 output (hidden unit
    // 32 w + 16 mt + 4 g + v of cell n in lane (g, n)) is, as it lies in the registers, the B
    // operand of fc2's k-tile (mt, v), whose A operand is W2[l16][32 w + 16 mt + 4 g + v]; the four
    // partial sums (wave 0's from b2) meet in the H region and the update adds them in wave order.
    // The stencil's kernel k runs on wave k, each output's tap chain in the order of `stencil`.
    // (Otherwise wave 0 alone ran the stencil and fc2: twice the other waves' MFMA time.)
    constexpr bool KSPLIT = !BF16 && C == 16 && HD == 128;
    float w2p[2][4], kwv[9];
    if constexpr (KSPLIT) {
        const float *w2 = reinterpret_cast<const float *>(a.packed + a.off_w2);
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
            for (int v = 0; v < 4; ++v) w2p[mt][v] = w2[(8 * wave + 4 * mt + g) * 64 + 16 * v + l16];
#pragma unroll
        for (int t9 = 0; t9 < 9; ++t9) kwv[t9] = kern[wave * 9 + t9];
    }
    float *RED = reinterpret_cast<float *>(Hb);  // [buffer][wave][cell][channel]
    // fc1 of the tile in Z buffer zb and this wave's part of fc2 -> RED buffer rb
    auto fc1_ks = [&](int zb, int rb) {
        fr_t zf[S::KT1];
#pragma unroll
        for (int kt = 0; kt < S::KT1; ++kt) zf[kt] = FR::load_lds(Zb, zb * S::ZBUF + l16 * S::ZS + kt * S::KT + g);
        f32x4 acc[S::MT1];
#pragma unroll
        for (int mt = 0; mt < S::MT1; ++mt) acc[mt] = b1v[mt];
#pragma unroll
        for (int kt = 0; kt < S::KT1; ++kt)
#pragma unroll
            for (int mt = 0; mt < S::MT1; ++mt) acc[mt] = FR::mfma(w1f[mt][kt], zf[kt], acc[mt]);
        f32x4 part = b2v[0];  // b2 on wave 0, zeros on the others
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const float h = acc[mt][v] > 0.0f ? acc[mt][v] : 0.0f;
                part = FR::mfma(w2p[mt][v], h, part);
            }
        *reinterpret_cast<float4 *>(RED + ((rb * 4 + wave) * 16 + l16) * 16 + 4 * g) =
            make_float4(part[0], part[1], part[2], part[3]);
    };
    // stencil kernel `wave` of tile t's cells (lane: cell l16, channel quad g) -> Z buffer zb
    auto stencil_ks = [&](int pc, int zb, int cur) {
        const int base = cur * PBUF + pc + 4 * g;
        float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int t9 = 0; t9 < 9; ++t9) {
            float v[4];
            lds_load4<false>(Pb, base + toff[t9], v);
#pragma unroll
            for (int c = 0; c < 4; ++c) acc[c] = __builtin_fmaf(kwv[t9], v[c], acc[c]);
        }
        lds_store4<false>(Zb, zb * S::ZBUF + l16 * S::ZS + wave * C + 4 * g, acc);
    };
    // the update of tile t from RED buffer rb: lanes 0-15 of each wave, cell 4 wave + lane / 4,
    // channel quad lane % 4
    auto update_ks = [&](int t, int rb, int cur, int nxt, bool full) {
        if (lane >= 16) return;
        const int n = 4 * wave + (lane >> 2), c0 = 4 * (lane & 3);
        const int gq = t * 16 + n, gc = gq < ncell ? gq : ncell - 1;
        const int pc = cinfo[gc];
        const float f = fireL[gc];
        const bool gv = givenL[gc] != 0;
        float xo[4];
        lds_load4<false>(Pb, cur * PBUF + pc + c0, xo);
        float4 pw[4];
#pragma unroll
        for (int w = 0; w < 4; ++w) pw[w] = *reinterpret_cast<const float4 *>(RED + ((rb * 4 + w) * 16 + n) * 16 + c0);
        float u[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const float *q0 = &pw[0].x, *q1 = &pw[1].x, *q2 = &pw[2].x, *q3 = &pw[3].x;
            const float dxv = __fadd_rn(__fadd_rn(__fadd_rn(q0[v], q1[v]), q2[v]), q3[v]);
            float uv = __fadd_rn(xo[v], __fmul_rn(f, dxv));
            if constexpr (NOISE) {
                const int r = gc / HWn;
                uv = __fadd_rn(uv, a.noise[((rbase + r) * C + c0 + v) * HWn + (gc - r * HWn)]);
            }
            const int c = c0 + v;
            u[v] = (gv && c >= in_off && c < in_off + c_in) ? xo[v] : uv;
        }
        if (full || gq < ncell) lds_store4<false>(Pb, nxt * PBUF + pc + c0, u);
    };

    // per-lane cell of the update of tile t: (cell, centre offset, fire, given)
    struct Upd {
        int gq, gc, pc;
        float f;
        bool gv;
    };
    auto upd_info = [&](int t) {
        Upd u;
        u.gq = t * 16 + l16;
        u.gc = u.gq < ncell ? u.gq : ncell - 1;
        u.pc = cinfo[u.gc];
        u.f = fireL[u.gc];
        u.gv = givenL[u.gc] != 0;
        return u;
    };
    // fc2 + update of one tile (H buffer hb), state buffers cur -> nxt. Input-slice channels of
    // given cells keep their value (the first step's clamp is applied by clamp_pass). With
    // `full` the tile has no padding cells and the stores are unconditional.
    auto fc2_update = [&](const Upd &ui, int hb, int cur, int nxt, bool full) {
#pragma unroll
        for (int jj = 0; jj < S::MT2W; ++jj) {
            const int mt2 = wave + S::NW * jj;
            if (S::MT2 % S::NW != 0 && mt2 >= S::MT2) continue;  // uniform per wave
            const int gc = ui.gc;
            const int c0 = 16 * mt2 + 4 * g;
            float xo[4];
            if constexpr (BF16) {
                const float4 m4 = *reinterpret_cast<const float4 *>(M + gc * S::MP + c0);
                xo[0] = m4.x;
                xo[1] = m4.y;
                xo[2] = m4.z;
                xo[3] = m4.w;
            } else {
                lds_load4<false>(Pb, cur * PBUF + ui.pc + c0, xo);
            }
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
                float uv = __fadd_rn(xo[v], __fmul_rn(ui.f, dxv));
                if constexpr (NOISE) {
                    const int r = gc / HWn;
                    uv = __fadd_rn(uv, a.noise[((rbase + r) * C + c0 + v) * HWn + (gc - r * HWn)]);
                }
                u[v] = (ui.gv && inslice[jj][v]) ? xo[v] : uv;
            }
            if (full || ui.gq < ncell) {
                if constexpr (BF16)
                    *reinterpret_cast<float4 *>(M + gc * S::MP + c0) = make_float4(u[0], u[1], u[2], u[3]);
                lds_store4<BF16>(Pb, nxt * PBUF + ui.pc + c0, u);
            }
        }
    };

    // the first step's clamp: input slice of given cells := clamp values (state buffer buf)
    auto clamp_pass = [&](int buf) {
        for (int e = tid; e < ncell * c_in; e += S::NT) {
            const int cell = e / c_in, ci = e - cell * c_in;
            if (!givenL[cell]) continue;
            const float v = clampL[e];
            const int c = in_off + ci;
            if constexpr (BF16) {
                M[cell * S::MP + c] = v;
                reinterpret_cast<__bf16 *>(Pb)[buf * PBUF + cinfo[cell] + c] = (__bf16)v;
            } else {
                reinterpret_cast<float *>(Pb)[buf * PBUF + cinfo[cell] + c] = v;
            }
        }
    };

    // fire mask of step s for every cell of the workgroup (state buffer cur holds the pre-step state)
    const int nq = (HWn + 3) >> 2;
    auto draw_fire = [&](int s, int cur) {
        for (int it = tid; it < Rw * nq; it += S::NT) {
            const int r = it / nq, qq = it - r * nq;
            float u[4] = {0.f, 0.f, 0.f, 0.f};
            if (!a.fire_u8 && !a.fire_f32) {
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
                } else if (a.fire_f32) {
                    f = a.fire_f32[(rbase + r) * HWn + q];
                } else {
                    float pcell = a.p;
                    if (a.adaptive) {
                        int am;
                        const float cf = cell_readout(state_ptr(cur, cell) + a.out_off, 1, a.c_out, a.n_out,
                                                      a.head_kind, headL, headL + a.n_out * a.c_out, &am);
                        const bool confident = cf > a.tau || (a.given_confident && givenL[cell]);
                        if (confident) pcell = a.p_low;
                    }
                    f = u[e] < pcell ? 1.0f : 0.0f;
                }
                fireL[cell] = f;
                cnt += f != 0.0f;
            }
            if (cnt) atomicAdd(&firedL[r], cnt);
        }
    };

    // ---- bf16 steady-state interval, hand-interleaved -----------------------------------
    // fc1 MFMAs of tile t are issued k-tile by k-tile, each group followed by a slice of the
    // stencil of tile t+1 (tap-pair packing first, then the dot2 chains) so that the VALU work
    // runs while the matrix core is busy; then fc2 of tile t-1 with the fc1 epilogue, then the
    // update of tile t-1. sched_barrier(0) keeps the groups in this order.
    auto interval_bf16 = [&](const Upd &ui, int spc, int zb, int hb1, int hb2, int zb_next, int cur, int nxt) {
        // ---- LDS loads
        fr_t zf[S::KT1];
#pragma unroll
        for (int kt = 0; kt < S::KT1; ++kt) zf[kt] = FR::load_lds(Zb, zb * S::ZBUF + l16 * S::ZS + kt * S::KT + 8 * g);
        const bool st_on = S::NSI == S::NT || tid < S::NSI;
        const int sbase = cur * PBUF + spc + 4 * st_qd;
        uint2 nb[9];
#pragma unroll
        for (int t9 = 0; t9 < 9; ++t9) nb[t9] = *reinterpret_cast<const uint2 *>(Pb + 2 * (sbase + toff[t9]));
        __builtin_amdgcn_sched_barrier(0);
        // ---- tap pairs
        uint32_t pr[5][4];
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
        // ---- fc1 MFMAs interleaved with the stencil's 16 dot2 chains (head k, channel c)
        f32x4 acc[S::MT1];
#pragma unroll
        for (int mt = 0; mt < S::MT1; ++mt) acc[mt] = b1v[mt];
        float zs[16];
        constexpr int CH = (16 + S::KT1 - 1) / S::KT1;  // chains per k-tile group
#pragma unroll
        for (int kt = 0; kt < S::KT1; ++kt) {
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int mt = 0; mt < S::MT1; ++mt) acc[mt] = FR::mfma(w1f[mt][kt], zf[kt], acc[mt]);
#pragma unroll
            for (int j = kt * CH; j < (kt + 1) * CH && j < 16; ++j) {
                const int k = j >> 2, c = j & 3;
                float sum = dot2_bf16_zero(pr[0][c], kp[k][0]);
#pragma unroll
                for (int p2 = 1; p2 < 5; ++p2)
                    sum = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(pr[p2][c]), as_bf16x2(kp[k][p2]), sum, false);
                zs[j] = sum;
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        // ---- fc2 of tile t-1 (H loads issued now; H of tile t-1 is complete since the last barrier)
        f32x4 acc2[S::MT2W];
        float xo[S::MT2W][4];
#pragma unroll
        for (int jj = 0; jj < S::MT2W; ++jj) {
            const int mt2 = wave + S::NW * jj;
            if (S::MT2 % S::NW != 0 && mt2 >= S::MT2) continue;
            const int c0 = 16 * mt2 + 4 * g;
            const float4 m4 = *reinterpret_cast<const float4 *>(M + ui.gc * S::MP + c0);
            xo[jj][0] = m4.x;
            xo[jj][1] = m4.y;
            xo[jj][2] = m4.z;
            xo[jj][3] = m4.w;
            fr_t hf[S::KT2];
#pragma unroll
            for (int kt = 0; kt < S::KT2; ++kt) hf[kt] = FR::load_lds(Hb, hb2 * S::HBUF + l16 * S::HS + kt * S::KT + 8 * g);
            acc2[jj] = b2v[jj];
#pragma unroll
            for (int kt = 0; kt < S::KT2; ++kt) acc2[jj] = FR::mfma(w2f[jj][kt], hf[kt], acc2[jj]);
        }
        // ---- fc1 epilogue -> H[hb1]; stencil results -> Z[zb_next]
#pragma unroll
        for (int mt = 0; mt < S::MT1; ++mt) {
            float h[4];
#pragma unroll
            for (int v = 0; v < 4; ++v) h[v] = acc[mt][v] > 0.0f ? acc[mt][v] : 0.0f;
            lds_store4<true>(Hb, hb1 * S::HBUF + l16 * S::HS + wave * S::HPW + 16 * mt + 4 * g, h);
        }
        if (st_on) {
#pragma unroll
            for (int k = 0; k < 4; ++k) lds_store4<true>(Zb, zb_next * S::ZBUF + st_n * S::ZS + k * C + 4 * st_qd, &zs[4 * k]);
        }
        __builtin_amdgcn_sched_barrier(0);
        // ---- update of tile t-1
#pragma unroll
        for (int jj = 0; jj < S::MT2W; ++jj) {
            const int mt2 = wave + S::NW * jj;
            if (S::MT2 % S::NW != 0 && mt2 >= S::MT2) continue;
            const int c0 = 16 * mt2 + 4 * g;
            float u[4];
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const float dxv = round_bf16(acc2[jj][v]);
                const float uv = __fadd_rn(xo[jj][v], __fmul_rn(ui.f, dxv));
                u[v] = (ui.gv && inslice[jj][v]) ? xo[jj][v] : uv;
            }
            *reinterpret_cast<float4 *>(M + ui.gc * S::MP + c0) = make_float4(u[0], u[1], u[2], u[3]);
            lds_store4<true>(Pb, nxt * PBUF + ui.pc + c0, u);
        }
    };

    // the steady-state interval of the split fp32 path, hand-interleaved: every LDS load first
    // (fc1's operands, the next tile's taps, the update's partial sums and state), then fc1's
    // MFMAs k-tile by k-tile, each followed by one tap of the stencil (its four FMA chains advance
    // one tap), then this wave's part of fc2 and the stores; the update's VALU last, beside the
    // MFMA tail. sched_barrier(0) keeps the groups in this order; the arithmetic is that of
    // update_ks, fc1_ks and stencil_ks.
    auto interval_ks = [&](int t, int spc, int cur, int nxt) {
        const int zb = t & 1;
        fr_t zf[S::KT1];
#pragma unroll
        for (int kt = 0; kt < S::KT1; ++kt) zf[kt] = FR::load_lds(Zb, zb * S::ZBUF + l16 * S::ZS + kt * S::KT + g);
        const int sbase = cur * PBUF + spc + 4 * g;
        float tp[9][4];
#pragma unroll
        for (int t9 = 0; t9 < 9; ++t9) lds_load4<false>(Pb, sbase + toff[t9], tp[t9]);
        // the update of tile t-1 (lanes 0-15): cell 4 wave + lane / 4, channel quad lane % 4
        const bool ul = lane < 16;
        const int un = 4 * wave + ((lane & 15) >> 2), uc0 = 4 * (lane & 3);
        const int ugq = (t - 1) * 16 + un, ugc = ugq < ncell ? ugq : ncell - 1;
        const int upc = cinfo[ugc];
        const float uf = fireL[ugc];
        const bool ugv = givenL[ugc] != 0;
        float uxo[4];
        lds_load4<false>(Pb, cur * PBUF + upc + uc0, uxo);
        float4 pw[4];
#pragma unroll
        for (int w = 0; w < 4; ++w)
            pw[w] = *reinterpret_cast<const float4 *>(RED + ((((t - 1) & 1) * 4 + w) * 16 + un) * 16 + uc0);
        __builtin_amdgcn_sched_barrier(0);
        f32x4 acc[S::MT1];
#pragma unroll
        for (int mt = 0; mt < S::MT1; ++mt) acc[mt] = b1v[mt];
        float sacc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int kt = 0; kt < S::KT1; ++kt) {
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int mt = 0; mt < S::MT1; ++mt) acc[mt] = FR::mfma(w1f[mt][kt], zf[kt], acc[mt]);
            if (kt < 9) {
#pragma unroll
                for (int c = 0; c < 4; ++c) sacc[c] = __builtin_fmaf(kwv[kt], tp[kt][c], sacc[c]);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        lds_store4<false>(Zb, ((t + 1) & 1) * S::ZBUF + l16 * S::ZS + wave * C + 4 * g, sacc);
        f32x4 part = b2v[0];
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const float h = acc[mt][v] > 0.0f ? acc[mt][v] : 0.0f;
                part = FR::mfma(w2p[mt][v], h, part);
            }
        __builtin_amdgcn_sched_barrier(0);
        float u[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const float *q0 = &pw[0].x, *q1 = &pw[1].x, *q2 = &pw[2].x, *q3 = &pw[3].x;
            const float dxv = __fadd_rn(__fadd_rn(__fadd_rn(q0[v], q1[v]), q2[v]), q3[v]);
            const float uv = __fadd_rn(uxo[v], __fmul_rn(uf, dxv));
            const int c = uc0 + v;
            u[v] = (ugv && c >= in_off && c < in_off + c_in) ? uxo[v] : uv;
        }
        if (ul) lds_store4<false>(Pb, nxt * PBUF + upc + uc0, u);
        *reinterpret_cast<float4 *>(RED + ((zb * 4 + wave) * 16 + l16) * 16 + 4 * g) =
            make_float4(part[0], part[1], part[2], part[3]);
    };

    auto stencil_any = [&](int pc, int zb, int cur) {
        if constexpr (KSPLIT)
            stencil_ks(pc, zb, cur);
        else
            stencil(pc, zb, cur);
    };
    auto fc1_any = [&](int zb, int hb) {
        if constexpr (KSPLIT)
            fc1_ks(zb, hb);
        else
            fc1(zb, hb);
    };
    auto update_any = [&](int t, int hb, int cur, int nxt, bool full) {
        if constexpr (KSPLIT)
            update_ks(t, hb, cur, nxt, full);
        else
            fc2_update(upd_info(t), hb, cur, nxt, full);
    };

    // ---- steps ------------------------------------------------------------------------------
    int cur = 0;
    for (int s = 0; s < a.n_steps; ++s) {
        const int nxt = cur ^ 1;
        draw_fire(s, cur);
        stencil_any(stencil_pc(0), 0, cur);
        __syncthreads();
        // interval 0: fc1(0) + stencil(1)
        fc1_any(0, 0);
        if (ntile > 1) stencil_any(stencil_pc(1), 1, cur);
        __syncthreads();
        // steady state: fc2/update(t-1), fc1(t), stencil(t+1) in one barrier interval; the cell
        // info of the next interval is read one interval ahead so that every LDS load of an
        // interval can be issued at its start
        Upd ui = upd_info(0);
        int spc = ntile > 2 ? stencil_pc(2) : 0;
        for (int t = 1; t + 1 < ntile; ++t) {
            const Upd ui_n = upd_info(t);
            const int spc_n = stencil_pc(t + 2 < ntile ? t + 2 : ntile - 1);
            if constexpr (BF16 && !NOISE) {
                interval_bf16(ui, spc, t & 1, t & 1, (t - 1) & 1, (t + 1) & 1, cur, nxt);
            } else if constexpr (KSPLIT && !NOISE) {
                interval_ks(t, spc, cur, nxt);
            } else if constexpr (KSPLIT) {
                update_ks(t - 1, (t - 1) & 1, cur, nxt, true);
                fc1_ks(t & 1, t & 1);
                stencil_ks(spc, (t + 1) & 1, cur);
            } else {
                fc2_update(ui, (t - 1) & 1, cur, nxt, true);
                fc1(t & 1, t & 1);
                stencil(spc, (t + 1) & 1, cur);
            }
            __syncthreads();
            ui = ui_n;
            spc = spc_n;
        }
        if (ntile > 1) {
            update_any(ntile - 2, (ntile - 2) & 1, cur, nxt, false);
            fc1_any((ntile - 1) & 1, (ntile - 1) & 1);
            __syncthreads();
        }
        update_any(ntile - 1, (ntile - 1) & 1, cur, nxt, false);
        __syncthreads();
        if (s == 0 && c_in > 0) {
            clamp_pass(nxt);
            __syncthreads();
        }
        if (a.padding == 2) {
            wrap_halo(nxt);
            __syncthreads();
        }
        cur = nxt;
    }

    // ---- write back the state, the board confidence and the fired counts
    for (int e = tid; e < Rw * C * HWn; e += S::NT) {
        const int r = e / (C * HWn), rem = e - r * C * HWn, c = rem / HWn, q = rem - c * HWn;
        a.x_out[rbase * C * HWn + e] = state_ptr(cur, r * HWn + q)[c];
    }
    if (a.conf_out) {
        for (int cell = tid; cell < ncell; cell += S::NT) {
            int am;
            confL[cell] = cell_readout(state_ptr(cur, cell) + a.out_off, 1, a.c_out, a.n_out, a.head_kind,
                                       headL, headL + a.n_out * a.c_out, &am);
        }
        __syncthreads();
        for (int r = tid; r < Rw; r += S::NT) {
            float sum = 0.0f;
            for (int q = 0; q < HWn; ++q) sum = __fadd_rn(sum, confL[r * HWn + q]);
            a.conf_out[rbase + r] = __fdiv_rn(sum, (float)HWn);
        }
    }
    if (a.fired_out)
        for (int r = tid; r < Rw; r += S::NT) a.fired_out[rbase + r] = firedL[r];
}

}  // namespace nca
