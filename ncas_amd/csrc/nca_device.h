// Device helpers shared by the NCA kernels: Philox4x32-10, bf16 packing, the fixed-order
// readout and the packed-weight layout.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace nca {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// ------------------------------------------------------------------------------------------
// bf16 <-> fp32. Conversion to bf16 rounds to nearest even (v_cvt_pk_bf16_f32 on gfx950), the
// rounding torch's .to(torch.bfloat16) and autocast use.
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
    bf16x2 v;
    v[0] = (__bf16)a;
    v[1] = (__bf16)b;
    return __builtin_bit_cast(uint32_t, v);
}
__device__ __forceinline__ float bf16_lo(uint32_t u) { return __uint_as_float(u << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t u) { return __uint_as_float(u & 0xffff0000u); }
__device__ __forceinline__ float round_bf16(float a) { return bf16_lo(pack_bf16x2(a, 0.0f)); }
// a0 b0 + a1 b1 of two bf16 pairs with a zero accumulator: the three-operand v_dot2_f32_bf16 with
// an inline zero, whose result equals the two-operand v_dot2c form's on a zeroed accumulator bit
// for bit (checked on 4M operand pairs with denormals and cancellations); the compiler opens a
// v_dot2 chain with a move of zero and v_dot2c otherwise
__device__ __forceinline__ float dot2_bf16_zero(uint32_t a, uint32_t b) {
    float s;
    asm("v_dot2_f32_bf16 %0, %1, %2, 0" : "=v"(s) : "v"(a), "v"(b));
    return s;
}

// ------------------------------------------------------------------------------------------
// Philox4x32-10 (Salmon et al., SC'11). Counter (c0..c3), key (k0, k1); result in c.
__device__ __forceinline__ void philox4x32_10(uint32_t c[4], uint32_t k0, uint32_t k1) {
#pragma unroll
    for (int r = 0; r < 10; ++r) {
        // one 32x32 -> 64-bit product gives both halves (a single v_mad_u64_u32)
        const uint64_t p0 = (uint64_t)0xD2511F53u * c[0], p1 = (uint64_t)0xCD9E8D57u * c[2];
        const uint32_t hi0 = (uint32_t)(p0 >> 32), lo0 = (uint32_t)p0;
        const uint32_t hi1 = (uint32_t)(p1 >> 32), lo1 = (uint32_t)p1;
        const uint32_t n0 = hi1 ^ c[1] ^ k0;
        const uint32_t n2 = hi0 ^ c[3] ^ k1;
        c[0] = n0;
        c[1] = lo1;
        c[2] = n2;
        c[3] = lo0;
        k0 += 0x9E3779B9u;
        k1 += 0xBB67AE85u;
    }
}

// The four uniforms of cells 4*quad .. 4*quad+3 of `row` at `step`: counter (quad, step, row, 0),
// key = seed; u = (word >> 8) * 2^-24.
__device__ __forceinline__ void cell_uniforms4(uint64_t seed, uint32_t row, uint32_t step,
                                               uint32_t quad, float u[4]) {
    uint32_t c[4] = {quad, step, row, 0u};
    philox4x32_10(c, (uint32_t)(seed & 0xffffffffu), (uint32_t)(seed >> 32));
#pragma unroll
    for (int i = 0; i < 4; ++i) u[i] = (float)(c[i] >> 8) * 5.9604644775390625e-08f;
}

// ------------------------------------------------------------------------------------------
// Readout with a fixed operation order; every operation is a single IEEE operation so that the
// CPU restatement computes the same bits. No contraction of a*b+c into fma is allowed here.
#pragma clang fp contract(off)

__host__ __device__ __forceinline__ float readout_expf(float x) {
    if (x < -87.0f) x = -87.0f;
    if (x > 0.0f) x = 0.0f;
    const float n = __builtin_rintf(x * 1.44269504088896341f);
    float r = __builtin_fmaf(-n, 0.693359375f, x);
    r = __builtin_fmaf(-n, -2.12194440e-4f, r);
    float p = __builtin_fmaf(1.9875691500e-4f, r, 1.3981999507e-3f);
    p = __builtin_fmaf(p, r, 8.3334519073e-3f);
    p = __builtin_fmaf(p, r, 4.1665795894e-2f);
    p = __builtin_fmaf(p, r, 1.6666665459e-1f);
    p = __builtin_fmaf(p, r, 5.0000001201e-1f);
    const float r2 = r * r;
    float y = __builtin_fmaf(p, r2, r);
    y = y + 1.0f;
    return __builtin_ldexpf(y, (int)n);
}

// Confidence and argmax of one cell whose output channel c (c < c_out) is xo(c).
// head_kind 0: mlp head (hw (n_out, c_out), hb (n_out)), conf = max softmax = 1 / sum exp(l - max).
// head_kind 1: l2 head (hw = token embeddings (n_out, c_out)), conf = max 1/(1 + |x - e|).
template <class X>
__device__ __forceinline__ float cell_readout_fn(X xo, int c_out, int n_out, int head_kind, const float *hw,
                                                 const float *hb, int *argmax) {
    float best = 0.0f;
    int bi = 0;
    if (head_kind == 0) {
        // pass 1: the maximum logit; pass 2: the sum of exponentials (logits recomputed in the
        // same order, so both passes see identical values)
        for (int v = 0; v < n_out; ++v) {
            float acc = hb[v];
            for (int c = 0; c < c_out; ++c) acc = __builtin_fmaf(hw[v * c_out + c], xo(c), acc);
            if (v == 0 || acc > best) {
                best = acc;
                bi = v;
            }
        }
        float s = 0.0f;
        for (int v = 0; v < n_out; ++v) {
            float acc = hb[v];
            for (int c = 0; c < c_out; ++c) acc = __builtin_fmaf(hw[v * c_out + c], xo(c), acc);
            s = s + readout_expf(acc - best);
        }
        float conf = __fdiv_rn(1.0f, s);
        if (conf > 1.0f) conf = 1.0f;
        if (conf < 0.0f) conf = 0.0f;
        *argmax = bi;
        return conf;
    }
    for (int v = 0; v < n_out; ++v) {
        float d2 = 0.0f;
        for (int c = 0; c < c_out; ++c) {
            const float d = xo(c) - hw[v * c_out + c];
            d2 = __builtin_fmaf(d, d, d2);
        }
        const float sc = __fdiv_rn(1.0f, 1.0f + __fsqrt_rn(d2 + 1e-8f));
        if (v == 0 || sc > best) {
            best = sc;
            bi = v;
        }
    }
    *argmax = bi;
    if (best > 1.0f) best = 1.0f;
    if (best < 0.0f) best = 0.0f;
    return best;
}

// The same for a head of at most 4 outputs over at most 4 channels, its parameters in registers
// (hw4[v][c], hb4[v]): the operations and their order are cell_readout_fn's.
__device__ __forceinline__ float cell_readout4(const float xo[4], int c_out, int n_out, int head_kind,
                                               const float hw4[4][4], const float hb4[4]) {
    float best = 0.0f;
    if (head_kind == 0) {
        float lg[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            float acc = hb4[v];
#pragma unroll
            for (int c = 0; c < 4; ++c)
                if (c < c_out) acc = __builtin_fmaf(hw4[v][c], xo[c], acc);
            lg[v] = acc;
            if (v < n_out && (v == 0 || acc > best)) best = acc;
        }
        float s = 0.0f;
#pragma unroll
        for (int v = 0; v < 4; ++v)
            if (v < n_out) s = s + readout_expf(lg[v] - best);
        float conf = __fdiv_rn(1.0f, s);
        if (conf > 1.0f) conf = 1.0f;
        if (conf < 0.0f) conf = 0.0f;
        return conf;
    }
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        if (v >= n_out) continue;
        float d2 = 0.0f;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            if (c >= c_out) continue;
            const float d = xo[c] - hw4[v][c];
            d2 = __builtin_fmaf(d, d, d2);
        }
        const float sc = __fdiv_rn(1.0f, 1.0f + __fsqrt_rn(d2 + 1e-8f));
        if (v == 0 || sc > best) best = sc;
    }
    if (best > 1.0f) best = 1.0f;
    if (best < 0.0f) best = 0.0f;
    return best;
}

// The same with the output slice at xo[c * cstride].
__device__ __forceinline__ float cell_readout(const float *xo, int cstride, int c_out, int n_out,
                                              int head_kind, const float *hw, const float *hb,
                                              int *argmax) {
    return cell_readout_fn([&](int c) { return xo[c * cstride]; }, c_out, n_out, head_kind, hw, hb, argmax);
}

#pragma clang fp contract(on)

}  // namespace nca
