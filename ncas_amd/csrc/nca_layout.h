// Packed-weight layout, shared by the host code and the kernels.
//
// The packed buffer holds, at 256-byte aligned offsets:
//   kern   float[heads * 9]   perception kernels (bf16-rounded values for bf16 cells)
//   b1     float[hidden]      fc1 bias (bf16-rounded for bf16 cells: autocast casts it)
//   b2     float[C]           fc2 bias (idem)
//   headw  float[n_out*c_out] readout head weight / l2 token embeddings (fp32: the readout
//                             runs outside autocast, reference src/nca/rollout.py:184-186)
//   headb  float[n_out]
//   padv   float[C]           wall border value
//   w1     MFMA A fragments of fc1: [m-tile (hidden/16)][k-tile][lane 64][slot]
//   w2     MFMA A fragments of fc2: [m-tile (C/16)][k-tile][lane 64][slot]
//   w2h    (bf16 only) fc2 fragments for the streamed kernel, whose hidden activations sit in
//          LDS in the order of fc1's accumulators: physical position p = 64 w + 16 g + 4 mt + v
//          holds hidden unit hl(p) = 64 w + 16 mt + 4 g + v. [m-tile][k-tile][lane][slot] with
//          A[i][slot] = W2[16 m + i][hl(32 k + 8 (lane / 16) + slot)]
//   w1q    (bf16 only) fc1 fragments like w1 with the feature (k) axis in quad-major order:
//          k = 16 iq + 4 head + ch holds feature head * C + 4 iq + ch
//   w2k    (bf16 only) fc2 fragments per quarter q of the hidden units, for kernels whose waves
//          each own a quarter and keep fc1's accumulators as the B operand:
//          [q][m-tile][k-tile][lane][slot], A[i][slot] = W2[16 m + i][q hidden/4 +
//          16 (2 k + slot / 4) + 4 (lane / 16) + slot % 4]
// bf16 cells use v_mfma_f32_16x16x32_bf16 fragments (k-tile 32, 8 bf16 slots per lane:
// A[i = lane % 16][k = 8 * (lane / 16) + slot]); fp32 cells use v_mfma_f32_16x16x4_f32
// fragments (k-tile 4, one float per lane: A[i = lane % 16][k = lane / 16]).
#pragma once

#include <stddef.h>

namespace nca {

struct PackedLayout {
    size_t kern, b1, b2, headw, headb, padv, w1, w2, w2h, w1q, w2k, total;
};

__host__ __device__ inline size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

__host__ __device__ inline PackedLayout packed_layout(int C, int heads, int hidden, int c_out,
                                                      int n_out, bool bf16) {
    PackedLayout L;
    size_t o = 0;
    L.kern = o;
    o = align256(o + sizeof(float) * heads * 9);
    L.b1 = o;
    o = align256(o + sizeof(float) * hidden);
    L.b2 = o;
    o = align256(o + sizeof(float) * C);
    L.headw = o;
    o = align256(o + sizeof(float) * n_out * c_out);
    L.headb = o;
    o = align256(o + sizeof(float) * n_out);
    L.padv = o;
    o = align256(o + sizeof(float) * C);
    const size_t esz = bf16 ? 2 : 4;
    L.w1 = o;
    o = align256(o + esz * (size_t)hidden * heads * C);
    L.w2 = o;
    o = align256(o + esz * (size_t)C * hidden);
    L.w2h = o;  // bf16 cells: fc2 fragments in the streamed kernel's hidden order
    o = align256(o + (bf16 ? 2 * (size_t)C * hidden : 0));
    L.w1q = o;  // bf16 cells: fc1 fragments in quad-major feature order
    o = align256(o + (bf16 ? 2 * (size_t)hidden * heads * C : 0));
    L.w2k = o;  // bf16 cells: fc2 fragments per hidden quarter
    o = align256(o + (bf16 ? 2 * (size_t)C * hidden : 0));
    L.total = o;
    return L;
}

}  // namespace nca
