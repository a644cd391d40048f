/*
 * CPU oracle (test infrastructure, never the product): the integer and bit-exact parts of the
 * NCA hot path, restated in plain C so that the HIP library can be checked against them bit for
 * bit. Only tests, the smoke check and the CPU-baseline leg of the benchmark load this file's
 * shared object.
 *
 * 1. Philox4x32-10 (Salmon, Moraes, Dror, Shaw, "Parallel Random Numbers: As Easy as 1, 2, 3",
 *    SC'11), the counter-based generator behind the fire mask. Pinned by the Random123
 *    known-answer vectors in tests/test_oracle_philox.py.
 * 2. The fire-mask rule. The reference draws `u = torch.rand(B, 1, H, W)` and fires where
 *    `u < p` (reference src/nca/engine/rng.py:66-69, src/nca/model.py:584-593); adaptive
 *    firing uses `p_low` where the pre-step confidence is `> tau` or the cell is given
 *    (model.py:589-593). Here u comes from Philox instead of torch's generator:
 *       key     = (seed & 0xffffffff, seed >> 32)
 *       counter = (cell >> 2, step, row, 0)        cell = i * W + j, row = board * K + trial
 *       u       = (word[cell & 3] >> 8) * 2^-24    (exact in fp32, in [0, 1))
 *       fire    = u < (float)p
 * 3. The readout used for decoding and confidence (model.py:596-633), with a fixed arithmetic
 *    order so that a GPU implementation can agree to the bit:
 *       mlp head: logit_v = fma chain over the output slice starting from the bias;
 *                 conf = 1 / sum_v exp(logit_v - max) (= max softmax), clamped to [0, 1];
 *       l2 head:  score_v = 1 / (1 + sqrt(sum_c (x_c - e_vc)^2 + 1e-8)), conf = max score;
 *       board confidence = sequential fp32 sum over cells in row-major order / (H * W);
 *       argmax: first maximum (torch.argmax / np.argmax tie rule).
 *    exp is the Cephes single-precision method (S. L. Moshier, "Methods and Programs for
 *    Mathematical Functions", 1989): Cody-Waite reduction by ln 2 in two parts and a degree-5
 *    polynomial, every step a single IEEE operation.
 * 4. conf@K selection (reference src/nca/rollout.py:317-334): per board, the first maximum of
 *    the alive trials' confidence among the first k trials.
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off; no -ffast-math).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#define PHILOX_M0 0xD2511F53u
#define PHILOX_M1 0xCD9E8D57u
#define PHILOX_W0 0x9E3779B9u
#define PHILOX_W1 0xBB67AE85u

void oracle_philox4x32_10(const uint32_t ctr_in[4], const uint32_t key_in[2], uint32_t out[4]) {
    uint32_t c0 = ctr_in[0], c1 = ctr_in[1], c2 = ctr_in[2], c3 = ctr_in[3];
    uint32_t k0 = key_in[0], k1 = key_in[1];
    for (int r = 0; r < 10; ++r) {
        uint64_t p0 = (uint64_t)PHILOX_M0 * c0;
        uint64_t p1 = (uint64_t)PHILOX_M1 * c2;
        uint32_t hi0 = (uint32_t)(p0 >> 32), lo0 = (uint32_t)p0;
        uint32_t hi1 = (uint32_t)(p1 >> 32), lo1 = (uint32_t)p1;
        uint32_t n0 = hi1 ^ c1 ^ k0;
        uint32_t n2 = hi0 ^ c3 ^ k1;
        c0 = n0;
        c1 = lo1;
        c2 = n2;
        c3 = lo0;
        k0 += PHILOX_W0;
        k1 += PHILOX_W1;
    }
    out[0] = c0;
    out[1] = c1;
    out[2] = c2;
    out[3] = c3;
}

/* Uniform draw of one cell: the 24 high bits of its Philox word, scaled by 2^-24. */
float oracle_cell_uniform(uint64_t seed, uint32_t row, uint32_t step, uint32_t cell) {
    uint32_t ctr[4] = {cell >> 2, step, row, 0u};
    uint32_t key[2] = {(uint32_t)(seed & 0xffffffffu), (uint32_t)(seed >> 32)};
    uint32_t w[4];
    oracle_philox4x32_10(ctr, key, w);
    return (float)(w[cell & 3u] >> 8) * 5.9604644775390625e-08f; /* 2^-24 */
}

/*
 * Fire mask of one step for rows [row0, row0 + rows): out[r * HW + cell] in {0, 1}.
 * conf / given may be NULL (uniform firing). conf is the per-cell confidence of the pre-step
 * state, given the clamped-cell mask (given_confident). A cell fires with p_low instead of p
 * when conf > tau or it is given.
 */
void oracle_fire_mask(uint64_t seed, int64_t row0, int64_t step, int rows, int hw, float p,
                      float p_low, float tau, const float *conf, const uint8_t *given,
                      uint8_t *out) {
    for (int r = 0; r < rows; ++r) {
        for (int q = 0; q < hw; ++q) {
            float u = oracle_cell_uniform(seed, (uint32_t)(row0 + r), (uint32_t)step, (uint32_t)q);
            float pc = p;
            if (conf != NULL) {
                int confident = conf[(int64_t)r * hw + q] > tau;
                if (given != NULL && given[(int64_t)r * hw + q]) confident = 1;
                if (confident) pc = p_low;
            }
            out[(int64_t)r * hw + q] = (uint8_t)(u < pc);
        }
    }
}

/* Cephes expf, restricted to the range the softmax needs (arguments <= 0). */
float oracle_expf(float x) {
    if (x < -87.0f) x = -87.0f;
    if (x > 0.0f) x = 0.0f;
    float n = rintf(x * 1.44269504088896341f);
    float r = fmaf(-n, 0.693359375f, x);
    r = fmaf(-n, -2.12194440e-4f, r);
    float p = fmaf(1.9875691500e-4f, r, 1.3981999507e-3f);
    p = fmaf(p, r, 8.3334519073e-3f);
    p = fmaf(p, r, 4.1665795894e-2f);
    p = fmaf(p, r, 1.6666665459e-1f);
    p = fmaf(p, r, 5.0000001201e-1f);
    float r2 = r * r;
    float y = fmaf(p, r2, r);
    y = y + 1.0f;
    return ldexpf(y, (int)n);
}

/*
 * Readout of one cell. xo points at the cell's output slice, read with stride `cstride`
 * (channel stride in floats). head_kind 0 = mlp (hw: n_out x c_out, hb: n_out), 1 = l2
 * (hw: n_out x c_out token embeddings restricted to the output slice, hb unused).
 * Returns the confidence and writes the argmax index.
 */
float oracle_cell_readout(const float *xo, int64_t cstride, int c_out, int n_out, int head_kind,
                          const float *hw, const float *hb, int *argmax) {
    float best = 0.0f;
    int bi = 0;
    if (head_kind == 0) {
        float logits[64];
        for (int v = 0; v < n_out; ++v) {
            float acc = hb[v];
            for (int c = 0; c < c_out; ++c) acc = fmaf(hw[v * c_out + c], xo[c * cstride], acc);
            logits[v] = acc;
            if (v == 0 || acc > best) {
                best = acc;
                bi = v;
            }
        }
        float s = 0.0f;
        for (int v = 0; v < n_out; ++v) s = s + oracle_expf(logits[v] - best);
        float conf = 1.0f / s;
        if (conf > 1.0f) conf = 1.0f;
        if (conf < 0.0f) conf = 0.0f;
        *argmax = bi;
        return conf;
    }
    for (int v = 0; v < n_out; ++v) {
        float d2 = 0.0f;
        for (int c = 0; c < c_out; ++c) {
            float d = xo[c * cstride] - hw[v * c_out + c];
            d2 = fmaf(d, d, d2);
        }
        float sc = 1.0f / (1.0f + sqrtf(d2 + 1e-8f));
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

/*
 * Readout of a batch of states x (rows, C, H, W) fp32 (NCHW, the reference layout).
 * conf_cell (rows*H*W), conf_board (rows), argmax (rows*H*W) may each be NULL.
 */
void oracle_readout(const float *x, int rows, int C, int H, int W, int out_offset, int c_out,
                    int n_out, int head_kind, const float *hw, const float *hb, float *conf_cell,
                    float *conf_board, int32_t *argmax) {
    const int64_t hwn = (int64_t)H * W;
    for (int r = 0; r < rows; ++r) {
        float sum = 0.0f;
        for (int64_t q = 0; q < hwn; ++q) {
            const float *xo = x + ((int64_t)r * C + out_offset) * hwn + q;
            int a;
            float c = oracle_cell_readout(xo, hwn, c_out, n_out, head_kind, hw, hb, &a);
            sum = sum + c;
            if (conf_cell) conf_cell[(int64_t)r * hwn + q] = c;
            if (argmax) argmax[(int64_t)r * hwn + q] = a;
        }
        if (conf_board) conf_board[r] = sum / (float)hwn;
    }
}

/* conf@K selection: best[n] = first argmax over the first k trials of board n, dead trials
 * (alive == 0) counting as -inf. alive may be NULL (all alive). */
void oracle_conf_select(const float *conf, const uint8_t *alive, int N, int K, int k,
                        int32_t *best) {
    if (k > K) k = K;
    for (int n = 0; n < N; ++n) {
        float bv = -INFINITY;
        int bi = 0;
        for (int t = 0; t < k; ++t) {
            float v = conf[(int64_t)n * K + t];
            if (alive && !alive[(int64_t)n * K + t]) v = -INFINITY;
            if (v > bv) {
                bv = v;
                bi = t;
            }
        }
        best[n] = bi;
    }
}
