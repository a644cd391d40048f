// The training step around the BPTT chunk, fused on the GPU:
//
// nca_adamw_ema - one launch per iteration after the backward: the L2 norm of the summed
//   gradient, clipping to max_norm, the finiteness test, AdamW with decoupled weight decay and
//   bias correction, the exponential moving average of the weights and the zeroing of the
//   gradient, over flat fp32 buffers (every parameter of the cell back to back). The reference
//   runs clip_grad_norm_ (src/nca/engine/engine.py), a host test of the norm, torch's AdamW, a
//   Python loop of EMA updates and zero_grad (src/nca/engine/train.py:262-273). Here the norm's
//   test and the count of applied steps (AdamW's `step`, which a skipped iteration does not
//   advance) live on the device, so an iteration needs no host synchronisation; the squares are
//   summed in a fixed order (fp64: each thread a strided run, fixed butterflies, the blocks'
//   sums in block order), so the update is deterministic and a run resumed from a checkpoint
//   repeats the uninterrupted run bit for bit. The per-element arithmetic is torch's multi-tensor AdamW's,
//   operation for operation in fp32 with the same scalars: p *= 1 - lr wd; m = lerp(m, g, 1 - b1);
//   v = v b2 + (1 - b2) g g; p += -(lr / bc1) m / (sqrt(v) / sqrt(bc2) + eps).
//
// nca_pool_rows - the replay pool's gathers and scatters of a training iteration (every key of a
//   batch, the fresh boards' rows and the age counters) in one launch: the reference indexes each
//   of the pool's tensors on its own (src/nca/pool.py:96-179), one kernel per tensor and step.
//
// nca_init_state - a batch's initial state (model.py:384-412): the noise scaled as the reference
//   scales it, the clamp values (the input tokens' embeddings, model.py:378-382) and their
//   application to the given cells' input channels (model.py:430-438) in one pass; the
//   reference's torch ops take six launches.
//
// nca_damage_clamp - the damage perturbation (src/nca/perturb.py:43-106: the state set to `fill`
//   inside discs) and the clamp of the given cells' input channels (model.py:430-438) in one pass
//   over the state, in place. The discs are drawn on the host (their random stream is the
//   trainer's numpy generator) and handed over as (row, cy, cx, r^2) in fp64; a cell is inside
//   when (y - cy)^2 + (x - cx)^2 <= r^2 with y, x its row and column ("ours"), or < r^2 with y, x
//   the numpy linspace(-1, 1) coordinates ("official"), evaluated in fp64 with one rounding per
//   operation, as numpy evaluates it.
#include <hip/hip_runtime.h>

#include <math.h>
#include <stdint.h>
#include <string.h>

#include "nca_hip.h"
#include "nca_status.h"

namespace {

// Two launches over a fixed grid: the first writes each block's sum of squares (the blocks'
// elements are a fixed grid-stride partition, a thread's squares are added in a fixed order, then
// fixed butterflies) and a copy of the applied-step count; the second has every block add the
// partial sums in the same order, so every block sees the same norm and decision, and update its
// elements. Only the second kernel's block 0 writes the counters, and no block reads them there
// (the copy stands in), so no block can see another's update.
constexpr int kOptBlocks = 64;
constexpr int kOptThreads = 256;
constexpr int kUnroll = 4;

__device__ __forceinline__ double wave_sum(double v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__global__ void __launch_bounds__(kOptThreads)
    adamw_norm_kernel(const float *__restrict__ g, int64_t n, const int64_t *__restrict__ counters,
                      double *__restrict__ ws) {
    __shared__ double part[kOptThreads / 64];
    const int tid = threadIdx.x;
    const int64_t stride = (int64_t)kOptBlocks * kOptThreads;
    double acc = 0.0;
    for (int64_t base = (int64_t)blockIdx.x * kOptThreads + tid; base < n; base += stride * kUnroll) {
        float gv[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const int64_t i = base + (int64_t)u * stride;
            gv[u] = i < n ? g[i] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) acc += (double)gv[u] * (double)gv[u];
    }
    acc = wave_sum(acc);
    if ((tid & 63) == 0) part[tid >> 6] = acc;
    __syncthreads();
    if (tid == 0) {
        double b = 0.0;
        for (int w = 0; w < kOptThreads / 64; ++w) b += part[w];
        ws[blockIdx.x] = b;
        if (blockIdx.x == 0) ws[kOptBlocks] = (double)counters[0];
    }
}

__global__ void __launch_bounds__(kOptThreads)
    adamw_ema_kernel(float *__restrict__ p, float *__restrict__ g, float *__restrict__ m, float *__restrict__ v,
                     float *__restrict__ e, int64_t n, nca_adamw_desc d, int64_t *__restrict__ counters,
                     float *__restrict__ grad_norm, const double *__restrict__ ws) {
    __shared__ float s_coef, s_wd, s_w1, s_b2, s_w2, s_bc2, s_eps, s_step, s_ed, s_ea;
    __shared__ int s_ok, s_clip, s_ema;
    const int tid = threadIdx.x;
    if (tid == 0) {
        double sum = 0.0;
        for (int b = 0; b < kOptBlocks; ++b) sum += ws[b];
        const float gn = (float)sqrt(sum);
        const bool ok = isfinite(gn);
        s_clip = d.max_norm > 0.0;
        const float coef = (float)d.max_norm / (gn + 1e-6f);
        s_coef = coef < 1.0f ? coef : 1.0f;
        s_ok = ok;
        s_ema = d.ema_decay >= 0.0;
        s_ed = (float)d.ema_decay;
        s_ea = (float)(1.0 - d.ema_decay);
        const int64_t t = (int64_t)ws[kOptBlocks] + 1;
        if (ok) {
            const double bc1 = 1.0 - pow(d.beta1, (double)t), bc2 = 1.0 - pow(d.beta2, (double)t);
            s_wd = (float)(1.0 - d.lr * d.weight_decay);
            s_w1 = (float)(1.0 - d.beta1);
            s_b2 = (float)d.beta2;
            s_w2 = (float)(1.0 - d.beta2);
            s_bc2 = (float)sqrt(bc2);
            s_eps = (float)d.eps;
            s_step = (float)(-(d.lr / bc1));
        }
        if (blockIdx.x == 0) {
            grad_norm[0] = gn;
            if (ok)
                counters[0] = t;
            else
                counters[1] += 1;
        }
    }
    __syncthreads();
    const bool ok = s_ok, clip = s_clip, ema = s_ema;
    const float coef = s_coef, wd = s_wd, w1 = s_w1, b2 = s_b2, w2 = s_w2, bc2 = s_bc2, eps = s_eps,
                step = s_step, ed = s_ed, ea = s_ea;
    const int64_t stride = (int64_t)kOptBlocks * kOptThreads;
    for (int64_t base = (int64_t)blockIdx.x * kOptThreads + tid; base < n; base += stride * kUnroll) {
        float pv[kUnroll], gv[kUnroll], mv[kUnroll], vv[kUnroll], ev[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const int64_t i = base + (int64_t)u * stride;
            const bool in = i < n;
            pv[u] = in ? p[i] : 0.0f;
            gv[u] = in && ok ? g[i] : 0.0f;
            mv[u] = in && ok ? m[i] : 0.0f;
            vv[u] = in && ok ? v[i] : 0.0f;
            ev[u] = in && ema ? e[i] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const int64_t i = base + (int64_t)u * stride;
            if (i >= n) break;
            float pi = pv[u];
            if (ok) {
                float gi = gv[u];
                if (clip) gi = gi * coef;
                pi = pi * wd;
                float mi = mv[u];
                mi = w1 < 0.5f ? mi + w1 * (gi - mi) : gi - (gi - mi) * (1.0f - w1);
                float vi = vv[u] * b2;
                vi = vi + w2 * (gi * gi);
                const float den = sqrtf(vi) / bc2 + eps;
                pi = pi + step * (mi / den);
                p[i] = pi;
                m[i] = mi;
                v[i] = vi;
            }
            if (ema) {
                const float ei = ev[u] * ed;
                e[i] = ei + ea * pi;
            }
            g[i] = 0.0f;
        }
    }
}

constexpr int kDamageThreads = 256;

__device__ __forceinline__ double linspace_pm1(int i, int num) {
    // numpy.linspace(-1, 1, num)[i]: i * (2 / (num - 1)) - 1, the last point exactly 1
    if (num == 1) return -1.0;
    if (i == num - 1) return 1.0;
    return __dadd_rn(__dmul_rn((double)i, __ddiv_rn(2.0, (double)(num - 1))), -1.0);
}

__global__ void __launch_bounds__(kDamageThreads)
    damage_clamp_kernel(float *__restrict__ x, int64_t rows, int C, int H, int W, const double *__restrict__ discs,
                        int n_discs, int official, float fill, const uint8_t *__restrict__ given,
                        const float *__restrict__ clamp, int c_in, int in_offset) {
    const int64_t HW = (int64_t)H * W;
    const int64_t cell = (int64_t)blockIdx.x * kDamageThreads + threadIdx.x;
    if (cell >= rows * HW) return;
    const int64_t row = cell / HW, rc = cell - row * HW;
    const int i = (int)(rc / W), j = (int)(rc - (int64_t)(rc / W) * W);
    const double y = official ? linspace_pm1(i, H) : (double)i;
    const double xx = official ? linspace_pm1(j, W) : (double)j;
    bool hit = false;
    for (int k = 0; k < n_discs && !hit; ++k) {
        const double *dk = discs + 4 * k;
        if ((int64_t)dk[0] != row) continue;
        const double dy = __dsub_rn(y, dk[1]), dx = __dsub_rn(xx, dk[2]);
        const double s = __dadd_rn(__dmul_rn(dy, dy), __dmul_rn(dx, dx));
        hit = official ? s < dk[3] : s <= dk[3];
    }
    float *xr = x + row * C * HW + rc;
    if (hit)
        for (int c = 0; c < C; ++c) xr[c * HW] = fill;
    if (given && given[row * HW + rc]) {
        const float *cr = clamp + row * c_in * HW + rc;
        for (int c = 0; c < c_in; ++c) xr[(in_offset + c) * HW] = cr[c * HW];
    }
}

// ---- replay-pool row copies: item i copies row src_row[r] (r when NULL; none when < 0) of its
// source to row dst_row[r] (r when NULL) of its destination, for r < n_rows, 16 bytes at a time
// where the rows and pointers allow it (else 4, else 1); mode 1 adds one to every int64 of the row,
// mode 2 writes zeros (no source)
constexpr int kRowItems = 16;
constexpr int kRowThreads = 256;
struct RowArgs {
    nca_pool_row_copy it[kRowItems];
    int n_items;
    int64_t n_rows;
};

// Workgroup (r, item, chunk) copies bytes [chunk kRowChunk, (chunk + 1) kRowChunk) of the item's
// row r: a 115 KB state row is 8 workgroups, and each thread issues its four 16-byte loads before
// its stores (one workgroup per row, looping, took 17 us for a training batch: a round trip per
// 4 KB).
constexpr int64_t kRowChunk = 16384;

__global__ void __launch_bounds__(kRowThreads) pool_rows_kernel(RowArgs a) {
    const int64_t r = blockIdx.x;
    const nca_pool_row_copy &c = a.it[blockIdx.y];
    const int64_t lo = (int64_t)blockIdx.z * kRowChunk;
    if (lo >= c.row_bytes) return;
    const int64_t hi = c.row_bytes - lo < kRowChunk ? c.row_bytes : lo + kRowChunk;
    const int64_t sr = c.src_row ? c.src_row[r] : r;
    if (sr < 0) return;
    const int64_t dr = c.dst_row ? c.dst_row[r] : r;
    unsigned char *dst = static_cast<unsigned char *>(c.dst) + dr * c.row_bytes;
    const unsigned char *src = c.mode == 2 ? nullptr : static_cast<const unsigned char *>(c.src) + sr * c.row_bytes;
    if (c.mode == 1) {
        for (int64_t e = lo / 8 + threadIdx.x; e < hi / 8; e += kRowThreads)
            reinterpret_cast<int64_t *>(dst)[e] = reinterpret_cast<const int64_t *>(src)[e] + 1;
        return;
    }
    const uintptr_t al = reinterpret_cast<uintptr_t>(dst) | reinterpret_cast<uintptr_t>(src) | (uintptr_t)c.row_bytes;
    if ((al & 15u) == 0) {
        constexpr int kU = (int)(kRowChunk / 16 / kRowThreads);  // 4 quads a thread
        const int64_t q0 = lo / 16 + threadIdx.x, qn = hi / 16;
        uint4 v[kU];
#pragma unroll
        for (int k = 0; k < kU; ++k) {
            const int64_t e = q0 + (int64_t)k * kRowThreads;
            v[k] = (src && e < qn) ? reinterpret_cast<const uint4 *>(src)[e] : make_uint4(0u, 0u, 0u, 0u);
        }
#pragma unroll
        for (int k = 0; k < kU; ++k) {
            const int64_t e = q0 + (int64_t)k * kRowThreads;
            if (e < qn) reinterpret_cast<uint4 *>(dst)[e] = v[k];
        }
    } else if ((al & 3u) == 0) {
        for (int64_t e = lo / 4 + threadIdx.x; e < hi / 4; e += kRowThreads)
            reinterpret_cast<uint32_t *>(dst)[e] = src ? reinterpret_cast<const uint32_t *>(src)[e] : 0u;
    } else {
        for (int64_t e = lo + threadIdx.x; e < hi; e += kRowThreads) dst[e] = src ? src[e] : (unsigned char)0;
    }
}

// One thread per state element (row, channel, cell): coalesced over the cells of a plane.
constexpr int kInitThreads = 256;

__global__ void __launch_bounds__(kInitThreads)
    init_state_kernel(const float *__restrict__ noise, const int64_t *__restrict__ tokens,
                      const uint8_t *__restrict__ given, const float *__restrict__ embed, int vocab, int64_t rows,
                      int C, int c_in, int in_off, int hw, int uniform, float sigma, float *__restrict__ x,
                      float *__restrict__ clamp) {
    const int64_t o = (int64_t)blockIdx.x * kInitThreads + threadIdx.x;
    if (o >= rows * C * (int64_t)hw) return;
    const int64_t bc = o / hw;
    const int q = (int)(o - bc * hw);
    const int64_t b = bc / C;
    const int c = (int)(bc - b * C);
    const float r = noise[o];
    // the reference's expressions, one rounding per operation: (rand * 2 - 1) * sigma or
    // randn * sigma
    float v = uniform ? __fmul_rn(__fsub_rn(__fmul_rn(r, 2.0f), 1.0f), sigma) : __fmul_rn(r, sigma);
    const int ci = c - in_off;
    if (ci >= 0 && ci < c_in) {
        const int64_t tok = tokens[b * hw + q];
        const float cv = tok >= 0 && tok < vocab ? embed[tok * c_in + ci] : __int_as_float(0x7fc00000);
        clamp[(b * c_in + ci) * hw + q] = cv;
        if (given[b * hw + q]) v = cv;
    }
    x[o] = v;
}

}  // namespace

extern "C" int nca_init_state(const float *noise, const int64_t *tokens, const uint8_t *given, const float *embed,
                              int32_t vocab, int64_t rows, int32_t channels, int32_t c_in, int32_t in_off,
                              int32_t hw, int32_t uniform, float sigma, float *x, float *clamp, void *stream) {
    nca::clear_error();
    if (rows < 0 || channels < 1 || c_in < 0 || in_off < 0 || in_off + c_in > channels || hw < 1 || vocab < 1)
        return nca::set_error(NCA_ERR_INVALID, "rows >= 0, 0 <= in_off, in_off + c_in <= channels, hw >= 1, vocab >= 1");
    if (rows == 0) return NCA_OK;
    if (!noise || !tokens || !given || !x || (c_in > 0 && (!embed || !clamp)))
        return nca::set_error(NCA_ERR_INVALID, "NULL pointer argument");
    const int64_t n = rows * (int64_t)channels * hw;
    if (n > 0x7fffffffll * kInitThreads) return nca::set_error(NCA_ERR_UNSUPPORTED, "too many state elements");
    const unsigned blocks = (unsigned)((n + kInitThreads - 1) / kInitThreads);
    hipLaunchKernelGGL(init_state_kernel, dim3(blocks), dim3(kInitThreads), 0, reinterpret_cast<hipStream_t>(stream),
                       noise, tokens, given, embed, (int)vocab, rows, (int)channels, (int)c_in, (int)in_off, (int)hw,
                       (int)uniform, sigma, x, clamp);
    return nca::hip_status(hipGetLastError(), "init state launch");
}

extern "C" int nca_pool_rows(const nca_pool_row_copy *items, int32_t n_items, int64_t n_rows, void *stream) {
    nca::clear_error();
    if (n_items < 0 || n_items > kRowItems || n_rows < 0)
        return nca::set_error(NCA_ERR_INVALID, "0 <= n_items <= 16, n_rows >= 0");
    if (n_items == 0 || n_rows == 0) return NCA_OK;
    if (!items) return nca::set_error(NCA_ERR_INVALID, "NULL items");
    if (n_rows > 0x7fffffffll) return nca::set_error(NCA_ERR_UNSUPPORTED, "n_rows < 2^31");
    RowArgs a;
    memset(&a, 0, sizeof(a));
    for (int i = 0; i < n_items; ++i) {
        const nca_pool_row_copy &c = items[i];
        if (!c.dst || (c.mode != 2 && !c.src) || c.row_bytes < 0 || c.mode < 0 || c.mode > 2)
            return nca::set_error(NCA_ERR_INVALID, "an item needs dst, src (modes 0, 1), row_bytes >= 0, mode 0-2");
        if (c.mode == 1 && c.row_bytes % 8 != 0) return nca::set_error(NCA_ERR_INVALID, "mode 1 rows hold int64 values");
        a.it[i] = c;
    }
    a.n_items = n_items;
    a.n_rows = n_rows;
    int64_t chunks = 1;
    for (int i = 0; i < n_items; ++i) {
        const int64_t k = (items[i].row_bytes + kRowChunk - 1) / kRowChunk;
        if (k > chunks) chunks = k;
    }
    if (chunks > 65535) return nca::set_error(NCA_ERR_UNSUPPORTED, "rows of at most 1 GiB");
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(pool_rows_kernel, dim3((unsigned)n_rows, (unsigned)n_items, (unsigned)chunks), dim3(kRowThreads),
                       0, st, a);
    return nca::hip_status(hipGetLastError(), "pool rows launch");
}

extern "C" int nca_adamw_ema(float *params, float *grads, float *exp_avg, float *exp_avg_sq, float *ema, int64_t n,
                             const nca_adamw_desc *desc, int64_t *counters, float *grad_norm, void *workspace,
                             void *stream) {
    nca::clear_error();
    if (!desc) return nca::set_error(NCA_ERR_INVALID, "NULL descriptor");
    if (n < 1) return nca::set_error(NCA_ERR_INVALID, "n >= 1");
    if (!params || !grads || !exp_avg || !exp_avg_sq || !counters || !grad_norm || !workspace)
        return nca::set_error(NCA_ERR_INVALID, "NULL pointer argument");
    static_assert((kOptBlocks + 1) * sizeof(double) <= NCA_ADAMW_WORKSPACE_BYTES, "workspace size");
    if (desc->ema_decay >= 0.0 && !ema) return nca::set_error(NCA_ERR_INVALID, "ema_decay >= 0 needs the EMA buffer");
    if (!(desc->beta1 >= 0.0 && desc->beta1 < 1.0 && desc->beta2 >= 0.0 && desc->beta2 < 1.0 && desc->eps >= 0.0 &&
          desc->lr >= 0.0 && desc->weight_decay >= 0.0 && desc->ema_decay <= 1.0))
        return nca::set_error(NCA_ERR_INVALID, "0 <= beta1, beta2 < 1; eps, lr, weight_decay >= 0; ema_decay <= 1");
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    double *ws = static_cast<double *>(workspace);
    hipLaunchKernelGGL(adamw_norm_kernel, dim3(kOptBlocks), dim3(kOptThreads), 0, st, grads, n, counters, ws);
    int rc = nca::hip_status(hipGetLastError(), "adamw norm launch");
    if (rc) return rc;
    hipLaunchKernelGGL(adamw_ema_kernel, dim3(kOptBlocks), dim3(kOptThreads), 0, st, params, grads, exp_avg, exp_avg_sq,
                       ema, n, *desc, counters, grad_norm, ws);
    return nca::hip_status(hipGetLastError(), "adamw launch");
}

extern "C" int nca_damage_clamp(float *x, int64_t rows, int32_t channels, int32_t height, int32_t width,
                                const double *discs, int32_t n_discs, int32_t geometry, float fill,
                                const uint8_t *given, const float *clamp, int32_t c_in, int32_t in_offset,
                                void *stream) {
    nca::clear_error();
    if (rows < 0 || channels < 1 || height < 1 || width < 1 || n_discs < 0)
        return nca::set_error(NCA_ERR_INVALID, "rows >= 0, channels, height, width >= 1, n_discs >= 0");
    if (geometry != NCA_DAMAGE_OURS && geometry != NCA_DAMAGE_OFFICIAL)
        return nca::set_error(NCA_ERR_INVALID, "geometry: NCA_DAMAGE_OURS or NCA_DAMAGE_OFFICIAL");
    if (given && (!clamp || c_in < 1 || in_offset < 0 || in_offset + c_in > channels))
        return nca::set_error(NCA_ERR_INVALID, "the clamp needs clamp values and 0 <= in_offset < in_offset + c_in <= channels");
    if (rows == 0) return NCA_OK;
    if (!x || (n_discs > 0 && !discs)) return nca::set_error(NCA_ERR_INVALID, "NULL pointer argument");
    const int64_t cells = rows * (int64_t)height * width;
    const int64_t blocks = (cells + kDamageThreads - 1) / kDamageThreads;
    if (blocks > 0x7fffffffll) return nca::set_error(NCA_ERR_UNSUPPORTED, "too many cells for one call");
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(damage_clamp_kernel, dim3((unsigned)blocks), dim3(kDamageThreads), 0, st, x, rows,
                       (int)channels, (int)height, (int)width, discs, (int)n_discs,
                       geometry == NCA_DAMAGE_OFFICIAL ? 1 : 0, fill, given, clamp, (int)c_in, (int)in_offset);
    return nca::hip_status(hipGetLastError(), "damage launch");
}
