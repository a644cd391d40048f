// Niche-capped diversity pruning (reference src/nca/pruning.py:22-65): the selection of the
// trials that survive a halving of the ensemble, on the GPU, one workgroup per board.
//
// For board n with a alive trials (a > 1), target = a / 2 trials survive:
//   niches  alive trials with identical decoded boards form a niche; its representative is its
//           first alive member (the reference's dict insertion order). Trials are grouped by a
//           64-bit hash of the decoded board and checked cell by cell against the candidate
//           representative, so a hash collision never merges two niches;
//   depth   a member's rank in its niche by confidence, highest first, ties to the lower trial
//           index (the reference's stable sort by -conf); members of depth >= n_cap are cut;
//   order   the niches in a random order: the reference draws numpy's rng.permutation; here a
//           niche's position is the rank of a Philox4x32-10 word keyed on (seed; representative,
//           event, board, 1), ties broken by the representative;
//   rounds  survivors are taken round-robin, depth 0 of every niche in niche order, then depth
//           1, ..., until target are chosen or no capped member is left. That is: the capped
//           members of lexicographically smallest (depth, niche position), min(target, capped
//           members) of them.
// Boards with at most one alive trial keep their alive set.
#include <hip/hip_runtime.h>

#include <stdint.h>

#include "nca_device.h"
#include "nca_hip.h"
#include "nca_status.h"

namespace {

constexpr int kPruneThreads = 256;
constexpr int kPruneMaxK = 1024;

// First index r in [0, n) with v[r] >= key (v increasing).
__device__ __forceinline__ int64_t lower_bound(const int64_t *v, int64_t n, int64_t key) {
    int64_t lo = 0, hi = n;
    while (lo < hi) {
        const int64_t mid = (lo + hi) >> 1;
        if (v[mid] < key) lo = mid + 1;
        else hi = mid;
    }
    return lo;
}

// COMPACT = false: the (n_boards, K) layout, trial k of board n at row n * K + k, alive flags in
// `alive`, the new alive mask written to out[n * K + k].
// COMPACT = true: only the alive trials are present, as rows whose flat (board, trial) index
// board * K + trial is row_trial[row] (strictly increasing over the rows); out[row] is 1 when
// the row's trial survives.
template <bool COMPACT>
__global__ void __launch_bounds__(kPruneThreads) prune_kernel(const int32_t *__restrict__ dec,
                                                               const float *__restrict__ conf,
                                                               const uint8_t *__restrict__ alive,
                                                               const int64_t *__restrict__ row_trial,
                                                               int64_t n_rows, int K, int cells, int n_cap,
                                                               uint64_t seed, uint32_t event,
                                                               uint8_t *__restrict__ out) {
    __shared__ int src[kPruneMaxK];     // row holding trial k, -1 when the trial is not alive
    __shared__ unsigned long long hsh[kPruneMaxK];
    __shared__ float cf[kPruneMaxK];
    __shared__ int rep[kPruneMaxK];     // niche representative of an alive trial, -1 if dead
    __shared__ int depth[kPruneMaxK];   // rank in its niche
    __shared__ uint32_t nkey[kPruneMaxK];  // random key of the niche whose representative it is
    __shared__ int npos[kPruneMaxK];    // position of the niche (representatives only)
    __shared__ int n_alive_s, n_capped_s;
    const int n = blockIdx.x, tid = threadIdx.x;
    const int64_t base = (int64_t)n * K;
    if (tid == 0) {
        n_alive_s = 0;
        n_capped_s = 0;
    }
    if (COMPACT) {
        for (int k = tid; k < K; k += kPruneThreads) src[k] = -1;
        __syncthreads();
        const int64_t lo = lower_bound(row_trial, n_rows, base), hi = lower_bound(row_trial, n_rows, base + K);
        for (int64_t r = lo + tid; r < hi; r += kPruneThreads) {
            const int64_t t = row_trial[r] - base;
            if (t >= 0 && t < K) src[t] = (int)r;
        }
    } else {
        for (int k = tid; k < K; k += kPruneThreads) src[k] = alive[base + k] ? (int)(base + k) : -1;
    }
    __syncthreads();
    // hash of every alive trial's board
    for (int k = tid; k < K; k += kPruneThreads) {
        const int s = src[k];
        unsigned long long h = 1469598103934665603ull;
        float c = 0.0f;
        if (s >= 0) {
            const int32_t *b = dec + (int64_t)s * cells;
            for (int q = 0; q < cells; ++q) {
                h ^= (uint32_t)b[q];
                h *= 1099511628211ull;
            }
            c = conf[s];
            atomicAdd(&n_alive_s, 1);
        }
        hsh[k] = h;
        cf[k] = c;
        rep[k] = s >= 0 ? k : -1;
    }
    __syncthreads();
    const int n_alive = n_alive_s;
    if (n_alive <= 1) {
        for (int k = tid; k < K; k += kPruneThreads) {
            if (COMPACT) {
                if (src[k] >= 0) out[src[k]] = 1;
            } else {
                out[base + k] = src[k] >= 0 ? 1 : 0;
            }
        }
        return;
    }
    // representative: the first alive trial with the same board
    for (int k = tid; k < K; k += kPruneThreads) {
        if (rep[k] < 0) continue;
        const int32_t *bk = dec + (int64_t)src[k] * cells;
        for (int j = 0; j < k; ++j) {
            if (rep[j] < 0 || hsh[j] != hsh[k]) continue;
            const int32_t *bj = dec + (int64_t)src[j] * cells;
            bool same = true;
            for (int c = 0; c < cells && same; ++c) same = bj[c] == bk[c];
            if (same) {
                rep[k] = j;
                break;
            }
        }
    }
    __syncthreads();
    // depth in the niche and the niche keys
    for (int k = tid; k < K; k += kPruneThreads) {
        depth[k] = 0;
        nkey[k] = 0;
        const int r = rep[k];
        if (r < 0) continue;
        int d = 0;
        for (int j = 0; j < K; ++j)
            if (j != k && rep[j] == r && (cf[j] > cf[k] || (cf[j] == cf[k] && j < k))) ++d;
        depth[k] = d;
        if (r == k) {
            uint32_t c[4] = {(uint32_t)k, event, (uint32_t)n, 1u};
            nca::philox4x32_10(c, (uint32_t)(seed & 0xffffffffu), (uint32_t)(seed >> 32));
            nkey[k] = c[0];
        }
        if (d < n_cap) atomicAdd(&n_capped_s, 1);
    }
    __syncthreads();
    // niche positions: rank of (key, representative) among the representatives
    for (int k = tid; k < K; k += kPruneThreads) {
        npos[k] = 0;
        if (rep[k] != k) continue;
        int p = 0;
        for (int j = 0; j < K; ++j)
            if (rep[j] == j && (nkey[j] < nkey[k] || (nkey[j] == nkey[k] && j < k))) ++p;
        npos[k] = p;
    }
    __syncthreads();
    const int target = n_alive / 2;
    const int keep_n = target < n_capped_s ? target : n_capped_s;
    // survivors: the capped members of smallest (depth, niche position)
    for (int k = tid; k < K; k += kPruneThreads) {
        bool keep = false;
        if (rep[k] >= 0 && depth[k] < n_cap) {
            const int dk = depth[k], pk = npos[rep[k]];
            int rank = 0;
            for (int j = 0; j < K; ++j) {
                if (rep[j] < 0 || depth[j] >= n_cap) continue;
                const int dj = depth[j], pj = npos[rep[j]];
                rank += (dj < dk || (dj == dk && pj < pk)) ? 1 : 0;
            }
            keep = rank < keep_n;
        }
        if (COMPACT) {
            if (src[k] >= 0) out[src[k]] = keep ? 1 : 0;
        } else {
            out[base + k] = keep ? 1 : 0;
        }
    }
}

}  // namespace

extern "C" int nca_prune_select(const int32_t *decoded, const float *conf, const uint8_t *alive, int32_t n_boards,
                                int32_t k_trials, int32_t cells, int32_t n_cap, uint64_t seed, int64_t event,
                                uint8_t *alive_out, void *stream) {
    nca::clear_error();
    if (n_boards < 0 || k_trials < 1 || cells < 1 || n_cap < 1)
        return nca::set_error(NCA_ERR_INVALID, "n_boards >= 0, k_trials >= 1, cells >= 1, n_cap >= 1");
    if (k_trials > kPruneMaxK) return nca::set_error(NCA_ERR_UNSUPPORTED, "pruning takes at most 1024 trials per board");
    if (n_boards == 0) return NCA_OK;
    if (!decoded || !conf || !alive || !alive_out) return nca::set_error(NCA_ERR_INVALID, "NULL pointer argument");
    if (event < 0 || event > 0xffffffffll) return nca::set_error(NCA_ERR_INVALID, "event out of range");
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(prune_kernel<false>, dim3((unsigned)n_boards), dim3(kPruneThreads), 0, st, decoded, conf,
                       alive, (const int64_t *)nullptr, (int64_t)0, (int)k_trials, (int)cells, (int)n_cap, seed,
                       (uint32_t)event, alive_out);
    return nca::hip_status(hipGetLastError(), "prune launch");
}

extern "C" int nca_prune_select_rows(const int32_t *decoded, const float *conf, const int64_t *row_trial,
                                     int64_t n_rows, int32_t n_boards, int32_t k_trials, int32_t cells,
                                     int32_t n_cap, uint64_t seed, int64_t event, uint8_t *keep, void *stream) {
    nca::clear_error();
    if (n_rows < 0 || n_boards < 0 || k_trials < 1 || cells < 1 || n_cap < 1)
        return nca::set_error(NCA_ERR_INVALID, "n_rows >= 0, n_boards >= 0, k_trials >= 1, cells >= 1, n_cap >= 1");
    if (k_trials > kPruneMaxK) return nca::set_error(NCA_ERR_UNSUPPORTED, "pruning takes at most 1024 trials per board");
    if (n_rows > (int64_t)n_boards * k_trials) return nca::set_error(NCA_ERR_INVALID, "more rows than (board, trial) pairs");
    if (n_rows == 0 || n_boards == 0) return NCA_OK;
    if (!decoded || !conf || !row_trial || !keep) return nca::set_error(NCA_ERR_INVALID, "NULL pointer argument");
    if (event < 0 || event > 0xffffffffll) return nca::set_error(NCA_ERR_INVALID, "event out of range");
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(prune_kernel<true>, dim3((unsigned)n_boards), dim3(kPruneThreads), 0, st, decoded, conf,
                       (const uint8_t *)nullptr, row_trial, n_rows, (int)k_trials, (int)cells, (int)n_cap, seed,
                       (uint32_t)event, keep);
    return nca::hip_status(hipGetLastError(), "prune launch");
}
