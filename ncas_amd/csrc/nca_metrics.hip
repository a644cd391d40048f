// Per-(board, trial) task metrics of decoded boards, on the GPU: maze path validity and
// optimality (reference src/nca/tasks/maze.py:251-295, 843-866) and Sudoku validity (reference
// src/nca/tasks/sudoku.py:151-164, 987-995). Decoded boards are int64 tokens (rows, H, W); a row
// belongs to board row / k_per_board of the per-board inputs / targets / given arrays, so a
// (N, K) rollout result is scored without repeating its boards K times.
//
// Maze, one workgroup per row. The predicted path is P = (pred == path_token and not given) or
// an endpoint input (inputs equal to end_a or end_b). The row is valid when
//   * the inputs hold exactly two endpoint cells a < b (row-major order),
//   * every cell of P has one or two 4-neighbours in P, a and b exactly one, and no other cell
//     exactly one,
//   * the walk from a, which those degrees force, reaches b after visiting every cell of P,
// and optimal when valid and |P| equals the target's path length (target cells equal to
// path_token plus the two endpoints). P is held in LDS as a byte grid with a one-cell border of
// zeros, so neighbour tests need no bounds checks; one lane walks it.
//
// Sudoku, one wave per row: the filled grid (inputs on given cells, pred elsewhere) is valid when
// every value is in 1..9 and every row, column and 3x3 box holds each digit once, i.e. the OR of
// the digit bits of each of the 27 units is 0x3fe.
#include <hip/hip_runtime.h>

#include <stdint.h>

#include "nca_hip.h"
#include "nca_status.h"

namespace {

constexpr int kMazeThreads = 256;
constexpr int kMazeMaxLds = 64 * 1024;  // the P grid: (H + 2) * (W + 2) bytes

__global__ void __launch_bounds__(kMazeThreads)
    maze_metrics_kernel(const int64_t *__restrict__ pred, const int64_t *__restrict__ inputs,
                        const int64_t *__restrict__ targets, const uint8_t *__restrict__ given, int k_per_board,
                        int H, int W, int64_t path_tok, int64_t end_a, int64_t end_b, uint8_t *__restrict__ valid,
                        uint8_t *__restrict__ optimal) {
    extern __shared__ uint8_t grid[];  // (H + 2) x (W + 2), border 0
    __shared__ int n_path, n_end, end_lo, end_hi, ref_len, n_deg1, bad;
    const int64_t row = blockIdx.x, board = row / k_per_board;
    const int tid = threadIdx.x, HW = H * W, Wp = W + 2, GP = (H + 2) * Wp;
    const int64_t *pr = pred + row * HW, *in = inputs + board * HW, *tg = targets + board * HW;
    const uint8_t *gv = given + board * HW;
    if (tid == 0) {
        n_path = n_end = ref_len = n_deg1 = bad = 0;
        end_lo = 0x7fffffff;
        end_hi = -1;
    }
    for (int c = tid; c < GP; c += kMazeThreads) grid[c] = 0;
    __syncthreads();
    int my_path = 0, my_end = 0, my_ref = 0;
    for (int c = tid; c < HW; c += kMazeThreads) {
        const int64_t t = in[c];
        const bool is_end = t == end_a || t == end_b;
        const bool on = is_end || (pr[c] == path_tok && gv[c] == 0);
        const int i = c / W, j = c - (c / W) * W;
        grid[(i + 1) * Wp + j + 1] = on ? 1 : 0;
        my_path += on ? 1 : 0;
        my_ref += (tg[c] == path_tok ? 1 : 0) + (is_end ? 1 : 0);
        if (is_end) {
            ++my_end;
            atomicMin(&end_lo, c);
            atomicMax(&end_hi, c);
        }
    }
    if (my_path) atomicAdd(&n_path, my_path);
    if (my_end) atomicAdd(&n_end, my_end);
    if (my_ref) atomicAdd(&ref_len, my_ref);
    __syncthreads();
    // degrees of the path cells
    int my_deg1 = 0, my_bad = 0;
    for (int c = tid; c < HW; c += kMazeThreads) {
        const int i = c / W, j = c - (c / W) * W, p = (i + 1) * Wp + j + 1;
        if (!grid[p]) continue;
        const int d = grid[p - Wp] + grid[p + Wp] + grid[p - 1] + grid[p + 1];
        my_deg1 += d == 1 ? 1 : 0;
        my_bad |= (d == 0 || d > 2) ? 1 : 0;
        if ((c == end_lo || c == end_hi) && d != 1) my_bad = 1;
    }
    if (my_deg1) atomicAdd(&n_deg1, my_deg1);
    if (my_bad) atomicOr(&bad, 1);
    __syncthreads();
    if (tid != 0) return;
    bool ok = n_end == 2 && !bad && n_deg1 == 2;
    if (ok) {
        // forced walk from a to b, neighbour order up, down, left, right
        const int a = end_lo, b = end_hi;
        int prev = -1, cur = (a / W + 1) * Wp + a % W + 1;
        const int target = (b / W + 1) * Wp + b % W + 1;
        int visited = 1;
        const int total = n_path;
        const int step[4] = {-Wp, Wp, -1, 1};
        while (cur != target) {
            int nxt = -1;
            for (int s = 0; s < 4; ++s) {
                const int nb = cur + step[s];
                if (grid[nb] && nb != prev) {
                    nxt = nb;
                    break;
                }
            }
            if (nxt < 0 || ++visited > total) {
                ok = false;
                break;
            }
            prev = cur;
            cur = nxt;
        }
        ok = ok && visited == total;
    }
    valid[row] = ok ? 1 : 0;
    optimal[row] = (ok && n_path == ref_len) ? 1 : 0;
}

constexpr int kSudokuWaves = 4;

__global__ void __launch_bounds__(64 * kSudokuWaves)
    sudoku_valid_kernel(const int64_t *__restrict__ pred, const int64_t *__restrict__ inputs,
                        const uint8_t *__restrict__ given, int64_t rows, int k_per_board, uint8_t *__restrict__ valid) {
    __shared__ uint32_t units[kSudokuWaves][27];
    __shared__ int bad[kSudokuWaves];
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * kSudokuWaves + w;
    if (lane < 27) units[w][lane] = 0;
    if (lane == 0) bad[w] = 0;
    __syncthreads();
    if (row < rows) {
        const int64_t board = row / k_per_board;
        for (int c = lane; c < 81; c += 64) {
            const int64_t v = given[board * 81 + c] ? inputs[board * 81 + c] : pred[row * 81 + c];
            if (v < 1 || v > 9) {
                atomicOr(&bad[w], 1);
                continue;
            }
            const uint32_t bit = 1u << (uint32_t)v;
            const int i = c / 9, j = c - (c / 9) * 9;
            atomicOr(&units[w][i], bit);
            atomicOr(&units[w][9 + j], bit);
            atomicOr(&units[w][18 + (i / 3) * 3 + j / 3], bit);
        }
    }
    __syncthreads();
    if (row < rows && lane == 0) {
        bool ok = bad[w] == 0;
        for (int u = 0; u < 27; ++u) ok = ok && units[w][u] == 0x3feu;
        valid[row] = ok ? 1 : 0;
    }
}

}  // namespace

extern "C" int nca_maze_metrics(const int64_t *pred, const int64_t *inputs, const int64_t *targets,
                                const uint8_t *given, int64_t rows, int32_t k_per_board, int32_t H, int32_t W,
                                int64_t path_token, int64_t end_token_a, int64_t end_token_b, uint8_t *valid,
                                uint8_t *optimal, void *stream) {
    nca::clear_error();
    if (rows < 0 || k_per_board < 1 || H < 1 || W < 1)
        return nca::set_error(NCA_ERR_INVALID, "rows >= 0, k_per_board >= 1, H >= 1, W >= 1");
    if ((int64_t)(H + 2) * (W + 2) > kMazeMaxLds)
        return nca::set_error(NCA_ERR_UNSUPPORTED, "maze metrics take grids with (H + 2) * (W + 2) <= 65536");
    if (rows > 0x7fffffffll) return nca::set_error(NCA_ERR_UNSUPPORTED, "at most 2^31 - 1 rows per call");
    if (rows == 0) return NCA_OK;
    if (!pred || !inputs || !targets || !given || !valid || !optimal)
        return nca::set_error(NCA_ERR_INVALID, "NULL pointer argument");
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const size_t lds = (size_t)(H + 2) * (W + 2);
    hipLaunchKernelGGL(maze_metrics_kernel, dim3((unsigned)rows), dim3(kMazeThreads), lds, st, pred, inputs, targets,
                       given, (int)k_per_board, (int)H, (int)W, path_token, end_token_a, end_token_b, valid, optimal);
    return nca::hip_status(hipGetLastError(), "maze metrics launch");
}

extern "C" int nca_sudoku_valid(const int64_t *pred, const int64_t *inputs, const uint8_t *given, int64_t rows,
                                int32_t k_per_board, uint8_t *valid, void *stream) {
    nca::clear_error();
    if (rows < 0 || k_per_board < 1) return nca::set_error(NCA_ERR_INVALID, "rows >= 0, k_per_board >= 1");
    if (rows == 0) return NCA_OK;
    if (!pred || !inputs || !given || !valid) return nca::set_error(NCA_ERR_INVALID, "NULL pointer argument");
    const int64_t blocks = (rows + kSudokuWaves - 1) / kSudokuWaves;
    if (blocks > 0x7fffffffll) return nca::set_error(NCA_ERR_UNSUPPORTED, "too many rows for one call");
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(sudoku_valid_kernel, dim3((unsigned)blocks), dim3(64 * kSudokuWaves), 0, st, pred, inputs,
                       given, rows, (int)k_per_board, valid);
    return nca::hip_status(hipGetLastError(), "sudoku validity launch");
}
