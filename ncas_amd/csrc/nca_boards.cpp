// Batched board generation on the host (C ABI in include/nca_hip.h): seeded random mazes and
// Sudoku boards, many at a time on several threads. The reference generates them in per-board
// Python loops (src/nca/tasks/maze.py:317-445, src/nca/tasks/sudoku.py:290-294).
//
// Every board draws from its own counter-based stream, Philox4x32-10 keyed on the seed with the
// counter (word index, board, stream tag, 0), so a board's contents depend only on (seed, board)
// and not on the thread count.
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <thread>
#include <vector>

#include "nca_hip.h"
#include "nca_status.h"

namespace {

constexpr int64_t kOpen = 0, kWall = 1, kStart = 2, kGoal = 3, kPath = 4;
constexpr uint32_t kMazeTag = 0x4d415a45u, kSudokuTag = 0x5355444bu;

void philox(uint32_t c[4], uint32_t k0, uint32_t k1) {
    for (int r = 0; r < 10; ++r) {
        const uint64_t p0 = 0xD2511F53ull * c[0], p1 = 0xCD9E8D57ull * c[2];
        const uint32_t n0 = (uint32_t)(p1 >> 32) ^ c[1] ^ k0, n2 = (uint32_t)(p0 >> 32) ^ c[3] ^ k1;
        c[0] = n0;
        c[1] = (uint32_t)p1;
        c[2] = n2;
        c[3] = (uint32_t)p0;
        k0 += 0x9E3779B9u;
        k1 += 0xBB67AE85u;
    }
}

// The uniform 32-bit words of one board.
struct Stream {
    uint32_t k0, k1, board, tag, ctr = 0, buf[4], left = 0;
    Stream(uint64_t seed, uint32_t b, uint32_t t) : k0((uint32_t)seed), k1((uint32_t)(seed >> 32)), board(b), tag(t) {}
    uint32_t next() {
        if (left == 0) {
            buf[0] = ctr++;
            buf[1] = board;
            buf[2] = tag;
            buf[3] = 0;
            philox(buf, k0, k1);
            left = 4;
        }
        return buf[4 - left--];
    }
    // uniform integer in [0, n), n >= 1 (64-bit multiply-shift of a 32-bit word)
    int below(int n) { return (int)(((uint64_t)next() * (uint64_t)n) >> 32); }
    double uniform() { return next() * (1.0 / 4294967296.0); }
};

template <class F>
void for_boards(int64_t n, int threads, F &&fn) {
    if (threads < 1) threads = (int)std::max(1u, std::thread::hardware_concurrency());
    if ((int64_t)threads > n) threads = (int)std::max<int64_t>(n, 1);
    std::vector<std::thread> pool;
    for (int t = 0; t < threads; ++t)
        pool.emplace_back([&, t]() {
            for (int64_t b = t; b < n; b += threads) fn(b);
        });
    for (auto &th : pool) th.join();
}

// One maze; false when no goal at distance >= need exists in this draw.
bool draw_maze(Stream &rs, int size, double extra, int need, int64_t *in, int64_t *tg, int64_t *plen) {
    const int k = size / 2, G = 2 * k + 1;
    std::vector<uint8_t> g((size_t)G * G, (uint8_t)kWall);
    for (int i = 1; i < G; i += 2)
        for (int j = 1; j < G; j += 2) g[(size_t)i * G + j] = (uint8_t)kOpen;
    if (k > 1) {  // spanning tree of the k x k lattice by randomised depth-first search
        std::vector<uint8_t> seen((size_t)k * k, 0);
        std::vector<int> stack;
        const int s0 = rs.below(k), s1 = rs.below(k);
        seen[(size_t)s0 * k + s1] = 1;
        stack.push_back(s0 * k + s1);
        while (!stack.empty()) {
            const int cur = stack.back(), ci = cur / k, cj = cur % k;
            int nb[4], nn = 0;
            const int di[4] = {-1, 1, 0, 0}, dj[4] = {0, 0, -1, 1};
            for (int d = 0; d < 4; ++d) {
                const int a = ci + di[d], b = cj + dj[d];
                if (a >= 0 && a < k && b >= 0 && b < k && !seen[(size_t)a * k + b]) nb[nn++] = a * k + b;
            }
            if (nn == 0) {
                stack.pop_back();
                continue;
            }
            const int nxt = nb[rs.below(nn)], ni = nxt / k, nj = nxt % k;
            seen[(size_t)nxt] = 1;
            g[(size_t)(ci + ni + 1) * G + (cj + nj + 1)] = (uint8_t)kOpen;  // the wall between them
            stack.push_back(nxt);
        }
    }
    if (extra > 0) {  // knock out a fraction of the interior walls between two lattice cells
        std::vector<int> cand;
        for (int i = 1; i < 2 * k; ++i)
            for (int j = 1; j < 2 * k; ++j)
                if (((i + j) & 1) && g[(size_t)i * G + j] == kWall) cand.push_back(i * G + j);
        const int m = (int)(extra * (double)cand.size() + 0.5);
        for (int t = 0; t < m; ++t) {  // partial Fisher-Yates
            const int r = t + rs.below((int)cand.size() - t);
            std::swap(cand[t], cand[r]);
            g[(size_t)cand[t]] = (uint8_t)kOpen;
        }
    }
    // crop to size x size; BFS from a random free cell (neighbour order up, down, left, right)
    const int HW = size * size;
    std::vector<int> free_cells;
    for (int i = 0; i < size; ++i)
        for (int j = 0; j < size; ++j)
            if (g[(size_t)i * G + j] != kWall) free_cells.push_back(i * size + j);
    if (free_cells.empty()) return false;
    const int src = free_cells[rs.below((int)free_cells.size())];
    std::vector<int> dist(HW, -1), parent(HW, -1), q;
    q.reserve(HW);
    dist[src] = 0;
    q.push_back(src);
    for (size_t h = 0; h < q.size(); ++h) {
        const int c = q[h], i = c / size, j = c % size;
        const int di[4] = {-1, 1, 0, 0}, dj[4] = {0, 0, -1, 1};
        for (int d = 0; d < 4; ++d) {
            const int a = i + di[d], b = j + dj[d];
            if (a < 0 || a >= size || b < 0 || b >= size) continue;
            const int nc = a * size + b;
            if (g[(size_t)a * G + b] == kWall || dist[nc] >= 0) continue;
            dist[nc] = dist[c] + 1;
            parent[nc] = c;
            q.push_back(nc);
        }
    }
    std::vector<int> far;
    for (int c = 0; c < HW; ++c)
        if (dist[c] >= need) far.push_back(c);
    if (far.empty()) return false;
    const int dst = far[rs.below((int)far.size())];
    for (int i = 0; i < size; ++i)
        for (int j = 0; j < size; ++j) in[i * size + j] = tg[i * size + j] = g[(size_t)i * G + j];
    int64_t length = 1;
    for (int cur = dst; parent[cur] >= 0;) {
        cur = parent[cur];
        tg[cur] = kPath;
        ++length;
    }
    in[src] = tg[src] = kStart;
    in[dst] = tg[dst] = kGoal;
    *plen = length;
    return true;
}

}  // namespace

extern "C" {

int nca_maze_boards(int64_t n, int32_t size, uint64_t seed, double extra_openings, int32_t min_path_len,
                    int32_t max_tries, int64_t *inputs, int64_t *targets, uint8_t *given, int64_t *path_len,
                    int32_t threads) {
    nca::clear_error();
    if (n < 0 || size < 2 || size > 4096 || extra_openings < 0 || extra_openings > 1 || max_tries < 1)
        return nca::set_error(NCA_ERR_INVALID, "n >= 0, 2 <= size <= 4096, 0 <= extra_openings <= 1, max_tries >= 1");
    if (n > 0 && (!inputs || !targets || !given || !path_len)) return nca::set_error(NCA_ERR_INVALID, "NULL pointer argument");
    const int need = min_path_len > 0 ? min_path_len - 1 : 1;
    const int64_t HW = (int64_t)size * size;
    std::vector<uint8_t> failed((size_t)n, 0);
    for_boards(n, threads, [&](int64_t b) {
        Stream rs(seed, (uint32_t)b, kMazeTag);
        int64_t *in = inputs + b * HW, *tg = targets + b * HW;
        for (int t = 0; t < max_tries; ++t)
            if (draw_maze(rs, size, extra_openings, need, in, tg, path_len + b)) {
                for (int64_t c = 0; c < HW; ++c) given[b * HW + c] = in[c] != kOpen;
                return;
            }
        failed[(size_t)b] = 1;
    });
    for (int64_t b = 0; b < n; ++b)
        if (failed[(size_t)b]) return nca::set_error(NCA_ERR_INVALID, "no maze satisfying min_path_len within max_tries");
    return NCA_OK;
}

int nca_sudoku_boards(int64_t n, uint64_t seed, int32_t clues_lo, int32_t clues_hi, int64_t *inputs,
                      int64_t *targets, uint8_t *given, int32_t threads) {
    nca::clear_error();
    if (n < 0 || clues_lo < 0 || clues_hi < clues_lo || clues_hi > 81)
        return nca::set_error(NCA_ERR_INVALID, "n >= 0, 0 <= clues_lo <= clues_hi <= 81");
    if (n > 0 && (!inputs || !targets || !given)) return nca::set_error(NCA_ERR_INVALID, "NULL pointer argument");
    for_boards(n, threads, [&](int64_t b) {
        Stream rs(seed, (uint32_t)b, kSudokuTag);
        auto perm = [&](int m, int *p) {
            for (int i = 0; i < m; ++i) p[i] = i;
            for (int i = m - 1; i > 0; --i) std::swap(p[i], p[rs.below(i + 1)]);
        };
        // a valid base pattern under the validity-preserving symmetries: row and column
        // permutations within bands / stacks, band and stack permutations, transposition and
        // digit relabelling
        int bands[3], stacks[3], rows[9], cols[9], digits[9];
        perm(3, bands);
        for (int a = 0; a < 3; ++a) {
            int p[3];
            perm(3, p);
            for (int r = 0; r < 3; ++r) rows[3 * a + r] = 3 * bands[a] + p[r];
        }
        perm(3, stacks);
        for (int a = 0; a < 3; ++a) {
            int p[3];
            perm(3, p);
            for (int c = 0; c < 3; ++c) cols[3 * a + c] = 3 * stacks[a] + p[c];
        }
        const bool transpose = rs.below(2) == 1;
        perm(9, digits);
        int64_t *tg = targets + b * 81, *in = inputs + b * 81;
        for (int r = 0; r < 9; ++r)
            for (int c = 0; c < 9; ++c) {
                const int rr = rows[transpose ? c : r], cc = cols[transpose ? r : c];
                tg[r * 9 + c] = digits[(3 * (rr % 3) + rr / 3 + cc) % 9] + 1;
            }
        const int m = clues_lo + rs.below(clues_hi - clues_lo + 1);
        int cells[81];
        for (int i = 0; i < 81; ++i) cells[i] = i;
        for (int t = 0; t < m; ++t) std::swap(cells[t], cells[t + rs.below(81 - t)]);
        for (int i = 0; i < 81; ++i) in[i] = 0;
        for (int t = 0; t < m; ++t) in[cells[t]] = tg[cells[t]];
        for (int i = 0; i < 81; ++i) given[b * 81 + i] = in[i] != 0;
    });
    return NCA_OK;
}

}  // extern "C"
