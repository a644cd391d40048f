/*
 * nca_hip.h - C ABI of the MI355X (gfx950) NCA step / rollout library `libnca_hip.so`.
 *
 * Every entry point takes plain device pointers and sizes, returns an int status (NCA_OK = 0)
 * and, on failure, leaves a message readable with nca_last_error() (thread-local). Calls are
 * ordered on the given HIP stream (a hipStream_t passed as void*, NULL = default stream) and
 * never synchronise the host. The library allocates no device memory: the caller owns every
 * buffer, including the packed weights (nca_packed_weights_bytes / nca_pack_weights).
 *
 * Tensor layouts are the reference's: states (rows, C, H, W) fp32 contiguous (NCHW), given
 * masks (rows, H, W) uint8, clamp values (rows, c_in, H, W) fp32. A "row" is one rollout,
 * i.e. one (board, trial) pair flattened board-major: row = board * K + trial (reference
 * src/nca/rollout.py:143-146).
 *
 * Reference interfaces replaced (paths relative to the reference repository):
 *   nca_step          <- the step protocol `step(x, given4, clamp, fire, noise, noise_mask,
 *                        clock) -> x` of make_step (src/nca/engine/step.py:74-209, call at
 *                        184-207) and NCA.step (src/nca/model.py:503-559)
 *   nca_rollout       <- the per-step loops inference_block / InferenceEngine.__call__
 *                        (src/nca/engine/inference.py:9-71) and rollout()'s step loop
 *                        (src/nca/rollout.py:203-247), fused into one launch
 *   nca_rollout_ws    <- the same loops for grids whose rows do not fit one workgroup's LDS
 *                        (the 201x201 mazes of src/nca/tasks/maze.py, max_cells batching of
 *                        rollout.py:101): one launch per step into a caller workspace
 *   nca_rollout_workspace_bytes <- nothing in the reference (PyTorch allocates its temporaries);
 *                        tells the caller how large that workspace must be
 *   nca_fire_mask     <- draw_step's fire mask (src/nca/engine/rng.py:51-69) and
 *                        NCA.sample_fire_mask (src/nca/model.py:567-593)
 *   nca_readout       <- NCA.scores / confidence / board_confidence / decode
 *                        (src/nca/model.py:596-633)
 *   nca_conf_select   <- conf_at_k's per-board selection (src/nca/rollout.py:317-334)
 *   nca_bptt_forward  <- the BPTT chunk's forward in Engine.train_iteration (run_steps with grad,
 *                        src/nca/engine/engine.py:478-489 -> run_block, step.py:212-246): the
 *                        chunk's states, kept instead of autograd's per-step activations
 *   nca_bptt_forward_ws <- the same, with a workspace that lets boards run in pieces of rows
 *   nca_bptt_backward <- its backward ((loss * scale).backward(), engine.py:497, through
 *                        _FusedCellUpdate.backward ops.py:269-294, the MLP and the shared-kernel
 *                        perception backward ops.py:79-94) with the loss of step.py:243-245 /
 *                        train.py:183-207 normalised as in engine.py:490
 *   nca_bptt_workspace_bytes <- nothing in the reference (autograd allocates); workspace size
 *   nca_step_backward <- the backward of one step of make_step's step function under autograd
 *                        (src/nca/engine/step.py:184-207): _FusedCellUpdate.backward
 *                        (src/nca/engine/ops.py:269-294), the MLP's backward and the shared-kernel
 *                        perception backward (ops.py:79-94); checked against the reference step's
 *                        gradients by tests/test_engine_ops.py:251-294
 *   nca_step_backward_workspace_bytes <- nothing in the reference (autograd allocates)
 *   nca_prune_select  <- niche_capped_pruning (src/nca/pruning.py:22-65) at the pruning steps of
 *                        rollout() (src/nca/rollout.py:249-275)
 *   nca_prune_select_rows <- the same on rollout()'s compacted batch (rollout.py:249-271)
 *   nca_maze_metrics  <- the maze tasks' "valid" / "optimal" metrics (src/nca/tasks/maze.py:
 *                        251-295, 843-866)
 *   nca_sudoku_valid  <- the Sudoku tasks' "valid" metric (src/nca/tasks/sudoku.py:151, 987-995)
 *   nca_adamw_ema     <- clip_grad_norm_ + AdamW.step + zero_grad + the EMA loop of train_fast's
 *                        update (src/nca/engine/train.py:262-273)
 *   nca_damage_clamp  <- apply_damage + apply_clamp of the training batch (src/nca/perturb.py:
 *                        43-106, src/nca/train.py:219-244)
 *   nca_pool_rows     <- the replay pool's per-tensor indexing of a training iteration
 *                        (src/nca/pool.py:96-179: sample's gathers and fresh boards, write_back's
 *                        scatters and the age counters)
 *   nca_init_state    <- NCA.init_state (src/nca/model.py:384-412) with clamp_values and
 *                        apply_clamp (model.py:378-382, 430-438)
 */
#ifndef NCA_HIP_H
#define NCA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    NCA_OK = 0,
    NCA_ERR_INVALID = 1,     /* bad argument (NULL pointer, inconsistent sizes) */
    NCA_ERR_UNSUPPORTED = 2, /* a cell shape or option this build does not implement */
    NCA_ERR_HIP = 3          /* a HIP runtime call failed */
};

enum { NCA_PAD_ZERO = 0, NCA_PAD_WALL = 1, NCA_PAD_WRAP = 2 };      /* model.py:140-152 */
enum { NCA_HEAD_MLP = 0, NCA_HEAD_L2 = 1 };                         /* model.py:596-609 */
enum { NCA_FP32 = 0, NCA_BF16 = 1 };

/* The cell: "kernels" perception with `heads` 3x3 kernels (head-major features, F = heads*C),
 * ReLU MLP F -> hidden -> C, no group normalisation, no time embedding (NCAConfig,
 * src/nca/model.py:47-137). precision NCA_BF16 reproduces the rounding points of bf16 autocast:
 * perception input, z, h and dx rounded to bf16, fp32 accumulation and fp32 state. */
typedef struct nca_cell_desc {
    int32_t channels;   /* C */
    int32_t heads;      /* perception kernels (4) */
    int32_t hidden;     /* MLP hidden width */
    int32_t c_in;       /* clamped input slice [in_offset, in_offset + c_in) */
    int32_t in_offset;
    int32_t c_out;      /* readout slice [out_offset, out_offset + c_out) */
    int32_t out_offset;
    int32_t n_out;      /* readout classes (logits of the mlp head, tokens of the l2 head) */
    int32_t padding;    /* NCA_PAD_* */
    int32_t head_kind;  /* NCA_HEAD_* */
    int32_t precision;  /* NCA_FP32 | NCA_BF16 */
} nca_cell_desc;

/* fp32 device pointers in the reference's parameter layouts. */
typedef struct nca_cell_weights {
    const float *kernels; /* perceive.weight (heads, 1, 3, 3) */
    const float *w1;      /* update.fc1.weight (hidden, F, 1, 1) */
    const float *b1;      /* update.fc1.bias (hidden) */
    const float *w2;      /* update.fc2.weight (C, hidden, 1, 1) */
    const float *b2;      /* update.fc2.bias (C) */
    const float *head_w;  /* mlp: head.weight (n_out, c_out, 1, 1); l2: out_embed (n_out, c_out) */
    const float *head_b;  /* mlp: head.bias (n_out); l2: NULL */
    const float *pad_vec; /* wall border value (C) (model.py:320-325); may be NULL unless WALL */
} nca_cell_weights;

/* Which rows and how they fire. */
typedef struct nca_fire_desc {
    uint64_t seed;              /* Philox key when step_seeds is NULL */
    const uint64_t *step_seeds; /* device (n_steps): per-step keys (engine/rng.py:37-39), or NULL */
    const uint8_t *fire_in;     /* device (n_steps, rows, H, W) injected masks in {0,1}, or NULL */
    int64_t row0;               /* global index of row 0 (Philox counter) */
    int64_t step0;              /* global index of the first step (Philox counter) */
    float p_fire;               /* firing probability */
    float p_low;                /* adaptive firing: probability of confident cells */
    float tau;                  /* adaptive firing: confidence threshold (strict >) */
    int32_t adaptive;           /* 0 = uniform p_fire, 1 = confidence-gated (model.py:589-593) */
    int32_t given_confident;    /* adaptive: given cells count as confident (rollout.py:36) */
} nca_fire_desc;

/* Bytes of the packed-weight buffer for this cell, 0 if the cell is unsupported. */
size_t nca_packed_weights_bytes(const nca_cell_desc *cell);

/* Convert the reference-layout fp32 weights into the kernels' MFMA fragment layout (bf16 or
 * fp32 per cell->precision). `packed` must hold nca_packed_weights_bytes(cell) bytes. */
int nca_pack_weights(const nca_cell_desc *cell, const nca_cell_weights *w, void *packed,
                     void *stream);

/* Run n_steps NCA steps on `rows` states of H x W cells: x_out = step^n(x_in). x_in and x_out
 * may alias. noise (rows, C, H, W) is added after the residual update when n_steps == 1
 * (model.py:544-546), NULL otherwise. conf_out (rows) receives the board confidence of the
 * final state (model.py:631-633), fired_out (rows) the number of fired cells over the call
 * (rollout.py:233); either may be NULL. */
int nca_rollout(const nca_cell_desc *cell, const void *packed, int64_t rows, int32_t height,
                int32_t width, const float *x_in, const uint8_t *given, const float *clamp,
                float *x_out, const nca_fire_desc *fire, int32_t n_steps, const float *noise,
                float *conf_out, int32_t *fired_out, void *stream);

/* Bytes of workspace that nca_rollout_ws needs for this call shape: 0 when the rows fit the
 * LDS-resident kernels (the whole rollout runs in one launch; bf16 cells with C=32, hidden 256
 * on boards up to 31 wide, such as 30x30, run one board per workgroup), else two state buffers
 * (2 * rows * C * H * W * 4 bytes) for the halo-tiled per-step path. An in-place single step
 * with noise always takes the tiled path and then needs one state buffer. */
size_t nca_rollout_workspace_bytes(const nca_cell_desc *cell, int64_t rows, int32_t height,
                                   int32_t width);

/* nca_rollout with a caller-owned device workspace. Grids whose rows do not fit the resident
 * kernels run one halo-tiled launch per step: the first step reads x_in, the steps in between
 * keep the state in the workspace (cell-major, two buffers), the last writes x_out. They need
 * workspace_bytes >= nca_rollout_workspace_bytes (one state buffer suffices for n_steps == 2
 * or an in-place single step, none for an out-of-place single step). The workspace must not
 * overlap x_in or x_out. The arithmetic per cell is the generic resident kernel's (nca_set_kernel_path(1)). */
int nca_rollout_ws(const nca_cell_desc *cell, const void *packed, int64_t rows, int32_t height,
                   int32_t width, const float *x_in, const uint8_t *given, const float *clamp,
                   float *x_out, const nca_fire_desc *fire, int32_t n_steps, const float *noise,
                   float *conf_out, int32_t *fired_out, void *workspace, size_t workspace_bytes,
                   void *stream);

/* Niche-capped diversity pruning of K trials per board (reference src/nca/pruning.py:22-65,
 * used by rollout() at its pruning steps, src/nca/rollout.py:249-275): decoded (n_boards,
 * k_trials, cells) int32 decoded boards, conf (n_boards, k_trials) board confidences, alive
 * (n_boards, k_trials) {0,1}; writes the trials that stay alive to alive_out (may alias alive).
 * A board with a > 1 alive trials keeps a / 2 of them: trials with identical decoded boards
 * form a niche, each niche's members by confidence (highest first, ties to the lower trial) with
 * at most n_cap kept, taken round-robin across the niches in a random order. The order is the
 * build's own (Philox4x32-10 keyed on (seed; niche representative, event, board, 1)), where the
 * reference draws numpy's rng.permutation. k_trials <= 1024. Deterministic. */
int nca_prune_select(const int32_t *decoded, const float *conf, const uint8_t *alive,
                     int32_t n_boards, int32_t k_trials, int32_t cells, int32_t n_cap,
                     uint64_t seed, int64_t event, uint8_t *alive_out, void *stream);

/* The same selection on a compacted batch (the rows rollout() still runs after earlier pruning
 * steps, src/nca/rollout.py:249-271): decoded (n_rows, cells) int32 and conf (n_rows) of the
 * alive trials only, row_trial (n_rows) int64 the flat (board, trial) index board * k_trials +
 * trial of each row, strictly increasing. keep (n_rows) gets 1 for the rows whose trial
 * survives. Results equal nca_prune_select's on the full layout with the absent trials dead. */
int nca_prune_select_rows(const int32_t *decoded, const float *conf, const int64_t *row_trial,
                          int64_t n_rows, int32_t n_boards, int32_t k_trials, int32_t cells,
                          int32_t n_cap, uint64_t seed, int64_t event, uint8_t *keep,
                          void *stream);

/* Task metrics of decoded boards, one value per row; row r belongs to board r / k_per_board of
 * the per-board arrays (k_per_board = K scores an (N, K) rollout result without repeating the
 * boards). Device buffers: pred (rows, H, W) int64 tokens; inputs / targets (boards, H, W)
 * int64; given (boards, H, W) {0,1}; outputs (rows) {0,1}.
 *
 * nca_maze_metrics <- _MazeTask._metrics' "valid" / "optimal" (src/nca/tasks/maze.py:843-866)
 * with path_validity (maze.py:251-295): the predicted path (pred == path_token on non-given
 * cells, plus the inputs' endpoint cells, tokens end_token_a / end_token_b) is one simple
 * 4-connected path between exactly two endpoints ("valid"), and as long as the target path,
 * i.e. the target's path_token cells plus the endpoints ("optimal"). (H + 2) * (W + 2) <= 65536. */
int nca_maze_metrics(const int64_t *pred, const int64_t *inputs, const int64_t *targets,
                     const uint8_t *given, int64_t rows, int32_t k_per_board, int32_t height,
                     int32_t width, int64_t path_token, int64_t end_token_a,
                     int64_t end_token_b, uint8_t *valid, uint8_t *optimal, void *stream);

/* nca_sudoku_valid <- SudokuOOD.metrics' "valid" (src/nca/tasks/sudoku.py:987-995) with
 * is_valid_solution (sudoku.py:151-164): the grid filled with the inputs on given cells and pred
 * elsewhere has values 1..9 and every row, column and 3x3 box holds each digit once. 9x9 boards. */
int nca_sudoku_valid(const int64_t *pred, const int64_t *inputs, const uint8_t *given,
                     int64_t rows, int32_t k_per_board, uint8_t *valid, void *stream);

/* The training step's update, fused: clip + AdamW + EMA + zero_grad in one launch
 * (<- the reference's clip_grad_norm_ in Engine.train_iteration, src/nca/engine/engine.py, and
 * its apply_update: the host test of the norm, torch.optim.AdamW.step, zero_grad and the EMA loop,
 * src/nca/engine/train.py:262-273). Flat fp32 device buffers of n elements: every parameter of
 * the cell back to back (params, their gradient, AdamW's two moments, the EMA weights).
 * counters (2) int64 on the device: [0] the number of applied AdamW steps (torch's `step`), [1]
 * the number of skipped iterations. One call: gn = ||grads||_2 (fixed summation order), written
 * to *grad_norm; with max_norm > 0 the gradient is scaled by min(1, max_norm / (gn + 1e-6));
 * when gn is finite counters[0] += 1 and AdamW updates params, exp_avg and exp_avg_sq with the
 * bias corrections of that count, else counters[1] += 1 and they keep their values; then
 * ema = d ema + (1 - d) params (ema_decay d >= 0; d < 0 leaves ema alone, which may be NULL) and
 * grads = 0. workspace: NCA_ADAMW_WORKSPACE_BYTES of device memory (nothing in it is kept). Two
 * launches, no host synchronisation; deterministic. */
typedef struct {
    double lr;           /* this iteration's learning rate (the schedule applied) */
    double beta1, beta2;
    double eps;
    double weight_decay; /* decoupled: params *= 1 - lr * weight_decay */
    double ema_decay;    /* this iteration's EMA decay, < 0 for none */
    double max_norm;     /* clip threshold, <= 0 for no clipping */
} nca_adamw_desc;

#define NCA_ADAMW_WORKSPACE_BYTES 1024 /* device workspace of nca_adamw_ema (the block sums) */

int nca_adamw_ema(float *params, float *grads, float *exp_avg, float *exp_avg_sq, float *ema,
                  int64_t n, const nca_adamw_desc *desc, int64_t *counters, float *grad_norm,
                  void *workspace, void *stream);

enum { NCA_DAMAGE_OURS = 0, NCA_DAMAGE_OFFICIAL = 1 };  /* perturb.py:43-83 geometries */

/* nca_damage_clamp <- apply_damage + apply_clamp of the training batch (src/nca/perturb.py:
 * 86-106, src/nca/train.py:219-244): in place on x (rows, channels, H, W) fp32, every channel of
 * a cell inside one of the discs is set to fill, then the channels [in_offset, in_offset + c_in)
 * of given cells take the clamp values (given (rows, H, W) {0,1} and clamp (rows, c_in, H, W);
 * given NULL: no clamp). discs (n_discs, 4) fp64 on the device: (row, cy, cx, r^2). Inside:
 * NCA_DAMAGE_OURS (y - cy)^2 + (x - cx)^2 <= r^2 with y, x the cell's row and column;
 * NCA_DAMAGE_OFFICIAL the same < r^2 with y, x = numpy linspace(-1, 1) coordinates; fp64, each
 * operation rounded once, as numpy evaluates it. */
int nca_damage_clamp(float *x, int64_t rows, int32_t channels, int32_t height, int32_t width,
                     const double *discs, int32_t n_discs, int32_t geometry, float fill,
                     const uint8_t *given, const float *clamp, int32_t c_in, int32_t in_offset,
                     void *stream);

/* nca_pool_rows <- the replay pool's indexing (src/nca/pool.py:96-179), every tensor of a batch
 * in one launch. Item i copies, for r < n_rows, row src_row[r] of src (row r when src_row is
 * NULL; nothing when src_row[r] < 0) to row dst_row[r] of dst (row r when NULL); rows are
 * row_bytes apart in both. mode 0 copies, mode 1 adds one to each int64 of the row (the pool's
 * age), mode 2 writes zeros (src unused). src_row / dst_row are device int64 arrays of n_rows;
 * at most 16 items; rows written by two items or two r race. */
typedef struct {
    const void *src;
    void *dst;
    const int64_t *src_row;
    const int64_t *dst_row;
    int64_t row_bytes;
    int32_t mode;
} nca_pool_row_copy;

int nca_pool_rows(const nca_pool_row_copy *items, int32_t n_items, int64_t n_rows, void *stream);

/* nca_init_state <- NCA.init_state (src/nca/model.py:384-412) for the noise drawn by the caller:
 * x (rows, channels, hw) = uniform ? (noise * 2 - 1) * sigma : noise * sigma, one rounding per
 * operation as the reference's torch expressions; clamp (rows, c_in, hw) = embed[token] (the
 * clamp values, model.py:378-382; embed is (vocab, c_in)); channels [in_off, in_off + c_in) of
 * given cells take the clamp values (apply_clamp, model.py:430-438). tokens int64 (rows, hw),
 * given (rows, hw) bytes, noise (rows, channels, hw) fp32; a token outside [0, vocab) gets NaN
 * clamp values. */
int nca_init_state(const float *noise, const int64_t *tokens, const uint8_t *given, const float *embed,
                   int32_t vocab, int64_t rows, int32_t channels, int32_t c_in, int32_t in_off, int32_t hw,
                   int32_t uniform, float sigma, float *x, float *clamp, void *stream);

/* Host-side batched board generation (the inputs of the workloads), on `threads` host threads
 * (0 = all). Every board draws from its own Philox4x32-10 stream keyed on `seed`, so the
 * output does not depend on the thread count. Buffers are host memory.
 *
 * nca_maze_boards <- generate_perfect_maze / generate_hard_maze (src/nca/tasks/maze.py:317-445):
 * n mazes of size x size: a spanning tree of the (size/2)^2 lattice by randomised depth-first
 * search, a fraction extra_openings of the interior walls between lattice cells removed, a
 * random start on an open cell and a random goal at BFS distance >= min_path_len - 1 (>= 1 when
 * min_path_len <= 0; up to max_tries draws per board). Tokens OPEN 0, WALL 1, START 2, GOAL 3,
 * PATH 4 (targets mark the BFS shortest path); inputs / targets (n, size, size) int64, given
 * (n, size, size) {0,1} (every non-open input), path_len (n) cells on the path. */
int nca_maze_boards(int64_t n, int32_t size, uint64_t seed, double extra_openings,
                    int32_t min_path_len, int32_t max_tries, int64_t *inputs, int64_t *targets,
                    uint8_t *given, int64_t *path_len, int32_t threads);

/* nca_sudoku_boards <- random_solution (src/nca/tasks/sudoku.py:290-294) plus a clue subset:
 * n solved grids (targets, values 1..9) with a uniformly random number of clues in
 * [clues_lo, clues_hi] kept at uniformly random cells (inputs, 0 elsewhere; given = clue). */
int nca_sudoku_boards(int64_t n, uint64_t seed, int32_t clues_lo, int32_t clues_hi,
                      int64_t *inputs, int64_t *targets, uint8_t *given, int32_t threads);

/* Bytes of the device scratch that nca_rollout_noalloc uses instead of a caller workspace. */
#define NCA_NOALLOC_SCRATCH_BYTES ((size_t)128 << 20)

/* nca_rollout_ws without a workspace argument and without any allocation. No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). The per-step path's state
 * buffers live in a device array of the library of NCA_NOALLOC_SCRATCH_BYTES (128 MiB: two
 * states of 16 boards of 201 x 201 cells with C = 16 take 83 MB), which every GPU the library
 * runs on holds from its first call until the process ends. A call whose per-step path needs
 * more (nca_rollout_workspace_bytes) returns NCA_ERR_UNSUPPORTED. Every call on one GPU shares
 * that array and the previous call's contents stay in it (nothing in it needs to start at
 * zero): calls that overlap on one GPU (other streams or threads) race, and the caller must
 * order them. Results equal nca_rollout_ws's bit for bit. */
int nca_rollout_noalloc(const nca_cell_desc *cell, const void *packed, int64_t rows,
                        int32_t height, int32_t width, const float *x_in, const uint8_t *given,
                        const float *clamp, float *x_out, const nca_fire_desc *fire,
                        int32_t n_steps, const float *noise, float *conf_out, int32_t *fired_out,
                        void *stream);

/* One step with an injected fire mask (rows, H, W) fp32 in {0,1}: the make_step drop-in. */
int nca_step(const nca_cell_desc *cell, const void *packed, int64_t rows, int32_t height,
             int32_t width, const float *x, const uint8_t *given, const float *clamp,
             const float *fire, const float *noise, float *x_out, void *stream);

/* Fire mask of one step: out (rows, H, W) uint8. conf_cell (rows, H, W) and given are read only
 * when fire->adaptive. fire->fire_in and fire->step_seeds are ignored (key = fire->seed). */
int nca_fire_mask(int64_t rows, int32_t height, int32_t width, const nca_fire_desc *fire,
                  int64_t step, const float *conf_cell, const uint8_t *given, uint8_t *out,
                  void *stream);

/* Readout of fp32 states x (rows, C, H, W): per-cell confidence (rows, H, W), board confidence
 * (rows) and argmax class index (rows, H, W); each output may be NULL. */
int nca_readout(const nca_cell_desc *cell, const void *packed, int64_t rows, int32_t height,
                int32_t width, const float *x, float *conf_cell, float *conf_board,
                int32_t *argmax, void *stream);

/* conf@K selection: best[n] = first argmax over trials t < k of conf[n, t] (alive[n, t] == 0
 * counts as -inf; alive may be NULL). conf (N, K) fp32, best (N) int32. */
int nca_conf_select(const float *conf, const uint8_t *alive, int32_t n_boards, int32_t k_trials,
                    int32_t k, int32_t *best, void *stream);

/* Gradients of the cell's parameters, fp32 device buffers in the reference's layouts. */
typedef struct nca_cell_grads {
    float *kernels; /* (heads, 1, 3, 3) */
    float *w1;      /* (hidden, F, 1, 1) */
    float *b1;      /* (hidden) */
    float *w2;      /* (C, hidden, 1, 1) */
    float *b2;      /* (C) */
    float *head_w;  /* (n_out, c_out, 1, 1) */
    float *head_b;  /* (n_out) */
    int32_t accumulate; /* 0: the gradients are written; 1: added to the buffers' contents (as
                           autograd adds into .grad) */
} nca_cell_grads;

/* The chunk loss: sum_t w_t * step_loss(x_{t+1}) / max(sum_t w_t, 1), step_loss = the mean over
 * cells (or the loss_mask-weighted mean, sum(l * mask) / max(sum(mask), 1)) of the per-cell
 * cross-entropy of the mlp head's logits against the target class. */
typedef struct nca_bptt_loss {
    const int32_t *targets;     /* device (rows, H, W) class index in [0, n_out) */
    const float *loss_mask;     /* device (rows, H, W) or NULL */
    const float *step_weights;  /* host (n_chunk): loss weight of each chunk step */
} nca_bptt_loss;

/* Workspace bytes of nca_bptt_backward for this shape (0 if the cell is unsupported). */
size_t nca_bptt_workspace_bytes(const nca_cell_desc *cell, int64_t rows, int32_t height,
                                int32_t width, int32_t n_chunk);

/* Forward of a BPTT chunk: states (n_chunk + 1, rows, C, H, W) receives x0 and the state after
 * every step, equal to nca_rollout's states bit for bit (bf16 C=32 boards up to 31 wide: one
 * fused launch of the streamed kernel that records every step; other cells and grids: one call
 * per step). fire->adaptive must be 0. States are all that the backward needs: it recomputes
 * everything else. */
int nca_bptt_forward(const nca_cell_desc *cell, const void *packed, int64_t rows, int32_t height,
                     int32_t width, const float *x0, const uint8_t *given, const float *clamp,
                     const nca_fire_desc *fire, int32_t n_chunk, float *states, void *stream);

/* nca_bptt_forward with a device workspace of workspace_bytes (the backward's, at least
 * nca_bptt_workspace_bytes of the same shape, may be passed; nothing in it is kept): the streamed
 * kernel then runs each board in two or three pieces of rows on as many workgroups, exchanging
 * their boundary rows through the workspace every step, when the device has a CU for every
 * piece. States are the same bit for bit in every case: a piece waits for its neighbour's rows
 * a bounded time (about a second); if the pieces of a board are not resident together (CUs held
 * by other work) and a wait runs out, the workspace's first 32-bit word is set to 1 and a repair
 * launch queued behind the pieces recomputes every board whole (when no wait ran out, that
 * launch's workgroups return at once). With workspace_bytes >= 256 the word is 0 otherwise, until
 * the workspace is next written (nca_bptt_backward overwrites it). Replaces the same reference
 * call as nca_bptt_forward (src/nca/engine/engine.py:478-489, the chunk's forward under
 * autograd). */
int nca_bptt_forward_ws(const nca_cell_desc *cell, const void *packed, int64_t rows, int32_t height,
                        int32_t width, const float *x0, const uint8_t *given, const float *clamp,
                        const nca_fire_desc *fire, int32_t n_chunk, float *states, void *workspace,
                        size_t workspace_bytes, void *stream);

/* Backward of the chunk whose forward wrote `states` (same cell, packed weights, fire desc).
 * w->w1 and w->w2 are the fp32 master weights (rounded to bf16 on load for bf16 cells, as the
 * forward used them). grad_final (rows, C, H, W), the gradient of a later loss w.r.t. the last
 * state, may be NULL (zero). Writes the parameter gradients of the chunk loss into `grads`
 * (overwritten, not accumulated), grad_x0 (rows, C, H, W; may be NULL), and the loss value into
 * loss_out (device scalar; may be NULL). Deterministic: every sum has a fixed order. */
int nca_bptt_backward(const nca_cell_desc *cell, const void *packed, const nca_cell_weights *w,
                      int64_t rows, int32_t height, int32_t width, const float *states,
                      const uint8_t *given, const nca_fire_desc *fire, int32_t n_chunk,
                      const nca_bptt_loss *loss, const float *grad_final, nca_cell_grads *grads,
                      float *grad_x0, float *loss_out, void *workspace, size_t workspace_bytes,
                      void *stream);

/* Bytes of workspace that nca_step_backward needs for this shape (0 if the cell is unsupported). */
size_t nca_step_backward_workspace_bytes(const nca_cell_desc *cell, int64_t rows, int32_t height,
                                         int32_t width);

/* Vector-Jacobian product of one nca_step: given the cotangent grad_out (rows, C, H, W) of the step's
 * output x_out = step(x, given, clamp, fire, noise), writes grads->kernels, w1, b1, w2, b2 (the
 * parameter gradients, overwritten) and grad_x (rows, C, H, W; may be NULL). fire (rows, H, W) fp32
 * is the step's fire value per cell (any real value: g_dx = g_u * fire); the noise and the clamp
 * values do not enter the gradient. grads->head_w / head_b are not written (the step does not use
 * the readout head). w->w1 and w->w2 are the fp32 weights (bf16 cells round them on load like the
 * forward). Any head kind. Deterministic. */
int nca_step_backward(const nca_cell_desc *cell, const void *packed, const nca_cell_weights *w,
                      int64_t rows, int32_t height, int32_t width, const float *x,
                      const uint8_t *given, const float *fire, const float *grad_out,
                      nca_cell_grads *grads, float *grad_x, void *workspace,
                      size_t workspace_bytes, void *stream);

/* Last error message of the calling thread ("" if none). */
const char *nca_last_error(void);

/* ABI version (major * 100 + minor). */
int nca_version(void);

/* Kernel selection: 0 = automatic (the streamed bf16 kernel where the grid allows it, the
 * resident kernel where the rows fit LDS, else the per-step path: the wave-per-tile kernel for
 * bf16 cells with 16 channels, the halo-window kernel for other cells; with
 * nca_set_window_steps(T >= 2), bf16 cells with 16 channels on the temporally blocked kernel, T
 * steps per launch on LDS-resident windows, for calls of two or more steps with uniform firing
 * and no noise), 1 = never the streamed kernel, 2 = always the per-step path with one step per
 * launch, 3 = always the per-step path on the halo-window kernel, 4 = the temporally blocked
 * kernel wherever it applies (2 steps per launch unless set), also on grids the resident kernels
 * take. Per calling thread (other threads keep their own setting); used by the tests to check
 * the paths against each other and by the bench to time each regime. No counterpart in the
 * reference. */
int nca_set_kernel_path(int path);

/* Steps per launch of the temporally blocked kernel (its windows' halo width), 1..8, or 0 for
 * the automatic choice (one step per launch: the per-step kernels). Per calling thread. No
 * counterpart in the reference (the reference has no temporal blocking). */
int nca_set_window_steps(int steps);

/* Pieces per board that nca_bptt_forward_ws plans for this shape on a device of `cus` CUs
 * (cus <= 0: the current device): 2 or 3 when every board's pieces fit the device at once, each
 * piece has enough rows and fits the LDS; 1 for whole boards; 0 for an unsupported cell or
 * grid. Host only. No counterpart in the reference. */
int32_t nca_bptt_forward_pieces(const nca_cell_desc *cell, int64_t rows, int32_t height,
                                int32_t width, int32_t cus);

/* Test settings of the pieces of nca_bptt_forward_ws, for every thread: spin_limit > 0 bounds a
 * wait for a neighbour's rows to that many re-reads; force_timeout != 0 makes every wait run out
 * (it looks for a tag that never comes), so a test sees the status word set and the repair run
 * while every kernel still ends; plan_cus > 0 plans pieces as for a device of that many CUs (more
 * workgroups than the device holds at once, so the pieces of some boards are not resident
 * together). (0, 0, 0) in use. No counterpart in the reference. */
int nca_set_piece_debug(int32_t spin_limit, int32_t force_timeout, int32_t plan_cus);

/* Test setting of nca_bptt_backward's path: 0 automatic (bf16 cells of 32 channels, 128 features
 * and 256 hidden units run the chunk's whole backward as one launch, on pieces of boards where
 * the device holds them, else on whole boards; other cells, three launches per step), 1 three
 * launches per step, 2 the one-launch backward on whole boards. The gradients of the paths agree
 * to fp32 rounding. No counterpart in the reference. */
int nca_set_bptt_backward_path(int32_t path);

#ifdef __cplusplus
}
#endif

#endif /* NCA_HIP_H */
