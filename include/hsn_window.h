/*
 * hsn_window.h -- the C ABI of the MI355X (gfx950) window hot path of HSN: the top-k cell
 * router, the forward sweep (sparse gather / gated update / scatter with the summary coupling),
 * the backward recurrence and the carried-state gradient.
 *
 * Conventions (every function)
 * ----------------------------
 * - Shapes: B rows, T positions of a window, N cells, d state width, K slots per position,
 *   M units. Tensors are dense, row-major and contiguous (the last index fastest), except where
 *   a function documents a row stride.
 * - The state (h, q and their cotangents A, R) is fp32. Inputs and per-slot outputs are stored
 *   in `io_dtype` (HSN_DTYPE_F32 or HSN_DTYPE_BF16) and computed in fp32.
 * - Cells and units: `index_bits` 32 (int32_t) or 64 (int64_t). valid, refreshed and reset are
 *   uint8_t holding 0 / 1 (torch.bool storage).
 * - Caller-allocated outputs; no function allocates device memory, so every call is legal
 *   under stream capture. A pointer documented as optional may be NULL.
 * - `stream` is a hipStream_t (NULL: the default stream). Functions return once the work is
 *   enqueued and check what needs no synchronisation (dimensions, dtypes, sizes, pointers);
 *   index preconditions (cells in [0, N), distinct valid cells per position) are the caller's.
 * - Return value: HSN_OK or an HSN_ERR_* code of hsn_ops.h (the same numbering).
 */
#ifndef HSN_WINDOW_H
#define HSN_WINDOW_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#ifndef HSN_OK
#define HSN_DTYPE_F32 0
#define HSN_DTYPE_F16 1
#define HSN_DTYPE_BF16 2
#define HSN_OK 0
#define HSN_ERR_INVALID_ARGUMENT 1
#define HSN_ERR_UNSUPPORTED_DTYPE 2
#define HSN_ERR_INDEX_OUT_OF_RANGE 3
#define HSN_ERR_DUPLICATE_INDEX 4
#define HSN_ERR_SIZE_OVERFLOW 5
#define HSN_ERR_BAD_GRAPH 6
#define HSN_ERR_BACKEND 7
#endif

/* ABI version of this header (bumped on any signature or semantic change). */
#define HSN_WINDOW_ABI_VERSION 2
int hsn_win_abi_version(void);

/* The last error message of the calling thread ("" if none); valid until the next call. */
const char* hsn_win_last_error(void);

/*
 * Whether an entry point takes a shape, decided on the host by the launchers' own checks and
 * geometry (no GPU work, no launch): HSN_OK, or HSN_ERR_INVALID_ARGUMENT with the reason in
 * hsn_win_last_error(). This is what the Python wrappers consult to decline (return None) as
 * the reference's wrappers do (python/hsn/kernels/window.py:119-128,557-565,626-640).
 *   op: HSN_OP_FORWARD, HSN_OP_BACKWARD, HSN_OP_RECURRENCE, HSN_OP_CELL_UPDATE, HSN_OP_ROUTE
 *   (hsn_win_route and hsn_win_select); T is ignored for the per-position ops.
 */
#define HSN_OP_FORWARD 0
#define HSN_OP_BACKWARD 1
#define HSN_OP_RECURRENCE 2
#define HSN_OP_CELL_UPDATE 3
#define HSN_OP_ROUTE 4
int hsn_win_supports(int op, int B, int T, int N, int d, int K);

/*
 * The three designs of the window's sweeps. No counterpart in the reference (its fused sweep is
 * one design); these choose between this library's three, which compute the same outputs to the
 * parity tolerance:
 *   HSN_PATH_SLICE  time-chunked slices of the state resident in LDS (a workgroup per row and
 *                   column slice): a wavefront's piece of a slot row is S columns, S * K <= 64;
 *   HSN_PATH_CHAIN  cell chains (a wavefront per cell walks the cell's events in time; whole
 *                   slot rows per load and store; the summary by a scan over time): any N, K
 *                   up to 255, d up to 256;
 *   HSN_PATH_EVMAP  event maps (a workgroup per row and 8 columns; a chunk of up to 16
 *                   positions per half-wavefront composes each touched cell's affine map over
 *                   the chunk, every cell is walked through the 16 chunks' maps, then each chunk
 *                   replays its positions from the cells' values at its edge; the backward
 *                   runs the same steps in reverse time after an fp64 scan of the summary
 *                   cotangent): fp32 rows, d a multiple of 8, T <= 256, K <= 8, the tables of
 *                   N cells within the LDS (N up to about 1000); no workspace.
 * hsn_win_set_path fixes the path of every later hsn_win_forward / hsn_win_forward_noalloc /
 * hsn_win_backward call of the process. HSN_PATH_AUTO, the default: the event maps where they
 * take the shape and their B * d / 8 workgroups run in one round of the 256 CUs; otherwise the
 * slices where their piece is a full sector and N * S <= 2048, else the chains. hsn_win_path reports the path a call of `op` (HSN_OP_FORWARD or
 * HSN_OP_BACKWARD) would take, or the reason none takes the shape.
 */
#define HSN_PATH_AUTO 0
#define HSN_PATH_SLICE 1
#define HSN_PATH_CHAIN 2
#define HSN_PATH_EVMAP 3
int hsn_win_set_path(int path);
int hsn_win_path(int op, int B, int T, int N, int d, int K, int io_dtype, int* path);

/*
 * The workspace hsn_win_forward / hsn_win_backward need, in bytes (0: none), for `op`
 * HSN_OP_FORWARD or HSN_OP_BACKWARD on the path the call takes: the RMS candidate's normalised
 * input (cand_norm 1) and, on the chain path, the row lists, the per-position sums, the
 * forward's fp32 per-slot deltas (used with bf16 rows, or where h_old or h_sel is omitted) and
 * its row-maximum table per workgroup of cells. No counterpart in the reference (its sweep keeps the state in
 * shared memory and allocates through torch).
 */
int hsn_win_workspace_bytes(int op, int B, int T, int N, int d, int K, int io_dtype,
                            int cand_norm, int64_t* bytes);

/*
 * Router: the hard top-k decision of every position of a window.
 * Replaces the per-position `hsn_win_select` launches of the fused sweep
 * (reference kernels/cuda/hsn_window.cu:533-749, wrapper python/hsn/kernels/window.py:356-423)
 * and restates Router.select(mode="topk") (python/hsn/model/router.py:1263-1417).
 *
 *   logits [B,T,N,width] (io_dtype f32 or bf16; the first M columns of each cell's row are the
 *          unit logits, width >= M; width = M for a plain tensor)
 *   cost [M] f32 (the cost table)
 *   age0 [B,N] int64, reset [B,T] u8: read only with probes (the ages evolve with the
 *          decisions, so a window with probes is walked position by position per row)
 *   cells, units [B,T,K] (index_bits), valid, refreshed [B,T,K] u8, theta [B,T] f32
 *   slots [B,T,K] int32, optional: the slot's cell where valid, -1 where padded (the packed
 *          decision the sweeps read)
 *   h_max_zero [B,T] f32, optional: set to 0 (the forward sweep max-reduces into it)
 * For every position: score_i = max_j (logit_ij - lambda cost_j) (fp32, no contraction), unit
 * the first maximiser; cells sorted by descending score, ties by index (NaN first, -0 = +0,
 * reserved cells 0..reserved-1 first); the first K slots; valid = shared + cumsum(overhead +
 * cost[unit]) <= limit (the prefix sums in double rounded to fp32, as the CPU oracle's torch
 * cumsum); padded slots cell 0 / unit 0; theta = (lowest selected + highest unselected) / 2;
 * with probes the stalest unselected cells over age_max replace the valid slots from the last
 * one backwards unless that exceeds the limit.
 */
int hsn_win_route(const void* logits, int io_dtype, int64_t width, const float* cost,
                  const int64_t* age0, const uint8_t* reset, void* cells, void* units,
                  int index_bits, uint8_t* valid, float* theta, uint8_t* refreshed,
                  int32_t* slots, float* h_max_zero, int B, int T, int N, int M, int K,
                  int age_max, int probes,
                  float lambda_cost, float cell_overhead, float shared_cost, float limit,
                  int reserved, int reserved_units, void* stream);

/*
 * One position's decision, the reference's per-position form (plain, tape and folded):
 * kernels/cuda/hsn_window.cu:533-749 `hsn_win_select`, wrappers select_op / select_tape_op /
 * select_fold_op (python/hsn/kernels/window.py:356-530).
 *   logits: [B*N, width] rows (io_dtype), the first M columns are the logits
 *   age [B, n_age, N] int64 (record t read; only with probes); cost [M] f32
 *   cells, units [B, n_out, K] int64; valid, refreshed [B, n_out, K] u8; theta [B, n_out] f32:
 *   record t is written in full, no other record is touched.
 */
int hsn_win_select(const void* logits, int io_dtype, int64_t width, const int64_t* age,
                   const float* cost, int64_t* cells, int64_t* units, uint8_t* valid,
                   float* theta, uint8_t* refreshed, int B, int N, int M, int K, int t, int n_out,
                   int n_age, int age_max, int probes, float lambda_cost, float cell_overhead,
                   float shared_cost, float limit, int reserved, int reserved_units, void* stream);

/*
 * Forward sweep of a window with the state resident on chip: per position reset -> candidate
 * and gate -> gated update of the valid slots' cells -> summary -> tick. Replaces the
 * per-position `hsn_win_cell_update` launches and the full-state tape of the fused sweep
 * (kernels/cuda/hsn_window.cu:751-954; python/hsn/train/compile.py:892-1024,1296-1362;
 * python/hsn/kernels/native.py:244-303; python/hsn/model/state.py:267-324).
 *   y, gate_pre [B,T,K,d] io_dtype: candidate input and write-gate pre-activation
 *   c = tanh(y) (cand_norm 0) or tanh(y * rsqrt(mean_d(y^2) + cand_eps) * cand_w) (cand_norm 1,
 *   cand_w [d] f32); b = sigmoid
 *   workspace: workspace_bytes >= what hsn_win_workspace_bytes(HSN_OP_FORWARD, ...) reports
 *   (may be NULL where that is 0)
 *   reset [B,T] u8; slots [B,T,K] int32 (hsn_win_route's packed decision: cell or -1)
 *   h0 [B,N,d], q0 [B,d] f32; age0 [B,N], pos0 [B] int64
 * Outputs (each optional): q_pre, q_post [B,T,d] io_dtype (summary before / after each
 * position), h_sel [B,T,K,d] io_dtype (the slots' cells after the update; cell 0 on padded
 * slots), h_old [B,T,K,d] io_dtype (the slots' cells before the update: the backward's tape),
 * h_max [B,T] f32 (row max |h| after each position, NaN-propagating; must hold 0 on entry:
 * hsn_win_route zeroes it), h_T [B,N,d], q_T [B,d] f32, age_T [B,N], pos_T [B] int64.
 */
int hsn_win_forward(const void* y, const void* gate_pre, int io_dtype, const float* cand_w,
                    int cand_norm, float cand_eps, void* workspace, int64_t workspace_bytes,
                    const uint8_t* reset,
                    const int32_t* slots, const float* h0, const float* q0, const int64_t* age0,
                    const int64_t* pos0, void* q_pre, void* q_post, void* h_sel, void* h_old,
                    float* h_max, float* h_T, float* q_T, int64_t* age_T, int64_t* pos_T, int B,
                    int T, int N, int d, int K, void* stream);

/*
 * hsn_win_forward without the workspace argument: an entry point that allocates nothing and
 * takes no workspace. It has no counterpart in the reference; it is for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc). The workspace hsn_win_forward would take (hsn_win_workspace_bytes, on the
 * same path) is a device array of 32 MiB that the library owns (one per GPU, held until the
 * process ends): shapes whose workspace exceeds it return HSN_ERR_SIZE_OVERFLOW (the slice
 * path needs one only for the RMS candidate: about 129,000 slots of d = 64 in fp32; the chain
 * path about 4 (d + 1 + d / K) bytes per slot). Every call on a GPU shares that GPU's array,
 * so calls that overlap on one GPU (other streams or threads) race; calls ordered on one
 * stream do not. Arguments, outputs and results are those of hsn_win_forward.
 */
int hsn_win_forward_noalloc(const void* y, const void* gate_pre, int io_dtype,
                            const float* cand_w, int cand_norm, float cand_eps,
                            const uint8_t* reset, const int32_t* slots, const float* h0,
                            const float* q0, const int64_t* age0, const int64_t* pos0,
                            void* q_pre, void* q_post, void* h_sel, void* h_old, float* h_max,
                            float* h_T, float* q_T, int64_t* age_T, int64_t* pos_T, int B, int T,
                            int N, int d, int K, void* stream);

/*
 * Route and forward sweep of a window as one call: hsn_win_route (without probes) followed by
 * hsn_win_forward on its slots, the two steps of every position of the reference's fused sweep
 * (the per-position `hsn_win_select` and `hsn_win_cell_update` launches,
 * kernels/cuda/hsn_window.cu:533-954; the position loop of python/hsn/train/compile.py:892-1024).
 * Arguments are those two calls' (the router's first, then the forward's; `slots` is required,
 * the backward's decisions; h_max needs no zeroing); outputs and results are bit for bit theirs.
 * With hsn_win_set_route_forward(HSN_ROUTE_FORWARD_ONE), where the event maps take the forward
 * (HSN_PATH_EVMAP), the router has one unit (M = 1), the logits and rows are f32, the decisions
 * int32 (index_bits 32), N <= 512, B * d / 8 <= 256 and the device's compute units, and
 * ceil(T / (d / 8)) <= 32, it is one launch: the forward's workgroups of a row each decide a
 * share of the row's positions and hand the decisions to each other through device memory the
 * library owns (one set a GPU). Those buffers serve one stream a GPU, the first that fuses;
 * calls on other streams, or on a capturing stream, take the two launches. The default,
 * HSN_ROUTE_FORWARD_AUTO, takes the two launches (faster at the ref shape on MI355X: the one
 * launch's wavefronts decide four positions each with two wavefronts a SIMD to hide the
 * decisions' latency); HSN_ROUTE_FORWARD_TWO always does. No counterpart in the reference for
 * the setting. hsn_win_route_forward_fuses reports which a call takes (without claiming the
 * buffers; the reason in hsn_win_last_error when it is two).
 */
#define HSN_ROUTE_FORWARD_AUTO 0
#define HSN_ROUTE_FORWARD_ONE 1
#define HSN_ROUTE_FORWARD_TWO 2
int hsn_win_set_route_forward(int mode);
int hsn_win_route_forward(const void* logits, int logits_dtype, int64_t width, const float* cost,
                          void* cells, void* units, int index_bits, uint8_t* valid, float* theta,
                          uint8_t* refreshed, int32_t* slots, int M, float lambda_cost,
                          float cell_overhead, float shared_cost, float limit, int reserved,
                          int reserved_units, const void* y, const void* gate_pre, int io_dtype,
                          const float* cand_w, int cand_norm, float cand_eps, void* workspace,
                          int64_t workspace_bytes, const uint8_t* reset, const float* h0,
                          const float* q0, const int64_t* age0, const int64_t* pos0, void* q_pre,
                          void* q_post, void* h_sel, void* h_old, float* h_max, float* h_T,
                          float* q_T, int64_t* age_T, int64_t* pos_T, int B, int T, int N, int d,
                          int K, void* stream);
int hsn_win_route_forward_fuses(int M, int logits_dtype, int index_bits, int io_dtype,
                                int cand_norm, int B, int T, int N, int d, int K, void* stream,
                                int* fuses);
/*
 * The one-launch route and forward's waits for another workgroup's word that reached their
 * limit (about a second each; only a grid whose workgroups cannot all be resident at once waits
 * that long, and its results are then not to be used), counted since the last clear. Waits for
 * the device's work to finish first. No counterpart in the reference.
 */
int hsn_win_exchange_timeouts(unsigned* count, int clear);

/*
 * Backward of the window with the activations fused and the carried-state gradient: the
 * reverse recurrence of python/hsn/train/split.py:128-174 (A [N,d], R [d] resident on chip),
 * seeded with the end-state cotangent (python/hsn/train/state_gradient.py:402-416), the VJPs
 * of tanh / RMSNorm and sigmoid (the replay's autograd, python/hsn/train/split.py:588-716),
 * and the start-state cotangent that split.py:173-174 drops.
 *   y, gate_pre, h_old [B,T,K,d] io_dtype; slots [B,T,K] int32; reset [B,T] u8
 *   d_q_pre, d_q_post [B,T,d], d_h_sel [B,T,K,d] io_dtype (optional: absent = zero)
 *   d_h_T [B,N,d], d_q_T [B,d] f32 (optional: absent = zero)
 * Outputs: dy, dgate [B,T,K,d] io_dtype (exact zeros on padded slots); d_h0 [B,N,d], d_q0 [B,d]
 * f32 (optional); d_cand_w [d] f32 (cand_norm 1).
 *   workspace: workspace_bytes >= what hsn_win_workspace_bytes(HSN_OP_BACKWARD, ...) reports.
 */
int hsn_win_backward(const void* y, const void* gate_pre, const void* h_old, int io_dtype,
                     const float* cand_w, int cand_norm, float cand_eps, void* workspace,
                     int64_t workspace_bytes,
                     const int32_t* slots, const uint8_t* reset, const void* d_q_pre,
                     const void* d_q_post, const void* d_h_sel, const float* d_h_T,
                     const float* d_q_T, void* dy, void* dgate, float* d_h0, float* d_q0,
                     float* d_cand_w, int B, int T, int N, int d, int K, void* stream);

/*
 * The reference's backward recurrence from the candidate and gate themselves (no activation):
 * kernels/cuda/hsn_window.cu:50-115 `hsn_win_recurrence`, wrapper recurrence_backward
 * (python/hsn/kernels/window.py:108-153), contract python/hsn/train/split.py:128-174.
 *   c, b, h_old [B,T,K,d] f32; cells [B,T,K] int64 (0 on padded); valid [B,T,K], reset [B,T] u8;
 *   d_q_pre, d_q_post [B,T,d], d_h_sel [B,T,K,d] f32 (optional); dc, db [B,T,K,d] f32.
 *   Carried state (optional, new): d_h_T [B,N,d], d_q_T [B,d] seed A, R; d_h0 [B,N,d],
 *   d_q0 [B,d] receive A, R after position 0.
 * No limit on N * d (the reference declines above 48 KiB of shared memory).
 */
int hsn_win_recurrence(const float* c, const float* b, const float* h_old, const int64_t* cells,
                       const uint8_t* valid, const uint8_t* reset, const float* d_q_pre,
                       const float* d_q_post, const float* d_h_sel, const float* d_h_T,
                       const float* d_q_T, float* dc, float* db, float* d_h0, float* d_q0, int B,
                       int T, int K, int d, int N, void* stream);

/*
 * The dense-fallback rows' recurrence: kernels/cuda/hsn_window.cu:117-163
 * `hsn_win_recurrence_dense`, wrapper python/hsn/kernels/window.py:156-192, contract
 * python/hsn/train/split.py:177-209.
 *   c, b, h_old [Bd,T,N,d] f32; reset [Bd,T] u8; d_q_pre, d_q_post [Bd,T,d] f32 (optional);
 *   dc, db [Bd,T,N,d] f32.
 */
int hsn_win_recurrence_dense(const float* c, const float* b, const float* h_old,
                             const uint8_t* reset, const float* d_q_pre, const float* d_q_post,
                             float* dc, float* db, int Bd, int T, int N, int d, void* stream);

/*
 * One position's end of round, the reference's per-position form (plain and tape):
 * kernels/cuda/hsn_window.cu:751-954 `hsn_win_cell_update`, wrappers cell_update_op /
 * update_tape_op (python/hsn/kernels/window.py:605-760).
 *   y [B,K,d], gate [B,K,d] io_dtype (the round's products); cand_w [d] f32 (cand_norm 1;
 *   rms_scratch a workspace of R(B*K) bytes, R(s) = align16(s*d*sizeof(io)) + 4*s)
 *   h [B,n_state,N,d], q [B,n_state,d] f32, age [B,n_state,N] int64: record t read
 *   pos [B] int64 (optional), cells [B,n_slot,K] int64, valid [B,n_slot,K] u8: record t
 *   h_next, q_next, age_next: record t_out written (may be the buffers above, t_out != t);
 *   pos_next [B] (optional); h_sel [B,n_slot,K,d] f32; h_max [B,n_slot] f32 (record t);
 *   reset [B,n_slot] u8 (optional: reset[:, t+1] zeroes the written record; never for the last
 *   record); q_post [B,n_slot,d] f32 (optional, the summary after the round).
 */
int hsn_win_cell_update(const void* y, const void* gate, int io_dtype, const float* cand_w,
                        int cand_norm, float cand_eps, void* rms_scratch, const float* h,
                        const float* q, const int64_t* age, const int64_t* pos,
                        const int64_t* cells, const uint8_t* valid, float* h_next,
                        float* q_next, int64_t* age_next, int64_t* pos_next, float* h_sel,
                        float* h_max, const uint8_t* reset, float* q_post, int B, int N, int d,
                        int K, int t, int n_state, int n_slot, int t_out, void* stream);

/*
 * The folded sweep's row (reference kernels/cuda/hsn_window.cu:770-779,887-920, the extra output
 * of update_fold_op, python/hsn/kernels/window.py:765-853): after hsn_win_cell_update has
 * written record t_next of the state tape, the next position's input row of the first product,
 *   x[t_next, b, :] = [z[b, t_next, :]; q[b, t_next, :]; context[b, t_next, :] (; f[b, :])],
 * every value rounded once to x_dtype (round to nearest even for bf16); f, present when
 * n_fast = F > 0, is the mean of cells 0 .. F-1 of state record t_next, summed in cell order
 * (the fast readout, model.fast_readout).
 *   x [n, B, d_z + d + d_c (+ d)] x_dtype (f32 or bf16); z [B, n, d_z] z_dtype; context
 *   [B, n, d_c] c_dtype; tape_q [B, n_state, d], tape_h [B, n_state, N, d] f32; 1 <= t_next < n.
 */
int hsn_win_fold_row(void* x, int x_dtype, const void* z, int z_dtype, int d_z,
                     const void* context, int c_dtype, int d_c, const float* tape_q,
                     const float* tape_h, int n_fast, int B, int N, int d, int n, int n_state,
                     int t_next, void* stream);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* HSN_WINDOW_H */
