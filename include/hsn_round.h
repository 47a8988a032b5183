/*
 * hsn_round.h -- the fused cell round of one position on MI355X (gfx950): the sparse round of
 * every row's K selected (cell, unit) slots and the tick, forward only, in fp32.
 *
 * Replaces the reference's five kernels hsn_win_cell_front / _routes / _mlp_hidden / _mlp_out /
 * _cell_back (kernels/cuda/hsn_window.cu:226-531), which its python/hsn/kernels/window.py:233-330
 * (cell_round_op, the custom op "hsn::window_cell_round") launches; the contract is the native
 * round PDGCell.step_sparse (python/hsn/model/cell.py:349-505) followed by the tick
 * (python/hsn/model/state.py:316-324), with a hard decision (alpha 1 on valid slots, as
 * window.py:1007-1048 cell_round passes it) and the cell norm and GELU the reference's round
 * implements (window.py:202-230, cell_round_error).
 *
 * Per valid slot (row r, cell i = cells[r, k], unit j = units[r, k]), from the pre-round state:
 *   m   = V (sum_e edge_w[i, e] h[r, pad_src[i, e]])          (the window's padded edges)
 *   x   = [u[r]; eps[r]; h[r, i]; m],  v = norm_w x / sqrt(mean(x^2) + norm_eps)
 *   b   = sigmoid(gate_w v + gate_b)
 *   F   = W2[j]^T gelu(W1[j]^T v + b1[j]) + b2[j]              (exact, erf GELU)
 *   y   = W_out F;  c = tanh(alpha y / sqrt(mean(y^2) + cand_eps) cand_w)   (cand_norm)
 *                   c = tanh(W_out (alpha F))                                 (otherwise)
 *   h_new[r, i] = (1 - b) h[r, i] + b c
 * then q_new = q + sum_k (h_new - h)[cells k] / N over the valid slots (in slot order), age_new =
 * age + 1 with 0 at the written cells, h_sel[r, k] = h_new[r, cells[r, k]] (cell 0 on padded
 * slots); every cell no valid slot names keeps its state bit for bit.
 *
 * A slot is valid when valid[] is set and its cell lies in [0, N); a unit outside [0, M) reads
 * as the nearest unit and a padded source outside [0, N) as an absent edge, so the kernels never
 * index outside a buffer. A row's valid slots must name distinct cells (the router's top-k).
 * The call returns once its three launches are enqueued on `stream` (a hipStream_t; NULL: the
 * default stream), with the status codes of hsn_ops.h and the message in hsn_win_last_error().
 * Nothing is allocated: `work` is the caller's scratch of hsn_win_cell_round_workspace() bytes.
 */
#ifndef HSN_ROUND_H
#define HSN_ROUND_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct hsn_cell_round {
    /* shape: rows, cells, width, slots, units, hidden units, padded in-degree (0: no edges) */
    int32_t B, N, d, K, M, H, D;
    int32_t cand_norm; /* 1: the candidate norm with cand_w and cand_eps */
    float norm_eps;    /* the cell norm's eps */
    float cand_eps;
    /* the position's inputs and the state before it */
    const float* u;         /* [B, d] */
    const float* eps;       /* [B, d] */
    const float* h;         /* [B, N, d] */
    const float* q;         /* [B, d] */
    const int64_t* age;     /* [B, N] */
    const int64_t* cells;   /* [B, K] */
    const int64_t* units;   /* [B, K] */
    const uint8_t* valid;   /* [B, K] */
    const float* alpha;     /* [B, K] */
    /* the cell's weights (nn.Linear layouts: out = W x with W [out, in] row-major) */
    const float* V;         /* [d, d] */
    const float* edge_w;    /* [N, D]: the padded edge weights, 0 on padding (NULL when D is 0) */
    const int64_t* pad_src; /* [N, D]: each cell's sources, 0 on padding (NULL when D is 0) */
    const float* norm_w;    /* [4 d] */
    const float* gate_w;    /* [d, 4 d] */
    const float* gate_b;    /* [d] */
    const float* W1;        /* [M, 4 d, H] */
    const float* b1;        /* [M, H] */
    const float* W2;        /* [M, H, d] */
    const float* b2;        /* [M, d] */
    const float* W_out;     /* [d, d] */
    const float* cand_w;    /* [d] (cand_norm; else unused) */
    void* work;             /* hsn_win_cell_round_workspace() bytes; work, u, eps, h and h_new
                             * 16-byte aligned */
    /* the state after the position and the selected slots' new states */
    float* h_new;      /* [B, N, d] */
    float* q_new;      /* [B, d] */
    int64_t* age_new;  /* [B, N] */
    float* h_sel;      /* [B, K, d] */
} hsn_cell_round;

/* Whether the fused round takes this shape: HSN_OK, or an error status with the reason in
 * hsn_win_last_error() (the reference's cell_round_error, window.py:202-230). Reads only the
 * sizes and whether the pointers are set. */
int hsn_win_cell_round_check(const hsn_cell_round* round);

/* The scratch bytes `work` must hold for this shape (*bytes; sizes only). */
int hsn_win_cell_round_workspace(const hsn_cell_round* round, int64_t* bytes);

/* The round of one position (reference window.py:233-330 cell_round_op's five launches). */
int hsn_win_cell_round(const hsn_cell_round* round, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* HSN_ROUND_H */
