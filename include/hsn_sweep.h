/*
 * hsn_sweep.h -- the state-gradient reverse sweep's glue steps on MI355X (gfx950): the head, the
 * middle and the tail of one position of the P2.10c sweep, between which the caller runs the two
 * transposed all-units products of the cell (plain GEMMs on the operands these steps write).
 *
 * Replaces the reference's hsn_win_back_head / _mid / _tail (kernels/cuda/hsn_window.cu:956-1427),
 * which its python/hsn/kernels/window.py:1182-1270 (back_head, back_mid, back_tail) launches on
 * the buffers of a ReverseSweep (python/hsn/train/state_sweep.py:112-662); the contract of each
 * step is the reference's PyTorch glue (state_sweep.py head_reference, middle_reference,
 * tail_reference). Here the buffers are described by one plain struct of device pointers and
 * sizes, `hsn_back_sweep`; every call returns once its work is enqueued on `stream` (a
 * hipStream_t; NULL: the default stream), with the status codes of hsn_ops.h and the message in
 * hsn_win_last_error(). Nothing is allocated, so a position's five launches can be captured in a
 * graph and replayed for every window of the shape.
 *
 * Per position t (T-1 down to 0):
 *   head    R += d_q_post[t]; A[fast cells] += d_h_fast[t]; A[cell_k] += d_h_sel[t, k];
 *           g = A[cell_k] + R / N; dc = b g; db = (c - h_old) g; A[cell_k] = (1 - b) A[cell_k]
 *           - b R / N; the candidate's backward (dz = dc (1 - c^2), the candidate norm's with
 *           alpha, cand_gain and the recorded y) into op1's unit block; the gate's backward
 *           dg = db b (1 - b) into op2's gate columns; sigma = <gate_pre - gate_bias, dg>
 *   (caller) act = op1 . w2_t                     [B K, M d] x [M d, H]
 *   middle  dh = act' (hidden) . act into op2's unit block; sigma += <hidden - b1, dh>
 *   (caller) dv = op2 . w1_state_t                [B K, M H + d] x [M H + d, 2 d]
 *   tail    ds = r dv - (r^2 / in_dim) sigma [h_old; m V] (the cell norm's backward; ds = dv
 *           without it); A[cell_k] += ds[:d]; every cell adds, in its out-adjacency's order, its
 *           edge weight times ds[d:] of each selected cell it is a message source of;
 *           R += d_q_pre[t]; a reset zeroes the row's A and R.
 * A routed slot writes its unit's block of op1 / op2 and clears the block position t + 1 used,
 * so the operands are zeroed once per window (by the caller), not per position. Padded slots
 * (slots[] < 0) give exact zeros and touch no state cotangent. A position's valid slots hold
 * distinct cells (the router's top-k). The kernels never index outside a buffer: a cell outside
 * [0, N) reads as a padded slot and a unit outside [0, M) as the nearest unit; the Python
 * wrapper rejects such values before it loads a window.
 */
#ifndef HSN_SWEEP_H
#define HSN_SWEEP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HSN_ACT_GELU 0 /* exact (erf) GELU */
#define HSN_ACT_RELU 1
#define HSN_ACT_SILU 2
#define HSN_ACT_TANH 3

typedef struct hsn_back_sweep {
    /* shape */
    int32_t B, T, K, N, d, H, M;
    int32_t n_read;        /* fast-read cells 0 .. n_read-1 (A8); 0: none */
    int32_t in_dim;        /* the cell norm's width n */
    int32_t d_out;         /* the out-adjacency's width */
    int32_t d_in;          /* the in-adjacency's width (the padded sources per cell) */
    int32_t product_dtype; /* HSN_DTYPE_F32 or HSN_DTYPE_BF16: hidden, op1, op2, act, dv */
    int32_t activation;    /* HSN_ACT_* */
    int32_t cand_norm;     /* 1: c = tanh(alpha RMSNorm(y)) with cand_gain, cand_eps */
    int32_t cell_norm;     /* 1: the cell norm's backward with rms */
    float cand_eps;
    /* the state's cotangent and the per-slot inner products (read and written) */
    float* A;     /* [B, N, d] */
    float* R;     /* [B, d] */
    float* sigma; /* [B, K] */
    /* the window's record */
    const float* c;        /* [B, T, K, d] */
    const float* b;        /* [B, T, K, d] */
    const float* h_old;    /* [B, T, K, d] */
    const float* y;        /* [B, T, K, d] (cand_norm) */
    const float* gate_pre; /* [B, T, K, d] */
    const float* mv;       /* [B, T, K, d]: the messages through V, m @ v (cell_norm) */
    const float* alpha;    /* [B, T, K] */
    const float* rms;      /* [B, T, K] (cell_norm) */
    const void* hidden;    /* [B, T, K, H] in product_dtype */
    const int32_t* slots;  /* [B, T, K]: the cell, -1 on padded slots */
    const int32_t* units;  /* [B, T, K]: the unit (0 on padded slots) */
    const uint8_t* reset;  /* [B, T] */
    /* the cotangents of the node's outputs */
    const float* d_q_pre;  /* [B, T, d] */
    const float* d_q_post; /* [B, T, d] */
    const float* d_h_sel;  /* [B, T, K, d] */
    const float* d_h_fast; /* [B, T, n_read, d]; NULL when n_read is 0 */
    /* the cell's constants */
    const float* cand_gain; /* [d] (cand_norm) */
    const float* gate_bias; /* [d] */
    const float* b1;        /* [M, H] */
    const int32_t* out_tgt; /* [N, d_out]: targets of each cell's out-edges, -1 on padding */
    const float* out_w;     /* [N, d_out]: their edge weights, 0 on padding */
    const int32_t* in_src;  /* [N, d_in]: each cell's message sources, -1 on padding */
    /* the products' operands and results, in product_dtype */
    void* op1;       /* [B K, M d] */
    void* op2;       /* [B K, M H + d] */
    const void* act; /* [B K, H] */
    const void* dv;  /* [B K, 2 d]: [g_h dv_h ; (g_m dv_m) V] */
    /* what the sweep returns */
    float* dc; /* [B, T, K, d] */
    float* db; /* [B, T, K, d] */
    /* the fused step's weights (hsn_win_back_cell), in product_dtype, each unit's matrix with
     * its reduction index contiguous: w2f [M, H, d] holds (W_out W2_j^T)^T, w1f [M, 2 d, H + d]
     * holds ([W1_s; G_s]^T blockdiag(diag(g_h), diag(g_m) V))^T restricted to unit j's rows */
    const void* w2f;
    const void* w1f;
    float* carry; /* [B K, d]: the fused step's (1 - b) carried - b R / N per slot, for its tail */
    float* ds;    /* [B K, 2 d]: the fused step's cell-norm backward [ds_h ; ds_m] per slot */
} hsn_back_sweep;

/* Whether the glue steps take this sweep (sizes, dtypes, LDS): HSN_OK, or an error status with
 * the reason in hsn_win_last_error() (the reference's back_unsupported, window.py:1165-1176). */
int hsn_win_back_check(const hsn_back_sweep* sweep);

/* The head of position t (reference hsn_window.cu hsn_win_back_head; state_sweep.py
 * head_reference). */
int hsn_win_back_head(const hsn_back_sweep* sweep, int t, void* stream);

/* The middle of position t (hsn_win_back_mid; state_sweep.py middle_reference). */
int hsn_win_back_mid(const hsn_back_sweep* sweep, int t, void* stream);

/* The tail of position t (hsn_win_back_tail; state_sweep.py tail_reference). */
int hsn_win_back_tail(const hsn_back_sweep* sweep, int t, void* stream);

/*
 * No counterpart in the reference: the head, both products and the middle of position t as one
 * launch on the matrix cores. A workgroup takes 16 slots of one unit (the slots of unit j in slot
 * order), runs the head on them, then act = du . (W_out W2_j^T) and dv = [dh ; dg] . w1f_j on
 * v_mfma tiles (bf16 in, fp32 accumulation; fp32 tiles for fp32 products) with only the unit's
 * own blocks (the all-units layout multiplies M times as much, mostly zeros), writing dc, db,
 * sigma, each slot's carry and its cell-norm backward ds (A itself is only read). The operands op1 / op2 and act are not
 * used; values are rounded to product_dtype where the reference's products store them. Follow it
 * with hsn_win_back_cell_tail (not hsn_win_back_tail): the tail writes the selected cells' rows
 * of A from the carry, R, and the unselected fast-read cells. hsn_win_back_cell_check says whether a sweep takes this step
 * (d % 8 == 0, H % 8 == 0 and its LDS).
 */
int hsn_win_back_cell_check(const hsn_back_sweep* sweep);
int hsn_win_back_cell(const hsn_back_sweep* sweep, int t, void* stream);

/* The tail after hsn_win_back_cell: hsn_win_back_tail's work, plus R += d_q_post[t] (before its
 * d_q_pre[t]) and the decoder's cotangent of the fast-read cells no slot selected. */
int hsn_win_back_cell_tail(const hsn_back_sweep* sweep, int t, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* HSN_SWEEP_H */
