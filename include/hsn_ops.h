/*
 * hsn_ops.h -- the numerical C ABI of HSN's sparse round for MI355X: the two ops on the window
 * hot path (the gated delta update and the gather of the selected cells) and the cell round's
 * grouped unit MLP and CSR neighbour messages.
 *
 * Same function names, argument order, dtype codes and status codes as the reference's ABI
 * (kernels/include/hsn_ops.h:64-187), so a host that binds that header binds this library
 * unchanged. Conventions as there: dense row-major tensors, int32_t indices, one float
 * dtype per call (f32, f16 or bf16), fp32 accumulation with one rounding per output, outputs written in full, `stream` a hipStream_t, functions return
 * once the work is enqueued. Tolerances against the reference's golden vectors: f32 1e-5,
 * f16 and bf16 1e-2 (atol = rtol).
 */
#ifndef HSN_OPS_H
#define HSN_OPS_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HSN_OPS_SPEC_VERSION 1

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

/*
 * v[r,k,:] = [u[r,:]; eps[r,:]; h[r, cell_idx[r,k], :]; m[r,k,:]]     (reference hsn_ops.h:79-87)
 * u, eps [B,d]; h [B,N,d]; m [B,K,d]; cell_idx [B,K]; v [B,K,4d].
 */
int hsn_gather_concat(const void* u, const void* eps, const void* h, const void* m,
                      const int32_t* cell_idx, void* v, int B, int N, int d, int K, int dtype,
                      void* stream);

/*
 * Backward of the gather (reference hsn_ops.h:88-99): grad_u, grad_eps [B,d] sum the slots'
 * first two blocks; grad_h [B,N,d] is the scatter-add of the third block over cell_idx (0 for
 * cells no slot names); grad_m [B,K,d] is the fourth block. `deterministic` is accepted for
 * the ABI's sake: every reduction here has a fixed order, so results are always reproducible.
 */
int hsn_gather_concat_bwd(const void* grad_v, const int32_t* cell_idx, void* grad_u,
                          void* grad_eps, void* grad_h, void* grad_m, int B, int N, int d, int K,
                          int dtype, int deterministic, void* stream);

/*
 * The grouped unit MLP (reference hsn_ops.h:101-112): unit j = unit_idx[p] in [0,M) on pair p,
 *   z1[p,:] = v[p,:] W1[j] + b1[j,:] (saved as hidden_saved [P,H], pre-GELU),
 *   out[p,:] = gelu(z1[p,:]) W2[j] + b2[j,:], gelu(x) = x/2 (1 + erf(x / sqrt 2)).
 * v [P,4d]; unit_idx [P]; W1 [M,4d,H] ([in, out]); b1 [M,H]; W2 [M,H,d]; b2 [M,d]; out [P,d];
 * d <= 256. The products run on the matrix cores (fp32 16x16x4 tiles, operands widened from
 * the storage dtype).
 */
int hsn_grouped_unit_mlp_fwd(const void* v, const int32_t* unit_idx, const void* W1,
                             const void* b1, const void* W2, const void* b2, void* hidden_saved,
                             void* out, int P, int M, int d, int H, int dtype, void* stream);

/*
 * Its backward (reference hsn_ops.h:114-130), from grad_out [P,d] and the saved z1:
 *   dz1 = (grad_out W2[j]^T) * gelu'(z1); grad_v = dz1 W1[j]^T;
 *   grad_W1[j] = sum_p v^T dz1, grad_b1[j] = sum_p dz1; grad_W2[j] = sum_p gelu(z1)^T grad_out,
 *   grad_b2[j] = sum_p grad_out; units without a pair get zeros.
 * The ABI has no workspace: grad_v's dz1 is kept in fp32 in grad_W2's memory when it has room
 * (P H floats), before grad_W2 is written, and is recomputed where it is consumed otherwise.
 * So grad_W2 must not overlap any input. Every sum has a fixed order, so `deterministic` holds
 * either way.
 */
int hsn_grouped_unit_mlp_bwd(const void* v, const int32_t* unit_idx, const void* W1,
                             const void* W2, const void* hidden_saved, const void* grad_out,
                             void* grad_v, void* grad_W1, void* grad_b1, void* grad_W2,
                             void* grad_b2, int P, int M, int d, int H, int dtype,
                             int deterministic, void* stream);

/*
 * The CSR neighbour messages (reference hsn_ops.h:132-143): i = cell_idx[r,k],
 *   m[r,k,:] = sum_{e in [indptr[i], indptr[i+1])} a[e] (V h[r, indices[e], :]),
 * V [d,d] as [d_out, d_in]. h [B,N,d]; indptr [N+1]; indices, a [E]; cell_idx [B,K] (repeats
 * allowed); m [B,K,d]; d <= 1024. Computed as V (sum_e a[e] h[r, indices[e]]) on the matrix
 * cores. Entries outside [0,N) / [0,E] contribute nothing (no out-of-bounds access); the CSR's
 * well-formedness is the caller's, as on the reference's GPU path (HSN_ERR_BAD_GRAPH is not
 * detected on the device).
 */
int hsn_csr_messages(const void* h, const int32_t* indptr, const int32_t* indices, const void* a,
                     const void* V, const int32_t* cell_idx, void* m, int B, int N, int d, int K,
                     int E, int dtype, void* stream);

/*
 * Its backward (reference hsn_ops.h:145-153), from grad_m [B,K,d]: over every slot (r,k) and
 * edge e of its row, source j = indices[e]:
 *   grad_h[r,j,:] = sum a[e] (V^T grad_m[r,k,:]); grad_V = sum a[e] grad_m[r,k,:] (outer)
 *   h[r,j,:]; grad_a[e] = sum grad_m[r,k,:] . (V h[r,j,:]).
 * Every sum has a fixed order (no atomics), so `deterministic` holds either way. grad_h must
 * not overlap any input: its memory holds intermediate fp32 sums before grad_h is written.
 */
int hsn_csr_messages_bwd(const void* h, const int32_t* indptr, const int32_t* indices,
                         const void* a, const void* V, const int32_t* cell_idx,
                         const void* grad_m, void* grad_h, void* grad_a, void* grad_V, int B,
                         int N, int d, int K, int E, int dtype, int deterministic, void* stream);

/*
 * The gated delta update, in place on h, q, age (reference hsn_ops.h:155-171): for every valid
 * slot, n = cell_idx[r,k]: h_old_saved = h[r,n,:]; h[r,n,:] = (1-b) h + b c; q[r,:] += sum of
 * the deltas / N; age[r,n] = 0. Padded slots (valid 0) are never read and get h_old_saved = 0.
 */
int hsn_gated_delta_update(void* h, void* q, int32_t* age, const int32_t* cell_idx,
                           const int32_t* valid, const void* c, const void* b, void* h_old_saved,
                           int B, int N, int d, int K, int dtype, void* stream);

/*
 * Its backward (reference hsn_ops.h:173-187), from G = grad_h_out [B,N,d], g = grad_q_out [B,d]:
 * for a valid slot grad_h[n] = (1-b) G[n] - b g/N, grad_c = b (G[n] + g/N),
 * grad_b = (c - h_old) (G[n] + g/N); grad_h = G on cells no valid slot names; grad_q = g;
 * zeros on padded slots.
 */
int hsn_gated_delta_update_bwd(const int32_t* cell_idx, const int32_t* valid, const void* c,
                               const void* b, const void* h_old_saved, const void* grad_h_out,
                               const void* grad_q_out, void* grad_h, void* grad_q, void* grad_c,
                               void* grad_b, int B, int N, int d, int K, int dtype, void* stream);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* HSN_OPS_H */
