// Entry points of the backward recurrence: the whole window with the activations fused and the
// carried state (hsn_win_backward), the reference's recurrence from c and b
// (hsn_win_recurrence) and the dense-fallback rows' recurrence (hsn_win_recurrence_dense).
#include <string>

#include "sweep.cuh"
#include "abi_util.h"
#include "chain_host.h"

using namespace hsn;

namespace {

// The dense-fallback rows (every cell written each position): the cotangent of one (row, cell,
// column) never meets another's, because R restarts from the position's own cotangents (reference
// python/hsn/train/split.py:177-209), so each thread walks its column chain alone.
__global__ __launch_bounds__(256) void dense_recurrence(const float* c, const float* bgate,
                                                        const float* h_old, const uint8_t* reset,
                                                        const float* dq_pre, const float* dq_post,
                                                        float* dc, float* db, int Bd, int T, int N,
                                                        int d) {
    const int64_t e = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    const int64_t per_row = int64_t(N) * d;
    if (e >= int64_t(Bd) * per_row) return;
    const int64_t r = e / per_row, nd = e - r * per_row;
    const int x = static_cast<int>(nd % d);
    const float n_f = static_cast<float>(N);
    float A = 0.0f, Rc = 0.0f;  // Rc: the summary cotangent carried from position t+1
    for (int t = T - 1; t >= 0; --t) {
        float R = Rc;
        if (dq_post) R += dq_post[(r * T + t) * d + x];
        const int64_t o = (r * T + t) * per_row + nd;
        const float gg = A + R / n_f;
        const float b = bgate[o];
        dc[o] = b * gg;
        db[o] = (c[o] - h_old[o]) * gg;
        A = (1.0f - b) * gg;
        Rc = dq_pre ? dq_pre[(r * T + t) * d + x] : 0.0f;
        if (reset[r * T + t]) {
            A = 0.0f;
            Rc = 0.0f;
        }
    }
}

void fill_common(BwdArgs& a, const void* y, const void* g, const void* h_old, const void* d_h_sel,
                 const void* d_q_pre, const void* d_q_post, const uint8_t* reset,
                 const float* d_h_T, const float* d_q_T, void* dy, void* dg, float* d_h0,
                 float* d_q0, int B, int T, int N, int d, int K, const Geometry& geo) {
    a.y = y, a.g = g, a.h_old = h_old, a.y_row = int64_t(T) * K * d;
    a.dsel = d_h_sel, a.dq_pre = d_q_pre, a.dq_post = d_q_post;  // absent: read as zero
    a.q_row = int64_t(T) * d;
    a.reset = reset, a.r_row = T, a.s_row = int64_t(T) * K;
    a.dh_T = d_h_T, a.dq_T = d_q_T, a.dy = dy, a.dg = dg, a.dh0 = d_h0, a.dq0 = d_q0;
    a.B = B, a.T = T, a.N = N, a.d = d, a.K = K;
    a.W = geo.W, a.Tc = geo.Tc, a.region = bwd_region(N, geo.S, geo.W), a.divn = make_divn(N);
}

}  // namespace

extern "C" int hsn_win_backward(const void* y, const void* gate_pre, const void* h_old,
                                int io_dtype, const float* cand_w, int cand_norm, float cand_eps,
                                void* workspace, int64_t workspace_bytes, const int32_t* slots,
                                const uint8_t* reset, const void* d_q_pre, const void* d_q_post,
                                const void* d_h_sel, const float* d_h_T, const float* d_q_T,
                                void* dy, void* dgate, float* d_h0, float* d_q0, float* d_cand_w,
                                int B, int T, int N, int d, int K, void* stream) {
    HSN_ABI_BEGIN
    HSN_REQUIRE(y && gate_pre && h_old && slots && reset && dy && dgate, HSN_ERR_INVALID_ARGUMENT,
                "hsn_win_backward: a required pointer is NULL");
    HSN_REQUIRE(B >= 1 && T >= 1 && N >= 1 && d >= 1 && K >= 1 && K <= N,
                HSN_ERR_INVALID_ARGUMENT, "hsn_win_backward: bad dimensions");
    HSN_REQUIRE(!cand_norm || cand_w, HSN_ERR_INVALID_ARGUMENT,
                "hsn_win_backward: the RMS candidate needs cand_w");
    HSN_REQUIRE(io_dtype == HSN_DTYPE_F32 || io_dtype == HSN_DTYPE_BF16,
                HSN_ERR_UNSUPPORTED_DTYPE, "hsn_win_backward: io_dtype must be f32 or bf16");
    HSN_REQUIRE(check_elems({int64_t(B) * T * K * d, int64_t(B) * N * d}) &&
                    int64_t(T) * K * d * 4 < (int64_t(1) << 31),
                HSN_ERR_SIZE_OVERFLOW,
                "hsn_win_backward: a tensor is too large");
    const size_t elem = io_dtype == HSN_DTYPE_F32 ? 4 : 2;
    const WorkspaceLayout L = workspace_layout(HSN_OP_BACKWARD, B, T, N, d, K, elem, cand_norm);
    HSN_REQUIRE(L.bytes == 0 || (workspace && workspace_bytes >= int64_t(L.bytes)),
                HSN_ERR_INVALID_ARGUMENT,
                "hsn_win_backward: the workspace must hold " + std::to_string(L.bytes) +
                    " bytes (hsn_win_workspace_bytes)");
    hipStream_t st = as_stream(stream);
    char* ws = static_cast<char*>(workspace);
    const int64_t nslots = int64_t(B) * T * K;
    const void* pre = y;
    float* inv = nullptr;
    if (cand_norm) {  // the normalised candidate input (the forward's, recomputed)
        void* rms_scratch = ws + L.rms;
        inv = reinterpret_cast<float*>(static_cast<char*>(rms_scratch) + rms_inv_offset(nslots, d, elem));
        const int blocks = static_cast<int>((nslots + 3) / 4);
        if (io_dtype == HSN_DTYPE_F32)
            hipLaunchKernelGGL((rms_prologue<float>), dim3(blocks), dim3(256), 0, st,
                               static_cast<const float*>(y), cand_w,
                               static_cast<float*>(rms_scratch), inv, nslots, d, cand_eps);
        else
            hipLaunchKernelGGL((rms_prologue<bf16_t>), dim3(blocks), dim3(256), 0, st,
                               static_cast<const bf16_t*>(y), cand_w,
                               static_cast<bf16_t*>(rms_scratch), inv, nslots, d, cand_eps);
        HSN_HIP(hipGetLastError());
        pre = rms_scratch;
    }
    if (L.evmap) {
        evmap_backward(pre, gate_pre, h_old, slots, reset, d_q_pre, d_q_post, d_h_sel, d_h_T,
                       d_q_T, dy, dgate, d_h0, d_q0, B, T, N, d, K, st);
    } else if (L.chain) {
        chain_backward(pre, gate_pre, h_old, io_dtype, slots, reset, d_q_pre, d_q_post, d_h_sel,
                       d_h_T, d_q_T, dy, dgate, d_h0, d_q0, B, T, N, d, K, ws, L, st);
    } else {
        Geometry g;
        HSN_REQUIRE(choose_geometry(B, T, N, d, K, bwd_lds_bytes, g), HSN_ERR_INVALID_ARGUMENT,
                    "hsn_win_backward: the cotangent slice does not fit the LDS (N too large)");
        const size_t lds = bwd_lds_bytes(N, g.S, g.W);
        BwdArgs a{};
        fill_common(a, pre, gate_pre, h_old, d_h_sel, d_q_pre, d_q_post, reset, d_h_T, d_q_T, dy,
                    dgate, d_h0, d_q0, B, T, N, d, K, g);
        a.cells = slots, a.valid = nullptr;
        if (io_dtype == HSN_DTYPE_F32)
            HSN_HIP((launch_bwd<float, Packed32, true>(a, g.S, lds, st)));
        else
            HSN_HIP((launch_bwd<bf16_t, Packed32, true>(a, g.S, lds, st)));
    }
    if (cand_norm) {  // the norm's VJP: dy holds dL/dpre
        const int blocks = static_cast<int>((nslots + 3) / 4);
        if (io_dtype == HSN_DTYPE_F32) {
            if (d_cand_w)
                hipLaunchKernelGGL((rms_weight_grad<float>), dim3(d), dim3(256), 0, st,
                                   static_cast<const float*>(y), static_cast<const float*>(dy), inv,
                                   d_cand_w, nslots, d);
            hipLaunchKernelGGL((rms_input_grad<float>), dim3(blocks), dim3(256), 0, st,
                               static_cast<const float*>(y), static_cast<float*>(dy), inv, cand_w,
                               nslots, d);
        } else {
            if (d_cand_w)
                hipLaunchKernelGGL((rms_weight_grad<bf16_t>), dim3(d), dim3(256), 0, st,
                                   static_cast<const bf16_t*>(y), static_cast<const bf16_t*>(dy),
                                   inv, d_cand_w, nslots, d);
            hipLaunchKernelGGL((rms_input_grad<bf16_t>), dim3(blocks), dim3(256), 0, st,
                               static_cast<const bf16_t*>(y), static_cast<bf16_t*>(dy), inv,
                               cand_w, nslots, d);
        }
        HSN_HIP(hipGetLastError());
    }
    HSN_ABI_END
}

extern "C" int hsn_win_recurrence(const float* c, const float* b, const float* h_old,
                                  const int64_t* cells, const uint8_t* valid,
                                  const uint8_t* reset, const float* d_q_pre,
                                  const float* d_q_post, const float* d_h_sel, const float* d_h_T,
                                  const float* d_q_T, float* dc, float* db, float* d_h0,
                                  float* d_q0, int B, int T, int K, int d, int N, void* stream) {
    HSN_ABI_BEGIN
    HSN_REQUIRE(c && b && h_old && cells && valid && reset && dc && db, HSN_ERR_INVALID_ARGUMENT,
                "hsn_win_recurrence: a required pointer is NULL");
    HSN_REQUIRE(B >= 1 && T >= 1 && N >= 1 && d >= 1 && K >= 1, HSN_ERR_INVALID_ARGUMENT,
                "hsn_win_recurrence: bad dimensions");
    HSN_REQUIRE(check_elems({int64_t(B) * T * K * d, int64_t(B) * N * d}) &&
                    int64_t(T) * K * d * 4 < (int64_t(1) << 31),
                HSN_ERR_SIZE_OVERFLOW,
                "hsn_win_recurrence: a tensor is too large");
    Geometry g;
    HSN_REQUIRE(choose_geometry(B, T, N, d, K, bwd_lds_bytes, g), HSN_ERR_INVALID_ARGUMENT,
                "hsn_win_recurrence: the cotangent slice does not fit the LDS (N too large)");
    const size_t lds = bwd_lds_bytes(N, g.S, g.W);
    BwdArgs a{};
    fill_common(a, c, b, h_old, d_h_sel, d_q_pre, d_q_post, reset, d_h_T, d_q_T, dc, db, d_h0,
                d_q0, B, T, N, d, K, g);
    a.cells = cells, a.valid = valid;
    HSN_HIP((launch_bwd<float, Cells64, false>(a, g.S, lds, as_stream(stream))));
    HSN_ABI_END
}

extern "C" int hsn_win_recurrence_dense(const float* c, const float* b, const float* h_old,
                                        const uint8_t* reset, const float* d_q_pre,
                                        const float* d_q_post, float* dc, float* db, int Bd,
                                        int T, int N, int d, void* stream) {
    HSN_ABI_BEGIN
    HSN_REQUIRE(c && b && h_old && reset && dc && db, HSN_ERR_INVALID_ARGUMENT,
                "hsn_win_recurrence_dense: a required pointer is NULL");
    HSN_REQUIRE(Bd >= 1 && T >= 1 && N >= 1 && d >= 1, HSN_ERR_INVALID_ARGUMENT,
                "hsn_win_recurrence_dense: bad dimensions");
    HSN_REQUIRE(check_elems({int64_t(Bd) * T * N * d}), HSN_ERR_SIZE_OVERFLOW,
                "hsn_win_recurrence_dense: a tensor is too large");
    const int64_t chains = int64_t(Bd) * N * d;
    const int blocks = static_cast<int>((chains + 255) / 256);
    hipLaunchKernelGGL(dense_recurrence, dim3(blocks), dim3(256), 0, as_stream(stream), c, b, h_old,
                       reset, d_q_pre, d_q_post, dc, db, Bd, T, N, d);
    HSN_HIP(hipGetLastError());
    HSN_ABI_END
}
