// The column-strip path of hsn_win_forward / hsn_win_backward (strip.cuh): the shapes it takes
// and its launchers.
#include "abi_util.h"
#include "chain_host.h"
#include "strip.cuh"

namespace hsn {

namespace {


template <typename IO>
void launch_strip_fwd(const strip::FwdArgs& a, hipStream_t st) {
    constexpr int S = strip::kCols;
    const size_t lds = size_t(strip::layout(a.T, a.N, a.K, true).words) * 4;
    auto k = a.h_max ? strip::strip_fwd<IO, true> : strip::strip_fwd<IO, false>;
    HSN_HIP(allow_lds(k, lds));
    hipLaunchKernelGGL(k, strip::strip_grid(a.B, (a.d + S - 1) / S), dim3(strip::kThreads), lds, st, a);
    HSN_HIP(hipGetLastError());
}

template <typename IO>
void launch_strip_bwd(const strip::BwdArgs& a, hipStream_t st) {
    constexpr int S = strip::kCols;
    const size_t lds = size_t(strip::layout(a.T, a.N, a.K, false).words) * 4;
    auto k = strip::strip_bwd<IO>;
    HSN_HIP(allow_lds(k, lds));
    hipLaunchKernelGGL(k, strip::strip_grid(a.B, (a.d + S - 1) / S), dim3(strip::kThreads), lds, st, a);
    HSN_HIP(hipGetLastError());
}

}  // namespace

bool strip_takes(int op, int B, int T, int N, int d, int K, const char** why) {
    (void)B;
    const char* r = nullptr;
    if (d % strip::kVec != 0) r = "the column strips take d a multiple of 4";
    else if (K > chain::kMaxK) r = "the column strips take K <= 255";
    else if (int64_t(T) * K > int64_t(strip::kThreads) * strip::kMaxU ||
             int64_t(T) * K > strip::kSlotMask + 1)
        r = "the column strips take T * K <= 8192 (the row's decisions in one workgroup)";
    else if (int64_t(strip::layout(T, N, K, op == HSN_OP_FORWARD).words) * 4 > kLdsMax)
        r = "the row's lists and per-slot sums do not fit the LDS";
    if (r && why) *why = r;
    return r == nullptr;
}

void strip_forward(const void* y, const void* gate_pre, int io_dtype, const uint8_t* reset,
                   const int32_t* slots, const float* h0, const float* q0, const int64_t* age0,
                   const int64_t* pos0, void* q_pre, void* q_post, void* h_sel, void* h_old,
                   float* h_max, float* h_T, float* q_T, int64_t* age_T, int64_t* pos_T, int B,
                   int T, int N, int d, int K, hipStream_t st) {
    strip::FwdArgs a{};
    a.y = y, a.g = gate_pre, a.slots = slots, a.reset = reset;
    a.h0 = h0, a.q0 = q0, a.age0 = age0, a.pos0 = pos0;
    a.q_pre = q_pre, a.q_post = q_post, a.h_old = h_old, a.h_sel = h_sel, a.h_max = h_max;
    a.h_T = h_T, a.q_T = q_T, a.age_T = age_T, a.pos_T = pos_T;
    a.B = B, a.T = T, a.N = N, a.d = d, a.K = K, a.divn = make_divn(N);
    if (io_dtype == HSN_DTYPE_F32) launch_strip_fwd<float>(a, st);
    else launch_strip_fwd<bf16_t>(a, st);
}

void strip_backward(const void* y, const void* gate_pre, const void* h_old, int io_dtype,
                    const int32_t* slots, const uint8_t* reset, const void* d_q_pre,
                    const void* d_q_post, const void* d_h_sel, const float* d_h_T,
                    const float* d_q_T, void* dy, void* dgate, float* d_h0, float* d_q0, int B,
                    int T, int N, int d, int K, hipStream_t st) {
    strip::BwdArgs a{};
    a.y = y, a.g = gate_pre, a.h_old = h_old, a.dsel = d_h_sel, a.slots = slots, a.reset = reset;
    a.dq_pre = d_q_pre, a.dq_post = d_q_post, a.dq_T = d_q_T, a.dh_T = d_h_T;
    a.dy = dy, a.dg = dgate, a.dh0 = d_h0, a.dq0 = d_q0;
    a.B = B, a.T = T, a.N = N, a.d = d, a.K = K, a.divn = make_divn(N);
    if (io_dtype == HSN_DTYPE_F32) launch_strip_bwd<float>(a, st);
    else launch_strip_bwd<bf16_t>(a, st);
}

}  // namespace hsn
