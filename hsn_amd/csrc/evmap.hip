// The event-map path of hsn_win_forward and hsn_win_backward (evmap.cuh): argument blocks and
// launches.
#include "abi_util.h"
#include "chain_host.h"
#include "evmap.cuh"

namespace hsn {

void evmap_forward(const void* y, const void* gate_pre, const uint8_t* reset,
                   const int32_t* slots, const float* h0, const float* q0, const int64_t* age0,
                   const int64_t* pos0, void* q_pre, void* q_post, void* h_sel, void* h_old,
                   float* h_max, float* h_T, float* q_T, int64_t* age_T, int64_t* pos_T, int B,
                   int T, int N, int d, int K, hipStream_t st) {
    evmap::FwdEv a{};
    a.y = static_cast<const float*>(y), a.g = static_cast<const float*>(gate_pre);
    a.slots = slots, a.reset = reset, a.h0 = h0, a.q0 = q0, a.age0 = age0, a.pos0 = pos0;
    a.q_pre = static_cast<float*>(q_pre), a.q_post = static_cast<float*>(q_post);
    a.h_sel = static_cast<float*>(h_sel), a.h_old = static_cast<float*>(h_old);
    a.h_max = h_max, a.h_T = h_T, a.q_T = q_T, a.age_T = age_T, a.pos_T = pos_T;
    a.T = T, a.N = N, a.d = d, a.K = K, a.P = (T + evmap::kChunks - 1) / evmap::kChunks;
    a.divn = make_divn(N);
    const size_t lds = evmap::fwd_layout(N).bytes;
    auto k = evmap::fwd<float>;
    HSN_HIP(allow_lds(k, lds));
    hipLaunchKernelGGL(k, sweep_grid(B, d / evmap::kS), dim3(kWave * evmap::kWaves), lds, st, a);
    HSN_HIP(hipGetLastError());
}

void evmap_backward(const void* y, const void* gate_pre, const void* h_old, const int32_t* slots,
                    const uint8_t* reset, const void* d_q_pre, const void* d_q_post,
                    const void* d_h_sel, const float* d_h_T, const float* d_q_T, void* dy,
                    void* dgate, float* d_h0, float* d_q0, int B, int T, int N, int d, int K,
                    hipStream_t st) {
    evmap::BwdEv a{};
    a.y = static_cast<const float*>(y), a.g = static_cast<const float*>(gate_pre);
    a.h_old = static_cast<const float*>(h_old), a.dsel = static_cast<const float*>(d_h_sel);
    a.slots = slots, a.reset = reset;
    a.dq_pre = static_cast<const float*>(d_q_pre), a.dq_post = static_cast<const float*>(d_q_post);
    a.dh_T = d_h_T, a.dq_T = d_q_T;
    a.dy = static_cast<float*>(dy), a.dg = static_cast<float*>(dgate);
    a.dh0 = d_h0, a.dq0 = d_q0;
    a.T = T, a.N = N, a.d = d, a.K = K, a.P = (T + evmap::kChunks - 1) / evmap::kChunks;
    a.divn = make_divn(N);
    const size_t lds = evmap::bwd_layout(N).bytes;
    auto k = evmap::bwd<float>;
    HSN_HIP(allow_lds(k, lds));
    hipLaunchKernelGGL(k, sweep_grid(B, d / evmap::kS), dim3(kWave * evmap::kWaves), lds, st, a);
    HSN_HIP(hipGetLastError());
}

}  // namespace hsn
