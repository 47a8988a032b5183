// The event-map path of hsn_win_forward (evmap.cuh): argument block and launch.
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

}  // namespace hsn
