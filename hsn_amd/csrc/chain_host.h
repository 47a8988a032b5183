// The choice between the three sweep designs of the window (the time-chunked slices of
// sweep.cuh, the cell chains of chain.cuh and the event-map slices of evmap.cuh), the workspace
// each entry point needs, and the chain and event-map paths' launchers.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace hsn {

enum PathCode : int { kPathAuto = 0, kPathSlice = 1, kPathChain = 2, kPathEvmap = 3 };

// The workspace of hsn_win_forward / hsn_win_backward, byte offsets into it (256-aligned):
// the RMS candidate's normalised input (both paths), and on the chain path the row lists, the
// per-position sums (the forward's D, the backward's share), the forward's fp32 per-slot deltas
// (used with bf16 rows, or where the caller omits h_old or h_sel) and its per-group row maxima.
struct WorkspaceLayout {
    bool chain = false, evmap = false;
    size_t ptr = 0, ev = 0, sum = 0, delta = 0, hmax = 0, rms = 0, bytes = 0;
};

int path_setting();
void set_path_setting(int path);
// Whether a path takes a shape (op: HSN_OP_FORWARD or HSN_OP_BACKWARD for the chains; every op
// for the slices), with the reason when it does not.
bool slice_takes(int op, int B, int T, int N, int d, int K, const char** why);
bool chain_takes(int B, int T, int N, int d, int K, const char** why);
bool evmap_takes(int op, int B, int T, int N, int d, int K, size_t elem, const char** why);
// The path hsn_win_forward / hsn_win_backward take (kPathSlice or kPathChain), or throws the
// reason neither does.
int choose_path(int op, int B, int T, int N, int d, int K, size_t elem);
WorkspaceLayout workspace_layout(int op, int B, int T, int N, int d, int K, size_t elem,
                                 int cand_norm);

void chain_forward(const void* y, const void* gate_pre, int io_dtype, const uint8_t* reset,
                   const int32_t* slots, const float* h0, const float* q0, const int64_t* age0,
                   const int64_t* pos0, void* q_pre, void* q_post, void* h_sel, void* h_old,
                   float* h_max, float* h_T, float* q_T, int64_t* age_T, int64_t* pos_T, int B,
                   int T, int N, int d, int K, char* ws, const WorkspaceLayout& L,
                   hipStream_t st);

void chain_backward(const void* y, const void* gate_pre, const void* h_old, int io_dtype,
                    const int32_t* slots, const uint8_t* reset, const void* d_q_pre,
                    const void* d_q_post, const void* d_h_sel, const float* d_h_T,
                    const float* d_q_T, void* dy, void* dgate, float* d_h0, float* d_q0, int B,
                    int T, int N, int d, int K, char* ws, const WorkspaceLayout& L,
                    hipStream_t st);

void evmap_forward(const void* y, const void* gate_pre, const uint8_t* reset,
                   const int32_t* slots, const float* h0, const float* q0, const int64_t* age0,
                   const int64_t* pos0, void* q_pre, void* q_post, void* h_sel, void* h_old,
                   float* h_max, float* h_T, float* q_T, int64_t* age_T, int64_t* pos_T, int B,
                   int T, int N, int d, int K, hipStream_t st);
// The router's settings where the forward routes its own window (hsn_win_route_forward: one
// unit, no probes, fp32 logits [B,T,N,width], int32 decisions).
struct WindowRouteSpec {
    const float* logits;
    int64_t width;
    const float* cost;
    int32_t* cells;
    int32_t* units;
    uint8_t* valid;
    float* theta;
    uint8_t* refreshed;
    int32_t* slots;
    int reserved;
    float lambda, overhead, shared, limit;
};
// Whether the routed forward takes the shape (the event maps' conditions, N <= 512, at most 256
// workgroups, at most 32 positions to decide a workgroup), with the reason when it does not.
bool evmap_routes(int B, int T, int N, int d, int K, const char** why);
// Whether this call may use the routed forward's device buffers: the device's first stream that
// takes them keeps them (`take`: this call takes them if free), a capturing stream never does,
// and the grid must fit the device's compute units at once; the reason when not.
bool evmap_route_claim(hipStream_t st, int B, int d, bool take, const char** why);
void evmap_route_forward(const WindowRouteSpec& rs, const void* y, const void* gate_pre,
                         const uint8_t* reset, const float* h0, const float* q0,
                         const int64_t* age0, const int64_t* pos0, void* q_pre, void* q_post,
                         void* h_sel, void* h_old, float* h_max, float* h_T, float* q_T,
                         int64_t* age_T, int64_t* pos_T, int B, int T, int N, int d, int K,
                         hipStream_t st);
// The routed forward's exchange waits that hit their limit since the last clear (the device is
// synchronised first).
unsigned evmap_exchange_timeouts(bool clear);

void evmap_backward(const void* y, const void* gate_pre, const void* h_old, const int32_t* slots,
                    const uint8_t* reset, const void* d_q_pre, const void* d_q_post,
                    const void* d_h_sel, const float* d_h_T, const float* d_q_T, void* dy,
                    void* dgate, float* d_h0, float* d_q0, int B, int T, int N, int d, int K,
                    hipStream_t st);

}  // namespace hsn
