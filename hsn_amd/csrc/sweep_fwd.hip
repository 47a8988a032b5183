// Entry points of the forward sweep: the whole window (hsn_win_forward) and the reference's
// per-position end of round (hsn_win_cell_update), over the kernels of sweep.cuh.
#include <atomic>
#include <mutex>
#include <string>

#include "sweep.cuh"
#include "abi_util.h"
#include "chain_host.h"

using namespace hsn;

namespace {

// The RMS candidate's prologue: writes the normalised candidate input into the workspace
// (layout: rms_inv_offset) and returns it.
const void* rms_normalise(const void* y, int io_dtype, const float* cand_w, float cand_eps,
                          void* ws, int64_t slots, int d, hipStream_t st) {
    const int blocks = static_cast<int>((slots + 3) / 4);
    const size_t elem = io_dtype == HSN_DTYPE_F32 ? 4 : 2;
    float* inv = reinterpret_cast<float*>(static_cast<char*>(ws) + rms_inv_offset(slots, d, elem));
    if (io_dtype == HSN_DTYPE_F32)
        hipLaunchKernelGGL((rms_prologue<float>), dim3(blocks), dim3(256), 0, st,
                           static_cast<const float*>(y), cand_w, static_cast<float*>(ws), inv,
                           slots, d, cand_eps);
    else
        hipLaunchKernelGGL((rms_prologue<bf16_t>), dim3(blocks), dim3(256), 0, st,
                           static_cast<const bf16_t*>(y), cand_w, static_cast<bf16_t*>(ws),
                           inv, slots, d, cand_eps);
    return ws;
}

// The checks every forward entry point makes before it touches the RMS workspace.
void forward_checks(const char* fn, const void* y, const void* gate_pre, int io_dtype,
                    const float* cand_w, int cand_norm, const uint8_t* reset,
                    const int32_t* slots, const float* h0, const float* q0, const int64_t* age0,
                    const int64_t* pos0, int64_t* age_T, int64_t* pos_T, int B, int T, int N,
                    int d, int K) {
    const std::string f(fn);
    HSN_REQUIRE(y && gate_pre && reset && slots && h0 && q0, HSN_ERR_INVALID_ARGUMENT,
                f + ": a required pointer is NULL");
    HSN_REQUIRE(B >= 1 && T >= 1 && N >= 1 && d >= 1 && K >= 1 && K <= N,
                HSN_ERR_INVALID_ARGUMENT, f + ": bad dimensions");
    HSN_REQUIRE(!age_T || age0, HSN_ERR_INVALID_ARGUMENT, f + ": age_T needs age0");
    HSN_REQUIRE(!pos_T || (pos0 && age_T), HSN_ERR_INVALID_ARGUMENT,
                f + ": pos_T needs pos0 and age_T");
    HSN_REQUIRE(!cand_norm || cand_w, HSN_ERR_INVALID_ARGUMENT,
                f + ": the RMS candidate needs cand_w");
    HSN_REQUIRE(io_dtype == HSN_DTYPE_F32 || io_dtype == HSN_DTYPE_BF16,
                HSN_ERR_UNSUPPORTED_DTYPE, f + ": io_dtype must be f32 or bf16");
    HSN_REQUIRE(check_elems({int64_t(B) * T * K * d, int64_t(B) * N * d}) &&
                    int64_t(T) * K * d * 4 < (int64_t(1) << 31),
                HSN_ERR_SIZE_OVERFLOW, f + ": a tensor is too large");
}

// The forward after the checks, on the path the layout names; `ws` is the workspace.
void forward_launch(const void* y, const void* gate_pre, int io_dtype, const float* cand_w,
                    int cand_norm, float cand_eps, char* ws, const WorkspaceLayout& L,
                    const uint8_t* reset, const int32_t* slots, const float* h0, const float* q0,
                    const int64_t* age0, const int64_t* pos0, void* q_pre, void* q_post,
                    void* h_sel, void* h_old, float* h_max, float* h_T, float* q_T,
                    int64_t* age_T, int64_t* pos_T, int B, int T, int N, int d, int K,
                    void* stream) {
    hipStream_t st = as_stream(stream);
    if (cand_norm) {
        y = rms_normalise(y, io_dtype, cand_w, cand_eps, ws + L.rms, int64_t(B) * T * K, d, st);
        HSN_HIP(hipGetLastError());
    }
    if (L.evmap) {
        evmap_forward(y, gate_pre, reset, slots, h0, q0, age0, pos0, q_pre, q_post, h_sel,
                      h_old, h_max, h_T, q_T, age_T, pos_T, B, T, N, d, K, st);
        return;
    }
    if (L.chain) {
        chain_forward(y, gate_pre, io_dtype, reset, slots, h0, q0, age0, pos0, q_pre, q_post,
                      h_sel, h_old, h_max, h_T, q_T, age_T, pos_T, B, T, N, d, K, ws, L, st);
        return;
    }
    Geometry g;
    HSN_REQUIRE(choose_geometry(B, T, N, d, K, fwd_lds_bytes, g), HSN_ERR_INVALID_ARGUMENT,
                "hsn_win_forward: the state slice does not fit the LDS (N too large)");
    const size_t lds = fwd_lds_bytes(N, g.S, g.W);
    FwdArgs a{};
    a.y = y, a.g = gate_pre, a.y_row = int64_t(T) * K * d;
    a.reset = reset, a.r_row = T, a.clear = nullptr, a.c_row = 0;
    a.cells = slots, a.valid = nullptr, a.s_row = int64_t(T) * K;
    a.h0 = h0, a.h0_row = int64_t(N) * d, a.q0 = q0, a.q0_row = d;
    a.age0 = age0, a.a0_row = N, a.pos0 = pos0;
    a.q_pre = q_pre, a.q_post = q_post, a.qo_row = int64_t(T) * d;
    a.h_sel = h_sel, a.h_old = h_old, a.o_row = int64_t(T) * K * d;
    a.h_max = h_max, a.hm_row = T;
    a.h_T = h_T, a.hT_row = int64_t(N) * d, a.q_T = q_T, a.qT_row = d;
    a.age_T = age_T, a.aT_row = N, a.pos_T = pos_T;
    a.B = B, a.T = T, a.N = N, a.d = d, a.K = K;
    a.W = g.W, a.Tc = g.Tc, a.region = fwd_region(N, g.S, g.W), a.divn = make_divn(N);
    if (io_dtype == HSN_DTYPE_F32)
        HSN_HIP((launch_fwd<float, float, Packed32>(a, g.S, lds, st)));
    else
        HSN_HIP((launch_fwd<bf16_t, bf16_t, Packed32>(a, g.S, lds, st)));
}

}  // namespace

extern "C" int hsn_win_forward(const void* y, const void* gate_pre, int io_dtype,
                               const float* cand_w, int cand_norm, float cand_eps,
                               void* workspace, int64_t workspace_bytes, const uint8_t* reset,
                               const int32_t* slots, const float* h0, const float* q0,
                               const int64_t* age0, const int64_t* pos0, void* q_pre,
                               void* q_post, void* h_sel, void* h_old, float* h_max, float* h_T,
                               float* q_T, int64_t* age_T, int64_t* pos_T, int B, int T, int N,
                               int d, int K, void* stream) {
    HSN_ABI_BEGIN
    forward_checks("hsn_win_forward", y, gate_pre, io_dtype, cand_w, cand_norm, reset, slots, h0,
                   q0, age0, pos0, age_T, pos_T, B, T, N, d, K);
    const WorkspaceLayout L = workspace_layout(HSN_OP_FORWARD, B, T, N, d, K,
                                               io_dtype == HSN_DTYPE_F32 ? 4 : 2, cand_norm);
    HSN_REQUIRE(L.bytes == 0 || (workspace && workspace_bytes >= int64_t(L.bytes)),
                HSN_ERR_INVALID_ARGUMENT,
                "hsn_win_forward: the workspace must hold " + std::to_string(L.bytes) +
                    " bytes (hsn_win_workspace_bytes)");
    forward_launch(y, gate_pre, io_dtype, cand_w, cand_norm, cand_eps,
                   static_cast<char*>(workspace), L, reset, slots, h0, q0, age0, pos0, q_pre,
                   q_post, h_sel, h_old, h_max, h_T, q_T, age_T, pos_T, B, T, N, d, K, stream);
    HSN_ABI_END
}

namespace {

// The workspace of hsn_win_forward_noalloc, owned by the library: every device the library runs
// on holds its own copy for the life of the process. Host code never uses the symbol itself
// (its host-side name is a stand-in, not a device address): each device's address comes from
// hipGetSymbolAddress, taken once per device with that device current.
constexpr size_t kNoAllocScratchBytes = size_t(32) << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_lock;
void* g_scratch_ptr[kMaxDevices] = {};

void* device_scratch() {
    int dev = 0;
    HSN_HIP(hipGetDevice(&dev));
    HSN_REQUIRE(dev >= 0 && dev < kMaxDevices, HSN_ERR_BACKEND,
                "hsn_win_forward_noalloc: device index above 63");
    std::lock_guard<std::mutex> guard(g_scratch_lock);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        HSN_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        HSN_REQUIRE(p != nullptr, HSN_ERR_BACKEND,
                    "hsn_win_forward_noalloc: no device address for the scratch array");
        g_scratch_ptr[dev] = p;
    }
    return g_scratch_ptr[dev];
}

}  // namespace

extern "C" int hsn_win_forward_noalloc(const void* y, const void* gate_pre, int io_dtype,
                                       const float* cand_w, int cand_norm, float cand_eps,
                                       const uint8_t* reset, const int32_t* slots,
                                       const float* h0, const float* q0, const int64_t* age0,
                                       const int64_t* pos0, void* q_pre, void* q_post,
                                       void* h_sel, void* h_old, float* h_max, float* h_T,
                                       float* q_T, int64_t* age_T, int64_t* pos_T, int B, int T,
                                       int N, int d, int K, void* stream) {
    HSN_ABI_BEGIN
    forward_checks("hsn_win_forward_noalloc", y, gate_pre, io_dtype, cand_w, cand_norm, reset,
                   slots, h0, q0, age0, pos0, age_T, pos_T, B, T, N, d, K);
    // the workspace hsn_win_forward would take: the library's array, within its size
    const WorkspaceLayout L = workspace_layout(HSN_OP_FORWARD, B, T, N, d, K,
                                               io_dtype == HSN_DTYPE_F32 ? 4 : 2, cand_norm);
    HSN_REQUIRE(L.bytes <= kNoAllocScratchBytes, HSN_ERR_SIZE_OVERFLOW,
                "hsn_win_forward_noalloc: the workspace of this shape needs " +
                    std::to_string(L.bytes) + " bytes, above the library's " +
                    std::to_string(kNoAllocScratchBytes) + "-byte scratch array");
    char* ws = L.bytes ? static_cast<char*>(device_scratch()) : nullptr;
    forward_launch(y, gate_pre, io_dtype, cand_w, cand_norm, cand_eps, ws, L, reset, slots, h0,
                   q0, age0, pos0, q_pre, q_post, h_sel, h_old, h_max, h_T, q_T, age_T, pos_T, B,
                   T, N, d, K, stream);
    HSN_ABI_END
}

namespace {

// hsn_win_route_forward's choice (hsn_win_set_route_forward): HSN_ROUTE_FORWARD_AUTO takes the
// two launches (the one launch measured slower at the ref shape: 42.8 against 9.3 + 30.3 us,
// its wavefronts deciding four positions each at two wavefronts a SIMD), ONE the one launch
// wherever it takes the call, TWO always the two.
std::atomic<int> g_route_forward_mode{HSN_ROUTE_FORWARD_AUTO};

// hsn_win_route's checks of the router's arguments (without probes).
void route_checks(const char* fn, const void* logits, int logits_dtype, int64_t width,
                  const float* cost, void* cells, void* units, int index_bits, uint8_t* valid,
                  float* theta, uint8_t* refreshed, int M, int reserved, int reserved_units,
                  int B, int T, int N, int K) {
    const std::string f(fn);
    HSN_REQUIRE(logits && cost && cells && units && valid && theta && refreshed,
                HSN_ERR_INVALID_ARGUMENT, f + ": a required router pointer is NULL");
    HSN_REQUIRE(M >= 1 && K <= kWave && N <= 64 * kWave, HSN_ERR_INVALID_ARGUMENT,
                f + ": need M >= 1, K <= 64 and N <= 4096");
    HSN_REQUIRE(width >= M, HSN_ERR_INVALID_ARGUMENT, f + ": width < M");
    HSN_REQUIRE(reserved >= 0 && (reserved == 0 || reserved < K), HSN_ERR_INVALID_ARGUMENT,
                f + ": reserved must be 0 or lie in [1, K)");
    HSN_REQUIRE(!reserved_units || reserved > 0, HSN_ERR_INVALID_ARGUMENT,
                f + ": reserved_units needs reserved > 0");
    HSN_REQUIRE(index_bits == 32 || index_bits == 64, HSN_ERR_INVALID_ARGUMENT,
                f + ": index_bits must be 32 or 64");
    HSN_REQUIRE(logits_dtype == HSN_DTYPE_F32 || logits_dtype == HSN_DTYPE_BF16,
                HSN_ERR_UNSUPPORTED_DTYPE, f + ": logits must be f32 or bf16");
    HSN_REQUIRE(check_elems({int64_t(B) * T * N * width}), HSN_ERR_SIZE_OVERFLOW,
                f + ": the logits are too large");
}

// Whether a call with these settings runs as one launch: the event maps' forward that routes
// its own window takes the shape, the router has one unit and fp32 logits, the decisions are
// int32, the rows fp32 (`claim`: and the call's stream may use the device's exchange buffers,
// which it then keeps; otherwise only reported).
bool route_forward_fuses(int M, int logits_dtype, int index_bits, int io_dtype, int cand_norm,
                         int B, int T, int N, int d, int K, hipStream_t st, bool claim,
                         const char** why) {
    const char* r = nullptr;
    const int mode = g_route_forward_mode.load(std::memory_order_relaxed);
    if (mode != HSN_ROUTE_FORWARD_ONE)
        r = mode == HSN_ROUTE_FORWARD_TWO ? "two launches are set (hsn_win_set_route_forward)"
                                          : "two launches are the library's choice (measured faster)";
    else if (M != 1) r = "the routed forward takes one unit";
    else if (logits_dtype != HSN_DTYPE_F32) r = "the routed forward takes fp32 logits";
    else if (index_bits != 32) r = "the routed forward writes int32 decisions";
    else if (io_dtype != HSN_DTYPE_F32) r = "the routed forward takes fp32 rows";
    else if (!workspace_layout(HSN_OP_FORWARD, B, T, N, d, K, 4, cand_norm).evmap)
        r = "the forward of this shape is not on the event maps";
    else if (!evmap_routes(B, T, N, d, K, &r)) {
    } else if (!evmap_route_claim(st, B, d, claim, &r)) {
    }
    if (r && why) *why = r;
    return r == nullptr;
}

}  // namespace

extern "C" int hsn_win_route_forward(
    const void* logits, int logits_dtype, int64_t width, const float* cost, void* cells,
    void* units, int index_bits, uint8_t* valid, float* theta, uint8_t* refreshed,
    int32_t* slots, int M, float lambda_cost, float cell_overhead, float shared_cost, float limit,
    int reserved, int reserved_units, const void* y, const void* gate_pre, int io_dtype,
    const float* cand_w, int cand_norm, float cand_eps, void* workspace, int64_t workspace_bytes,
    const uint8_t* reset, const float* h0, const float* q0, const int64_t* age0,
    const int64_t* pos0, void* q_pre, void* q_post, void* h_sel, void* h_old, float* h_max,
    float* h_T, float* q_T, int64_t* age_T, int64_t* pos_T, int B, int T, int N, int d, int K,
    void* stream) {
    HSN_ABI_BEGIN
    const char* fn = "hsn_win_route_forward";
    HSN_REQUIRE(slots != nullptr, HSN_ERR_INVALID_ARGUMENT,
                "hsn_win_route_forward: slots (the backward's decisions) is required");
    route_checks(fn, logits, logits_dtype, width, cost, cells, units, index_bits, valid, theta,
                 refreshed, M, reserved, reserved_units, B, T, N, K);
    forward_checks(fn, y, gate_pre, io_dtype, cand_w, cand_norm, reset, slots, h0, q0, age0,
                   pos0, age_T, pos_T, B, T, N, d, K);
    const WorkspaceLayout L = workspace_layout(HSN_OP_FORWARD, B, T, N, d, K,
                                               io_dtype == HSN_DTYPE_F32 ? 4 : 2, cand_norm);
    HSN_REQUIRE(L.bytes == 0 || (workspace && workspace_bytes >= int64_t(L.bytes)),
                HSN_ERR_INVALID_ARGUMENT,
                "hsn_win_route_forward: the workspace must hold " + std::to_string(L.bytes) +
                    " bytes (hsn_win_workspace_bytes)");
    hipStream_t st = as_stream(stream);
    if (route_forward_fuses(M, logits_dtype, index_bits, io_dtype, cand_norm, B, T, N, d, K, st,
                            true, nullptr)) {
        if (cand_norm) {
            y = rms_normalise(y, io_dtype, cand_w, cand_eps, static_cast<char*>(workspace) + L.rms,
                              int64_t(B) * T * K, d, st);
            HSN_HIP(hipGetLastError());
        }
        WindowRouteSpec rs{};
        rs.logits = static_cast<const float*>(logits), rs.width = width, rs.cost = cost;
        rs.cells = static_cast<int32_t*>(cells), rs.units = static_cast<int32_t*>(units);
        rs.valid = valid, rs.theta = theta, rs.refreshed = refreshed, rs.slots = slots;
        rs.reserved = reserved;
        rs.lambda = lambda_cost, rs.overhead = cell_overhead, rs.shared = shared_cost, rs.limit = limit;
        evmap_route_forward(rs, y, gate_pre, reset, h0, q0, age0, pos0, q_pre, q_post, h_sel,
                            h_old, h_max, h_T, q_T, age_T, pos_T, B, T, N, d, K, st);
    } else {  // the two launches, the router zeroing h_max for the sweep's max-reduction
        int rc = hsn_win_route(logits, logits_dtype, width, cost, nullptr, nullptr, cells, units,
                               index_bits, valid, theta, refreshed, slots, h_max, B, T, N, M, K, 0,
                               0, lambda_cost, cell_overhead, shared_cost, limit, reserved,
                               reserved_units, stream);
        if (rc != HSN_OK) throw AbiError{rc, hsn_win_last_error()};
        rc = hsn_win_forward(y, gate_pre, io_dtype, cand_w, cand_norm, cand_eps, workspace,
                             workspace_bytes, reset, slots, h0, q0, age0, pos0, q_pre, q_post,
                             h_sel, h_old, h_max, h_T, q_T, age_T, pos_T, B, T, N, d, K, stream);
        if (rc != HSN_OK) throw AbiError{rc, hsn_win_last_error()};
    }
    HSN_ABI_END
}

extern "C" int hsn_win_route_forward_fuses(int M, int logits_dtype, int index_bits, int io_dtype,
                                           int cand_norm, int B, int T, int N, int d, int K,
                                           void* stream, int* fuses) {
    HSN_ABI_BEGIN
    HSN_REQUIRE(fuses != nullptr, HSN_ERR_INVALID_ARGUMENT, "fuses is NULL");
    HSN_REQUIRE(B >= 1 && T >= 1 && N >= 1 && d >= 1 && K >= 1 && K <= N, HSN_ERR_INVALID_ARGUMENT,
                "bad dimensions");
    const char* why = nullptr;
    *fuses = route_forward_fuses(M, logits_dtype, index_bits, io_dtype, cand_norm, B, T, N, d, K,
                                 as_stream(stream), false, &why) ? 1 : 0;
    if (!*fuses && why) set_last_error(why);  // the reason, for hsn_win_last_error
    HSN_ABI_END
}

extern "C" int hsn_win_set_route_forward(int mode) {
    HSN_ABI_BEGIN
    HSN_REQUIRE(mode == HSN_ROUTE_FORWARD_AUTO || mode == HSN_ROUTE_FORWARD_ONE ||
                    mode == HSN_ROUTE_FORWARD_TWO,
                HSN_ERR_INVALID_ARGUMENT, "hsn_win_set_route_forward: unknown mode");
    g_route_forward_mode.store(mode, std::memory_order_relaxed);
    HSN_ABI_END
}

extern "C" int hsn_win_exchange_timeouts(unsigned* count, int clear) {
    HSN_ABI_BEGIN
    HSN_REQUIRE(count != nullptr, HSN_ERR_INVALID_ARGUMENT, "count is NULL");
    *count = evmap_exchange_timeouts(clear != 0);
    HSN_ABI_END
}

extern "C" int hsn_win_cell_update(const void* y, const void* gate, int io_dtype,
                                   const float* cand_w, int cand_norm, float cand_eps,
                                   void* rms_scratch, const float* h, const float* q,
                                   const int64_t* age, const int64_t* pos, const int64_t* cells,
                                   const uint8_t* valid, float* h_next, float* q_next,
                                   int64_t* age_next, int64_t* pos_next, float* h_sel,
                                   float* h_max, const uint8_t* reset, float* q_post, int B,
                                   int N, int d, int K, int t, int n_state, int n_slot, int t_out,
                                   void* stream) {
    HSN_ABI_BEGIN
    HSN_REQUIRE(y && gate && h && q && age && cells && valid && h_next && q_next && age_next &&
                    h_sel && h_max,
                HSN_ERR_INVALID_ARGUMENT, "hsn_win_cell_update: a required pointer is NULL");
    HSN_REQUIRE(B >= 1 && N >= 1 && d >= 1 && K >= 1 && K <= N, HSN_ERR_INVALID_ARGUMENT,
                "hsn_win_cell_update: bad dimensions");
    HSN_REQUIRE(t >= 0 && t < n_state && t_out >= 0 && t_out < n_state && t < n_slot,
                HSN_ERR_INVALID_ARGUMENT, "hsn_win_cell_update: record outside the tapes");
    HSN_REQUIRE(!pos_next || pos, HSN_ERR_INVALID_ARGUMENT,
                "hsn_win_cell_update: pos_next needs pos");
    HSN_REQUIRE(!cand_norm || (cand_w && rms_scratch), HSN_ERR_INVALID_ARGUMENT,
                "hsn_win_cell_update: the RMS candidate needs cand_w and rms_scratch");
    HSN_REQUIRE(io_dtype == HSN_DTYPE_F32 || io_dtype == HSN_DTYPE_BF16,
                HSN_ERR_UNSUPPORTED_DTYPE, "hsn_win_cell_update: io_dtype must be f32 or bf16");
    Geometry g;
    HSN_REQUIRE(choose_geometry(B, 1, N, d, K, fwd_lds_bytes, g), HSN_ERR_INVALID_ARGUMENT,
                "hsn_win_cell_update: the state slice does not fit the LDS (N too large)");
    const size_t lds = fwd_lds_bytes(N, g.S, g.W);
    hipStream_t st = as_stream(stream);
    if (cand_norm) {
        y = rms_normalise(y, io_dtype, cand_w, cand_eps, rms_scratch, int64_t(B) * K, d, st);
        HSN_HIP(hipGetLastError());
    }
    FwdArgs a{};
    a.y = y, a.g = gate, a.y_row = int64_t(K) * d;
    a.reset = nullptr, a.r_row = 0;
    const bool clear = reset && t + 1 < n_slot;
    a.clear = clear ? reset + t + 1 : nullptr, a.c_row = n_slot;
    a.cells = cells + int64_t(t) * K, a.valid = valid + int64_t(t) * K, a.s_row = int64_t(n_slot) * K;
    a.h0 = h + int64_t(t) * N * d, a.h0_row = int64_t(n_state) * N * d;
    a.q0 = q + int64_t(t) * d, a.q0_row = int64_t(n_state) * d;
    a.age0 = age + int64_t(t) * N, a.a0_row = int64_t(n_state) * N, a.pos0 = pos;
    a.q_pre = nullptr, a.q_post = q_post ? q_post + int64_t(t) * d : nullptr;
    a.qo_row = int64_t(n_slot) * d;
    a.h_sel = h_sel + int64_t(t) * K * d, a.h_old = nullptr, a.o_row = int64_t(n_slot) * K * d;
    a.h_max = h_max + t, a.hm_row = n_slot;
    a.h_T = h_next + int64_t(t_out) * N * d, a.hT_row = int64_t(n_state) * N * d;
    a.q_T = q_next + int64_t(t_out) * d, a.qT_row = int64_t(n_state) * d;
    a.age_T = age_next + int64_t(t_out) * N, a.aT_row = int64_t(n_state) * N, a.pos_T = pos_next;
    a.B = B, a.T = 1, a.N = N, a.d = d, a.K = K;
    a.W = g.W, a.Tc = g.Tc, a.region = fwd_region(N, g.S, g.W), a.divn = make_divn(N);
    // h_max is max-reduced across the row's slices: zero it first (a kernel, not a memset, so
    // the call stays capturable)
    hipLaunchKernelGGL(zero_strided_kernel, dim3((B + 255) / 256), dim3(256), 0, st, a.h_max,
                       int64_t(B), int64_t(n_slot));
    HSN_HIP(hipGetLastError());
    if (io_dtype == HSN_DTYPE_F32)
        HSN_HIP((launch_fwd<float, float, Cells64>(a, g.S, lds, st)));
    else
        HSN_HIP((launch_fwd<bf16_t, float, Cells64>(a, g.S, lds, st)));
    HSN_ABI_END
}

extern "C" int hsn_win_supports(int op, int B, int T, int N, int d, int K) {
    HSN_ABI_BEGIN
    HSN_REQUIRE(B >= 1 && T >= 1 && N >= 1 && d >= 1 && K >= 1, HSN_ERR_INVALID_ARGUMENT,
                "dimensions must be >= 1");
    const char* why = nullptr;
    switch (op) {
        case HSN_OP_FORWARD:
        case HSN_OP_BACKWARD:  // either path (the one the call would take)
            HSN_REQUIRE(K <= N, HSN_ERR_INVALID_ARGUMENT, "K exceeds N");
            choose_path(op, B, T, N, d, K, 4);
            break;
        case HSN_OP_CELL_UPDATE:
            HSN_REQUIRE(K <= N, HSN_ERR_INVALID_ARGUMENT, "K exceeds N");
            HSN_REQUIRE(slice_takes(op, B, 1, N, d, K, &why), HSN_ERR_INVALID_ARGUMENT, why);
            break;
        case HSN_OP_RECURRENCE:
            HSN_REQUIRE(slice_takes(op, B, T, N, d, K, &why), HSN_ERR_INVALID_ARGUMENT, why);
            break;
        case HSN_OP_ROUTE:
            HSN_REQUIRE(K <= N, HSN_ERR_INVALID_ARGUMENT, "K exceeds N");
            HSN_REQUIRE(K <= kWave, HSN_ERR_INVALID_ARGUMENT, "K above 64 (one lane per slot)");
            HSN_REQUIRE(N <= 64 * kWave, HSN_ERR_INVALID_ARGUMENT,
                        "N above 4096 (64 cells per lane)");
            break;
        default:
            HSN_REQUIRE(false, HSN_ERR_INVALID_ARGUMENT, "unknown op");
    }
    HSN_ABI_END
}
