// The cell-chain path of hsn_win_forward / hsn_win_backward (chain.cuh): the path choice, the
// workspace layout and the launchers.
#include <atomic>
#include <string>

#include "abi_util.h"
#include "chain.cuh"
#include "evmap.cuh"
#include "chain_host.h"

namespace hsn {

namespace {

std::atomic<int> g_path{kPathAuto};

constexpr size_t kAlign = 256;
inline size_t align_up(size_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

// Cells per workgroup: the smallest power of two from 16 that brings the grid to about 2048
// workgroups (eight per CU of the 256-CU chip), at most N.
inline int chain_cells(int B, int N) {
    int C = 16;
    while (C < N && int64_t(B) * ((N + C - 1) / C) > 2048) C *= 2;
    return C < N ? C : N;
}

// Events staged in LDS per workgroup: twice the group's expected count, 256..8192.
inline int chain_stage(int T, int N, int K, int C) {
    const int64_t expect = int64_t(C) * T * K / N;
    int64_t s = (2 * expect + 63) / 64 * 64;
    if (s < 256) s = 256;
    if (s > 8192) s = 8192;
    return static_cast<int>(s);
}

}  // namespace

int path_setting() { return g_path.load(std::memory_order_relaxed); }
void set_path_setting(int path) { g_path.store(path, std::memory_order_relaxed); }

bool slice_takes(int op, int B, int T, int N, int d, int K, const char** why) {
    Geometry g;
    const bool fwd = op == HSN_OP_FORWARD || op == HSN_OP_CELL_UPDATE;
    const int t = op == HSN_OP_CELL_UPDATE ? 1 : T;
    const bool ok = fwd ? choose_geometry(B, t, N, d, K, fwd_lds_bytes, g)
                        : choose_geometry(B, t, N, d, K, bwd_lds_bytes, g);
    if (!ok && why)
        *why = fwd ? "no state slice fits the LDS with one slot per lane (N or K too large)"
                   : "no cotangent slice fits the LDS with one slot per lane (N or K too large)";
    return ok;
}

bool chain_takes(int B, int T, int N, int d, int K, const char** why) {
    const char* r = nullptr;
    if (d > 64 * chain::kMaxV) r = "the cell chains take d <= 256";
    else if (K > chain::kMaxK) r = "the cell chains take K <= 255";
    else if (T >= (1 << 23)) r = "the cell chains take T < 2^23";
    else if (int64_t(chain::list_words(N, T, K)) * 4 > kLdsMax) r = "the row lists do not fit the LDS (N too large)";
    else {
        const int C = chain_cells(B, N);
        if (int64_t(chain::chain_words(T, C, chain_stage(T, N, K, C))) * 4 > kLdsMax)
            r = "the chains' reset table does not fit the LDS (T too large)";
    }
    if (r && why) *why = r;
    return r == nullptr;
}

bool evmap_takes(int op, int B, int T, int N, int d, int K, size_t elem, const char** why) {
    (void)B;
    const char* r = nullptr;
    if (op != HSN_OP_FORWARD && op != HSN_OP_BACKWARD) r = "the event maps take the window forward and backward";
    else if (elem != 4) r = "the event maps take fp32 rows only";
    else if (d % evmap::kS != 0) r = "the event maps take d a multiple of 8";
    else if (T > evmap::kChunks * evmap::kP) r = "the event maps take T <= 256";
    else if (K > evmap::kK) r = "the event maps take K <= 8";
    else if ((op == HSN_OP_FORWARD ? evmap::fwd_layout(N).bytes : evmap::bwd_layout(N).bytes) > size_t(kLdsMax))
        r = "the event maps' tables of N cells do not fit the LDS";
    else if ((int64_t(T) + 32) * K * d * 4 >= (int64_t(1) << 31)) r = "the event maps take (T + 32) K d * 4 < 2^31 bytes a row";
    if (r && why) *why = r;
    return r == nullptr;
}

// MI355X's compute units: the event maps' grid in one round
constexpr int64_t kEvmapOneRound = 256;

int choose_path(int op, int B, int T, int N, int d, int K, size_t elem) {
    const char* why_s = nullptr;
    const char* why_c = nullptr;
    const char* why_e = nullptr;
    const int setting = path_setting();
    const bool any = setting == kPathAuto;
    const bool e_ok = (any || setting == kPathEvmap) && evmap_takes(op, B, T, N, d, K, elem, &why_e);
    if (setting == kPathEvmap && !e_ok)
        throw AbiError{HSN_ERR_INVALID_ARGUMENT, std::string("(event-map path) ") + why_e};
    // The event maps first where they take the shape and their grid of B d / 8 workgroups (one
    // a CU: the maps hold most of the LDS) runs in one round on MI355X's 256 CUs: every
    // workgroup carries a fixed cost (the tables, the walk over all N cells), which a single
    // round pays once. Measured: B32 T256 N256 d64 K8 fp32 (256 workgroups) 28.2 + 28.3 us
    // against the slices' 30.2 + 29.0; B128 T128 N512 d128 K8 fp32 (2048, eight rounds) 213 +
    // 240 us against the chains' 127 + 139.
    if (e_ok && (setting == kPathEvmap || int64_t(B) * (d / evmap::kS) <= kEvmapOneRound))
        return kPathEvmap;
    const bool s_ok = (any || setting == kPathSlice) && slice_takes(op, B, T, N, d, K, &why_s);
    const bool c_ok = (any || setting == kPathChain) && chain_takes(B, T, N, d, K, &why_c);
    if (!s_ok && !c_ok) {
        std::string msg;
        if (setting == kPathSlice) msg = std::string("(slice path) ") + why_s;
        else if (setting == kPathChain) msg = std::string("(chain path) ") + why_c;
        else msg = std::string(why_s) + "; and " + why_c;
        throw AbiError{HSN_ERR_INVALID_ARGUMENT, msg};
    }
    if (!c_ok) return kPathSlice;
    if (!s_ok) return kPathChain;
    // Both slices and chains take it: the slices where a wavefront's piece of a slot row is a
    // full 32-byte sector and the state slice (N * S words) leaves room for chunks of the row in
    // LDS; the chains where the piece would be narrower (K large against d) or the slice large
    // (N large). Measured on MI355X: slices at B32 T256 N256 d64 K8 fp32 (S 8, 68 against 95 us
    // per step), chains at B64 T512 N1024 d64 K16 bf16 (S 4: 0.45 against 1.62 ms) and B128 T128
    // N512 d128 K8 fp32 (S 8, N S 4096: 0.31 against 0.43 ms).
    Geometry g;
    const bool fwd = op == HSN_OP_FORWARD;
    if (fwd) choose_geometry(B, T, N, d, K, fwd_lds_bytes, g);
    else choose_geometry(B, T, N, d, K, bwd_lds_bytes, g);
    return size_t(g.S) * elem >= 32 && int64_t(N) * g.S <= 2048 ? kPathSlice : kPathChain;
}

WorkspaceLayout workspace_layout(int op, int B, int T, int N, int d, int K, size_t elem,
                                 int cand_norm) {
    WorkspaceLayout L;
    const int path = choose_path(op, B, T, N, d, K, elem);
    L.chain = path == kPathChain;
    L.evmap = path == kPathEvmap;
    const int64_t slots = int64_t(B) * T * K;
    size_t at = 0;
    if (L.chain) {
        L.ptr = at;
        at = align_up(at + size_t(B) * (N + 1) * 4);
        L.ev = at;
        at = align_up(at + size_t(slots) * 4);
        L.sum = at;
        at = align_up(at + size_t(B) * T * d * 4);
        if (op == HSN_OP_FORWARD) {
            L.delta = at;
            at = align_up(at + size_t(slots) * d * 4);
            const int C = chain_cells(B, N);
            L.hmax = at;
            at = align_up(at + size_t(B) * T * ((N + C - 1) / C) * 4);
        }
    }
    L.rms = at;
    if (cand_norm) at = align_up(at + rms_inv_offset(slots, d, elem) + 4 * size_t(slots));
    L.bytes = at;
    return L;
}

namespace {

void build_lists(const int32_t* slots, int32_t* ptr, int32_t* ev, int B, int T, int N, int K,
                 hipStream_t st) {
    chain::ListArgs la{slots, ptr, ev, B, T, N, K};
    const size_t lds = size_t(chain::list_words(N, T, K)) * 4;
    HSN_HIP(allow_lds(chain::row_lists, lds));
    hipLaunchKernelGGL(chain::row_lists, dim3(B), dim3(chain::kListThreads), lds, st, la);
    HSN_HIP(hipGetLastError());
}

template <typename IO, int V>
void launch_chain_fwd(const chain::FwdArgs& a, size_t lds, hipStream_t st) {
    constexpr int NB = 4;  // measured: 4 ahead of 8 and 16 (most cells hold a few events)
    auto k = a.delta ? (a.hm_groups ? chain::chain_fwd<IO, V, NB, true, true>
                                    : chain::chain_fwd<IO, V, NB, true, false>)
                     : (a.hm_groups ? chain::chain_fwd<IO, V, NB, false, true>
                                    : chain::chain_fwd<IO, V, NB, false, false>);
    HSN_HIP(allow_lds(k, lds));
    hipLaunchKernelGGL(k, chain::chain_grid(a.B, (a.N + a.C - 1) / a.C),
                       dim3(chain::kChainThreads), lds, st, a);
    HSN_HIP(hipGetLastError());
}

template <typename IO, int V>
void launch_chain_bwd(const chain::BwdArgs& a, size_t lds, hipStream_t st) {
    auto k = chain::chain_bwd<IO, V, 4>;
    HSN_HIP(allow_lds(k, lds));
    hipLaunchKernelGGL(k, chain::chain_grid(a.B, (a.N + a.C - 1) / a.C),
                       dim3(chain::kChainThreads), lds, st, a);
    HSN_HIP(hipGetLastError());
}

template <typename IO, int V>
void launch_delta(const chain::DeltaArgs& a, bool pair, hipStream_t st) {
    const dim3 grid((a.T + 3) / 4, a.B);
    if (pair) hipLaunchKernelGGL((chain::summary_delta<IO, V, true>), grid, dim3(256), 0, st, a);
    else hipLaunchKernelGGL((chain::summary_delta<IO, V, false>), grid, dim3(256), 0, st, a);
    HSN_HIP(hipGetLastError());
}

template <typename IO>
void forward_io(const chain::FwdArgs& fa, const chain::DeltaArgs& da, const chain::ScanArgs& sa,
                bool pair, size_t lds, hipStream_t st) {
    const int V = (fa.d + 63) / 64;
    switch (V) {
        case 1: launch_chain_fwd<IO, 1>(fa, lds, st); launch_delta<IO, 1>(da, pair, st); break;
        case 2: launch_chain_fwd<IO, 2>(fa, lds, st); launch_delta<IO, 2>(da, pair, st); break;
        case 3: launch_chain_fwd<IO, 3>(fa, lds, st); launch_delta<IO, 3>(da, pair, st); break;
        default: launch_chain_fwd<IO, 4>(fa, lds, st); launch_delta<IO, 4>(da, pair, st); break;
    }
    hipLaunchKernelGGL((chain::summary_scan_fwd<IO>), dim3((fa.d + 63) / 64, fa.B),
                       dim3(64 * chain::kScanWaves), 0, st, sa);
    HSN_HIP(hipGetLastError());
}

template <typename IO>
void backward_io(const chain::BwdArgs& ba, const chain::ScanArgs& sa, size_t lds,
                 hipStream_t st) {
    hipLaunchKernelGGL((chain::summary_scan_bwd<IO>), dim3((ba.d + 63) / 64, ba.B),
                       dim3(64 * chain::kScanWaves), 0, st, sa);
    HSN_HIP(hipGetLastError());
    const int V = (ba.d + 63) / 64;
    switch (V) {
        case 1: launch_chain_bwd<IO, 1>(ba, lds, st); break;
        case 2: launch_chain_bwd<IO, 2>(ba, lds, st); break;
        case 3: launch_chain_bwd<IO, 3>(ba, lds, st); break;
        default: launch_chain_bwd<IO, 4>(ba, lds, st); break;
    }
}

}  // namespace

void chain_forward(const void* y, const void* gate_pre, int io_dtype, const uint8_t* reset,
                   const int32_t* slots, const float* h0, const float* q0, const int64_t* age0,
                   const int64_t* pos0, void* q_pre, void* q_post, void* h_sel, void* h_old,
                   float* h_max, float* h_T, float* q_T, int64_t* age_T, int64_t* pos_T, int B,
                   int T, int N, int d, int K, char* ws, const WorkspaceLayout& L,
                   hipStream_t st) {
    int32_t* ptr = reinterpret_cast<int32_t*>(ws + L.ptr);
    int32_t* ev = reinterpret_cast<int32_t*>(ws + L.ev);
    float* D = reinterpret_cast<float*>(ws + L.sum);
    // the summary reads the fp32 rows themselves; else the chains' fp32 deltas (bf16 rows are
    // rounded: summing them would leave q off the mean of h by up to a rounding of |h|)
    const bool pair = io_dtype == HSN_DTYPE_F32 && h_sel && h_old;
    float* delta = pair ? nullptr : reinterpret_cast<float*>(ws + L.delta);
    build_lists(slots, ptr, ev, B, T, N, K, st);
    chain::FwdArgs fa{};
    fa.y = y, fa.g = gate_pre, fa.ptr = ptr, fa.ev = ev, fa.reset = reset;
    fa.h0 = h0, fa.age0 = age0, fa.pos0 = pos0;
    fa.h_old = h_old, fa.h_sel = h_sel, fa.delta = delta;
    uint32_t* hm_groups = h_max ? reinterpret_cast<uint32_t*>(ws + L.hmax) : nullptr;
    fa.hm_groups = hm_groups, fa.h_T = h_T, fa.age_T = age_T, fa.pos_T = pos_T;
    fa.B = B, fa.T = T, fa.N = N, fa.d = d, fa.K = K;
    fa.C = chain_cells(B, N), fa.stage = chain_stage(T, N, K, fa.C);
    const size_t lds = size_t(chain::chain_words(T, fa.C, fa.stage)) * 4;
    chain::DeltaArgs da{};
    da.h_old = h_old, da.h_sel = h_sel, da.delta = delta, da.slots = slots, da.D = D;
    da.hm_groups = hm_groups, da.h_max = h_max;
    da.B = B, da.T = T, da.N = N, da.d = d, da.K = K, da.G = (N + fa.C - 1) / fa.C;
    chain::ScanArgs sa{};
    sa.D = D, sa.q0 = q0, sa.q_pre = q_pre, sa.q_post = q_post, sa.q_T = q_T;
    sa.reset = reset, sa.B = B, sa.T = T, sa.d = d, sa.divn = make_divn(N);
    if (io_dtype == HSN_DTYPE_F32) forward_io<float>(fa, da, sa, pair, lds, st);
    else forward_io<bf16_t>(fa, da, sa, pair, lds, st);
}

void chain_backward(const void* y, const void* gate_pre, const void* h_old, int io_dtype,
                    const int32_t* slots, const uint8_t* reset, const void* d_q_pre,
                    const void* d_q_post, const void* d_h_sel, const float* d_h_T,
                    const float* d_q_T, void* dy, void* dgate, float* d_h0, float* d_q0, int B,
                    int T, int N, int d, int K, char* ws, const WorkspaceLayout& L,
                    hipStream_t st) {
    int32_t* ptr = reinterpret_cast<int32_t*>(ws + L.ptr);
    int32_t* ev = reinterpret_cast<int32_t*>(ws + L.ev);
    float* share = reinterpret_cast<float*>(ws + L.sum);
    build_lists(slots, ptr, ev, B, T, N, K, st);
    chain::ScanArgs sa{};
    sa.dq_pre = d_q_pre, sa.dq_post = d_q_post, sa.dq_T = d_q_T, sa.share = share, sa.dq0 = d_q0;
    sa.reset = reset, sa.B = B, sa.T = T, sa.d = d, sa.divn = make_divn(N);
    chain::BwdArgs ba{};
    ba.y = y, ba.g = gate_pre, ba.h_old = h_old, ba.dsel = d_h_sel, ba.ptr = ptr, ba.ev = ev;
    ba.reset = reset, ba.share = share, ba.dh_T = d_h_T, ba.dy = dy, ba.dg = dgate, ba.dh0 = d_h0;
    ba.B = B, ba.T = T, ba.N = N, ba.d = d, ba.K = K;
    ba.C = chain_cells(B, N), ba.stage = chain_stage(T, N, K, ba.C);
    const size_t lds = size_t(chain::chain_words(T, ba.C, ba.stage)) * 4;
    if (io_dtype == HSN_DTYPE_F32) backward_io<float>(ba, sa, lds, st);
    else backward_io<bf16_t>(ba, sa, lds, st);
}

}  // namespace hsn

extern "C" int hsn_win_set_path(int path) {
    HSN_ABI_BEGIN
    HSN_REQUIRE(path == hsn::kPathAuto || path == hsn::kPathSlice || path == hsn::kPathChain ||
                    path == hsn::kPathEvmap,
                HSN_ERR_INVALID_ARGUMENT, "hsn_win_set_path: path must be 0 (auto), 1, 2 or 3");
    hsn::set_path_setting(path);
    HSN_ABI_END
}

extern "C" int hsn_win_path(int op, int B, int T, int N, int d, int K, int io_dtype, int* path) {
    HSN_ABI_BEGIN
    HSN_REQUIRE(path != nullptr, HSN_ERR_INVALID_ARGUMENT, "hsn_win_path: path is NULL");
    HSN_REQUIRE(op == HSN_OP_FORWARD || op == HSN_OP_BACKWARD, HSN_ERR_INVALID_ARGUMENT,
                "hsn_win_path: op must be HSN_OP_FORWARD or HSN_OP_BACKWARD");
    HSN_REQUIRE(B >= 1 && T >= 1 && N >= 1 && d >= 1 && K >= 1 && K <= N,
                HSN_ERR_INVALID_ARGUMENT, "hsn_win_path: bad dimensions");
    HSN_REQUIRE(io_dtype == HSN_DTYPE_F32 || io_dtype == HSN_DTYPE_BF16,
                HSN_ERR_UNSUPPORTED_DTYPE, "hsn_win_path: io_dtype must be f32 or bf16");
    *path = hsn::choose_path(op, B, T, N, d, K, io_dtype == HSN_DTYPE_F32 ? 4 : 2);
    HSN_ABI_END
}

extern "C" int hsn_win_workspace_bytes(int op, int B, int T, int N, int d, int K, int io_dtype,
                                       int cand_norm, int64_t* bytes) {
    HSN_ABI_BEGIN
    HSN_REQUIRE(bytes != nullptr, HSN_ERR_INVALID_ARGUMENT, "hsn_win_workspace_bytes: bytes is NULL");
    HSN_REQUIRE(op == HSN_OP_FORWARD || op == HSN_OP_BACKWARD, HSN_ERR_INVALID_ARGUMENT,
                "hsn_win_workspace_bytes: op must be HSN_OP_FORWARD or HSN_OP_BACKWARD");
    HSN_REQUIRE(B >= 1 && T >= 1 && N >= 1 && d >= 1 && K >= 1 && K <= N,
                HSN_ERR_INVALID_ARGUMENT, "hsn_win_workspace_bytes: bad dimensions");
    HSN_REQUIRE(io_dtype == HSN_DTYPE_F32 || io_dtype == HSN_DTYPE_BF16,
                HSN_ERR_UNSUPPORTED_DTYPE, "hsn_win_workspace_bytes: io_dtype must be f32 or bf16");
    HSN_REQUIRE(hsn::check_elems({int64_t(B) * T * K * d, int64_t(B) * N * d}),
                HSN_ERR_SIZE_OVERFLOW, "hsn_win_workspace_bytes: a tensor is too large");
    *bytes = static_cast<int64_t>(hsn::workspace_layout(op, B, T, N, d, K,
                                                        io_dtype == HSN_DTYPE_F32 ? 4 : 2,
                                                        cand_norm ? 1 : 0)
                                      .bytes);
    HSN_ABI_END
}
