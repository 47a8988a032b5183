// The sparse round's gated delta update and gather (the reference's four-op ABI, the two ops on
// the window path: kernels/include/hsn_ops.h:79-99,155-187), for f32 / f16 / bf16 storage with
// fp32 arithmetic and one rounding per output.
//
// Threads own (row, column) pairs and walk the row's K slots in slot order: the in-place update
// needs no atomics (valid slots name distinct cells) and every sum has a fixed order, so the
// results are reproducible run to run whatever `deterministic` says.
#include "common.cuh"

#include <type_traits>

namespace hsn {

namespace {

// grad_h = G (the copy the slot pass then overwrites), or zero when G is NULL.
template <typename F>
__global__ __launch_bounds__(256) void copy_or_zero(const F* src, F* dst, int64_t n) {
    const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) dst[i] = src ? src[i] : from_f32<F>(0.0f);
}

// A thread per (row, column) walks the row's K slots in order, 8 at a time: the group's valid
// flags, cells, gates and candidates are loaded first, then the group's old values of h in one
// batch; a cell that an earlier slot of the group already updated takes that slot's stored value
// (in-place order, as if each slot read h after the slots before it).
template <typename F>
__global__ __launch_bounds__(256) void gated_update_fwd(F* h, F* q, int32_t* age,
                                                        const int32_t* cell_idx,
                                                        const int32_t* valid, const F* c,
                                                        const F* bgate, F* h_old_saved, int B,
                                                        int N, int d, int K) {
    const int64_t e = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (e >= int64_t(B) * d) return;
    const int r = static_cast<int>(e / d), x = static_cast<int>(e - int64_t(r) * d);
    constexpr int G = 8;
    float delta = 0.0f;
    for (int k0 = 0; k0 < K; k0 += G) {
        bool on[G];
        int cell[G];
        float cv[G], bv[G], old[G], stored[G];
#pragma unroll
        for (int i = 0; i < G; ++i) {
            const int64_t s = int64_t(r) * K + k0 + i;
            on[i] = k0 + i < K && valid[s] != 0;
            cell[i] = on[i] ? cell_idx[s] : -1;
            cv[i] = on[i] ? to_f32(c[s * d + x]) : 0.0f;
            bv[i] = on[i] ? to_f32(bgate[s * d + x]) : 0.0f;
        }
#pragma unroll
        for (int i = 0; i < G; ++i)
            old[i] = on[i] ? to_f32(h[(int64_t(r) * N + cell[i]) * d + x]) : 0.0f;
#pragma unroll
        for (int i = 0; i < G; ++i) {
            stored[i] = 0.0f;
            if (k0 + i >= K) continue;
            const int64_t o = (int64_t(r) * K + k0 + i) * d + x;
            if (on[i]) {
                float prev = old[i];
#pragma unroll
                for (int t = 0; t < i; ++t)
                    if (on[t] && cell[t] == cell[i]) prev = stored[t];  // the latest earlier slot
                const F st = from_f32<F>((1.0f - bv[i]) * prev + bv[i] * cv[i]);
                stored[i] = to_f32(st);
                h[(int64_t(r) * N + cell[i]) * d + x] = st;
                h_old_saved[o] = from_f32<F>(prev);
                delta += stored[i] - prev;
                if (x == 0) age[int64_t(r) * N + cell[i]] = 0;
            } else {
                h_old_saved[o] = from_f32<F>(0.0f);
            }
        }
    }
    const int64_t qi = int64_t(r) * d + x;
    q[qi] = from_f32<F>(to_f32(q[qi]) + delta / static_cast<float>(N));
}

template <typename F>
__global__ __launch_bounds__(256) void gated_update_bwd(const int32_t* cell_idx,
                                                        const int32_t* valid, const F* c,
                                                        const F* bgate, const F* h_old,
                                                        const F* G, const F* g, F* grad_h,
                                                        F* grad_q, F* grad_c, F* grad_b, int B,
                                                        int N, int d, int K) {
    const int64_t e = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (e >= int64_t(B) * d) return;
    const int r = static_cast<int>(e / d), x = static_cast<int>(e - int64_t(r) * d);
    const float gq = to_f32(g[int64_t(r) * d + x]);
    const float share = gq / static_cast<float>(N);
    grad_q[int64_t(r) * d + x] = g[int64_t(r) * d + x];
    constexpr int S = 8;  // slots a batch: every load of the batch issued before its stores
    for (int k0 = 0; k0 < K; k0 += S) {
        bool on[S];
        int64_t hi[S];
        float Gn[S], bv[S], cv[S], ov[S];
#pragma unroll
        for (int i = 0; i < S; ++i) {
            const int64_t s = int64_t(r) * K + k0 + i;
            on[i] = k0 + i < K && valid[s] != 0;
            hi[i] = on[i] ? (int64_t(r) * N + cell_idx[s]) * d + x : 0;
        }
#pragma unroll
        for (int i = 0; i < S; ++i) {
            const int64_t o = (int64_t(r) * K + k0 + i) * d + x;
            Gn[i] = on[i] ? to_f32(G[hi[i]]) : 0.0f;
            bv[i] = on[i] ? to_f32(bgate[o]) : 0.0f;
            cv[i] = on[i] ? to_f32(c[o]) : 0.0f;
            ov[i] = on[i] ? to_f32(h_old[o]) : 0.0f;
        }
#pragma unroll
        for (int i = 0; i < S; ++i) {
            if (k0 + i >= K) continue;
            const int64_t o = (int64_t(r) * K + k0 + i) * d + x;
            if (on[i]) {
                const float total = Gn[i] + share;
                grad_h[hi[i]] = from_f32<F>((1.0f - bv[i]) * Gn[i] - bv[i] * share);
                grad_c[o] = from_f32<F>(bv[i] * total);
                grad_b[o] = from_f32<F>((cv[i] - ov[i]) * total);
            } else {
                grad_c[o] = from_f32<F>(0.0f);
                grad_b[o] = from_f32<F>(0.0f);
            }
        }
    }
}

template <typename F>
__global__ __launch_bounds__(256) void gather_fwd(const F* u, const F* eps, const F* h, const F* m,
                                                  const int32_t* cell_idx, F* v, int B, int N,
                                                  int d, int K) {
    const int64_t e = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    const int64_t w = 4 * int64_t(d);
    if (e >= int64_t(B) * K * w) return;
    const int64_t s = e / w;
    const int c = static_cast<int>(e - s * w);
    const int r = static_cast<int>(s / K);
    const int part = c / d, x = c - part * d;
    F out;
    if (part == 0) out = u[int64_t(r) * d + x];
    else if (part == 1) out = eps[int64_t(r) * d + x];
    else if (part == 2) out = h[(int64_t(r) * N + cell_idx[s]) * d + x];
    else out = m[s * d + x];
    v[e] = out;
}

template <typename F>
__global__ __launch_bounds__(256) void gather_bwd(const F* grad_v, const int32_t* cell_idx,
                                                  F* grad_u, F* grad_eps, F* grad_h, F* grad_m,
                                                  int B, int N, int d, int K) {
    const int64_t e = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (e >= int64_t(B) * d) return;
    const int r = static_cast<int>(e / d), x = static_cast<int>(e - int64_t(r) * d);
    const int64_t w = 4 * int64_t(d);
    float su = 0.0f, se = 0.0f;
    // slot order, 8 slots at a time: the batch's cells and grad_v values, then its reads of
    // grad_h, are issued together; repeats of one cell add in slot order, a repeat inside the
    // batch taking the earlier slot's stored sum
    constexpr int G = 8;
    for (int k0 = 0; k0 < K; k0 += G) {
        int64_t hi[G];
        float gu[G], ge[G], gh[G], old[G], stored[G];
        F gm[G];
#pragma unroll
        for (int i = 0; i < G; ++i) {
            const int64_t s = int64_t(r) * K + min(k0 + i, K - 1);
            const F* gv = grad_v + s * w;
            hi[i] = (int64_t(r) * N + cell_idx[s]) * d + x;
            gu[i] = to_f32(gv[x]);
            ge[i] = to_f32(gv[d + x]);
            gh[i] = to_f32(gv[2 * d + x]);
            gm[i] = gv[3 * d + x];
        }
#pragma unroll
        for (int i = 0; i < G; ++i) old[i] = k0 + i < K ? to_f32(grad_h[hi[i]]) : 0.0f;
#pragma unroll
        for (int i = 0; i < G; ++i) {
            stored[i] = 0.0f;
            if (k0 + i >= K) continue;
            su += gu[i];
            se += ge[i];
            float prev = old[i];
#pragma unroll
            for (int t = 0; t < i; ++t)
                if (hi[t] == hi[i]) prev = stored[t];  // the latest earlier slot of the batch
            const F st = from_f32<F>(prev + gh[i]);
            stored[i] = to_f32(st);
            grad_h[hi[i]] = st;
            grad_m[(int64_t(r) * K + k0 + i) * d + x] = gm[i];
        }
    }
    grad_u[int64_t(r) * d + x] = from_f32<F>(su);
    grad_eps[int64_t(r) * d + x] = from_f32<F>(se);
}

// The 16-bit gather backward: a repeated cell's grad_h is the fp32 sum over its slots in slot
// order, rounded once to F (the ABI's accumulation). A thread per (row, column) walks the slots;
// each slot writes its cell's sum over the slots up to it (the same cells found by a scan of the
// earlier slots), so the cell's last slot writes the whole sum.
template <typename F>
__global__ __launch_bounds__(256) void gather_bwd_narrow(const F* grad_v, const int32_t* cell_idx,
                                                         F* grad_u, F* grad_eps, F* grad_h,
                                                         F* grad_m, int B, int N, int d, int K) {
    const int64_t e = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (e >= int64_t(B) * d) return;
    const int r = static_cast<int>(e / d), x = static_cast<int>(e - int64_t(r) * d);
    const int64_t w = 4 * int64_t(d);
    const int32_t* cells = cell_idx + int64_t(r) * K;
    const F* gv = grad_v + int64_t(r) * K * w;
    float su = 0.0f, se = 0.0f;
    for (int i = 0; i < K; ++i) {
        const F* g = gv + i * w;
        su += to_f32(g[x]);
        se += to_f32(g[d + x]);
        grad_m[(int64_t(r) * K + i) * d + x] = g[3 * d + x];
        const int c = cells[i];
        float sum = 0.0f;
        for (int j = 0; j <= i; ++j)
            if (cells[j] == c) sum += to_f32(gv[j * w + 2 * d + x]);
        grad_h[(int64_t(r) * N + c) * d + x] = from_f32<F>(sum);
    }
    grad_u[int64_t(r) * d + x] = from_f32<F>(su);
    grad_eps[int64_t(r) * d + x] = from_f32<F>(se);
}

inline int grid_of(int64_t n) { return static_cast<int>((n + 255) / 256); }

}  // namespace
}  // namespace hsn

#include "../../include/hsn_ops.h"
#include "abi_util.h"

using namespace hsn;

namespace {

void check_dims(int B, int N, int d, int K, const char* who) {
    HSN_REQUIRE(B >= 1 && N >= 1 && d >= 1 && K >= 1, HSN_ERR_INVALID_ARGUMENT,
                std::string(who) + ": dimensions must be >= 1");
    HSN_REQUIRE(int64_t(B) * N * d <= INT32_MAX && int64_t(B) * K * 4 * d <= INT32_MAX,
                HSN_ERR_SIZE_OVERFLOW, std::string(who) + ": an element count exceeds INT32_MAX");
}

void check_dtype(int dtype, const char* who) {
    HSN_REQUIRE(dtype == HSN_DTYPE_F32 || dtype == HSN_DTYPE_F16 || dtype == HSN_DTYPE_BF16,
                HSN_ERR_UNSUPPORTED_DTYPE, std::string(who) + ": unknown dtype code");
}

template <template <typename> class Fn, typename... Args>
void by_dtype(int dtype, Args&&... args) {
    if (dtype == HSN_DTYPE_F32) Fn<float>::run(args...);
    else if (dtype == HSN_DTYPE_F16) Fn<_Float16>::run(args...);
    else Fn<bf16_t>::run(args...);
}

template <typename F>
struct RunUpdate {
    static void run(void* h, void* q, int32_t* age, const int32_t* cell_idx, const int32_t* valid,
                    const void* c, const void* b, void* h_old_saved, int B, int N, int d, int K,
                    hipStream_t st) {
        hipLaunchKernelGGL((gated_update_fwd<F>), dim3(grid_of(int64_t(B) * d)), dim3(256), 0, st,
                           static_cast<F*>(h), static_cast<F*>(q), age, cell_idx, valid,
                           static_cast<const F*>(c), static_cast<const F*>(b),
                           static_cast<F*>(h_old_saved), B, N, d, K);
    }
};

template <typename F>
struct RunUpdateBwd {
    static void run(const int32_t* cell_idx, const int32_t* valid, const void* c, const void* b,
                    const void* h_old, const void* G, const void* g, void* grad_h, void* grad_q,
                    void* grad_c, void* grad_b, int B, int N, int d, int K, hipStream_t st) {
        const int64_t n = int64_t(B) * N * d;
        hipLaunchKernelGGL((copy_or_zero<F>), dim3(grid_of(n)), dim3(256), 0, st,
                           static_cast<const F*>(G), static_cast<F*>(grad_h), n);
        hipLaunchKernelGGL((gated_update_bwd<F>), dim3(grid_of(int64_t(B) * d)), dim3(256), 0, st,
                           cell_idx, valid, static_cast<const F*>(c), static_cast<const F*>(b),
                           static_cast<const F*>(h_old), static_cast<const F*>(G),
                           static_cast<const F*>(g), static_cast<F*>(grad_h),
                           static_cast<F*>(grad_q), static_cast<F*>(grad_c),
                           static_cast<F*>(grad_b), B, N, d, K);
    }
};

template <typename F>
struct RunGather {
    static void run(const void* u, const void* eps, const void* h, const void* m,
                    const int32_t* cell_idx, void* v, int B, int N, int d, int K, hipStream_t st) {
        hipLaunchKernelGGL((gather_fwd<F>), dim3(grid_of(int64_t(B) * K * 4 * d)), dim3(256), 0,
                           st, static_cast<const F*>(u), static_cast<const F*>(eps),
                           static_cast<const F*>(h), static_cast<const F*>(m), cell_idx,
                           static_cast<F*>(v), B, N, d, K);
    }
};

template <typename F>
struct RunGatherBwd {
    static void run(const void* grad_v, const int32_t* cell_idx, void* grad_u, void* grad_eps,
                    void* grad_h, void* grad_m, int B, int N, int d, int K, hipStream_t st) {
        const int64_t n = int64_t(B) * N * d;
        hipLaunchKernelGGL((copy_or_zero<F>), dim3(grid_of(n)), dim3(256), 0, st,
                           static_cast<const F*>(nullptr), static_cast<F*>(grad_h), n);
        // fp32 rows: repeats forwarded in registers in slot order (exact); 16-bit rows: each
        // cell's sum kept in fp32 and rounded once
        auto kernel = std::is_same<F, float>::value ? gather_bwd<F> : gather_bwd_narrow<F>;
        hipLaunchKernelGGL(kernel, dim3(grid_of(int64_t(B) * d)), dim3(256), 0, st,
                           static_cast<const F*>(grad_v), cell_idx, static_cast<F*>(grad_u),
                           static_cast<F*>(grad_eps), static_cast<F*>(grad_h),
                           static_cast<F*>(grad_m), B, N, d, K);
    }
};

}  // namespace

extern "C" int hsn_gather_concat(const void* u, const void* eps, const void* h, const void* m,
                                 const int32_t* cell_idx, void* v, int B, int N, int d, int K,
                                 int dtype, void* stream) {
    HSN_ABI_BEGIN
    check_dims(B, N, d, K, "hsn_gather_concat");
    check_dtype(dtype, "hsn_gather_concat");
    HSN_REQUIRE(u && eps && h && m && cell_idx && v, HSN_ERR_INVALID_ARGUMENT,
                "hsn_gather_concat: a pointer is NULL");
    by_dtype<RunGather>(dtype, u, eps, h, m, cell_idx, v, B, N, d, K, as_stream(stream));
    HSN_HIP(hipGetLastError());
    HSN_ABI_END
}

extern "C" int hsn_gather_concat_bwd(const void* grad_v, const int32_t* cell_idx, void* grad_u,
                                     void* grad_eps, void* grad_h, void* grad_m, int B, int N,
                                     int d, int K, int dtype, int deterministic, void* stream) {
    HSN_ABI_BEGIN
    check_dims(B, N, d, K, "hsn_gather_concat_bwd");
    check_dtype(dtype, "hsn_gather_concat_bwd");
    HSN_REQUIRE(deterministic == 0 || deterministic == 1, HSN_ERR_INVALID_ARGUMENT,
                "hsn_gather_concat_bwd: deterministic must be 0 or 1");
    HSN_REQUIRE(grad_v && cell_idx && grad_u && grad_eps && grad_h && grad_m,
                HSN_ERR_INVALID_ARGUMENT, "hsn_gather_concat_bwd: a pointer is NULL");
    by_dtype<RunGatherBwd>(dtype, grad_v, cell_idx, grad_u, grad_eps, grad_h, grad_m, B, N, d, K,
                           as_stream(stream));
    HSN_HIP(hipGetLastError());
    HSN_ABI_END
}

extern "C" int hsn_gated_delta_update(void* h, void* q, int32_t* age, const int32_t* cell_idx,
                                      const int32_t* valid, const void* c, const void* b,
                                      void* h_old_saved, int B, int N, int d, int K, int dtype,
                                      void* stream) {
    HSN_ABI_BEGIN
    check_dims(B, N, d, K, "hsn_gated_delta_update");
    check_dtype(dtype, "hsn_gated_delta_update");
    HSN_REQUIRE(h && q && age && cell_idx && valid && c && b && h_old_saved,
                HSN_ERR_INVALID_ARGUMENT, "hsn_gated_delta_update: a pointer is NULL");
    by_dtype<RunUpdate>(dtype, h, q, age, cell_idx, valid, c, b, h_old_saved, B, N, d, K,
                        as_stream(stream));
    HSN_HIP(hipGetLastError());
    HSN_ABI_END
}

extern "C" int hsn_gated_delta_update_bwd(const int32_t* cell_idx, const int32_t* valid,
                                          const void* c, const void* b, const void* h_old_saved,
                                          const void* grad_h_out, const void* grad_q_out,
                                          void* grad_h, void* grad_q, void* grad_c, void* grad_b,
                                          int B, int N, int d, int K, int dtype, void* stream) {
    HSN_ABI_BEGIN
    check_dims(B, N, d, K, "hsn_gated_delta_update_bwd");
    check_dtype(dtype, "hsn_gated_delta_update_bwd");
    HSN_REQUIRE(cell_idx && valid && c && b && h_old_saved && grad_h_out && grad_q_out &&
                    grad_h && grad_q && grad_c && grad_b,
                HSN_ERR_INVALID_ARGUMENT, "hsn_gated_delta_update_bwd: a pointer is NULL");
    by_dtype<RunUpdateBwd>(dtype, cell_idx, valid, c, b, h_old_saved, grad_h_out, grad_q_out,
                           grad_h, grad_q, grad_c, grad_b, B, N, d, K, as_stream(stream));
    HSN_HIP(hipGetLastError());
    HSN_ABI_END
}
