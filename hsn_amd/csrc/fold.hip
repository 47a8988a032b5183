// The folded sweep's glue (reference kernels/cuda/hsn_window.cu:770-779,887-920, wrapper
// update_fold_op in python/hsn/kernels/window.py:765-853): after a position's round has written
// record t + 1 of the state tape, the next position's input row of the first product,
// x[t + 1, b, :] = [z[b, t + 1, :]; q[b, t + 1, :]; context[b, t + 1, :] (; f[b, :])], each value
// rounded once to x's dtype, f the mean of cells 0 .. F - 1 of record t + 1's state (the fast
// readout).
#include "abi_util.h"
#include "common.cuh"

namespace hsn {
namespace {

template <typename X>
__device__ __forceinline__ void put(void* x, int64_t i, float v) {
    static_cast<X*>(x)[i] = from_f32<X>(v);
}

__device__ __forceinline__ float get(const void* p, int dtype, int64_t i) {
    return dtype == HSN_DTYPE_BF16 ? to_f32(static_cast<const bf16_t*>(p)[i])
                                   : static_cast<const float*>(p)[i];
}

// One workgroup per row b; threads over the row's columns.
template <typename X>
__global__ __launch_bounds__(256) void fold_row(void* x, const void* z, int z_dtype, int d_z,
                                                const void* context, int c_dtype, int d_c,
                                                const float* tape_q, const float* tape_h,
                                                int n_fast, int B, int N, int d, int n,
                                                int n_state, int t_next) {
    const int b = blockIdx.x;
    const int width = d_z + d + d_c + (n_fast > 0 ? d : 0);
    const int64_t row = (int64_t(t_next) * B + b) * width;
    const float* q = tape_q + (int64_t(b) * n_state + t_next) * d;
    const float* h = tape_h + (int64_t(b) * n_state + t_next) * N * d;
    for (int c = threadIdx.x; c < width; c += blockDim.x) {
        float v;
        if (c < d_z) {
            v = get(z, z_dtype, (int64_t(b) * n + t_next) * d_z + c);
        } else if (c < d_z + d) {
            v = q[c - d_z];
        } else if (c < d_z + d + d_c) {
            v = get(context, c_dtype, (int64_t(b) * n + t_next) * d_c + (c - d_z - d));
        } else {  // the fast cells' mean, summed in cell order
            const int col = c - d_z - d - d_c;
            float s = 0.0f;
            for (int cell = 0; cell < n_fast; ++cell) s += h[int64_t(cell) * d + col];
            v = s / static_cast<float>(n_fast);
        }
        put<X>(x, row + c, v);
    }
}

}  // namespace
}  // namespace hsn

using namespace hsn;

extern "C" int hsn_win_fold_row(void* x, int x_dtype, const void* z, int z_dtype, int d_z,
                                const void* context, int c_dtype, int d_c, const float* tape_q,
                                const float* tape_h, int n_fast, int B, int N, int d, int n,
                                int n_state, int t_next, void* stream) {
    HSN_ABI_BEGIN
    HSN_REQUIRE(x && tape_q && (d_z == 0 || z) && (d_c == 0 || context) && (n_fast == 0 || tape_h),
                HSN_ERR_INVALID_ARGUMENT, "hsn_win_fold_row: a required pointer is NULL");
    HSN_REQUIRE(B >= 1 && N >= 1 && d >= 1 && n >= 1 && d_z >= 0 && d_c >= 0,
                HSN_ERR_INVALID_ARGUMENT, "hsn_win_fold_row: bad dimensions");
    HSN_REQUIRE(t_next >= 1 && t_next < n && t_next < n_state, HSN_ERR_INVALID_ARGUMENT,
                "hsn_win_fold_row: t_next must name a record of x and of the state tape");
    HSN_REQUIRE(n_fast >= 0 && n_fast <= N, HSN_ERR_INVALID_ARGUMENT,
                "hsn_win_fold_row: n_fast must lie in [0, N]");
    for (int dt : {x_dtype, z_dtype, c_dtype})
        HSN_REQUIRE(dt == HSN_DTYPE_F32 || dt == HSN_DTYPE_BF16, HSN_ERR_UNSUPPORTED_DTYPE,
                    "hsn_win_fold_row: dtypes must be f32 or bf16");
    HSN_REQUIRE(check_elems({int64_t(n) * B * (d_z + 2 * d + d_c), int64_t(B) * n_state * N * d}),
                HSN_ERR_SIZE_OVERFLOW, "hsn_win_fold_row: a tensor is too large");
    hipStream_t st = as_stream(stream);
    if (x_dtype == HSN_DTYPE_F32)
        hipLaunchKernelGGL(fold_row<float>, dim3(B), dim3(256), 0, st, x, z, z_dtype, d_z, context,
                           c_dtype, d_c, tape_q, tape_h, n_fast, B, N, d, n, n_state, t_next);
    else
        hipLaunchKernelGGL(fold_row<bf16_t>, dim3(B), dim3(256), 0, st, x, z, z_dtype, d_z,
                           context, c_dtype, d_c, tape_q, tape_h, n_fast, B, N, d, n, n_state,
                           t_next);
    HSN_HIP(hipGetLastError());
    HSN_ABI_END
}
