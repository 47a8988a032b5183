// The trainer's per-step passes after backward() on gfx950 (reference kernels/cuda/hsn_trainer.cu:
// 60-182; wrappers python/hsn/kernels/trainer.py:111-229): the AdamW step of ordinary and of
// stacked unit tensors, the weight average's lerp, the float64 clip's scaling, a copy, and the
// update caps' two passes, each one launch over a list of fp32 tensors.
//
// Each pass equals, value for value, the sequence of PyTorch multi-tensor operations it replaces
// (python/hsn/train/lazy_adam.py:462-486,573-626, weight_ema.py, grad_norm.py, update_limit.py).
// Every PyTorch operation rounds once, so each step below is one correctly rounded operation, and
// a fused multiply-add stands exactly where PyTorch's kernel has one (its lerp, addcmul and
// addcdiv contract a product into the sum): no other contraction. The arithmetic is written with
// plain operators in this file, under the pragma below, with __builtin_fmaf for the fused forms
// and __builtin_sqrtf (correctly rounded, as hipcc's default -fhip-fp32-correctly-rounded-divide-
// sqrt makes it and '/'): the header intrinsics __fadd_rn, __fmul_rn, ... are plain operators
// compiled under the header's own contraction setting, and __fsqrt_rn is the native (1 ulp)
// square root, so neither gives these guarantees.
//
// Work: the tensors of a launch form one index space of 1024-element chunks; a workgroup takes one
// chunk (its tensor found by a binary search over the tensors' first chunks, uniform per
// workgroup), a thread four elements 256 apart, so every load and store of a wavefront is one
// coalesced run. The passes are HBM-bound: AdamW moves 28 bytes an element (four rows read, three
// written).
#include <string>
#include <type_traits>

#include "../../include/hsn_trainer.h"
#include "abi_util.h"
#include "common.cuh"

#pragma clang fp contract(off)

namespace hsn {
namespace {

constexpr int kTrRows = 4;      // operands per tensor
constexpr int kTrUnits = 64;    // units of a stacked unit tensor (the reference's HSN_TR_UNITS)
constexpr int kTrThreads = 256;
constexpr int kTrPer = 4;       // elements per thread
constexpr int kTrChunk = kTrThreads * kTrPer;

enum TrOp : int { kAdamW, kAdamWUnits, kLerp, kScale64, kCopy, kLimitSquares, kLimitProject };

// The by-value launch descriptor (under the 4 KiB of kernel arguments): T tensors a launch (a
// longer list takes several), and with U the unit coefficients of the stacked-unit AdamW, whose
// 1.5 KiB leave room for 48 tensors; the other passes take 88 (the model's 198 tensors in three
// launches, not five).
template <int T, bool U>
struct TrArgsT {
    static constexpr int kTensors = T;
    float* p[kTrRows][T];  // operand r of tensor j
    int64_t numel[T];
    int32_t chunk0[T + 1];  // the first chunk of tensor j; chunk0[n] = all chunks
    int32_t n;              // tensors
    int32_t flag;           // AdamW: weight decay on
    int32_t units;          // AdamW units: M
    float f[8];
    float u[U ? 6 : 1][U ? kTrUnits : 1];
    const double* coef;  // scale64: the coefficient, one f64 on the device
};
using TrArgsUnits = TrArgsT<48, true>;
using TrArgs = TrArgsT<88, false>;
static_assert(sizeof(TrArgsUnits) <= 4096 && sizeof(TrArgs) <= 4096,
              "kernel arguments take at most 4 KiB");
template <int OP>
using TrArgsOf = std::conditional_t<OP == kAdamWUnits, TrArgsUnits, TrArgs>;

// at::native::lerp (ATen/native/Lerp.h) as the device compiles it: the small-weight form
// self + w (end - self) and the large one end - (end - self)(1 - w), each with its product
// contracted into the sum.
__device__ __forceinline__ float tr_lerp(float self, float end, float w) {
    const float diff = end - self;
    if (fabsf(w) < 0.5f) return __builtin_fmaf(w, diff, self);
    return __builtin_fmaf(-diff, 1.0f - w, end);
}
// addcmul / addcdiv as PyTorch's pointwise kernels: input + value * (t1 op t2), contracted;
// with value 1 the product of t1 and t2 itself (addcmul) or a plain sum (addcdiv).
__device__ __forceinline__ float tr_addcmul(float input, float t1, float t2, float value) {
    if (value == 1.0f) return __builtin_fmaf(t1, t2, input);
    return __builtin_fmaf(value, t1 * t2, input);
}
__device__ __forceinline__ float tr_addcdiv(float input, float t1, float t2, float value) {
    const float q = t1 / t2;
    if (value == 1.0f) return input + q;
    return __builtin_fmaf(value, q, input);
}

// The operand rows each pass reads and writes (bit r: row r).
template <int OP>
struct TrRows;
template <> struct TrRows<kAdamW> { static constexpr int rd = 0xF, wr = 0xD; };
template <> struct TrRows<kAdamWUnits> { static constexpr int rd = 0xF, wr = 0xD; };
template <> struct TrRows<kLerp> { static constexpr int rd = 0x3, wr = 0x1; };
template <> struct TrRows<kScale64> { static constexpr int rd = 0x1, wr = 0x1; };
template <> struct TrRows<kCopy> { static constexpr int rd = 0x2, wr = 0x1; };
template <> struct TrRows<kLimitSquares> { static constexpr int rd = 0x3, wr = 0xC; };
template <> struct TrRows<kLimitProject> { static constexpr int rd = 0x3, wr = 0x5; };

// What stays fixed over a workgroup's elements: the tensor's unit size, the clip's coefficient,
// the projection's group.
struct TrUniform {
    int64_t base;      // the chunk's first element
    int64_t per_unit;  // a unit's elements
    int64_t rem0;      // base's place in its unit (base = unit0 per_unit + rem0)
    int unit0;         // base's unit
    const float (*u)[kTrUnits];  // the unit coefficients, staged in LDS
    double coef;
    float scale;
    bool clipped;
};

// One element: x[r] holds row r's value on entry (the rows the pass reads) and on exit (the
// rows it writes); o is the element's index in its tensor.
template <int OP, typename A>
__device__ __forceinline__ void tr_op(const A& a, const TrUniform& q, int64_t o, float (&x)[4]) {
    if constexpr (OP == kAdamW) {
        // lazy_adam._dense_steps: p *= 1 - lr wd; m = lerp(m, g, 1 - beta1); v *= beta2;
        // v = addcmul(v, g, g, 1 - beta2); den = sqrt(v) * (1 / sqrt(1 - beta2^t)) + eps;
        // p = addcdiv(p, m, den, -lr / (1 - beta1^t))
        const float g = x[1];
        float p = x[0];
        if (a.flag) p = p * a.f[0];
        const float m = tr_lerp(x[2], g, a.f[1]);
        const float v = tr_addcmul(x[3] * a.f[2], g, g, a.f[3]);
        const float den = __builtin_sqrtf(v) * a.f[4] + a.f[5];
        x[0] = tr_addcdiv(p, m, den, a.f[6]);
        x[2] = m;
        x[3] = v;
    } else if constexpr (OP == kAdamWUnits) {
        // lazy_adam._unit_step with the unit's coefficients (an inactive unit: gradient 0,
        // factors 1 and 0): g = active ? grad : 0; p *= decay; m = lerp(m, g, w); v *= b2f;
        // v = addcmul(v, g, g, 1 - beta2); den = sqrt(v) / bc2s + eps;
        // p = addcdiv(p, m * step, den, -1)
        // the element's unit from the chunk's: rel < kTrChunk + per_unit, so a unit longer
        // than a chunk is crossed at most once and a shorter one needs a 32-bit division
        const int64_t rel = o - q.base + q.rem0;
        const int unit = q.per_unit > kTrChunk
                             ? q.unit0 + (rel >= q.per_unit ? 1 : 0)
                             : q.unit0 + static_cast<int>(static_cast<uint32_t>(rel) /
                                                          static_cast<uint32_t>(q.per_unit));
        const float g = q.u[0][unit] != 0.0f ? x[1] : 0.0f;
        float p = x[0];
        if (a.flag) p = p * q.u[1][unit];
        const float m = tr_lerp(x[2], g, q.u[2][unit]);
        const float v = tr_addcmul(x[3] * q.u[3][unit], g, g, a.f[3]);
        const float den = __builtin_sqrtf(v) / q.u[4][unit] + a.f[5];
        x[0] = tr_addcdiv(p, m * q.u[5][unit], den, -1.0f);
        x[2] = m;
        x[3] = v;
    } else if constexpr (OP == kLerp) {  // weight_ema: self = lerp(self, end, w)
        x[0] = tr_lerp(x[0], x[1], a.f[0]);
    } else if constexpr (OP == kScale64) {  // grad_norm (float64): grad = f32(f64(grad) * c)
        x[0] = static_cast<float>(static_cast<double>(x[0]) * q.coef);
    } else if constexpr (OP == kCopy) {
        x[0] = x[1];
    } else if constexpr (OP == kLimitSquares) {  // update_limit: old^2, (param - old)^2
        const float delta = x[0] - x[1];
        x[2] = x[1] * x[1];
        x[3] = delta * delta;
    } else {  // kLimitProject: param = old + (param - old) scale where clipped; (param - old)^2
        if (q.clipped) x[0] = x[1] + (x[0] - x[1]) * q.scale;
        const float applied = x[0] - x[1];
        x[2] = applied * applied;
    }
}

// One workgroup per chunk of kTrChunk elements of one tensor, a thread kTrPer elements 256 apart.
// Measured on an AdamW pass over 1 GiB rows: 5.77 TB/s, against 6.16 TB/s for a plain copy; 16-byte
// accesses (runs of four elements a thread, loads issued together or per run) and sixteen elements
// a thread measured 5.3-5.4 TB/s, a grid-stride loop 4.5 TB/s.
template <int OP>
__global__ __launch_bounds__(kTrThreads) void tr_pass(TrArgsOf<OP> a) {
    constexpr int kRd = TrRows<OP>::rd;
    const int c = blockIdx.x;
    int lo = 0, hi = a.n - 1;  // the tensor holding chunk c: the last j with chunk0[j] <= c
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (a.chunk0[mid] <= c) lo = mid;
        else hi = mid - 1;
    }
    const int j = uniform(lo);
    const int64_t base = int64_t(c - a.chunk0[j]) * kTrChunk;
    const int64_t numel = a.numel[j];
    TrUniform q{};
    if constexpr (OP == kAdamWUnits) {
        __shared__ float su[6][kTrUnits];
        for (int i = threadIdx.x; i < 6 * kTrUnits; i += kTrThreads)
            su[i / kTrUnits][i % kTrUnits] = a.u[i / kTrUnits][i % kTrUnits];
        __syncthreads();
        q.u = su;
        q.base = base;
        q.per_unit = numel / a.units;
        q.unit0 = static_cast<int>(base / q.per_unit);
        q.rem0 = base - int64_t(q.unit0) * q.per_unit;
    }
    if constexpr (OP == kScale64) q.coef = *a.coef;
    if constexpr (OP == kLimitProject) {
        const float* group = a.p[3][j];
        q.scale = group[0];
        q.clipped = group[1] != 0.0f;
    }
    // rows the pass writes: the projection rewrites the parameter only in a clipped group
    int wr = TrRows<OP>::wr;
    if constexpr (OP == kLimitProject) wr = q.clipped ? 0x5 : 0x4;
#pragma unroll
    for (int k = 0; k < kTrPer; ++k) {
        const int64_t o = base + threadIdx.x + int64_t(k) * kTrThreads;
        if (o >= numel) break;
        float x[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) x[r] = (kRd >> r & 1) ? a.p[r][j][o] : 0.0f;
        tr_op<OP>(a, q, o, x);
#pragma unroll
        for (int r = 0; r < 4; ++r)
            if (wr >> r & 1) a.p[r][j][o] = x[r];
    }
}

// The list, in launches of at most TrArgsOf<OP>::kTensors tensors (empty tensors skipped).
template <int OP>
void tr_launch(TrArgsOf<OP>& a, float* const* const rows[kTrRows], const int64_t* numels, int n,
               hipStream_t st) {
    int j = 0;
    while (j < n) {
        int m = 0, chunks = 0;
        for (; j < n && m < TrArgsOf<OP>::kTensors; ++j) {
            if (numels[j] == 0) continue;
            for (int r = 0; r < kTrRows; ++r) a.p[r][m] = rows[r] ? rows[r][j] : nullptr;
            a.numel[m] = numels[j];
            a.chunk0[m] = chunks;
            const int64_t c = (numels[j] + kTrChunk - 1) / kTrChunk;
            HSN_REQUIRE(int64_t(chunks) + c < (int64_t(1) << 31), HSN_ERR_SIZE_OVERFLOW,
                        "trainer pass: a launch's tensors are too large");
            chunks += static_cast<int>(c);
            ++m;
        }
        if (m == 0) break;
        a.n = m;
        a.chunk0[m] = chunks;
        hipLaunchKernelGGL(tr_pass<OP>, dim3(chunks), dim3(kTrThreads), 0, st, a);
        HSN_HIP(hipGetLastError());
    }
}

void tr_check_list(const char* f, const int64_t* numels, int n) {
    HSN_REQUIRE(n >= 0 && (n == 0 || numels), HSN_ERR_INVALID_ARGUMENT,
                std::string(f) + ": bad tensor list");
    for (int j = 0; j < n; ++j)
        HSN_REQUIRE(numels[j] >= 0, HSN_ERR_INVALID_ARGUMENT,
                    std::string(f) + ": a tensor's element count is negative");
}

void tr_check_rows(const char* f, std::initializer_list<const void* const*> rows,
                   const int64_t* numels, int n) {
    for (const void* const* row : rows) {
        HSN_REQUIRE(n == 0 || row, HSN_ERR_INVALID_ARGUMENT,
                    std::string(f) + ": a required pointer list is NULL");
        for (int j = 0; j < n; ++j)  // an empty tensor's pointer may be NULL
            HSN_REQUIRE(row[j] != nullptr || numels[j] == 0, HSN_ERR_INVALID_ARGUMENT,
                        std::string(f) + ": a required tensor pointer is NULL");
    }
}

}  // namespace
}  // namespace hsn

using namespace hsn;

extern "C" int hsn_tr_adamw(float* const* params, float* const* grads, float* const* exp_avgs,
                            float* const* exp_avg_sqs, const int64_t* numels, int n,
                            int weight_decay_on, const float* coefs, void* stream) {
    HSN_ABI_BEGIN
    tr_check_list("hsn_tr_adamw", numels, n);
    tr_check_rows("hsn_tr_adamw",
                  {(const void* const*)params, (const void* const*)grads,
                   (const void* const*)exp_avgs, (const void* const*)exp_avg_sqs},
                  numels, n);
    HSN_REQUIRE(coefs != nullptr, HSN_ERR_INVALID_ARGUMENT, "hsn_tr_adamw: coefs is NULL");
    TrArgs a{};
    a.flag = weight_decay_on ? 1 : 0;
    for (int k = 0; k < 7; ++k) a.f[k] = coefs[k];
    float* const* const rows[kTrRows] = {params, grads, exp_avgs, exp_avg_sqs};
    tr_launch<kAdamW>(a, rows, numels, n, as_stream(stream));
    HSN_ABI_END
}

extern "C" int hsn_tr_adamw_units(float* const* params, float* const* grads,
                                  float* const* exp_avgs, float* const* exp_avg_sqs,
                                  const int64_t* numels, int n, int n_units, int weight_decay_on,
                                  const float* unit_coefs, float one_minus_beta2, float eps,
                                  void* stream) {
    HSN_ABI_BEGIN
    tr_check_list("hsn_tr_adamw_units", numels, n);
    tr_check_rows("hsn_tr_adamw_units",
                  {(const void* const*)params, (const void* const*)grads,
                   (const void* const*)exp_avgs, (const void* const*)exp_avg_sqs},
                  numels, n);
    HSN_REQUIRE(n_units >= 1 && n_units <= kTrUnits, HSN_ERR_INVALID_ARGUMENT,
                "hsn_tr_adamw_units: n_units must lie in [1, 64]");
    HSN_REQUIRE(unit_coefs != nullptr, HSN_ERR_INVALID_ARGUMENT,
                "hsn_tr_adamw_units: unit_coefs is NULL");
    for (int j = 0; j < n; ++j)
        HSN_REQUIRE(numels[j] % n_units == 0, HSN_ERR_INVALID_ARGUMENT,
                    "hsn_tr_adamw_units: a tensor's elements are not a whole number per unit");
    TrArgsUnits a{};
    a.flag = weight_decay_on ? 1 : 0;
    a.units = n_units;
    a.f[3] = one_minus_beta2;
    a.f[5] = eps;
    for (int c = 0; c < 6; ++c)
        for (int m = 0; m < n_units; ++m) a.u[c][m] = unit_coefs[c * n_units + m];
    float* const* const rows[kTrRows] = {params, grads, exp_avgs, exp_avg_sqs};
    tr_launch<kAdamWUnits>(a, rows, numels, n, as_stream(stream));
    HSN_ABI_END
}

extern "C" int hsn_tr_lerp(float* const* selfs, float* const* ends, const int64_t* numels, int n,
                           float weight, void* stream) {
    HSN_ABI_BEGIN
    tr_check_list("hsn_tr_lerp", numels, n);
    tr_check_rows("hsn_tr_lerp", {(const void* const*)selfs, (const void* const*)ends}, numels,
                  n);
    TrArgs a{};
    a.f[0] = weight;
    float* const* const rows[kTrRows] = {selfs, ends, nullptr, nullptr};
    tr_launch<kLerp>(a, rows, numels, n, as_stream(stream));
    HSN_ABI_END
}

extern "C" int hsn_tr_scale64(float* const* grads, const int64_t* numels, int n,
                              const double* coefficient, void* stream) {
    HSN_ABI_BEGIN
    tr_check_list("hsn_tr_scale64", numels, n);
    tr_check_rows("hsn_tr_scale64", {(const void* const*)grads}, numels, n);
    HSN_REQUIRE(coefficient != nullptr, HSN_ERR_INVALID_ARGUMENT,
                "hsn_tr_scale64: coefficient is NULL");
    TrArgs a{};
    a.coef = coefficient;
    float* const* const rows[kTrRows] = {grads, nullptr, nullptr, nullptr};
    tr_launch<kScale64>(a, rows, numels, n, as_stream(stream));
    HSN_ABI_END
}

extern "C" int hsn_tr_copy(float* const* dsts, float* const* srcs, const int64_t* numels, int n,
                           void* stream) {
    HSN_ABI_BEGIN
    tr_check_list("hsn_tr_copy", numels, n);
    tr_check_rows("hsn_tr_copy", {(const void* const*)dsts, (const void* const*)srcs}, numels, n);
    TrArgs a{};
    float* const* const rows[kTrRows] = {dsts, srcs, nullptr, nullptr};
    tr_launch<kCopy>(a, rows, numels, n, as_stream(stream));
    HSN_ABI_END
}

extern "C" int hsn_tr_limit_squares(float* const* params, float* const* olds,
                                    float* const* old_squares, float* const* delta_squares,
                                    const int64_t* numels, int n, void* stream) {
    HSN_ABI_BEGIN
    tr_check_list("hsn_tr_limit_squares", numels, n);
    tr_check_rows("hsn_tr_limit_squares",
                  {(const void* const*)params, (const void* const*)olds,
                   (const void* const*)old_squares, (const void* const*)delta_squares},
                  numels, n);
    TrArgs a{};
    float* const* const rows[kTrRows] = {params, olds, old_squares, delta_squares};
    tr_launch<kLimitSquares>(a, rows, numels, n, as_stream(stream));
    HSN_ABI_END
}

extern "C" int hsn_tr_limit_project(float* const* params, float* const* olds,
                                    float* const* applied_squares, float* const* groups,
                                    const int64_t* numels, int n, void* stream) {
    HSN_ABI_BEGIN
    tr_check_list("hsn_tr_limit_project", numels, n);
    tr_check_rows("hsn_tr_limit_project",
                  {(const void* const*)params, (const void* const*)olds,
                   (const void* const*)applied_squares, (const void* const*)groups},
                  numels, n);
    TrArgs a{};
    float* const* const rows[kTrRows] = {params, olds, applied_squares, groups};
    tr_launch<kLimitProject>(a, rows, numels, n, as_stream(stream));
    HSN_ABI_END
}
