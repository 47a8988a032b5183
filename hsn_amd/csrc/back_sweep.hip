// The state-gradient reverse sweep's glue steps on gfx950 (reference kernels/cuda/hsn_window.cu:
// 956-1427, hsn_win_back_head / _mid / _tail; their contract is python/hsn/train/state_sweep.py's
// head_reference, middle_reference and tail_reference). One position of the sweep is
// head -> product -> middle -> product -> tail, the products being the caller's GEMMs on the
// operands written here.
//
// Work per launch (B rows, K slots, d columns, H hidden units):
//   head    one workgroup per row, a wavefront per slot (slots k, k + 4, ...), lanes over the
//           columns (at most 4 a lane): the carry, dc / db, the candidate's and the gate's
//           backward, the operand rows. Two wavefront reductions per slot for the candidate norm
//           (mean y^2 and mean y * scaled) and one for the gate's part of sigma.
//   middle  a wavefront per slot row, lanes over H: the activation's derivative, the unit block of
//           op2, sigma's hidden part (one reduction).
//   tail    (row, cell range) workgroups: every workgroup rebuilds the row's slot-of-cell table and
//           the cells the position touches (the selected cells and their message sources) in
//           LDS, then updates its cells' rows of A in column order with the selected cells'
//           ds terms in the out-adjacency's order, a fixed summation order per element.
// These are launch- and latency-bound (a few MB a position); the products carry the FLOPs.
// The file keeps every operation separately rounded (no contraction), as the PyTorch glue does.
#include <string>

#include "../../include/hsn_ops.h"
#include "../../include/hsn_sweep.h"
#include "abi_util.h"
#include "common.cuh"

#pragma clang fp contract(off)

namespace hsn {
namespace {

constexpr int kBackThreads = 256;
constexpr int kBackWaves = kBackThreads / kWave;
constexpr int kMaxColsPerLane = 4;  // d <= 256
constexpr int kTailCells = 64;      // cells per tail workgroup
constexpr int kMaxLds = 64 * 1024;

template <typename P>
__device__ __forceinline__ float ld(const void* p, int64_t i) {
    return to_f32(static_cast<const P*>(p)[i]);
}
template <typename P>
__device__ __forceinline__ void st(void* p, int64_t i, float v) {
    static_cast<P*>(p)[i] = from_f32<P>(v);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += wave_shfl_xor(v, m);
    return v;
}

// state_gradient.activation_grad: the derivative of the cell's activation at x.
__device__ __forceinline__ float act_grad(int code, float x) {
    if (code == HSN_ACT_GELU) {
        const float cdf = 0.5f * (1.0f + erff(x / 1.41421356237309515f));
        return cdf + x * expf(-0.5f * x * x) / 2.50662827463100024f;
    }
    if (code == HSN_ACT_RELU) return x > 0.0f ? 1.0f : 0.0f;
    if (code == HSN_ACT_SILU) {
        const float s = 1.0f / (1.0f + expf(-x));
        return s * (1.0f + x * (1.0f - s));
    }
    const float th = tanhf(x);
    return 1.0f - th * th;
}

// ------------------------------------------------------------------------------------------
// head: the carry of position t and the candidate's and gate's backward
// ------------------------------------------------------------------------------------------
template <typename P>
__global__ __launch_bounds__(kBackThreads) void back_head(hsn_back_sweep s, int t) {
    const int row = blockIdx.x;
    const int tid = threadIdx.x;
    const int wave = tid / kWave, lane = tid % kWave;
    const int d = s.d, K = s.K, N = s.N;
    float* A = s.A + int64_t(row) * N * d;
    float* R = s.R + int64_t(row) * d;
    const int64_t bt = int64_t(row) * s.T + t;
    // R += d_q_post[t]; the fast cells' rows of A take the decoder's read of them
    for (int x = tid; x < d; x += kBackThreads) R[x] = R[x] + s.d_q_post[bt * d + x];
    if (s.n_read > 0) {
        const float* dh_fast = s.d_h_fast + bt * s.n_read * d;
        for (int i = tid; i < s.n_read * d; i += kBackThreads) A[i] = A[i] + dh_fast[i];
    }
    __syncthreads();
    for (int k = wave; k < K; k += kBackWaves) {
        const int64_t slot = bt * K + k;
        const int cell = s.slots[slot];
        const bool ok = cell >= 0 && cell < N;  // out of range reads as padded, never faults
        const int unit = min(max(s.units[slot], 0), s.M - 1);
        const float alpha = s.alpha[slot];
        const int64_t base = slot * d;
        float dgv[kMaxColsPerLane], yv[kMaxColsPerLane], scaled[kMaxColsPerLane];
        float sum_yy = 0.0f, sum_ys = 0.0f, sum_gate = 0.0f;
#pragma unroll
        for (int j = 0; j < kMaxColsPerLane; ++j) {
            const int x = lane + j * kWave;
            dgv[j] = yv[j] = scaled[j] = 0.0f;
            if (x >= d) continue;
            const float bx = s.b[base + x];
            const float cx = s.c[base + x];
            float dc = 0.0f, db = 0.0f;
            if (ok) {
                // A[cell] += d_h_sel; g = A[cell] + R / N
                const float carried = A[int64_t(cell) * d + x] + s.d_h_sel[base + x];
                const float share = R[x] / static_cast<float>(N);
                const float g = carried + share;
                dc = bx * g;
                db = (cx - s.h_old[base + x]) * g;
                A[int64_t(cell) * d + x] = (1.0f - bx) * carried - bx * share;
            }
            s.dc[base + x] = dc;
            s.db[base + x] = db;
            // the candidate: dz = dc (1 - c^2); the norm's scaled cotangent gain (alpha dz)
            const float dz = dc * (1.0f - cx * cx);
            if (s.cand_norm) {
                const float y = s.y[base + x];
                yv[j] = y;
                scaled[j] = s.cand_gain[x] * (alpha * dz);
                sum_yy += y * y;
                sum_ys += y * scaled[j];
            } else {
                scaled[j] = alpha * dz;
            }
            // the gate: dg = db b (1 - b); its part of sigma
            const float dg = db * bx * (1.0f - bx);
            dgv[j] = ok ? dg : 0.0f;
            if (ok) sum_gate += dgv[j] * (s.gate_pre[base + x] - s.gate_bias[x]);
        }
        float rho = 0.0f, mean_ys = 0.0f;
        if (s.cand_norm) {
            sum_yy = wave_sum(sum_yy);
            sum_ys = wave_sum(sum_ys);
            rho = 1.0f / sqrtf(sum_yy / static_cast<float>(d) + s.cand_eps);
            mean_ys = sum_ys / static_cast<float>(d);
        }
        sum_gate = wave_sum(sum_gate);
        if (lane == 0) s.sigma[int64_t(row) * K + k] = ok ? sum_gate : 0.0f;
        // operand rows: op1's unit block (the block of t + 1 cleared first), op2's gate columns
        const int64_t op_row = int64_t(row) * K + k;
        const int64_t w1 = int64_t(s.M) * d;
        const int64_t w2 = int64_t(s.M) * s.H + d;
        const int prev_unit = t + 1 < s.T ? min(max(s.units[slot + K], 0), s.M - 1) : -1;
#pragma unroll
        for (int j = 0; j < kMaxColsPerLane; ++j) {
            const int x = lane + j * kWave;
            if (x >= d) continue;
            float du;
            if (s.cand_norm) {
                const float rho3 = rho * rho * rho;
                du = rho * scaled[j] - rho3 * yv[j] * mean_ys;
            } else {
                du = scaled[j];
            }
            du = ok ? du : 0.0f;
            if (prev_unit >= 0) st<P>(s.op1, op_row * w1 + int64_t(prev_unit) * d + x, 0.0f);
            st<P>(s.op1, op_row * w1 + int64_t(unit) * d + x, du);
            st<P>(s.op2, op_row * w2 + int64_t(s.M) * s.H + x, dgv[j]);
        }
    }
}

// ------------------------------------------------------------------------------------------
// middle: the activation's derivative into op2's unit block, sigma's hidden part
// ------------------------------------------------------------------------------------------
template <typename P>
__global__ __launch_bounds__(kBackThreads) void back_mid(hsn_back_sweep s, int t) {
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    const int64_t op_row = int64_t(blockIdx.x) * kBackWaves + wave;  // row * K + k
    if (op_row >= int64_t(s.B) * s.K) return;
    const int row = static_cast<int>(op_row / s.K), k = static_cast<int>(op_row % s.K);
    const int64_t slot = (int64_t(row) * s.T + t) * s.K + k;
    const bool ok = s.slots[slot] >= 0 && s.slots[slot] < s.N;
    const int unit = min(max(s.units[slot], 0), s.M - 1);
    const int prev_unit = t + 1 < s.T ? min(max(s.units[slot + s.K], 0), s.M - 1) : -1;
    const int H = s.H;
    const int64_t w2 = int64_t(s.M) * H + s.d;
    float part = 0.0f;
    for (int h = lane; h < H; h += kWave) {
        const float hid = ld<P>(s.hidden, slot * H + h);
        float dh = 0.0f;
        if (ok) dh = ld<P>(s.act, op_row * H + h) * act_grad(s.activation, hid);
        if (ok) part += dh * (hid - s.b1[int64_t(unit) * H + h]);
        if (prev_unit >= 0) st<P>(s.op2, op_row * w2 + int64_t(prev_unit) * H + h, 0.0f);
        st<P>(s.op2, op_row * w2 + int64_t(unit) * H + h, dh);
    }
    part = wave_sum(part);
    if (lane == 0) s.sigma[int64_t(row) * s.K + k] = s.sigma[int64_t(row) * s.K + k] + part;
}

// ------------------------------------------------------------------------------------------
// tail: the cell norm's backward, the scatter into the cells and their messages' sources
// ------------------------------------------------------------------------------------------
struct TailLds {
    int slot_of, touched, dsh, dvm, bytes;
};
__host__ __device__ inline TailLds tail_lds(int N, int K, int d) {
    TailLds L;
    L.slot_of = 0;                          // int [N]
    L.touched = L.slot_of + 4 * N;          // int [N]
    L.dsh = L.touched + 4 * N;              // float [K, d]
    L.dvm = L.dsh + 4 * K * d;              // float [K, d]
    L.bytes = L.dvm + 4 * K * d;
    return L;
}

template <typename P>
__global__ __launch_bounds__(kBackThreads) void back_tail(hsn_back_sweep s, int t) {
    extern __shared__ __align__(16) unsigned char lds[];
    const int row = blockIdx.y;
    const int cell0 = blockIdx.x * kTailCells;
    const int tid = threadIdx.x;
    const int wave = tid / kWave, lane = tid % kWave;
    const int d = s.d, K = s.K, N = s.N;
    const TailLds L = tail_lds(N, K, d);
    int* slot_of = reinterpret_cast<int*>(lds + L.slot_of);
    int* touched = reinterpret_cast<int*>(lds + L.touched);
    float* dsh = reinterpret_cast<float*>(lds + L.dsh);
    float* dvm = reinterpret_cast<float*>(lds + L.dvm);
    const int64_t bt = int64_t(row) * s.T + t;
    const bool reset = s.reset[bt] != 0;
    float* A = s.A + int64_t(row) * N * d;
    const int cell_end = min(cell0 + kTailCells, N);
    if (reset) {  // the row restarts: its cotangent before position t is zero
        for (int64_t i = int64_t(cell0) * d + tid; i < int64_t(cell_end) * d; i += kBackThreads)
            A[i] = 0.0f;
        if (blockIdx.x == 0)
            for (int x = tid; x < d; x += kBackThreads) s.R[int64_t(row) * d + x] = 0.0f;
        return;
    }
    for (int n = tid; n < N; n += kBackThreads) {
        slot_of[n] = -1;
        touched[n] = 0;
    }
    __syncthreads();
    // the selected cells and their message sources; each slot's ds = [ds_h ; ds_m]
    for (int k = wave; k < K; k += kBackWaves) {
        const int64_t slot = bt * K + k;
        const int cell = s.slots[slot];
        const bool ok = cell >= 0 && cell < N;
        if (ok && lane == 0) {
            slot_of[cell] = k;
            touched[cell] = 1;
        }
        if (ok)
            for (int e = lane; e < s.d_in; e += kWave) {
                const int src = s.in_src[int64_t(cell) * s.d_in + e];
                if (src >= 0 && src < N) touched[src] = 1;
            }
        const int64_t op_row = int64_t(row) * K + k;
        float r = 0.0f, back = 0.0f;
        if (s.cell_norm) {
            r = s.rms[slot];
            back = (r * r / static_cast<float>(s.in_dim)) * s.sigma[op_row];
        }
        for (int x = lane; x < d; x += kWave) {
            float h = ld<P>(s.dv, op_row * 2 * d + x);
            float m = ld<P>(s.dv, op_row * 2 * d + d + x);
            if (s.cell_norm) {
                h = r * h - back * s.h_old[slot * d + x];
                m = r * m - back * s.mv[slot * d + x];
            }
            dsh[k * d + x] = ok ? h : 0.0f;
            dvm[k * d + x] = ok ? m : 0.0f;
        }
    }
    __syncthreads();
    // A[n] (+ ds_h of its slot) + sum_j w_nj ds_m[slot of target_j], in j's order
    for (int i = tid; i < (cell_end - cell0) * d; i += kBackThreads) {
        const int n = cell0 + i / d, x = i % d;
        if (!touched[n]) continue;
        float a = A[int64_t(n) * d + x];
        const int own = slot_of[n];
        if (own >= 0) a = a + dsh[own * d + x];
        for (int j = 0; j < s.d_out; ++j) {
            const int target = s.out_tgt[int64_t(n) * s.d_out + j];
            const int k = target >= 0 && target < N ? slot_of[target] : -1;
            const float add = k >= 0 ? s.out_w[int64_t(n) * s.d_out + j] * dvm[k * d + x] : 0.0f;
            a = a + add;
        }
        A[int64_t(n) * d + x] = a;
    }
    if (blockIdx.x == 0)
        for (int x = tid; x < d; x += kBackThreads)
            s.R[int64_t(row) * d + x] = s.R[int64_t(row) * d + x] + s.d_q_pre[bt * d + x];
}

void back_check(const hsn_back_sweep* s) {
    HSN_REQUIRE(s != nullptr, HSN_ERR_INVALID_ARGUMENT, "hsn_back_sweep: NULL");
    HSN_REQUIRE(s->B >= 1 && s->T >= 1 && s->K >= 1 && s->N >= 1 && s->d >= 1 && s->H >= 1 &&
                    s->M >= 1,
                HSN_ERR_INVALID_ARGUMENT, "reverse sweep: every size must be positive");
    HSN_REQUIRE(s->d <= kMaxColsPerLane * kWave, HSN_ERR_INVALID_ARGUMENT,
                "reverse sweep: model.d above 256 (four columns a lane)");
    HSN_REQUIRE(s->n_read >= 0 && s->n_read <= s->N, HSN_ERR_INVALID_ARGUMENT,
                "reverse sweep: n_read outside [0, N]");
    HSN_REQUIRE(s->n_read == 0 || s->d_h_fast != nullptr, HSN_ERR_INVALID_ARGUMENT,
                "reverse sweep: d_h_fast is NULL with fast-read cells");
    HSN_REQUIRE(s->d_out >= 1 && s->d_in >= 1, HSN_ERR_INVALID_ARGUMENT,
                "reverse sweep: the adjacency widths must be positive");
    HSN_REQUIRE(s->product_dtype == HSN_DTYPE_F32 || s->product_dtype == HSN_DTYPE_BF16,
                HSN_ERR_UNSUPPORTED_DTYPE, "reverse sweep: products in f32 or bf16 only");
    HSN_REQUIRE(s->activation >= HSN_ACT_GELU && s->activation <= HSN_ACT_TANH,
                HSN_ERR_INVALID_ARGUMENT, "reverse sweep: unknown activation");
    HSN_REQUIRE(!s->cell_norm || (s->rms != nullptr && s->mv != nullptr && s->in_dim > 0),
                HSN_ERR_INVALID_ARGUMENT, "reverse sweep: the cell norm needs rms, m V, in_dim");
    HSN_REQUIRE(!s->cand_norm || (s->y != nullptr && s->cand_gain != nullptr),
                HSN_ERR_INVALID_ARGUMENT, "reverse sweep: the candidate norm needs y, its gain");
    HSN_REQUIRE(tail_lds(s->N, s->K, s->d).bytes <= kMaxLds, HSN_ERR_INVALID_ARGUMENT,
                "reverse sweep: a row's slot table and slot terms (8 N + 8 K d bytes) exceed "
                "64 KiB of LDS");
    const int64_t elems = int64_t(s->B) * s->T * s->K * s->H;
    HSN_REQUIRE(check_elems({int64_t(s->B) * s->N * s->d, elems,
                             int64_t(s->B) * s->K * (int64_t(s->M) * s->H + s->d)}),
                HSN_ERR_SIZE_OVERFLOW, "reverse sweep: a buffer is too large");
    const void* need[] = {s->A, s->R, s->sigma, s->c, s->b, s->h_old, s->gate_pre, s->alpha,
                          s->hidden, s->slots, s->units, s->reset, s->d_q_pre, s->d_q_post,
                          s->d_h_sel, s->gate_bias, s->b1, s->out_tgt, s->out_w, s->in_src,
                          s->op1, s->op2, s->act, s->dv, s->dc, s->db};
    for (const void* p : need)
        HSN_REQUIRE(p != nullptr, HSN_ERR_INVALID_ARGUMENT, "reverse sweep: a buffer is NULL");
}

void check_t(const hsn_back_sweep* s, int t) {
    HSN_REQUIRE(t >= 0 && t < s->T, HSN_ERR_INVALID_ARGUMENT, "reverse sweep: t outside [0, T)");
}

}  // namespace
}  // namespace hsn

using namespace hsn;

extern "C" int hsn_win_back_check(const hsn_back_sweep* sweep) {
    HSN_ABI_BEGIN
    back_check(sweep);
    HSN_ABI_END
}

extern "C" int hsn_win_back_head(const hsn_back_sweep* sweep, int t, void* stream) {
    HSN_ABI_BEGIN
    back_check(sweep);
    check_t(sweep, t);
    const hsn_back_sweep s = *sweep;
    if (s.product_dtype == HSN_DTYPE_BF16)
        hipLaunchKernelGGL(back_head<bf16_t>, dim3(s.B), dim3(kBackThreads), 0, as_stream(stream),
                           s, t);
    else
        hipLaunchKernelGGL(back_head<float>, dim3(s.B), dim3(kBackThreads), 0, as_stream(stream),
                           s, t);
    HSN_HIP(hipGetLastError());
    HSN_ABI_END
}

extern "C" int hsn_win_back_mid(const hsn_back_sweep* sweep, int t, void* stream) {
    HSN_ABI_BEGIN
    back_check(sweep);
    check_t(sweep, t);
    const hsn_back_sweep s = *sweep;
    const int64_t rows = int64_t(s.B) * s.K;
    const dim3 grid(static_cast<unsigned>((rows + kBackWaves - 1) / kBackWaves));
    if (s.product_dtype == HSN_DTYPE_BF16)
        hipLaunchKernelGGL(back_mid<bf16_t>, grid, dim3(kBackThreads), 0, as_stream(stream), s, t);
    else
        hipLaunchKernelGGL(back_mid<float>, grid, dim3(kBackThreads), 0, as_stream(stream), s, t);
    HSN_HIP(hipGetLastError());
    HSN_ABI_END
}

extern "C" int hsn_win_back_tail(const hsn_back_sweep* sweep, int t, void* stream) {
    HSN_ABI_BEGIN
    back_check(sweep);
    check_t(sweep, t);
    const hsn_back_sweep s = *sweep;
    const dim3 grid(static_cast<unsigned>((s.N + kTailCells - 1) / kTailCells),
                    static_cast<unsigned>(s.B));
    const size_t lds = static_cast<size_t>(tail_lds(s.N, s.K, s.d).bytes);
    if (s.product_dtype == HSN_DTYPE_BF16)
        hipLaunchKernelGGL(back_tail<bf16_t>, grid, dim3(kBackThreads), lds, as_stream(stream), s,
                           t);
    else
        hipLaunchKernelGGL(back_tail<float>, grid, dim3(kBackThreads), lds, as_stream(stream), s,
                           t);
    HSN_HIP(hipGetLastError());
    HSN_ABI_END
}
