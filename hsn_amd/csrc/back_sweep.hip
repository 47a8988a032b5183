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
#include "dpp.cuh"

#pragma clang fp contract(off)

namespace hsn {
// Raise a kernel's dynamic-LDS limit to 160 KiB once per (kernel, device) (runtime.cpp).
hipError_t allow_lds_raw(const void* kernel, size_t lds);

namespace {

constexpr int kBackThreads = 256;
constexpr int kBackWaves = kBackThreads / kWave;
constexpr int kMaxColsPerLane = 4;  // d <= 256
constexpr int kTailCells = 64;      // cells per tail workgroup
constexpr int kMaxLds = 64 * 1024;
constexpr int kCellMaxLds = 160 * 1024;  // the fused step raises its kernels' dynamic-LDS limit

template <typename P>
__device__ __forceinline__ float ld(const void* p, int64_t i) {
    return to_f32(static_cast<const P*>(p)[i]);
}
template <typename P>
__device__ __forceinline__ void st(void* p, int64_t i, float v) {
    static_cast<P*>(p)[i] = from_f32<P>(v);
}

// The wavefront's sum in every lane: DPP within the rows, permlane swaps across them (no LDS).
__device__ __forceinline__ float wave_sum(float v) { return group_sum<kWave>(v); }

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
        for (int x = tid; x < d; x += kBackThreads) {
            s.R[int64_t(row) * d + x] = s.R[int64_t(row) * d + x] + s.d_q_pre[bt * d + x];
        }
}

// ------------------------------------------------------------------------------------------
// back_cell: head, both products and middle for 16 slots of one unit on the matrix cores
// ------------------------------------------------------------------------------------------
typedef float v4f __attribute__((ext_vector_type(4)));
typedef __bf16 bf8 __attribute__((ext_vector_type(8)));

constexpr int kCellRows = 16;  // slots per workgroup: the MFMA tile's rows
constexpr int kCellCols = 16;  // dv columns per workgroup: one MFMA tile's columns
constexpr int kCellThreads = 512;
constexpr int kCellWaves = kCellThreads / kWave;
constexpr int kCellMaxCpl = 2;  // d <= 128 on the fused step
constexpr int kDvChunk = 4;     // dv reduction steps whose loads a wavefront issues together

// act column tiles whose loads a wavefront issues together: at most 64 registers of weights
template <typename P, int CPL>
constexpr int act_tiles() {
    return sizeof(P) == 2 ? 4 : (CPL == 1 ? 4 : 2);
}

// The MFMA tile of a product dtype. Lane l supplies A[l % 16][kq .. kq + kPer) and
// B[kq .. kq + kPer)[l % 16] with kq = kPer (l / 16), and receives D[4 (l / 16) + r][l % 16] in
// result register r; a step covers kStep of the reduction index (the lane layout checked on the
// card for both instructions).
template <typename P>
struct Tile;
template <>
struct Tile<bf16_t> {  // v_mfma_f32_16x16x32_bf16
    static constexpr int kPer = 8, kStep = 32;
    typedef bf8 frag;
    static __device__ __forceinline__ frag lds(const bf16_t* p) {
        return *reinterpret_cast<const bf8*>(p);
    }
    static __device__ __forceinline__ frag glb(const bf16_t* p, bool ok) {
        if (!ok) return frag{};
        return *reinterpret_cast<const bf8*>(p);
    }
    static __device__ __forceinline__ v4f mma(frag a, frag b, v4f c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
    }
};
template <>
struct Tile<float> {  // v_mfma_f32_16x16x4_f32
    static constexpr int kPer = 1, kStep = 4;
    typedef float frag;
    static __device__ __forceinline__ frag lds(const float* p) { return *p; }
    static __device__ __forceinline__ frag glb(const float* p, bool ok) { return ok ? *p : 0.0f; }
    static __device__ __forceinline__ v4f mma(frag a, frag b, v4f c) {
        return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
    }
};

// The activation's derivative with the activation fixed at compile time (one branch of code),
// with products by reciprocal constants and exp from the hardware's exp2 (a few ulps; the exact
// divisions and the correctly rounded expf cost more instructions than the rest of the step's
// epilogue): Phi(x) + x phi(x) for the exact GELU, s (1 + x (1 - s)) for SiLU, 1 - tanh^2.
constexpr float kRsqrt2f = 0.70710678118654752f;
constexpr float kRsqrt2Pif = 0.39894228040143268f;
constexpr float kLog2ef = 1.44269504088896341f;
__device__ __forceinline__ float exp_fast(float x) {
    return __builtin_amdgcn_exp2f(x * kLog2ef);
}
template <int ACT>
__device__ __forceinline__ float act_grad_t(float x) {
    if constexpr (ACT == HSN_ACT_GELU) {
        const float cdf = 0.5f * (1.0f + erff(x * kRsqrt2f));
        return cdf + x * (exp_fast(-0.5f * x * x) * kRsqrt2Pif);
    } else if constexpr (ACT == HSN_ACT_RELU) {
        return x > 0.0f ? 1.0f : 0.0f;
    } else if constexpr (ACT == HSN_ACT_SILU) {
        const float sg = __builtin_amdgcn_rcpf(1.0f + exp_fast(-x));
        return sg * (1.0f + x * (1.0f - sg));
    } else {
        const float th = tanhf(x);
        return 1.0f - th * th;
    }
}

__host__ __device__ inline int round_up(int x, int m) { return (x + m - 1) / m * m; }

constexpr int kCellMaxSlots = 4096;  // B K on the fused step: the position's slots in LDS

struct CellLds {
    int rows, meta, sig_part, sig_gate, sig_row, red, ucache, ccache, hid, du, dh, du_stride,
        dh_stride, bytes;
};
template <typename P>
__host__ __device__ inline CellLds cell_lds(int d, int H, int BK) {
    constexpr int kStep = sizeof(P) == 2 ? 32 : 4;
    CellLds L;
    L.du_stride = round_up(d, kStep) + 8;  // + 8 elements: consecutive rows off the same banks
    L.dh_stride = round_up(H + d, kStep) + 8;
    L.rows = 0;                                            // int [16]
    L.meta = L.rows + 4 * kCellRows;                       // int [4]
    L.sig_part = L.meta + 16;                              // float [8][16]
    L.sig_gate = L.sig_part + 4 * kCellWaves * kCellRows;  // float [16]
    L.sig_row = L.sig_gate + 4 * kCellRows;                // float [16]
    L.red = L.sig_row + 4 * kCellRows;                     // float [8][64][4]
    L.ucache = L.red + 4 * kCellWaves * kWave * 4;         // uint8 [B K]: each slot's unit
    L.ccache = round_up(L.ucache + BK, 16);                // int [B K]: each slot's cell
    L.hid = round_up(L.ccache + 4 * BK, 16);               // P [16][H]: the rows' hidden values
    L.du = round_up(L.hid + static_cast<int>(sizeof(P)) * kCellRows * H, 16);  // P [16][du_stride]
    L.dh = L.du + round_up(static_cast<int>(sizeof(P)) * kCellRows * L.du_stride, 16);
    L.bytes = L.dh + static_cast<int>(sizeof(P)) * kCellRows * L.dh_stride;
    return L;
}

template <typename P>
__device__ __forceinline__ float round_p(float v) {
    return to_f32(from_f32<P>(v));
}

__device__ __forceinline__ int64_t slot_at(const hsn_back_sweep& s, int t, int q) {
    return (int64_t(q / s.K) * s.T + t) * s.K + q % s.K;
}

// Grid (ceil(B K / 16) + M, 1, 2d / 16): the row tiles of every unit's slots at position t (in
// slot order q = b K + k), 16 slots a tile, laid end to end unit after unit (at most
// ceil(B K / 16) + M of them; a workgroup past the last exits); workgroup (i, 0, ct) takes row
// tile i and dv's columns 16 ct .. 16 ct + 15. Every workgroup of a row tile computes the head and
// act of its slots (act is a quarter of the FLOPs); the ct = 0 one writes their dc, db, sigma and
// carry. A is only read here.
//
// Latency is what bounds a position (a few MB of traffic, microseconds of arithmetic): the
// position's units and cells come into LDS in one round trip, then every load of the head, of
// act's first batch (weights, hidden values, biases) and of dv's weights is issued before the
// head's arithmetic, and the reductions are DPP / permlane (no LDS round trips).
template <typename P, int CPL, int ACT>
__global__ __launch_bounds__(kCellThreads) void back_cell(hsn_back_sweep s, int t) {
    extern __shared__ __align__(16) unsigned char lds[];
    using TL = Tile<P>;
    using frag = typename TL::frag;
    constexpr int kActSteps = TL::kStep == 32 ? 2 * CPL : 16 * CPL;  // d <= 64 CPL
    constexpr int kActTiles = act_tiles<P, CPL>();
    constexpr int R = kCellRows / kCellWaves;  // head rows per wavefront
    const int ct = blockIdx.z;
    const bool lead = ct == 0;
    const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
    const int lr = lane & 15, lq = lane >> 4;
    const int d = s.d, K = s.K, N = s.N, H = s.H, M = s.M;
    const int BK = s.B * K;
    const CellLds L = cell_lds<P>(d, H, BK);
    int* rows = reinterpret_cast<int*>(lds + L.rows);
    int* meta = reinterpret_cast<int*>(lds + L.meta);
    float* sig_part = reinterpret_cast<float*>(lds + L.sig_part);
    float* sig_gate = reinterpret_cast<float*>(lds + L.sig_gate);
    float* sig_row = reinterpret_cast<float*>(lds + L.sig_row);
    float* red = reinterpret_cast<float*>(lds + L.red);
    uint8_t* ucache = lds + L.ucache;
    int* ccache = reinterpret_cast<int*>(lds + L.ccache);
    P* hid_lds = reinterpret_cast<P*>(lds + L.hid);
    P* du = reinterpret_cast<P*>(lds + L.du);
    P* dh = reinterpret_cast<P*>(lds + L.dh);

    // ---- the position's units and cells; which unit's which row tile this workgroup takes ----
    for (int q = tid; q < BK; q += kCellThreads) {
        const int64_t slot = slot_at(s, t, q);
        ucache[q] = static_cast<uint8_t>(min(max(s.units[slot], 0), M - 1));
        const int cell = s.slots[slot];
        ccache[q] = cell >= 0 && cell < N ? cell : -1;
    }
    __syncthreads();
    if (wave == 0) {
        int tiles_before = 0, unit = -1, tile = 0;
        for (int j = 0; j < M && unit < 0; ++j) {
            int cnt = 0;
            for (int q0 = 0; q0 < BK; q0 += kWave)
                cnt += __popcll(ballot(q0 + lane < BK && ucache[q0 + lane] == j));
            const int tiles = (cnt + kCellRows - 1) / kCellRows;
            if (static_cast<int>(blockIdx.x) < tiles_before + tiles) {
                unit = j;
                tile = blockIdx.x - tiles_before;
            }
            tiles_before += tiles;
        }
        if (lane < kCellRows) rows[lane] = -1;
        if (unit >= 0) {
            const int first = tile * kCellRows;
            int base = 0;
            for (int q0 = 0; q0 < BK && base < first + kCellRows; q0 += kWave) {
                const int q = q0 + lane;
                const bool mine = q < BK && ucache[q] == unit;
                const uint64_t m = ballot(mine);
                const int rank = base + lanes_below(m);
                if (mine && rank >= first && rank < first + kCellRows) rows[rank - first] = q;
                base += __popcll(m);
            }
        }
        if (lane == 0) meta[0] = unit;
    }
    __syncthreads();
    const int j = meta[0];
    if (j < 0) return;  // past the last tile (uniform)

    // ---- every load up to the products: the head's rows, act's first batch, dv's weights ----
    float vb[R][CPL], vc[R][CPL], vh[R][CPL], vs[R][CPL], vy[R][CPL], vg[R][CPL];
    float va[R][CPL], vf[R][CPL], vr[R][CPL], gain[CPL], gbias[CPL];
    int64_t slotv[R];
    bool okv[R], fastv[R];
    float alv[R];
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
        const int x = lane + c * kWave;
        gain[c] = x < d && s.cand_norm ? s.cand_gain[x] : 0.0f;
        gbias[c] = x < d ? s.gate_bias[x] : 0.0f;
    }
#pragma unroll
    for (int i = 0; i < R; ++i) {
        const int q = rows[R * wave + i];
        slotv[i] = q >= 0 ? slot_at(s, t, q) : 0;
        const int cell = q >= 0 ? ccache[q] : -1;
        okv[i] = cell >= 0;
        fastv[i] = okv[i] && cell < s.n_read;
        alv[i] = q >= 0 ? s.alpha[slotv[i]] : 0.0f;
        const int b = q >= 0 ? q / K : 0;
        const int64_t bt = int64_t(b) * s.T + t;
        const int64_t base = slotv[i] * d;
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            const int x = lane + c * kWave;
            const bool in = q >= 0 && x < d;
            vb[i][c] = in ? s.b[base + x] : 0.0f;
            vc[i][c] = in ? s.c[base + x] : 0.0f;
            vh[i][c] = in ? s.h_old[base + x] : 0.0f;
            vs[i][c] = in ? s.d_h_sel[base + x] : 0.0f;
            vg[i][c] = in ? s.gate_pre[base + x] : 0.0f;
            vy[i][c] = in && s.cand_norm ? s.y[base + x] : 0.0f;
            va[i][c] = in && okv[i] ? s.A[(int64_t(b) * N + cell) * d + x] : 0.0f;
            vf[i][c] = in && fastv[i] ? s.d_h_fast[(bt * s.n_read + cell) * d + x] : 0.0f;
            vr[i][c] = in ? s.R[int64_t(b) * d + x] + s.d_q_post[bt * d + x] : 0.0f;
        }
    }
    int qrow[4];
    bool okrow[4];
    int64_t srow[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        qrow[i] = rows[4 * lq + i];
        srow[i] = qrow[i] >= 0 ? slot_at(s, t, qrow[i]) : 0;
        okrow[i] = qrow[i] >= 0 && ccache[qrow[i]] >= 0;
    }
    const int ka = round_up(d, TL::kStep);
    const int steps = ka / TL::kStep;
    const P* w2 = static_cast<const P*>(s.w2f) + int64_t(j) * H * d;
    const P* hidden = static_cast<const P*>(s.hidden);
    // the tile's hidden rows, 16 bytes a thread per load (H * sizeof(P) % 16 == 0: H % 8 == 0)
    constexpr int kHidPer = 16 / static_cast<int>(sizeof(P));
    constexpr int kHidLoads = 2;  // per thread per batch
    typedef uint32_t u4 __attribute__((ext_vector_type(4)));
    const int hid_chunks = kCellRows * H / kHidPer;
    u4 hv[kHidLoads];
    auto load_hid = [&](int c0) {
#pragma unroll
        for (int u = 0; u < kHidLoads; ++u) {
            const int c = c0 + u * kCellThreads + tid;
            hv[u] = u4{0u, 0u, 0u, 0u};
            if (c < hid_chunks) {
                const int r = c / (H / kHidPer), e = (c % (H / kHidPer)) * kHidPer;
                const int q = rows[r];
                if (q >= 0 && ccache[q] >= 0)
                    hv[u] = *reinterpret_cast<const u4*>(hidden + slot_at(s, t, q) * H + e);
            }
        }
    };
    auto store_hid = [&](int c0) {
#pragma unroll
        for (int u = 0; u < kHidLoads; ++u) {
            const int c = c0 + u * kCellThreads + tid;
            if (c < hid_chunks) *reinterpret_cast<u4*>(hid_lds + c * kHidPer) = hv[u];
        }
    };
    load_hid(0);
    frag bf[kActTiles][kActSteps];
    float bias[kActTiles];
    auto load_act = [&](int c00) {
#pragma unroll
        for (int u = 0; u < kActTiles; ++u) {
            const int h = c00 + 16 * kCellWaves * u + lr;
            const bool hin = h < H;
#pragma unroll
            for (int st = 0; st < kActSteps; ++st) {
                const int kq = st * TL::kStep + TL::kPer * lq;
                bf[u][st] = TL::glb(w2 + int64_t(hin ? h : 0) * d + kq,
                                    st < steps && hin && kq < d);
            }
            bias[u] = hin ? s.b1[int64_t(j) * H + h] : 0.0f;
        }
    };
    load_act(16 * wave);
    const int kt = H + d;
    const int dv_steps = round_up(kt, TL::kStep) / TL::kStep;
    const int col = ct * kCellCols + lr;
    const bool cin = col < 2 * d;
    const P* w1 = static_cast<const P*>(s.w1f) + (int64_t(j) * 2 * d + (cin ? col : 0)) * kt;
    frag bv[kDvChunk];
    auto load_dv = [&](int s0) {
#pragma unroll
        for (int u = 0; u < kDvChunk; ++u) {
            const int st = s0 + u * kCellWaves;
            const int kq = st * TL::kStep + TL::kPer * lq;
            bv[u] = TL::glb(w1 + kq, st < dv_steps && cin && kq < kt);
        }
    };
    load_dv(wave);

    // ---- head: the carry, dc / db, the candidate's and the gate's backward ----
#pragma unroll
    for (int i = 0; i < R; ++i) {
        const int r = R * wave + i;
        const int q = rows[r];
        P* du_row = du + r * L.du_stride;
        P* dg_row = dh + r * L.dh_stride + H;
        const bool ok = okv[i];
        float dgv[CPL], scaled[CPL];
        float sum_yy = 0.0f, sum_ys = 0.0f, sum_gate = 0.0f;
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            const int x = lane + c * kWave;
            dgv[c] = scaled[c] = 0.0f;
            if (q < 0 || x >= d) continue;
            const float bx = vb[i][c], cx = vc[i][c];
            float dc = 0.0f, db = 0.0f;
            if (ok) {
                float a = va[i][c];
                if (fastv[i]) a = a + vf[i][c];  // the decoder's read of a fast cell
                const float carried = a + vs[i][c];
                const float share = vr[i][c] / static_cast<float>(N);
                const float g = carried + share;
                dc = bx * g;
                db = (cx - vh[i][c]) * g;
                if (lead) s.carry[int64_t(q) * d + x] = (1.0f - bx) * carried - bx * share;
            }
            if (lead) {
                s.dc[slotv[i] * d + x] = dc;
                s.db[slotv[i] * d + x] = db;
            }
            const float dz = dc * (1.0f - cx * cx);
            if (s.cand_norm) {
                scaled[c] = gain[c] * (alv[i] * dz);
                sum_yy += vy[i][c] * vy[i][c];
                sum_ys += vy[i][c] * scaled[c];
            } else {
                scaled[c] = alv[i] * dz;
            }
            const float dg = db * bx * (1.0f - bx);
            dgv[c] = ok ? dg : 0.0f;
            if (ok) sum_gate += dgv[c] * (vg[i][c] - gbias[c]);
        }
        float rho = 0.0f, mean_ys = 0.0f;
        if (s.cand_norm) {
            sum_yy = wave_sum(sum_yy);
            sum_ys = wave_sum(sum_ys);
            rho = 1.0f / sqrtf(sum_yy / static_cast<float>(d) + s.cand_eps);
            mean_ys = sum_ys / static_cast<float>(d);
        }
        sum_gate = wave_sum(sum_gate);
        if (lane == 0) sig_gate[r] = ok ? sum_gate : 0.0f;
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            const int x = lane + c * kWave;
            if (x >= d) continue;
            float v = scaled[c];
            if (s.cand_norm) v = rho * scaled[c] - rho * rho * rho * vy[i][c] * mean_ys;
            du_row[x] = from_f32<P>(ok ? v : 0.0f);
            dg_row[x] = from_f32<P>(dgv[c]);
        }
        for (int x = d + lane; x < L.du_stride; x += kWave) du_row[x] = from_f32<P>(0.0f);
        for (int x = d + lane; x < L.dh_stride - H; x += kWave) dg_row[x] = from_f32<P>(0.0f);
    }
    store_hid(0);  // the first batch was in flight under the head
    for (int c0 = kHidLoads * kCellThreads; c0 < hid_chunks; c0 += kHidLoads * kCellThreads) {
        load_hid(c0);
        store_hid(c0);
    }
    __syncthreads();

    // ---- act = du . (W_out W2_j^T); dh = act'(hidden) act; sigma's hidden part ----
    float part[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int c00 = 16 * wave; c00 < H; c00 += 16 * kCellWaves * kActTiles) {
        if (c00 != 16 * wave) load_act(c00);  // the first batch is in flight already
#pragma unroll
        for (int u = 0; u < kActTiles; ++u) {
            const int h = c00 + 16 * kCellWaves * u + lr;
            const bool hin = h < H;
            v4f acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int st = 0; st < kActSteps; ++st)
                if (st < steps)
                    acc = TL::mma(
                        TL::lds(du + lr * L.du_stride + st * TL::kStep + TL::kPer * lq),
                        bf[u][st], acc);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                float v = 0.0f;
                if (okrow[i] && hin) {
                    const float hv1 = to_f32(hid_lds[(4 * lq + i) * H + h]);
                    v = round_p<P>(acc[i]) * act_grad_t<ACT>(hv1);
                    part[i] += v * (hv1 - bias[u]);
                }
                if (hin) dh[(4 * lq + i) * L.dh_stride + h] = from_f32<P>(v);
            }
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {  // the 16 lanes of a row group hold the same rows
        const float v = group_sum<16>(part[i]);
        if (lr == 0) sig_part[wave * kCellRows + 4 * lq + i] = v;
    }
    // the ds epilogue's operands, in flight under the dv product
    float rms4[4], st4[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        rms4[i] = 0.0f;
        st4[i] = 0.0f;
        if (wave == 0 && s.cell_norm && qrow[i] >= 0 && cin) {
            rms4[i] = s.rms[srow[i]];
            st4[i] = col < d ? s.h_old[srow[i] * d + col] : s.mv[srow[i] * d + col - d];
        }
    }
    __syncthreads();
    if (tid < kCellRows) {
        float sg = sig_gate[tid];
        for (int w = 0; w < kCellWaves; ++w) sg = sg + sig_part[w * kCellRows + tid];
        sig_row[tid] = sg;
        if (lead && rows[tid] >= 0) s.sigma[rows[tid]] = sg;
    }

    // ---- dv's column tile ct = [dh ; dg] . w1f_j; the reduction split over the wavefronts ----
    v4f acc = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int s0 = wave; s0 < dv_steps; s0 += kCellWaves * kDvChunk) {
        if (s0 != wave) load_dv(s0);  // the first chunk is in flight already
#pragma unroll
        for (int u = 0; u < kDvChunk; ++u) {
            const int st = s0 + u * kCellWaves;
            if (st < dv_steps)
                acc = TL::mma(TL::lds(dh + lr * L.dh_stride + st * TL::kStep + TL::kPer * lq),
                              bv[u], acc);
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) red[(wave * kWave + lane) * 4 + i] = acc[i];
    __syncthreads();
    if (wave == 0) {
        // the product's value as the reference's product dtype stores it, then the cell norm's
        // backward: ds = r dv - (r^2 / in_dim) sigma [h_old ; m V] (ds = dv without the norm)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float v = red[lane * 4 + i];
            for (int w = 1; w < kCellWaves; ++w) v = v + red[(w * kWave + lane) * 4 + i];
            if (qrow[i] < 0 || !cin) continue;
            v = round_p<P>(v);
            if (s.cell_norm) {
                const float r = rms4[i];
                const float back = (r * r / static_cast<float>(s.in_dim)) * sig_row[4 * lq + i];
                v = r * v - back * st4[i];
            }
            s.ds[int64_t(qrow[i]) * 2 * d + col] = okrow[i] ? v : 0.0f;
        }
    }
}

// ------------------------------------------------------------------------------------------
// back_cell_tail: the tail after back_cell, a wavefront per touched cell
// ------------------------------------------------------------------------------------------
constexpr int kCellTailCells = 32;  // cells per workgroup

struct CellTailLds {
    int slot_of, ds, carry, bytes;
};
__host__ __device__ inline CellTailLds cell_tail_lds(int N, int K, int d, int d_out) {
    (void)d_out;
    CellTailLds L;
    L.slot_of = 0;                           // int [N]
    L.ds = round_up(L.slot_of + 4 * N, 16);  // float [K][2d]
    L.carry = L.ds + 4 * K * 2 * d;          // float [K][d]
    L.bytes = L.carry + 4 * K * d;
    return L;
}

// Grid (N / 32, B): workgroup (i, b) updates row b's cells 32 i .. 32 i + 31, a wavefront per
// cell (cells w, w + 4, ...), a lane per column and per out-edge. Every load it needs is issued at
// once (its cells' rows of A and out-edges, the position's slots, carries and ds rows, the fast
// reads, R); then each cell resolves its out-edges' target slots in one LDS read across lanes and
// skips itself when nothing touches it. Per touched cell n and column x, in this order: a = the
// carry of n's slot if n is selected, else A[n] (+ d_h_fast if n is a fast-read cell); + ds_h of
// n's slot; + the edge weight times ds_m of each selected target of n, in n's out-adjacency
// order. Then R = (R + d_q_post) + d_q_pre, and a reset zeroes the row.
template <int CPL>
__global__ __launch_bounds__(kBackThreads) void back_cell_tail(hsn_back_sweep s, int t) {
    extern __shared__ __align__(16) unsigned char lds[];
    constexpr int kCellsPerWave = kCellTailCells / kBackWaves;
    const int row = blockIdx.y;
    const int cell0 = blockIdx.x * kCellTailCells;
    const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
    const int d = s.d, K = s.K, N = s.N, D = s.d_out;
    const int64_t bt = int64_t(row) * s.T + t;
    float* A = s.A + int64_t(row) * N * d;
    const CellTailLds L = cell_tail_lds(N, K, d, D);
    int* slot_of = reinterpret_cast<int*>(lds + L.slot_of);
    float* ds = reinterpret_cast<float*>(lds + L.ds);
    float* carry = reinterpret_cast<float*>(lds + L.carry);
    for (int n = tid; n < N; n += kBackThreads) slot_of[n] = -1;
    // ---- every load at once ----
    const bool reset = s.reset[bt] != 0;
    int cell_k = -1;
    if (tid < K) {
        const int c = s.slots[bt * K + tid];
        cell_k = c >= 0 && c < N ? c : -1;
    }
    float av[kCellsPerWave][CPL], fv[kCellsPerWave][CPL], ew[kCellsPerWave];
    int et[kCellsPerWave];
#pragma unroll
    for (int ci = 0; ci < kCellsPerWave; ++ci) {
        const int n = cell0 + wave + ci * kBackWaves;
        const bool in = n < N;
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            const int x = lane + c * kWave;
            av[ci][c] = in && x < d ? A[int64_t(n) * d + x] : 0.0f;
            fv[ci][c] = in && x < d && n < s.n_read
                            ? s.d_h_fast[(bt * s.n_read + n) * d + x] : 0.0f;
        }
        et[ci] = in && lane < D ? s.out_tgt[int64_t(n) * D + lane] : -1;
        ew[ci] = in && lane < D ? s.out_w[int64_t(n) * D + lane] : 0.0f;
    }
    for (int i = tid; i < K * 2 * d; i += kBackThreads)
        ds[i] = s.ds[int64_t(row) * K * 2 * d + i];
    for (int i = tid; i < K * d; i += kBackThreads) carry[i] = s.carry[int64_t(row) * K * d + i];
    float rv = 0.0f;
    if (blockIdx.x == 0 && tid < d)
        rv = (s.R[int64_t(row) * d + tid] + s.d_q_post[bt * d + tid]) + s.d_q_pre[bt * d + tid];
    __syncthreads();
    if (cell_k >= 0) slot_of[cell_k] = tid;
    __syncthreads();
    // ---- the cells' rows ----
#pragma unroll
    for (int ci = 0; ci < kCellsPerWave; ++ci) {
        const int n = cell0 + wave + ci * kBackWaves;
        if (n >= N) continue;  // uniform per wavefront
        if (reset) {  // the row restarts: its cotangent before position t is zero
#pragma unroll
            for (int c = 0; c < CPL; ++c)
                if (lane + c * kWave < d) A[int64_t(n) * d + lane + c * kWave] = 0.0f;
            continue;
        }
        const int ke = et[ci] >= 0 && et[ci] < N ? slot_of[et[ci]] : -1;  // lane e: edge e's slot
        const uint64_t hit = ballot(ke >= 0);
        const int own = slot_of[n];
        if (hit == 0 && own < 0 && n >= s.n_read) continue;  // nothing touches n (uniform)
        float a[CPL];
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            const int x = lane + c * kWave;
            if (x >= d) continue;
            a[c] = own >= 0 ? carry[own * d + x] : av[ci][c];
            if (own < 0 && n < s.n_read) a[c] = a[c] + fv[ci][c];
            if (own >= 0) a[c] = a[c] + ds[own * 2 * d + x];
        }
        for (uint64_t m = hit; m != 0; m &= m - 1) {  // the selected targets, in edge order
            const int e = __builtin_ctzll(m);
            const int kj = __builtin_amdgcn_readlane(ke, e);
            const float wj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ew[ci]), e));
#pragma unroll
            for (int c = 0; c < CPL; ++c) {
                const int x = lane + c * kWave;
                if (x < d) a[c] = a[c] + wj * ds[kj * 2 * d + d + x];
            }
        }
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            const int x = lane + c * kWave;
            if (x < d) A[int64_t(n) * d + x] = a[c];
        }
    }
    if (blockIdx.x == 0 && tid < d) s.R[int64_t(row) * d + tid] = reset ? 0.0f : rv;
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

void cell_check(const hsn_back_sweep* s) {
    back_check(s);
    HSN_REQUIRE(s->d % 8 == 0 && s->H % 8 == 0, HSN_ERR_INVALID_ARGUMENT,
                "fused reverse sweep step: d and H must be multiples of 8");
    HSN_REQUIRE(s->d <= kCellMaxCpl * kWave, HSN_ERR_INVALID_ARGUMENT,
                "fused reverse sweep step: d above 128");
    HSN_REQUIRE(int64_t(s->B) * s->K <= kCellMaxSlots && s->M <= 256, HSN_ERR_INVALID_ARGUMENT,
                "fused reverse sweep step: more than 4096 slots a position, or more than 256 "
                "units");
    const int BK = s->B * s->K;
    const int lds = s->product_dtype == HSN_DTYPE_BF16 ? cell_lds<bf16_t>(s->d, s->H, BK).bytes
                                                       : cell_lds<float>(s->d, s->H, BK).bytes;
    HSN_REQUIRE(lds <= kCellMaxLds, HSN_ERR_INVALID_ARGUMENT,
                "fused reverse sweep step: 16 slots' operand rows exceed 160 KiB of LDS");
    HSN_REQUIRE(s->w2f != nullptr && s->w1f != nullptr && s->carry != nullptr &&
                    s->ds != nullptr,
                HSN_ERR_INVALID_ARGUMENT,
                "fused reverse sweep step: w2f / w1f / carry / ds is NULL");
    HSN_REQUIRE(cell_tail_lds(s->N, s->K, s->d, s->d_out).bytes <= kMaxLds,
                HSN_ERR_INVALID_ARGUMENT,
                "fused reverse sweep step: the tail's slot table and slot terms (4 N + 12 K d "
                "bytes) exceed 64 KiB of LDS");
    HSN_REQUIRE(s->K <= kBackThreads && s->d_out <= kWave, HSN_ERR_INVALID_ARGUMENT,
                "fused reverse sweep step: more than 256 slots a row or 64 out-edges a cell");
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
        hipLaunchKernelGGL((back_tail<bf16_t>), grid, dim3(kBackThreads), lds,
                           as_stream(stream), s, t);
    else
        hipLaunchKernelGGL((back_tail<float>), grid, dim3(kBackThreads), lds,
                           as_stream(stream), s, t);
    HSN_HIP(hipGetLastError());
    HSN_ABI_END
}

extern "C" int hsn_win_back_cell_check(const hsn_back_sweep* sweep) {
    HSN_ABI_BEGIN
    cell_check(sweep);
    HSN_ABI_END
}

template <typename P, int CPL, int ACT>
void launch_cell_act(const hsn_back_sweep& s, int t, dim3 grid, size_t lds, hipStream_t st) {
    if (lds > static_cast<size_t>(kMaxLds))
        HSN_HIP(allow_lds_raw(reinterpret_cast<const void*>(back_cell<P, CPL, ACT>), lds));
    hipLaunchKernelGGL((back_cell<P, CPL, ACT>), grid, dim3(kCellThreads), lds, st, s, t);
}

template <typename P, int CPL>
void launch_cell(const hsn_back_sweep& s, int t, dim3 grid, size_t lds, hipStream_t st) {
    switch (s.activation) {
        case HSN_ACT_GELU:
            launch_cell_act<P, CPL, HSN_ACT_GELU>(s, t, grid, lds, st);
            break;
        case HSN_ACT_RELU:
            launch_cell_act<P, CPL, HSN_ACT_RELU>(s, t, grid, lds, st);
            break;
        case HSN_ACT_SILU:
            launch_cell_act<P, CPL, HSN_ACT_SILU>(s, t, grid, lds, st);
            break;
        default:
            launch_cell_act<P, CPL, HSN_ACT_TANH>(s, t, grid, lds, st);
    }
}

extern "C" int hsn_win_back_cell(const hsn_back_sweep* sweep, int t, void* stream) {
    HSN_ABI_BEGIN
    cell_check(sweep);
    check_t(sweep, t);
    const hsn_back_sweep s = *sweep;
    const int64_t rows = int64_t(s.B) * s.K;
    const dim3 grid(static_cast<unsigned>((rows + kCellRows - 1) / kCellRows + s.M), 1u,
                    static_cast<unsigned>((2 * s.d + kCellCols - 1) / kCellCols));
    const int cpl = (s.d + kWave - 1) / kWave;
    const bool bf = s.product_dtype == HSN_DTYPE_BF16;
    const int BK = s.B * s.K;
    const size_t lds = static_cast<size_t>(bf ? cell_lds<bf16_t>(s.d, s.H, BK).bytes
                                              : cell_lds<float>(s.d, s.H, BK).bytes);
    hipStream_t st = as_stream(stream);
    if (bf) {
        if (cpl == 1) launch_cell<bf16_t, 1>(s, t, grid, lds, st);
        else launch_cell<bf16_t, 2>(s, t, grid, lds, st);
    } else {
        if (cpl == 1) launch_cell<float, 1>(s, t, grid, lds, st);
        else launch_cell<float, 2>(s, t, grid, lds, st);
    }
    HSN_HIP(hipGetLastError());
    HSN_ABI_END
}

extern "C" int hsn_win_back_cell_tail(const hsn_back_sweep* sweep, int t, void* stream) {
    HSN_ABI_BEGIN
    cell_check(sweep);
    check_t(sweep, t);
    const hsn_back_sweep s = *sweep;
    const dim3 grid(static_cast<unsigned>((s.N + kCellTailCells - 1) / kCellTailCells),
                    static_cast<unsigned>(s.B));
    const size_t lds = static_cast<size_t>(cell_tail_lds(s.N, s.K, s.d, s.d_out).bytes);
    const int cpl = (s.d + kWave - 1) / kWave;
    hipStream_t st = as_stream(stream);
#define HSN_TAIL(C) \
    hipLaunchKernelGGL((back_cell_tail<C>), grid, dim3(kBackThreads), lds, st, s, t)
    if (cpl == 1) HSN_TAIL(1);
    else if (cpl == 2) HSN_TAIL(2);
    else if (cpl == 3) HSN_TAIL(3);
    else HSN_TAIL(4);
#undef HSN_TAIL
    HSN_HIP(hipGetLastError());
    HSN_ABI_END
}
