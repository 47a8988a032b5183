// The window's forward sweep and backward recurrence on gfx950, with the state resident in LDS.
//
// Both directions are separable over the state's d columns: the gated update
// h'[n,x] = (1-b) h[n,x] + b c touches column x only, the summary q[x] sums column x over the
// slots, and the reverse recurrence (A[n,x], R[x]) likewise (reference
// python/hsn/kernels/native.py:292-302, python/hsn/train/split.py:154-173). So one 64-lane
// wavefront owns (row b, a slice of S columns) for the whole window and keeps that slice of the
// state -- h[N][S] forward, the cotangent A[N][S] backward -- in LDS from the first position to
// the last: HBM is read for the inputs, the decisions and the start state once, and written for
// the per-slot outputs and the end state once. Lanes are (slot lane, column): lane = kl*S + x,
// slot k = kl + j*L (L = 64/S slot lanes, j < KPL), so a slot's S columns are contiguous in HBM
// and in LDS. Valid slots of one position name distinct cells, so no two lanes write one LDS
// word; every LDS read of a position is issued before its writes (a padded slot reads cell 0
// before the update, as the reference's gather does).
//
// The inputs of the next D positions are prefetched into registers while a block of D
// positions runs, so the sequential chain per position is LDS read -> FMA -> LDS write.
#include "common.cuh"

namespace hsn {
namespace {

// Positions per prefetch block: about 8 slot-loads of y/gate in flight per lane forward and 4
// backward (which loads twice as much per slot), whatever the slots per lane.
constexpr int fwd_depth(int kpl) { return kpl >= 8 ? 1 : 8 / kpl; }
constexpr int bwd_depth(int kpl) { return kpl >= 4 ? 1 : 4 / kpl; }

// (row, slice) of a workgroup. With B a multiple of 8 the slices of one row go to one XCD
// (workgroups are dealt to the 8 XCDs round-robin by id), so the row's shared cache lines (the
// slots' rows of y/gate, the decisions) are fetched into one L2 instead of several.
__device__ __forceinline__ void block_coords(int bid, int nslices, int xcd_rows, int& b,
                                             int& slice) {
    if (xcd_rows > 0) {
        const int x8 = bid & 7, q = bid >> 3;
        const int rl = q / nslices;
        slice = q - rl * nslices;
        b = x8 * xcd_rows + rl;
    } else {
        b = bid / nslices;
        slice = bid - b * nslices;
    }
}

__device__ __forceinline__ float div_n(float v, float inv_n, float n, bool pow2) {
    return pow2 ? v * inv_n : v / n;
}

// ------------------------------------------------------------------------------------------
// Forward
// ------------------------------------------------------------------------------------------

struct FwdArgs {
    const void* y;
    const void* g;
    int64_t y_row;  // row stride of y and g; position stride K*d
    const float* cand_w;
    const float* inv_rms;
    int64_t rms_row;  // [., T, K]
    const uint8_t* reset;
    int64_t r_row;  // reset[b*r_row + t] zeroes the state before position t (NULL: none)
    const uint8_t* clear;
    int64_t c_row;  // clear[b*c_row] zeroes the written end state (NULL: none)
    const void* cells;
    const uint8_t* valid;
    int64_t s_row;  // [., T, K]
    const float* h0;
    int64_t h0_row;  // [., N, d]
    const float* q0;
    int64_t q0_row;
    const int64_t* age0;
    int64_t a0_row;
    const int64_t* pos0;
    void* q_pre;
    void* q_post;
    int64_t qo_row;  // [., T, d]
    void* h_sel;
    void* h_old;
    int64_t o_row;  // [., T, K, d]
    float* h_max;
    int64_t hm_row;  // [., T]
    float* h_T;
    int64_t hT_row;
    float* q_T;
    int64_t qT_row;
    int64_t* age_T;
    int64_t aT_row;
    int64_t* pos_T;
    int B, T, N, d, K, s_shift, rms, xcd_rows, n_pow2;
    float inv_n, n_f;
};

template <typename IN, typename IDX, int KPL, int D>
struct FwdBlock {
    IN y[D][KPL];
    IN g[D][KPL];
    IDX c[D][KPL];
    uint8_t v[D][KPL];
    float ir[D][KPL];
    uint8_t r[D];
};

template <typename IN, typename IDX, int KPL, int D>
__device__ __forceinline__ void fwd_load(const FwdArgs& a, FwdBlock<IN, IDX, KPL, D>& blk, int b,
                                         int t0, int kl, int L, int col) {
    const IN* y = static_cast<const IN*>(a.y) + b * a.y_row;
    const IN* g = static_cast<const IN*>(a.g) + b * a.y_row;
    const IDX* cells = static_cast<const IDX*>(a.cells) + b * a.s_row;
    const uint8_t* valid = a.valid + b * a.s_row;
    const int64_t kd = int64_t(a.K) * a.d;
#pragma unroll
    for (int p = 0; p < D; ++p) {
        const int t = t0 + p;
        if (t < a.T) {
            blk.r[p] = a.reset ? a.reset[b * a.r_row + t] : 0;
#pragma unroll
            for (int j = 0; j < KPL; ++j) {
                const int k = kl + j * L;
                if (k < a.K) {
                    const int64_t o = t * kd + int64_t(k) * a.d + col;
                    blk.y[p][j] = y[o];
                    blk.g[p][j] = g[o];
                    blk.c[p][j] = cells[int64_t(t) * a.K + k];
                    blk.v[p][j] = valid[int64_t(t) * a.K + k];
                    if (a.rms) blk.ir[p][j] = a.inv_rms[b * a.rms_row + int64_t(t) * a.K + k];
                }
            }
        }
    }
}

template <typename IN, typename OUT, typename IDX, int KPL, int D>
__device__ __forceinline__ void fwd_process(const FwdArgs& a, const FwdBlock<IN, IDX, KPL, D>& blk,
                                            int b, int t0, int kl, int L, int x, int col,
                                            int S, float* lds_h, uint32_t* lds_m, int* lds_last,
                                            bool track_age, float cw, float& q, int& last_reset) {
    const int lane = lane_id();
    const int N = a.N, K = a.K;
    const int64_t kd = int64_t(K) * a.d;
#pragma unroll
    for (int p = 0; p < D; ++p) {
        const int t = t0 + p;
        if (t >= a.T) break;
        if (uniform(blk.r[p])) {  // a document boundary: h, q (and the ages) restart at zero
            for (int e = lane; e < N * S; e += kWave) lds_h[e] = 0.0f;
            if (lds_m)
                for (int n = lane; n < N; n += kWave) lds_m[n] = 0u;
            q = 0.0f;
            last_reset = t;
        }
        if (a.q_pre && kl == 0) store_f32(static_cast<OUT*>(a.q_pre), b * a.qo_row + int64_t(t) * a.d + col, q);
        int cell[KPL];
        float hold[KPL];
#pragma unroll
        for (int j = 0; j < KPL; ++j) {
            const int k = kl + j * L;
            cell[j] = (k < K) ? (blk.v[p][j] ? static_cast<int>(blk.c[p][j]) : -1) : -2;
            const int nr = cell[j] >= 0 ? cell[j] : 0;
            hold[j] = lds_h[nr * S + x];
        }
        float hnew[KPL];
        float delta = 0.0f;
#pragma unroll
        for (int j = 0; j < KPL; ++j) {
            float pre = to_f32(blk.y[p][j]);
            if (a.rms) pre = pre * blk.ir[p][j] * cw;
            const float c = act_tanh(pre);
            const float bg = act_sigmoid(to_f32(blk.g[p][j]));
            hnew[j] = (1.0f - bg) * hold[j] + bg * c;
        }
#pragma unroll
        for (int j = 0; j < KPL; ++j) {
            if (cell[j] >= 0) {
                lds_h[cell[j] * S + x] = hnew[j];
                delta += hnew[j] - hold[j];
            }
        }
        // the slots' outputs: the pre-round state (the backward's tape) and the updated one
        bool padded = false;
#pragma unroll
        for (int j = 0; j < KPL; ++j) padded |= cell[j] == -1;
        float cell0 = 0.0f;
        if (ballot(padded)) cell0 = lds_h[x];  // a padded slot shows cell 0 after the update
#pragma unroll
        for (int j = 0; j < KPL; ++j) {
            const int k = kl + j * L;
            if (cell[j] != -2) {
                const int64_t o = b * a.o_row + t * kd + int64_t(k) * a.d + col;
                if (a.h_old) store_f32(static_cast<OUT*>(a.h_old), o, hold[j]);
                if (a.h_sel) store_f32(static_cast<OUT*>(a.h_sel), o, cell[j] >= 0 ? hnew[j] : cell0);
            }
        }
        // the summary: q' = q + sum_k (h' - h)[k] / N over the slot lanes of this column
        for (int m = S; m < kWave; m <<= 1) delta += wave_shfl_xor(delta, m);
        q = q + div_n(delta, a.inv_n, a.n_f, a.n_pow2);
        if (a.q_post && kl == 0) store_f32(static_cast<OUT*>(a.q_post), b * a.qo_row + int64_t(t) * a.d + col, q);
        // the row's max |h| after the position: per cell over this slice, then over cells
        if (lds_m) {
#pragma unroll
            for (int j = 0; j < KPL; ++j) {
                uint32_t mm = abs_bits(hnew[j]);
                for (int m = 1; m < S; m <<= 1) {
                    const uint32_t o = wave_shfl_xor(mm, m);
                    mm = o > mm ? o : mm;
                }
                if (x == 0 && cell[j] >= 0) lds_m[cell[j]] = mm;
            }
            uint32_t top = 0u;
            for (int n = lane; n < N; n += kWave) {
                const uint32_t v = lds_m[n];
                top = v > top ? v : top;
            }
            for (int m = 1; m < kWave; m <<= 1) {
                const uint32_t o = wave_shfl_xor(top, m);
                top = o > top ? o : top;
            }
            if (lane == 0) atomicMax(reinterpret_cast<unsigned int*>(a.h_max + b * a.hm_row + t), top);
        }
        if (track_age && x == 0) {
#pragma unroll
            for (int j = 0; j < KPL; ++j)
                if (cell[j] >= 0) lds_last[cell[j]] = t;
        }
    }
}

template <typename IN, typename OUT, typename IDX, int KPL>
__global__ __launch_bounds__(64) void fwd_sweep(FwdArgs a) {
    extern __shared__ float lds[];
    constexpr int D = fwd_depth(KPL);
    const int lane = lane_id();
    const int sh = a.s_shift, S = 1 << sh, L = kWave >> sh;
    const int x = lane & (S - 1), kl = lane >> sh;
    const int nslices = a.d >> sh;
    int b, slice;
    block_coords(blockIdx.x, nslices, a.xcd_rows, b, slice);
    const int col = slice * S + x;
    const int N = a.N, d = a.d;
    float* lds_h = lds;
    uint32_t* lds_m = a.h_max ? reinterpret_cast<uint32_t*>(lds + N * S) : nullptr;
    int* lds_last = reinterpret_cast<int*>(lds + N * S + (a.h_max ? N : 0));
    const bool track_age = slice == 0 && (a.age_T != nullptr);

    // the start state of this slice, and its per-cell max |h|
    for (int e = lane; e < N * S; e += kWave) {
        const int n = e >> sh, xx = e & (S - 1);
        const float v = a.h0[b * a.h0_row + int64_t(n) * d + slice * S + xx];
        lds_h[e] = v;
        if (lds_m) {
            uint32_t mm = abs_bits(v);
            for (int m = 1; m < S; m <<= 1) {
                const uint32_t o = wave_shfl_xor(mm, m);
                mm = o > mm ? o : mm;
            }
            if (xx == 0) lds_m[n] = mm;
        }
    }
    if (track_age)
        for (int n = lane; n < N; n += kWave) lds_last[n] = -1;
    float q = a.q0[b * a.q0_row + col];
    int last_reset = -1;
    const float cw = a.rms ? a.cand_w[col] : 1.0f;

    FwdBlock<IN, IDX, KPL, D> A, Bk;
    fwd_load(a, A, b, 0, kl, L, col);
    for (int t0 = 0; t0 < a.T; t0 += 2 * D) {
        fwd_load(a, Bk, b, t0 + D, kl, L, col);
        fwd_process<IN, OUT, IDX, KPL, D>(a, A, b, t0, kl, L, x, col, S, lds_h, lds_m, lds_last,
                                          track_age, cw, q, last_reset);
        if (t0 + D >= a.T) break;
        fwd_load(a, A, b, t0 + 2 * D, kl, L, col);
        fwd_process<IN, OUT, IDX, KPL, D>(a, Bk, b, t0 + D, kl, L, x, col, S, lds_h, lds_m,
                                          lds_last, track_age, cw, q, last_reset);
    }

    // the end state (zeroed when the caller's next record resets this row)
    const bool clear = a.clear ? a.clear[b * a.c_row] != 0 : false;
    if (a.h_T) {
        for (int e = lane; e < N * S; e += kWave) {
            const int n = e >> sh, xx = e & (S - 1);
            a.h_T[b * a.hT_row + int64_t(n) * d + slice * S + xx] = clear ? 0.0f : lds_h[e];
        }
    }
    if (a.q_T && kl == 0) a.q_T[b * a.qT_row + col] = clear ? 0.0f : q;
    if (track_age) {
        const int T = a.T;
        for (int n = lane; n < N; n += kWave) {
            const int ls = lds_last[n];
            int64_t age;
            if (ls >= 0 && ls >= last_reset) age = (T - 1) - ls;
            else if (last_reset >= 0) age = T - last_reset;
            else age = a.age0[b * a.a0_row + n] + T;
            a.age_T[b * a.aT_row + n] = clear ? 0 : age;
        }
        if (a.pos_T && lane == 0)
            a.pos_T[b] = last_reset >= 0 ? int64_t(T - last_reset) : a.pos0[b] + T;
    }
}

// 1 / rms of every slot's candidate input: inv[b,t,k] = rsqrt(mean_x y^2 + eps), one wavefront
// per slot (the only cross-column quantity of the round, and it reads inputs only).
template <typename IN>
__global__ __launch_bounds__(256) void rms_prologue(const IN* y, float* inv, int64_t slots, int d,
                                                    float eps) {
    const int64_t s = int64_t(blockIdx.x) * (blockDim.x / kWave) + threadIdx.x / kWave;
    if (s >= slots) return;
    const int lane = lane_id();
    float sum = 0.0f;
    for (int x = lane; x < d; x += kWave) {
        const float v = to_f32(y[s * d + x]);
        sum += v * v;
    }
    for (int m = 1; m < kWave; m <<= 1) sum += wave_shfl_xor(sum, m);
    if (lane == 0) inv[s] = rsqrtf(sum / static_cast<float>(d) + eps);
}

// ------------------------------------------------------------------------------------------
// Backward
// ------------------------------------------------------------------------------------------

enum Act { kActNone = 0, kActTanh = 1, kActRms = 2 };

struct BwdArgs {
    const void* y;  // the candidate input (kActNone: c itself)
    const void* g;  // the gate pre-activation (kActNone: b itself)
    const void* h_old;
    const void* dsel;
    int64_t y_row;  // row stride of y, g, h_old, dsel, dy, dg ([., T, K, d])
    const float* cand_w;
    const float* inv_rms;
    const void* cells;
    const uint8_t* valid;
    int64_t s_row;
    const uint8_t* reset;
    int64_t r_row;
    const void* dq_pre;
    const void* dq_post;
    int64_t q_row;  // [., T, d]
    const float* dh_T;
    const float* dq_T;
    void* dy;
    void* dg;
    float* dh0;
    float* dq0;
    int B, T, N, d, K, s_shift, act, xcd_rows, n_pow2;
    float inv_n, n_f;
};

template <typename IN, typename IDX, int KPL, int D>
struct BwdBlock {
    IN y[D][KPL];
    IN g[D][KPL];
    IN ho[D][KPL];
    IN ds[D][KPL];
    IDX c[D][KPL];
    uint8_t v[D][KPL];
    float ir[D][KPL];
    IN qpre[D];
    IN qpost[D];
    uint8_t r[D];
};

template <typename IN, typename IDX, int KPL, int D>
__device__ __forceinline__ void bwd_load(const BwdArgs& a, BwdBlock<IN, IDX, KPL, D>& blk, int b,
                                         int t0, int kl, int L, int col) {
    const int64_t base = b * a.y_row;
    const IN* y = static_cast<const IN*>(a.y) + base;
    const IN* g = static_cast<const IN*>(a.g) + base;
    const IN* ho = static_cast<const IN*>(a.h_old) + base;
    const IN* ds = a.dsel ? static_cast<const IN*>(a.dsel) + base : nullptr;
    const IDX* cells = static_cast<const IDX*>(a.cells) + b * a.s_row;
    const uint8_t* valid = a.valid + b * a.s_row;
    const int64_t kd = int64_t(a.K) * a.d;
#pragma unroll
    for (int p = 0; p < D; ++p) {
        const int t = t0 - p;  // walking backwards
        if (t >= 0) {
            blk.r[p] = a.reset[b * a.r_row + t];
            if (a.dq_pre) blk.qpre[p] = static_cast<const IN*>(a.dq_pre)[b * a.q_row + int64_t(t) * a.d + col];
            if (a.dq_post) blk.qpost[p] = static_cast<const IN*>(a.dq_post)[b * a.q_row + int64_t(t) * a.d + col];
#pragma unroll
            for (int j = 0; j < KPL; ++j) {
                const int k = kl + j * L;
                if (k < a.K) {
                    const int64_t o = t * kd + int64_t(k) * a.d + col;
                    blk.y[p][j] = y[o];
                    blk.g[p][j] = g[o];
                    blk.ho[p][j] = ho[o];
                    if (ds) blk.ds[p][j] = ds[o];
                    blk.c[p][j] = cells[int64_t(t) * a.K + k];
                    blk.v[p][j] = valid[int64_t(t) * a.K + k];
                    if (a.act == kActRms) blk.ir[p][j] = a.inv_rms[b * int64_t(a.T) * a.K + int64_t(t) * a.K + k];
                }
            }
        }
    }
}

template <typename IN, typename IDX, int KPL, int D>
__device__ __forceinline__ void bwd_process(const BwdArgs& a, const BwdBlock<IN, IDX, KPL, D>& blk,
                                            int b, int t0, int kl, int L, int x, int col, int S,
                                            float* lds_A, float cw, float& R) {
    const int lane = lane_id();
    const int N = a.N, K = a.K;
    const int64_t kd = int64_t(K) * a.d;
#pragma unroll
    for (int p = 0; p < D; ++p) {
        const int t = t0 - p;
        if (t < 0) break;
        if (a.dq_post) R += to_f32(blk.qpost[p]);
        const float share = div_n(R, a.inv_n, a.n_f, a.n_pow2);
        int cell[KPL];
        float aold[KPL];
#pragma unroll
        for (int j = 0; j < KPL; ++j) {
            const int k = kl + j * L;
            cell[j] = (k < K) ? (blk.v[p][j] ? static_cast<int>(blk.c[p][j]) : -1) : -2;
            aold[j] = cell[j] >= 0 ? lds_A[cell[j] * S + x] : 0.0f;
        }
#pragma unroll
        for (int j = 0; j < KPL; ++j) {
            const int k = kl + j * L;
            float c, bg, pre = 0.0f;
            if (a.act == kActNone) {
                c = to_f32(blk.y[p][j]);
                bg = to_f32(blk.g[p][j]);
            } else {
                pre = to_f32(blk.y[p][j]);
                if (a.act == kActRms) pre = pre * blk.ir[p][j] * cw;
                c = act_tanh(pre);
                bg = act_sigmoid(to_f32(blk.g[p][j]));
            }
            float carried = aold[j];
            if (a.dsel) carried += to_f32(blk.ds[p][j]);
            const float gg = carried + share;
            float dc = bg * gg;
            float db = (c - to_f32(blk.ho[p][j])) * gg;
            const float anew = (1.0f - bg) * carried - bg * share;
            if (cell[j] >= 0) {
                lds_A[cell[j] * S + x] = anew;
            } else {
                dc = 0.0f;
                db = 0.0f;
            }
            float o1 = dc, o2 = db;
            if (a.act != kActNone) {
                o1 = dc * (1.0f - c * c);   // tanh' (kActRms: the cotangent of the norm's output)
                o2 = db * (1.0f - bg) * bg;  // sigmoid'
            }
            if (cell[j] != -2) {
                const int64_t o = b * a.y_row + t * kd + int64_t(k) * a.d + col;
                store_f32(static_cast<IN*>(a.dy), o, o1);
                store_f32(static_cast<IN*>(a.dg), o, o2);
            }
        }
        if (a.dq_pre) R += to_f32(blk.qpre[p]);
        if (uniform(blk.r[p])) {  // the boundary: nothing before it reaches past the reset
            for (int e = lane; e < N * S; e += kWave) lds_A[e] = 0.0f;
            R = 0.0f;
        }
    }
}

template <typename IN, typename IDX, int KPL>
__global__ __launch_bounds__(64) void bwd_sweep(BwdArgs a) {
    extern __shared__ float lds[];
    constexpr int D = bwd_depth(KPL);
    const int lane = lane_id();
    const int sh = a.s_shift, S = 1 << sh, L = kWave >> sh;
    const int x = lane & (S - 1), kl = lane >> sh;
    const int nslices = a.d >> sh;
    int b, slice;
    block_coords(blockIdx.x, nslices, a.xcd_rows, b, slice);
    const int col = slice * S + x;
    const int N = a.N, d = a.d;
    float* lds_A = lds;
    for (int e = lane; e < N * S; e += kWave) {
        const int n = e >> sh, xx = e & (S - 1);
        lds_A[e] = a.dh_T ? a.dh_T[int64_t(b) * N * d + int64_t(n) * d + slice * S + xx] : 0.0f;
    }
    float R = a.dq_T ? a.dq_T[int64_t(b) * d + col] : 0.0f;
    const float cw = a.act == kActRms ? a.cand_w[col] : 1.0f;

    BwdBlock<IN, IDX, KPL, D> A, Bk;
    const int last = a.T - 1;
    bwd_load(a, A, b, last, kl, L, col);
    for (int t0 = last; t0 >= 0; t0 -= 2 * D) {
        bwd_load(a, Bk, b, t0 - D, kl, L, col);
        bwd_process<IN, IDX, KPL, D>(a, A, b, t0, kl, L, x, col, S, lds_A, cw, R);
        if (t0 - D < 0) break;
        bwd_load(a, A, b, t0 - 2 * D, kl, L, col);
        bwd_process<IN, IDX, KPL, D>(a, Bk, b, t0 - D, kl, L, x, col, S, lds_A, cw, R);
    }
    if (a.dh0) {
        for (int e = lane; e < N * S; e += kWave) {
            const int n = e >> sh, xx = e & (S - 1);
            a.dh0[int64_t(b) * N * d + int64_t(n) * d + slice * S + xx] = lds_A[e];
        }
    }
    if (a.dq0 && kl == 0) a.dq0[int64_t(b) * d + col] = R;
}

// The RMSNorm candidate's backward, after the sweep left dL/dpre in dy (pre = y * inv * w):
// dL/dw[x] = sum over slots of dpre[x] y[x] inv, in a fixed order (one workgroup per column,
// a fixed-shape tree), then dy[x] = inv w[x] dpre[x] - inv^3 y[x] / d * sum_x' dpre w y.
template <typename IN>
__global__ __launch_bounds__(256) void rms_weight_grad(const IN* y, const IN* dpre, const float* inv,
                                                       float* dw, int64_t slots, int d) {
    __shared__ float part[256];
    const int x = blockIdx.x;
    float acc = 0.0f;
    for (int64_t s = threadIdx.x; s < slots; s += blockDim.x)
        acc += to_f32(dpre[s * d + x]) * to_f32(y[s * d + x]) * inv[s];
    part[threadIdx.x] = acc;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
        if (threadIdx.x < w) part[threadIdx.x] += part[threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x == 0) dw[x] = part[0];
}

template <typename IN>
__global__ __launch_bounds__(256) void rms_input_grad(const IN* y, IN* dy, const float* inv,
                                                      const float* w, int64_t slots, int d) {
    const int64_t s = int64_t(blockIdx.x) * (blockDim.x / kWave) + threadIdx.x / kWave;
    if (s >= slots) return;
    const int lane = lane_id();
    const float r = inv[s];
    float dot = 0.0f;
    for (int x = lane; x < d; x += kWave) dot += to_f32(dy[s * d + x]) * w[x] * to_f32(y[s * d + x]);
    for (int m = 1; m < kWave; m <<= 1) dot += wave_shfl_xor(dot, m);
    const float k3 = r * r * r * dot / static_cast<float>(d);
    for (int x = lane; x < d; x += kWave) {
        const float v = r * w[x] * to_f32(dy[s * d + x]) - k3 * to_f32(y[s * d + x]);
        store_f32(dy, s * d + x, v);
    }
}

// The dense-fallback rows (every cell written each position): the cotangent of one (row, cell,
// column) never meets another's, because R restarts from the position's own cotangents (reference
// python/hsn/train/split.py:177-209), so each thread walks its column chain alone.
__global__ __launch_bounds__(256) void dense_recurrence(const float* c, const float* bgate,
                                                        const float* h_old, const uint8_t* reset,
                                                        const float* dq_pre, const float* dq_post,
                                                        float* dc, float* db, int Bd, int T, int N,
                                                        int d) {
    const int64_t e = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    const int64_t per_row = int64_t(N) * d;
    if (e >= int64_t(Bd) * per_row) return;
    const int64_t r = e / per_row, nd = e - r * per_row;
    const int x = static_cast<int>(nd % d);
    const float n_f = static_cast<float>(N);
    float A = 0.0f, Rc = 0.0f;  // Rc: the summary cotangent carried from position t+1
    for (int t = T - 1; t >= 0; --t) {
        float R = Rc;
        if (dq_post) R += dq_post[(r * T + t) * d + x];
        const int64_t o = (r * T + t) * per_row + nd;
        const float gg = A + R / n_f;
        const float b = bgate[o];
        dc[o] = b * gg;
        db[o] = (c[o] - h_old[o]) * gg;
        A = (1.0f - b) * gg;
        Rc = dq_pre ? dq_pre[(r * T + t) * d + x] : 0.0f;
        if (reset[r * T + t]) {
            A = 0.0f;
            Rc = 0.0f;
        }
    }
}

// ------------------------------------------------------------------------------------------
// Launch helpers
// ------------------------------------------------------------------------------------------

__global__ __launch_bounds__(256) void zero_strided_kernel(float* p, int64_t count,
                                                          int64_t stride) {
    const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < count) p[i * stride] = 0.0f;
}

inline void zero_strided(float* p, int64_t count, int64_t stride, hipStream_t st) {
    hipLaunchKernelGGL(zero_strided_kernel, dim3(static_cast<int>((count + 255) / 256)), dim3(256),
                       0, st, p, count, stride);
}

struct SliceShape {
    int s_shift;  // S = 1 << s_shift columns per wavefront
    int kpl;      // slots per lane (1, 2, 4 or 8)
};

// S (columns per wavefront): one slot per lane (S <= 64 / K) keeps the most wavefronts in
// flight for small batches; wider slices (up to 16 columns, 64-byte fp32 segments) are taken
// while the grid still holds >= 2048 wavefronts. Narrowed while the slice's LDS does not fit
// (then each lane takes up to 8 slots).
inline bool choose_shape(int B, int d, int K, int64_t lds_per_col, int64_t lds_fixed,
                         SliceShape& out) {
    constexpr int64_t kLdsMax = 160 * 1024;
    int dmax = 0;  // the largest power of two <= 16 dividing d
    while (dmax < 4 && d % (2 << dmax) == 0) ++dmax;
    int sh = 0;
    while (sh < dmax && (2 << sh) * K <= kWave) ++sh;
    while (sh < dmax && int64_t(B) * (d >> (sh + 1)) >= 2048) ++sh;
    for (; sh >= 0; --sh) {
        const int S = 1 << sh, L = kWave / S;
        const int kpl_need = (K + L - 1) / L;
        if (kpl_need > 8) continue;
        if (lds_per_col * S + lds_fixed > kLdsMax) continue;
        int kpl = 1;
        while (kpl < kpl_need) kpl <<= 1;
        out.s_shift = sh;
        out.kpl = kpl;
        return true;
    }
    return false;
}

inline int xcd_rows_of(int B) { return (B % 8 == 0) ? B / 8 : 0; }

template <typename IN, typename OUT, typename IDX>
hipError_t launch_fwd(const FwdArgs& a, int kpl, size_t lds, hipStream_t st) {
    const int blocks = a.B * (a.d >> a.s_shift);
    switch (kpl) {
        case 1: hipLaunchKernelGGL((fwd_sweep<IN, OUT, IDX, 1>), dim3(blocks), dim3(kWave), lds, st, a); break;
        case 2: hipLaunchKernelGGL((fwd_sweep<IN, OUT, IDX, 2>), dim3(blocks), dim3(kWave), lds, st, a); break;
        case 4: hipLaunchKernelGGL((fwd_sweep<IN, OUT, IDX, 4>), dim3(blocks), dim3(kWave), lds, st, a); break;
        case 8: hipLaunchKernelGGL((fwd_sweep<IN, OUT, IDX, 8>), dim3(blocks), dim3(kWave), lds, st, a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <typename IN, typename IDX>
hipError_t launch_bwd(const BwdArgs& a, int kpl, size_t lds, hipStream_t st) {
    const int blocks = a.B * (a.d >> a.s_shift);
    switch (kpl) {
        case 1: hipLaunchKernelGGL((bwd_sweep<IN, IDX, 1>), dim3(blocks), dim3(kWave), lds, st, a); break;
        case 2: hipLaunchKernelGGL((bwd_sweep<IN, IDX, 2>), dim3(blocks), dim3(kWave), lds, st, a); break;
        case 4: hipLaunchKernelGGL((bwd_sweep<IN, IDX, 4>), dim3(blocks), dim3(kWave), lds, st, a); break;
        case 8: hipLaunchKernelGGL((bwd_sweep<IN, IDX, 8>), dim3(blocks), dim3(kWave), lds, st, a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// Every instantiation a kernel may be launched with needs its LDS ceiling raised once per
// device; the launch helpers do it lazily (hipFuncSetAttribute is cheap and idempotent).
template <typename K>
hipError_t allow_lds(K kernel, size_t lds) {
    if (lds <= 64 * 1024) return hipSuccess;
    return hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                               hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
}

template <typename IN, typename OUT, typename IDX>
hipError_t prepare_fwd(int kpl, size_t lds) {
    switch (kpl) {
        case 1: return allow_lds(fwd_sweep<IN, OUT, IDX, 1>, lds);
        case 2: return allow_lds(fwd_sweep<IN, OUT, IDX, 2>, lds);
        case 4: return allow_lds(fwd_sweep<IN, OUT, IDX, 4>, lds);
        case 8: return allow_lds(fwd_sweep<IN, OUT, IDX, 8>, lds);
    }
    return hipErrorInvalidValue;
}

template <typename IN, typename IDX>
hipError_t prepare_bwd(int kpl, size_t lds) {
    switch (kpl) {
        case 1: return allow_lds(bwd_sweep<IN, IDX, 1>, lds);
        case 2: return allow_lds(bwd_sweep<IN, IDX, 2>, lds);
        case 4: return allow_lds(bwd_sweep<IN, IDX, 4>, lds);
        case 8: return allow_lds(bwd_sweep<IN, IDX, 8>, lds);
    }
    return hipErrorInvalidValue;
}

}  // namespace
}  // namespace hsn

#include "abi_util.h"

using namespace hsn;

namespace {

void fill_n_consts(int N, int& pow2, float& inv_n, float& n_f) {
    pow2 = (N & (N - 1)) == 0 ? 1 : 0;
    inv_n = 1.0f / static_cast<float>(N);
    n_f = static_cast<float>(N);
}

}  // namespace

extern "C" int hsn_win_forward(const void* y, const void* gate_pre, int io_dtype,
                               const float* cand_w, int cand_norm, float cand_eps,
                               float* rms_scratch, const uint8_t* reset, const void* cells,
                               const uint8_t* valid, int index_bits, const float* h0,
                               const float* q0, const int64_t* age0, const int64_t* pos0,
                               void* q_pre, void* q_post, void* h_sel, void* h_old, float* h_max,
                               float* h_T, float* q_T, int64_t* age_T, int64_t* pos_T, int B,
                               int T, int N, int d, int K, void* stream) {
    HSN_ABI_BEGIN
    HSN_REQUIRE(y && gate_pre && reset && cells && valid && h0 && q0, HSN_ERR_INVALID_ARGUMENT,
                "hsn_win_forward: a required pointer is NULL");
    HSN_REQUIRE(B >= 1 && T >= 1 && N >= 1 && d >= 1 && K >= 1 && K <= N,
                HSN_ERR_INVALID_ARGUMENT, "hsn_win_forward: bad dimensions");
    HSN_REQUIRE(!age_T || age0, HSN_ERR_INVALID_ARGUMENT, "hsn_win_forward: age_T needs age0");
    HSN_REQUIRE(!pos_T || (pos0 && age_T), HSN_ERR_INVALID_ARGUMENT,
                "hsn_win_forward: pos_T needs pos0 and age_T");
    HSN_REQUIRE(!cand_norm || (cand_w && rms_scratch), HSN_ERR_INVALID_ARGUMENT,
                "hsn_win_forward: the RMS candidate needs cand_w and rms_scratch");
    HSN_REQUIRE(index_bits == 32 || index_bits == 64, HSN_ERR_INVALID_ARGUMENT,
                "hsn_win_forward: index_bits must be 32 or 64");
    HSN_REQUIRE(io_dtype == HSN_DTYPE_F32 || io_dtype == HSN_DTYPE_BF16,
                HSN_ERR_UNSUPPORTED_DTYPE, "hsn_win_forward: io_dtype must be f32 or bf16");
    HSN_REQUIRE(check_elems({int64_t(B) * T * K * d, int64_t(B) * N * d}), HSN_ERR_SIZE_OVERFLOW,
                "hsn_win_forward: a tensor is too large");
    SliceShape sh;
    const int64_t fixed = int64_t(N) * 4 * ((h_max ? 1 : 0) + 1);
    HSN_REQUIRE(choose_shape(B, d, K, int64_t(N) * 4, fixed, sh), HSN_ERR_INVALID_ARGUMENT,
                "hsn_win_forward: the state slice does not fit the LDS (N too large)");
    const size_t lds = size_t(N) * 4 * (size_t(1) << sh.s_shift) + size_t(fixed);
    hipStream_t st = as_stream(stream);
    FwdArgs a{};
    a.y = y, a.g = gate_pre, a.y_row = int64_t(T) * K * d;
    a.cand_w = cand_w, a.inv_rms = rms_scratch, a.rms_row = int64_t(T) * K, a.rms = cand_norm ? 1 : 0;
    a.reset = reset, a.r_row = T, a.clear = nullptr, a.c_row = 0;
    a.cells = cells, a.valid = valid, a.s_row = int64_t(T) * K;
    a.h0 = h0, a.h0_row = int64_t(N) * d, a.q0 = q0, a.q0_row = d;
    a.age0 = age0, a.a0_row = N, a.pos0 = pos0;
    a.q_pre = q_pre, a.q_post = q_post, a.qo_row = int64_t(T) * d;
    a.h_sel = h_sel, a.h_old = h_old, a.o_row = int64_t(T) * K * d;
    a.h_max = h_max, a.hm_row = T;
    a.h_T = h_T, a.hT_row = int64_t(N) * d, a.q_T = q_T, a.qT_row = d;
    a.age_T = age_T, a.aT_row = N, a.pos_T = pos_T;
    a.B = B, a.T = T, a.N = N, a.d = d, a.K = K, a.s_shift = sh.s_shift, a.xcd_rows = xcd_rows_of(B);
    fill_n_consts(N, a.n_pow2, a.inv_n, a.n_f);
    if (cand_norm) {
        const int64_t slots = int64_t(B) * T * K;
        const int blocks = static_cast<int>((slots + 3) / 4);
        if (io_dtype == HSN_DTYPE_F32)
            hipLaunchKernelGGL((rms_prologue<float>), dim3(blocks), dim3(256), 0, st,
                               static_cast<const float*>(y), rms_scratch, slots, d, cand_eps);
        else
            hipLaunchKernelGGL((rms_prologue<bf16_t>), dim3(blocks), dim3(256), 0, st,
                               static_cast<const bf16_t*>(y), rms_scratch, slots, d, cand_eps);
        HSN_HIP(hipGetLastError());
    }
    if (io_dtype == HSN_DTYPE_F32) {
        if (index_bits == 32) {
            HSN_HIP((prepare_fwd<float, float, int32_t>(sh.kpl, lds)));
            HSN_HIP((launch_fwd<float, float, int32_t>(a, sh.kpl, lds, st)));
        } else {
            HSN_HIP((prepare_fwd<float, float, int64_t>(sh.kpl, lds)));
            HSN_HIP((launch_fwd<float, float, int64_t>(a, sh.kpl, lds, st)));
        }
    } else {
        HSN_REQUIRE(index_bits == 32, HSN_ERR_INVALID_ARGUMENT,
                    "hsn_win_forward: bf16 storage takes int32 cells");
        HSN_HIP((prepare_fwd<bf16_t, bf16_t, int32_t>(sh.kpl, lds)));
        HSN_HIP((launch_fwd<bf16_t, bf16_t, int32_t>(a, sh.kpl, lds, st)));
    }
    HSN_ABI_END
}

extern "C" int hsn_win_backward(const void* y, const void* gate_pre, const void* h_old,
                                int io_dtype, const float* cand_w, int cand_norm, float cand_eps,
                                float* rms_scratch, const void* cells, const uint8_t* valid,
                                int index_bits, const uint8_t* reset, const void* d_q_pre,
                                const void* d_q_post, const void* d_h_sel, const float* d_h_T,
                                const float* d_q_T, void* dy, void* dgate, float* d_h0,
                                float* d_q0, float* d_cand_w, int B, int T, int N, int d, int K,
                                void* stream) {
    HSN_ABI_BEGIN
    HSN_REQUIRE(y && gate_pre && h_old && cells && valid && reset && dy && dgate,
                HSN_ERR_INVALID_ARGUMENT, "hsn_win_backward: a required pointer is NULL");
    HSN_REQUIRE(B >= 1 && T >= 1 && N >= 1 && d >= 1 && K >= 1 && K <= N,
                HSN_ERR_INVALID_ARGUMENT, "hsn_win_backward: bad dimensions");
    HSN_REQUIRE(!cand_norm || (cand_w && rms_scratch), HSN_ERR_INVALID_ARGUMENT,
                "hsn_win_backward: the RMS candidate needs cand_w and rms_scratch");
    HSN_REQUIRE(index_bits == 32, HSN_ERR_INVALID_ARGUMENT,
                "hsn_win_backward: the window form takes int32 cells");
    HSN_REQUIRE(io_dtype == HSN_DTYPE_F32 || io_dtype == HSN_DTYPE_BF16,
                HSN_ERR_UNSUPPORTED_DTYPE, "hsn_win_backward: io_dtype must be f32 or bf16");
    HSN_REQUIRE(check_elems({int64_t(B) * T * K * d, int64_t(B) * N * d}), HSN_ERR_SIZE_OVERFLOW,
                "hsn_win_backward: a tensor is too large");
    SliceShape sh;
    HSN_REQUIRE(choose_shape(B, d, K, int64_t(N) * 4, 0, sh), HSN_ERR_INVALID_ARGUMENT,
                "hsn_win_backward: the cotangent slice does not fit the LDS (N too large)");
    const size_t lds = size_t(N) * 4 * (size_t(1) << sh.s_shift);
    hipStream_t st = as_stream(stream);
    const int64_t slots = int64_t(B) * T * K;
    if (cand_norm) {  // the forward's 1 / rms (recomputed: the scratch may have been reused)
        const int blocks = static_cast<int>((slots + 3) / 4);
        if (io_dtype == HSN_DTYPE_F32)
            hipLaunchKernelGGL((rms_prologue<float>), dim3(blocks), dim3(256), 0, st,
                               static_cast<const float*>(y), rms_scratch, slots, d, cand_eps);
        else
            hipLaunchKernelGGL((rms_prologue<bf16_t>), dim3(blocks), dim3(256), 0, st,
                               static_cast<const bf16_t*>(y), rms_scratch, slots, d, cand_eps);
        HSN_HIP(hipGetLastError());
    }
    BwdArgs a{};
    a.y = y, a.g = gate_pre, a.h_old = h_old, a.dsel = d_h_sel, a.y_row = int64_t(T) * K * d;
    a.cand_w = cand_w, a.inv_rms = rms_scratch;
    a.cells = cells, a.valid = valid, a.s_row = int64_t(T) * K;
    a.reset = reset, a.r_row = T;
    a.dq_pre = d_q_pre, a.dq_post = d_q_post, a.q_row = int64_t(T) * d;
    a.dh_T = d_h_T, a.dq_T = d_q_T, a.dy = dy, a.dg = dgate, a.dh0 = d_h0, a.dq0 = d_q0;
    a.B = B, a.T = T, a.N = N, a.d = d, a.K = K, a.s_shift = sh.s_shift;
    a.act = cand_norm ? kActRms : kActTanh, a.xcd_rows = xcd_rows_of(B);
    fill_n_consts(N, a.n_pow2, a.inv_n, a.n_f);
    if (io_dtype == HSN_DTYPE_F32) {
        HSN_HIP((prepare_bwd<float, int32_t>(sh.kpl, lds)));
        HSN_HIP((launch_bwd<float, int32_t>(a, sh.kpl, lds, st)));
    } else {
        HSN_HIP((prepare_bwd<bf16_t, int32_t>(sh.kpl, lds)));
        HSN_HIP((launch_bwd<bf16_t, int32_t>(a, sh.kpl, lds, st)));
    }
    if (cand_norm) {
        const int blocks = static_cast<int>((slots + 3) / 4);
        if (io_dtype == HSN_DTYPE_F32) {
            if (d_cand_w)
                hipLaunchKernelGGL((rms_weight_grad<float>), dim3(d), dim3(256), 0, st,
                                   static_cast<const float*>(y), static_cast<const float*>(dy),
                                   rms_scratch, d_cand_w, slots, d);
            hipLaunchKernelGGL((rms_input_grad<float>), dim3(blocks), dim3(256), 0, st,
                               static_cast<const float*>(y), static_cast<float*>(dy), rms_scratch,
                               cand_w, slots, d);
        } else {
            if (d_cand_w)
                hipLaunchKernelGGL((rms_weight_grad<bf16_t>), dim3(d), dim3(256), 0, st,
                                   static_cast<const bf16_t*>(y), static_cast<const bf16_t*>(dy),
                                   rms_scratch, d_cand_w, slots, d);
            hipLaunchKernelGGL((rms_input_grad<bf16_t>), dim3(blocks), dim3(256), 0, st,
                               static_cast<const bf16_t*>(y), static_cast<bf16_t*>(dy),
                               rms_scratch, cand_w, slots, d);
        }
        HSN_HIP(hipGetLastError());
    }
    HSN_ABI_END
}

extern "C" int hsn_win_recurrence(const float* c, const float* b, const float* h_old,
                                  const int64_t* cells, const uint8_t* valid,
                                  const uint8_t* reset, const float* d_q_pre,
                                  const float* d_q_post, const float* d_h_sel, const float* d_h_T,
                                  const float* d_q_T, float* dc, float* db, float* d_h0,
                                  float* d_q0, int B, int T, int K, int d, int N, void* stream) {
    HSN_ABI_BEGIN
    HSN_REQUIRE(c && b && h_old && cells && valid && reset && dc && db, HSN_ERR_INVALID_ARGUMENT,
                "hsn_win_recurrence: a required pointer is NULL");
    HSN_REQUIRE(B >= 1 && T >= 1 && N >= 1 && d >= 1 && K >= 1, HSN_ERR_INVALID_ARGUMENT,
                "hsn_win_recurrence: bad dimensions");
    HSN_REQUIRE(check_elems({int64_t(B) * T * K * d, int64_t(B) * N * d}), HSN_ERR_SIZE_OVERFLOW,
                "hsn_win_recurrence: a tensor is too large");
    SliceShape sh;
    HSN_REQUIRE(choose_shape(B, d, K, int64_t(N) * 4, 0, sh), HSN_ERR_INVALID_ARGUMENT,
                "hsn_win_recurrence: the cotangent slice does not fit the LDS (N too large)");
    const size_t lds = size_t(N) * 4 * (size_t(1) << sh.s_shift);
    BwdArgs a{};
    a.y = c, a.g = b, a.h_old = h_old, a.dsel = d_h_sel, a.y_row = int64_t(T) * K * d;
    a.cells = cells, a.valid = valid, a.s_row = int64_t(T) * K;
    a.reset = reset, a.r_row = T;
    a.dq_pre = d_q_pre, a.dq_post = d_q_post, a.q_row = int64_t(T) * d;
    a.dh_T = d_h_T, a.dq_T = d_q_T, a.dy = dc, a.dg = db, a.dh0 = d_h0, a.dq0 = d_q0;
    a.B = B, a.T = T, a.N = N, a.d = d, a.K = K, a.s_shift = sh.s_shift, a.act = kActNone;
    a.xcd_rows = xcd_rows_of(B);
    fill_n_consts(N, a.n_pow2, a.inv_n, a.n_f);
    HSN_HIP((prepare_bwd<float, int64_t>(sh.kpl, lds)));
    HSN_HIP((launch_bwd<float, int64_t>(a, sh.kpl, lds, as_stream(stream))));
    HSN_ABI_END
}

extern "C" int hsn_win_recurrence_dense(const float* c, const float* b, const float* h_old,
                                        const uint8_t* reset, const float* d_q_pre,
                                        const float* d_q_post, float* dc, float* db, int Bd,
                                        int T, int N, int d, void* stream) {
    HSN_ABI_BEGIN
    HSN_REQUIRE(c && b && h_old && reset && dc && db, HSN_ERR_INVALID_ARGUMENT,
                "hsn_win_recurrence_dense: a required pointer is NULL");
    HSN_REQUIRE(Bd >= 1 && T >= 1 && N >= 1 && d >= 1, HSN_ERR_INVALID_ARGUMENT,
                "hsn_win_recurrence_dense: bad dimensions");
    HSN_REQUIRE(check_elems({int64_t(Bd) * T * N * d}), HSN_ERR_SIZE_OVERFLOW,
                "hsn_win_recurrence_dense: a tensor is too large");
    const int64_t chains = int64_t(Bd) * N * d;
    const int blocks = static_cast<int>((chains + 255) / 256);
    hipLaunchKernelGGL(dense_recurrence, dim3(blocks), dim3(256), 0, as_stream(stream), c, b, h_old,
                       reset, d_q_pre, d_q_post, dc, db, Bd, T, N, d);
    HSN_HIP(hipGetLastError());
    HSN_ABI_END
}

extern "C" int hsn_win_cell_update(const void* y, const void* gate, int io_dtype,
                                   const float* cand_w, int cand_norm, float cand_eps,
                                   float* rms_scratch, const float* h, const float* q,
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
    HSN_REQUIRE(!pos_next || pos, HSN_ERR_INVALID_ARGUMENT, "hsn_win_cell_update: pos_next needs pos");
    HSN_REQUIRE(!cand_norm || (cand_w && rms_scratch), HSN_ERR_INVALID_ARGUMENT,
                "hsn_win_cell_update: the RMS candidate needs cand_w and rms_scratch");
    HSN_REQUIRE(io_dtype == HSN_DTYPE_F32 || io_dtype == HSN_DTYPE_BF16,
                HSN_ERR_UNSUPPORTED_DTYPE, "hsn_win_cell_update: io_dtype must be f32 or bf16");
    SliceShape sh;
    const int64_t fixed = int64_t(N) * 8;
    HSN_REQUIRE(choose_shape(B, d, K, int64_t(N) * 4, fixed, sh), HSN_ERR_INVALID_ARGUMENT,
                "hsn_win_cell_update: the state slice does not fit the LDS (N too large)");
    const size_t lds = size_t(N) * 4 * (size_t(1) << sh.s_shift) + size_t(fixed);
    hipStream_t st = as_stream(stream);
    // h_max is max-reduced across the row's slices: zero it first (a kernel, not a memset, so
    // the call stays capturable)
    FwdArgs a{};
    a.y = y, a.g = gate, a.y_row = int64_t(K) * d;
    a.cand_w = cand_w, a.inv_rms = rms_scratch, a.rms_row = K, a.rms = cand_norm ? 1 : 0;
    a.reset = nullptr, a.r_row = 0;
    const bool clear = reset && t + 1 < n_slot;
    a.clear = clear ? reset + t + 1 : nullptr, a.c_row = n_slot;
    a.cells = cells + int64_t(t) * K, a.valid = valid + int64_t(t) * K, a.s_row = int64_t(n_slot) * K;
    a.h0 = h + int64_t(t) * N * d, a.h0_row = int64_t(n_state) * N * d;
    a.q0 = q + int64_t(t) * d, a.q0_row = int64_t(n_state) * d;
    a.age0 = age + int64_t(t) * N, a.a0_row = int64_t(n_state) * N, a.pos0 = pos;
    a.q_pre = nullptr, a.q_post = q_post ? q_post + int64_t(t) * d : nullptr, a.qo_row = int64_t(n_slot) * d;
    a.h_sel = h_sel + int64_t(t) * K * d, a.h_old = nullptr, a.o_row = int64_t(n_slot) * K * d;
    a.h_max = h_max + t, a.hm_row = n_slot;
    a.h_T = h_next + int64_t(t_out) * N * d, a.hT_row = int64_t(n_state) * N * d;
    a.q_T = q_next + int64_t(t_out) * d, a.qT_row = int64_t(n_state) * d;
    a.age_T = age_next + int64_t(t_out) * N, a.aT_row = int64_t(n_state) * N, a.pos_T = pos_next;
    a.B = B, a.T = 1, a.N = N, a.d = d, a.K = K, a.s_shift = sh.s_shift, a.xcd_rows = xcd_rows_of(B);
    fill_n_consts(N, a.n_pow2, a.inv_n, a.n_f);
    zero_strided(a.h_max, B, n_slot, st);
    HSN_HIP(hipGetLastError());
    if (cand_norm) {
        const int64_t slots = int64_t(B) * K;
        const int blocks = static_cast<int>((slots + 3) / 4);
        if (io_dtype == HSN_DTYPE_F32)
            hipLaunchKernelGGL((rms_prologue<float>), dim3(blocks), dim3(256), 0, st,
                               static_cast<const float*>(y), rms_scratch, slots, d, cand_eps);
        else
            hipLaunchKernelGGL((rms_prologue<bf16_t>), dim3(blocks), dim3(256), 0, st,
                               static_cast<const bf16_t*>(y), rms_scratch, slots, d, cand_eps);
        HSN_HIP(hipGetLastError());
    }
    if (io_dtype == HSN_DTYPE_F32) {
        HSN_HIP((prepare_fwd<float, float, int64_t>(sh.kpl, lds)));
        HSN_HIP((launch_fwd<float, float, int64_t>(a, sh.kpl, lds, st)));
    } else {
        HSN_HIP((prepare_fwd<bf16_t, float, int64_t>(sh.kpl, lds)));
        HSN_HIP((launch_fwd<bf16_t, float, int64_t>(a, sh.kpl, lds, st)));
    }
    HSN_ABI_END
}
