// The window's forward sweep and backward recurrence on gfx950, with the state resident in LDS.
//
// Both directions are separable over the state's d columns: the gated update
// h'[n,x] = (1-b) h[n,x] + b c touches column x only, the summary q[x] sums column x over the
// slots, and the reverse recurrence (A[n,x], R[x]) likewise (reference
// python/hsn/kernels/native.py:292-302, python/hsn/train/split.py:154-173). So one 64-lane
// wavefront owns (row b, a slice of S columns) for the whole window and keeps that slice of the
// state -- h[N][S] forward, the cotangent A[N][S] backward -- in LDS from the first position to
// the last: HBM is read for the inputs, the decisions and the start state once, and written for
// the per-slot outputs and the end state once.
//
// Lanes are (column, slot lane) with the slot fastest: lane = x*L + kl, L = 64/S, slot
// k = kl + j*L (j < KPL). A column's L slot lanes are consecutive, so the per-column sums and
// maxima reduce with DPP inside a row. Valid slots of one position name distinct cells, so no
// two lanes write one LDS word, and every LDS read of a position is issued before its writes (a
// padded slot reads cell 0 before the update, as the reference's gather does).
//
// Latency: the only sequential chain is LDS read -> FMA -> LDS write per position. The inputs of
// the next P positions stay in flight in a rolling register buffer: every load is unconditional
// (indices clamped into the window, optional inputs aimed at a valid dummy and masked at use), so
// the compiler's wait counts stay exact and a position waits only for its own loads.
#pragma once

#include "common.cuh"
#include "bufio.cuh"
#include "dpp.cuh"

namespace hsn {

// The decisions of a slot as the sweeps read them: `Packed32` is one int32 per slot, the cell
// where the slot is valid and -1 where it is padded (hsn_win_route's `slots`); `Cells64` is the
// reference's pair of arrays, int64 cells and uint8 valid flags.
struct Packed32 {
    using Raw = int32_t;
};
struct Cells64 {
    using Raw = int64_t;
};

// Decode a slot: the cell where valid, -1 where padded.
template <typename SLOT>
__device__ __forceinline__ int slot_cell(typename SLOT::Raw c, uint8_t v) {
    if constexpr (sizeof(typename SLOT::Raw) == 4) return static_cast<int>(c);
    else return v ? static_cast<int>(c) : -1;
}

// (row, slice) of a workgroup, from a grid (G, nslices, B/G), G = 8 when B is a multiple of 8
// (else 1). Workgroups are dealt to the 8 XCDs round-robin by linear id, so blockIdx.x is the
// XCD and all slices of a row land on one XCD: the row's shared cache lines (the slots' rows of
// y/gate, the decisions) are fetched into one L2 instead of several. No division: the resources
// built from (row, slice) stay in SGPRs.
__device__ __forceinline__ void block_coords(int& b, int& slice) {
    b = blockIdx.x * gridDim.z + blockIdx.z;
    slice = blockIdx.y;
}

inline dim3 sweep_grid(int B, int nslices) {
    const int g = B % 8 == 0 ? 8 : 1;
    return dim3(g, nslices, B / g);
}

constexpr int fwd_depth(int kpl) { return kpl >= 8 ? 2 : 8 / kpl; }
constexpr int bwd_depth(int kpl) { return kpl >= 4 ? 2 : (kpl == 2 ? 3 : 6); }

// Select element `i` (a lane-dependent index) of a register array without indexing memory.
template <int P, typename T>
__device__ __forceinline__ T pick(const T (&v)[P], int i) {
    T r = v[0];
#pragma unroll
    for (int p = 1; p < P; ++p) r = i == p ? v[p] : r;
    return r;
}

// ------------------------------------------------------------------------------------------
// Forward
// ------------------------------------------------------------------------------------------

struct FwdArgs {
    const void* y;  // the candidate's pre-activation (the RMS prologue's output with the norm)
    const void* g;
    int64_t y_row;  // row stride of y and g (elements); position stride K*d
    const uint8_t* reset;  // reset[b*r_row + t] zeroes the state before position t (NULL: none)
    int64_t r_row;
    const uint8_t* clear;  // clear[b*c_row] zeroes the written end state (NULL: none)
    int64_t c_row;
    const void* cells;  // Packed32: slots; Cells64: cells
    const uint8_t* valid;  // Cells64 only
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
    int B, T, N, d, K, xcd_rows, n_pow2;
    float inv_n, n_f;
};

template <typename IN, typename SLOT, int KPL>
struct FwdStage {
    IN y[KPL];
    IN g[KPL];
    typename SLOT::Raw c[KPL];
    uint8_t v[KPL];
    uint8_t r;  // the position's reset flag (the same in every lane)
};

template <typename IN, typename OUT, typename SLOT, int S, int KPL>
__global__ __launch_bounds__(64) void fwd_sweep(FwdArgs a) {
    using Raw = typename SLOT::Raw;
    extern __shared__ float lds[];
    constexpr int L = kWave / S;
    constexpr int P = fwd_depth(KPL);
    const int lane = lane_id();
    const int x = lane / L, kl = lane % L;
    int b, slice;
    block_coords(b, slice);
    const int col = slice * S + x;
    const int N = a.N, d = a.d, K = a.K, T = a.T;
    float* lds_h = lds;                                  // [N*S], then one dummy word
    int* lds_last = reinterpret_cast<int*>(lds + N * S + 1);  // [N], then one dummy word
    const int dummy_h = N * S;
    const bool track_age = slice == 0 && a.age_T != nullptr;
    const bool want_max = a.h_max != nullptr;
    const bool has_reset = a.reset != nullptr;

    // the row's tensors as buffer resources: per position a uniform soffset, per lane a voffset
    const uint32_t kd = uint32_t(K) * d;
    const rsrc_t ry = make_rsrc(static_cast<const IN*>(a.y) + b * a.y_row, T * kd * sizeof(IN));
    const rsrc_t rg = make_rsrc(static_cast<const IN*>(a.g) + b * a.y_row, T * kd * sizeof(IN));
    const rsrc_t rc = make_rsrc(static_cast<const Raw*>(a.cells) + b * a.s_row, T * K * sizeof(Raw));
    const rsrc_t rv = make_rsrc(a.valid ? a.valid + b * a.s_row : nullptr, a.valid ? T * K : 0);
    const rsrc_t rr = make_rsrc(has_reset ? a.reset + b * a.r_row : nullptr, has_reset ? T : 0);
    // outputs: uniform row pointers, a per-position uniform offset, per-lane element offsets
    OUT* const ho_row = a.h_old ? static_cast<OUT*>(a.h_old) + b * a.o_row : nullptr;
    OUT* const hs_row = a.h_sel ? static_cast<OUT*>(a.h_sel) + b * a.o_row : nullptr;
    OUT* const qa_row = a.q_pre ? static_cast<OUT*>(a.q_pre) + b * a.qo_row : nullptr;
    OUT* const qb_row = a.q_post ? static_cast<OUT*>(a.q_post) + b * a.qo_row : nullptr;
    bool active[KPL];
    uint32_t vy[KPL], vc[KPL], vv[KPL], eo[KPL];
#pragma unroll
    for (int j = 0; j < KPL; ++j) {
        const int k = kl + j * L;
        active[j] = k < K;
        vy[j] = active[j] ? uint32_t(k * d + col) * sizeof(IN) : kOob;
        eo[j] = uint32_t((active[j] ? k : 0) * d + col);
        vc[j] = active[j] ? uint32_t(k) * sizeof(Raw) : kOob;
        vv[j] = active[j] ? uint32_t(k) : kOob;
    }

    // the start state of this slice and the column maxima of |h|
    // (every loop below runs a uniform trip count with a per-lane guard: a divergent loop exit
    // would make the values defined in it divergent, row pointers included)
    uint32_t colmax = 0u;
    const float* h0_row = a.h0 + b * a.h0_row;
    for (int n0 = 0; n0 < N; n0 += L) {
        const int n = n0 + kl;
        if (n < N) {
            const float v = h0_row[int64_t(n) * d + col];
            lds_h[n * S + x] = v;
            colmax = umax(colmax, abs_bits(v));
        }
    }
    colmax = group_max<L>(colmax);
    if (track_age)
        for (int n0 = 0; n0 < N; n0 += kWave)
            if (n0 + lane < N) lds_last[n0 + lane] = -1;
    float q = a.q0[b * a.q0_row + col];
    int last_reset = -1;

    auto load = [&](FwdStage<IN, SLOT, KPL>& st, int t) {
        t = uniform(t < T ? t : T - 1);
        const uint32_t sy = uint32_t(t) * kd * sizeof(IN);
        const uint32_t sc = uint32_t(t) * K;
#pragma unroll
        for (int j = 0; j < KPL; ++j) {
            st.y[j] = bload<IN>(ry, vy[j], sy);
            st.g[j] = bload<IN>(rg, vy[j], sy);
            st.c[j] = bload<Raw>(rc, vc[j], sc * sizeof(Raw));
            if constexpr (sizeof(Raw) == 8) st.v[j] = bload<uint8_t>(rv, vv[j], sc);
            else st.v[j] = 1;
        }
        st.r = bload<uint8_t>(rr, 0u, uint32_t(t));
    };

    // the prologue keeps its loads in stage order (the scheduler would otherwise reorder
    // them, and the loop's first waits would then have to drain the whole pipeline)
    FwdStage<IN, SLOT, KPL> stage[P];
#pragma unroll
    for (int p = 0; p < P; ++p) {
        load(stage[p], p);
        __builtin_amdgcn_sched_barrier(0);
    }

    for (int t0 = 0; t0 < T; t0 += P) {
        uint32_t hm_b[P];  // the row max |h| of each position of the block (uniform)
#pragma unroll
        for (int p = 0; p < P; ++p) {
            const int t = t0 + p;
            hm_b[p] = 0u;
            if (t < T) {
                if (has_reset && uniform(stage[p].r)) {
                    // a document boundary: h, q (and the ages) restart at zero before t reads them
                    for (int e0 = 0; e0 < N * S; e0 += kWave)
                        if (e0 + lane < N * S) lds_h[e0 + lane] = 0.0f;
                    colmax = 0u;
                    q = 0.0f;
                    last_reset = t;
                }
                const uint32_t tq = uint32_t(uniform(t)) * d;
                if (qa_row && kl == 0) store_f32(qa_row + tq, col, q);
                int cell[KPL];
                float hold[KPL];
#pragma unroll
                for (int j = 0; j < KPL; ++j) {
                    cell[j] = active[j] ? slot_cell<SLOT>(stage[p].c[j], stage[p].v[j]) : -2;
                    hold[j] = lds_h[(cell[j] > 0 ? cell[j] : 0) * S + x];
                }
                float delta = 0.0f;
                bool padded = false, drop = false;
                uint32_t up = 0u;
                float hnew[KPL];
#pragma unroll
                for (int j = 0; j < KPL; ++j) {
                    const float c = fast_tanh(to_f32(stage[p].y[j]));
                    const float bg = fast_sigmoid(to_f32(stage[p].g[j]));
                    hnew[j] = (1.0f - bg) * hold[j] + bg * c;
                    const bool ok = cell[j] >= 0;
                    lds_h[ok ? cell[j] * S + x : dummy_h] = hnew[j];
                    delta += ok ? hnew[j] - hold[j] : 0.0f;
                    const uint32_t ob = abs_bits(hold[j]), nb = abs_bits(hnew[j]);
                    drop |= ok && ob == colmax && nb < ob;
                    up = umax(up, ok ? nb : 0u);
                    padded |= cell[j] == -1;
                }
                float cell0 = 0.0f;
                if (ballot(padded)) cell0 = lds_h[x];  // a padded slot shows cell 0 after the update
                const uint32_t to = uint32_t(uniform(t)) * kd;
#pragma unroll
                for (int j = 0; j < KPL; ++j) {
                    if (active[j]) {
                        if (ho_row) store_f32(ho_row + to, eo[j], hold[j]);
                        if (hs_row) store_f32(hs_row + to, eo[j], cell[j] >= 0 ? hnew[j] : cell0);
                    }
                }
                // q' = q + sum_k (h' - h)[k] / N over the column's slot lanes
                delta = group_sum<L>(delta);
                q = q + (a.n_pow2 ? delta * a.inv_n : delta / a.n_f);
                if (qb_row && kl == 0) store_f32(qb_row + tq, col, q);
                if (want_max) {
                    // the column's max |h|: raised by the new values, rescanned only when a cell
                    // that held it shrank; the row's is the max over the slice's columns
                    colmax = umax(colmax, group_max<L>(up));
                    if (ballot(drop)) {
                        uint32_t m = 0u;
                        for (int n0 = 0; n0 < N; n0 += L)
                            if (n0 + kl < N) m = umax(m, abs_bits(lds_h[(n0 + kl) * S + x]));
                        colmax = group_max<L>(m);
                    }
                    hm_b[p] = wave_max_from_groups<L>(colmax);
                }
                if (track_age) {
#pragma unroll
                    for (int j = 0; j < KPL; ++j)
                        lds_last[(cell[j] >= 0 && x == 0) ? cell[j] : N] = t;
                }
            }
            load(stage[p], t + P);
        }
        if (want_max) {  // lane p sends position t0 + p's row max
            uint32_t m = 0u;
#pragma unroll
            for (int p = 0; p < P; ++p) m = lane == p ? hm_b[p] : m;
            if (lane < P && t0 + lane < T)
                atomicMax(reinterpret_cast<unsigned int*>(a.h_max + b * a.hm_row) + (t0 + lane), m);
        }
    }

    // the end state (zeroed when the caller's next record resets this row)
    const bool clear = a.clear ? a.clear[b * a.c_row] != 0 : false;
    if (a.h_T) {
        float* hT_row = a.h_T + b * a.hT_row;
        for (int n0 = 0; n0 < N; n0 += L)
            if (n0 + kl < N) hT_row[int64_t(n0 + kl) * d + col] = clear ? 0.0f : lds_h[(n0 + kl) * S + x];
    }
    if (a.q_T && kl == 0) a.q_T[b * a.qT_row + col] = clear ? 0.0f : q;
    if (track_age) {
        const int64_t* age0_row = a.age0 + b * a.a0_row;
        int64_t* ageT_row = a.age_T + b * a.aT_row;
        for (int n0 = 0; n0 < N; n0 += kWave) {
            const int n = n0 + lane;
            if (n < N) {
                const int ls = lds_last[n];
                int64_t age;
                if (ls >= 0 && ls >= last_reset) age = (T - 1) - ls;
                else if (last_reset >= 0) age = T - last_reset;
                else age = age0_row[n] + T;
                ageT_row[n] = clear ? 0 : age;
            }
        }
        if (a.pos_T && lane == 0)
            a.pos_T[b] = last_reset >= 0 ? int64_t(T - last_reset) : a.pos0[b] + T;
    }
}

// ------------------------------------------------------------------------------------------
// Backward
// ------------------------------------------------------------------------------------------

struct BwdArgs {
    const void* y;  // the candidate's pre-activation (ACT false: the candidate c itself)
    const void* g;  // the gate's pre-activation (ACT false: the gate b itself)
    const void* h_old;
    const void* dsel;  // optional (NULL: zero)
    int64_t y_row;  // row stride of y, g, h_old, dsel, dy, dg ([., T, K, d])
    const void* cells;
    const uint8_t* valid;
    int64_t s_row;
    const uint8_t* reset;
    int64_t r_row;
    const void* dq_pre;  // optional
    const void* dq_post;  // optional
    int64_t q_row;  // [., T, d]
    const float* dh_T;
    const float* dq_T;
    void* dy;
    void* dg;
    float* dh0;
    float* dq0;
    int B, T, N, d, K, S, xcd_rows, n_pow2;
    float inv_n, n_f;
};

template <typename IN, typename SLOT, int KPL>
struct BwdStage {
    IN y[KPL];
    IN g[KPL];
    IN ho[KPL];
    IN ds[KPL];
    typename SLOT::Raw c[KPL];
    uint8_t v[KPL];
    IN qpre;
    IN qpost;
    uint8_t r;
};

template <typename IN, typename SLOT, bool ACT, int KPL>
__global__ __launch_bounds__(64) void bwd_sweep(BwdArgs a) {
    using Raw = typename SLOT::Raw;
    extern __shared__ float lds[];
    constexpr int P = bwd_depth(KPL);
    const int lane = lane_id();
    const int S = a.S, L = kWave / S;
    const int x = lane / L, kl = lane % L;
    int b, slice;
    block_coords(b, slice);
    const int col = slice * S + x;
    const int N = a.N, d = a.d, K = a.K, T = a.T;
    float* lds_A = lds;  // [N*S], then one dummy word
    const int dummy = N * S;
    // (uniform trip counts with per-lane guards: a divergent loop exit would make the values
    // defined in it divergent, row pointers included)
    const float* dhT_row = a.dh_T ? a.dh_T + int64_t(b) * N * d : nullptr;
    for (int n0 = 0; n0 < N; n0 += L)
        if (n0 + kl < N) lds_A[(n0 + kl) * S + x] = dhT_row ? dhT_row[int64_t(n0 + kl) * d + col] : 0.0f;
    float R = a.dq_T ? a.dq_T[int64_t(b) * d + col] : 0.0f;

    const uint32_t kd = uint32_t(K) * d;
    const uint32_t row_bytes = T * kd * sizeof(IN);
    const int64_t base = b * a.y_row;
    const rsrc_t ry = make_rsrc(static_cast<const IN*>(a.y) + base, row_bytes);
    const rsrc_t rg = make_rsrc(static_cast<const IN*>(a.g) + base, row_bytes);
    const rsrc_t rho = make_rsrc(static_cast<const IN*>(a.h_old) + base, row_bytes);
    const rsrc_t rds = make_rsrc(a.dsel ? static_cast<const IN*>(a.dsel) + base : nullptr,
                                 a.dsel ? row_bytes : 0);
    IN* const dy_row = static_cast<IN*>(a.dy) + base;
    IN* const dg_row = static_cast<IN*>(a.dg) + base;
    const rsrc_t rc = make_rsrc(static_cast<const Raw*>(a.cells) + b * a.s_row, T * K * sizeof(Raw));
    const rsrc_t rv = make_rsrc(a.valid ? a.valid + b * a.s_row : nullptr, a.valid ? T * K : 0);
    const rsrc_t rr = make_rsrc(a.reset + b * a.r_row, T);
    const uint32_t qbytes = T * uint32_t(d) * sizeof(IN);
    const rsrc_t rqa = make_rsrc(a.dq_pre ? static_cast<const IN*>(a.dq_pre) + b * a.q_row : nullptr,
                                 a.dq_pre ? qbytes : 0);
    const rsrc_t rqb = make_rsrc(a.dq_post ? static_cast<const IN*>(a.dq_post) + b * a.q_row : nullptr,
                                 a.dq_post ? qbytes : 0);
    bool active[KPL];
    uint32_t vy[KPL], vc[KPL], vv[KPL], eo[KPL];
#pragma unroll
    for (int j = 0; j < KPL; ++j) {
        const int k = kl + j * L;
        active[j] = k < K;
        vy[j] = active[j] ? uint32_t(k * d + col) * sizeof(IN) : kOob;
        eo[j] = uint32_t((active[j] ? k : 0) * d + col);
        vc[j] = active[j] ? uint32_t(k) * sizeof(Raw) : kOob;
        vv[j] = active[j] ? uint32_t(k) : kOob;
    }
    const uint32_t vq = uint32_t(col) * sizeof(IN);

    auto load = [&](BwdStage<IN, SLOT, KPL>& st, int t) {
        t = uniform(t >= 0 ? t : 0);
        const uint32_t sy = uint32_t(t) * kd * sizeof(IN);
        const uint32_t sc = uint32_t(t) * K;
#pragma unroll
        for (int j = 0; j < KPL; ++j) {
            st.y[j] = bload<IN>(ry, vy[j], sy);
            st.g[j] = bload<IN>(rg, vy[j], sy);
            st.ho[j] = bload<IN>(rho, vy[j], sy);
            st.ds[j] = bload<IN>(rds, vy[j], sy);
            st.c[j] = bload<Raw>(rc, vc[j], sc * sizeof(Raw));
            if constexpr (sizeof(Raw) == 8) st.v[j] = bload<uint8_t>(rv, vv[j], sc);
            else st.v[j] = 1;
        }
        const uint32_t sq = uint32_t(t) * d * sizeof(IN);
        st.qpre = bload<IN>(rqa, vq, sq);
        st.qpost = bload<IN>(rqb, vq, sq);
        st.r = bload<uint8_t>(rr, 0u, uint32_t(t));
    };

    BwdStage<IN, SLOT, KPL> stage[P];
#pragma unroll
    for (int p = 0; p < P; ++p) {
        load(stage[p], T - 1 - p);
        __builtin_amdgcn_sched_barrier(0);
    }

    for (int t0 = T - 1; t0 >= 0; t0 -= P) {
#pragma unroll
        for (int p = 0; p < P; ++p) {
            const int t = t0 - p;
            if (t >= 0) {
                R += to_f32(stage[p].qpost);  // absent cotangents read as zero
                const float share = a.n_pow2 ? R * a.inv_n : R / a.n_f;
                int cell[KPL];
                float aold[KPL];
#pragma unroll
                for (int j = 0; j < KPL; ++j) {
                    cell[j] = active[j] ? slot_cell<SLOT>(stage[p].c[j], stage[p].v[j]) : -2;
                    aold[j] = lds_A[(cell[j] > 0 ? cell[j] : 0) * S + x];
                }
                const uint32_t to = uint32_t(uniform(t)) * kd;
#pragma unroll
                for (int j = 0; j < KPL; ++j) {
                    float c, bg;
                    if constexpr (ACT) {
                        c = fast_tanh(to_f32(stage[p].y[j]));
                        bg = fast_sigmoid(to_f32(stage[p].g[j]));
                    } else {
                        c = to_f32(stage[p].y[j]);
                        bg = to_f32(stage[p].g[j]);
                    }
                    const bool ok = cell[j] >= 0;
                    const float carried = aold[j] + to_f32(stage[p].ds[j]);
                    const float gg = carried + share;
                    float dc = ok ? bg * gg : 0.0f;
                    float db = ok ? (c - to_f32(stage[p].ho[j])) * gg : 0.0f;
                    lds_A[ok ? cell[j] * S + x : dummy] = (1.0f - bg) * carried - bg * share;
                    if constexpr (ACT) {
                        dc = dc * (1.0f - c * c);    // tanh'
                        db = db * (1.0f - bg) * bg;  // sigmoid'
                    }
                    if (active[j]) {
                        store_f32(dy_row + to, eo[j], dc);
                        store_f32(dg_row + to, eo[j], db);
                    }
                }
                R += to_f32(stage[p].qpre);
                if (uniform(stage[p].r)) {
                    // the boundary: nothing before it reaches past the reset
                    for (int e0 = 0; e0 < N * S; e0 += kWave)
                        if (e0 + lane < N * S) lds_A[e0 + lane] = 0.0f;
                    R = 0.0f;
                }
            }
            load(stage[p], t - P);
        }
    }
    if (a.dh0) {
        float* dh0_row = a.dh0 + int64_t(b) * N * d;
        for (int n0 = 0; n0 < N; n0 += L)
            if (n0 + kl < N) dh0_row[int64_t(n0 + kl) * d + col] = lds_A[(n0 + kl) * S + x];
    }
    if (a.dq0 && kl == 0) a.dq0[int64_t(b) * d + col] = R;
}

// ------------------------------------------------------------------------------------------
// The RMS candidate: a prologue normalises the candidate input once (the only cross-column
// quantity of the round, computed from inputs only), an epilogue applies the norm's VJP.
// ------------------------------------------------------------------------------------------

// ynorm[s, x] = y[s, x] * inv[s] * w[x],  inv[s] = rsqrt(mean_x y^2 + eps): a wavefront per slot
template <typename IN>
__global__ __launch_bounds__(256) void rms_prologue(const IN* y, const float* w, IN* ynorm,
                                                    float* inv, int64_t slots, int d, float eps) {
    const int64_t s = int64_t(blockIdx.x) * (blockDim.x / kWave) + threadIdx.x / kWave;
    if (s >= slots) return;
    const int lane = lane_id();
    float sum = 0.0f;
    for (int x = lane; x < d; x += kWave) {
        const float v = to_f32(y[s * d + x]);
        sum += v * v;
    }
    for (int m = 1; m < kWave; m <<= 1) sum += __shfl_xor(sum, m, kWave);
    const float r = rsqrtf(sum / static_cast<float>(d) + eps);
    if (lane == 0) inv[s] = r;
    for (int x = lane; x < d; x += kWave) store_f32(ynorm, s * d + x, to_f32(y[s * d + x]) * r * w[x]);
}

// dL/dw[x] = sum over slots of dpre[x] y[x] inv (one workgroup per column, fixed-shape tree)
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

// dy[x] = inv w[x] dpre[x] - inv^3 y[x] / d * sum_x' dpre[x'] w[x'] y[x'], in place over dpre
template <typename IN>
__global__ __launch_bounds__(256) void rms_input_grad(const IN* y, IN* dy, const float* inv,
                                                      const float* w, int64_t slots, int d) {
    const int64_t s = int64_t(blockIdx.x) * (blockDim.x / kWave) + threadIdx.x / kWave;
    if (s >= slots) return;
    const int lane = lane_id();
    const float r = inv[s];
    float dot = 0.0f;
    for (int x = lane; x < d; x += kWave) dot += to_f32(dy[s * d + x]) * w[x] * to_f32(y[s * d + x]);
    for (int m = 1; m < kWave; m <<= 1) dot += __shfl_xor(dot, m, kWave);
    const float k3 = r * r * r * dot / static_cast<float>(d);
    for (int x = lane; x < d; x += kWave) {
        const float v = r * w[x] * to_f32(dy[s * d + x]) - k3 * to_f32(y[s * d + x]);
        store_f32(dy, s * d + x, v);
    }
}

namespace {
__global__ __launch_bounds__(256) void zero_strided_kernel(float* p, int64_t count, int64_t stride) {
    const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < count) p[i * stride] = 0.0f;
}
}  // namespace

// ------------------------------------------------------------------------------------------
// Host-side shape choice
// ------------------------------------------------------------------------------------------

struct SliceShape {
    int S;    // columns per wavefront (1, 4, 8 or 16)
    int kpl;  // slots per lane (1, 2, 4 or 8)
};

// S: one slot per lane (S <= 64 / K) keeps the most wavefronts in flight for small batches;
// wider slices (up to 16 columns, 64-byte fp32 segments) are taken while the grid still holds
// >= 2048 wavefronts. Narrowed while the slice's LDS does not fit.
inline bool choose_shape(int B, int d, int K, int64_t lds_per_col, int64_t lds_fixed,
                         SliceShape& out) {
    constexpr int64_t kLdsMax = 160 * 1024;
    const int cand[4] = {16, 8, 4, 1};
    int best = -1;
    for (int i = 0; i < 4; ++i) {  // the widest S dividing d with one slot per lane
        const int S = cand[i];
        if (d % S == 0 && S * K <= kWave) {
            best = i;
            break;
        }
    }
    if (best < 0) best = 3;
    // widen while many wavefronts remain
    while (best > 0 && d % cand[best - 1] == 0 && int64_t(B) * (d / cand[best - 1]) >= 2048) --best;
    for (int i = best; i < 4; ++i) {
        const int S = cand[i];
        if (d % S) continue;
        const int L = kWave / S;
        const int kpl_need = (K + L - 1) / L;
        if (kpl_need > 8) continue;
        if (lds_per_col * S + lds_fixed > kLdsMax) continue;
        int kpl = 1;
        while (kpl < kpl_need) kpl <<= 1;
        out.S = S;
        out.kpl = kpl;
        return true;
    }
    return false;
}

inline int xcd_rows_of(int B) { return (B % 8 == 0) ? B / 8 : 0; }

inline void fill_n_consts(int N, int& pow2, float& inv_n, float& n_f) {
    pow2 = (N & (N - 1)) == 0 ? 1 : 0;
    inv_n = 1.0f / static_cast<float>(N);
    n_f = static_cast<float>(N);
}

template <typename K>
hipError_t allow_lds(K kernel, size_t lds) {
    if (lds <= 64 * 1024) return hipSuccess;
    return hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                               hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
}

template <typename IN, typename OUT, typename SLOT, int S>
hipError_t launch_fwd_s(const FwdArgs& a, int kpl, size_t lds, hipStream_t st) {
    const dim3 blocks = sweep_grid(a.B, a.d / S);
#define HSN_FWD_CASE(KP)                                                                          \
    case KP: {                                                                                    \
        auto k = fwd_sweep<IN, OUT, SLOT, S, KP>;                                                 \
        hipError_t e = allow_lds(k, lds);                                                         \
        if (e != hipSuccess) return e;                                                            \
        hipLaunchKernelGGL(k, blocks, dim3(kWave), lds, st, a);                             \
        return hipGetLastError();                                                                 \
    }
    switch (kpl) {
        HSN_FWD_CASE(1)
        HSN_FWD_CASE(2)
        HSN_FWD_CASE(4)
        HSN_FWD_CASE(8)
    }
#undef HSN_FWD_CASE
    return hipErrorInvalidValue;
}

template <typename IN, typename OUT, typename SLOT>
hipError_t launch_fwd(const FwdArgs& a, SliceShape sh, size_t lds, hipStream_t st) {
    switch (sh.S) {
        case 1: return launch_fwd_s<IN, OUT, SLOT, 1>(a, sh.kpl, lds, st);
        case 4: return launch_fwd_s<IN, OUT, SLOT, 4>(a, sh.kpl, lds, st);
        case 8: return launch_fwd_s<IN, OUT, SLOT, 8>(a, sh.kpl, lds, st);
        case 16: return launch_fwd_s<IN, OUT, SLOT, 16>(a, sh.kpl, lds, st);
    }
    return hipErrorInvalidValue;
}

template <typename IN, typename SLOT, bool ACT>
hipError_t launch_bwd(const BwdArgs& a, int kpl, size_t lds, hipStream_t st) {
    const dim3 blocks = sweep_grid(a.B, a.d / a.S);
#define HSN_BWD_CASE(KP)                                                                          \
    case KP: {                                                                                    \
        auto k = bwd_sweep<IN, SLOT, ACT, KP>;                                                         \
        hipError_t e = allow_lds(k, lds);                                                         \
        if (e != hipSuccess) return e;                                                            \
        hipLaunchKernelGGL(k, blocks, dim3(kWave), lds, st, a);                             \
        return hipGetLastError();                                                                 \
    }
    switch (kpl) {
        HSN_BWD_CASE(1)
        HSN_BWD_CASE(2)
        HSN_BWD_CASE(4)
        HSN_BWD_CASE(8)
    }
#undef HSN_BWD_CASE
    return hipErrorInvalidValue;
}

}  // namespace hsn
