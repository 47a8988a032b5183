// The window's forward sweep and backward recurrence on gfx950, time-chunked, with the state
// resident in LDS.
//
// Columns. Both directions are separable over the state's d columns: the gated update
// h'[n,x] = (1-b) h[n,x] + b c touches column x only, the summary q[x] sums column x over the
// cells, and the reverse recurrence (A[n,x], R[x]) likewise (reference
// python/hsn/kernels/native.py:292-302, python/hsn/train/split.py:154-173). A workgroup owns
// (row b, a slice of S columns) and keeps that slice of the state in LDS.
//
// Time. One wavefront walking all T positions of a row leaves most of the chip idle at small
// batch (B*d/S wavefronts), so the workgroup splits the window into W chunks of Tc positions,
// one wavefront each. For a fixed chunk, each cell's state maps affinely from the chunk's start
// to its end: forward h_end = alpha h_start + beta, backward A_before = mu A_after + nu (the
// product of the (1-b) factors of the cell's updates, and the run from zero; a reset zeroes
// both). The kernel runs
//   phase A  every wavefront composes its chunk's per-cell maps in LDS (independent of the
//            start state, so all chunks run at once),
//   phase B  the workgroup walks the W maps per (cell, column) to every chunk's exact start
//            state (W steps per element, all elements in parallel),
//   phase C  every wavefront replays its chunk from its start state with the real outputs.
// The summary q needs no map: q - sum_n h[n]/N is constant between resets (q starts at q0,
// every update adds its delta / N, a reset zeroes both), so a chunk's start q follows from the
// column sums of its start state. The backward's R depends on the cotangents only, so a
// chunk-sum pre-pass gives every chunk its start R. W = 1 is the plain sequential sweep.
//
// Lanes. Lane = k*S + x: slot k of the position, column x of the slice (columns fastest), one
// slot per lane (S*K <= 64). A slot's S columns are an aligned group of lanes, so the max over
// a cell's columns reduces with DPP. Valid slots of one position name distinct cells, so no two
// lanes write one LDS word, and every LDS read of a position is issued before its writes (a
// padded slot reads cell 0 before the update, as the reference's gather does).
//
// Registers. A sub-block of TB positions of a chunk is loaded at once (every load unconditional,
// clamped into the chunk, so the compiler's wait counts are exact and the loads of all TB
// positions are in flight together) and its activations are kept in registers for the phases;
// a chunk longer than TB reloads its sub-blocks in phase C.
#pragma once

#include "common.cuh"
#include "bufio.cuh"
#include "dpp.cuh"

namespace hsn {

// The decisions of a slot as the sweeps read them: `Packed32` is one int32 per slot, the cell
// where the slot is valid and -1 where it is padded (hsn_win_route's `slots`); `Cells64` is the
// reference's pair of arrays, int64 cells and uint8 valid flags (the low word of a cell in
// [0, N) is the cell).
struct Packed32 {
    using Raw = int32_t;
};
struct Cells64 {
    using Raw = int64_t;
};

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

constexpr int kMaxChunks = 8;  // wavefronts (chunks) per workgroup

// v / N as the reference divides (an exact reciprocal product when N is a power of two)
struct DivN {
    int pow2;
    float inv, n;
    __device__ __forceinline__ float operator()(float v) const { return pow2 ? v * inv : v / n; }
    __device__ __forceinline__ double operator()(double v) const {
        return pow2 ? v * double(inv) : v / double(n);
    }
};

// Sum over the lanes with equal lane % S (a column's slot lanes).
template <int S>
__device__ __forceinline__ float col_sum(float v) {
#pragma unroll
    for (int m = S; m < kWave; m <<= 1) {
        if (m == 8) v += dpp_f32<dpp::kRor8>(v);  // xor 8 inside a 16-lane row
        else v += __shfl_xor(v, m, kWave);
    }
    return v;
}

// Zero `count` words of LDS from `p` with the wavefront (a uniform trip count).
__device__ __forceinline__ void lds_zero(float* p, int count, int lane) {
    for (int e0 = 0; e0 < count; e0 += kWave)
        if (e0 + lane < count) p[e0 + lane] = 0.0f;
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
    int B, T, N, d, K;
    int W, Tc;   // chunks per row and positions per chunk
    int region;  // LDS words per wavefront
    DivN divn;
};

// LDS words of the forward: per wavefront the state slice h [N*S] (alpha in phase A) and a
// second array (beta in phase A, the cells' max |h| in phase C), each with a dummy word; then
// the ages' last-selection table [N+1], the column-sum partials [W][W][S] and two flags per chunk.
inline int fwd_region(int N, int S, int W) {
    const int ns = N * S + 1;
    return W > 1 ? 2 * ns : ns + N + 1;
}
inline size_t fwd_lds_bytes(int N, int S, int W) {
    return 4 * (size_t(W) * fwd_region(N, S, W) + (N + 1) + size_t(W) * W * S + 2 * W);
}

template <typename IN, typename OUT, typename SLOT, int S, int TB>
__global__ __launch_bounds__(kWave* kMaxChunks) void fwd_chunk(FwdArgs a) {
    using Raw = typename SLOT::Raw;
    constexpr bool kWide = sizeof(Raw) == 8;
    extern __shared__ float lds[];
    const int lane = lane_id();
    const int gl = threadIdx.x;
    const int w = uniform(gl / kWave);
    const int W = a.W;
    const int kslot = lane / S, x = lane % S;
    int b, slice;
    block_coords(b, slice);
    const int col = slice * S + x;
    const int N = a.N, d = a.d, K = a.K, T = a.T;
    const int NS = N * S;
    const bool active = kslot < K;
    float* st = lds + w * a.region;  // alpha, then h: [NS] + a dummy word
    float* st2 = st + NS + 1;        // beta, then the cells' max |h| over the slice (as bits)
    uint32_t* cm = reinterpret_cast<uint32_t*>(st2);
    float* shared = lds + W * a.region;
    int* last = reinterpret_cast<int*>(shared);  // [N] + a dummy
    float* part = shared + N + 1;                // [W waves][W chunks][S]
    int* rflag = reinterpret_cast<int*>(part + W * W * S);
    int* rlast = rflag + W;
    const int t_begin = w * a.Tc;
    const int t_end = min(T, t_begin + a.Tc);
    const int nsb = (t_end - t_begin + TB - 1) / TB;
    const bool track_age = slice == 0 && a.age_T != nullptr;
    const bool want_max = a.h_max != nullptr;
    const DivN divn = a.divn;

    const uint32_t kd = uint32_t(K) * d;
    const uint32_t row_elems = uint32_t(T) * kd;
    const rsrc_t ry = make_rsrc(static_cast<const IN*>(a.y) + b * a.y_row, row_elems * sizeof(IN));
    const rsrc_t rg = make_rsrc(static_cast<const IN*>(a.g) + b * a.y_row, row_elems * sizeof(IN));
    const rsrc_t rc = make_rsrc(static_cast<const Raw*>(a.cells) + b * a.s_row, T * K * sizeof(Raw));
    const rsrc_t rv = make_rsrc(a.valid ? a.valid + b * a.s_row : nullptr, a.valid ? T * K : 0);
    const rsrc_t rr = make_rsrc(a.reset ? a.reset + b * a.r_row : nullptr, a.reset ? T : 0);
    // outputs: an absent one is a resource of size 0 (its stores are dropped)
    const rsrc_t rho = make_rsrc(a.h_old ? static_cast<OUT*>(a.h_old) + b * a.o_row : nullptr,
                                 a.h_old ? row_elems * sizeof(OUT) : 0);
    const rsrc_t rhs = make_rsrc(a.h_sel ? static_cast<OUT*>(a.h_sel) + b * a.o_row : nullptr,
                                 a.h_sel ? row_elems * sizeof(OUT) : 0);
    const uint32_t qbytes = uint32_t(T) * d * sizeof(OUT);
    const rsrc_t rqa = make_rsrc(a.q_pre ? static_cast<OUT*>(a.q_pre) + b * a.qo_row : nullptr,
                                 a.q_pre ? qbytes : 0);
    const rsrc_t rqb = make_rsrc(a.q_post ? static_cast<OUT*>(a.q_post) + b * a.qo_row : nullptr,
                                 a.q_post ? qbytes : 0);
    const uint32_t vy = active ? uint32_t(kslot * d + col) * sizeof(IN) : kOob;
    const uint32_t vo = active ? uint32_t(kslot * d + col) * sizeof(OUT) : kOob;
    const uint32_t vc = active ? uint32_t(kslot) * sizeof(Raw) : kOob;
    const uint32_t vv = active ? uint32_t(kslot) : kOob;
    const uint32_t vq = kslot == 0 ? uint32_t(col) * sizeof(OUT) : kOob;  // one lane per column

    if (track_age)
        for (int n0 = 0; n0 <= N; n0 += kWave * W)
            if (n0 + gl <= N) last[n0 + gl] = -1;

    // the sub-block in registers: (1 - b), b*c and the decoded cell of every position
    float omb[TB], bcv[TB];
    int cl[TB];
    uint32_t rmask = 0u;
    auto fetch = [&](int tb0) {
        const int tl = t_end - 1;
        IN yv[TB], gv[TB];
        int32_t cv[TB];
        uint8_t vb[TB];
#pragma unroll
        for (int i = 0; i < TB; ++i) {
            const int t = uniform(min(tb0 + i, tl));
            const uint32_t sy = uint32_t(t) * kd * sizeof(IN);
            yv[i] = bload<IN>(ry, vy, sy);
            gv[i] = bload<IN>(rg, vy, sy);
            cv[i] = bload<int32_t>(rc, vc, uint32_t(t) * K * sizeof(Raw));
            if constexpr (kWide) vb[i] = bload<uint8_t>(rv, vv, uint32_t(t) * K);
        }
        const bool rin = lane < TB && tb0 + lane < t_end;
        const uint8_t r = bload<uint8_t>(rr, rin ? uint32_t(lane) : kOob, uint32_t(tb0));
        rmask = static_cast<uint32_t>(ballot(r != 0));
#pragma unroll
        for (int i = 0; i < TB; ++i) {
            const float bg = fast_sigmoid(to_f32(gv[i]));
            omb[i] = 1.0f - bg;
            bcv[i] = bg * fast_tanh(to_f32(yv[i]));
            int c = cv[i];
            if constexpr (kWide) c = vb[i] ? c : -1;
            cl[i] = active ? c : -2;
        }
    };

    float q_run = a.q0[b * a.q0_row + col];
    const float* h0_row = a.h0 + b * a.h0_row;

    if (W > 1) {
        // phase A: the chunk's per-cell maps, alpha (st) and beta (st2), from the identity
        for (int e0 = 0; e0 < NS; e0 += kWave) {
            const int e = e0 + lane;
            if (e < NS) {
                st[e] = 1.0f;
                st2[e] = 0.0f;
            }
        }
        bool any_reset = false;
        for (int sb = 0; sb < nsb; ++sb) {
            const int tb0 = t_begin + sb * TB;
            const int n = min(TB, t_end - tb0);
            fetch(tb0);
#pragma unroll
            for (int i = 0; i < TB; ++i) {
                if (i < n) {
                    if ((rmask >> i) & 1u) {  // the state restarts from zero before t
                        lds_zero(st, NS, lane);
                        lds_zero(st2, NS, lane);
                        any_reset = true;
                    }
                    const int ci = cl[i];
                    const int ri = (ci > 0 ? ci : 0) * S + x;
                    const float al = st[ri], be = st2[ri];
                    const int wi = ci >= 0 ? ci * S + x : NS;
                    st[wi] = omb[i] * al;
                    st2[wi] = omb[i] * be + bcv[i];
                }
            }
        }
        if (lane == 0) rflag[w] = any_reset ? 1 : 0;
        __syncthreads();

        // phase B: every chunk's start state (into its alpha's place), and its column sums
        float ps[kMaxChunks];
#pragma unroll
        for (int j = 0; j < kMaxChunks; ++j) ps[j] = 0.0f;
        for (int e0 = 0; e0 < NS; e0 += kWave * W) {
            const int e = e0 + gl;
            if (e < NS) {
                float h = h0_row[int64_t(e / S) * d + slice * S + e % S];
#pragma unroll
                for (int j = 0; j < kMaxChunks; ++j) {
                    if (j < W) {
                        float* sj = lds + j * a.region;
                        const float al = sj[e], be = sj[NS + 1 + e];
                        sj[e] = h;
                        ps[j] += h;
                        h = al * h + be;
                    }
                }
            }
        }
#pragma unroll
        for (int j = 0; j < kMaxChunks; ++j) {
            if (j < W) {
                const float v = col_sum<S>(ps[j]);  // lanes with equal lane % S hold column x
                if (lane < S) part[(w * W + j) * S + lane] = v;
            }
        }
        __syncthreads();
        if (w > 0) {
            float cs_w = 0.0f, cs_0 = 0.0f;
            for (int wp = 0; wp < W; ++wp) {
                cs_w += part[(wp * W + w) * S + x];
                cs_0 += part[(wp * W) * S + x];
            }
            bool reset_before = false;
            for (int j = 0; j < w; ++j) reset_before |= rflag[j] != 0;
            // q - sum_n h[n] / N is constant between resets, zero after one
            q_run = (reset_before ? 0.0f : q_run - divn(cs_0)) + divn(cs_w);
        }
    } else {
        for (int e0 = 0; e0 < NS; e0 += kWave) {
            const int e = e0 + lane;
            if (e < NS) st[e] = h0_row[int64_t(e / S) * d + slice * S + e % S];
        }
    }

    // phase C: the replay with the outputs
    uint32_t M = 0u;  // the slice's max |h| (bits), the max over cm
    if (want_max) {
        for (int n0 = 0; n0 < N; n0 += kWave) {
            const int n = n0 + lane;
            if (n < N) {
                uint32_t m = 0u;
#pragma unroll
                for (int xx = 0; xx < S; ++xx) m = umax(m, abs_bits(st[n * S + xx]));
                cm[n] = m;
                M = umax(M, m);
            }
        }
        M = wave_max_from_groups<1>(M);
    }
    int lr = -1;  // the chunk's last reset
    for (int sb = 0; sb < nsb; ++sb) {
        const int tb0 = t_begin + sb * TB;
        const int n = min(TB, t_end - tb0);
        if (W == 1 || nsb > 1) fetch(tb0);
        float delta[TB];
        uint32_t hmv = 0u;
#pragma unroll
        for (int i = 0; i < TB; ++i) {
            delta[i] = 0.0f;
            if (i < n) {
                const int t = tb0 + i;
                if ((rmask >> i) & 1u) {  // a document boundary: h, q (and the ages) restart at zero
                    lds_zero(st, NS, lane);
                    if (want_max) {
                        lds_zero(st2, N, lane);
                        M = 0u;
                    }
                    lr = t;
                }
                const int ci = cl[i];
                const bool ok = ci >= 0;
                const float hold = st[(ci > 0 ? ci : 0) * S + x];
                const uint32_t mo = (want_max && ok) ? cm[ci] : 0u;
                const float hnew = omb[i] * hold + bcv[i];
                st[ok ? ci * S + x : NS] = hnew;
                const uint32_t so = uint32_t(t) * kd * sizeof(OUT);
                bstore_f32<OUT>(hold, rho, vo, so);
                float hs = hnew;
                if (ballot(ci == -1)) {  // a padded slot shows cell 0 after the update
                    const float c0 = st[x];
                    hs = ci == -1 ? c0 : hnew;
                }
                bstore_f32<OUT>(hs, rhs, vo, so);
                delta[i] = ok ? hnew - hold : 0.0f;
                if (want_max) {
                    // the cell's max over the slice's columns replaces its old one; the slice max
                    // rises with it, and is rescanned only when the cell that held it shrank
                    const uint32_t mn = group_max<S>(abs_bits(hnew));
                    if (ok && x == 0) cm[ci] = mn;
                    const bool drop = ok && mo == M && mn < M;
                    M = umax(M, wave_max_from_groups<S>(ok ? mn : 0u));
                    if (ballot(drop)) {
                        uint32_t m = 0u;
                        for (int n0 = 0; n0 < N; n0 += kWave)
                            if (n0 + lane < N) m = umax(m, cm[n0 + lane]);
                        M = wave_max_from_groups<1>(m);
                    }
                    hmv = lane == i ? M : hmv;
                }
                if (track_age && ok && x == 0) atomicMax(&last[ci], t);
            }
        }
        // the summary before and after each position: q' = q + sum_k (h' - h)[k] / N
#pragma unroll
        for (int i = 0; i < TB; ++i) {
            const float s = col_sum<S>(delta[i]);
            if (i < n) {
                if ((rmask >> i) & 1u) q_run = 0.0f;
                const uint32_t sq = uint32_t(tb0 + i) * d * sizeof(OUT);
                bstore_f32<OUT>(q_run, rqa, vq, sq);
                q_run = q_run + divn(s);
                bstore_f32<OUT>(q_run, rqb, vq, sq);
            }
        }
        if (want_max && lane < n)  // lane i sends position tb0 + i's slice max
            atomicMax(reinterpret_cast<unsigned int*>(a.h_max + b * a.hm_row) + (tb0 + lane), hmv);
    }

    // the end state (zeroed when the caller's next record resets this row)
    const bool clear = a.clear ? a.clear[b * a.c_row] != 0 : false;
    if (w == W - 1) {
        if (a.h_T) {
            float* hT_row = a.h_T + b * a.hT_row;
            for (int e0 = 0; e0 < NS; e0 += kWave) {
                const int e = e0 + lane;
                if (e < NS) hT_row[int64_t(e / S) * d + slice * S + e % S] = clear ? 0.0f : st[e];
            }
        }
        if (a.q_T && kslot == 0) a.q_T[b * a.qT_row + col] = clear ? 0.0f : q_run;
    }
    if (track_age) {
        if (lane == 0) rlast[w] = lr;
        __syncthreads();
        int last_reset = -1;
        for (int j = 0; j < W; ++j) last_reset = max(last_reset, rlast[j]);
        const int64_t* age0_row = a.age0 + b * a.a0_row;
        int64_t* ageT_row = a.age_T + b * a.aT_row;
        for (int n0 = 0; n0 < N; n0 += kWave * W) {
            const int n = n0 + gl;
            if (n < N) {
                const int ls = last[n];
                int64_t age;
                if (ls >= 0 && ls >= last_reset) age = (T - 1) - ls;
                else if (last_reset >= 0) age = T - last_reset;
                else age = age0_row[n] + T;
                ageT_row[n] = clear ? 0 : age;
            }
        }
        if (a.pos_T && gl == 0)
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
    int B, T, N, d, K;
    int W, Tc, region;
    DivN divn;
};

// LDS words of the backward: per wavefront the cotangent slice A [N*S] (mu in phase A) and, when
// chunked, nu [N*S], each with a dummy word; then the chunks' summary-cotangent sums [W][S]
// (fp64) and reset flags [W].
inline int bwd_region(int N, int S, int W) {
    const int ns = N * S + 1;
    return W > 1 ? 2 * ns : ns;
}
inline size_t bwd_lds_bytes(int N, int S, int W) {
    return 4 * (size_t(W) * bwd_region(N, S, W) + 2 * size_t(W) * S + W);
}

template <typename IN, typename SLOT, bool ACT, int S, int TB>
__global__ __launch_bounds__(kWave* kMaxChunks) void bwd_chunk(BwdArgs a) {
    using Raw = typename SLOT::Raw;
    constexpr bool kWide = sizeof(Raw) == 8;
    extern __shared__ float lds[];
    const int lane = lane_id();
    const int gl = threadIdx.x;
    const int w = uniform(gl / kWave);
    const int W = a.W;
    const int kslot = lane / S, x = lane % S;
    int b, slice;
    block_coords(b, slice);
    const int col = slice * S + x;
    const int N = a.N, d = a.d, K = a.K, T = a.T;
    const int NS = N * S;
    const bool active = kslot < K;
    float* st = lds + w * a.region;  // mu, then A: [NS] + a dummy word
    float* st2 = st + NS + 1;        // nu (chunked only)
    // [W][S]: the chunks' summary-cotangent sums (the region is an even number of words, so
    // this is 8-byte aligned); [W]: whether the chunk resets R
    double* rl = reinterpret_cast<double*>(lds + W * a.region);
    int* rf = reinterpret_cast<int*>(rl + W * S);
    const int t_begin = w * a.Tc;
    const int t_end = min(T, t_begin + a.Tc);
    const int nsb = (t_end - t_begin + TB - 1) / TB;
    const DivN divn = a.divn;

    const uint32_t kd = uint32_t(K) * d;
    const uint32_t row_bytes = uint32_t(T) * kd * sizeof(IN);
    const int64_t base = b * a.y_row;
    const rsrc_t ry = make_rsrc(static_cast<const IN*>(a.y) + base, row_bytes);
    const rsrc_t rg = make_rsrc(static_cast<const IN*>(a.g) + base, row_bytes);
    const rsrc_t rho = make_rsrc(static_cast<const IN*>(a.h_old) + base, row_bytes);
    const rsrc_t rds = make_rsrc(a.dsel ? static_cast<const IN*>(a.dsel) + base : nullptr,
                                 a.dsel ? row_bytes : 0);
    const rsrc_t rdy = make_rsrc(static_cast<IN*>(a.dy) + base, row_bytes);
    const rsrc_t rdg = make_rsrc(static_cast<IN*>(a.dg) + base, row_bytes);
    const rsrc_t rc = make_rsrc(static_cast<const Raw*>(a.cells) + b * a.s_row, T * K * sizeof(Raw));
    const rsrc_t rv = make_rsrc(a.valid ? a.valid + b * a.s_row : nullptr, a.valid ? T * K : 0);
    const rsrc_t rr = make_rsrc(a.reset + b * a.r_row, T);
    const uint32_t qbytes = uint32_t(T) * d * sizeof(IN);
    const rsrc_t rqa = make_rsrc(a.dq_pre ? static_cast<const IN*>(a.dq_pre) + b * a.q_row : nullptr,
                                 a.dq_pre ? qbytes : 0);
    const rsrc_t rqb = make_rsrc(a.dq_post ? static_cast<const IN*>(a.dq_post) + b * a.q_row : nullptr,
                                 a.dq_post ? qbytes : 0);
    const uint32_t vy = active ? uint32_t(kslot * d + col) * sizeof(IN) : kOob;
    const uint32_t vc = active ? uint32_t(kslot) * sizeof(Raw) : kOob;
    const uint32_t vv = active ? uint32_t(kslot) : kOob;
    const uint32_t vq = uint32_t(col) * sizeof(IN);  // every lane reads its column's cotangent

    // the summary cotangents of a sub-block and its reset mask
    float qa[TB], qb[TB];
    uint32_t rmask = 0u;
    auto fetch_q = [&](int tb0) {
        const int tl = t_end - 1;
#pragma unroll
        for (int i = 0; i < TB; ++i) {
            const uint32_t sq = uint32_t(uniform(min(tb0 + i, tl))) * d * sizeof(IN);
            qa[i] = to_f32(bload<IN>(rqa, vq, sq));
            qb[i] = to_f32(bload<IN>(rqb, vq, sq));
        }
        const bool rin = lane < TB && tb0 + lane < t_end;
        const uint8_t r = bload<uint8_t>(rr, rin ? uint32_t(lane) : kOob, uint32_t(tb0));
        rmask = static_cast<uint32_t>(ballot(r != 0));
    };

    // The summary cotangent R is a running sum of 2T cotangents; it is accumulated in fp64 (its
    // chunked sums would otherwise round differently from a sequential fp32 sum by about
    // sqrt(2T) ulps of its largest partial), and every position's share R/N is rounded to fp32.
    // R at the chunk's end (its later side): the end-state cotangent, then the later chunks'
    double R_in = a.dq_T ? double(a.dq_T[int64_t(b) * d + col]) : 0.0;
    double R_out = 0.0;  // R after the chunk (its position t_begin)
    if (W > 1) {
        // pre-pass: each chunk's own sum (restarted at its resets, processed latest first)
        double Rl = 0.0;
        bool hasr = false;
        for (int sb = nsb - 1; sb >= 0; --sb) {
            const int tb0 = t_begin + sb * TB;
            const int n = min(TB, t_end - tb0);
            fetch_q(tb0);
#pragma unroll
            for (int i = TB - 1; i >= 0; --i) {
                if (i < n) {
                    Rl += double(qb[i]);
                    Rl += double(qa[i]);
                    if ((rmask >> i) & 1u) {
                        Rl = 0.0;
                        hasr = true;
                    }
                }
            }
        }
        if (kslot == 0) rl[w * S + x] = Rl;
        if (lane == 0) rf[w] = hasr ? 1 : 0;
        __syncthreads();
        for (int j = W - 1; j > w; --j) R_in = (rf[j] ? 0.0 : R_in) + rl[j * S + x];
        R_out = (hasr ? 0.0 : R_in) + Rl;
    }

    // the sub-block in registers: (1 - b), the A update's constant term, dsel + share, and the
    // output factors dc = p1 g, db = p2 g (activation derivatives folded in)
    float omb[TB], e2[TB], e3[TB], p1[TB], p2[TB];
    int cl[TB];
    // positions' shares and A-update terms from the running R (latest position first)
    auto fetch_a = [&](int tb0, int n, double& R) {
        const int tl = t_end - 1;
        IN gv[TB], dv[TB];
        int32_t cv[TB];
        uint8_t vb[TB];
#pragma unroll
        for (int i = 0; i < TB; ++i) {
            const int t = uniform(min(tb0 + i, tl));
            const uint32_t sy = uint32_t(t) * kd * sizeof(IN);
            gv[i] = bload<IN>(rg, vy, sy);
            dv[i] = bload<IN>(rds, vy, sy);
            cv[i] = bload<int32_t>(rc, vc, uint32_t(t) * K * sizeof(Raw));
            if constexpr (kWide) vb[i] = bload<uint8_t>(rv, vv, uint32_t(t) * K);
        }
        fetch_q(tb0);
#pragma unroll
        for (int i = TB - 1; i >= 0; --i) {
            float share = 0.0f;
            if (i < n) {
                R += double(qb[i]);
                share = static_cast<float>(divn(R));
                R += double(qa[i]);
                if ((rmask >> i) & 1u) R = 0.0;
            }
            const float bg = ACT ? fast_sigmoid(to_f32(gv[i])) : to_f32(gv[i]);
            const float ds = to_f32(dv[i]);
            omb[i] = 1.0f - bg;
            e2[i] = omb[i] * ds - bg * share;
            e3[i] = ds + share;
            p1[i] = bg;  // the gate, until fetch_c folds the candidate in
            int c = cv[i];
            if constexpr (kWide) c = vb[i] ? c : -1;
            cl[i] = active ? c : -2;
        }
    };
    auto fetch_c = [&](int tb0) {
        const int tl = t_end - 1;
        IN yv[TB], hv[TB];
#pragma unroll
        for (int i = 0; i < TB; ++i) {
            const uint32_t sy = uint32_t(uniform(min(tb0 + i, tl))) * kd * sizeof(IN);
            yv[i] = bload<IN>(ry, vy, sy);
            hv[i] = bload<IN>(rho, vy, sy);
        }
#pragma unroll
        for (int i = 0; i < TB; ++i) {
            const float bg = p1[i];
            const float c = ACT ? fast_tanh(to_f32(yv[i])) : to_f32(yv[i]);
            const float diff = c - to_f32(hv[i]);
            if constexpr (ACT) {
                p1[i] = bg * (1.0f - c * c);         // tanh'
                p2[i] = diff * (omb[i] * bg);        // sigmoid'
            } else {
                p2[i] = diff;
            }
        }
    };

    double R = R_in;
    if (W > 1) {
        // phase A: the chunk's per-cell maps A_before = mu A_after + nu, latest position first
        for (int e0 = 0; e0 < NS; e0 += kWave) {
            const int e = e0 + lane;
            if (e < NS) {
                st[e] = 1.0f;
                st2[e] = 0.0f;
            }
        }
        for (int sb = nsb - 1; sb >= 0; --sb) {
            const int tb0 = t_begin + sb * TB;
            const int n = min(TB, t_end - tb0);
            fetch_a(tb0, n, R);
#pragma unroll
            for (int i = TB - 1; i >= 0; --i) {
                if (i < n) {
                    const int ci = cl[i];
                    const int ri = (ci > 0 ? ci : 0) * S + x;
                    const float mu = st[ri], nu = st2[ri];
                    const int wi = ci >= 0 ? ci * S + x : NS;
                    st[wi] = omb[i] * mu;
                    st2[wi] = omb[i] * nu + e2[i];
                    if ((rmask >> i) & 1u) {  // nothing before the boundary reaches past it
                        lds_zero(st, NS, lane);
                        lds_zero(st2, NS, lane);
                    }
                }
            }
        }
        __syncthreads();
        // phase B: every chunk's end cotangent (into its mu's place), latest chunk first
        const float* dhT_row = a.dh_T ? a.dh_T + int64_t(b) * N * d : nullptr;
        for (int e0 = 0; e0 < NS; e0 += kWave * W) {
            const int e = e0 + gl;
            if (e < NS) {
                float A = dhT_row ? dhT_row[int64_t(e / S) * d + slice * S + e % S] : 0.0f;
#pragma unroll
                for (int j = kMaxChunks - 1; j >= 0; --j) {
                    if (j < W) {
                        float* sj = lds + j * a.region;
                        const float mu = sj[e], nu = sj[NS + 1 + e];
                        sj[e] = A;
                        A = mu * A + nu;
                    }
                }
            }
        }
        __syncthreads();
        R = R_in;
    } else {
        const float* dhT_row = a.dh_T ? a.dh_T + int64_t(b) * N * d : nullptr;
        for (int e0 = 0; e0 < NS; e0 += kWave) {
            const int e = e0 + lane;
            if (e < NS) st[e] = dhT_row ? dhT_row[int64_t(e / S) * d + slice * S + e % S] : 0.0f;
        }
    }

    // phase C: the replay with the outputs, latest position first
    for (int sb = nsb - 1; sb >= 0; --sb) {
        const int tb0 = t_begin + sb * TB;
        const int n = min(TB, t_end - tb0);
        if (W == 1 || nsb > 1) fetch_a(tb0, n, R);
        fetch_c(tb0);
#pragma unroll
        for (int i = TB - 1; i >= 0; --i) {
            if (i < n) {
                const int ci = cl[i];
                const bool ok = ci >= 0;
                const float aold = st[(ci > 0 ? ci : 0) * S + x];
                const float gg = aold + e3[i];
                st[ok ? ci * S + x : NS] = omb[i] * aold + e2[i];
                const uint32_t so = uint32_t(tb0 + i) * kd * sizeof(IN);
                bstore_f32<IN>(ok ? p1[i] * gg : 0.0f, rdy, vy, so);
                bstore_f32<IN>(ok ? p2[i] * gg : 0.0f, rdg, vy, so);
                if ((rmask >> i) & 1u) lds_zero(st, NS, lane);
            }
        }
    }
    if (W == 1) R_out = R;

    // the carried-state gradient: A and R after position 0
    if (w == 0) {
        if (a.dh0) {
            float* dh0_row = a.dh0 + int64_t(b) * N * d;
            for (int e0 = 0; e0 < NS; e0 += kWave) {
                const int e = e0 + lane;
                if (e < NS) dh0_row[int64_t(e / S) * d + slice * S + e % S] = st[e];
            }
        }
        if (a.dq0 && kslot == 0) a.dq0[int64_t(b) * d + col] = static_cast<float>(R_out);
    }
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
// Host-side geometry
// ------------------------------------------------------------------------------------------

struct Geometry {
    int S;   // columns per wavefront (1, 2, 4, 8 or 16), S * K <= 64
    int W;   // chunks (wavefronts) per workgroup
    int Tc;  // positions per chunk
};

constexpr int64_t kLdsMax = 160 * 1024;
constexpr int64_t kTargetWaves = 2048;  // two wavefronts per SIMD of the 256-CU chip

// The widest S dividing d with one slot per lane; then as many chunks as bring the grid to
// about two wavefronts per SIMD, within the LDS. `lds_of(N, S, W)` is the kernel's LDS bytes.
template <typename F>
inline bool choose_geometry(int B, int T, int N, int d, int K, F lds_of, Geometry& g) {
    const int cand[5] = {16, 8, 4, 2, 1};
    for (int i = 0; i < 5; ++i) {
        const int S = cand[i];
        if (d % S || S * K > kWave) continue;
        if (int64_t(lds_of(N, S, 1)) > kLdsMax) continue;
        const int64_t waves = int64_t(B) * (d / S);
        int W = 1;
        while (W < kMaxChunks && W < T && waves * W < kTargetWaves &&
               int64_t(lds_of(N, S, 2 * W)) <= kLdsMax)
            W *= 2;
        if (W > T) W = T;
        const int Tc = (T + W - 1) / W;
        g.S = S;
        g.W = (T + Tc - 1) / Tc;  // no empty chunk
        g.Tc = Tc;
        return true;
    }
    return false;
}

inline DivN make_divn(int N) {
    DivN v;
    v.pow2 = (N & (N - 1)) == 0 ? 1 : 0;
    v.inv = 1.0f / static_cast<float>(N);
    v.n = static_cast<float>(N);
    return v;
}

template <typename K>
hipError_t allow_lds(K kernel, size_t lds) {
    if (lds <= 64 * 1024) return hipSuccess;
    return hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                               hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
}

template <typename IN, typename OUT, typename SLOT, int S>
hipError_t launch_fwd_s(const FwdArgs& a, size_t lds, hipStream_t st) {
    constexpr int TB = sizeof(typename SLOT::Raw) == 8 ? 16 : 32;
    auto k = fwd_chunk<IN, OUT, SLOT, S, TB>;
    hipError_t e = allow_lds(k, lds);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k, sweep_grid(a.B, a.d / S), dim3(kWave * a.W), lds, st, a);
    return hipGetLastError();
}

template <typename IN, typename OUT, typename SLOT>
hipError_t launch_fwd(const FwdArgs& a, int S, size_t lds, hipStream_t st) {
    switch (S) {
        case 1: return launch_fwd_s<IN, OUT, SLOT, 1>(a, lds, st);
        case 2: return launch_fwd_s<IN, OUT, SLOT, 2>(a, lds, st);
        case 4: return launch_fwd_s<IN, OUT, SLOT, 4>(a, lds, st);
        case 8: return launch_fwd_s<IN, OUT, SLOT, 8>(a, lds, st);
        case 16: return launch_fwd_s<IN, OUT, SLOT, 16>(a, lds, st);
    }
    return hipErrorInvalidValue;
}

template <typename IN, typename SLOT, bool ACT, int S>
hipError_t launch_bwd_s(const BwdArgs& a, size_t lds, hipStream_t st) {
    constexpr int TB = 16;
    auto k = bwd_chunk<IN, SLOT, ACT, S, TB>;
    hipError_t e = allow_lds(k, lds);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k, sweep_grid(a.B, a.d / S), dim3(kWave * a.W), lds, st, a);
    return hipGetLastError();
}

template <typename IN, typename SLOT, bool ACT>
hipError_t launch_bwd(const BwdArgs& a, int S, size_t lds, hipStream_t st) {
    switch (S) {
        case 1: return launch_bwd_s<IN, SLOT, ACT, 1>(a, lds, st);
        case 2: return launch_bwd_s<IN, SLOT, ACT, 2>(a, lds, st);
        case 4: return launch_bwd_s<IN, SLOT, ACT, 4>(a, lds, st);
        case 8: return launch_bwd_s<IN, SLOT, ACT, 8>(a, lds, st);
        case 16: return launch_bwd_s<IN, SLOT, ACT, 16>(a, lds, st);
    }
    return hipErrorInvalidValue;
}

}  // namespace hsn
