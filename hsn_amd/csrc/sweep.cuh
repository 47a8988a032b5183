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

#include <stddef.h>
#include <type_traits>

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
constexpr int kResTB = 32;     // positions per chunk held in registers (resident kernels)
constexpr int kStreamTB = 16;  // positions per streamed sub-block

// v / N as the reference divides (an exact reciprocal product when N is a power of two)
struct DivN {
    int pow2;
    float inv, n;
    __device__ __forceinline__ float operator()(float v) const { return pow2 ? v * inv : v / n; }
    __device__ __forceinline__ double operator()(double v) const {
        return pow2 ? v * double(inv) : v / double(n);
    }
};


// Sums over the lanes with equal lane % S (a column's slot lanes) of every element of an array,
// step by step across the array so the cross-lane moves of all elements are in flight together.
template <int S, int M>
__device__ __forceinline__ void col_sums(float (&v)[M]) {
#pragma unroll
    for (int m = S; m < kWave; m <<= 1) {
#pragma unroll
        for (int i = 0; i < M; ++i) {
            if (m == 8) v[i] += dpp_f32<dpp::kRor8>(v[i]);  // xor 8 inside a 16-lane row
            else if (m == 16) v[i] = sum16(v[i]);
            else if (m == 32) v[i] = sum32(v[i]);
            else v[i] += __shfl_xor(v[i], m, kWave);
        }
    }
}

// The column sums of a sub-block's per-position values, scattered: v[0..M) holds lane l's values
// of positions 0..M-1; on return v[0..P) holds the sums over the column's lanes (equal lane % S)
// of positions base .. base+P-1, P = M*S/64 (M*S >= 64). Recursive halving, from the lanes
// 32 apart down to S apart: at each step a lane keeps the lower or the upper half of its
// positions (by the step's lane bit) and adds its partner's copy of that half. The gfx950 row
// swaps exchange a pair of halves in one instruction, so the whole reduction is about as many
// instructions as positions (an all-lanes reduction of every position is S..32 steps each).
template <int S, int M>
__device__ __forceinline__ void col_scatter(float (&v)[M], int lane, int& base) {
    static_assert(M * S >= kWave, "at least one position per lane");
    base = 0;
    int c = M;
#pragma unroll
    for (int m = 32; m >= S; m >>= 1) {
        const int h = c / 2;
        const bool up = (lane & m) != 0;
#pragma unroll
        for (int i = 0; i < M / 2; ++i) {
            if (i < h) {
                const float a = v[i], b = v[h + i];
                if (m == 32 || m == 16) {
                    // the lower row's lanes end with their a and the partner's a, the upper
                    // row's with the partner's b and their b
                    const auto r = m == 32 ? __builtin_amdgcn_permlane32_swap(__float_as_uint(a),
                                                                              __float_as_uint(b),
                                                                              false, false)
                                           : __builtin_amdgcn_permlane16_swap(__float_as_uint(a),
                                                                              __float_as_uint(b),
                                                                              false, false);
                    v[i] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
                } else {
                    const float send = up ? a : b;
                    const float recv = m == 8 ? dpp_f32<dpp::kRor8>(send) : __shfl_xor(send, m, kWave);
                    v[i] = (up ? b : a) + recv;
                }
            }
        }
        base += up ? h : 0;
        c = h;
    }
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

// LDS words of the forward: per wavefront the state slice h [N*S] (alpha in phase A) with a
// dummy word, and beta [N*S] with a dummy (the cells' maxima in phase C); then the ages'
// last-selection table [N+1], the column-sum partials [W][W][S], two flags per chunk and, when
// chunked, the start state [N*S] staged for phase B.
inline int fwd_region(int N, int S, int W) {  // a multiple of 4 words: 16-byte aligned slices
    (void)W;
    const int ns = N * S + 1;
    return (2 * ns + 3) & ~3;
}
inline size_t fwd_lds_bytes(int N, int S, int W) {
    const size_t h0_stage = W > 1 ? size_t(N) * S : 0;  // the start state, for phase B
    return 4 * (size_t(W) * fwd_region(N, S, W) + (N + 1) + size_t(W) * W * S + 2 * W + h0_stage);
}

// An LDS word by byte address.
__device__ __forceinline__ float& lds_at(float* lds, uint32_t byte) {
    return *reinterpret_cast<float*>(reinterpret_cast<char*>(lds) + byte);
}

__device__ __forceinline__ uint32_t& lds_at_u(float* lds, uint32_t byte) {
    return *reinterpret_cast<uint32_t*>(reinterpret_cast<char*>(lds) + byte);
}

constexpr uint32_t kNoCell = 0xffffffffu;  // no tracked cell

// RES: the whole chunk is one register sub-block (W > 1, Tc <= TB): phase C replays what phase A
// loaded. Otherwise every phase streams its sub-blocks from memory.
// A row's state [N*S] out of LDS by the whole workgroup: element e = i*stride + t (t the thread),
// U elements a thread per pass, all read before any is stored (one LDS wait a pass).
template <int S, int U, typename Rd, typename Wr>
__device__ __forceinline__ void write_state(int NS, int t, int stride, Rd rd, Wr wr) {
    for (int e0 = t; e0 < NS; e0 += U * stride) {
        float v[U];
#pragma unroll
        for (int j = 0; j < U; ++j) {
            const int e = e0 + j * stride;
            v[j] = e < NS ? rd(e) : 0.0f;
        }
#pragma unroll
        for (int j = 0; j < U; ++j) {
            const int e = e0 + j * stride;
            if (e < NS) wr(e, v[j]);
        }
    }
}

// The wavefront maximum of each of M per-position values, scattered the same way: lane l ends
// with position l / (64/M) (64/M lanes per position, all with the same value). Halving from the
// lanes 32 apart (row swaps) down to 2*(64/M)... then a plain exchange for the last steps; the
// partners inside 8 lanes are the half-mirror and quad permutations (each pairs lanes across
// the step's bit, with the same positions so far).
template <int M>
__device__ __forceinline__ uint32_t max_scatter(uint32_t (&v)[M], int lane) {
    static_assert(M >= 1 && M <= kWave && (M & (M - 1)) == 0, "M");
    int c = M;
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        auto xchg = [&](uint32_t u) __attribute__((always_inline)) -> uint32_t {
            if (m == 8) return dpp_u32<dpp::kRor8>(u);
            if (m == 4) return dpp_u32<dpp::kHalfMirror>(u);
            if (m == 2) return dpp_u32<dpp::kXor2>(u);
            return dpp_u32<dpp::kXor1>(u);
        };
        if (c > 1) {
            const int h = c / 2;
            const bool up = (lane & m) != 0;
#pragma unroll
            for (int i = 0; i < M / 2; ++i) {
                if (i < h) {
                    const uint32_t a = v[i], b = v[h + i];
                    if (m == 32 || m == 16) {
                        const auto r = m == 32 ? __builtin_amdgcn_permlane32_swap(a, b, false, false)
                                               : __builtin_amdgcn_permlane16_swap(a, b, false, false);
                        v[i] = umax(static_cast<uint32_t>(r[0]), static_cast<uint32_t>(r[1]));
                    } else {
                        v[i] = umax(up ? b : a, xchg(up ? a : b));
                    }
                }
            }
            c = h;
        } else {
            v[0] = umax(v[0], xchg(v[0]));
        }
    }
    return v[0];
}

template <typename IN, typename OUT, typename SLOT, int S, int TB, bool RES, bool CM>
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
    float* st2 = st + NS + 1;        // beta (chunked only)
    const uint32_t rb = uint32_t(w * a.region) * 4u;  // byte address of st
    const uint32_t boff = uint32_t(NS + 1) * 4u;      // st2 - st, bytes
    const uint32_t dummy = rb + uint32_t(NS) * 4u;    // where padded and idle lanes write
    const uint32_t x0 = rb + uint32_t(x) * 4u;        // cell 0, this lane's column
    float* shared = lds + W * a.region;
    int* last = reinterpret_cast<int*>(shared);  // [N] + a dummy
    float* part = shared + N + 1;                // [W waves][W chunks][S]
    int* rflag = reinterpret_cast<int*>(part + W * W * S);
    int* rlast = rflag + W;
    float* h0s = reinterpret_cast<float*>(rlast + W);  // [NS] when chunked
    const int t_begin = w * a.Tc;
    const int t_end = min(T, t_begin + a.Tc);
    const int nsb = RES ? 1 : (t_end - t_begin + TB - 1) / TB;
    const bool track_age = slice == 0 && a.age_T != nullptr;
    const bool want_max = CM || a.h_max != nullptr;  // CM: launched only with the maxima
    const uint32_t qbytes = uint32_t(T) * d * sizeof(OUT);
    const DivN divn = a.divn;

    const uint32_t kd = uint32_t(K) * d;
    const uint32_t row_elems = uint32_t(T) * kd;
    const rsrc_t ry = make_rsrc(static_cast<const IN*>(a.y) + b * a.y_row, row_elems * sizeof(IN));
    const rsrc_t rg = make_rsrc(static_cast<const IN*>(a.g) + b * a.y_row, row_elems * sizeof(IN));
    const rsrc_t rc = make_rsrc(static_cast<const Raw*>(a.cells) + b * a.s_row, T * K * sizeof(Raw));
    const rsrc_t rv = make_rsrc(a.valid ? a.valid + b * a.s_row : nullptr, a.valid ? T * K : 0);
    const rsrc_t rr = make_rsrc(a.reset ? a.reset + b * a.r_row : nullptr, a.reset ? T : 0);
    // the outputs as resources, made where phase C starts (an absent output is a resource of
    // size 0: its stores are dropped)
    auto out_rsrc = [&](void* p, int64_t row, uint32_t bytes) __attribute__((always_inline)) {
        OUT* const q = static_cast<OUT*>(p);
        return make_rsrc(q ? q + b * row : nullptr, q ? bytes : 0u);
    };
    const uint32_t vy = active ? uint32_t(kslot * d + col) * sizeof(IN) : kOob;
    const uint32_t vo = active ? uint32_t(kslot * d + col) * sizeof(OUT) : kOob;
    const uint32_t vc = active ? uint32_t(kslot) * sizeof(Raw) : kOob;
    const uint32_t vv = active ? uint32_t(kslot) : kOob;

    if (track_age)
        for (int n0 = 0; n0 <= N; n0 += kWave * W)
            if (n0 + gl <= N) last[n0 + gl] = -1;
    // the first pass of the ages' starting values, loaded now: the ages are the kernel's last work
    const int64_t* const age0_row = track_age ? a.age0 + b * a.a0_row : nullptr;
    const int64_t age0_first = track_age && gl < N ? age0_row[gl] : 0;

    // A sub-block: the raw loads, then per position (1 - b), b*c and the LDS byte address of
    // the slot's (cell, column) word. Padded and idle lanes get the identity update (1, 0) on
    // the dummy word, so no step of the loops below tests them.
    IN yv[TB], gv[TB];
    int32_t cv[TB];
    uint8_t vb[TB];
    uint32_t rmask = 0u;
    float omb[TB], bcv[TB];
    uint32_t ca[TB];
    // the loads of position i of the sub-block at tb0, unconditional (the compiler's wait counts
    // stay exact). A position past the chunk reads data the preparation ignores; one past the
    // row is clamped to the row's last position (the soffset must stay inside the row).
    auto fetch_at = [&](int i, int tb0) __attribute__((always_inline)) {
        const int t = uniform(min(tb0 + i, T - 1));
        const uint32_t sy = uint32_t(t) * kd * sizeof(IN);
        yv[i] = bload<IN>(ry, vy, sy);
        gv[i] = bload<IN>(rg, vy, sy);
        cv[i] = bload<int32_t>(rc, vc, uint32_t(t) * K * sizeof(Raw));
        if constexpr (kWide) vb[i] = bload<uint8_t>(rv, vv, uint32_t(t) * K);
    };
    // the sub-block's resets (lane i: position tb0 + i), loaded before its other inputs and
    // turned into a bit mask of its positions after they are issued: the ballot waits for the
    // oldest load only, not for a round trip before the others go out
    uint8_t rbyte = 0;
    auto fetch_rst = [&](int tb0) __attribute__((always_inline)) {
        const bool rin = lane < TB && tb0 + lane < t_end;
        rbyte = bload<uint8_t>(rr, rin ? uint32_t(lane) : kOob, uint32_t(tb0));
    };
    auto rst_mask = [&]() __attribute__((always_inline)) {
        rmask = static_cast<uint32_t>(ballot(rbyte != 0));
    };
    auto fetch = [&](int tb0) __attribute__((always_inline)) {
        fetch_rst(tb0);
#pragma unroll
        for (int i = 0; i < TB; ++i) fetch_at(i, tb0);
        rst_mask();
    };
    // positions whose loads are in flight ahead of the one being composed in phase A
    constexpr int kAhead = kWide ? 12 : 8;
    // returns whether the lane's slot is padded (the activations are computed for every lane,
    // then selected: a conditional tanh would cost a divergent branch per position)
    auto prep = [&](int i, bool in_block) __attribute__((always_inline)) -> bool {
        int c = cv[i];
        if constexpr (kWide) c = vb[i] ? c : -1;
        const bool ok = in_block && active && c >= 0;
        const float bg = fast_sigmoid(to_f32(gv[i]));
        const float cand = fast_tanh(to_f32(yv[i]));
        const float bc = bg * cand;
        omb[i] = ok ? 1.0f - bg : 1.0f;
        bcv[i] = ok ? bc : 0.0f;
        ca[i] = ok ? rb + uint32_t(c * S + x) * 4u : dummy;
        return in_block && active && c < 0;
    };

    float q_run = a.q0[b * a.q0_row + col];
    const float* h0_row = a.h0 + b * a.h0_row;
    bool pad_lane = false;
    // The start state for phase B is staged in LDS during phase A: the first kPre elements of
    // each lane are fetched before the sub-block's loads and written after them (so waiting for
    // them waits for nothing else), the rest after phase A's first sub-block.
    constexpr int kPre = 4;
    float h0v[kPre];
    auto h0_elem = [&](int e) __attribute__((always_inline)) -> float {
        return h0_row[int64_t(e / S) * d + slice * S + e % S];
    };
    if (RES || W > 1) {
        // phase A: the chunk's per-cell maps, alpha (st) and beta (st2).
        // The loads are software-pipelined, kAhead positions ahead of the one being composed, so
        // the composition overlaps the sub-block's later loads (issuing them all first would
        // hold the wavefront at issue until most of them had returned). A reset makes what
        // came before it irrelevant to the chunk's map: the maps restart from zero at the
        // sub-block's last reset and only the positions from there are composed.
        bool any_reset = false;
        for (int sb = 0; sb < nsb; ++sb) {
            const int tb0 = t_begin + sb * TB;
            const int n = min(TB, t_end - tb0);
            fetch_rst(tb0);  // the oldest load: waiting for it waits for nothing else
            if (sb == 0) {
#pragma unroll
                for (int q = 0; q < kPre; ++q) {
                    const int e = q * kWave * W + gl;
                    h0v[q] = h0_elem(min(e, NS - 1));
                }
            }
#pragma unroll
            for (int i = 0; i < kAhead && i < TB; ++i) fetch_at(i, tb0);
            __builtin_amdgcn_sched_barrier(0);
            rst_mask();
            if (sb == 0) {
#pragma unroll
                for (int q = 0; q < kPre; ++q) {
                    const int e = q * kWave * W + gl;
                    if (e < NS) h0s[e] = h0v[q];
                }
                for (int e = kPre * kWave * W + gl; e < NS; e += kWave * W) h0s[e] = h0_elem(e);
            }
            any_reset |= rmask != 0u;
            const int start = rmask != 0u ? 31 - __builtin_clz(rmask) : 0;
            if (sb == 0 || rmask != 0u) {
                const float a0 = sb == 0 && rmask == 0u ? 1.0f : 0.0f;
                for (int e0 = 0; e0 < NS; e0 += kWave) {
                    const int e = e0 + lane;
                    if (e < NS) {
                        st[e] = a0;
                        st2[e] = 0.0f;
                    }
                }
            }
            pad_lane = false;
            auto compose = [&](auto full_c) __attribute__((always_inline)) {
                constexpr bool kFull = decltype(full_c)::value;  // n == TB: no position test
#pragma unroll
                for (int i = 0; i < TB; ++i) {
                    if (i + kAhead < TB) fetch_at(i + kAhead, tb0);
                    pad_lane |= prep(i, kFull || i < n);  // the loads of position i arrive in order
                    if (i >= start) {
                        // alpha's sign bit marks a cell written in the chunk (a plain 1 or the
                        // restart's 0 is unwritten): -(omb |alpha|), free input modifiers
                        float& al = lds_at(lds, ca[i]);
                        float& be = lds_at(lds, ca[i] + boff);
                        const float va = al, vbe = be;
                        al = -omb[i] * fabsf(va);
                        be = omb[i] * vbe + bcv[i];
                    }
                }
            };
            if (n == TB) compose(std::true_type{});
            else compose(std::false_type{});
        }
        if (lane == 0) rflag[w] = any_reset ? 1 : 0;
        __syncthreads();

        // phase B: every chunk's start state (into its alpha's place), and the summary's change
        // over each chunk. Chunk by chunk over all of the lane's elements, so each chunk's reads
        // are in flight together (a chunk's store may alias the next chunk's reads as far as the
        // compiler knows). A chunk that resets ends at beta whatever its start (a select, not
        // 0 * h: a NaN in the start state must not cross the reset, as the reference's
        // masked_fill). The summary moves only by the deltas of written cells (q' = q + sum of
        // the slots' deltas / N), so a chunk adds the sum of its written cells' end - start, or,
        // after a reset, restarts from the sum of its end state: an unwritten NaN or inf cell
        // reaches neither.
        float ps[kMaxChunks];
#pragma unroll
        for (int j = 0; j < kMaxChunks; ++j) ps[j] = 0.0f;
        for (int g0 = 0; g0 < NS; g0 += kWave * W * kPre) {  // groups of kPre elements per lane
            float h[kPre];
#pragma unroll
            for (int q = 0; q < kPre; ++q) h[q] = h0s[min(g0 + q * kWave * W + gl, NS - 1)];
#pragma unroll
            for (int j = 0; j < kMaxChunks; ++j) {
                if (j < W) {
                    float* sj = lds + j * a.region;
                    const bool rj = rflag[j] != 0;
                    float al[kPre], be[kPre];
#pragma unroll
                    for (int q = 0; q < kPre; ++q) {
                        const int e = min(g0 + q * kWave * W + gl, NS);  // NS: the dummy
                        al[q] = sj[e];
                        be[q] = sj[NS + 1 + e];
                    }
#pragma unroll
                    for (int q = 0; q < kPre; ++q) {  // past the end: the dummy word
                        const int e = g0 + q * kWave * W + gl;
                        sj[min(e, NS)] = h[q];
                        const float hn = rj ? be[q] : fabsf(al[q]) * h[q] + be[q];
                        const float dq = rj ? hn : (signbit(al[q]) ? hn - h[q] : 0.0f);
                        ps[j] += e < NS ? dq : 0.0f;
                        h[q] = hn;
                    }
                }
            }
        }
        col_sums<S>(ps);  // lanes with equal lane % S hold column x
#pragma unroll
        for (int j = 0; j < kMaxChunks; ++j)
            if (j < W && lane < S) part[(w * W + j) * S + lane] = ps[j];
        __syncthreads();
        if (w > 0) {
            float q = q_run;  // q0, then the summary at each earlier chunk's end
            for (int j = 0; j < w; ++j) {
                float cs = 0.0f;
                for (int wp = 0; wp < W; ++wp) cs += part[(wp * W + j) * S + x];
                q = (rflag[j] != 0 ? 0.0f : q) + divn(cs);
            }
            q_run = q;
        }
    } else {
        for (int e0 = 0; e0 < NS; e0 += kWave) {
            const int e = e0 + lane;
            if (e < NS) st[e] = h0_row[int64_t(e / S) * d + slice * S + e % S];
        }
    }
    if (lane == 0) st[NS] = 0.0f;  // the dummy: idle lanes read it as a zero state

    // phase C: the replay with the outputs.
    // The slice's max |h| per position (bits, NaN above +inf), two ways:
    //  CM (N <= 256): every cell's max over the slice's columns, cm[c], lives in the beta
    //     region (free in phase C) as 256 words, those past N zero. Each position writes its
    //     cells' new maxima (a DPP max over the slot's lanes, stored by the slot's first lane;
    //     the other lanes store to words of their own past the cells, so no two lanes of a store
    //     share a word) and every lane reads the cells lane, lane+64, lane+128 and lane+192
    //     (consecutive words across the lanes: no bank conflict); its maximum per position stays
    //     in a register, and one batched wavefront reduction after the steps gives every
    //     position's slice maximum. No branch, whatever the data.
    //  otherwise: M, held by the tracked cell (cw: its word in this lane's column, kNoCell when
    //     none); a position changes it only when a new value exceeds it or the tracked cell is
    //     written, and then leaves the steps for a rescan or a raise.
    uint32_t M = 0u, cw = kNoCell;
    constexpr int kLgS = S == 1 ? 0 : S == 2 ? 1 : S == 4 ? 2 : S == 8 ? 3 : 4;
    constexpr int kCmCells = 256;
    uint32_t* const cmw = reinterpret_cast<uint32_t*>(st2);  // [256] + the dummy N's + [64]
    const uint32_t cm_base = rb + boff;
    // a slot's cm word from its state word: cell c = (ca - rb) >> (2 + lg S) (the dummy gives N,
    // a cell past the real ones: its padded and idle lanes store zero there)
    const uint32_t cm_own = cm_base + uint32_t(kCmCells + 1 + lane) * 4u;
    const uint32_t cm_rd = cm_base + uint32_t(lane) * 4u;
    auto cm_init = [&]() __attribute__((always_inline)) {
        for (int c0 = 0; c0 < kCmCells; c0 += kWave) {
            const int c = c0 + lane;
            uint32_t m = 0u;
            if (c < N) {
                if constexpr (S % 4 == 0) {
#pragma unroll
                    for (int q = 0; q < S; q += 4) {
                        const float4 v = *reinterpret_cast<const float4*>(st + c * S + q);
                        m = umax(umax(m, umax(abs_bits(v.x), abs_bits(v.y))),
                                 umax(abs_bits(v.z), abs_bits(v.w)));
                    }
                } else {
#pragma unroll
                    for (int q = 0; q < S; ++q) m = umax(m, abs_bits(st[c * S + q]));
                }
            }
            cmw[c] = m;
        }
    };
    auto cm_zero = [&]() __attribute__((always_inline)) {
        for (int c0 = 0; c0 < kCmCells; c0 += kWave) cmw[c0 + lane] = 0u;
    };
    auto rescan = [&]() __attribute__((always_inline)) {  // the max and a cell holding it, over the whole slice
        constexpr int U = 8;  // reads in flight per lane (the dummy word NS reads as zero)
        uint32_t best = 0u;
        int bi = 0;
        if (NS % (kWave * 4) == 0) {  // four words per lane and read
            for (int e0 = 0; e0 < NS; e0 += kWave * 4 * U) {
                float4 v[U];
#pragma unroll
                for (int u = 0; u < U; ++u)
                    v[u] = *reinterpret_cast<const float4*>(st + min(e0 + (u * kWave + lane) * 4, NS - 4));
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    const int e = e0 + (u * kWave + lane) * 4;
                    const float c4[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
#pragma unroll
                    for (int c = 0; c < 4; ++c) {
                        const uint32_t a = e < NS ? abs_bits(c4[c]) : 0u;
                        if (a > best) {
                            best = a;
                            bi = e + c;
                        }
                    }
                }
            }
        } else {
            for (int e0 = 0; e0 < NS; e0 += kWave * U) {
                uint32_t v[U];
#pragma unroll
                for (int u = 0; u < U; ++u) v[u] = abs_bits(st[min(e0 + u * kWave + lane, NS)]);
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    if (v[u] > best) {
                        best = v[u];
                        bi = e0 + u * kWave + lane;
                    }
                }
            }
        }
        M = wave_max_from_groups<1>(best);
        const uint64_t who = ballot(best == M);
        const int src = __builtin_ctzll(who);
        const int e_max = __builtin_amdgcn_readlane(bi, src);
        cw = M == 0u ? kNoCell : rb + uint32_t((e_max / S) * S + x) * 4u;
    };
    auto raise = [&](uint32_t av, uint32_t cai) __attribute__((always_inline)) {  // new values above M, none on the tracked cell
        const uint32_t m = wave_max_from_groups<1>(av > M ? av : 0u);
        const uint64_t who = ballot(av == m);
        const int src = __builtin_ctzll(who);
        const uint32_t cell_x = static_cast<uint32_t>(__builtin_amdgcn_readlane(
                                    static_cast<int>(cai), src)) - uint32_t(src % S) * 4u;
        M = m;
        cw = cell_x + uint32_t(x) * 4u;
    };
    if constexpr (CM) cm_init();
    else if (want_max) rescan();

    int lr = -1;  // the chunk's last reset
    const rsrc_t rho = out_rsrc(a.h_old, a.o_row, row_elems * sizeof(OUT));
    const rsrc_t rhs = out_rsrc(a.h_sel, a.o_row, row_elems * sizeof(OUT));
    const rsrc_t rqa = out_rsrc(a.q_pre, a.qo_row, qbytes);
    const rsrc_t rqb = out_rsrc(a.q_post, a.qo_row, qbytes);
    // One sub-block of phase C: the steps, then the summaries, the slice maxima and the cells'
    // last selections.
    //
    // The steps run straight through the unrolled positions. A position that needs more than the
    // update (a reset before it, a change of the tracked maximum after it) leaves the unrolled
    // code for the one handler after it, which re-enters at the next position to do. The rare
    // work is compiled once instead of once per position, so the hot path is contiguous code
    // (an inlined copy per position put a jump over cold code, and an instruction-cache miss,
    // into every step).
    auto block = [&](int tb0, int n) __attribute__((always_inline)) {
        const bool pad = ballot(pad_lane) != 0u;
        float delta[TB];
        uint32_t lmv[TB];  // CM: this lane's cells' maximum after each position
#pragma unroll
        for (int i = 0; i < TB; ++i) {
            delta[i] = 0.0f;
            lmv[i] = 0u;
        }
        uint32_t hmv = 0u;
        const uint32_t live = n >= 32 ? 0xffffffffu : (1u << n) - 1u;
        const uint32_t so0 = uint32_t(tb0) * kd * sizeof(OUT);
        const uint32_t sstep = kd * sizeof(OUT);
        auto steps = [&](auto pad_c) __attribute__((always_inline)) {
            constexpr bool kPad = decltype(pad_c)::value;
            uint32_t todo = live;
            uint32_t rpend = rmask & live;  // resets not applied yet
            for (;;) {
                int ev = -1;
                bool ev_reset = false;
                uint32_t ev_av = 0u, ev_ca = 0u;
#pragma unroll
                for (int i = 0; i < TB; ++i) {
                    if ((todo >> i) & 1u) {
                        if (unlikely((rpend >> i) & 1u)) {  // a boundary before position i
                            ev = i;
                            ev_reset = true;
                            break;
                        }
                        const bool ok = !kPad || ca[i] != dummy;
                        const float hold = lds_at(lds, kPad && !ok ? x0 : ca[i]);
                        const float hnew = omb[i] * hold + bcv[i];
                        lds_at(lds, ca[i]) = kPad && !ok ? 0.0f : hnew;
                        const uint32_t so = so0 + uint32_t(i) * sstep;
                        bstore_f32<OUT>(hold, rho, vo, so);
                        float hs = hnew;
                        if (kPad) {  // a padded slot shows cell 0 after the update
                            const float c0 = lds_at(lds, x0);
                            hs = ok ? hnew : c0;
                        }
                        bstore_f32<OUT>(hs, rhs, vo, so);
                        delta[i] = kPad && !ok ? 0.0f : hnew - hold;
                        if constexpr (CM) {
                            const uint32_t av = kPad && !ok ? 0u : abs_bits(hnew);
                            const uint32_t cma = x == 0 ? cm_base + (((ca[i] - rb) >> (2 + kLgS)) << 2) : cm_own;
                            lds_at_u(lds, cma) = group_max<S>(av);
                            const uint32_t m0 = lds_at_u(lds, cm_rd), m1 = lds_at_u(lds, cm_rd + 256u);
                            const uint32_t m2 = lds_at_u(lds, cm_rd + 512u), m3 = lds_at_u(lds, cm_rd + 768u);
                            lmv[i] = umax(umax(m0, m1), umax(m2, m3));
                        } else if (want_max) {
                            const uint32_t av = kPad && !ok ? 0u : abs_bits(hnew);
                            if (unlikely(ballot(av > M || ca[i] == cw) != 0u)) {
                                ev = i;
                                ev_av = av;
                                ev_ca = ca[i];
                                break;
                            }
                            hmv = lane == i ? M : hmv;
                        }
                    }
                }
                if (ev < 0) break;
                if (ev_reset) {  // h, q and ages restart; position ev runs next
                    lds_zero(st, NS, lane);
                    if constexpr (CM) cm_zero();
                    M = 0u;
                    cw = kNoCell;
                    lr = tb0 + ev;
                    rpend &= ~(1u << ev);
                    todo = live & ~((1u << ev) - 1u);
                } else {  // position ev is done but for its maximum
                    if (ballot(ev_ca == cw)) rescan();  // the tracked cell changed
                    else raise(ev_av, ev_ca);
                    hmv = lane == ev ? M : hmv;
                    todo = live & ~((2u << ev) - 1u);
                }
            }
        };
        if (pad) steps(std::true_type{});
        else steps(std::false_type{});
        // CM: every position's slice maximum, lane l holding position l / (64 / TB)'s
        if constexpr (CM) hmv = max_scatter<TB>(lmv, lane);

        // the summary before and after each position: q' = q + sum_k (h' - h)[k] / N
        if constexpr (TB * S >= kWave) {
            // scattered: lane (g, x) = (lane / S, lane % S) sums, and stores, positions
            // base .. base+kP-1 of column x (a full-width store per kP positions instead of a
            // column's eight lanes per position). A run of positions maps q to (rs ? 0 : q) + c
            // (a reset zeroes q before its position); a scan over the groups, earlier first,
            // gives each lane the map of the positions before its own.
            constexpr int kP = TB * S / kWave;
            constexpr int kG = kWave / S;
            int base;
            col_scatter<S, TB>(delta, lane, base);
            float ctb[kP];
            if (divn.pow2) {
#pragma unroll
                for (int j = 0; j < kP; ++j) ctb[j] = delta[j] * divn.inv;
            } else {
#pragma unroll
                for (int j = 0; j < kP; ++j) ctb[j] = delta[j] / divn.n;
            }
            bool rs = false;
            float c = 0.0f;
#pragma unroll
            for (int j = 0; j < kP; ++j) {
                const int i = base + j;
                if (i < n) {
                    if ((rmask >> i) & 1u) {
                        c = 0.0f;
                        rs = true;
                    }
                    c += ctb[j];
                }
            }
            const int g = lane / S;
#pragma unroll
            for (int k = 1; k < kG; k <<= 1) {  // inclusive over the groups 0..g
                const float ce = __shfl_up(c, k * S, kWave);
                const int re = __shfl_up(rs ? 1 : 0, k * S, kWave);
                if (g >= k) {
                    c = rs ? c : ce + c;
                    rs = rs || re != 0;
                }
            }
            float cx = __shfl_up(c, S, kWave);
            int rx = __shfl_up(rs ? 1 : 0, S, kWave);
            if (g == 0) {
                cx = 0.0f;
                rx = 0;
            }
            const float c_all = __shfl(c, (kG - 1) * S + x, kWave);
            const bool rs_all = __shfl(rs ? 1 : 0, (kG - 1) * S + x, kWave) != 0;
            float q = (rx ? 0.0f : q_run) + cx;
            const uint32_t qstep = uint32_t(d) * sizeof(OUT);
            const uint32_t sq = uint32_t(tb0) * qstep;
#pragma unroll
            for (int j = 0; j < kP; ++j) {
                const int i = base + j;
                const uint32_t vq = i < n ? uint32_t(i) * qstep + uint32_t(col) * sizeof(OUT) : kOob;
                if (i < n && ((rmask >> i) & 1u)) q = 0.0f;
                bstore_f32<OUT>(q, rqa, vq, sq);
                q = i < n ? q + ctb[j] : q;
                bstore_f32<OUT>(q, rqb, vq, sq);
            }
            q_run = (rs_all ? 0.0f : q_run) + c_all;
        } else {
        col_sums<S>(delta);
        auto summaries = [&](auto pow2_c, auto reset_c) __attribute__((always_inline)) {
            constexpr bool kPow2 = decltype(pow2_c)::value;
            constexpr bool kReset = decltype(reset_c)::value;
            const uint32_t qstep = uint32_t(d) * sizeof(OUT);
            uint32_t vqt = uint32_t(col) * sizeof(OUT) + uint32_t(tb0) * qstep;
#pragma unroll
            for (int i = 0; i < TB; ++i, vqt += qstep) {
                if (i < n) {
                    if (kReset && ((rmask >> i) & 1u)) q_run = 0.0f;
                    bstore_f32<OUT>(q_run, rqa, vqt, 0u);
                    q_run = q_run + (kPow2 ? delta[i] * divn.inv : delta[i] / divn.n);
                    bstore_f32<OUT>(q_run, rqb, vqt, 0u);
                }
            }
        };
        if (kslot == 0) {
            if (divn.pow2 && rmask == 0u) summaries(std::true_type{}, std::false_type{});
            else if (divn.pow2) summaries(std::true_type{}, std::true_type{});
            else summaries(std::false_type{}, std::true_type{});
        }
        }
        if constexpr (CM) {  // the first lane of each position's group sends its slice max
            constexpr int kDup = kWave / TB;
            const int pos = lane / kDup;
            if (lane % kDup == 0 && pos < n)
                atomicMax(reinterpret_cast<unsigned int*>(a.h_max + b * a.hm_row) + (tb0 + pos),
                          hmv);
        } else if (want_max && lane < n) {  // lane i sends position tb0 + i's slice max
            atomicMax(reinterpret_cast<unsigned int*>(a.h_max + b * a.hm_row) + (tb0 + lane),
                      hmv);
        }
        if (track_age && x == 0) {  // the cells' last selection (idle and padded: the dummy N)
#pragma unroll
            for (int i = 0; i < TB; ++i)
                if (i < n) atomicMax(&last[(ca[i] - rb) / (4u * S)], tb0 + i);
        }
    };
    if constexpr (RES) {
        block(t_begin, t_end - t_begin);  // the chunk is in registers since phase A
    } else {
        for (int sb = 0; sb < nsb; ++sb) {
            const int tb0 = t_begin + sb * TB;
            const int n = min(TB, t_end - tb0);
            fetch(tb0);
            pad_lane = false;
#pragma unroll
            for (int i = 0; i < TB; ++i) pad_lane |= prep(i, i < n);
            block(tb0, n);
        }
    }

    // the end state (zeroed when the caller's next record resets this row). h is the last
    // chunk's state, in wave W-1's region; every wavefront writes a share of it (wave W-1 alone,
    // an LDS wait per store, made the kernel's tail).
    const uint8_t* const clear_p = a.clear;
    const bool clear = clear_p ? clear_p[b * a.c_row] != 0 : false;
    float* const hT = a.h_T;
    if (hT || track_age) {  // uniform in the workgroup
        if (track_age && lane == 0) rlast[w] = lr;
        __syncthreads();
    }
    if (hT) {
        const float* const stl = lds + (W - 1) * a.region;
        float* const hT_row = hT + b * a.hT_row;
        write_state<S, 4>(NS, gl, kWave * W, [&](int e) __attribute__((always_inline)) {
            return clear ? 0.0f : stl[e];
        }, [&](int e, float v) __attribute__((always_inline)) {
            hT_row[int64_t(e / S) * d + slice * S + e % S] = v;
        });
    }
    float* const qT = a.q_T;
    if (w == W - 1 && qT && kslot == 0) qT[b * a.qT_row + col] = clear ? 0.0f : q_run;
    if (track_age) {
        int last_reset = -1;
        for (int j = 0; j < W; ++j) last_reset = max(last_reset, rlast[j]);
        int64_t* ageT_row = a.age_T + b * a.aT_row;
        for (int n0 = 0; n0 < N; n0 += kWave * W) {
            const int n = n0 + gl;
            if (n < N) {
                const int ls = last[n];
                const int64_t a0 = n0 == 0 ? age0_first : age0_row[n];
                int64_t age;
                if (ls >= 0 && ls >= last_reset) age = (T - 1) - ls;
                else if (last_reset >= 0) age = T - last_reset;
                else age = a0 + T;
                ageT_row[n] = clear ? 0 : age;
            }
        }
        int64_t* const posT = a.pos_T;
        if (posT && gl == 0) posT[b] = last_reset >= 0 ? int64_t(T - last_reset) : a.pos0[b] + T;
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

// LDS words of the backward: per wavefront the cotangent slice A [N*S] (mu in phase A) with a
// dummy word, and nu [N*S] with a dummy (the cells' tags in phase C); then the chunks'
// summary-cotangent sums [W][S] (fp64), reset flags [W], per wavefront the shares of a sub-block
// [S][TB] and, when chunked, the end cotangent [N*S] staged for phase B.
inline int bwd_region(int N, int S, int W) {  // a multiple of 4 words
    (void)W;  // phase C keeps the cells' tags in the nu region, chunked or not
    const int ns = N * S + 1;
    return (2 * ns + 3) & ~3;
}
inline size_t bwd_lds_bytes(int N, int S, int W) {
    const size_t dh_stage = W > 1 ? size_t(N) * S : 0;  // the end cotangent, for phase B
    return 4 * (size_t(W) * bwd_region(N, S, W) + 2 * size_t(W) * S + W + size_t(W) * S * kResTB +
                dh_stage) + 8;
}

// RES: as the forward's (the whole chunk is one register sub-block, W > 1).
template <typename IN, typename SLOT, bool ACT, int S, int TB, bool RES>
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
    const uint32_t rb = uint32_t(w * a.region) * 4u;
    const uint32_t boff = uint32_t(NS + 1) * 4u;
    const uint32_t dummy = rb + uint32_t(NS) * 4u;
    // [W][S]: the chunks' summary-cotangent sums, 8-byte aligned; [W]: whether a chunk resets R
    const uint32_t rl_word = (uint32_t(W * a.region) + 1u) & ~1u;
    double* rl = reinterpret_cast<double*>(lds + rl_word);
    int* rf = reinterpret_cast<int*>(rl + W * S);
    float* shl = reinterpret_cast<float*>(rf + W) + w * S * TB + x * TB;  // this column's shares
    float* dhs = reinterpret_cast<float*>(rf + W) + W * S * kResTB;       // [NS] when chunked
    const int t_begin = w * a.Tc;
    const int t_end = min(T, t_begin + a.Tc);
    const int nsb = RES ? 1 : (t_end - t_begin + TB - 1) / TB;
    const DivN divn = a.divn;

    const uint32_t kd = uint32_t(K) * d;
    const uint32_t row_bytes = uint32_t(T) * kd * sizeof(IN);
    const int64_t base = b * a.y_row;
    const rsrc_t ry = make_rsrc(static_cast<const IN*>(a.y) + base, row_bytes);
    const rsrc_t rg = make_rsrc(static_cast<const IN*>(a.g) + base, row_bytes);
    const rsrc_t rho = make_rsrc(static_cast<const IN*>(a.h_old) + base, row_bytes);
    const rsrc_t rds = make_rsrc(a.dsel ? static_cast<const IN*>(a.dsel) + base : nullptr,
                                 a.dsel ? row_bytes : 0);
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

    // raw loads of a sub-block. The summary cotangents are transposed: lane (g, x) = (lane / S,
    // lane % S) holds positions g*kQP .. g*kQP + kQP - 1 of column x, so a sub-block takes
    // 2*kQP loads instead of one per position at every slot (the same column's value, eight times
    // over at S = 8, and enough loads to fill a wavefront's 63 in flight with phase A's prologue).
    constexpr int kQG = kWave / S;                               // position groups
    constexpr int kQP = TB * S >= kWave ? TB * S / kWave : 1;    // positions per group
    const int qg = lane / S;
    float qa[kQP], qb[kQP];
    IN gv[TB], dv[TB], yv[TB], hv[TB];
    int32_t cv[TB];
    uint8_t vb[TB];
    uint32_t rmask = 0u;
    // the summary cotangents and the resets (lane i: position tb0 + i; loaded first, turned into
    // a bit mask of the positions by rst_mask once the sub-block's other loads are issued)
    uint8_t rbyte = 0;
    auto fetch_q = [&](int tb0) __attribute__((always_inline)) {
        const bool rin = lane < TB && tb0 + lane < t_end;
        rbyte = bload<uint8_t>(rr, rin ? uint32_t(lane) : kOob, uint32_t(tb0));
        const uint32_t sq = uint32_t(tb0) * d * sizeof(IN);
#pragma unroll
        for (int j = 0; j < kQP; ++j) {  // past the row: masked by the lane offset (reads 0)
            const int i = qg * kQP + j;
            const uint32_t v = i < TB && tb0 + i < a.T ? uint32_t(i * d + col) * sizeof(IN) : kOob;
            qa[j] = to_f32(bload<IN>(rqa, v, sq));
            qb[j] = to_f32(bload<IN>(rqb, v, sq));
        }
    };
    auto rst_mask = [&]() __attribute__((always_inline)) {
        rmask = static_cast<uint32_t>(ballot(rbyte != 0));
    };
    // the gate, the selection cotangent and the decision of position i of the sub-block at tb0
    auto fetch_a_at = [&](int i, int tb0) __attribute__((always_inline)) {
        const int t = uniform(min(tb0 + i, t_end - 1));
        const uint32_t sy = uint32_t(t) * kd * sizeof(IN);
        gv[i] = bload<IN>(rg, vy, sy);
        dv[i] = bload<IN>(rds, vy, sy);
        cv[i] = bload<int32_t>(rc, vc, uint32_t(t) * K * sizeof(Raw));
        if constexpr (kWide) vb[i] = bload<uint8_t>(rv, vv, uint32_t(t) * K);
    };
    // the candidate and the gathered old state of positions [lo, hi) of the sub-block, latest
    // position first (phase C's order)
    auto fetch_c_at = [&](int i, int tb0) __attribute__((always_inline)) {
        const uint32_t sy = uint32_t(uniform(min(tb0 + i, t_end - 1))) * kd * sizeof(IN);
        yv[i] = bload<IN>(ry, vy, sy);
        hv[i] = bload<IN>(rho, vy, sy);
    };
    auto fetch_c = [&](int tb0, int lo = 0, int hi = TB) __attribute__((always_inline)) {
#pragma unroll
        for (int i = TB - 1; i >= 0; --i)
            if (i >= lo && i < hi) fetch_c_at(i, tb0);
    };
    // positions whose loads are in flight ahead of the one being composed in phase A (fewer than
    // the forward's: this kernel keeps more per position in registers)
    constexpr int kAhead = kWide ? 8 : 12;

    // The summary cotangent R is a running sum of 2T cotangents, latest position first: R += qb,
    // the position's share is R/N, R += qa, and a reset zeroes R. It is accumulated in fp64 (its
    // chunked sums would otherwise round differently from a sequential fp32 sum by about
    // sqrt(2T) ulps of its largest partial), and every share is rounded to fp32.
    // A run of positions maps R to (rs ? 0 : R) + c. Each lane composes its own positions' map,
    // and a scan over the position groups (later groups first: shuffles of the column's lanes)
    // gives every lane the map of the positions after its own. The running sum is a few
    // dependent adds instead of one per position.
    auto lane_map = [&](int n, bool& rs, double& c) __attribute__((always_inline)) {
        rs = false;
        c = 0.0;
#pragma unroll
        for (int j = kQP - 1; j >= 0; --j) {
            const int i = qg * kQP + j;
            if (i < n) {
                c += double(qb[j]);
                c += double(qa[j]);
                if ((rmask >> i) & 1u) {
                    c = 0.0;
                    rs = true;
                }
            }
        }
    };
    // inclusive: the map of the groups g .. kQG-1 (applied latest first)
    auto scan_maps = [&](bool& rs, double& c) __attribute__((always_inline)) {
#pragma unroll
        for (int k = 1; k < kQG; k <<= 1) {
            const double cu = __shfl_down(c, k * S, kWave);
            const int ru = __shfl_down(rs ? 1 : 0, k * S, kWave);
            if (qg + k < kQG) {
                c = rs ? c : cu + c;
                rs = rs || ru != 0;
            }
        }
    };
    // the column's whole run (group 0's inclusive map), in every lane of the column
    auto run_map = [&](bool rs, double c, bool& rs0, double& c0) __attribute__((always_inline)) {
        c0 = __shfl(c, x, kWave);
        rs0 = __shfl(rs ? 1 : 0, x, kWave) != 0;
    };
    // the sub-block's shares into LDS (shl: this column's [TB]), and R carried past it
    auto shares = [&](int n, double& R) __attribute__((always_inline)) {
        bool rs;
        double c;
        lane_map(n, rs, c);
        scan_maps(rs, c);
        bool rs0;
        double c0;
        run_map(rs, c, rs0, c0);
        // exclusive: the map of the groups after this one
        double ce = __shfl_down(c, S, kWave);
        int re = __shfl_down(rs ? 1 : 0, S, kWave);
        if (qg + 1 >= kQG) {
            ce = 0.0;
            re = 0;
        }
        double Rg = (re ? 0.0 : R) + ce;
        const double inv = double(divn.inv), nf = double(divn.n);
        auto run = [&](auto pow2_c) __attribute__((always_inline)) {
            constexpr bool kPow2 = decltype(pow2_c)::value;
#pragma unroll
            for (int j = kQP - 1; j >= 0; --j) {
                const int i = qg * kQP + j;
                float sh = 0.0f;
                if (i < n) {
                    Rg += double(qb[j]);
                    sh = static_cast<float>(kPow2 ? Rg * inv : Rg / nf);
                    Rg += double(qa[j]);
                    if ((rmask >> i) & 1u) Rg = 0.0;
                }
                if (i < TB) shl[i] = sh;
            }
        };
        if (divn.pow2) run(std::true_type{});
        else run(std::false_type{});
        R = (rs0 ? 0.0 : R) + c0;
    };
    // per position: (1 - b), the selection cotangent and the LDS byte address of the slot's word.
    // Padded and idle lanes get the identity update (1, no cotangent) on the dummy word.
    float omb[TB], dsv[TB];
    uint32_t ca[TB];
    auto prep = [&](int i, bool in_block) __attribute__((always_inline)) -> bool {
        int c = cv[i];
        if constexpr (kWide) c = vb[i] ? c : -1;
        const bool ok = in_block && active && c >= 0;
        const float bg = ACT ? fast_sigmoid(to_f32(gv[i])) : to_f32(gv[i]);
        omb[i] = ok ? 1.0f - bg : 1.0f;
        dsv[i] = ok ? to_f32(dv[i]) : 0.0f;
        ca[i] = ok ? rb + uint32_t(c * S + x) * 4u : dummy;
        return in_block && active && c < 0;
    };

    // The end cotangent for phase B is staged in LDS during the pre-pass (the first kPre elements
    // of each lane fetched before the pre-pass's loads and written after them).
    const float* dhT_row = a.dh_T ? a.dh_T + int64_t(b) * N * d : nullptr;
    constexpr int kPre = 4;
    auto dh_elem = [&](int e) __attribute__((always_inline)) -> float {
        return dhT_row ? dhT_row[int64_t(e / S) * d + slice * S + e % S] : 0.0f;
    };

    // R at the chunk's end (its later side): the end-state cotangent, then the later chunks'
    double R_in = a.dq_T ? double(a.dq_T[int64_t(b) * d + col]) : 0.0;
    double R_out = 0.0;  // R after the chunk (its position t_begin)
    bool pad_lane = false;
    if (RES || W > 1) {
        // pre-pass: each chunk's own sum (restarted at its resets, latest position first). The
        // first kAhead positions of phase A (resident kernels) are fetched with it, so their
        // loads are in flight through the pre-pass and its barrier.
        double Rl = 0.0;
        bool hasr = false;
        float dhv[kPre];
        for (int sb = nsb - 1; sb >= 0; --sb) {
            const int tb0 = t_begin + sb * TB;
            const int n = min(TB, t_end - tb0);
            fetch_q(tb0);
            if (sb == nsb - 1) {
#pragma unroll
                for (int q = 0; q < kPre; ++q) {
                    const int e = q * kWave * W + gl;
                    dhv[q] = dh_elem(min(e, NS - 1));
                }
            }
            if (RES) {
#pragma unroll
                for (int i = TB - 1; i >= TB - kAhead && i >= 0; --i) fetch_a_at(i, tb0);
            }
            __builtin_amdgcn_sched_barrier(0);
            rst_mask();
            bool rs, rs0;
            double c, c0;
            lane_map(n, rs, c);
            scan_maps(rs, c);
            run_map(rs, c, rs0, c0);
            Rl = (rs0 ? 0.0 : Rl) + c0;
            hasr = hasr || rs0;
        }
        if (kslot == 0) rl[w * S + x] = Rl;
        if (lane == 0) rf[w] = hasr ? 1 : 0;
#pragma unroll
        for (int q = 0; q < kPre; ++q) {
            const int e = q * kWave * W + gl;
            if (e < NS) dhs[e] = dhv[q];
        }
        for (int e = kPre * kWave * W + gl; e < NS; e += kWave * W) dhs[e] = dh_elem(e);
        __syncthreads();
        for (int j = W - 1; j > w; --j) R_in = (rf[j] ? 0.0 : R_in) + rl[j * S + x];
        R_out = (hasr ? 0.0 : R_in) + Rl;
        // phase A: the chunk's per-cell maps A_before = mu A_after + nu, latest position first,
        // the loads kAhead positions ahead. A reset at t cuts what comes after it from what comes
        // before: the maps restart from zero at the sub-block's earliest reset, and only the
        // positions before it are composed (the later ones are still prepared for phase C).
        double R = R_in;
        for (int sb = nsb - 1; sb >= 0; --sb) {
            const int tb0 = t_begin + sb * TB;
            const int n = min(TB, t_end - tb0);
            if (!RES) {
                fetch_q(tb0);
#pragma unroll
                for (int i = TB - 1; i >= TB - kAhead && i >= 0; --i) fetch_a_at(i, tb0);
                rst_mask();
            }
            shares(n, R);  // phase A reads them back from LDS (registers are scarce here)
            __builtin_amdgcn_wave_barrier();
            const int stop = rmask != 0u ? __builtin_ctz(rmask) : TB;  // compose positions < stop
            if (sb == nsb - 1 || rmask != 0u) {
                const float m0 = sb == nsb - 1 && rmask == 0u ? 1.0f : 0.0f;
                for (int e0 = 0; e0 < NS; e0 += kWave) {
                    const int e = e0 + lane;
                    if (e < NS) {
                        st[e] = m0;
                        st2[e] = 0.0f;
                    }
                }
            }
            pad_lane = false;
#pragma unroll
            for (int i = TB - 1; i >= 0; --i) {
                if (i - kAhead >= 0) fetch_a_at(i - kAhead, tb0);
                // RES: the last kAhead steps have no loads of their own left to issue; the
                // replay's latest inputs go out there instead (through the barrier and phase B)
                else if (RES && TB - kAhead + i >= TB / 2) fetch_c_at(TB - kAhead + i, tb0);
                pad_lane |= prep(i, i < n);  // the loads of position i arrive in order
                if (i < stop) {
                    float& mu = lds_at(lds, ca[i]);
                    float& nu = lds_at(lds, ca[i] + boff);
                    const float vm = mu, vn = nu;
                    mu = omb[i] * vm;
                    nu = omb[i] * (vn + dsv[i]) - (1.0f - omb[i]) * shl[i];
                }
            }
        }
        if (RES) {  // the rest of the replay's first inputs, in flight during phase B (the
                    // earlier half after it: registers)
            __builtin_amdgcn_sched_barrier(0);
            fetch_c(t_begin, TB / 2, TB - kAhead);
        }
        __syncthreads();
        // phase B: every chunk's end cotangent (into its mu's place), latest chunk first, chunk
        // by chunk over all of the lane's elements
        for (int g0 = 0; g0 < NS; g0 += kWave * W * kPre) {  // groups of kPre elements per lane
            float A[kPre];
#pragma unroll
            for (int q = 0; q < kPre; ++q) A[q] = dhs[min(g0 + q * kWave * W + gl, NS - 1)];
#pragma unroll
            for (int j = kMaxChunks - 1; j >= 0; --j) {
                if (j < W) {
                    float* sj = lds + j * a.region;
                    float mu[kPre], nu[kPre];
#pragma unroll
                    for (int q = 0; q < kPre; ++q) {
                        const int e = min(g0 + q * kWave * W + gl, NS);  // NS: the dummy
                        mu[q] = sj[e];
                        nu[q] = sj[NS + 1 + e];
                    }
                    const bool rj = rf[j] != 0;  // a reset in the chunk: A before it is nu
#pragma unroll
                    for (int q = 0; q < kPre; ++q) {  // past the end: the dummy word
                        const int e = g0 + q * kWave * W + gl;
                        sj[min(e, NS)] = A[q];
                        A[q] = rj ? nu[q] : mu[q] * A[q] + nu[q];  // a select: no 0 * NaN
                    }
                }
            }
        }
        // the replay's later inputs, issued before the barrier: a stall at issue (the earlier
        // half is still in flight) then overlaps the wait for the other chunks
        if constexpr (RES) fetch_c(t_begin, 0, TB / 2);
        __syncthreads();
    } else {
        for (int e0 = 0; e0 < NS; e0 += kWave) {
            const int e = e0 + lane;
            if (e < NS) st[e] = dh_elem(e);
        }
    }
    if (lane == 0) st[NS] = 0.0f;  // the dummy: idle lanes read it as a zero cotangent

    // phase C: the replay with the outputs, latest position first
    const rsrc_t rdy = make_rsrc(static_cast<IN*>(a.dy) + base, row_bytes);
    const rsrc_t rdg = make_rsrc(static_cast<IN*>(a.dg) + base, row_bytes);
    // Resets without a branch: every cell's word in the (now free) nu region tags the position
    // of its last update in this replay (the chunk's start state: t_end), and rcur is the
    // latest reset passed (positions run latest first; t_end + 1: none yet). A reset at t zeroes
    // the cotangent of every cell after position t is replayed, so a cell's value counts only
    // if it was updated after the latest reset passed: tag < rcur, else it reads as zero.
    int* const tagw = reinterpret_cast<int*>(st2);
    const uint32_t tag_base = rb + boff;
    constexpr int kLgS = S == 1 ? 0 : S == 2 ? 1 : S == 4 ? 2 : S == 8 ? 3 : 4;
    for (int c0 = 0; c0 <= N; c0 += kWave)
        if (c0 + lane <= N) tagw[c0 + lane] = t_end;
    int rcur = t_end + 1;
    // One sub-block of phase C, straight through the positions (no branch: the registers of a
    // position are free once it is replayed).
    auto block = [&](int tb0, int n) __attribute__((always_inline)) {
        const bool pad = ballot(pad_lane) != 0u;
        auto steps = [&](auto pad_c) __attribute__((always_inline)) {
            constexpr bool kPad = decltype(pad_c)::value;
#pragma unroll
            for (int i = TB - 1; i >= 0; --i) {
                if (i < n) {
                    const int t = tb0 + i;
                    // the slot's cell's tag (the dummy's for padded and idle lanes: cell N)
                    const uint32_t ta = tag_base + (((ca[i] - rb) >> (2 + kLgS)) << 2);
                    float& Aref = lds_at(lds, ca[i]);
                    const float Ar = Aref;
                    const int tg = *reinterpret_cast<const int*>(reinterpret_cast<const char*>(lds) + ta);
                    const float A = tg < rcur ? Ar : 0.0f;
                    const float share = shl[i];
                    const float carried = A + dsv[i];
                    const float gg = carried + share;
                    const float bg = 1.0f - omb[i];
                    Aref = omb[i] * carried - bg * share;
                    *reinterpret_cast<int*>(reinterpret_cast<char*>(lds) + ta) = t;
                    const float c = ACT ? fast_tanh(to_f32(yv[i])) : to_f32(yv[i]);
                    const float diff = c - to_f32(hv[i]);
                    float dc, db;
                    if constexpr (ACT) {
                        dc = bg * (1.0f - c * c) * gg;   // tanh'
                        db = diff * (omb[i] * bg) * gg;  // sigmoid'
                    } else {
                        dc = bg * gg;
                        db = diff * gg;
                    }
                    if (kPad) {  // exact zeros on padded slots, whatever their inputs hold
                        const bool ok = ca[i] != dummy;
                        dc = ok ? dc : 0.0f;
                        db = ok ? db : 0.0f;
                    }
                    const uint32_t so = uint32_t(t) * kd * sizeof(IN);
                    bstore_f32<IN>(dc, rdy, vy, so);
                    bstore_f32<IN>(db, rdg, vy, so);
                    rcur = ((rmask >> i) & 1u) ? t : rcur;  // nothing before it reaches past t
                }
            }
        };
        if (pad) steps(std::true_type{});
        else steps(std::false_type{});
    };
    double R = R_in;
    if constexpr (RES) {
        block(t_begin, t_end - t_begin);  // the chunk is in registers since phase A
    } else {
        for (int sb = nsb - 1; sb >= 0; --sb) {
            const int tb0 = t_begin + sb * TB;
            const int n = min(TB, t_end - tb0);
            fetch_q(tb0);
#pragma unroll
            for (int i = TB - 1; i >= 0; --i) fetch_a_at(i, tb0);
            rst_mask();
            shares(n, R);
            __builtin_amdgcn_wave_barrier();
            pad_lane = false;
#pragma unroll
            for (int i = TB - 1; i >= 0; --i) pad_lane |= prep(i, i < n);
            fetch_c(tb0);
            block(tb0, n);
        }
    }
    if (!RES && W == 1) R_out = R;

    // the carried-state gradient: A and R after position 0. A is wave 0's state; every
    // wavefront writes a share of it (wave 0 alone, an LDS wait per store, made the kernel's tail),
    // and wave 0 passes its latest reset in its region's dummy word.
    if (float* const dh0 = a.dh0) {
        if (w == 0 && lane == 0) reinterpret_cast<int*>(st)[NS] = rcur;
        __syncthreads();
        const float* const st0 = lds;
        const int* const tag0 = reinterpret_cast<const int*>(lds + NS + 1);
        const int rcur0 = reinterpret_cast<const int*>(lds)[NS];
        float* const dh0_row = dh0 + int64_t(b) * N * d;
        write_state<S, 4>(NS, gl, kWave * W, [&](int e) __attribute__((always_inline)) {
            // a cell last updated before the latest reset passed reads as zero
            return tag0[e / S] < rcur0 ? st0[e] : 0.0f;
        }, [&](int e, float v) __attribute__((always_inline)) {
            dh0_row[int64_t(e / S) * d + slice * S + e % S] = v;
        });
    }
    float* const dq0 = a.dq0;
    if (w == 0 && dq0 && kslot == 0) dq0[int64_t(b) * d + col] = static_cast<float>(R_out);
}

// ------------------------------------------------------------------------------------------
// The RMS candidate: a prologue normalises the candidate input once (the only cross-column
// quantity of the round, computed from inputs only), an epilogue applies the norm's VJP.
// ------------------------------------------------------------------------------------------

// The RMS workspace: [slots, d] of the storage type, then [slots] fp32 of 1/rms at a 16-byte
// aligned offset.
inline size_t rms_inv_offset(int64_t slots, int d, size_t elem) {
    return (size_t(slots) * size_t(d) * elem + 15) & ~size_t(15);
}

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

// Raise a kernel's dynamic-LDS limit to the full 160 KiB once per (kernel, device) and process
// (not a stream operation, and never repeated inside a stream capture). Every instantiation is
// its own kernel, so the record is keyed by the kernel's address.
hipError_t allow_lds_raw(const void* kernel, size_t lds);

template <typename K>
hipError_t allow_lds(K kernel, size_t lds) {
    if (lds <= 64 * 1024) return hipSuccess;
    return allow_lds_raw(reinterpret_cast<const void*>(kernel), lds);
}

template <typename IN, typename OUT, typename SLOT, int S>
hipError_t launch_fwd_s(const FwdArgs& a, size_t lds, hipStream_t st) {
    const bool res = a.W > 1 && a.Tc <= kResTB;
    // see fwd_chunk's phase C: 256 cells' maxima, a dummy and 64 words more fit the beta region
    const bool cm = a.h_max != nullptr && a.N <= 256 && a.N * S >= 321;
    auto k = res ? (cm ? fwd_chunk<IN, OUT, SLOT, S, kResTB, true, true>
                       : fwd_chunk<IN, OUT, SLOT, S, kResTB, true, false>)
                 : (cm ? fwd_chunk<IN, OUT, SLOT, S, kStreamTB, false, true>
                       : fwd_chunk<IN, OUT, SLOT, S, kStreamTB, false, false>);
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
    auto k = (a.W > 1 && a.Tc <= kResTB) ? bwd_chunk<IN, SLOT, ACT, S, kResTB, true>
                                         : bwd_chunk<IN, SLOT, ACT, S, kStreamTB, false>;
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

// The kernels of each storage type are instantiated in a translation unit of their own
// (sweep_inst_*.hip), so they compile in parallel; every other unit only declares them.
#ifndef HSN_SWEEP_INSTANTIATE
extern template hipError_t launch_fwd<float, float, Packed32>(const FwdArgs&, int, size_t, hipStream_t);
extern template hipError_t launch_fwd<bf16_t, bf16_t, Packed32>(const FwdArgs&, int, size_t, hipStream_t);
extern template hipError_t launch_fwd<float, float, Cells64>(const FwdArgs&, int, size_t, hipStream_t);
extern template hipError_t launch_fwd<bf16_t, float, Cells64>(const FwdArgs&, int, size_t, hipStream_t);
extern template hipError_t launch_bwd<float, Packed32, true>(const BwdArgs&, int, size_t, hipStream_t);
extern template hipError_t launch_bwd<bf16_t, Packed32, true>(const BwdArgs&, int, size_t, hipStream_t);
extern template hipError_t launch_bwd<float, Cells64, false>(const BwdArgs&, int, size_t, hipStream_t);
#endif

}  // namespace hsn
