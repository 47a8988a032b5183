// The window's forward sweep and backward recurrence as time-chunked slices with event maps.
//
// A workgroup owns (row b, a slice of 8 state columns) and the whole window. The window splits
// into 16 chunks of P = ceil(T / 16) positions; each chunk belongs to a half-wavefront (32 lanes:
// lane = 4 k + p, slot k of the position, column pair p of the slice, two fp32 columns a lane,
// 8-byte loads and stores). The state recurrence is separable over columns and, for a fixed
// chunk, affine in each cell's value at the chunk's start (h_end = alpha h_start + beta; a reset
// zeroes both), so the forward runs
//   phase A  every half-wave loads its chunk, computes the activations and composes the maps of
//            the cells its chunk touches,
//   phase B  the workgroup walks every (cell, column pair) through the 16 chunks from h0: each
//            touched chunk receives the cell's start value (and its |h| maximum), the untouched
//            cells' maximum per chunk is reduced, and the end state goes out,
//   phase C  every half-wave replays its chunk from those start values with the outputs.
// Event maps. A chunk touches at most P K cells, so its maps live in a table of P K entries
// instead of N: a cell's entry is the index i K + k of its first event in the chunk (position i,
// slot k), found without a search: the chunk's half-wave writes every event's index into the
// cell's byte of a [cell][chunk] table from the last position to the first, so the first
// event's index is the one left (LDS executes one wave's accesses in order). The table's row of
// a cell is its 16 chunks' entries, one 16-byte read in phase B.
// The row maximum of |h| after each position is the larger of the chunk's untouched cells'
// maximum at its start (fixed until a reset) and the current maxima of its touched cells, kept
// per entry. The summary q: the replay sums each position's slot deltas across the 8 slots (a
// reduce-scatter), each position maps q to (reset ? 0 : q) + D / N, and the maps are scanned
// within the chunk and then across the chunks from q0.
// The backward (below `bwd`) runs the same three phases in reverse time: a cell's entry is its
// last event in the chunk, the maps carry the state's cotangent from the chunk's end to its
// start, and the summary cotangent (which reads no state) is scanned first, in fp64.
#pragma once

#include "sweep.cuh"

// Phase stamps: a measurement build (hsn_amd/probes/evmap_phases.hip) defines HSN_EVMAP_STAMPS
// and these hooks, which record the real-time counter at the kernels' phase edges (and a value
// that tells the wavefronts apart, HSN_EVMAP_NOTE); in the library they compile to nothing.
#ifndef HSN_EVMAP_STAMPS
#define HSN_EVMAP_STAMPS_BEGIN()
#define HSN_EVMAP_STAMP(i)
#define HSN_EVMAP_NOTE(i, v)
#define HSN_EVMAP_STAMPS_END(which)
#endif

namespace hsn {
namespace evmap {

constexpr int kS = 8;          // state columns per workgroup
constexpr int kK = 8;          // slots per position, at most
constexpr int kWaves = 8;      // wavefronts per workgroup
constexpr int kChunks = 16;    // chunks per workgroup: two per wavefront
constexpr int kP = 16;         // positions per chunk, at most (T <= 256)
constexpr int kEv = kP * kK;   // event indices of a chunk
constexpr int kConst = kEv;    // entry holding cell 0's value at the chunk's start
constexpr int kDummy = kEv + 1;  // entry the padded and idle slots update, never read
constexpr int kEnt = kEv + 2;  // entries of a chunk's table
constexpr uint32_t kNone = 0xffu;
constexpr uint32_t kEntBytes = kS * 4;                 // one entry's 8 columns
constexpr uint32_t kMapBytes = 2u * kEnt * kEntBytes;  // a chunk's alpha and beta tables

// LDS byte offsets: the chunks' maps [16][alpha, beta][kEnt][8] f32 (alpha becomes the entry's
// value in phase C), the first-event table [N + 1][16] u8 (row N: kDummy, read by idle and
// padded slots), the entries' current maxima [16][kEnt] u32 (|h| bits), the last-event table
// [N + 1][16] u8 (the ages), per chunk its untouched cells' maximum and last reset, each chunk's
// summary map
// q -> (reset ? 0 : q) + c ([16][8] c and [16] reset flags) and start q [16][8], and 8 bytes a
// thread where a lane with nothing to store writes.
struct Layout {
    uint32_t maps, idx, cmx, lastev, umax, rlast, qmap, qreset, qstart, tdummy, bytes;
};

__host__ __device__ inline Layout fwd_layout(int N) {
    Layout L{};
    uint32_t at = 0;
    L.maps = at;
    at += kChunks * kMapBytes;
    L.idx = at;
    at += (uint32_t(N + 1) * kChunks + 15u) & ~15u;
    L.cmx = at;
    at += kChunks * kEnt * 4u;
    L.lastev = at;
    at += (uint32_t(N + 1) * kChunks + 15u) & ~15u;
    L.umax = at;
    at += kChunks * 4u;
    L.rlast = at;
    at += kChunks * 4u;
    L.qmap = at;
    at += kChunks * kS * 4u;
    L.qreset = at;
    at += kChunks * 4u;
    L.qstart = at;
    at += kChunks * kS * 4u;
    L.tdummy = at;
    at += kWave * kWaves * 8u;
    L.bytes = at;
    return L;
}

__device__ __forceinline__ float2 ld2(rsrc_t r, uint32_t vo) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, vo, 0u, 0);
    return make_float2(__uint_as_float(v[0]), __uint_as_float(v[1]));
}
__device__ __forceinline__ void st2(float2 x, rsrc_t r, uint32_t vo) {
    decltype(__builtin_amdgcn_raw_buffer_load_b64(r, 0u, 0u, 0)) v;
    v[0] = __float_as_uint(x.x);
    v[1] = __float_as_uint(x.y);
    __builtin_amdgcn_raw_buffer_store_b64(v, r, vo, 0u, 0);
}

template <typename T>
__device__ __forceinline__ T& lds_ref(unsigned char* lds, uint32_t byte) {
    return *reinterpret_cast<T*>(lds + byte);
}

__device__ __forceinline__ uint32_t abs2_bits(float2 v) {
    return umax(abs_bits(v.x), abs_bits(v.y));
}

// Sum with the lane m apart, the same column pair (m = 16, 8 or 4: a slot bit of the lane).
template <int M>
__device__ __forceinline__ float partner_f32(float v, int lane) {
    if constexpr (M == 16) {
        // the swap hands every lane {even row's value, odd row's value} of its row pair
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v),
                                                       false, false);
        return __uint_as_float((lane & 16) ? static_cast<uint32_t>(r[0]) : static_cast<uint32_t>(r[1]));
    } else if constexpr (M == 8) {
        return dpp_f32<dpp::kRor8>(v);
    } else {
        return __shfl_xor(v, M, kWave);
    }
}

template <int M>
__device__ __forceinline__ uint32_t partner_u32(uint32_t v, int lane) {
    if constexpr (M == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
        return (lane & 16) ? static_cast<uint32_t>(r[0]) : static_cast<uint32_t>(r[1]);
    } else if constexpr (M == 8) {
        return dpp_u32<dpp::kRor8>(v);
    } else if constexpr (M == 4) {
        // inside 8 lanes the half mirror pairs lane i with 7 - i: across bit 2, the same
        // higher bits (what a maximum over the lanes needs; the columns do not matter here)
        return dpp_u32<dpp::kHalfMirror>(v);
    } else if constexpr (M == 2) {
        return dpp_u32<dpp::kXor2>(v);
    } else {
        return dpp_u32<dpp::kXor1>(v);
    }
}

// ------------------------------------------------------------------------------------------
// Forward
// ------------------------------------------------------------------------------------------

// The forward's arguments: the window's tensors at their row starts (the kernel adds b times
// the row size), 32-bit sizes, and the summary's 1/N (an exact product when N is a power of two).
struct FwdEv {
    const float* y;         // [B, T, K, d], also the gate's pre-activation g
    const float* g;
    const int32_t* slots;   // [B, T, K]: the cell, or -1 where padded
    const uint8_t* reset;   // [B, T] or NULL
    const float* h0;        // [B, N, d]
    const float* q0;        // [B, d]
    const int64_t* age0;    // [B, N]
    const int64_t* pos0;    // [B]
    float* q_pre;           // [B, T, d]
    float* q_post;
    float* h_sel;           // [B, T, K, d] (each may be NULL)
    float* h_old;
    float* h_max;           // [B, T], holding 0 on entry, or NULL
    float* h_T;             // [B, N, d] or NULL
    float* q_T;             // [B, d] or NULL
    int64_t* age_T;         // [B, N] or NULL
    int64_t* pos_T;         // [B] or NULL
    int T, N, d, K, P;      // P: positions per chunk
    DivN divn;
};

// A per-lane bit of a word as an all-ones or all-zero word: a mask for bitwise selects, so the
// condition stays in a VGPR instead of a lane mask.
__device__ __forceinline__ uint32_t bitmask_at(uint32_t word, int i) { return 0u - ((word >> i) & 1u); }
__device__ __forceinline__ float and_f32(float v, uint32_t m) {
    return __uint_as_float(__float_as_uint(v) & m);
}
__device__ __forceinline__ float sel_f32(uint32_t m, float x, float y) {  // m ? x : y, bitwise
    return __uint_as_float((__float_as_uint(x) & m) | (__float_as_uint(y) & ~m));
}
// The maximum over lanes l, l ^ 16, l ^ 32, l ^ 48 (a cell's four column pairs in phase B).
__device__ __forceinline__ uint32_t max_of_rows(uint32_t v) {
    RowPair r = pair16(v);
    v = umax(r.lo, r.hi);
    r = pair32(v);
    return umax(r.lo, r.hi);
}

// The decisions are the `slots` input.
struct NoRoute {
    static constexpr bool kOn = false;
};

// The forward of one (row, 8-column slice). With Route::kOn the row's workgroups route the
// window themselves instead of reading `slots`; Route provides this launch's stamp,
// the prefetch of the logits of the workgroup's share of positions, their decisions (each
// handed to the row through a stamped word), the row's decisions gathered into LDS, and the
// exchange of the row maxima's per-slice parts at the end.
template <typename IN, typename Route>
__device__ __forceinline__ void fwd_body(const FwdEv& a, Route& route) {
    static_assert(sizeof(IN) == 4, "fp32 rows");
    extern __shared__ __align__(16) unsigned char lds[];
    HSN_EVMAP_STAMPS_BEGIN();
    const int N = a.N, d = a.d, K = a.K, T = a.T;
    const Layout Lo = fwd_layout(N);
    const int lane = lane_id();
    const int gl = threadIdx.x;
    const int w = uniform(gl / kWave);
    const int half = lane >> 5, hl = lane & 31;
    const int ch = 2 * w + half;  // this half-wave's chunk
    const int k = hl >> 2, cp = hl & 3;
    int b, slice;
    block_coords(b, slice);
    const int P = a.P;
    const int t0 = ch * P;
    const int n = max(0, min(P, T - t0));  // positions of the chunk (uniform in the half)
    const bool active = k < K;
    const int col = slice * kS + 2 * cp;
    const bool track_age = slice == 0 && a.age_T != nullptr;
    const DivN divn = a.divn;

    const uint32_t pos_bytes = uint32_t(K) * d * 4u;  // one position's slot rows
    const size_t orow = size_t(b) * T * K * d;  // element offset of row b of [B, T, K, d]
    const rsrc_t ry = make_rsrc(a.y + orow, uint32_t(T) * pos_bytes);
    const rsrc_t rg = make_rsrc(a.g + orow, uint32_t(T) * pos_bytes);
    const rsrc_t rc = make_rsrc(a.slots + size_t(b) * T * K, uint32_t(T) * K * 4u);
    const rsrc_t rr = make_rsrc(a.reset ? a.reset + size_t(b) * T : nullptr, a.reset ? uint32_t(T) : 0u);
    // a lane's piece of position i is vrow + i * pos_bytes: out of range (loads read zero, stores
    // are dropped) for an idle lane (kOob) and for a position past the window (its offset is at
    // least T * pos_bytes; the host keeps (T + 32) * pos_bytes < 2^31, so nothing wraps); a
    // position past a short chunk (P < 16) reads the next chunk's data, which the chunk ignores,
    // and its stores are sent out of range
    const uint32_t vrow = (active ? uint32_t(k * d + col) * 4u : kOob) + uint32_t(t0) * pos_bytes;

    // the routing's loads (the logits of the workgroup's positions) go out first, so that the
    // decisions wait for them and not for the slot rows
    uint64_t stamp = 0;
    if constexpr (Route::kOn) {
        stamp = route.stamp(b);
        route.prefetch(b, slice, w);
    }

    // ---- phase B's first start values and the chunk's resets, loaded first --------------------
    // phase B's threads: thread 2 c + q holds columns 4q .. 4q + 3 of cell c (+ 256 per pass)
    const int bq = gl & 1;
    const float* const h0_row = a.h0 + size_t(b) * N * d;
    auto h0_at = [&](int cell) __attribute__((always_inline)) -> float4 {
        return cell < N ? *reinterpret_cast<const float4*>(h0_row + int64_t(cell) * d + slice * kS + 4 * bq)
                        : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    };
    const float4 h0a = h0_at(gl >> 1);
    const uint8_t rbyte = __builtin_amdgcn_raw_buffer_load_b8(rr, hl < n ? uint32_t(t0 + hl) : kOob, 0u, 0);

    HSN_EVMAP_STAMP(1);
    // ---- phase A: the chunk's decisions first (its tables need them all), then the slot rows 6
    // positions ahead, each position's activations and composition as its row arrives ---------
    // (6 ahead measured 0.4 us faster than 8: fewer rows in flight before the decisions return;
    // 5, 7, 12 and 16 were slower)
    constexpr int kAhead = 6;
    float2 yv[kP], gv[kP];
    int32_t cv[kP];
    if constexpr (!Route::kOn) {
#pragma unroll
        for (int i = 0; i < kP; ++i)
            cv[i] = static_cast<int32_t>(__builtin_amdgcn_raw_buffer_load_b32(
                rc, active ? uint32_t((t0 + i) * K + k) * 4u : kOob, 0u, 0));
    }
    // (issued in position order, the scheduler held at each: position i's wait is then for its
    // own row and the older ones only)
    auto fetch = [&](int i) __attribute__((always_inline)) {
        const uint32_t vo = vrow + uint32_t(i) * pos_bytes;
        yv[i] = ld2(ry, vo);
        gv[i] = ld2(rg, vo);
        __builtin_amdgcn_sched_barrier(0);
    };
#pragma unroll
    for (int i = 0; i < kAhead; ++i) fetch(i);

    // this chunk's columns of the tables while the loads are in flight (no other half-wave
    // reads them before phase B): no event (0xff; kDummy in row N; cell 0 kConst, below) in the
    // first-event table and in the last-event table, zero maxima, the dummy entry's identity map
    // (1, 0) that idle slots compose, and the chunk's untouched maximum (phase B max-reduces
    // into it). Cell 0 without an event in the chunk keeps kConst, an entry with the identity map:
    // phase B then stores cell 0's start value there as for any touched cell (padded slots read
    // it), with no write of its own (that one branch a chunk measured 0.7 us of the walk).
    unsigned char* const idx = lds + Lo.idx;
    for (int c = hl; c <= N; c += 32)
        idx[c * kChunks + ch] = c == 0 ? uint8_t(kConst) : c < N ? 0xffu : uint8_t(kDummy);
    if (track_age)
        for (int c = hl; c < N; c += 32) lds[Lo.lastev + uint32_t(c * kChunks + ch)] = 0xffu;
    const uint32_t cmx_base = Lo.cmx + uint32_t(ch) * kEnt * 4u;
    for (int e = hl; e < kEnt; e += 32) lds_ref<uint32_t>(lds, cmx_base + 4u * e) = 0u;
    const uint32_t cbase = Lo.maps + uint32_t(ch) * kMapBytes;
    if (hl < kS) {
        lds_ref<float>(lds, cbase + kDummy * kEntBytes + 4u * hl) = 1.0f;
        lds_ref<float>(lds, cbase + kEnt * kEntBytes + kDummy * kEntBytes + 4u * hl) = 0.0f;
    } else if (hl < 2 * kS) {
        lds_ref<float>(lds, cbase + kConst * kEntBytes + 4u * (hl - kS)) = 1.0f;
        lds_ref<float>(lds, cbase + kEnt * kEntBytes + kConst * kEntBytes + 4u * (hl - kS)) = 0.0f;
    }
    if (hl == 0) lds_ref<uint32_t>(lds, Lo.umax + 4u * ch) = 0u;

    // the wavefront's share of the decisions while the first slot rows load (its LDS scratch in
    // its first chunk's maps, clear of the dummy entries, before the chunk composes them)
    if constexpr (Route::kOn) {
        route.decide(b, slice, w, stamp, lds + Lo.maps + uint32_t(2 * w) * kMapBytes);
        HSN_EVMAP_STAMP(9);
    }

    if constexpr (Route::kOn) {
        // the row's decisions as int16 in chunk 0's maps, below its dummy entry (T K <= 2048):
        // the maps are free until the composition, and the gather's barrier orders its writes
        // after every wavefront's decisions (whose scratch is there too)
        route.gather(b, stamp, lds + Lo.maps);
        __syncthreads();
#pragma unroll
        for (int i = 0; i < kP; ++i)
            cv[i] = active && i < n ? int32_t(lds_ref<int16_t>(lds, Lo.maps + 2u * uint32_t((t0 + i) * K + k)))
                                    : -1;
        __syncthreads();  // every read of the table before chunk 0 composes over it
    }
    uint32_t vmask = 0u, pmask = 0u;  // valid and padded positions of this lane's slot
#pragma unroll
    for (int i = 0; i < kP; ++i) {
        const int c = cv[i];
        const bool inb = active && i < n;
        const bool ok = inb && c >= 0;
        vmask |= ok ? 1u << i : 0u;
        pmask |= inb && c < 0 ? 1u << i : 0u;
        cv[i] = ok ? c : N;  // the first-event table's row (N: the idle slots' row)
    }
    const uint32_t rmask = static_cast<uint32_t>(ballot(rbyte != 0) >> (32 * half));

    // first events: every event writes its index into its cell's byte of this chunk, latest
    // position first, so each byte ends with the cell's first event; one lane a slot writes,
    // the others into their own dummy byte; idle and padded slots read row N (kDummy)
    const uint32_t my_dummy = Lo.tdummy + 8u * uint32_t(gl);
#pragma unroll
    for (int i = kP - 1; i >= 0; --i)
        lds[(vmask >> i) & 1u && cp == 0 ? Lo.idx + uint32_t(cv[i] * kChunks + ch) : my_dummy] =
            static_cast<unsigned char>(i * kK + k);
    uint32_t entw[kP / 4] = {};
#pragma unroll
    for (int i = 0; i < kP; ++i) entw[i / 4] |= uint32_t(idx[cv[i] * kChunks + ch]) << (8 * (i % 4));
    auto ent = [&](int i) __attribute__((always_inline)) -> uint32_t {
        return (entw[i / 4] >> (8 * (i % 4))) & 0xffu;
    };
    const uint32_t e0raw = idx[ch];  // cell 0's entry in this chunk
    const uint32_t e0 = e0raw == kNone ? uint32_t(kConst) : e0raw;
    // the entry a position's slot reads before its update: its own, or cell 0's if padded
    uint32_t rentw[kP / 4] = {};
#pragma unroll
    for (int i = 0; i < kP; ++i) rentw[i / 4] |= ((pmask >> i) & 1u ? e0 : ent(i)) << (8 * (i % 4));
    auto rent = [&](int i) __attribute__((always_inline)) -> uint32_t {
        return (rentw[i / 4] >> (8 * (i % 4))) & 0xffu;
    };
    if (track_age)  // last events, earliest position first: each byte ends with the last one
#pragma unroll
        for (int i = 0; i < kP; ++i)
            lds[(vmask >> i) & 1u && cp == 0 ? Lo.lastev + uint32_t(cv[i] * kChunks + ch) : my_dummy] =
                static_cast<unsigned char>(i * kK + k);
    if (hl == 0) lds_ref<int32_t>(lds, Lo.rlast + 4u * ch) = rmask ? t0 + 31 - __builtin_clz(rmask) : -1;

    const uint32_t lofs = uint32_t(cp) * 8u;
    auto al_at = [&](uint32_t e) __attribute__((always_inline)) -> float2& {
        return lds_ref<float2>(lds, cbase + e * kEntBytes + lofs);
    };
    auto be_at = [&](uint32_t e) __attribute__((always_inline)) -> float2& {
        return lds_ref<float2>(lds, cbase + kEnt * kEntBytes + e * kEntBytes + lofs);
    };
    // zero the maps (or values) of the entries below `e_end`, by the half-wave (a reset)
    auto zero_entries = [&](int e_end, bool with_beta) __attribute__((always_inline)) {
        for (int e = hl; e < e_end * 4; e += 32) {
            const uint32_t at = cbase + uint32_t(e >> 2) * kEntBytes + uint32_t(e & 3) * 8u;
            lds_ref<float2>(lds, at) = make_float2(0.0f, 0.0f);
            if (with_beta) lds_ref<float2>(lds, at + kEnt * kEntBytes) = make_float2(0.0f, 0.0f);
        }
    };

    // compose the chunk's maps: alpha' = (1 - b) alpha, beta' = (1 - b) beta + b c, an entry's
    // first event starting from (1, 0), or (0, 0) after a reset in the chunk; a reset zeroes the
    // entries created before it (idle and padded slots compose the identity on kDummy). Position
    // i's activations come first: its row is the oldest load in flight, and the loads kAhead
    // positions on go out as each position is taken, so the composition runs while the rows
    // arrive.
    HSN_EVMAP_STAMP(2);
    float2 omb[kP], bcv[kP];
    auto compose = [&](auto rs_c) __attribute__((always_inline)) {
        constexpr bool kRs = decltype(rs_c)::value;
        float ainit = 1.0f;
#pragma unroll
        for (int i = 0; i < kP; ++i) {
            if (i + kAhead < kP) fetch(i + kAhead);
            {
                const bool ok = (vmask >> i) & 1u;
                const float b0 = fast_sigmoid(gv[i].x), b1 = fast_sigmoid(gv[i].y);
                const float c0 = fast_tanh(yv[i].x), c1 = fast_tanh(yv[i].y);
                omb[i] = ok ? make_float2(1.0f - b0, 1.0f - b1) : make_float2(1.0f, 1.0f);
                bcv[i] = ok ? make_float2(b0 * c0, b1 * c1) : make_float2(0.0f, 0.0f);
            }
            if (kRs && ((rmask >> i) & 1u)) {
                zero_entries(i * kK, true);
                ainit = 0.0f;
            }
            const uint32_t e = ent(i);
            const bool first = e == uint32_t(i * kK + k);
            const float2 al = al_at(e), be = be_at(e);
            const float2 o = omb[i];
            al_at(e) = make_float2(o.x * (first ? ainit : al.x), o.y * (first ? ainit : al.y));
            be_at(e) = make_float2(o.x * (first ? 0.0f : be.x) + bcv[i].x,
                                   o.y * (first ? 0.0f : be.y) + bcv[i].y);
        }
    };
    const bool wave_rs = ballot(rmask != 0u) != 0u;
    if constexpr (!Route::kOn) HSN_EVMAP_NOTE(9, wave_rs ? 1u : 0u);
    if (wave_rs) compose(std::true_type{});
    else compose(std::false_type{});
    __syncthreads();

    HSN_EVMAP_STAMP(3);
    // ---- phase B: every cell through the 16 chunks, two threads a cell -----------------------
    {
        uint32_t rflags = 0u;  // chunks with a reset
#pragma unroll
        for (int j = 0; j < kChunks; ++j)
            rflags |= lds_ref<int32_t>(lds, Lo.rlast + 4u * j) >= 0 ? 1u << j : 0u;
        rflags = uniform(rflags);
        uint32_t um[kChunks];  // the untouched cells' maxima over this thread's cells
#pragma unroll
        for (int j = 0; j < kChunks; ++j) um[j] = 0u;
        float* const hT_row = a.h_T ? a.h_T + size_t(b) * N * d : nullptr;
        const uint32_t qofs = uint32_t(bq) * 16u;  // the thread's half of an entry
        for (int c0 = 0; c0 < N; c0 += kWave * kWaves / 2) {
            const int cell = c0 + (gl >> 1);
            const bool ok = cell < N;
            float4 s = c0 == 0 ? h0a : h0_at(cell);
            const uint4 iw = lds_ref<uint4>(lds, Lo.idx + uint32_t(ok ? cell : N) * kChunks);
            const uint32_t words[4] = {ok ? iw.x : ~0u, ok ? iw.y : ~0u, ok ? iw.z : ~0u, ok ? iw.w : ~0u};
#pragma unroll
            for (int jh = 0; jh < kChunks; jh += kChunks / 4) {  // four chunks' reads at once
                float4 al[kChunks / 4], be[kChunks / 4];
#pragma unroll
                for (int jj = 0; jj < kChunks / 4; ++jj) {
                    const int j = jh + jj;
                    const uint32_t ej = (words[j / 4] >> (8 * (j % 4))) & 0xffu;
                    const uint32_t e = ej == kNone ? uint32_t(kDummy) : ej;  // the identity (1, 0)
                    const uint32_t at = Lo.maps + uint32_t(j) * kMapBytes + e * kEntBytes + qofs;
                    al[jj] = lds_ref<float4>(lds, at);
                    be[jj] = lds_ref<float4>(lds, at + kEnt * kEntBytes);
                }
#pragma unroll
                for (int jj = 0; jj < kChunks / 4; ++jj) {
                    const int j = jh + jj;
                    const uint32_t ej = (words[j / 4] >> (8 * (j % 4))) & 0xffu;
                    const bool touched = ej != kNone;
                    // the thread's 4 columns (the cell's other half comes in through the atomic
                    // maximum below, and through the reduction of the untouched maxima)
                    uint32_t m = umax(umax(abs_bits(s.x), abs_bits(s.y)), umax(abs_bits(s.z), abs_bits(s.w)));
                    m = ok ? m : 0u;
                    const uint32_t jb = Lo.maps + uint32_t(j) * kMapBytes;
                    // the entry's start value for the replay and its maximum (kConst: cell 0 where
                    // the chunk leaves it untouched, which still counts among the untouched)
                    if (touched) {
                        lds_ref<float4>(lds, jb + ej * kEntBytes + qofs) = s;
                        atomicMax(&lds_ref<uint32_t>(lds, Lo.cmx + 4u * (j * kEnt + ej)), m);
                    }
                    um[j] = umax(um[j], touched && ej != uint32_t(kConst) ? 0u : m);
                    // a chunk with a reset ends at beta whatever the start (not 0 * s: a NaN in
                    // the start state must not cross the reset, as masked_fill); an untouched
                    // cell's map is the dummy entry's identity (1, 0)
                    if ((rflags >> j) & 1u) s = be[jj];
                    else s = make_float4(al[jj].x * s.x + be[jj].x, al[jj].y * s.y + be[jj].y,
                                         al[jj].z * s.z + be[jj].z, al[jj].w * s.w + be[jj].w);
                }
            }
            if (ok && hT_row)
                *reinterpret_cast<float4*>(hT_row + int64_t(cell) * d + slice * kS + 4 * bq) = s;
        }
        // the untouched cells' maxima: a max reduce-scatter over the wave (lane l ends with
        // chunk l / 4), then one atomic a chunk and wave
        const uint32_t mj = max_scatter<kChunks>(um, lane);
        if ((lane & 3) == 0) atomicMax(&lds_ref<uint32_t>(lds, Lo.umax + 4u * uint32_t(lane >> 2)), mj);
    }
    if (track_age) {  // the ages and position at the window's end
        int last_reset = -1;
        for (int j = 0; j < kChunks; ++j) last_reset = max(last_reset, lds_ref<int32_t>(lds, Lo.rlast + 4u * j));
        int64_t* const ageT_row = a.age_T + size_t(b) * N;
        const int64_t* const age0_row = a.age0 + size_t(b) * N;
        for (int c = gl; c < N; c += kWave * kWaves) {
            // the cell's last selection: the latest chunk with an event, at that event's position
            const uint4 lw = lds_ref<uint4>(lds, Lo.lastev + uint32_t(c) * kChunks);
            const uint32_t words[4] = {lw.x, lw.y, lw.z, lw.w};
            int ls = -1;
#pragma unroll
            for (int j = 0; j < kChunks; ++j) {
                const uint32_t e = (words[j / 4] >> (8 * (j % 4))) & 0xffu;
                ls = e != kNone ? j * P + int(e / kK) : ls;
            }
            int64_t age;
            if (ls >= 0 && ls >= last_reset) age = (T - 1) - ls;
            else if (last_reset >= 0) age = T - last_reset;
            else age = age0_row[c] + T;
            ageT_row[c] = age;
        }
        if (a.pos_T && gl == 0) a.pos_T[b] = last_reset >= 0 ? int64_t(T - last_reset) : a.pos0[b] + T;
    }
    __syncthreads();

    HSN_EVMAP_STAMP(4);
    // ---- phase C: the replay -------------------------------------------------------------------
    // b c moves to the chunk's beta table (free after phase B): 32 lanes x 16 positions x 8 bytes,
    // the 4160 bytes of the table less 64, so the replay holds only 1 - b in registers
    const uint32_t bc_base = cbase + kEnt * kEntBytes + uint32_t(hl) * 8u;
#pragma unroll
    for (int i = 0; i < kP; ++i) lds_ref<float2>(lds, bc_base + uint32_t(i) * 256u) = bcv[i];
    const rsrc_t rho = make_rsrc(a.h_old ? a.h_old + orow : nullptr, a.h_old ? uint32_t(T) * pos_bytes : 0u);
    const rsrc_t rhs = make_rsrc(a.h_sel ? a.h_sel + orow : nullptr, a.h_sel ? uint32_t(T) * pos_bytes : 0u);
    const rsrc_t rqa = make_rsrc(a.q_pre ? a.q_pre + size_t(b) * T * d : nullptr, a.q_pre ? uint32_t(T) * d * 4u : 0u);
    const rsrc_t rqb = make_rsrc(a.q_post ? a.q_post + size_t(b) * T * d : nullptr, a.q_post ? uint32_t(T) * d * 4u : 0u);
    const bool wave_pad = ballot(pmask != 0u) != 0u;
    uint32_t vrow_c = vrow;
    asm volatile("" : "+v"(vrow_c));  // recomputed here, not held from phase A's loads
    const uint32_t u = lds_ref<uint32_t>(lds, Lo.umax + 4u * ch);
    const int first_reset = rmask ? __builtin_ctz(rmask) : 32;
    const int g = hl >> 2;  // the lane group holding one position after the reductions
    const uint32_t vq = uint32_t(col) * 4u;
    // the summaries of the lane's positions g and 8 + g: D / N, the reset before it, the map of
    // the half's earlier positions (rx ? 0 : q) + cx, and each half's whole map
    float2 qc[2], qx[2], hc[2];
    bool qr[2], qxr[2], hr[2];

    // positions 8 H .. 8 H + 7: the steps, then each position's row maximum and summaries
    auto eight = [&](auto h_c) __attribute__((always_inline)) {
        constexpr int H = decltype(h_c)::value;
        float2 dl[8];
        uint32_t lmv[8];
        // the next position's read goes out after this position's write and its row-maximum
        // reads (its entry may be the one just written: LDS keeps one wave's accesses in order);
        // at a reset the entries are zeroed after that read, so the value is taken as zero
        float2 h = al_at(rent(8 * H));
        float2 bc = lds_ref<float2>(lds, bc_base + uint32_t(8 * H) * 256u);
#pragma unroll
        for (int ii = 0; ii < 8; ++ii) {
            const int i = 8 * H + ii;
            if ((rmask >> i) & 1u) {  // every value of the chunk restarts at zero
                // the entries, cell 0's start value and their maxima, in straight-line writes
                // (as a loop, the writes measured 0.4 us more on the wavefronts with a reset)
#pragma unroll
                for (int q = 0; q < ((kEnt - 1) * 4 + 31) / 32; ++q) {
                    const int ee = hl + 32 * q;
                    if (ee < (kEnt - 1) * 4)
                        lds_ref<float2>(lds, cbase + uint32_t(ee >> 2) * kEntBytes + uint32_t(ee & 3) * 8u) =
                            make_float2(0.0f, 0.0f);
                }
#pragma unroll
                for (int q = 0; q < (kEnt + 31) / 32; ++q)
                    if (hl + 32 * q < kEnt) lds_ref<uint32_t>(lds, cmx_base + 4u * uint32_t(hl + 32 * q)) = 0u;
                h = make_float2(0.0f, 0.0f);
            }
            const uint32_t e = ent(i);
            const float2 hn = make_float2(omb[i].x * h.x + bc.x, omb[i].y * h.y + bc.y);
            al_at(e) = hn;
            float2 hs = hn;
            if (wave_pad) {  // a padded slot shows cell 0 after the position
                const float2 c0 = al_at(e0);
                const uint32_t pm = bitmask_at(pmask, i);
                hs = make_float2(sel_f32(pm, c0.x, hn.x), sel_f32(pm, c0.y, hn.y));
            }
            const float2 hcur = h;
            auto read_ahead = [&]() __attribute__((always_inline)) {
                if (ii + 1 < 8) {
                    h = al_at(rent(i + 1));
                    bc = lds_ref<float2>(lds, bc_base + uint32_t(i + 1) * 256u);
                }
            };
            // past the chunk (P < 16): out of range, not the next chunk's rows
            const uint32_t vo = i < n ? vrow_c + uint32_t(i) * pos_bytes : kOob;
            st2(hcur, rho, vo);
            st2(hs, rhs, vo);
            const uint32_t vm = bitmask_at(vmask, i);
            dl[ii] = make_float2(and_f32(hn.x - hcur.x, vm), and_f32(hn.y - hcur.y, vm));
            const uint32_t mg = group_max<4>(abs2_bits(hn) & vm);
            lds_ref<uint32_t>(lds, (vm & 1u) && cp == 0 ? cmx_base + 4u * e : my_dummy) = mg;
            const uint32_t m0 = lds_ref<uint32_t>(lds, cmx_base + 4u * hl);
            const uint32_t m1 = lds_ref<uint32_t>(lds, cmx_base + 4u * (hl + 32));
            const uint32_t m2 = lds_ref<uint32_t>(lds, cmx_base + 4u * (hl + 64));
            const uint32_t m3 = lds_ref<uint32_t>(lds, cmx_base + 4u * (hl + 96));
            // each position starts with the reset's branch, past which the compiler cannot move
            // this position's reductions: the read-ahead goes out after the maxima's reads, so
            // that taking them waits for these reads only
            read_ahead();
            lmv[ii] = umax(umax(m0, m1), umax(m2, m3));
        }
        const int pos = 8 * H + g;
        // the row maximum: a max reduce-scatter over the lane bits 4, 3, 2 (lane group g ends
        // with position pos), then the group's four lanes, with the untouched cells' maximum
        // until a reset
        {
            int cnt = 8;
#pragma unroll
            for (int m = 16; m >= 4; m >>= 1) {
                const int h2 = cnt / 2;
                const bool up = (hl & m) != 0;
#pragma unroll
                for (int ii = 0; ii < 4; ++ii) {
                    if (ii < h2) {
                        const uint32_t lo = lmv[ii], hi = lmv[h2 + ii];
                        const uint32_t send = up ? lo : hi;
                        uint32_t recv;
                        if (m == 16) recv = partner_u32<16>(send, lane);
                        else if (m == 8) recv = partner_u32<8>(send, lane);
                        else recv = partner_u32<4>(send, lane);
                        lmv[ii] = umax(up ? hi : lo, recv);
                    }
                }
                cnt = h2;
            }
            uint32_t mx = lmv[0];
            mx = umax(mx, partner_u32<2>(mx, lane));
            mx = umax(mx, partner_u32<1>(mx, lane));
            mx = umax(mx, pos < first_reset ? u : 0u);
            if (a.h_max && (hl & 3) == 0 && pos < n) {
                if constexpr (Route::kOn) route.put_hmax(b, t0 + pos, slice, mx, stamp);
                else atomicMax(reinterpret_cast<unsigned int*>(a.h_max + size_t(b) * T) + (t0 + pos), mx);
            }
        }
        // the summaries: the slots' deltas summed by a reduce-scatter over the slot bits (lane
        // group g ends with position pos, its column pair), then a scan of the positions' maps
        // q -> (reset ? 0 : q) + D / N over the groups
        {
#pragma unroll
            for (int m = 16; m >= 4; m >>= 1) {
                const int h2 = m / 4;  // positions held before the step: 8, 4, 2
                const bool up = (hl & m) != 0;
#pragma unroll
                for (int ii = 0; ii < 4; ++ii) {
                    if (ii < h2) {
                        const float2 lo = dl[ii], hi = dl[h2 + ii];
                        const float2 send = up ? lo : hi;
                        float rx, ry2;
                        if (m == 16) rx = partner_f32<16>(send.x, lane), ry2 = partner_f32<16>(send.y, lane);
                        else if (m == 8) rx = partner_f32<8>(send.x, lane), ry2 = partner_f32<8>(send.y, lane);
                        else rx = partner_f32<4>(send.x, lane), ry2 = partner_f32<4>(send.y, lane);
                        const float2 keep = up ? hi : lo;
                        dl[ii] = make_float2(keep.x + rx, keep.y + ry2);
                    }
                }
            }
            const bool in = pos < n;
            const float2 c = make_float2(divn(dl[0].x), divn(dl[0].y));
            const bool r = in && ((rmask >> pos) & 1u);
            bool rs = r;
            float2 cg = in ? c : make_float2(0.0f, 0.0f);
#pragma unroll
            for (int sft = 1; sft < 8; sft <<= 1) {  // inclusive scan over the groups 0..g
                const float px = __shfl_up(cg.x, 4 * sft, kWave), py = __shfl_up(cg.y, 4 * sft, kWave);
                const int pr = __shfl_up(rs ? 1 : 0, 4 * sft, kWave);
                if (g >= sft) {
                    cg = rs ? cg : make_float2(px + cg.x, py + cg.y);
                    rs = rs || pr != 0;
                }
            }
            float cx = __shfl_up(cg.x, 4, kWave), cy = __shfl_up(cg.y, 4, kWave);
            int rx = __shfl_up(rs ? 1 : 0, 4, kWave);
            if (g == 0) cx = cy = 0.0f, rx = 0;
            qc[H] = c, qr[H] = r, qx[H] = make_float2(cx, cy), qxr[H] = rx != 0;
            const int src = (lane & 32) | (28 + cp);  // group 7: the half's whole map
            hc[H] = make_float2(__shfl(cg.x, src, kWave), __shfl(cg.y, src, kWave));
            hr[H] = __shfl(rs ? 1 : 0, src, kWave) != 0;
        }
    };
    // one code path for every wavefront, with or without a reset in its chunks: a separate path
    // for the few wavefronts with resets ran from a cold instruction cache and ended their
    // workgroups about 1.5 us after the others
    eight(std::integral_constant<int, 0>{});
    eight(std::integral_constant<int, 1>{});

    HSN_EVMAP_STAMP(5);
    // the chunks' maps (half 0, then half 1), scanned across the chunks from q0, give each chunk
    // its start q; then each lane's two positions
    if (g == 0) {
        const float2 c = hr[1] ? hc[1] : make_float2(hc[0].x + hc[1].x, hc[0].y + hc[1].y);
        lds_ref<float2>(lds, Lo.qmap + 4u * (ch * kS + 2 * cp)) = c;
        if (cp == 0) lds_ref<int32_t>(lds, Lo.qreset + 4u * ch) = hr[0] || hr[1] ? 1 : 0;
    }
    __syncthreads();
    if (gl < kS) {  // one column a thread, the chunks in order
        float cm[kChunks];
        bool rm[kChunks];
#pragma unroll
        for (int j = 0; j < kChunks; ++j) {
            cm[j] = lds_ref<float>(lds, Lo.qmap + 4u * (j * kS + gl));
            rm[j] = lds_ref<int32_t>(lds, Lo.qreset + 4u * j) != 0;
        }
        float q = a.q0[size_t(b) * d + slice * kS + gl];
#pragma unroll
        for (int j = 0; j < kChunks; ++j) {
            lds_ref<float>(lds, Lo.qstart + 4u * (j * kS + gl)) = q;
            q = (rm[j] ? 0.0f : q) + cm[j];
        }
        if (a.q_T) a.q_T[size_t(b) * d + slice * kS + gl] = q;
    }
    __syncthreads();
    {
        const float2 qs = lds_ref<float2>(lds, Lo.qstart + 4u * (ch * kS + 2 * cp));
        const float2 q1s = make_float2((hr[0] ? 0.0f : qs.x) + hc[0].x, (hr[0] ? 0.0f : qs.y) + hc[0].y);
#pragma unroll
        for (int H = 0; H < 2; ++H) {
            const float2 qin = H == 0 ? qs : q1s;
            float2 q = make_float2((qxr[H] ? 0.0f : qin.x) + qx[H].x, (qxr[H] ? 0.0f : qin.y) + qx[H].y);
            if (qr[H]) q = make_float2(0.0f, 0.0f);
            const int pos = 8 * H + g;
            const uint32_t vqp = pos < n ? vq + uint32_t(t0 + pos) * d * 4u : kOob;
            st2(q, rqa, vqp);
            st2(make_float2(q.x + qc[H].x, q.y + qc[H].y), rqb, vqp);
        }
    }
    HSN_EVMAP_STAMP(6);
    HSN_EVMAP_STAMPS_END(0);
    // the maps are free again: the row maxima's exchange accumulates in chunk 0's
    if constexpr (Route::kOn) route.finish(b, slice, stamp, a.h_max, lds + Lo.maps);
}

template <typename IN>
__global__ __launch_bounds__(kWave* kWaves) void fwd(FwdEv a) {
    NoRoute route;
    fwd_body<IN>(a, route);
}

// ------------------------------------------------------------------------------------------
// Backward
// ------------------------------------------------------------------------------------------
//
// The reverse recurrence of one cell and column is affine per event too: with A the cotangent
// of the cell's value after the event, the value before it gets A' = (1 - b) (A + dsel) - b s,
// where dsel is the slot's h_sel cotangent and s = R / N the position's share of the summary
// cotangent R (the summary's cotangent enters every update once with + and once with -); a
// reset at t zeroes every cell's A once position t is processed, and R as well. R depends on the
// cotangents only, so the kernel first scans it (fp64, latest position first, one barrier across
// the chunks) into every position's share; then, time reversed, the same three phases as the
// forward: each chunk composes its cells' maps A_start = mu A_end + nu over its events latest
// first (a cell's entry is its last event in the chunk), the cells are walked from d_h_T back
// through the 16 chunks to d_h0, and each chunk replays its positions from the cells' end values
// with the outputs d y = b (1 - c^2) G and d gate = (c - h_old) b (1 - b) G, G = A + dsel + s.
// Padded and idle slots take part in nothing and write exact zeros.

struct BwdEv {
    const float* y;         // [B, T, K, d]: the candidate's pre-activation (tanh)
    const float* g;         // the gate's pre-activation (sigmoid)
    const float* h_old;     // the forward's gathered old values
    const float* dsel;      // [B, T, K, d] cotangent of h_sel, or NULL (zero)
    const int32_t* slots;   // [B, T, K]: the cell, or -1 where padded
    const uint8_t* reset;   // [B, T] or NULL
    const float* dq_pre;    // [B, T, d] or NULL
    const float* dq_post;
    const float* dh_T;      // [B, N, d] or NULL
    const float* dq_T;      // [B, d] or NULL
    float* dy;              // [B, T, K, d]
    float* dg;
    float* dh0;             // [B, N, d] or NULL
    float* dq0;             // [B, d] or NULL
    int T, N, d, K, P;
    DivN divn;
};

// LDS byte offsets: the chunks' maps [16][mu, nu][kEnt][8] f32 (mu becomes the entry's cotangent
// in phase C, nu the slots' h_sel cotangents), the last-event table [N + 1][16] u8 (row N:
// kDummy), the positions' shares [16][16][8] f32, each chunk's summary-cotangent map
// R -> (reset ? 0 : R) + c ([16][8] fp64 c, [16] reset flags), and 8 bytes a thread where a lane
// with nothing to write does.
struct BwdLayout {
    uint32_t maps, idx, share, rsum, rflag, tdummy, bytes;
};

__host__ __device__ inline BwdLayout bwd_layout(int N) {
    BwdLayout L{};
    uint32_t at = 0;
    L.maps = at;
    at += kChunks * kMapBytes;
    L.idx = at;
    at += (uint32_t(N + 1) * kChunks + 15u) & ~15u;
    L.share = at;
    at += kChunks * kP * kS * 4u;
    L.rsum = at;
    at += kChunks * kS * 8u;
    L.rflag = at;
    at += kChunks * 4u;
    L.tdummy = at;
    at += kWave * kWaves * 8u;
    L.bytes = at;
    return L;
}

template <typename IN>
__global__ __launch_bounds__(kWave* kWaves) void bwd(BwdEv a) {
    static_assert(sizeof(IN) == 4, "fp32 rows");
    extern __shared__ __align__(16) unsigned char lds[];
    HSN_EVMAP_STAMPS_BEGIN();
    const int N = a.N, d = a.d, K = a.K, T = a.T;
    const BwdLayout Lo = bwd_layout(N);
    const int lane = lane_id();
    const int gl = threadIdx.x;
    const int half = lane >> 5, hl = lane & 31;
    const int ch = 2 * uniform(gl / kWave) + half;  // this half-wave's chunk
    const int k = hl >> 2, cp = hl & 3;
    int b, slice;
    block_coords(b, slice);
    const int P = a.P;
    const int t0 = ch * P;
    const int n = max(0, min(P, T - t0));  // positions of the chunk (uniform in the half)
    const bool active = k < K;
    const int col = slice * kS + 2 * cp;
    const DivN divn = a.divn;

    const uint32_t pos_bytes = uint32_t(K) * d * 4u;
    const size_t orow = size_t(b) * T * K * d;
    const uint32_t row_bytes = uint32_t(T) * pos_bytes;
    const rsrc_t rg = make_rsrc(a.g + orow, row_bytes);
    const rsrc_t rds = make_rsrc(a.dsel ? a.dsel + orow : nullptr, a.dsel ? row_bytes : 0u);
    const rsrc_t rc = make_rsrc(a.slots + size_t(b) * T * K, uint32_t(T) * K * 4u);
    const rsrc_t rr = make_rsrc(a.reset ? a.reset + size_t(b) * T : nullptr, a.reset ? uint32_t(T) : 0u);
    const uint32_t qbytes = uint32_t(T) * d * 4u;
    const rsrc_t rqa = make_rsrc(a.dq_pre ? a.dq_pre + size_t(b) * T * d : nullptr, a.dq_pre ? qbytes : 0u);
    const rsrc_t rqb = make_rsrc(a.dq_post ? a.dq_post + size_t(b) * T * d : nullptr, a.dq_post ? qbytes : 0u);
    // a lane's piece of position i is vrow + i * pos_bytes, out of range for an idle lane and
    // past the window (as the forward's)
    const uint32_t vrow = (active ? uint32_t(k * d + col) * 4u : kOob) + uint32_t(t0) * pos_bytes;

    // ---- first loads: phase B's first end cotangents, the resets, the summary cotangents ----
    const int bq = gl & 1;  // phase B: thread 2 c + q holds columns 4q .. 4q + 3 of cell c
    const float* const dhT_row = a.dh_T ? a.dh_T + size_t(b) * N * d : nullptr;
    auto dhT_at = [&](int cell) __attribute__((always_inline)) -> float4 {
        return dhT_row && cell < N
                   ? *reinterpret_cast<const float4*>(dhT_row + int64_t(cell) * d + slice * kS + 4 * bq)
                   : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    };
    const float4 dha = dhT_at(gl >> 1);
    const uint8_t rbyte = __builtin_amdgcn_raw_buffer_load_b8(rr, hl < n ? uint32_t(t0 + hl) : kOob, 0u, 0);
    // the summary cotangents of the lane's positions g and 8 + g, its column pair
    const int g = hl >> 2;
    const uint32_t vq = uint32_t(col) * 4u;
    float2 qa[2], qb[2];
#pragma unroll
    for (int H = 0; H < 2; ++H) {
        const int pos = 8 * H + g;
        const uint32_t vqp = pos < n ? vq + uint32_t(t0 + pos) * d * 4u : kOob;
        qa[H] = ld2(rqa, vqp);
        qb[H] = ld2(rqb, vqp);
    }
    // the window-end summary cotangent of the column pair (the chunks' R starts there): loaded
    // here, before the gates, so that the wait for it after the barrier holds none of them
    const rsrc_t rqT = make_rsrc(a.dq_T ? a.dq_T + size_t(b) * d : nullptr, a.dq_T ? uint32_t(d) * 4u : 0u);
    const float2 dqT = ld2(rqT, vq);

    HSN_EVMAP_STAMP(1);
    // ---- phase A: the chunk's decisions first (its tables need them all), then the gates and
    // the selection cotangents latest position first, 6 positions ahead of the composition ----
    constexpr int kAhead = 6;
    float2 gv[kP], dv[kP];
    int32_t cv[kP];
#pragma unroll
    for (int i = 0; i < kP; ++i)
        cv[i] = static_cast<int32_t>(__builtin_amdgcn_raw_buffer_load_b32(
            rc, active ? uint32_t((t0 + i) * K + k) * 4u : kOob, 0u, 0));
    // (issued in the composition's order, the scheduler held at each: a position's wait is then
    // for its own rows and the ones issued before)
    auto fetch = [&](int i) __attribute__((always_inline)) {
        const uint32_t vo = vrow + uint32_t(i) * pos_bytes;
        gv[i] = ld2(rg, vo);
        dv[i] = ld2(rds, vo);
        __builtin_amdgcn_sched_barrier(0);
    };
#pragma unroll
    for (int i = kP - 1; i >= kP - kAhead; --i) fetch(i);

    // this chunk's columns of the tables while the loads are in flight (no other half-wave reads
    // them before phase B): no event (0xff; row N kDummy) and the dummy entry's identity (1, 0)
    unsigned char* const idx = lds + Lo.idx;
    for (int c = hl; c <= N; c += 32) idx[c * kChunks + ch] = c < N ? 0xffu : uint8_t(kDummy);
    const uint32_t cbase = Lo.maps + uint32_t(ch) * kMapBytes;
    if (hl < kS) {
        lds_ref<float>(lds, cbase + kDummy * kEntBytes + 4u * hl) = 1.0f;
        lds_ref<float>(lds, cbase + kEnt * kEntBytes + kDummy * kEntBytes + 4u * hl) = 0.0f;
    }

    // the summary cotangent's maps, latest position first: position p takes R to
    // (reset ? 0 : R + dq_post + dq_pre); an inclusive scan over the lane groups g .. 7 of each
    // half (later positions applied first), in fp64
    const uint32_t rmask = static_cast<uint32_t>(ballot(rbyte != 0) >> (32 * half));
    bool ir[2], er[2], wr[2];  // inclusive, exclusive (groups after g) and the whole half's
    double icx[2], icy[2], ecx[2], ecy[2], wcx[2], wcy[2];
#pragma unroll
    for (int H = 0; H < 2; ++H) {
        const int pos = 8 * H + g;
        const bool in = pos < n;
        bool r = in && ((rmask >> pos) & 1u);
        double cx = in && !r ? double(qb[H].x) + double(qa[H].x) : 0.0;
        double cy = in && !r ? double(qb[H].y) + double(qa[H].y) : 0.0;
#pragma unroll
        for (int sft = 1; sft < 8; sft <<= 1) {
            const double nx = __shfl_down(cx, 4 * sft, kWave), ny = __shfl_down(cy, 4 * sft, kWave);
            const int nr = __shfl_down(r ? 1 : 0, 4 * sft, kWave);
            if (g + sft < 8) {
                cx = r ? cx : cx + nx;
                cy = r ? cy : cy + ny;
                r = r || nr != 0;
            }
        }
        ir[H] = r, icx[H] = cx, icy[H] = cy;
        const double ex = __shfl_down(cx, 4, kWave), ey = __shfl_down(cy, 4, kWave);
        const int ex_r = __shfl_down(r ? 1 : 0, 4, kWave);
        er[H] = g < 7 && ex_r != 0;
        ecx[H] = g < 7 ? ex : 0.0;
        ecy[H] = g < 7 ? ey : 0.0;
        const int src = (lane & 32) | cp;  // group 0 of this half: the half's whole map
        wcx[H] = __shfl(cx, src, kWave);
        wcy[H] = __shfl(cy, src, kWave);
        wr[H] = __shfl(r ? 1 : 0, src, kWave) != 0;
    }
    if (g == 0) {  // the chunk's map: the later half first
        const double cx = wr[0] ? wcx[0] : wcx[0] + wcx[1];
        const double cy = wr[0] ? wcy[0] : wcy[0] + wcy[1];
        lds_ref<double>(lds, Lo.rsum + 8u * (ch * kS + 2 * cp)) = cx;
        lds_ref<double>(lds, Lo.rsum + 8u * (ch * kS + 2 * cp + 1)) = cy;
        if (cp == 0) lds_ref<int32_t>(lds, Lo.rflag + 4u * ch) = wr[0] || wr[1] ? 1 : 0;
    }

    uint32_t vmask = 0u;  // the lane's valid positions
#pragma unroll
    for (int i = 0; i < kP; ++i) {
        const int c = cv[i];
        const bool ok = active && i < n && c >= 0;
        vmask |= ok ? 1u << i : 0u;
        cv[i] = ok ? c : N;  // the last-event table's row (N: the idle slots' row)
    }

    // last events: every event writes its index into its cell's byte of this chunk, earliest
    // position first, so each byte ends with the cell's last event (one lane a slot writes)
    const uint32_t my_dummy = Lo.tdummy + 8u * uint32_t(gl);
#pragma unroll
    for (int i = 0; i < kP; ++i)
        lds[(vmask >> i) & 1u && cp == 0 ? Lo.idx + uint32_t(cv[i] * kChunks + ch) : my_dummy] =
            static_cast<unsigned char>(i * kK + k);
    uint32_t entw[kP / 4] = {};
#pragma unroll
    for (int i = 0; i < kP; ++i) entw[i / 4] |= uint32_t(idx[cv[i] * kChunks + ch]) << (8 * (i % 4));
    auto ent = [&](int i) __attribute__((always_inline)) -> uint32_t {
        return (entw[i / 4] >> (8 * (i % 4))) & 0xffu;
    };
    // the replay's inputs, latest position first, spread over the barrier and the composition
    // (issued at once they stall the wave until the memory system drains them)
    const rsrc_t ry = make_rsrc(a.y + orow, row_bytes);
    const rsrc_t rho = make_rsrc(a.h_old + orow, row_bytes);
    float2 yv[kP], hv[kP];
    auto fetch_c = [&](int i) __attribute__((always_inline)) {
        const uint32_t vo = vrow + uint32_t(i) * pos_bytes;
        yv[i] = ld2(ry, vo);
        hv[i] = ld2(rho, vo);
    };
    // positions issued before the barrier (8 measured 0.3 us faster than 4 once the gates went
    // 6 ahead; 2 and 3 were slower)
    constexpr int kEarly = 8;
#pragma unroll
    for (int i = kP - 1; i >= kP - kEarly; --i) {
        fetch_c(i);
        __builtin_amdgcn_sched_barrier(0);
    }
    HSN_EVMAP_STAMP(2);
    __syncthreads();  // every chunk's summary map

    // R at the chunk's end: d q_T through the later chunks' maps; then each position's share
    // (R after the later positions, plus the position's d q_post, over N), rounded once to fp32
    {
        double Rx = double(dqT.x), Ry = double(dqT.y);
#pragma unroll
        for (int j = kChunks - 1; j > 0; --j) {
            if (j > ch) {
                const bool rj = lds_ref<int32_t>(lds, Lo.rflag + 4u * j) != 0;
                const double cx = lds_ref<double>(lds, Lo.rsum + 8u * (j * kS + 2 * cp));
                const double cy = lds_ref<double>(lds, Lo.rsum + 8u * (j * kS + 2 * cp + 1));
                Rx = (rj ? 0.0 : Rx) + cx;
                Ry = (rj ? 0.0 : Ry) + cy;
            }
        }
        double Rhx[2], Rhy[2];  // R at each half's end
        Rhx[1] = Rx, Rhy[1] = Ry;
        Rhx[0] = (wr[1] ? 0.0 : Rx) + wcx[1];
        Rhy[0] = (wr[1] ? 0.0 : Ry) + wcy[1];
        const double inv = double(divn.inv), nf = double(divn.n);
#pragma unroll
        for (int H = 0; H < 2; ++H) {
            const double bx = (er[H] ? 0.0 : Rhx[H]) + ecx[H] + double(qb[H].x);
            const double by = (er[H] ? 0.0 : Rhy[H]) + ecy[H] + double(qb[H].y);
            const float sx = static_cast<float>(divn.pow2 ? bx * inv : bx / nf);
            const float sy = static_cast<float>(divn.pow2 ? by * inv : by / nf);
            lds_ref<float2>(lds, Lo.share + 4u * uint32_t((ch * kP + 8 * H + g) * kS + 2 * cp)) =
                make_float2(sx, sy);
        }
        if (a.dq0 && ch == 0 && g == 0) {  // R after position 0
            const double sx = (wr[0] ? 0.0 : Rhx[0]) + wcx[0], sy = (wr[0] ? 0.0 : Rhy[0]) + wcy[0];
            a.dq0[size_t(b) * d + col] = static_cast<float>(sx);
            a.dq0[size_t(b) * d + col + 1] = static_cast<float>(sy);
        }
    }
    HSN_EVMAP_STAMP(3);
    const uint32_t sh_base = Lo.share + 4u * uint32_t(ch * kP * kS + 2 * cp);
    auto share_at = [&](int i) __attribute__((always_inline)) -> float2 {
        return lds_ref<float2>(lds, sh_base + uint32_t(i) * kS * 4u);
    };
    const uint32_t lofs = uint32_t(cp) * 8u;
    auto mu_at = [&](uint32_t e) __attribute__((always_inline)) -> float2& {
        return lds_ref<float2>(lds, cbase + e * kEntBytes + lofs);
    };
    auto nu_at = [&](uint32_t e) __attribute__((always_inline)) -> float2& {
        return lds_ref<float2>(lds, cbase + kEnt * kEntBytes + e * kEntBytes + lofs);
    };
    // zero the maps of entries [e_begin, kEv) (a reset: the entries created so far)
    auto zero_from = [&](int e_begin, bool with_nu) __attribute__((always_inline)) {
        for (int e = e_begin * 4 + hl; e < kEv * 4; e += 32) {
            const uint32_t at = cbase + uint32_t(e >> 2) * kEntBytes + uint32_t(e & 3) * 8u;
            lds_ref<float2>(lds, at) = make_float2(0.0f, 0.0f);
            if (with_nu) lds_ref<float2>(lds, at + kEnt * kEntBytes) = make_float2(0.0f, 0.0f);
        }
    };

    // compose the chunk's maps latest position first: mu' = (1 - b) mu, nu' = (1 - b) (nu + dsel)
    // - b s, an entry's first (latest) event from (1, 0), or (0, 0) once a reset has passed; a
    // reset zeroes the entries created so far. Idle and padded slots compose the identity on
    // kDummy (their b s term is an exact zero, whatever the share holds). Each position's gate
    // comes first (its rows are the oldest of the gates in flight); the gates kAhead positions on
    // and the replay's rows kEarly on go out as each position is taken.
    // One code path for chunks with and without resets: the replay's loads issued here stay in
    // flight through the barrier below, where two paths would join with different loads pending
    // and the join would wait for all of them.
    [[maybe_unused]] const bool wave_rs = ballot(rmask != 0u) != 0u;  // a reset in the wave's chunks
    HSN_EVMAP_NOTE(9, wave_rs ? 1u : 0u);
    float2 omb[kP], dsv[kP];
    {
        float ainit = 1.0f;
#pragma unroll
        for (int i = kP - 1; i >= 0; --i) {
            if (i - kAhead >= 0) fetch(i - kAhead);
            if (i - kEarly >= 0) {
                fetch_c(i - kEarly);
                __builtin_amdgcn_sched_barrier(0);
            }
            {
                const bool ok = (vmask >> i) & 1u;
                const float b0 = fast_sigmoid(gv[i].x), b1 = fast_sigmoid(gv[i].y);
                omb[i] = ok ? make_float2(1.0f - b0, 1.0f - b1) : make_float2(1.0f, 1.0f);
                dsv[i] = ok ? dv[i] : make_float2(0.0f, 0.0f);
            }
            const uint32_t e = ent(i);
            const bool first = e == uint32_t(i * kK + k);
            const float2 sh = share_at(i);
            const float2 mu = mu_at(e), nu = nu_at(e);
            const float2 o = omb[i];
            const uint32_t vm = bitmask_at(vmask, i);
            const float bsx = and_f32((1.0f - o.x) * sh.x, vm), bsy = and_f32((1.0f - o.y) * sh.y, vm);
            mu_at(e) = make_float2(o.x * (first ? ainit : mu.x), o.y * (first ? ainit : mu.y));
            nu_at(e) = make_float2(o.x * ((first ? 0.0f : nu.x) + dsv[i].x) - bsx,
                                   o.y * ((first ? 0.0f : nu.y) + dsv[i].y) - bsy);
            if ((rmask >> i) & 1u) {
                zero_from(i * kK, true);
                ainit = 0.0f;
            }
            // the replay reads the slot's validity from here: 1 - b is never -1 (it is in [0, 1],
            // or NaN from a NaN gate, which the replay propagates as before)
            omb[i] = (vmask >> i) & 1u ? o : make_float2(-1.0f, -1.0f);
        }
    }

    __syncthreads();

    HSN_EVMAP_STAMP(4);
    // ---- phase B: every cell from d_h_T back through the 16 chunks, two threads a cell -------
    {
        uint32_t rflags = 0u;  // chunks with a reset
#pragma unroll
        for (int j = 0; j < kChunks; ++j)
            rflags |= lds_ref<int32_t>(lds, Lo.rflag + 4u * j) != 0 ? 1u << j : 0u;
        rflags = uniform(rflags);
        float* const dh0_row = a.dh0 ? a.dh0 + size_t(b) * N * d : nullptr;
        const uint32_t qofs = uint32_t(bq) * 16u;
        auto walk = [&](int cell, float4 s) __attribute__((always_inline)) {
            const bool ok = cell < N;
            const uint4 iw = lds_ref<uint4>(lds, Lo.idx + uint32_t(ok ? cell : N) * kChunks);
            const uint32_t words[4] = {ok ? iw.x : ~0u, ok ? iw.y : ~0u, ok ? iw.z : ~0u, ok ? iw.w : ~0u};
#pragma unroll
            for (int jh = kChunks - kChunks / 4; jh >= 0; jh -= kChunks / 4) {  // four chunks at once
                float4 mu[kChunks / 4], nu[kChunks / 4];
#pragma unroll
                for (int jj = 0; jj < kChunks / 4; ++jj) {
                    const int j = jh + jj;
                    const uint32_t ej = (words[j / 4] >> (8 * (j % 4))) & 0xffu;
                    const uint32_t e = ej == kNone ? uint32_t(kDummy) : ej;  // the identity (1, 0)
                    const uint32_t at = Lo.maps + uint32_t(j) * kMapBytes + e * kEntBytes + qofs;
                    mu[jj] = lds_ref<float4>(lds, at);
                    nu[jj] = lds_ref<float4>(lds, at + kEnt * kEntBytes);
                }
#pragma unroll
                for (int jj = kChunks / 4 - 1; jj >= 0; --jj) {
                    const int j = jh + jj;
                    const uint32_t ej = (words[j / 4] >> (8 * (j % 4))) & 0xffu;
                    // the entry's cotangent at the chunk's end, for the replay
                    if (ej != kNone)
                        lds_ref<float4>(lds, Lo.maps + uint32_t(j) * kMapBytes + ej * kEntBytes + qofs) = s;
                    // a chunk with a reset ends at nu whatever came after (a select, not 0 * A)
                    if ((rflags >> j) & 1u) s = nu[jj];
                    else s = make_float4(mu[jj].x * s.x + nu[jj].x, mu[jj].y * s.y + nu[jj].y,
                                         mu[jj].z * s.z + nu[jj].z, mu[jj].w * s.w + nu[jj].w);
                }
            }
            if (ok && dh0_row)
                *reinterpret_cast<float4*>(dh0_row + int64_t(cell) * d + slice * kS + 4 * bq) = s;
        };
        // the first 256 cells from the values loaded at the start, in straight-line code: a
        // load inside the loop would make its first use wait for every load in flight, the
        // replay's inputs included
        walk(gl >> 1, dha);
        for (int c0 = kWave * kWaves / 2; c0 < N; c0 += kWave * kWaves / 2)
            walk(c0 + (gl >> 1), dhT_at(c0 + (gl >> 1)));
    }
    __syncthreads();

    HSN_EVMAP_STAMP(5);
    // ---- phase C: the replay, latest position first ------------------------------------------
    // the selection cotangents move to the chunk's nu table (free after phase B): 32 lanes x 16
    // positions x 8 bytes
    const uint32_t ds_base = cbase + kEnt * kEntBytes + uint32_t(hl) * 8u;
#pragma unroll
    for (int i = 0; i < kP; ++i) lds_ref<float2>(lds, ds_base + uint32_t(i) * 256u) = dsv[i];
    const rsrc_t rdy = make_rsrc(a.dy + orow, row_bytes);
    const rsrc_t rdg = make_rsrc(a.dg + orow, row_bytes);
    uint32_t vrow_c = vrow;
    asm volatile("" : "+v"(vrow_c));  // recomputed here, not held from phase A's loads
    // One code path for every wavefront, as in the forward's replay. The next position's entry,
    // selection cotangent and share are read right after this position's write (its entry may
    // be the one just written: LDS keeps one wave's accesses in order); a reset zeroes the entries
    // after that read, so the value is taken as zero.
    {
        float2 A = mu_at(ent(kP - 1));
        float2 ds = lds_ref<float2>(lds, ds_base + uint32_t(kP - 1) * 256u);
        float2 sh = share_at(kP - 1);
#pragma unroll
        for (int i = kP - 1; i >= 0; --i) {
            const uint32_t e = ent(i);
            const float2 o = omb[i];
            const float2 carried = make_float2(A.x + ds.x, A.y + ds.y);
            const float2 G = make_float2(carried.x + sh.x, carried.y + sh.y);
            const float bgx = 1.0f - o.x, bgy = 1.0f - o.y;
            mu_at(e) = make_float2(o.x * carried.x - bgx * sh.x, o.y * carried.y - bgy * sh.y);
            if (i > 0) {
                A = mu_at(ent(i - 1));
                ds = lds_ref<float2>(lds, ds_base + uint32_t(i - 1) * 256u);
                sh = share_at(i - 1);
            }
            const float cx = fast_tanh(yv[i].x), cy = fast_tanh(yv[i].y);
            const uint32_t vm = o.x == -1.0f ? 0u : ~0u;  // -1 marks an idle or padded slot
            const float dcx = and_f32(bgx * (1.0f - cx * cx) * G.x, vm);
            const float dcy = and_f32(bgy * (1.0f - cy * cy) * G.y, vm);
            const float dbx = and_f32((cx - hv[i].x) * (o.x * bgx) * G.x, vm);
            const float dby = and_f32((cy - hv[i].y) * (o.y * bgy) * G.y, vm);
            const uint32_t vo = i < n ? vrow_c + uint32_t(i) * pos_bytes : kOob;
            st2(make_float2(dcx, dcy), rdy, vo);
            st2(make_float2(dbx, dby), rdg, vo);
            if ((rmask >> i) & 1u) {  // every cotangent restarts at 0 (straight-line writes)
#pragma unroll
                for (int q = 0; q < kEv * 4 / 32; ++q) {
                    const int ee = hl + 32 * q;
                    lds_ref<float2>(lds, cbase + uint32_t(ee >> 2) * kEntBytes + uint32_t(ee & 3) * 8u) =
                        make_float2(0.0f, 0.0f);
                }
                A = make_float2(0.0f, 0.0f);
            }
        }
    }
    HSN_EVMAP_STAMP(6);
    HSN_EVMAP_STAMPS_END(1);
}

}  // namespace evmap
}  // namespace hsn
