// The window's sweeps by column strips (gfx950), for rows whose decisions fit a workgroup's LDS.
//
// A workgroup owns (row b, strip of S = 8 consecutive columns; the last strip may hold 4) for
// every cell of the row. Everything the row needs beyond its own inputs and outputs stays in the
// workgroup, so each direction is one kernel with no workspace:
//   lists    the row's decisions as per-cell event lists in LDS, in time order (an event word is
//            t << 13 | the slot's index t K + k), the padded slots after them; ranks from a bit
//            per (cell, position): deterministic;
//   walk     each cell's chain in an aligned pair of lanes, 4 columns per lane (one 16-byte
//            access per lane and row), 32 consecutive cells per wavefront; a batch's event words,
//            next resets and rows are fetched ahead of the batch before it;
//   summary  forward: each valid slot's fp32 delta h_sel - h_old goes to its own LDS words (a
//            padded slot's hold +0), so the position's sum D[t] over its slots in slot order is
//            the chains' exact arithmetic (as the cell-chain path's summary), then a scan over
//            time of D / N with the resets; backward: the summary cotangent's reverse scan (fp64)
//            first, its share R / N per position kept in LDS for the chains;
//   maxima   (forward) the row maximum of |h| per position: every cell's value is constant
//            between its events, so each interval [lo, hi) of a value v is a range-max update.
//            The walk records one (lo, hi, v) per event and per cell's last interval; a pass
//            over the records (a record per lane) posts each as two LDS atomics on a sparse
//            table (level k = floor(log2(hi - lo)) at lo and at hi - 2^k), pushed down level by
//            level, then max-reduced across the row's strips with a global atomic (h_max holds 0
//            on entry).
//
// Reference: as the cell-chain path (chain.cuh): the forward restates
// python/hsn/kernels/native.py:244-303 with python/hsn/model/state.py:267-324 per position, the
// backward python/hsn/train/split.py:128-174 with the carried state
// (python/hsn/train/state_gradient.py:402-416).
#pragma once

#include "chain.cuh"

namespace hsn {
namespace strip {

constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kCols = 8;         // columns per strip
constexpr int kVec = 4;          // columns per lane
constexpr int kPair = kCols / kVec;  // lanes per cell
constexpr int kCPW = 64 / kPair;     // cells per wavefront
constexpr int kMaxU = 16;        // slots of the row per thread: T * K <= 8192, 4 per load
constexpr int kSlotBits = 13;    // an event word: t << 13 | slot index (T * K <= 8192)
constexpr int kSlotMask = (1 << kSlotBits) - 1;
constexpr int kNBF = 8;          // events per fetched batch of a sub-chain: forward
constexpr int kNBB = 4;          // backward (four rows per event)

using f4 = float __attribute__((ext_vector_type(4)));
using u4 = uint32_t __attribute__((ext_vector_type(4)));
using u2 = uint32_t __attribute__((ext_vector_type(2)));

// Four consecutive columns of a row as one buffer access: fp32 rows 16 bytes, bf16 rows 8 (the
// raw words are kept until use; widened exactly, narrowed round-to-nearest-even).
template <typename IO>
struct Vec4;
template <>
struct Vec4<float> {
    using Raw = u4;
    __device__ static Raw load(rsrc_t r, uint32_t vo) {
        return __builtin_amdgcn_raw_buffer_load_b128(r, vo, 0u, 0);
    }
    __device__ static f4 widen(Raw v) {
        return f4{__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z),
                  __uint_as_float(v.w)};
    }
    __device__ static void store(f4 v, rsrc_t r, uint32_t vo) {
        const u4 w{__float_as_uint(v.x), __float_as_uint(v.y), __float_as_uint(v.z),
                   __float_as_uint(v.w)};
        __builtin_amdgcn_raw_buffer_store_b128(w, r, vo, 0u, 0);
    }
};
template <>
struct Vec4<bf16_t> {
    using Raw = u2;
    __device__ static Raw load(rsrc_t r, uint32_t vo) {
        return __builtin_amdgcn_raw_buffer_load_b64(r, vo, 0u, 0);
    }
    __device__ static f4 widen(Raw v) {
        return f4{__uint_as_float(v.x << 16), __uint_as_float(v.x & 0xffff0000u),
                  __uint_as_float(v.y << 16), __uint_as_float(v.y & 0xffff0000u)};
    }
    __device__ static void store(f4 v, rsrc_t r, uint32_t vo) {
        const u2 w{uint32_t(from_f32<bf16_t>(v.x).bits) | (uint32_t(from_f32<bf16_t>(v.y).bits) << 16),
                   uint32_t(from_f32<bf16_t>(v.z).bits) | (uint32_t(from_f32<bf16_t>(v.w).bits) << 16)};
        __builtin_amdgcn_raw_buffer_store_b64(w, r, vo, 0u, 0);
    }
};

__device__ __forceinline__ f4 f4_load_f32(rsrc_t r, uint32_t vo) {
    return Vec4<float>::widen(Vec4<float>::load(r, vo));
}

__host__ __device__ inline int levels_of(int T) {  // sparse-table levels: floor(log2 T) + 1
    int l = 1;
    while ((2 << (l - 1)) <= T) ++l;
    return l;
}

// LDS word offsets of a strip workgroup (regions of 16-byte multiples).
struct Layout {
    int nr, rbits, nx, cnt, ptr, misc, pbits, ppre, ev, xch, traj, share, sparse, rec, uni, words;
};
__host__ __device__ inline int al4(int v) { return (v + 3) & ~3; }
__host__ __device__ inline Layout layout(int T, int N, int K, bool fwd) {
    const int S = kCols;
    const int TW = (T + 31) / 32, PW = (T * K + 31) / 32;
    Layout L{};
    int at = 0;
    L.nr = at, at = al4(at + T + 2);
    L.rbits = at, at = al4(at + TW);
    L.nx = at, at = al4(at + TW + 1);
    L.cnt = at, at = al4(at + N);
    L.ptr = at, at = al4(at + N + 1);
    L.misc = at, at = al4(at + 4);
    L.pbits = at, at = al4(at + PW);
    L.ppre = at, at = al4(at + PW + 1);
    L.ev = at, at = al4(at + T * K);
    L.xch = at, at = al4(at + 3 * kWaves * S);  // the scan's per-wavefront maps (fp64: backward)
    L.rec = at, at = al4(at + (fwd ? 2 * (T * K + N) : 0));  // (lo | hi << 16, v) per interval
    L.traj = at, at = al4(at + (fwd ? T * S : 0));   // cell 0's state after each of its events
    L.share = at, at = al4(at + (fwd ? 0 : T * S));  // the summary cotangent's share per position
    L.sparse = at, at = al4(at + (fwd ? T * levels_of(T) : 0));
    // the list build's bits per (cell, position), then the forward's slot deltas (a position's
    // K * S words and S words of padding, so a wavefront over 8 positions reads 8 bank groups;
    // 4 spare words per lane) or the backward's staged summary cotangents (2 T S words)
    L.uni = at;
    const int mask = N * TW, other = fwd ? T * (K + 1) * S + 64 * kVec : 2 * T * S;
    at += mask > other ? mask : other;
    L.words = at;
    return L;
}

// (row, strip) from the grid (8, nstrips, B/8) (or (1, nstrips, B)): a row's strips share an XCD,
// so the row's decisions and its slot rows' cache lines are fetched into one L2.
__device__ __forceinline__ void strip_coords(int& b, int& sp) {
    b = blockIdx.x * gridDim.z + blockIdx.z;
    sp = blockIdx.y;
}
inline dim3 strip_grid(int B, int nstrips) {
    const int x = B % 8 == 0 ? 8 : 1;
    return dim3(x, nstrips, B / x);
}

// Inclusive prefix sum over the wavefront with DPP (row shifts, then the gfx9 row broadcasts);
// every lane active.
__device__ __forceinline__ int wave_incl_sum(int v) {
    v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, false);  // row_shr:1
    v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, false);  // row_shr:2
    v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, false);  // row_shr:4
    v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, false);  // row_shr:8
    v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false);  // row_bcast:15
    v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false);  // row_bcast:31
    return v;
}

// Exclusive prefix sum of val(0 .. n) into put(i, prefix) by one wavefront, a chunk of
// consecutive entries per lane; returns the total.
template <typename F, typename G>
__device__ __forceinline__ int wave_scan_chunks(int n, int lane, F val, G put) {
    const int per = (n + 63) / 64;
    const int i0 = min(n, lane * per), i1 = min(n, i0 + per);
    int s = 0;
    for (int i = i0; i < i1; ++i) s += val(i);
    const int incl = wave_incl_sum(s);
    int run = incl - s;
    for (int i = i0; i < i1; ++i) {
        const int v = val(i);
        put(i, run);
        run += v;
    }
    return readlane(incl, 63);
}

// Slot u of this thread: i = 4 (tid + (u / 4) kThreads) + u % 4 (four consecutive slots per
// 16-byte load).
__device__ __forceinline__ int slot_of(int tid, int u) {
    return 4 * (tid + (u / 4) * kThreads) + (u & 3);
}

// The row's decisions, kMaxU slots per thread: the cell, -1 on a padded slot (or a cell outside
// [0, N)), -2 past the row.
__device__ __forceinline__ void load_slots(int (&cs)[kMaxU], const int32_t* slots_row,
                                           int n_slots, int N, int tid) {
    const rsrc_t rs = make_rsrc(slots_row, uint32_t(n_slots) * 4u);
#pragma unroll
    for (int gq = 0; gq < kMaxU / 4; ++gq) {
        const int i0 = slot_of(tid, 4 * gq);
        // the row's end masks whole groups (n_slots % 4 == 0 is not assumed: a partial group
        // loads lane by lane)
        if (i0 + 4 <= n_slots) {
            const u4 v = __builtin_amdgcn_raw_buffer_load_b128(rs, uint32_t(i0) * 4u, 0u, 0);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int c = int(v[e]);
                cs[4 * gq + e] = c >= 0 && c < N ? c : -1;
            }
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int i = i0 + e;
                const int c = i < n_slots ? slots_row[i] : -2;
                cs[4 * gq + e] = c == -2 ? -2 : (c >= 0 && c < N ? c : -1);
            }
        }
    }
}

// t = i / K for i < 8192, K <= 255: the high word of i * ceil(2^32 / K) (exact: the rounding of
// the multiplier adds less than 2^-19 to i / K, below the gap 1 / K to the next integer).
__device__ __forceinline__ int div_k(int i, uint32_t magic) { return int(__umulhi(uint32_t(i), magic)); }

// The row's per-cell event lists in LDS: cnt[c] events of cell c at ev[ptr[c] ..), in time
// order, the padded slots at ev[ptr[N] ..) in time order, their bits per slot in pbits. Ends with
// a barrier. `mask` [N][TW] is scratch; cnt, pbits and mask must hold zeros on entry (behind a
// barrier).
struct Lists {
    int* cnt;
    int* ptr;
    uint32_t* pbits;
    int* ppre;
    int* ev;
    uint32_t* mask;
};
__device__ __forceinline__ void build_lists(const Lists& l, const int (&cs)[kMaxU], int T, int N,
                                            int K, int tid) {
    const int TW = (T + 31) / 32, PW = (T * K + 31) / 32;
    const int lane = tid & 63, wv = tid >> 6;
    const uint32_t magic = uint32_t((0x100000000ull + K - 1) / K);
#pragma unroll
    for (int u = 0; u < kMaxU; ++u) {
        const int i = slot_of(tid, u);
        if (cs[u] >= 0) {
            const int t = div_k(i, magic);
            atomicAdd(&l.cnt[cs[u]], 1);
            atomicOr(&l.mask[cs[u] * TW + (t >> 5)], 1u << (t & 31));
        } else if (cs[u] == -1) {
            atomicOr(&l.pbits[i >> 5], 1u << (i & 31));
        }
    }
    __syncthreads();
    if (wv == 0) {
        const int total = wave_scan_chunks(
            N, lane, [&](int c) { return l.cnt[c]; }, [&](int c, int p) { l.ptr[c] = p; });
        if (lane == 0) l.ptr[N] = total;
    } else if (wv == 1) {  // the padded slots' prefix per word
        const int total = wave_scan_chunks(
            PW, lane, [&](int w) { return __popc(l.pbits[w]); },
            [&](int w, int p) { l.ppre[w] = p; });
        if (lane == 0) l.ppre[PW] = total;
    }
    __syncthreads();
    const int n_valid = l.ptr[N];
#pragma unroll
    for (int u = 0; u < kMaxU; ++u) {
        const int i = slot_of(tid, u);
        const int c = cs[u];
        if (c == -2) continue;
        const int t = div_k(i, magic);
        const int word = (t << kSlotBits) | i;
        if (c >= 0) {
            const uint32_t* m = l.mask + c * TW;
            int rank = __popc(m[t >> 5] & ((1u << (t & 31)) - 1u));
            for (int w = 0; w < (t >> 5); ++w) rank += __popc(m[w]);
            l.ev[l.ptr[c] + rank] = word;
        } else {
            const int r = l.ppre[i >> 5] + __popc(l.pbits[i >> 5] & ((1u << (i & 31)) - 1u));
            l.ev[n_valid + r] = word;
        }
    }
    __syncthreads();
}

__device__ __forceinline__ int wave_max_int(int v) {  // v >= 0
    return int(wave_max_from_groups<1>(uint32_t(v)));
}

__device__ __forceinline__ uint32_t umax4(f4 v) {
    return umax(umax(abs_bits(v.x), abs_bits(v.y)), umax(abs_bits(v.z), abs_bits(v.w)));
}
__device__ __forceinline__ f4 sel4(bool c, f4 a, f4 b) {
    return f4{c ? a.x : b.x, c ? a.y : b.y, c ? a.z : b.z, c ? a.w : b.w};
}

// ------------------------------------------------------------------------------------------
// Forward
// ------------------------------------------------------------------------------------------

struct FwdArgs {
    const void* y;  // [B, T, K, d] io: the candidate's pre-activation (the RMS prologue's output)
    const void* g;  // the write gate's pre-activation
    const int32_t* slots;  // [B, T, K]: the cell, or -1 on a padded slot
    const uint8_t* reset;  // [B, T] (null: none)
    const float* h0;       // [B, N, d]
    const float* q0;       // [B, d]
    const int64_t* age0;   // [B, N] (with age_T)
    const int64_t* pos0;   // [B] (with pos_T)
    void* q_pre;           // [B, T, d] io (optional)
    void* q_post;          // (optional)
    void* h_old;           // [B, T, K, d] io (optional)
    void* h_sel;           // (optional)
    float* h_max;          // [B, T] (optional; holds 0 on entry)
    float* h_T;            // [B, N, d] (optional)
    float* q_T;            // [B, d] (optional)
    int64_t* age_T;        // [B, N] (optional)
    int64_t* pos_T;        // [B] (optional)
    int B, T, N, d, K;
    DivN divn;
};

template <typename IO, bool HMAX>
__global__ __launch_bounds__(kThreads) void strip_fwd(FwdArgs a) {
    extern __shared__ uint32_t lds_u[];
    constexpr int S = kCols, NB = kNBF;
    using VI = Vec4<IO>;
    int b, sp;
    strip_coords(b, sp);
    const int tid = threadIdx.x, lane = lane_id(), wv = tid >> 6;
    const int T = a.T, N = a.N, d = a.d, K = a.K;
    const int n_slots = T * K;
    int cs[kMaxU];  // the row's decisions, in flight while the LDS is prepared
    load_slots(cs, a.slots + int64_t(b) * n_slots, n_slots, N, tid);
    const Layout Lo = layout(T, N, K, true);
    int* nr = reinterpret_cast<int*>(lds_u + Lo.nr);
    uint32_t* rbits = lds_u + Lo.rbits;
    int* nx = reinterpret_cast<int*>(lds_u + Lo.nx);
    int* cnt = reinterpret_cast<int*>(lds_u + Lo.cnt);
    int* ptr = reinterpret_cast<int*>(lds_u + Lo.ptr);
    int* misc = reinterpret_cast<int*>(lds_u + Lo.misc);
    uint32_t* pbits = lds_u + Lo.pbits;
    int* ppre = reinterpret_cast<int*>(lds_u + Lo.ppre);
    int* ev = reinterpret_cast<int*>(lds_u + Lo.ev);
    float* xch = reinterpret_cast<float*>(lds_u + Lo.xch);
    uint2* rec = reinterpret_cast<uint2*>(lds_u + Lo.rec);
    float* traj = reinterpret_cast<float*>(lds_u + Lo.traj);
    uint32_t* sparse = lds_u + Lo.sparse;
    uint32_t* mask = lds_u + Lo.uni;
    float* dk = reinterpret_cast<float*>(lds_u + Lo.uni);
    const int TW = (T + 31) / 32, PW = (T * K + 31) / 32;
    const int LV = levels_of(T);
    for (int i = tid; i < N; i += kThreads) cnt[i] = 0;
    for (int i = tid; i < PW; i += kThreads) pbits[i] = 0u;
    for (int i = tid; i < N * TW; i += kThreads) mask[i] = 0u;
    if constexpr (HMAX)
        for (int i = tid; i < T * LV; i += kThreads) sparse[i] = 0u;
    if (tid == 0) misc[0] = 0;
    const int lrT = chain::reset_table(a.reset ? a.reset + int64_t(b) * T : nullptr, T, nr, rbits,
                                       nx, tid, kThreads);
    build_lists(Lists{cnt, ptr, pbits, ppre, ev, mask}, cs, T, N, K, tid);
    const int n_valid = ptr[N];
    // a padded slot's deltas are +0 (the list build's bits, aliased here, are dead); the deltas
    // of slot i = t K + k sit at (i + t) S
    const uint32_t magic = uint32_t((0x100000000ull + K - 1) / K);
#pragma unroll
    for (int u = 0; u < kMaxU; ++u)
        if (cs[u] == -1) {
            const int i = slot_of(tid, u);
            f4* p = reinterpret_cast<f4*>(dk + (i + div_k(i, magic)) * S);
#pragma unroll
            for (int v = 0; v < S / kVec; ++v) p[v] = f4{0.0f, 0.0f, 0.0f, 0.0f};
        }

    // the walk
    const int64_t slot0 = int64_t(b) * n_slots;
    const uint32_t row_bytes = uint32_t(n_slots) * d * sizeof(IO);
    const rsrc_t ry = make_rsrc(static_cast<const IO*>(a.y) + slot0 * d, row_bytes);
    const rsrc_t rg = make_rsrc(static_cast<const IO*>(a.g) + slot0 * d, row_bytes);
    const rsrc_t rho = make_rsrc(a.h_old ? static_cast<IO*>(a.h_old) + slot0 * d : nullptr,
                                 a.h_old ? row_bytes : 0u);
    const rsrc_t rhs = make_rsrc(a.h_sel ? static_cast<IO*>(a.h_sel) + slot0 * d : nullptr,
                                 a.h_sel ? row_bytes : 0u);
    const rsrc_t rh0 = make_rsrc(a.h0 + int64_t(b) * N * d, uint32_t(N) * d * 4u);
    const rsrc_t rhT = make_rsrc(a.h_T ? a.h_T + int64_t(b) * N * d : nullptr,
                                 a.h_T ? uint32_t(N) * d * 4u : 0u);
    const int x = lane % kPair, j = lane / kPair;
    const int col = sp * S + x * kVec;  // the lane's first column (d % 4 == 0)
    const bool colok = col < d;
    const uint32_t srow = uint32_t(d) * sizeof(IO), colb = uint32_t(col) * sizeof(IO);
    const int ntask = (N + kCPW - 1) / kCPW;
    const bool track_age = a.age_T != nullptr && sp == 0;
    const int spare = (n_slots + T) * S + lane * kVec;  // a lane without an event writes here
    for (;;) {
        int task = lane == 0 ? atomicAdd(&misc[0], 1) : 0;
        task = uniform(task);
        if (task >= ntask) break;
        const int oi = task * kCPW + j;
        const bool has = oi < N;
        const int c = oi;
        const int n = has ? cnt[c] : 0;
        const int base = has ? ptr[c] : 0;
        const int nmax = wave_max_int(n);
        const int elast = max(n - 1, 0);
        const bool is0 = has && c == 0;
        const uint32_t vc = has && colok ? uint32_t(c * d + col) * 4u : kOob;
        f4 h = f4_load_f32(rh0, vc);
        int s = 0;            // the latest event's position (0 before the first)
        int nrprev = nr[0];   // the first reset after it
        uint32_t vprev = 0u;  // the bits of max |h| over the cell's strip columns since s
        struct Batch {
            int q[NB];        // event word (-1: none)
            int nq[NB];       // the first reset after its position
            uint32_t vo[NB];  // its row's byte offset (kOob: none)
            typename VI::Raw y[NB], g[NB];
        };
        // every lane reads an event word (its own, or its list's last: no branch), then selects
        auto fetch = [&](int e0, Batch& bt) __attribute__((always_inline)) {
#pragma unroll
            for (int i = 0; i < NB; ++i) bt.q[i] = ev[base + min(e0 + i, elast)];
#pragma unroll
            for (int i = 0; i < NB; ++i) {
                const bool ok = e0 + i < n;
                const int q = bt.q[i];
                bt.q[i] = ok ? q : -1;
                bt.nq[i] = nr[ok ? (q >> kSlotBits) + 1 : 0];
                bt.vo[i] = ok && colok ? uint32_t(q & kSlotMask) * srow + colb : kOob;
                bt.y[i] = VI::load(ry, bt.vo[i]);
                bt.g[i] = VI::load(rg, bt.vo[i]);
            }
        };
        auto step = [&](int e0, const Batch& bt) __attribute__((always_inline)) {
#pragma unroll
            for (int i = 0; i < NB; ++i) {
                if (e0 + i >= nmax) break;
                const int q = bt.q[i];
                const bool ok = q >= 0;
                const int t = q >> kSlotBits, sl = q & kSlotMask;
                const bool zero = nrprev <= t;  // a reset since the cell's latest event
                if constexpr (HMAX)
                    if (x == 0 && ok)
                        rec[base + e0 + i] =
                            make_uint2(uint32_t(s) | (uint32_t(min(t, nrprev)) << 16), vprev);
                const f4 hold = zero ? f4{0.0f, 0.0f, 0.0f, 0.0f} : h;
                const f4 yv = VI::widen(bt.y[i]), gv = VI::widen(bt.g[i]);
                f4 hn;
#pragma unroll
                for (int v = 0; v < kVec; ++v) {
                    const float bg = fast_sigmoid(gv[v]);
                    const float cand = fast_tanh(yv[v]);
                    hn[v] = (1.0f - bg) * hold[v] + bg * cand;
                }
                VI::store(hold, rho, bt.vo[i]);
                VI::store(hn, rhs, bt.vo[i]);
                *reinterpret_cast<f4*>(dk + (ok ? (sl + t) * S + x * kVec : spare)) = hn - hold;
                if (unlikely(is0 && ok)) *reinterpret_cast<f4*>(traj + (e0 + i) * S + x * kVec) = hn;
                h = sel4(ok, hn, h);
                if constexpr (HMAX) {
                    const uint32_t vm = group_max<kPair>(umax4(h));
                    vprev = ok ? vm : vprev;
                }
                s = ok ? t : s;
                nrprev = ok ? bt.nq[i] : nrprev;
            }
        };
        Batch b0, b1;
        fetch(0, b0);
        if constexpr (HMAX) vprev = group_max<kPair>(umax4(h));  // (after the fetch is issued)
        for (int e0 = 0; e0 < nmax; e0 += 2 * NB) {
            if (e0 + NB < nmax) fetch(e0 + NB, b1);
            step(e0, b0);
            if (e0 + NB >= nmax) break;
            if (e0 + 2 * NB < nmax) fetch(e0 + 2 * NB, b0);
            step(e0 + NB, b1);
        }
        if constexpr (HMAX)  // the cell's last interval
            if (has && x == 0)
                rec[n_slots + c] = make_uint2(uint32_t(s) | (uint32_t(min(T, nrprev)) << 16), vprev);
        const bool cleared = nrprev < T;  // a reset after the cell's latest event
        Vec4<float>::store(cleared ? f4{0.0f, 0.0f, 0.0f, 0.0f} : h, rhT, vc);
        if (track_age && has && x == 0) {
            const int tprev = n > 0 ? s : -1;
            int64_t age;
            if (tprev >= 0 && tprev >= lrT) age = (T - 1) - tprev;
            else if (lrT >= 0) age = T - lrT;
            else age = a.age0[int64_t(b) * N + c] + T;
            a.age_T[int64_t(b) * N + c] = age;
        }
    }
    if (a.pos_T && sp == 0 && tid == 0) a.pos_T[b] = lrT >= 0 ? int64_t(T - lrT) : a.pos0[b] + T;
    __syncthreads();

    // the padded slots: cell 0's state before and after the position's update (a column per
    // thread)
    const int n_pad = n_slots - n_valid;
    if (n_pad > 0 && (a.h_old || a.h_sel)) {
        const int xs = tid % S, colp = sp * S + xs;
        const bool cok = colp < d;
        const int n0 = cnt[0], e00 = ptr[0];
        const float h0x = cok ? a.h0[int64_t(b) * N * d + colp] : 0.0f;
        for (int pi = tid / S; pi < n_pad; pi += kThreads / S) {
            const int q = ev[n_valid + pi];
            const int t = q >> kSlotBits;
            int lo = 0, hi = n0;  // the number of cell 0's events at or before t
            while (lo < hi) {
                const int mid = (lo + hi) >> 1;
                if ((ev[e00 + mid] >> kSlotBits) <= t) lo = mid + 1;
                else hi = mid;
            }
            float before, after;
            if (lo > 0 && (ev[e00 + lo - 1] >> kSlotBits) == t) {  // cell 0 was updated at t
                after = traj[(lo - 1) * S + xs];
                const int tp = lo >= 2 ? (ev[e00 + lo - 2] >> kSlotBits) : -1;
                const float prior = lo >= 2 ? traj[(lo - 2) * S + xs] : h0x;
                before = nr[tp + 1] <= t ? 0.0f : prior;
            } else {
                const int tp = lo > 0 ? (ev[e00 + lo - 1] >> kSlotBits) : -1;
                const float v = lo > 0 ? traj[(lo - 1) * S + xs] : h0x;
                before = after = nr[tp + 1] <= t ? 0.0f : v;
            }
            const uint32_t vo = cok ? uint32_t(q & kSlotMask) * srow + uint32_t(colp) * sizeof(IO) : kOob;
            bstore_f32<IO>(before, rho, vo, 0u);
            bstore_f32<IO>(after, rhs, vo, 0u);
        }
    }

    // the row maxima: post the intervals (a record per lane), push the sparse table down, then
    // max-reduce across the strips
    if constexpr (HMAX) {
        for (int r = tid; r < n_valid + N; r += kThreads) {
            const uint2 v = rec[r < n_valid ? r : n_slots + (r - n_valid)];
            const int lo = int(v.x & 0xffffu), hi = int(v.x >> 16);
            if (hi > lo && v.y != 0u) {
                const int k = 31 - __builtin_clz(hi - lo);
                atomicMax(&sparse[k * T + lo], v.y);
                atomicMax(&sparse[k * T + hi - (1 << k)], v.y);
            }
        }
        __syncthreads();
        for (int k = LV - 1; k >= 1; --k) {
            const int half = 1 << (k - 1);
            for (int p = tid; p < T; p += kThreads) {
                uint32_t v = sparse[(k - 1) * T + p];
                v = umax(v, sparse[k * T + p]);
                if (p >= half) v = umax(v, sparse[k * T + p - half]);
                sparse[(k - 1) * T + p] = v;
            }
            __syncthreads();
        }
        for (int p = tid; p < T; p += kThreads) {
            const uint32_t v = sparse[p];
            if (v != 0u)
                atomicMax(reinterpret_cast<unsigned int*>(a.h_max + int64_t(b) * T) + p, v);
        }
    }

    // the summary: D[t] per column, summed in slot order into the position's first slot word
    // (a wavefront over 8 positions x 8 columns), then the scan over time in runs of positions
    __syncthreads();
    for (int p = tid; p < T * S; p += kThreads) {
        const int t = p / S, xs = p - t * S;
        float* dp = dk + t * (K + 1) * S + xs;
        float D = 0.0f;
#pragma unroll 8
        for (int k = 0; k < K; ++k) D += dp[k * S];
        dp[0] = D;
    }
    __syncthreads();
    {
        constexpr int R = kThreads / S;  // runs
        const int Lr = (T + R - 1) / R;
        const int xs = tid % S, r = tid / S;
        const int cols = sp * S + xs;
        const int t0 = min(T, r * Lr), t1 = min(T, t0 + Lr);
        const DivN divn = a.divn;
        float cmap = 0.0f;  // the run's map q -> (rs ? 0 : q) + c
        int ri = 0;
        for (int t = t0; t < t1; ++t) {
            if ((rbits[t >> 5] >> (t & 31)) & 1u) {
                cmap = 0.0f;
                ri = 1;
            }
            cmap += divn(dk[t * (K + 1) * S + xs]);
        }
        // inclusive scan of the runs' maps over the wavefront's runs
        float ci = cmap;
#pragma unroll
        for (int o = S; o < 64; o <<= 1) {
            const float cu = __shfl_up(ci, o, 64);
            const int ru = __shfl_up(ri, o, 64);
            if (lane >= o) {
                ci = ri ? ci : cu + ci;
                ri |= ru;
            }
        }
        float* xc = xch;                                   // [kWaves][S]
        int* xr = reinterpret_cast<int*>(xch + kWaves * S);  // [kWaves][S]
        if (lane >= 64 - S) {
            xc[wv * S + xs] = ci;
            xr[wv * S + xs] = ri;
        }
        __syncthreads();
        const bool cok = cols < d;
        float q = cok ? a.q0[int64_t(b) * d + cols] : 0.0f;
        for (int w = 0; w < wv; ++w) q = (xr[w * S + xs] ? 0.0f : q) + xc[w * S + xs];
        const float ce = __shfl_up(ci, S, 64);  // the earlier runs of this wavefront
        const int re = __shfl_up(ri, S, 64);
        if (lane >= S) q = (re ? 0.0f : q) + ce;
        const int64_t qrow = int64_t(b) * T * d;
        const rsrc_t rqa = make_rsrc(a.q_pre ? static_cast<IO*>(a.q_pre) + qrow : nullptr,
                                     a.q_pre ? uint32_t(T) * d * sizeof(IO) : 0u);
        const rsrc_t rqb = make_rsrc(a.q_post ? static_cast<IO*>(a.q_post) + qrow : nullptr,
                                     a.q_post ? uint32_t(T) * d * sizeof(IO) : 0u);
        for (int t = t0; t < t1; ++t) {
            const uint32_t vo = cok ? uint32_t(t * d + cols) * sizeof(IO) : kOob;
            if ((rbits[t >> 5] >> (t & 31)) & 1u) q = 0.0f;
            bstore_f32<IO>(q, rqa, vo, 0u);
            q = q + divn(dk[t * (K + 1) * S + xs]);
            bstore_f32<IO>(q, rqb, vo, 0u);
        }
        if (a.q_T && r == R - 1 && cok) a.q_T[int64_t(b) * d + cols] = q;
    }
}

// ------------------------------------------------------------------------------------------
// Backward
// ------------------------------------------------------------------------------------------

struct BwdArgs {
    const void* y;      // [B, T, K, d] io: the candidate's pre-activation (RMS: normalised)
    const void* g;      // the gate's pre-activation
    const void* h_old;
    const void* dsel;   // optional
    const int32_t* slots;
    const uint8_t* reset;
    const void* dq_pre;   // [B, T, d] io (optional)
    const void* dq_post;  // (optional)
    const float* dq_T;    // [B, d] (optional)
    const float* dh_T;    // [B, N, d] (optional)
    void* dy;
    void* dg;
    float* dh0;  // optional
    float* dq0;  // optional
    int B, T, N, d, K;
    DivN divn;
};

// Per cell, latest event first (python/hsn/train/split.py:154-173), as chain_bwd: with the
// cotangent A of the cell's state after the event and the share R / N of its position,
// g = A + d_h_sel + R / N; dc = b g, db = (c - h_old) g, then through c = tanh(y) and
// b = sigmoid(gate); the state before the event gets (1 - b)(A + d_h_sel) - b R / N.
template <typename IO>
__global__ __launch_bounds__(kThreads) void strip_bwd(BwdArgs a) {
    extern __shared__ uint32_t lds_u[];
    constexpr int S = kCols, NB = kNBB;
    using VI = Vec4<IO>;
    int b, sp;
    strip_coords(b, sp);
    const int tid = threadIdx.x, lane = lane_id(), wv = tid >> 6;
    const int T = a.T, N = a.N, d = a.d, K = a.K;
    const int n_slots = T * K;
    int cs[kMaxU];
    load_slots(cs, a.slots + int64_t(b) * n_slots, n_slots, N, tid);
    const Layout Lo = layout(T, N, K, false);
    int* nr = reinterpret_cast<int*>(lds_u + Lo.nr);
    uint32_t* rbits = lds_u + Lo.rbits;
    int* nx = reinterpret_cast<int*>(lds_u + Lo.nx);
    int* cnt = reinterpret_cast<int*>(lds_u + Lo.cnt);
    int* ptr = reinterpret_cast<int*>(lds_u + Lo.ptr);
    int* misc = reinterpret_cast<int*>(lds_u + Lo.misc);
    uint32_t* pbits = lds_u + Lo.pbits;
    int* ppre = reinterpret_cast<int*>(lds_u + Lo.ppre);
    int* ev = reinterpret_cast<int*>(lds_u + Lo.ev);
    float* share = reinterpret_cast<float*>(lds_u + Lo.share);
    uint32_t* mask = lds_u + Lo.uni;
    const int TW = (T + 31) / 32, PW = (T * K + 31) / 32;

    // the strip's summary cotangents, in flight with the decisions while the LDS is prepared
    // (a wavefront loads 8 positions x 8 columns per instruction)
    constexpr int kStage = 4;  // (position, column) pairs per thread and round
    float* dqa = reinterpret_cast<float*>(lds_u + Lo.uni);  // [T][S]: dq_pre, then dq_post
    float* dqb = dqa + T * S;
    const int64_t qrow = int64_t(b) * T * d;
    const rsrc_t rpa = make_rsrc(a.dq_pre ? static_cast<const IO*>(a.dq_pre) + qrow : nullptr,
                                 a.dq_pre ? uint32_t(T) * d * sizeof(IO) : 0u);
    const rsrc_t rpb = make_rsrc(a.dq_post ? static_cast<const IO*>(a.dq_post) + qrow : nullptr,
                                 a.dq_post ? uint32_t(T) * d * sizeof(IO) : 0u);
    float sa[kStage], sb[kStage];
    auto stage_fetch = [&](int p0) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < kStage; ++u) {
            const int p = p0 + u * kThreads;
            const int t = p / S, xs = p - t * S;
            const uint32_t vo =
                p < T * S && sp * S + xs < d ? uint32_t(t * d + sp * S + xs) * sizeof(IO) : kOob;
            sa[u] = to_f32(bload<IO>(rpa, vo, 0u));
            sb[u] = to_f32(bload<IO>(rpb, vo, 0u));
        }
    };
    stage_fetch(tid);
    for (int i = tid; i < N; i += kThreads) cnt[i] = 0;
    for (int i = tid; i < PW; i += kThreads) pbits[i] = 0u;
    if (tid == 0) misc[0] = 0;
    chain::reset_table(a.reset ? a.reset + int64_t(b) * T : nullptr, T, nr, rbits, nx, tid,
                       kThreads);
    for (int p0 = tid;; p0 += kStage * kThreads) {
#pragma unroll
        for (int u = 0; u < kStage; ++u) {
            const int p = p0 + u * kThreads;
            if (p < T * S) {
                dqa[p] = sa[u];
                dqb[p] = sb[u];
            }
        }
        if (p0 + kStage * kThreads >= T * S) break;
        stage_fetch(p0 + kStage * kThreads);
    }
    __syncthreads();

    // the summary cotangent's reverse scan in runs of positions (fp64), its share R / N per
    // position into LDS: latest first, R += dq_post[t]; share[t] = R / N; R += dq_pre[t]; a reset
    // at t zeroes R after it
    {
        constexpr int R = kThreads / S;
        const int Lr = (T + R - 1) / R;
        const int xs = tid % S, r = tid / S;
        const int cols = sp * S + xs;
        const int t0 = min(T, r * Lr), t1 = min(T, t0 + Lr);
        const DivN divn = a.divn;
        double cmap = 0.0;  // the run's map on R, latest first: R -> (rs ? 0 : R) + c
        int ri = 0;
        for (int t = t1 - 1; t >= t0; --t) {
            cmap += double(dqb[t * S + xs]);
            cmap += double(dqa[t * S + xs]);
            if ((rbits[t >> 5] >> (t & 31)) & 1u) {
                ri = 1;
                cmap = 0.0;
            }
        }
        // inclusive suffix scan over the wavefront's runs (a later run's map applies first)
        double ci = cmap;
#pragma unroll
        for (int o = S; o < 64; o <<= 1) {
            const double cu = __shfl_down(ci, o, 64);
            const int ru = __shfl_down(ri, o, 64);
            if (lane + o < 64) {
                ci = ri ? ci : cu + ci;
                ri |= ru;
            }
        }
        double* xc = reinterpret_cast<double*>(lds_u + Lo.xch);             // [kWaves][S]
        int* xr = reinterpret_cast<int*>(lds_u + Lo.xch + 2 * kWaves * S);  // [kWaves][S]
        if (lane < S) {
            xc[wv * S + xs] = ci;
            xr[wv * S + xs] = ri;
        }
        __syncthreads();
        double Rv = (a.dq_T != nullptr && cols < d) ? double(a.dq_T[int64_t(b) * d + cols]) : 0.0;
        for (int w = kWaves - 1; w > wv; --w) Rv = (xr[w * S + xs] ? 0.0 : Rv) + xc[w * S + xs];
        const double ce = __shfl_down(ci, S, 64);  // the later runs of this wavefront
        const int re = __shfl_down(ri, S, 64);
        if (lane + S < 64) Rv = (re ? 0.0 : Rv) + ce;
        for (int t = t1 - 1; t >= t0; --t) {
            Rv += double(dqb[t * S + xs]);
            share[t * S + xs] = static_cast<float>(divn(Rv));
            Rv += double(dqa[t * S + xs]);
            if ((rbits[t >> 5] >> (t & 31)) & 1u) Rv = 0.0;
        }
        if (a.dq0 && r == 0 && cols < d) a.dq0[int64_t(b) * d + cols] = static_cast<float>(Rv);
    }
    __syncthreads();  // the staged cotangents are dead: the list build's bits take their place
    for (int i = tid; i < N * TW; i += kThreads) mask[i] = 0u;
    __syncthreads();
    build_lists(Lists{cnt, ptr, pbits, ppre, ev, mask}, cs, T, N, K, tid);
    const int n_valid = ptr[N];

    const int64_t slot0 = int64_t(b) * n_slots;
    const uint32_t row_bytes = uint32_t(n_slots) * d * sizeof(IO);
    const rsrc_t ry = make_rsrc(static_cast<const IO*>(a.y) + slot0 * d, row_bytes);
    const rsrc_t rg = make_rsrc(static_cast<const IO*>(a.g) + slot0 * d, row_bytes);
    const rsrc_t rho = make_rsrc(static_cast<const IO*>(a.h_old) + slot0 * d, row_bytes);
    const rsrc_t rds = make_rsrc(a.dsel ? static_cast<const IO*>(a.dsel) + slot0 * d : nullptr,
                                 a.dsel ? row_bytes : 0u);
    const rsrc_t rdy = make_rsrc(static_cast<IO*>(a.dy) + slot0 * d, row_bytes);
    const rsrc_t rdg = make_rsrc(static_cast<IO*>(a.dg) + slot0 * d, row_bytes);
    const rsrc_t rhT = make_rsrc(a.dh_T ? a.dh_T + int64_t(b) * N * d : nullptr,
                                 a.dh_T ? uint32_t(N) * d * 4u : 0u);
    const rsrc_t rh0 = make_rsrc(a.dh0 ? a.dh0 + int64_t(b) * N * d : nullptr,
                                 a.dh0 ? uint32_t(N) * d * 4u : 0u);
    const int x = lane % kPair, j = lane / kPair;
    const int col = sp * S + x * kVec;
    const bool colok = col < d;
    const uint32_t srow = uint32_t(d) * sizeof(IO), colb = uint32_t(col) * sizeof(IO);
    const int ntask = (N + kCPW - 1) / kCPW;
    for (;;) {
        int task = lane == 0 ? atomicAdd(&misc[0], 1) : 0;
        task = uniform(task);
        if (task >= ntask) break;
        const int oi = task * kCPW + j;
        const bool has = oi < N;
        const int c = oi;
        const int n = has ? cnt[c] : 0;
        const int base = has ? ptr[c] : 0;
        const int nmax = wave_max_int(n);
        const uint32_t vc = has && colok ? uint32_t(c * d + col) * 4u : kOob;
        // the end cotangent, cut by a reset after the cell's last event
        const int t_last = n > 0 ? (ev[base + n - 1] >> kSlotBits) : -1;
        const bool cut = nr[t_last + 1] < T;
        f4 A = f4_load_f32(rhT, cut ? kOob : vc);
        int tnext = T;  // the later event's position
        struct Batch {
            int q[NB];        // event word (-1: none)
            int nq[NB];       // the first reset after its position
            uint32_t vo[NB];  // its row's byte offset (kOob: none)
            f4 sh[NB];        // its position's share
            typename VI::Raw y[NB], g[NB], h[NB], s[NB];
        };
        // batch i0 holds the events n - 1 - i0 - i, i < NB (latest first)
        auto fetch = [&](int i0, Batch& bt) __attribute__((always_inline)) {
#pragma unroll
            for (int i = 0; i < NB; ++i) bt.q[i] = ev[base + max(n - 1 - (i0 + i), 0)];
#pragma unroll
            for (int i = 0; i < NB; ++i) {
                const bool ok = n - 1 - (i0 + i) >= 0;
                const int q = bt.q[i];
                const int t = ok ? q >> kSlotBits : 0;
                bt.q[i] = ok ? q : -1;
                bt.nq[i] = nr[t + 1];
                bt.sh[i] = *reinterpret_cast<const f4*>(share + t * S + x * kVec);
                bt.vo[i] = ok && colok ? uint32_t(q & kSlotMask) * srow + colb : kOob;
                bt.y[i] = VI::load(ry, bt.vo[i]);
                bt.g[i] = VI::load(rg, bt.vo[i]);
                bt.h[i] = VI::load(rho, bt.vo[i]);
                bt.s[i] = VI::load(rds, bt.vo[i]);
            }
        };
        auto step = [&](int i0, const Batch& bt) __attribute__((always_inline)) {
#pragma unroll
            for (int i = 0; i < NB; ++i) {
                if (i0 + i >= nmax) break;
                const int q = bt.q[i];
                const bool ok = q >= 0;
                const int t = q >> kSlotBits;
                const bool zero = bt.nq[i] <= tnext && tnext < T;  // a reset in (t, tnext]
                const f4 yv = VI::widen(bt.y[i]), gv = VI::widen(bt.g[i]);
                const f4 hv = VI::widen(bt.h[i]), sv = VI::widen(bt.s[i]);
                f4 dc, db, An;
#pragma unroll
                for (int v = 0; v < kVec; ++v) {
                    const float carried = (zero ? 0.0f : A[v]) + sv[v];
                    const float sh = bt.sh[i][v];
                    const float gg = carried + sh;
                    const float bgt = fast_sigmoid(gv[v]);
                    const float cc = fast_tanh(yv[v]);
                    dc[v] = bgt * gg * (1.0f - cc * cc);
                    db[v] = (cc - hv[v]) * gg * (bgt * (1.0f - bgt));
                    An[v] = (1.0f - bgt) * carried - bgt * sh;
                }
                VI::store(dc, rdy, bt.vo[i]);
                VI::store(db, rdg, bt.vo[i]);
                A = sel4(ok, An, A);
                tnext = ok ? t : tnext;
            }
        };
        Batch b0, b1;
        fetch(0, b0);
        for (int i0 = 0; i0 < nmax; i0 += 2 * NB) {
            if (i0 + NB < nmax) fetch(i0 + NB, b1);
            step(i0, b0);
            if (i0 + NB >= nmax) break;
            if (i0 + 2 * NB < nmax) fetch(i0 + 2 * NB, b0);
            step(i0 + NB, b1);
        }
        // the start state's cotangent: cut by a reset at or before the first event
        const bool z = nr[0] <= min(tnext, T - 1);
        Vec4<float>::store(z ? f4{0.0f, 0.0f, 0.0f, 0.0f} : A, rh0, vc);
    }
    // exact zeros on the row's padded slots (a column per thread)
    const int n_pad = n_slots - n_valid;
    {
        const int xs = tid % S, colp = sp * S + xs;
        const bool cok = colp < d;
        for (int pi = tid / S; pi < n_pad; pi += kThreads / S) {
            const int q = ev[n_valid + pi];
            const uint32_t vo = cok ? uint32_t(q & kSlotMask) * srow + uint32_t(colp) * sizeof(IO) : kOob;
            bstore_f32<IO>(0.0f, rdy, vo, 0u);
            bstore_f32<IO>(0.0f, rdg, vo, 0u);
        }
    }
}

}  // namespace strip
}  // namespace hsn
