// The window's sweeps cell by cell (gfx950). Each cell's updates form a chain in time; chains of
// different cells are independent but for the summary q, which adds every slot's delta of a
// position. So the state needs no shared memory: a wavefront walks one cell's chain with the
// cell's d columns in its lanes (column x in lane x % 64, register x / 64), and every load and
// store is a whole row of a [B, T, K, d] tensor (d * sizeof(io) contiguous bytes), against the
// S-column pieces of the time-chunked sweeps (sweep.cuh), whose slices shrink as K grows.
//
//   row_lists     (row): the row's decisions as per-cell event lists (CSR): ptr[N + 1], then
//                 the events (t << 8 | k) of each cell in time order, then the padded slots in
//                 time order. Counts by LDS atomics (integers: any order), ranks within a block
//                 of positions from a bit per position per cell (popcount below t):
//                 deterministic.
//   chain_fwd     (row, group of cells; a wavefront per cell): h_old, h_sel, the end state, the
//                 ages, each valid slot's delta h_sel - h_old in fp32 where the rows are bf16
//                 or omitted; the row maximum of |h| per position from each cell's value on the
//                 intervals between its events (LDS atomic max), a table per group.
//   summary_delta (row, position): D[t] = the sum of the valid slots' deltas; the row maximum,
//                 the largest of the groups'.
//   summary_scan_fwd (row, 64 columns): q before and after every position, a scan over time
//                 of D / N with the resets.
//   summary_scan_bwd (row, 64 columns): the summary cotangent R, a reverse scan in fp64, as the
//                 per-position share R / N and d_q0.
//   chain_bwd     (row, group of cells): the reverse chains of the cotangent A with the
//                 activations' VJPs; d_h0.
//
// Reference: the forward restates python/hsn/kernels/native.py:244-303 and
// python/hsn/model/state.py:267-324 per position (python/hsn/train/compile.py:1296-1344); the
// backward restates python/hsn/train/split.py:128-174 with the carried state
// (python/hsn/train/state_gradient.py:402-416). A reset at r zeroes the state before position
// r reads it (forward) and the cotangents after position r is processed (backward): for a
// cell's consecutive events t' < t, the chain restarts from zero exactly when a reset lies in
// (t', t], i.e. when the first reset after t' is at or before t. Padded slots gather cell 0
// (h_old shows cell 0 before the position's update, h_sel after it) and get exact zeros in the
// backward.
#pragma once

#include <stddef.h>

#include <type_traits>

#include "sweep.cuh"

namespace hsn {
namespace chain {

constexpr int kMaxV = 4;   // columns per lane: d <= 256
constexpr int kMaxK = 255;  // slots per position (the event's slot field is 8 bits)
constexpr int kEvWin = 64;  // events per window: one event per lane

// ------------------------------------------------------------------------------------------
// The per-row event lists
// ------------------------------------------------------------------------------------------

constexpr int kListThreads = 1024;
constexpr int kListU = 8;  // slots per thread and block of positions

// positions per block of the rank pass (a multiple of 32): a bit per position per cell in at most
// 64 KiB, and at most 2048 slots unless one word of positions has more (32 K <= 8160 slots, within
// the kListU * kListThreads a block's threads hold)
__host__ __device__ inline int list_block(int N, int T, int K) {
    int P = 32;
    while (P < T && int64_t(N) * (2 * P / 32) * 4 <= 65536 && 2 * P * K <= 2048) P *= 2;
    return P;
}
// the scan partials' words: the 16 wavefronts' and the row's total, or a prefix per word of the
// block's padded-slot bits and their total
__host__ __device__ inline int list_partials(int P, int K) {
    const int pkw = (P * K + 31) / 32 + 1;
    return pkw > 65 ? pkw : 65;
}
__host__ __device__ inline int list_words(int N, int T, int K) {  // LDS words of row_lists
    const int P = list_block(N, T, K);
    return 2 * N + N * (P / 32) + (P * K + 31) / 32 + list_partials(P, K) + 4;
}

struct ListArgs {
    const int32_t* slots;  // [B, T, K]: the cell, or -1 on a padded slot
    int32_t* ptr;          // [B, N + 1]
    int32_t* ev;           // [B, T * K]
    int B, T, N, K;
};

__device__ __forceinline__ int slot_cell(const int32_t* slots, int64_t i, int N) {
    const int c = slots[i];
    return c >= 0 && c < N ? c : -1;
}

static __global__ __launch_bounds__(kListThreads) void row_lists(ListArgs a) {
    extern __shared__ uint32_t lds_u[];
    const int b = blockIdx.x;
    const int tid = threadIdx.x;
    const int T = a.T, N = a.N, K = a.K;
    const int P = list_block(N, T, K), PW = P / 32;
    int* cnt = reinterpret_cast<int*>(lds_u);  // [N]: counts, then the events placed so far
    int* base = cnt + N;                       // [N]: the list starts
    uint32_t* mask = reinterpret_cast<uint32_t*>(base + N);  // [N][PW]
    const int PKW = (P * K + 31) / 32;
    uint32_t* pmask = mask + N * PW;                  // [PKW]: the block's padded slots
    int* wsum = reinterpret_cast<int*>(pmask + PKW);  // scan partials
    int* misc = wsum + list_partials(P, K);           // [0]: padded slots placed so far
    const int64_t row = int64_t(b) * T * K;
    for (int c = tid; c < N; c += kListThreads) cnt[c] = 0;
    if (tid == 0) misc[0] = 0;
    __syncthreads();
    const int n_slots = T * K;
    for (int i0 = tid; i0 < n_slots; i0 += kListThreads * kListU) {  // kListU loads in flight
        int cs[kListU];
#pragma unroll
        for (int u = 0; u < kListU; ++u) {
            const int i = i0 + u * kListThreads;
            cs[u] = i < n_slots ? slot_cell(a.slots, row + i, N) : -1;
        }
#pragma unroll
        for (int u = 0; u < kListU; ++u)
            if (cs[u] >= 0) atomicAdd(&cnt[cs[u]], 1);
    }
    __syncthreads();
    // exclusive scan of the counts (a chunk of cells per thread, then the chunks' prefix)
    const int per = (N + kListThreads - 1) / kListThreads;
    const int c0 = min(N, tid * per), c1 = min(N, c0 + per);
    int s = 0;
    for (int c = c0; c < c1; ++c) s += cnt[c];
    const int lane = tid & 63, wv = tid >> 6;
    int incl = s;
    for (int o = 1; o < 64; o <<= 1) {
        const int u = __shfl_up(incl, o, 64);
        if (lane >= o) incl += u;
    }
    if (lane == 63) wsum[wv] = incl;
    __syncthreads();
    if (tid == 0) {
        int acc = 0;
        for (int w = 0; w < kListThreads / 64; ++w) {
            const int v = wsum[w];
            wsum[w] = acc;
            acc += v;
        }
        wsum[kListThreads / 64] = acc;  // the row's valid events
    }
    __syncthreads();
    int run = wsum[wv] + incl - s;
    for (int c = c0; c < c1; ++c) {
        const int v = cnt[c];
        base[c] = run;
        cnt[c] = 0;
        a.ptr[int64_t(b) * (N + 1) + c] = run;
        run += v;
    }
    const int n_valid = wsum[kListThreads / 64];
    if (tid == 0) a.ptr[int64_t(b) * (N + 1) + N] = n_valid;
    int32_t* ev = a.ev + row;
    // blocks of P positions (P * K <= kListU * kListThreads slots): a thread's slots of the next
    // block are loaded while the current one is ranked
    int cur[kListU], nxt[kListU];
    auto fetch = [&](int t0, int (&cs)[kListU]) __attribute__((always_inline)) {
        const int n = min(P, T - t0) * K;
#pragma unroll
        for (int u = 0; u < kListU; ++u) {
            const int i = tid + u * kListThreads;
            cs[u] = t0 < T && i < n ? slot_cell(a.slots, row + int64_t(t0) * K + i, N) : -2;
        }
    };
    fetch(0, cur);
    for (int t0 = 0; t0 < T; t0 += P) {
        const int pn = min(P, T - t0);
        fetch(t0 + P, nxt);
        __syncthreads();
        for (int i = tid; i < N * PW; i += kListThreads) mask[i] = 0u;
        for (int i = tid; i < PKW; i += kListThreads) pmask[i] = 0u;
        __syncthreads();
#pragma unroll
        for (int u = 0; u < kListU; ++u) {
            const int i = tid + u * kListThreads, c = cur[u];
            if (c == -2) continue;  // past the block
            const int tl = i / K;
            if (c >= 0) atomicOr(&mask[c * PW + (tl >> 5)], 1u << (tl & 31));
            else atomicOr(&pmask[i >> 5], 1u << (i & 31));
        }
        __syncthreads();
        if (tid < 64) {  // the padded slots' exclusive prefix per word, in wsum (wavefront 0)
            int acc = 0;
            for (int w0 = 0; w0 < PKW; w0 += 64) {
                const int w = w0 + tid;
                const int v = w < PKW ? __popc(pmask[w]) : 0;
                int incl = v;
                for (int o = 1; o < 64; o <<= 1) {
                    const int u = __shfl_up(incl, o, 64);
                    if (tid >= o) incl += u;
                }
                if (w < PKW) wsum[w] = acc + incl - v;
                acc += __shfl(incl, 63, 64);
            }
            if (tid == 0) wsum[PKW] = acc;  // the block's padded slots
        }
        __syncthreads();
        const int pad0 = misc[0];
#pragma unroll
        for (int u = 0; u < kListU; ++u) {
            const int i = tid + u * kListThreads, c = cur[u];
            if (c == -2) continue;
            const int tl = i / K, k = i - tl * K;
            const int t = t0 + tl;
            if (c >= 0) {
                int rank = cnt[c];
                const uint32_t* m = mask + c * PW;
                for (int w = 0; w < (tl >> 5); ++w) rank += __popc(m[w]);
                rank += __popc(m[tl >> 5] & ((1u << (tl & 31)) - 1u));
                ev[base[c] + rank] = (t << 8) | k;
            } else {
                const int r = wsum[i >> 5] + __popc(pmask[i >> 5] & ((1u << (i & 31)) - 1u));
                ev[n_valid + pad0 + r] = (t << 8) | k;
            }
        }
        (void)pn;
        __syncthreads();
        for (int c = tid; c < N; c += kListThreads) {
            int v = 0;
            for (int w = 0; w < PW; ++w) v += __popc(mask[c * PW + w]);
            cnt[c] += v;
        }
        if (tid == 0) misc[0] = pad0 + wsum[PKW];
#pragma unroll
        for (int u = 0; u < kListU; ++u) cur[u] = nxt[u];
    }
}

// ------------------------------------------------------------------------------------------
// Shared pieces of the chain kernels
// ------------------------------------------------------------------------------------------

constexpr int kChainWaves = 8;
constexpr int kChainThreads = 64 * kChainWaves;

// The row's reset table in LDS: nr[p] = the first reset at or after position p (T: none),
// p = 0..T, and the last reset of the row (-1: none), returned. `bits` [TW] and `nx` [TW + 1]
// are scratch.
__device__ __forceinline__ int reset_table(const uint8_t* reset_row, int T, int* nr,
                                           uint32_t* bits, int* nx, int tid, int nthreads) {
    const int TW = (T + 31) / 32;
    for (int t0 = 0; t0 < T; t0 += nthreads) {  // every wavefront ballots its 64 positions
        const int t = t0 + tid;
        const bool r = t < T && reset_row != nullptr && reset_row[t] != 0;
        const uint64_t m = ballot(r);
        if ((tid & 63) == 0 && t < T) {
            const int w = t / 32;
            bits[w] = static_cast<uint32_t>(m);
            if (w + 1 < TW) bits[w + 1] = static_cast<uint32_t>(m >> 32);
        }
    }
    __syncthreads();
    if (tid == 0) {
        int next = T;
        nx[TW] = T;
        for (int w = TW - 1; w >= 0; --w) {  // nx[w]: the first reset in words >= w
            const uint32_t v = bits[w];
            next = v ? w * 32 + __builtin_ctz(v) : next;
            nx[w] = next;
        }
        int last = -1;
        for (int w = TW - 1; w >= 0 && last < 0; --w)
            if (bits[w]) last = w * 32 + 31 - __builtin_clz(bits[w]);
        nr[T + 1] = last;  // passed on through LDS
    }
    __syncthreads();
    for (int p = tid; p <= T; p += nthreads) {
        if (p == T) {
            nr[T] = T;
        } else {
            const int w = p / 32;
            const uint32_t above = bits[w] & (0xffffffffu << (p & 31));  // positions >= p
            nr[p] = above ? w * 32 + __builtin_ctz(above) : nx[w + 1];
        }
    }
    __syncthreads();
    return nr[T + 1];
}

// (row, group) of a chain workgroup from the grid (8, G, B/8) (or (1, G, B)): the rows with the
// same blockIdx.x share an XCD, so a row's lists and shares stay in one L2.
__device__ __forceinline__ void group_coords(int& b, int& g) {
    b = blockIdx.x * gridDim.z + blockIdx.z;
    g = blockIdx.y;
}
inline dim3 chain_grid(int B, int G) {
    const int x = B % 8 == 0 ? 8 : 1;
    return dim3(x, G, B / x);
}

// LDS words of a chain workgroup: nr [T + 2], the reset bits [TW], their word table [TW + 1],
// the row maxima [T], the next cell to take, the group's list starts [C + 1], its staged events
// [stage] and its cells in the order they are taken [C].
__host__ __device__ inline int chain_words(int T, int C, int stage) {
    const int TW = (T + 31) / 32;
    return (T + 2) + TW + (TW + 1) + T + 1 + (C + 1) + stage + C;
}

// The group's cells heaviest first (most events; ties by cell), into order[0 .. nc): the
// wavefronts take cells in this order, so the long chains start first and the workgroup's
// wavefronts finish together (a workgroup holds its CU slot until its last wavefront ends).
// cptr must be visible to every thread; ends with a barrier.
__device__ __forceinline__ void heavy_first(const int* cptr, int nc, int* order, int tid,
                                            int nthreads) {
    for (int i = tid; i < nc; i += nthreads) {
        const int ni = cptr[i + 1] - cptr[i];
        int rank = 0;
        for (int j = 0; j < nc; ++j) {
            const int nj = cptr[j + 1] - cptr[j];
            rank += (nj > ni || (nj == ni && j < i)) ? 1 : 0;
        }
        order[rank] = i;
    }
    __syncthreads();
}

// The wavefront maximum of the bit patterns of |h| over the cell's columns (a NaN above +inf).
template <int V>
__device__ __forceinline__ uint32_t cell_abs_max(const float (&h)[V], int lane, int d) {
    uint32_t m = 0u;
#pragma unroll
    for (int v = 0; v < V; ++v) m = umax(m, lane + 64 * v < d ? abs_bits(h[v]) : 0u);
    return wave_max_from_groups<1>(m);
}

// The row maxima over positions [p0, p1) from one cell's value (bits): the first 64 positions
// inline (intervals are mostly shorter than a wavefront), the rest out of line.
__device__ __attribute__((noinline)) void max_interval_tail(uint32_t* hm, int p0, int p1,
                                                           uint32_t val, int lane) {
    for (int p = p0 + lane; p < p1; p += 64) atomicMax(&hm[p], val);
}
__device__ __forceinline__ void max_interval(uint32_t* hm, int p0, int p1, uint32_t val,
                                             int lane) {
    if (p0 + lane < p1) atomicMax(&hm[p0 + lane], val);
    if (unlikely(uniform(p1 - p0) > 64)) max_interval_tail(hm, p0 + 64, p1, val, lane);
}

// ------------------------------------------------------------------------------------------
// Forward chains
// ------------------------------------------------------------------------------------------

struct FwdArgs {
    const void* y;  // [B, T, K, d] io: the candidate's pre-activation (the RMS prologue's output)
    const void* g;  // the write gate's pre-activation
    const int32_t* ptr;  // the lists: [B, N + 1], [B, T * K]
    const int32_t* ev;
    const uint8_t* reset;  // [B, T] (null: none)
    const float* h0;       // [B, N, d]
    const int64_t* age0;   // [B, N] (with age_T)
    const int64_t* pos0;   // [B] (with pos_T)
    void* h_old;           // [B, T, K, d] io (optional)
    void* h_sel;           // (optional)
    float* delta;          // [B, T, K, d] fp32: h_sel - h_old of the valid slots (optional)
    uint32_t* hm_groups;   // [B, T, G]: each group's row maximum per position, |h| bits
                           // (optional: with the row maxima)
    float* h_T;            // [B, N, d] (optional)
    int64_t* age_T;        // [B, N] (optional)
    int64_t* pos_T;        // [B] (optional)
    int B, T, N, d, K;
    int C, stage;  // cells per workgroup, staged events per workgroup
};

template <typename IO, int V>
__device__ __forceinline__ void fetch_rows(IO (&yv)[V], IO (&gv)[V], rsrc_t ry, rsrc_t rg,
                                           const uint32_t (&voff)[V], uint32_t so, bool in) {
#pragma unroll
    for (int v = 0; v < V; ++v) {
        const uint32_t vo = in ? voff[v] : kOob;
        yv[v] = bload<IO>(ry, vo, so);
        gv[v] = bload<IO>(rg, vo, so);
    }
}

template <typename IO, int V, int NB, bool DELTA, bool HMAX>
__global__ __launch_bounds__(kChainThreads) void chain_fwd(FwdArgs a) {
    extern __shared__ uint32_t lds_u[];
    int b, g;
    group_coords(b, g);
    const int tid = threadIdx.x, lane = lane_id();
    const int T = a.T, N = a.N, d = a.d, K = a.K;
    const int TW = (T + 31) / 32;
    int* nr = reinterpret_cast<int*>(lds_u);             // [T + 2]
    uint32_t* rbits = lds_u + (T + 2);                   // [TW]
    int* nx = reinterpret_cast<int*>(rbits + TW);        // [TW + 1]
    uint32_t* hm = reinterpret_cast<uint32_t*>(nx + TW + 1);  // [T]
    int* next = reinterpret_cast<int*>(hm + T);          // [1]
    int* cptr = next + 1;                                // [C + 1]
    int* cev = cptr + a.C + 1;                           // [stage]
    int* order = cev + a.stage;                          // [C]
    constexpr bool want_max = HMAX;
    const int c_begin = g * a.C, c_end = min(N, c_begin + a.C);
    const int nc = c_end - c_begin;
    const int32_t* ptr = a.ptr + int64_t(b) * (N + 1);
    const int32_t* ev = a.ev + int64_t(b) * T * K;
    // the group's list starts and its first `stage` events, staged once for every wavefront
    const int pc0 = ptr[c_begin];
    const int nst = min(ptr[c_end] - pc0, a.stage);
    for (int i = tid; i <= nc; i += kChainThreads) cptr[i] = ptr[c_begin + i];
    for (int i = tid; i < nst; i += kChainThreads) cev[i] = ev[pc0 + i];
    for (int p = tid; p < T; p += kChainThreads) hm[p] = 0u;
    if (tid == 0) next[0] = 0;
    const int lrT = reset_table(a.reset ? a.reset + int64_t(b) * T : nullptr, T, nr, rbits, nx,
                                tid, kChainThreads);
    heavy_first(cptr, nc, order, tid, kChainThreads);
    const int64_t slot0 = int64_t(b) * T * K;
    const uint32_t row_bytes = uint32_t(T) * K * d * sizeof(IO);
    const rsrc_t ry = make_rsrc(static_cast<const IO*>(a.y) + slot0 * d, row_bytes);
    const rsrc_t rg = make_rsrc(static_cast<const IO*>(a.g) + slot0 * d, row_bytes);
    const rsrc_t rho = make_rsrc(a.h_old ? static_cast<IO*>(a.h_old) + slot0 * d : nullptr,
                                 a.h_old ? row_bytes : 0u);
    const rsrc_t rhs = make_rsrc(a.h_sel ? static_cast<IO*>(a.h_sel) + slot0 * d : nullptr,
                                 a.h_sel ? row_bytes : 0u);
    const rsrc_t rdl = make_rsrc(a.delta ? a.delta + slot0 * d : nullptr,
                                 a.delta ? uint32_t(T) * K * d * 4u : 0u);
    uint32_t voff[V], voff4[V];
#pragma unroll
    for (int v = 0; v < V; ++v) {
        const bool in = lane + 64 * v < d;
        voff[v] = in ? uint32_t(lane + 64 * v) * sizeof(IO) : kOob;
        voff4[v] = in ? uint32_t(lane + 64 * v) * 4u : kOob;
    }
    const uint32_t srow = uint32_t(d) * sizeof(IO), srow4 = uint32_t(d) * 4u;
    const int n_slots = T * K;
    const int pad_begin = ptr[N];

    for (;;) {
        int slot = lane == 0 ? atomicAdd(next, 1) : 0;
        slot = __builtin_amdgcn_readfirstlane(slot);
        if (slot >= nc) break;
        const int ci = uniform(order[slot]);
        const int c = c_begin + ci;
        const int e_beg = uniform(cptr[ci]), e_end = uniform(cptr[ci + 1]);
        float h[V];
        const float* h0c = a.h0 + (int64_t(b) * N + c) * d;
#pragma unroll
        for (int v = 0; v < V; ++v) h[v] = lane + 64 * v < d ? h0c[lane + 64 * v] : 0.0f;
        float hold_last[V];  // the state before the latest event (cell 0's padded slots)
#pragma unroll
        for (int v = 0; v < V; ++v) hold_last[v] = 0.0f;
        uint32_t vprev = want_max ? cell_abs_max<V>(h, lane, d) : 0u;
        int tprev = -1, s = 0;
        int nrprev = nr[0];  // the first reset after the latest event
        // cell 0's padded slots at positions below `limit`, in time order (a window of 64 of
        // them in the lanes)
        int pp = pad_begin, pwb = -1, pwv = 0;
        auto flush = [&](int limit) __attribute__((always_inline)) {
            while (pp < n_slots) {
                if (pwb < 0 || pp >= pwb + kEvWin) {
                    pwb = pp;
                    pwv = lane < n_slots - pp ? ev[pp + lane] : 0x7fffffff;
                }
                const int off = pp - pwb;
                const uint64_t below = ballot(lane >= off && (pwv >> 8) < limit);
                const int n = __popcll(below);
                for (int i = 0; i < n; ++i) {
                    const int q = __builtin_amdgcn_readlane(pwv, off + i);
                    const int t = q >> 8;
                    const uint32_t so = uint32_t(t * K + (q & 255)) * srow;
                    const bool same = t == tprev;
                    const bool zero = nrprev <= t;
#pragma unroll
                    for (int v = 0; v < V; ++v) {
                        const float now = zero ? 0.0f : h[v];
                        bstore_f32<IO>(same ? hold_last[v] : now, rho, voff[v], so);
                        bstore_f32<IO>(same ? h[v] : now, rhs, voff[v], so);
                    }
                }
                pp += n;
                if (off + n < kEvWin) break;  // the next one is at or after `limit`
            }
        };
        const bool pad_here = c == 0 && pad_begin < n_slots;
        // one event: position t, its slot's byte offsets (so: storage rows, so4: fp32 rows) and
        // the first reset after t
        auto update = [&](auto pad_c, int t, uint32_t so, uint32_t so4, int nrq, const IO (&yv)[V],
                          const IO (&gv)[V]) __attribute__((always_inline)) {
            constexpr bool kPad = decltype(pad_c)::value;
            const bool zero = nrprev <= t;  // a reset since the cell's last event
            if constexpr (want_max) max_interval(hm, s, min(t, nrprev), vprev, lane);
            if constexpr (kPad) flush(t);
#pragma unroll
            for (int v = 0; v < V; ++v) {
                const float hold = zero ? 0.0f : h[v];
                const float bg = fast_sigmoid(to_f32(gv[v]));
                const float cand = fast_tanh(to_f32(yv[v]));
                const float hn = (1.0f - bg) * hold + bg * cand;
                bstore_f32<IO>(hold, rho, voff[v], so);
                bstore_f32<IO>(hn, rhs, voff[v], so);
                if constexpr (DELTA) bstore(hn - hold, rdl, voff4[v], so4);
                if constexpr (kPad) hold_last[v] = hold;
                h[v] = hn;
            }
            if constexpr (want_max) vprev = cell_abs_max<V>(h, lane, d);
            s = t;
            tprev = t;
            nrprev = nrq;
            if constexpr (kPad) flush(t + 1);
        };
        // windows of 64 events (one per lane), in batches of NB with two batches in flight; a
        // window's positions, slot offsets and next resets are computed for all its events at
        // once (lane i: event i) and read per event with readlane
        auto walk = [&](auto staged_c, auto pad_c) __attribute__((always_inline)) {
            constexpr bool kStaged = decltype(staged_c)::value;
            for (int w0 = e_beg; w0 < e_end; w0 += kEvWin) {
                const int m = min(kEvWin, e_end - w0);
                int evw;
                if constexpr (kStaged) evw = lane < m ? cev[w0 - pc0 + lane] : 0;
                else evw = lane < m ? ev[w0 + lane] : 0;
                const int tw = evw >> 8;
                const int slw = tw * K + (evw & 255);
                const uint32_t sow = uint32_t(slw) * srow;
                const uint32_t so4w = uint32_t(slw) * srow4;
                const int nrw = lane < m ? nr[tw + 1] : T;
                IO ya[NB][V], ga[NB][V], yb[NB][V], gb[NB][V];
                auto fetch = [&](int j, IO (&yv)[NB][V], IO (&gv)[NB][V])
                                 __attribute__((always_inline)) {
#pragma unroll
                    for (int i = 0; i < NB; ++i) {
                        const uint32_t so = __builtin_amdgcn_readlane(sow, min(j + i, kEvWin - 1));
                        fetch_rows<IO, V>(yv[i], gv[i], ry, rg, voff, so, j + i < m);
                    }
                };
                auto step = [&](int j, const IO (&yv)[NB][V], const IO (&gv)[NB][V])
                                __attribute__((always_inline)) {
#pragma unroll
                    for (int i = 0; i < NB; ++i) {
                        if (j + i < m) {
                            const int idx = j + i;
                            update(pad_c, __builtin_amdgcn_readlane(tw, idx),
                                   __builtin_amdgcn_readlane(sow, idx),
                                   DELTA ? __builtin_amdgcn_readlane(so4w, idx) : 0u,
                                   __builtin_amdgcn_readlane(nrw, idx), yv[i], gv[i]);
                        }
                    }
                };
                fetch(0, ya, ga);
                for (int j = 0; j < m; j += 2 * NB) {
                    fetch(j + NB, yb, gb);
                    step(j, ya, ga);
                    if (j + NB >= m) break;
                    fetch(j + 2 * NB, ya, ga);
                    step(j + NB, yb, gb);
                }
            }
        };
        if (pad_here) walk(std::false_type{}, std::true_type{});
        else if (e_end - pc0 <= nst) walk(std::true_type{}, std::false_type{});
        else walk(std::false_type{}, std::false_type{});
        if (pad_here) flush(T);
        if (want_max) max_interval(hm, s, min(T, nrprev), vprev, lane);
        const bool cleared = nrprev < T;  // a reset after the cell's last event
        if (a.h_T) {
            float* hTc = a.h_T + (int64_t(b) * N + c) * d;
#pragma unroll
            for (int v = 0; v < V; ++v)
                if (lane + 64 * v < d) hTc[lane + 64 * v] = cleared ? 0.0f : h[v];
        }
        if (a.age_T && lane == 0) {
            int64_t age;
            if (tprev >= 0 && tprev >= lrT) age = (T - 1) - tprev;
            else if (lrT >= 0) age = T - lrT;
            else age = a.age0[int64_t(b) * N + c] + T;
            a.age_T[int64_t(b) * N + c] = age;
        }
    }
    if (a.pos_T && g == 0 && tid == 0) a.pos_T[b] = lrT >= 0 ? int64_t(T - lrT) : a.pos0[b] + T;
    if (want_max) {  // the group's maxima, reduced over the groups by summary_delta
        __syncthreads();
        const int G = gridDim.y;
        uint32_t* hg = a.hm_groups + int64_t(b) * T * G + g;
        for (int p = tid; p < T; p += kChainThreads) hg[int64_t(p) * G] = hm[p];
    }
}

// ------------------------------------------------------------------------------------------
// The summary: the valid slots' delta sum per position, then a scan over time
// ------------------------------------------------------------------------------------------

struct DeltaArgs {
    const void* h_old;    // [B, T, K, d] io (PAIR)
    const void* h_sel;
    const float* delta;   // [B, T, K, d] fp32 (not PAIR)
    const int32_t* slots; // [B, T, K]
    float* D;             // [B, T, d]
    const uint32_t* hm_groups;  // [B, T, G] (optional)
    float* h_max;         // [B, T]: the maximum over the groups (with hm_groups)
    int B, T, N, d, K, G;
};

// A wavefront per (row, position), lanes over the columns: D[t] = the sum over the position's
// valid slots, in slot order, of h_sel - h_old as stored (PAIR: fp32 rows, the forward's own
// values) or of the chains' fp32 deltas (bf16 rows, or an omitted h_old / h_sel).
template <typename IO, int V, bool PAIR>
__global__ __launch_bounds__(256) void summary_delta(DeltaArgs a) {
    const int pos = blockIdx.x * 4 + uniform(threadIdx.x / 64);
    const int b = blockIdx.y;
    if (pos >= a.T) return;
    const int lane = lane_id();
    const int d = a.d, K = a.K;
    const int64_t slot0 = (int64_t(b) * a.T + pos) * K;
    const rsrc_t r1 = PAIR ? make_rsrc(static_cast<const IO*>(a.h_sel) + slot0 * d, uint32_t(K) * d * sizeof(IO))
                           : make_rsrc(a.delta + slot0 * d, uint32_t(K) * d * 4u);
    const rsrc_t r0 = make_rsrc(PAIR ? static_cast<const IO*>(a.h_old) + slot0 * d : nullptr,
                                PAIR ? uint32_t(K) * d * sizeof(IO) : 0u);
    constexpr uint32_t E = PAIR ? sizeof(IO) : 4u;
    uint32_t voff[V];
#pragma unroll
    for (int v = 0; v < V; ++v) voff[v] = lane + 64 * v < d ? uint32_t(lane + 64 * v) * E : kOob;
    float D[V];
#pragma unroll
    for (int v = 0; v < V; ++v) D[v] = 0.0f;
    constexpr int kU = 8;
    for (int k64 = 0; k64 < K; k64 += 64) {
        const uint64_t okm = ballot(k64 + lane < K && slot_cell(a.slots, slot0 + k64 + lane, a.N) >= 0);
        for (int k0 = 0; k0 < min(64, K - k64); k0 += kU) {
            float s1[kU][V], s0[kU][V];
#pragma unroll
            for (int i = 0; i < kU; ++i) {
                const int k = k64 + k0 + i;
                const bool ok = k0 + i < 64 && ((okm >> min(k0 + i, 63)) & 1ull) && k < K;
                const uint32_t so = uint32_t(min(k, K - 1)) * d * E;
#pragma unroll
                for (int v = 0; v < V; ++v) {
                    const uint32_t vo = ok ? voff[v] : kOob;
                    if constexpr (PAIR) {
                        s1[i][v] = to_f32(bload<IO>(r1, vo, so));
                        s0[i][v] = to_f32(bload<IO>(r0, vo, so));
                    } else {
                        s1[i][v] = bload<float>(r1, vo, so);
                        s0[i][v] = 0.0f;
                    }
                }
            }
#pragma unroll
            for (int i = 0; i < kU; ++i)
#pragma unroll
                for (int v = 0; v < V; ++v) D[v] += PAIR ? s1[i][v] - s0[i][v] : s1[i][v];
        }
    }
    float* Dp = a.D + (int64_t(b) * a.T + pos) * d;
#pragma unroll
    for (int v = 0; v < V; ++v)
        if (lane + 64 * v < d) Dp[lane + 64 * v] = D[v];
    if (a.hm_groups) {  // the row maximum: the largest of the groups' (|h| bits, NaN above inf)
        const uint32_t* hg = a.hm_groups + (int64_t(b) * a.T + pos) * a.G;
        uint32_t m = 0u;
        for (int g = lane; g < a.G; g += 64) m = umax(m, hg[g]);
        m = wave_max_from_groups<1>(m);
        if (lane == 0) a.h_max[int64_t(b) * a.T + pos] = __uint_as_float(m);
    }
}

constexpr int kScanWaves = 16;

struct ScanArgs {
    // forward: D [B, T, d] fp32 -> q_pre, q_post [B, T, d] io (optional), q_T [B, d] from q0
    const float* D;
    const float* q0;
    void* q_pre;
    void* q_post;
    float* q_T;
    // backward: dq_pre, dq_post [B, T, d] io (optional), dq_T [B, d] (optional) -> the share
    // R / N [B, T, d] fp32 and d_q0 [B, d] (optional)
    const void* dq_pre;
    const void* dq_post;
    const float* dq_T;
    float* share;
    float* dq0;
    const uint8_t* reset;  // [B, T] (optional)
    int B, T, d;
    DivN divn;
};

// (row, 64 columns): 16 wavefronts over consecutive ranges of 32 positions, in rounds of 512
// positions. A range maps the summary q to (reset in range ? 0 : q) + c, c its D / N sum after
// its last reset; the wavefronts exchange (reset, c) through LDS, each folds the earlier ones'
// into its start value and replays its positions in the reference's order per position
// (python/hsn/kernels/native.py:302 with state.py:267-283): q_pre[t] = (reset[t] ? 0 : q),
// q_post[t] = q_pre[t] + D[t] / N. Rows of [., T, d] tensors are buffer resources: a lane's
// column is its voffset, the position a uniform soffset (kept inside the row: only the voffset
// masks an access).
template <typename IO>
__global__ __launch_bounds__(64 * kScanWaves) void summary_scan_fwd(ScanArgs a) {
    __shared__ int rss[kScanWaves];
    __shared__ float cx[kScanWaves][64];
    const int b = blockIdx.y, z = blockIdx.x;
    const int lane = lane_id(), w = uniform(threadIdx.x / 64);
    const int x = z * 64 + lane;
    const bool col = x < a.d;
    const int T = a.T, d = a.d;
    const DivN divn = a.divn;
    const int64_t row = int64_t(b) * T * d;
    const rsrc_t rD = make_rsrc(a.D + row, uint32_t(T) * d * 4u);
    const rsrc_t rqa = make_rsrc(a.q_pre ? static_cast<IO*>(a.q_pre) + row : nullptr,
                                 a.q_pre ? uint32_t(T) * d * sizeof(IO) : 0u);
    const rsrc_t rqb = make_rsrc(a.q_post ? static_cast<IO*>(a.q_post) + row : nullptr,
                                 a.q_post ? uint32_t(T) * d * sizeof(IO) : 0u);
    const uint32_t vo4 = col ? uint32_t(x) * 4u : kOob, vo = col ? uint32_t(x) * sizeof(IO) : kOob;
    float q = col ? a.q0[int64_t(b) * d + x] : 0.0f;
    constexpr int kR = 32;
    for (int r0 = 0; r0 < T; r0 += kR * kScanWaves) {
        const int t0 = r0 + w * kR;
        float Dv[kR];
#pragma unroll
        for (int j = 0; j < kR; ++j) {  // past T: the lane offset masks the load (reads 0)
            const bool in = t0 + j < T;
            Dv[j] = bload<float>(rD, in ? vo4 : kOob, uint32_t(in ? t0 + j : 0) * d * 4u);
        }
        const uint32_t rsm = static_cast<uint32_t>(ballot(
            lane < kR && t0 + lane < T && a.reset != nullptr && a.reset[int64_t(b) * T + t0 + lane] != 0));
        float c = 0.0f;
#pragma unroll
        for (int j = 0; j < kR; ++j) {
            if ((rsm >> j) & 1u) c = 0.0f;
            c += divn(Dv[j]);
        }
        if (lane == 0) rss[w] = rsm != 0u ? 1 : 0;
        cx[w][lane] = c;
        __syncthreads();
        float qs = q;  // this range's start value
        for (int j = 0; j < w; ++j) qs = (rss[j] ? 0.0f : qs) + cx[j][lane];
        float qe = qs;  // the round's end value
        for (int j = w; j < kScanWaves; ++j) qe = (rss[j] ? 0.0f : qe) + cx[j][lane];
        float qq = qs;
#pragma unroll
        for (int j = 0; j < kR; ++j) {  // past T: the lane offset drops the stores
            const bool in = t0 + j < T;
            const uint32_t so = uint32_t(in ? t0 + j : 0) * d * sizeof(IO);
            const uint32_t vj = in ? vo : kOob;
            if ((rsm >> j) & 1u) qq = 0.0f;
            bstore_f32<IO>(qq, rqa, vj, so);
            qq = qq + divn(Dv[j]);
            bstore_f32<IO>(qq, rqb, vj, so);
        }
        q = qe;
        __syncthreads();  // before the next round reuses the exchange
    }
    if (a.q_T && w == 0 && col) a.q_T[int64_t(b) * d + x] = q;
}

// The reverse scan of the summary cotangent (python/hsn/train/split.py:154-173): latest first,
// R += dq_post[t]; share[t] = R / N; R += dq_pre[t]; a reset at t zeroes R after it. In fp64
// (so the ranges' composition rounds no differently from a sequential sum), each share rounded
// once to fp32.
template <typename IO>
__global__ __launch_bounds__(64 * kScanWaves) void summary_scan_bwd(ScanArgs a) {
    __shared__ int rss[kScanWaves];
    __shared__ double cx[kScanWaves][64];
    const int b = blockIdx.y, z = blockIdx.x;
    const int lane = lane_id(), w = uniform(threadIdx.x / 64);
    const int x = z * 64 + lane;
    const bool col = x < a.d;
    const int T = a.T, d = a.d;
    const DivN divn = a.divn;
    const int64_t row = int64_t(b) * T * d;
    const rsrc_t rpa = make_rsrc(a.dq_pre ? static_cast<const IO*>(a.dq_pre) + row : nullptr,
                                 a.dq_pre ? uint32_t(T) * d * sizeof(IO) : 0u);
    const rsrc_t rpb = make_rsrc(a.dq_post ? static_cast<const IO*>(a.dq_post) + row : nullptr,
                                 a.dq_post ? uint32_t(T) * d * sizeof(IO) : 0u);
    const rsrc_t rsh = make_rsrc(a.share + row, uint32_t(T) * d * 4u);
    const uint32_t vo4 = col ? uint32_t(x) * 4u : kOob, vo = col ? uint32_t(x) * sizeof(IO) : kOob;
    double R = (col && a.dq_T) ? double(a.dq_T[int64_t(b) * d + x]) : 0.0;
    constexpr int kR = 16;  // two values per position, within 128 registers
    const int span = kR * kScanWaves;
    const int rounds = (T + span - 1) / span;
    for (int rr = rounds - 1; rr >= 0; --rr) {
        const int t0 = rr * span + w * kR;
        float va[kR], vb[kR];
#pragma unroll
        for (int j = 0; j < kR; ++j) {  // past T: the lane offset masks the loads (reads 0)
            const bool in = t0 + j < T;
            const uint32_t so = uint32_t(in ? t0 + j : 0) * d * sizeof(IO);
            va[j] = to_f32(bload<IO>(rpa, in ? vo : kOob, so));
            vb[j] = to_f32(bload<IO>(rpb, in ? vo : kOob, so));
        }
        const uint32_t rsm = static_cast<uint32_t>(ballot(
            lane < kR && t0 + lane < T && a.reset != nullptr && a.reset[int64_t(b) * T + t0 + lane] != 0));
        double c = 0.0;  // this range's map on R, latest first: R -> (reset ? 0 : R) + c
#pragma unroll
        for (int j = kR - 1; j >= 0; --j) {
            c += double(vb[j]);
            c += double(va[j]);
            if ((rsm >> j) & 1u) c = 0.0;
        }
        if (lane == 0) rss[w] = rsm != 0u ? 1 : 0;
        cx[w][lane] = c;
        __syncthreads();
        double Rs = R;  // R entering this range: the later ranges' maps applied
        for (int j = kScanWaves - 1; j > w; --j) Rs = (rss[j] ? 0.0 : Rs) + cx[j][lane];
        double Re = Rs;
        for (int j = w; j >= 0; --j) Re = (rss[j] ? 0.0 : Re) + cx[j][lane];
        double Rr = Rs;
#pragma unroll
        for (int j = kR - 1; j >= 0; --j) {
            Rr += double(vb[j]);
            const bool in = t0 + j < T;
            bstore(static_cast<float>(divn(Rr)), rsh, in ? vo4 : kOob, uint32_t(in ? t0 + j : 0) * d * 4u);
            Rr += double(va[j]);
            if ((rsm >> j) & 1u) Rr = 0.0;
        }
        R = Re;
        __syncthreads();
    }
    if (a.dq0 && w == 0 && col) a.dq0[int64_t(b) * d + x] = static_cast<float>(R);
}

// ------------------------------------------------------------------------------------------
// Backward chains
// ------------------------------------------------------------------------------------------

struct BwdArgs {
    const void* y;      // [B, T, K, d] io: the candidate's pre-activation (RMS: normalised)
    const void* g;      // the gate's pre-activation
    const void* h_old;
    const void* dsel;   // optional
    const int32_t* ptr;
    const int32_t* ev;
    const uint8_t* reset;
    const float* share;  // [B, T, d]
    const float* dh_T;   // optional [B, N, d]
    void* dy;
    void* dg;
    float* dh0;  // optional
    int B, T, N, d, K;
    int C, stage;
};

// Per cell, latest event first (python/hsn/train/split.py:154-173): with the cotangent A of the
// cell's state after the event and the share R / N of its position, g = A + d_h_sel + R / N;
// dc = b g, db = (c - h_old) g, then through c = tanh(y) and b = sigmoid(gate); the state before
// the event gets (1 - b)(A + d_h_sel) - b R / N (h_old enters the summary's delta with -1 / N).
template <typename IO, int V, int NB>
__global__ __launch_bounds__(kChainThreads) void chain_bwd(BwdArgs a) {
    extern __shared__ uint32_t lds_u[];
    int b, g;
    group_coords(b, g);
    const int tid = threadIdx.x, lane = lane_id();
    const int T = a.T, N = a.N, d = a.d, K = a.K;
    const int TW = (T + 31) / 32;
    int* nr = reinterpret_cast<int*>(lds_u);
    uint32_t* rbits = lds_u + (T + 2);
    int* nx = reinterpret_cast<int*>(rbits + TW);
    int* next = nx + TW + 1 + T;  // the layout of chain_fwd (no row maxima used)
    int* cptr = next + 1;
    int* cev = cptr + a.C + 1;
    int* order = cev + a.stage;
    const int c_begin = g * a.C, c_end = min(N, c_begin + a.C);
    const int nc = c_end - c_begin;
    const int32_t* ptr = a.ptr + int64_t(b) * (N + 1);
    const int32_t* ev = a.ev + int64_t(b) * T * K;
    const int pc0 = ptr[c_begin];
    const int nst = min(ptr[c_end] - pc0, a.stage);
    for (int i = tid; i <= nc; i += kChainThreads) cptr[i] = ptr[c_begin + i];
    for (int i = tid; i < nst; i += kChainThreads) cev[i] = ev[pc0 + i];
    if (tid == 0) next[0] = 0;
    reset_table(a.reset ? a.reset + int64_t(b) * T : nullptr, T, nr, rbits, nx, tid, kChainThreads);
    heavy_first(cptr, nc, order, tid, kChainThreads);
    const int64_t slot0 = int64_t(b) * T * K;
    const uint32_t row_bytes = uint32_t(T) * K * d * sizeof(IO);
    const rsrc_t ry = make_rsrc(static_cast<const IO*>(a.y) + slot0 * d, row_bytes);
    const rsrc_t rg = make_rsrc(static_cast<const IO*>(a.g) + slot0 * d, row_bytes);
    const rsrc_t rho = make_rsrc(static_cast<const IO*>(a.h_old) + slot0 * d, row_bytes);
    const rsrc_t rds = make_rsrc(a.dsel ? static_cast<const IO*>(a.dsel) + slot0 * d : nullptr,
                                 a.dsel ? row_bytes : 0u);
    const rsrc_t rdy = make_rsrc(static_cast<IO*>(a.dy) + slot0 * d, row_bytes);
    const rsrc_t rdg = make_rsrc(static_cast<IO*>(a.dg) + slot0 * d, row_bytes);
    const rsrc_t rsh = make_rsrc(a.share + int64_t(b) * T * d, uint32_t(T) * d * 4u);
    uint32_t voff[V], voff4[V];
#pragma unroll
    for (int v = 0; v < V; ++v) {
        const bool in = lane + 64 * v < d;
        voff[v] = in ? uint32_t(lane + 64 * v) * sizeof(IO) : kOob;
        voff4[v] = in ? uint32_t(lane + 64 * v) * 4u : kOob;
    }
    const uint32_t srow = uint32_t(d) * sizeof(IO), srow4 = uint32_t(d) * 4u;
    const int n_slots = T * K;
    const int pad_begin = ptr[N];

    struct Rows {
        IO y[NB][V], g[NB][V], h[NB][V], s[NB][V];
        float r[NB][V];
    };
    for (;;) {
        int slot = lane == 0 ? atomicAdd(next, 1) : 0;
        slot = __builtin_amdgcn_readfirstlane(slot);
        if (slot >= nc) break;
        const int ci = uniform(order[slot]);
        const int c = c_begin + ci;
        const int e_beg = uniform(cptr[ci]), e_end = uniform(cptr[ci + 1]);
        const bool staged = e_end - pc0 <= nst;
        float A[V];
        {  // the end cotangent, cut by a reset after the cell's last event
            const int t_last = e_end > e_beg
                                   ? (uniform(staged ? cev[e_end - 1 - pc0] : ev[e_end - 1]) >> 8)
                                   : -1;
            const bool cut = nr[t_last + 1] < T;
            const float* dhc = a.dh_T ? a.dh_T + (int64_t(b) * N + c) * d : nullptr;
#pragma unroll
            for (int v = 0; v < V; ++v)
                A[v] = (dhc && !cut && lane + 64 * v < d) ? dhc[lane + 64 * v] : 0.0f;
        }
        int tnext = T;  // the later event's position
        int t_first = T;
        auto walk = [&](auto staged_c) __attribute__((always_inline)) {
            constexpr bool kStaged = decltype(staged_c)::value;
            for (int w1 = e_end; w1 > e_beg; w1 -= kEvWin) {
                const int m = min(kEvWin, w1 - e_beg);
                const int w0 = w1 - m;
                int evw;
                if constexpr (kStaged) evw = lane < m ? cev[w0 - pc0 + lane] : 0;
                else evw = lane < m ? ev[w0 + lane] : 0;
                // the window's positions, slot offsets, share offsets and next resets, for all
                // its events at once (lane i: event i), read per event with readlane
                const int tw = evw >> 8;
                const uint32_t sow = uint32_t(tw * K + (evw & 255)) * srow;
                const uint32_t stw = uint32_t(tw) * srow4;
                const int nrw = lane < m ? nr[tw + 1] : T;
                Rows ra, rb;
                // batch j holds window indices [j - NB + 1, j], fetched latest first
                auto fetch = [&](int j, Rows& r) __attribute__((always_inline)) {
#pragma unroll
                    for (int i = 0; i < NB; ++i) {
                        const int idx = j - i;
                        const uint32_t so = __builtin_amdgcn_readlane(sow, max(idx, 0));
                        const uint32_t st = __builtin_amdgcn_readlane(stw, max(idx, 0));
                        const bool in = idx >= 0;
#pragma unroll
                        for (int v = 0; v < V; ++v) {
                            const uint32_t vo = in ? voff[v] : kOob;
                            r.y[i][v] = bload<IO>(ry, vo, so);
                            r.g[i][v] = bload<IO>(rg, vo, so);
                            r.h[i][v] = bload<IO>(rho, vo, so);
                            r.s[i][v] = bload<IO>(rds, vo, so);
                            r.r[i][v] = bload<float>(rsh, in ? voff4[v] : kOob, st);
                        }
                    }
                };
                auto step = [&](int j, const Rows& r) __attribute__((always_inline)) {
#pragma unroll
                    for (int i = 0; i < NB; ++i) {
                        const int idx = j - i;
                        if (idx >= 0) {
                            const int t = __builtin_amdgcn_readlane(tw, idx);
                            const int nrq = __builtin_amdgcn_readlane(nrw, idx);
                            const uint32_t so = __builtin_amdgcn_readlane(sow, idx);
                            const bool zero = nrq <= tnext && tnext < T;  // a reset in (t, tnext]
#pragma unroll
                            for (int v = 0; v < V; ++v) {
                                const float carried = (zero ? 0.0f : A[v]) + to_f32(r.s[i][v]);
                                const float share = r.r[i][v];
                                const float gg = carried + share;
                                const float bg = fast_sigmoid(to_f32(r.g[i][v]));
                                const float cc = fast_tanh(to_f32(r.y[i][v]));
                                const float dc = bg * gg * (1.0f - cc * cc);
                                const float db = (cc - to_f32(r.h[i][v])) * gg * (bg * (1.0f - bg));
                                bstore_f32<IO>(dc, rdy, voff[v], so);
                                bstore_f32<IO>(db, rdg, voff[v], so);
                                A[v] = (1.0f - bg) * carried - bg * share;
                            }
                            tnext = t;
                        }
                    }
                };
                fetch(m - 1, ra);
                for (int j = m - 1; j >= 0; j -= 2 * NB) {
                    fetch(j - NB, rb);
                    step(j, ra);
                    if (j - NB < 0) break;
                    fetch(j - 2 * NB, ra);
                    step(j - NB, rb);
                }
            }
        };
        if (staged) walk(std::true_type{});
        else walk(std::false_type{});
        t_first = tnext;
        if (a.dh0) {  // the start state's cotangent: cut by a reset at or before the first event
            const bool z = nr[0] <= min(t_first, T - 1);
            float* d0 = a.dh0 + (int64_t(b) * N + c) * d;
#pragma unroll
            for (int v = 0; v < V; ++v)
                if (lane + 64 * v < d) d0[lane + 64 * v] = z ? 0.0f : A[v];
        }
    }
    if (g == 0) {  // exact zeros on the row's padded slots, every wavefront a share
        const int wv = tid >> 6;
        for (int pw = pad_begin + wv * kEvWin; pw < n_slots; pw += kEvWin * kChainWaves) {
            const int m = min(kEvWin, n_slots - pw);
            const int pe = lane < m ? ev[pw + lane] : 0;
            for (int i = 0; i < m; ++i) {
                const int q = __builtin_amdgcn_readlane(pe, i);
                const uint32_t so = uint32_t((q >> 8) * K + (q & 255)) * srow;
#pragma unroll
                for (int v = 0; v < V; ++v) {
                    bstore_f32<IO>(0.0f, rdy, voff[v], so);
                    bstore_f32<IO>(0.0f, rdg, voff[v], so);
                }
            }
        }
    }
}

}  // namespace chain
}  // namespace hsn
