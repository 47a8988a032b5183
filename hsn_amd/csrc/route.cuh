// The router's shared device code: its argument block, wavefront reductions, the float
// images and keys of the scores, and the selection of one position without probes
// (decide_select), used by the router's kernels and by the forward sweep that routes its own
// window (evmap.cuh).
//
// The CPU path rounds every product and sum on its own, so this header turns floating-point
// contraction off for the rest of any file that includes it: a file that includes it after
// its other kernels keeps their contraction.
#pragma once

#include "common.cuh"
#include "bufio.cuh"
#include "dpp.cuh"

#include <type_traits>

// The CPU path rounds every product and sum on its own (scores - lambda * cost is a multiply,
// then a subtract): no fused multiply-adds anywhere in the router.
#pragma clang fp contract(off)

namespace hsn {
namespace {
// one rounding each (written here, below the pragma: the header's mul_rn and friends carry
// their own contraction state into the caller when inlined)
__device__ __forceinline__ float mul_rn(float x, float y) { return x * y; }
__device__ __forceinline__ float sub_rn(float x, float y) { return x - y; }
__device__ __forceinline__ float add_rn(float x, float y) { return x + y; }
}  // namespace
}  // namespace hsn

namespace hsn {
namespace {

struct RouteArgs {
    const void* logits;
    int64_t l_row, l_pos, width;  // element offset of (b, p, n, j) = b*l_row + p*l_pos + n*width + j
    const float* cost;
    const int64_t* age;  // per-position form: [B, n_age, N], record `age_rec` of row b
    int64_t age_row, age_rec;
    const int64_t* age0;  // window form with probes: [B, N]
    const uint8_t* reset;  // window form with probes: [B, P]
    void* cells;
    void* units;
    uint8_t* valid;
    uint8_t* refreshed;
    int32_t* slots;  // optional: the cell where valid, -1 where padded (the sweeps' input)
    int64_t o_row, o_pos;  // output slot offset of (b, p, k) = b*o_row + p*o_pos + k
    float* theta;
    int64_t th_row, th_pos;
    float* h_max_zero;  // [B, P] (optional)
    // optional: the decisions handed to the other workgroups of a row by the forward sweep
    // that routes its own window, one word a slot at the slot's output offset:
    // (stamp << 16) | (cell + 1), 0 in the low bits where the slot is padded
    uint64_t* box;
    int B, P, N, M, K, age_max, probes, reserved, fixed_units;
    float lambda, overhead, shared, limit;
};

// Wavefront reductions with DPP (no LDS traffic): the four steps inside each 16-lane row are
// symmetric (every lane ends with the row's result), row_bcast:15 / row_bcast:31 then fold the
// rows into lane 63, which is read as a uniform value.
template <typename F>
__device__ __forceinline__ uint32_t wave_reduce_u32(uint32_t v, F op, uint32_t identity) {
    v = op(v, dpp_u32<dpp::kXor1>(v));
    v = op(v, dpp_u32<dpp::kXor2>(v));
    v = op(v, dpp_u32<dpp::kHalfMirror>(v));
    v = op(v, dpp_u32<dpp::kRor8>(v));
    v = op(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(
                  static_cast<int>(identity), static_cast<int>(v), 0x142, 0xa, 0xf, false)));
    v = op(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(
                  static_cast<int>(identity), static_cast<int>(v), 0x143, 0xc, 0xf, false)));
    return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 63));
}
template <typename F>
__device__ __forceinline__ float wave_reduce_f32(float v, F op, float identity) {
    auto u = [](float f) { return static_cast<uint32_t>(__float_as_int(f)); };
    auto f = [](uint32_t x) { return __int_as_float(static_cast<int>(x)); };
    const uint32_t r = wave_reduce_u32(
        u(v), [&](uint32_t a, uint32_t b) { return u(op(f(a), f(b))); }, u(identity));
    return f(r);
}

// Wavefront argmax of this lane's best (key, n): the largest key, the smallest n among equal
// keys. Cells are laid out in blocks (lane l holds n = l*NPL + i), so among equal keys the
// lowest lane holds the smallest n, and a lane's best is its first maximum.
__device__ __forceinline__ void wave_argmax(uint32_t k, int n, uint32_t& wk, int& wn) {
    wk = wave_reduce_u32(k, [](uint32_t a, uint32_t b) { return a > b ? a : b; }, 0u);
    const int src = __builtin_ctzll(ballot(k == wk));
    wn = __builtin_amdgcn_readlane(n, src);
}

__device__ __forceinline__ float wave_nan_min(float v) {
    return wave_reduce_f32(v, [](float a, float b) { return nan_min(a, b); }, INFINITY);
}
__device__ __forceinline__ float wave_nan_max(float v) {
    return wave_reduce_f32(v, [](float a, float b) { return nan_max(a, b); }, -INFINITY);
}
__device__ __forceinline__ int wave_sum(int v) {
    return static_cast<int>(wave_reduce_u32(
        static_cast<uint32_t>(v), [](uint32_t a, uint32_t b) { return a + b; }, 0u));
}

template <typename IDX>
__device__ __forceinline__ void store_index(void* p, int64_t i, int v) {
    static_cast<IDX*>(p)[i] = static_cast<IDX>(v);
}

// The order-preserving signed-integer image of a non-NaN float (an involution): non-negative
// floats keep their bits and negative ones flip their magnitude bits, so -0 (-1) sorts just
// below +0 (0) and a float min / max is a signed-integer one.
__device__ __forceinline__ int32_t ford(float f) {
    const int32_t u = __float_as_int(f);
    return u ^ ((u >> 31) & 0x7fffffff);
}
__device__ __forceinline__ float ford_inv(int32_t k) {
    return __int_as_float(k ^ ((k >> 31) & 0x7fffffff));
}
// NaN-propagating wavefront amin / amax (torch's: NaN when any lane holds one) of float images:
// a ballot finds a NaN, the rest is a signed-integer min / max, one DPP instruction a step (a
// float tree needs the neighbour's value canonicalised first). Of -0 and +0 the min is -0 and
// the max +0, whichever lane holds them.
__device__ __forceinline__ float wave_amin_k(int32_t k, bool nan) {
    const bool any_nan = ballot(nan) != 0u;
    const uint32_t m = wave_reduce_u32(
        static_cast<uint32_t>(k),
        [](uint32_t x, uint32_t y) { return static_cast<int32_t>(x) < static_cast<int32_t>(y) ? x : y; },
        static_cast<uint32_t>(ford(INFINITY)));
    return any_nan ? __int_as_float(0x7fc00000) : ford_inv(static_cast<int32_t>(m));
}
__device__ __forceinline__ float wave_amax_k(int32_t k, bool nan) {
    const bool any_nan = ballot(nan) != 0u;
    const uint32_t m = wave_reduce_u32(
        static_cast<uint32_t>(k),
        [](uint32_t x, uint32_t y) { return static_cast<int32_t>(x) > static_cast<int32_t>(y) ? x : y; },
        static_cast<uint32_t>(ford(-INFINITY)));
    return any_nan ? __int_as_float(0x7fc00000) : ford_inv(static_cast<int32_t>(m));
}

// A lane's NPL consecutive logits as one buffer load (the row's resource bounds it).
template <int NPL, typename IO>
__device__ __forceinline__ void load_run(IO (&raw)[NPL], rsrc_t r, uint32_t voff) {
    constexpr int kBytes = NPL * static_cast<int>(sizeof(IO));
    if constexpr (kBytes == 16) {
        const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, 0, 0);
        __builtin_memcpy(raw, &v, 16);
    } else if constexpr (kBytes == 8) {
        const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, voff, 0, 0);
        __builtin_memcpy(raw, &v, 8);
    } else if constexpr (kBytes == 4) {
        const uint32_t v = __builtin_amdgcn_raw_buffer_load_b32(r, voff, 0, 0);
        __builtin_memcpy(raw, &v, 4);
    } else {
        const uint16_t v = __builtin_amdgcn_raw_buffer_load_b16(r, voff, 0, 0);
        __builtin_memcpy(raw, &v, 2);
    }
}

// A lane's NPL consecutive logits, any multiple of 16 bytes or a power of two below, as vector
// buffer loads (a lane past the row reads zeros).
template <int NPL, typename IO>
__device__ __forceinline__ void load_block(IO (&raw)[NPL], rsrc_t r, uint32_t voff) {
    constexpr int kBytes = NPL * static_cast<int>(sizeof(IO));
    if constexpr (kBytes <= 16) {
        load_run<NPL, IO>(raw, r, voff);
    } else {
        static_assert(kBytes % 16 == 0, "whole 16-byte runs");
        constexpr int kPer = 16 / static_cast<int>(sizeof(IO));
#pragma unroll
        for (int c = 0; c < kBytes / 16; ++c) {
            const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, voff + 16u * c, 0, 0);
            __builtin_memcpy(&raw[c * kPer], &v, 16);
        }
    }
}

// The float of a score key below the NaN key (score_key's inverse; the key of -0 is +0's).
__device__ __forceinline__ float key_score(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k ^ 0x80000000u) : ~k);
}

// The slot table's budget, threshold and outputs (steps 4 and on of decide_select): `tab` holds
// the K slots in the selection's order, `pool` / `pool_nan` theta's highest unselected score
// over the cells outside the table.
template <bool kOne, typename IDX>
__device__ __forceinline__ void finish_select(const RouteArgs& a, int b, int p, const uint4* tab,
                                              int32_t pool, bool pool_nan, float cost0,
                                              uint64_t stamp = 0) {
    const int lane = lane_id();
    const int K = a.K, R = a.reserved, M = a.M;
    (void)M;
    __builtin_amdgcn_wave_barrier();  // the slot table's writes before its reads
    const bool is_slot = lane < K;
    const uint4 e = is_slot ? tab[lane] : make_uint4(0u, 0u, 0u, 0u);
    const int my_cell = static_cast<int>(e.y);
    const float my_score = __uint_as_float(e.z);

    // 4. the budget (as decide)
    int my_unit = 0;
    float cumulative;
    if constexpr (kOne) {
        const float ps = add_rn(a.overhead, cost0);
        cumulative = add_rn(a.shared, static_cast<float>(static_cast<double>(ps) * (lane + 1)));
    } else {
        my_unit = (a.fixed_units && lane < R) ? lane % M : static_cast<int>(e.w);
        const float my_cost = is_slot ? a.cost[my_unit] : 0.0f;
        const float per_slot = is_slot ? add_rn(a.overhead, my_cost) : 0.0f;
        double acc = 0.0;
        for (int j = 0; j < K; ++j) {
            const float v = readlane(per_slot, j);
            if (j <= lane) acc += static_cast<double>(v);
        }
        cumulative = add_rn(a.shared, static_cast<float>(acc));
    }
    const bool ok = is_slot && cumulative <= a.limit;

    // the threshold: the lowest selected scored slot, the highest unselected cell (the pool and
    // the table's slots past the budget)
    const bool in_low = ok && my_cell >= R;
    const float low = wave_amin_k(in_low ? ford(my_score) : ford(INFINITY), in_low && my_score != my_score);
    const bool cut = is_slot && !ok;
    const int32_t hk = max(pool, cut ? ford(my_score) : ford(-INFINITY));
    const float high = wave_amax_k(hk, pool_nan | (cut && my_score != my_score));
    const float th = 0.5f * (low + high);

    if (is_slot) {
        const int64_t o = b * a.o_row + p * a.o_pos + lane;
        store_index<IDX>(a.cells, o, ok ? my_cell : 0);
        store_index<IDX>(a.units, o, ok ? my_unit : 0);
        a.valid[o] = ok ? 1 : 0;
        a.refreshed[o] = 0;
        if (a.slots) a.slots[o] = ok ? my_cell : -1;
        if (a.box)  // one relaxed agent-scope word: the reader needs no fence, only the stamp
            __hip_atomic_store(a.box + o, (stamp << 16) | uint64_t(ok ? my_cell + 1 : 0),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (lane == 0) {
        a.theta[b * a.th_row + p * a.th_pos] = th;
        if (a.h_max_zero) a.h_max_zero[static_cast<int64_t>(b) * a.P + p] = 0.0f;
    }
}

// A lane's one-unit logits of position (b, p): cells lane * NPL .. lane * NPL + NPL - 1 as one
// vector load where the row is contiguous and aligned (lanes past the row read zeros, which
// the selection masks), else one load a cell (cells past N read cell N - 1).
template <int NPL, typename IO>
__device__ __forceinline__ void load_logits(const RouteArgs& a, int b, int p, IO (&raw)[NPL]) {
    const int lane = lane_id();
    const int N = a.N;
    const IO* logits = static_cast<const IO*>(a.logits) + b * a.l_row + p * a.l_pos;
    constexpr uint32_t kRun = NPL * sizeof(IO);
    const bool vec = a.width == 1 && N % NPL == 0 &&
                     (reinterpret_cast<uintptr_t>(logits) & (kRun >= 16 ? 15 : kRun - 1)) == 0;
    if (vec) {
        const rsrc_t r = make_rsrc(logits, uint32_t(N) * sizeof(IO));
        load_block<NPL, IO>(raw, r, lane * NPL < N ? uint32_t(lane) * kRun : kOob);
    } else {
#pragma unroll
        for (int i = 0; i < NPL; ++i)
            raw[i] = logits[int64_t(min(lane * NPL + i, N - 1)) * a.width];
    }
}

// The decision of one position without probes, any NPL: a threshold, then an exact order of
// the few cells at or above it.
//  1. Every lane's largest key; L = the largest 16-bit key prefix that at least Kc = K + 1 (K
//     when K = N) lanes' maxima reach, by 16 steps of ballot and popcount. The Kc-th largest
//     lane maximum is at most the Kc-th largest key overall (a subset's Kc-th largest is at most
//     the set's), so every cell of the top Kc, reserved and NaN keys included, has a key >= L.
//  2. The candidates, every cell with key >= L (about Kc and a few more), go to LDS, compacted
//     with ballot and mbcnt. More than 64 (heavy ties) take K rounds of a wavefront argmax over
//     the keys in registers instead.
//  3. Each candidate's rank is its count of candidates before it in the selection's order (key
//     descending, cell ascending): the stable order exactly. Rank k < K is slot k.
//  4. The budget as `decide`; theta's highest unselected score is the largest of the unselected
//     candidates (NaN-propagating) and of the keys below L (no NaN there: a NaN key is the
//     largest), whose float is exact but for -0 reading as +0, which changes no threshold (a zero
//     below L means every selected score is positive).
// VALU work per position is about 10 per cell and 6 per candidate, against 16 per slot for the
// K rounds of a wavefront argmax.
template <int NPL, bool kOne, typename IO, typename IDX>
__device__ void decide_select_from(const RouteArgs& a, int b, int p, const IO (&raw)[kOne ? NPL : 1],
                                   uint4* cand, uint4* tab, uint64_t* ord, uint64_t stamp = 0) {
    const int lane = lane_id();
    const int N = a.N, M = a.M, K = a.K, R = a.reserved;
    const IO* logits = static_cast<const IO*>(a.logits) + b * a.l_row + p * a.l_pos;
    const bool scale_cost = a.lambda > 0.0f;

    // kOne keeps the raw logits and recomputes a score where one is needed (a candidate, the
    // pool): scores, keys and logits together would hold three registers per cell
    constexpr int kS = kOne ? 1 : NPL;
    float scv[kS];
    int unit[kS];
    uint32_t key[NPL];
    const float cost0 = kOne ? a.cost[0] : 0.0f;
    const float lc = kOne && scale_cost ? mul_rn(a.lambda, cost0) : 0.0f;
    auto score = [&](int i) __attribute__((always_inline)) -> float {
        if constexpr (kOne) {
            const float v = to_f32(raw[i]);
            return scale_cost ? sub_rn(v, lc) : v;
        } else {
            return scv[i];
        }
    };
    auto unit_of = [&](int i) __attribute__((always_inline)) -> int {
        if constexpr (kOne) return 0;
        else return unit[i];
    };
    if constexpr (kOne) {
        if (N == kWave * NPL && R == 0 && !scale_cost) {  // uniform: every lane full, no masks
#pragma unroll
            for (int i = 0; i < NPL; ++i) key[i] = score_key(to_f32(raw[i]));
        } else {
#pragma unroll
            for (int i = 0; i < NPL; ++i) {
                const int n = lane * NPL + i;
                const uint32_t in = 0u - static_cast<uint32_t>(n < N);
                const uint32_t rsv = 0u - static_cast<uint32_t>(n < R);
                key[i] = ((score_key(score(i)) & ~rsv) | (kKeyPosInf & rsv)) & in;
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < NPL; ++i) {
            const int n = lane * NPL + i;
            scv[i] = -INFINITY;
            unit[i] = 0;
            key[i] = 0u;
            if (n < N) {
                const IO* row = logits + static_cast<int64_t>(n) * a.width;
                float best = to_f32(row[0]);
                if (scale_cost) best = sub_rn(best, mul_rn(a.lambda, a.cost[0]));
                int arg = 0;
                for (int j = 1; j < M; ++j) {
                    float s = to_f32(row[j]);
                    if (scale_cost) s = sub_rn(s, mul_rn(a.lambda, a.cost[j]));
                    if (best == best && (s > best || s != s)) {
                        best = s;
                        arg = j;
                    }
                }
                scv[i] = best;
                unit[i] = arg;
                key[i] = n < R ? kKeyPosInf : score_key(best);
            }
        }
    }

    // 1. the threshold prefix from the lanes' maxima
    uint32_t hb = 0u;
#pragma unroll
    for (int i = 0; i < NPL; ++i) hb = umax(hb, key[i]);
    const int Kc = K < N ? K + 1 : K;
    const uint32_t top = hb >> 16;
    uint32_t pfx = 0u;
#pragma unroll
    for (int bit = 15; bit >= 0; --bit) {
        const uint32_t c = pfx | (1u << bit);
        pfx = __popcll(ballot(top >= c)) >= Kc ? c : pfx;
    }
    const uint32_t L = pfx > 0u ? pfx << 16 : 1u;  // 1: every real key (a cell past N has key 0)

    // 2. the candidates into LDS, and the largest key below L
    uint32_t below = 0u;
    int C = 0;
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
        const bool c = key[i] >= L;
        below = umax(below, c ? 0u : key[i]);
        const uint64_t m = ballot(c);
        if (m != 0u) {  // uniform
            const int at = C + lanes_below(m);
            if (c && at < kWave) {
                const uint32_t n = uint32_t(lane * NPL + i);
                cand[at] = make_uint4(key[i], n, __float_as_uint(score(i)), uint32_t(unit_of(i)));
                ord[at] = (uint64_t(key[i]) << 32) | ~n;  // the selection's order as one integer
            }
            C += __popcll(m);
        }
    }
    // Theta's highest unselected score over the cells outside the slot table (`pool`: a signed
    // image, `pool_nan`); the table's slots past the budget join it below.
    int32_t pool;
    bool pool_nan;
    if (C <= kWave) {
        __builtin_amdgcn_wave_barrier();  // the candidates' writes before their reads
        const bool is_c = lane < C;
        const uint4 me = is_c ? cand[lane] : make_uint4(0u, 0xffffffffu, 0u, 0u);
        // 3. each candidate's place in the selection's order: (key, ~cell) as one unsigned
        // integer, the other candidates' read by broadcast from LDS, four a step (the slots past
        // C hold 0, below every candidate)
        const uint64_t mine = (uint64_t(me.x) << 32) | ~me.y;
        if (lane >= C) ord[lane] = 0u;
        __builtin_amdgcn_wave_barrier();
        int rank = 0;
        for (int j = 0; j < C; j = uniform(j + 4)) {
            const uint64_t o0 = ord[j], o1 = ord[j + 1], o2 = ord[j + 2], o3 = ord[j + 3];
            rank += static_cast<int>(o0 > mine) + static_cast<int>(o1 > mine) +
                    static_cast<int>(o2 > mine) + static_cast<int>(o3 > mine);
        }
        if (is_c && rank < K) tab[rank] = me;
        const bool out = is_c && rank >= K;
        const float cs = __uint_as_float(me.z);
        pool = max(out ? ford(cs) : ford(-INFINITY), below != 0u ? ford(key_score(below)) : ford(-INFINITY));
        pool_nan = out && cs != cs;
    } else {
        // Heavy ties: K rounds of a wavefront argmax over the keys in registers (the largest
        // key, the lowest cell of it: cells are in blocks, so the first lane and its first
        // entry); the winner's entry leaves the pool.
        uint32_t bk = 0u;
        int bi = 0;
#pragma unroll
        for (int i = 0; i < NPL; ++i) {
            const bool gt = key[i] > bk;
            bk = gt ? key[i] : bk;
            bi = gt ? i : bi;
        }
        for (int r = 0; r < K; r = uniform(r + 1)) {
            const uint32_t wk = wave_reduce_u32(bk, [](uint32_t x, uint32_t y) { return x > y ? x : y; }, 0u);
            const int src = __builtin_ctzll(ballot(bk == wk));
            if (lane == src) {
#pragma unroll
                for (int i = 0; i < NPL; ++i) {
                    if (i == bi) {
                        tab[r] = make_uint4(key[i], uint32_t(lane * NPL + i), __float_as_uint(score(i)),
                                            uint32_t(unit_of(i)));
                        key[i] = 0u;
                    }
                }
                bk = 0u;
                bi = 0;
#pragma unroll
                for (int i = 0; i < NPL; ++i) {
                    const bool gt = key[i] > bk;
                    bk = gt ? key[i] : bk;
                    bi = gt ? i : bi;
                }
            }
        }
        pool = ford(-INFINITY);
        pool_nan = false;
#pragma unroll
        for (int i = 0; i < NPL; ++i) {  // every real cell still in the pool
            const bool out = key[i] != 0u;
            const float si = score(i);
            pool = max(pool, out ? ford(si) : ford(-INFINITY));
            pool_nan = pool_nan | (out & (si != si));
        }
    }
    finish_select<kOne, IDX>(a, b, p, tab, pool, pool_nan, cost0, stamp);
}

// decide_select_from with the position's logits loaded here (kOne: a lane's cells; otherwise
// the selection reads each cell's unit logits itself).
template <int NPL, bool kOne, typename IO, typename IDX>
__device__ __forceinline__ void decide_select(const RouteArgs& a, int b, int p, uint4* cand,
                                              uint4* tab, uint64_t* ord) {
    IO raw[kOne ? NPL : 1];
    if constexpr (kOne) load_logits<NPL, IO>(a, b, p, raw);
    decide_select_from<NPL, kOne, IO, IDX>(a, b, p, raw, cand, tab, ord);
}

}  // namespace
}  // namespace hsn
