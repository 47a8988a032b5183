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
                                              uint4* tab, uint64_t* ord, uint64_t stamp = 0) {
    IO raw[kOne ? NPL : 1];
    if constexpr (kOne) load_logits<NPL, IO>(a, b, p, raw);
    decide_select_from<NPL, kOne, IO, IDX>(a, b, p, raw, cand, tab, ord, stamp);
}

// ---- the selection of G = 64 / LP positions a wavefront ------------------------------------
//
// Group g of LP lanes (lanes g LP .. g LP + LP - 1) decides position q0 + g, lane gl of the group
// holding cells gl CPL .. gl CPL + CPL - 1, so each instruction serves G positions. The steps of
// decide_select, group-wise:
//  1. the keys; L = the Kc-th largest of the group's lane maxima (a bitonic sort of the LP
//     maxima), so every cell of the top Kc has a key >= L (as the prefix of decide_select);
//  2. the candidates (key >= L) compacted into the group's LDS list by a scan of the lanes'
//     counts, the scores read back from the lanes' LDS rows;
//  3. each candidate's rank in the group's list, the slot table, the pool of unselected scores;
//  4. the budget, the threshold and the outputs of finish_select over the group's lanes.
// A group with more than LP candidates (heavy ties) is left to decide_select (the returned mask).

// Reduction over each aligned group of LP lanes with a commutative, idempotent or associative
// `op`; every lane of a group ends with the group's result.
template <int LP, typename F>
__device__ __forceinline__ uint32_t group_reduce_u32(uint32_t v, F op) {
    if constexpr (LP >= 2) v = op(v, dpp_u32<dpp::kXor1>(v));
    if constexpr (LP >= 4) v = op(v, dpp_u32<dpp::kXor2>(v));
    if constexpr (LP >= 8) v = op(v, dpp_u32<dpp::kHalfMirror>(v));
    if constexpr (LP >= 16) v = op(v, dpp_u32<dpp::kRor8>(v));
    if constexpr (LP >= 32) {
        const RowPair r = pair16(v);
        v = op(r.lo, r.hi);
    }
    if constexpr (LP >= 64) {
        const RowPair r = pair32(v);
        v = op(r.lo, r.hi);
    }
    return v;
}

template <int LP>
__device__ __forceinline__ uint64_t group_lanes(int g) {
    if constexpr (LP >= kWave) return ~uint64_t(0);
    else return ((uint64_t(1) << LP) - 1u) << (g * LP);
}

// Inclusive prefix sum over each aligned group of LP lanes (16-lane rows by row shifts, then the
// rows joined by row broadcasts).
template <int LP>
__device__ __forceinline__ uint32_t group_scan_u32(uint32_t v) {
    auto shr = [](uint32_t x, auto s_c) __attribute__((always_inline)) {
        return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(
            0, static_cast<int>(x), 0x110 + decltype(s_c)::value, 0xf, 0xf, false));
    };
    v += shr(v, std::integral_constant<int, 1>{});
    v += shr(v, std::integral_constant<int, 2>{});
    v += shr(v, std::integral_constant<int, 4>{});
    v += shr(v, std::integral_constant<int, 8>{});
    if constexpr (LP >= 32)  // row_bcast:15 into rows 1 and 3
        v += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x142, 0xa, 0xf, false));
    if constexpr (LP >= 64)  // row_bcast:31 into rows 2 and 3
        v += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x143, 0xc, 0xf, false));
    return v;
}

// The value of lane (lane ^ J) (J a power of two below LP <= 64).
template <int J>
__device__ __forceinline__ uint32_t xor_partner(uint32_t v, int lane) {
    if constexpr (J == 1) {
        return dpp_u32<dpp::kXor1>(v);
    } else if constexpr (J == 2) {
        return dpp_u32<dpp::kXor2>(v);
    } else if constexpr (J == 4) {
        // row_ror:r hands lane i the value of lane (i - r) mod 16 (as row_shr:1 gives lane i - 1)
        const uint32_t from_below = dpp_u32<0x124>(v), from_above = dpp_u32<0x12C>(v);
        return (lane & 4) ? from_below : from_above;
    } else if constexpr (J == 8) {
        return dpp_u32<dpp::kRor8>(v);
    } else if constexpr (J == 16) {
        const RowPair r = pair16(v);
        return (lane & 16) ? r.lo : r.hi;
    } else {
        const RowPair r = pair32(v);
        return (lane & 32) ? r.lo : r.hi;
    }
}

// Bitonic sort of each group's LP values, descending (group lane 0 ends with the largest).
template <int LP, int K2 = 2, int J = 1>
__device__ __forceinline__ uint32_t group_sort_desc(uint32_t v, int gl, int lane) {
    if constexpr (K2 > LP) {
        return v;
    } else {
        const uint32_t p = xor_partner<J>(v, lane);
        const bool keep_max = ((gl & J) == 0) == ((gl & K2) == 0);
        v = keep_max ? (v > p ? v : p) : (v < p ? v : p);
        if constexpr (J > 1) return group_sort_desc<LP, K2, J / 2>(v, gl, lane);
        else return group_sort_desc<LP, K2 * 2, K2>(v, gl, lane);
    }
}

template <int LP>
__device__ __forceinline__ float group_amin_k(int32_t k, bool nan, int g) {
    const bool any_nan = (ballot(nan) & group_lanes<LP>(g)) != 0u;
    const uint32_t m = group_reduce_u32<LP>(static_cast<uint32_t>(k), [](uint32_t x, uint32_t y) {
        return static_cast<int32_t>(x) < static_cast<int32_t>(y) ? x : y;
    });
    return any_nan ? __int_as_float(0x7fc00000) : ford_inv(static_cast<int32_t>(m));
}
template <int LP>
__device__ __forceinline__ float group_amax_k(int32_t k, bool nan, int g) {
    const bool any_nan = (ballot(nan) & group_lanes<LP>(g)) != 0u;
    const uint32_t m = group_reduce_u32<LP>(static_cast<uint32_t>(k), [](uint32_t x, uint32_t y) {
        return static_cast<int32_t>(x) > static_cast<int32_t>(y) ? x : y;
    });
    return any_nan ? __int_as_float(0x7fc00000) : ford_inv(static_cast<int32_t>(m));
}

// A lane's CPL one-unit logits of a row (cells gl CPL ..): vector loads where the row is
// contiguous and aligned, else one load a cell (cells past N read cell N - 1).
template <int CPL, typename IO>
__device__ __forceinline__ void load_cells(const RouteArgs& a, const IO* logits, int gl, IO (&raw)[CPL]) {
    constexpr uint32_t kRun = CPL * sizeof(IO);
    const int N = a.N;
    const bool vec = a.width == 1 && N % CPL == 0 &&
                     (reinterpret_cast<uintptr_t>(logits) & (kRun >= 16 ? 15 : kRun - 1)) == 0;
    if (vec) {
        const int n0 = gl * CPL < N ? gl * CPL : 0;  // a lane past the row reads cell 0's run
        const unsigned char* src = reinterpret_cast<const unsigned char*>(logits + n0);
        if constexpr (kRun >= 16) {
#pragma unroll
            for (uint32_t c = 0; c < kRun / 16; ++c) {
                const uint4 v = *reinterpret_cast<const uint4*>(src + 16 * c);
                __builtin_memcpy(reinterpret_cast<unsigned char*>(raw) + 16 * c, &v, 16);
            }
        } else if constexpr (kRun == 8) {
            const uint2 v = *reinterpret_cast<const uint2*>(src);
            __builtin_memcpy(raw, &v, 8);
        } else if constexpr (kRun == 4) {
            const uint32_t v = *reinterpret_cast<const uint32_t*>(src);
            __builtin_memcpy(raw, &v, 4);
        } else {
            const uint16_t v = *reinterpret_cast<const uint16_t*>(src);
            __builtin_memcpy(raw, &v, 2);
        }
    } else {
#pragma unroll
        for (int i = 0; i < CPL; ++i)
            raw[i] = logits[int64_t(min(gl * CPL + i, N - 1)) * a.width];
    }
}

// decide_grouped's LDS scratch for one wavefront: the lanes' scores [CPL][64] f32, the groups'
// candidate lists [G][LP] uint4, order words [G][LP + 4] u64 and slot tables [G][LP] uint4 (the
// last three, at least 1024, 544 and 1024 bytes, also serve decide_select's full-wavefront
// scratch for a fallback).
struct GroupedScratch {
    float* sc;
    uint4* cand;
    uint64_t* ord;
    uint4* tab;
};
template <int LP, int CPL>
constexpr int grouped_scratch_bytes() {
    return CPL * kWave * 4 + kWave * 16 + (kWave / LP) * (LP + 4) * 8 + kWave * 16;
}
template <int LP, int CPL>
__device__ __forceinline__ GroupedScratch grouped_scratch(unsigned char* smem) {
    GroupedScratch s;
    s.sc = reinterpret_cast<float*>(smem);
    s.cand = reinterpret_cast<uint4*>(smem + CPL * kWave * 4);
    s.ord = reinterpret_cast<uint64_t*>(s.cand + kWave);
    s.tab = reinterpret_cast<uint4*>(s.ord + (kWave / LP) * (LP + 4));
    return s;
}

// The flattened position of a lane's group, its row and position, and its row of logits (a
// group at or past `q_end` is not live).
template <int LP, typename IO>
__device__ __forceinline__ const IO* grouped_row(const RouteArgs& a, int q0, int q_end, bool& live,
                                                 int& b, int& p) {
    const int g = lane_id() / LP;
    live = q0 + g < q_end;
    // q0's row and position once (uniform), then the group's: at most G - 1 <= 3 positions on,
    // each wrap into the next row
    const int b0 = uniform(q0 / a.P);
    int pg = uniform(q0 - b0 * a.P) + g, bg = b0;
#pragma unroll
    for (int w = 1; w < kWave / LP; ++w) {
        const bool wrap = pg >= a.P;
        pg = wrap ? pg - a.P : pg;
        bg = wrap ? bg + 1 : bg;
    }
    b = live ? bg : 0;
    p = live ? pg : 0;
    return static_cast<const IO*>(a.logits) + b * a.l_row + p * a.l_pos;
}

// A lane's logits for decide_grouped_from (its group's position q0 + g, cells gl CPL ..).
template <int LP, int CPL, typename IO>
__device__ __forceinline__ void load_grouped(const RouteArgs& a, int q0, int q_end, IO (&raw)[CPL]) {
    bool live;
    int b, p;
    const IO* logits = grouped_row<LP, IO>(a, q0, q_end, live, b, p);
    load_cells<CPL, IO>(a, logits, lane_id() % LP, raw);
}

// G positions q0 .. q0 + G - 1 of the flattened [B, P] window (positions at or past q_end are
// skipped), the lane's logits in `raw`; returns the mask of groups whose position
// decide_select must decide (more candidates than lanes), uniform over the wavefront. With
// a.box, every slot's word goes out as in finish_select, with `stamp`.
template <int LP, int CPL, typename IO, typename IDX>
__device__ uint32_t decide_grouped_from(const RouteArgs& a, int q0, int q_end, const IO (&raw)[CPL],
                                        const GroupedScratch& sm, uint64_t stamp = 0) {
    static_assert(LP == 16 || LP == 32 || LP == 64, "LP");
    static_assert(CPL == 1 || CPL == 2 || CPL == 4 || CPL == 8 || CPL == 16, "CPL");
    constexpr int G = kWave / LP;
    const int lane = lane_id();
    const int g = lane / LP, gl = lane % LP;
    const int N = a.N, K = a.K, R = a.reserved;
    bool live;
    int b, p;
    grouped_row<LP, IO>(a, q0, q_end, live, b, p);
    const bool scale_cost = a.lambda > 0.0f;
    const float cost0 = a.cost[0];
    const float lc = scale_cost ? mul_rn(a.lambda, cost0) : 0.0f;
    float* const sc_lds = sm.sc;
    uint4* const cand = sm.cand;
    uint64_t* const ord = sm.ord;
    uint4* const tab = sm.tab;

    // 1. scores, keys (reserved cells at +inf, cells past N at 0), and the threshold
    uint32_t key[CPL];
    uint32_t hb = 0u;
    if (N == LP * CPL && R == 0 && !scale_cost) {  // uniform: every lane full, the score the logit
        const uint32_t in = 0u - static_cast<uint32_t>(live);
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
            const float s = to_f32(raw[i]);
            sc_lds[i * kWave + lane] = s;
            key[i] = score_key(s) & in;
            hb = umax(hb, key[i]);
        }
    } else {
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
            const int n = gl * CPL + i;
            const float v = to_f32(raw[i]);
            const float s = scale_cost ? sub_rn(v, lc) : v;
            sc_lds[i * kWave + lane] = s;
            const uint32_t in = 0u - static_cast<uint32_t>(live && n < N);
            const uint32_t rsv = 0u - static_cast<uint32_t>(n < R);
            key[i] = ((score_key(s) & ~rsv) | (kKeyPosInf & rsv)) & in;
            hb = umax(hb, key[i]);
        }
    }
    const int Kc = K < N ? K + 1 : K;
    uint32_t L = 0u;
    if (Kc <= LP) {
        const uint32_t sorted = group_sort_desc<LP>(hb, gl, lane);
        L = group_reduce_u32<LP>(gl >= Kc - 1 ? sorted : 0u, [](uint32_t x, uint32_t y) { return x > y ? x : y; });
    }
    L = L > 0u ? L : 1u;  // too few lanes for Kc: every real key

    // 2. the candidates into the group's list (their order words alongside), the largest key
    // below L
    uint32_t m = 0u, below = 0u;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
        const bool c = key[i] >= L;
        m |= c ? 1u << i : 0u;
        below = umax(below, c ? 0u : key[i]);
    }
    const uint32_t cnt = static_cast<uint32_t>(__popc(m));
    const uint32_t incl = group_scan_u32<LP>(cnt);
    const uint32_t C = group_reduce_u32<LP>(incl, [](uint32_t x, uint32_t y) { return x > y ? x : y; });
    const bool fits = live && C <= uint32_t(LP);
    uint32_t at = incl - cnt;
    __builtin_amdgcn_wave_barrier();  // the scores' writes before their reads
    while (m != 0u) {
        const int i = __builtin_ctz(m);
        m &= m - 1u;
        const float s = sc_lds[i * kWave + lane];
        const uint32_t n = uint32_t(gl * CPL + i);
        const uint32_t k = n < uint32_t(R) ? kKeyPosInf : score_key(s);
        if (fits) {
            cand[g * LP + at] = make_uint4(k, n, __float_as_uint(s), 0u);
            ord[g * (LP + 4) + at] = (uint64_t(k) << 32) | ~n;
        }
        ++at;
    }

    // 3. each candidate's rank: its count of the group's candidates before it in the selection's
    // order (the words past C hold 0, below every candidate)
    const bool is_c = fits && uint32_t(gl) < C;
    if (!is_c) ord[g * (LP + 4) + gl] = 0u;
    if (gl < 4) ord[g * (LP + 4) + LP + gl] = 0u;
    __builtin_amdgcn_wave_barrier();
    const uint4 me = is_c ? cand[g * LP + gl] : make_uint4(0u, 0xffffffffu, 0u, 0u);
    const uint64_t mine = (uint64_t(me.x) << 32) | ~me.y;
    int cmax = 0;  // the longest list of the wavefront's groups that fit
#pragma unroll
    for (int gg = 0; gg < G; ++gg) cmax = max(cmax, readlane(fits ? int(C) : 0, gg * LP));
    int rank = 0;
    const uint64_t* const og = ord + g * (LP + 4);
    for (int j = 0; j < cmax; j = uniform(j + 4)) {
        rank += static_cast<int>(og[j] > mine) + static_cast<int>(og[j + 1] > mine) +
                static_cast<int>(og[j + 2] > mine) + static_cast<int>(og[j + 3] > mine);
    }
    if (is_c && rank < K) tab[g * LP + rank] = me;
    const bool out = is_c && rank >= K;
    const float cs = __uint_as_float(me.z);
    const int32_t pool = max(out ? ford(cs) : ford(-INFINITY),
                             below != 0u ? ford(key_score(below)) : ford(-INFINITY));
    const bool pool_nan = out && cs != cs;

    // 4. the budget (one unit: the running sum a product), the threshold, the outputs
    __builtin_amdgcn_wave_barrier();  // the slot tables' writes before their reads
    const bool is_slot = fits && gl < K;
    const uint4 e = is_slot ? tab[g * LP + gl] : make_uint4(0u, 0u, 0u, 0u);
    const int my_cell = static_cast<int>(e.y);
    const float my_score = __uint_as_float(e.z);
    const float ps = add_rn(a.overhead, cost0);
    const float cumulative = add_rn(a.shared, static_cast<float>(static_cast<double>(ps) * (gl + 1)));
    const bool ok = is_slot && cumulative <= a.limit;
    const bool in_low = ok && my_cell >= R;
    const float low = group_amin_k<LP>(in_low ? ford(my_score) : ford(INFINITY),
                                       in_low && my_score != my_score, g);
    const bool cut = is_slot && !ok;
    const int32_t hk = max(pool, cut ? ford(my_score) : ford(-INFINITY));
    const float high = group_amax_k<LP>(hk, pool_nan | (cut && my_score != my_score), g);
    const float th = 0.5f * (low + high);
    if (is_slot) {
        const int64_t o = b * a.o_row + p * a.o_pos + gl;
        store_index<IDX>(a.cells, o, ok ? my_cell : 0);
        store_index<IDX>(a.units, o, 0);
        a.valid[o] = ok ? 1 : 0;
        a.refreshed[o] = 0;
        if (a.slots) a.slots[o] = ok ? my_cell : -1;
        if (a.box)
            __hip_atomic_store(a.box + o, (stamp << 16) | uint64_t(ok ? my_cell + 1 : 0),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (fits && gl == 0) {
        a.theta[b * a.th_row + p * a.th_pos] = th;
        if (a.h_max_zero) a.h_max_zero[static_cast<int64_t>(b) * a.P + p] = 0.0f;
    }
    const uint64_t lead = ballot(gl == 0 && live && !fits);
    uint32_t need = 0u;
#pragma unroll
    for (int gg = 0; gg < G; ++gg) need |= ((lead >> (gg * LP)) & 1u) ? 1u << gg : 0u;
    return need;
}

// decide_grouped_from with the lanes' logits loaded here.
template <int LP, int CPL, typename IO, typename IDX>
__device__ __forceinline__ uint32_t decide_grouped(const RouteArgs& a, int q0, unsigned char* smem) {
    IO raw[CPL];
    const int q_end = a.B * a.P;
    load_grouped<LP, CPL, IO>(a, q0, q_end, raw);
    return decide_grouped_from<LP, CPL, IO, IDX>(a, q0, q_end, raw, grouped_scratch<LP, CPL>(smem));
}

}  // namespace
}  // namespace hsn
