// The router's hard top-k decision on gfx950: one 64-lane wavefront per position.
//
// Restates Router.select(mode="topk") (reference python/hsn/model/router.py:1263-1417: scores
// :1246-1252, _topk :1640-1648, _truncate :1650-1657, _ste_threshold :1771-1786, the refresh
// probes of _post_process :1788-1850) so that the integer outputs are bit-identical to the CPU
// path on the same inputs.
//
// Layout: lane l holds the block of cells n = l*NPL + i (i < NPL), so a position's logits are one
// contiguous read per wavefront and, among equal keys, the lowest lane holds the smallest cell.
// The K winners are found by K rounds of a wavefront argmax over a total-order key (descending
// score, ties by ascending index, NaN above +inf, -0 equal to +0, reserved cells at +inf): a DPP
// max of the lanes' bests, the first lane holding it by ballot, and that lane's rescan. Without probes the positions are independent (the logits are inputs), so the
// whole window is one launch with a wavefront per (row, position); with probes the ages evolve
// with the decisions and one wavefront walks a row's positions in order, its ages in VGPRs.
#include "route.cuh"

#include <type_traits>

namespace hsn {
namespace {

// The decision of one position. `ages` (probes only) are this lane's cells' ages on entry and
// are ticked in place on exit when `tick` is set (the window form walks a row).
template <int NPL, typename IO, typename IDX>
__device__ void decide(const RouteArgs& a, int b, int p, int64_t (&ages)[NPL], bool tick) {
    const int lane = lane_id();
    const int N = a.N, M = a.M, K = a.K, R = a.reserved;
    const IO* logits = static_cast<const IO*>(a.logits) + b * a.l_row + p * a.l_pos;
    const bool scale_cost = a.lambda > 0.0f;

    // The cost table in lanes (lane j holds cost[j], j < M <= 64), loaded with the logits so
    // the position waits for memory once: cost[u] for a lane's own u is a shuffle, called with
    // every lane active.
    const float cost_lane = lane < M ? a.cost[lane] : 0.0f;
    auto cost_of = [&](int u) __attribute__((always_inline)) -> float {
        return M <= kWave ? __shfl(cost_lane, u, kWave) : a.cost[u];
    };

    // scores, units and sort keys of this lane's cells
    float sc[NPL];
    int unit[NPL];
    uint32_t key[NPL];
    int slot_of[NPL];  // 1 + the scored slot that took the cell, 0 if none
    if (M == 1) {  // one unit: every cell's logit read at once (cells past N read cell N-1)
        IO raw[NPL];
#pragma unroll
        for (int i = 0; i < NPL; ++i) {
            const int n = min(lane * NPL + i, N - 1);
            raw[i] = logits[static_cast<int64_t>(n) * a.width];
        }
        const float lc = scale_cost ? mul_rn(a.lambda, a.cost[0]) : 0.0f;
#pragma unroll
        for (int i = 0; i < NPL; ++i) {
            const int n = lane * NPL + i;
            float best = to_f32(raw[i]);
            if (scale_cost) best = sub_rn(best, lc);
            sc[i] = n < N ? best : -INFINITY;
            unit[i] = 0;
            key[i] = n < N ? (n < R ? kKeyPosInf : score_key(best)) : 0u;  // 0: never chosen
            slot_of[i] = 0;
        }
    } else {
#pragma unroll
        for (int i = 0; i < NPL; ++i) {
            const int n = lane * NPL + i;
            sc[i] = -INFINITY;
            unit[i] = 0;
            key[i] = 0u;  // below every real key: never chosen
            slot_of[i] = 0;
            if (n < N) {
                const IO* row = logits + static_cast<int64_t>(n) * a.width;
                float best = to_f32(row[0]);
                if (scale_cost) best = sub_rn(best, mul_rn(a.lambda, a.cost[0]));
                int arg = 0;
                for (int j = 1; j < M; ++j) {
                    float s = to_f32(row[j]);
                    if (scale_cost) s = sub_rn(s, mul_rn(a.lambda, a.cost[j]));
                    // amax / argmax: the first maximiser, a NaN counts as the maximum (first NaN)
                    if (best == best && (s > best || s != s)) {
                        best = s;
                        arg = j;
                    }
                }
                sc[i] = best;
                unit[i] = arg;
                key[i] = n < R ? kKeyPosInf : score_key(best);
            }
        }
    }

    // this lane's best remaining (key, n)
    uint32_t bk = 0u;
    int bn = 0x7fffffff;
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
        if (key[i] > bk) {  // strict: the first (smallest n) of equal keys stays
            bk = key[i];
            bn = lane * NPL + i;
        }
    }

    // K rounds of a wavefront argmax; lane k keeps slot k's cell, score and unit
    int my_cell = 0, my_unit = 0;
    float my_score = 0.0f;
    for (int r = 0; r < K; ++r) {
        uint32_t wk;
        int wn;
        wave_argmax(bk, bn, wk, wn);
        const int wl = wn / NPL, wi = wn % NPL;
        float ws = 0.0f;
        int wu = 0;
        if (lane == wl) {
#pragma unroll
            for (int i = 0; i < NPL; ++i) {
                if (i == wi) {
                    ws = sc[i];
                    wu = unit[i];
                    key[i] = 0u;
                    slot_of[i] = r + 1;
                }
            }
            bk = 0u;
            bn = 0x7fffffff;
#pragma unroll
            for (int i = 0; i < NPL; ++i) {
                if (key[i] > bk) {
                    bk = key[i];
                    bn = lane * NPL + i;
                }
            }
        }
        ws = readlane(ws, wl);
        wu = readlane(wu, wl);
        if (lane == r) {
            my_cell = wn;
            my_score = ws;
            my_unit = (a.fixed_units && r < R) ? r % M : wu;
        }
    }

    // the budget: per-slot cost, prefix sums accumulated in double in slot order and rounded to
    // fp32 per slot (torch's CPU cumsum of fp32), then the shared cost and the limit in fp32
    const bool is_slot = lane < K;
    const float my_cost = cost_of(is_slot ? my_unit : 0);
    const float per_slot = is_slot ? add_rn(a.overhead, my_cost) : 0.0f;
    double acc = 0.0;
    for (int j = 0; j < K; ++j) {
        const float v = readlane(per_slot, j);
        if (j <= lane) acc += static_cast<double>(v);
    }
    const float cumulative = add_rn(a.shared, static_cast<float>(acc));
    const bool ok = is_slot && cumulative <= a.limit;
    const uint64_t vmask = ballot(ok);
    const int n_valid = __popcll(vmask);

    // the threshold of the scored decision: lowest selected (scored slots only) and highest
    // unselected score, NaN-propagating
    float low = (ok && my_cell >= R) ? my_score : INFINITY;
    low = wave_nan_min(low);
    float high = -INFINITY;
    int n_stale = 0;
    bool stale[NPL];
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
        const int n = lane * NPL + i;
        const bool sel = slot_of[i] > 0 && ((vmask >> (slot_of[i] - 1)) & 1ull);
        if (n < N && !sel) high = nan_max(high, sc[i]);
        stale[i] = a.probes && n < N && !sel && ages[i] > static_cast<int64_t>(a.age_max);
        n_stale += stale[i] ? 1 : 0;
    }
    high = wave_nan_max(high);
    const float th = 0.5f * (low + high);

    int out_cell = ok ? my_cell : 0;
    int out_unit = ok ? my_unit : 0;
    bool out_refreshed = false;
    int probe_of[NPL];
#pragma unroll
    for (int i = 0; i < NPL; ++i) probe_of[i] = 0;
    bool over = true;  // no probes taken yet: the scored selection stands

    if (a.probes) {
        n_stale = wave_sum(n_stale);
        const int scored_slots = n_valid > R ? n_valid - R : 0;
        const int n_force = n_stale < scored_slots ? n_stale : scored_slots;
        if (n_force > 0) {
            // the stalest first (age as fp32, descending), equal ages in index order
            uint32_t pk[NPL];
            uint32_t qk = 0u;
            int qn = 0x7fffffff;
#pragma unroll
            for (int i = 0; i < NPL; ++i) {
                pk[i] = stale[i] ? __float_as_uint(static_cast<float>(ages[i])) + 1u : 0u;
                if (pk[i] > qk) {
                    qk = pk[i];
                    qn = lane * NPL + i;
                }
            }
            int new_cell = out_cell, new_unit = out_unit;
            bool replaced = false;
            for (int j = 0; j < n_force; ++j) {
                uint32_t wk;
                int wn;
                wave_argmax(qk, qn, wk, wn);
                const int wl = wn / NPL, wi = wn % NPL;
                int wu = 0;
                if (lane == wl) {
#pragma unroll
                    for (int i = 0; i < NPL; ++i) {
                        if (i == wi) {
                            wu = unit[i];
                            pk[i] = 0u;
                            probe_of[i] = j + 1;
                        }
                    }
                    qk = 0u;
                    qn = 0x7fffffff;
#pragma unroll
                    for (int i = 0; i < NPL; ++i) {
                        if (pk[i] > qk) {
                            qk = pk[i];
                            qn = lane * NPL + i;
                        }
                    }
                }
                wu = readlane(wu, wl);
                if (lane == n_valid - 1 - j) {
                    new_cell = wn;
                    new_unit = wu;
                    replaced = true;
                }
            }
            // the budget guarantee: over the limit after the probes, keep the scored selection
            const float new_cost = cost_of(ok ? new_unit : 0);
            const float cost_k = ok ? add_rn(a.overhead, new_cost) : 0.0f;
            float spent = 0.0f;
            for (int j = 0; j < K; ++j) spent = add_rn(spent, readlane(cost_k, j));
            over = add_rn(a.shared, spent) > a.limit;
            if (!over) {
                out_cell = new_cell;
                out_unit = new_unit;
                out_refreshed = replaced;
            }
        }
    }

    if (is_slot) {
        const int64_t o = b * a.o_row + p * a.o_pos + lane;
        store_index<IDX>(a.cells, o, out_cell);
        store_index<IDX>(a.units, o, out_unit);
        a.valid[o] = ok ? 1 : 0;
        a.refreshed[o] = out_refreshed ? 1 : 0;
        if (a.slots) a.slots[o] = ok ? out_cell : -1;
    }
    if (lane == 0) {
        a.theta[b * a.th_row + p * a.th_pos] = th;
        if (a.h_max_zero) a.h_max_zero[static_cast<int64_t>(b) * a.P + p] = 0.0f;
    }

    if (tick) {
        // CellGraphState.tick: the final selection's cells restart at 0, every other cell ages
        const uint64_t refreshed_slots = ballot(is_slot && out_refreshed);
#pragma unroll
        for (int i = 0; i < NPL; ++i) {
            bool sel = slot_of[i] > 0 && ((vmask >> (slot_of[i] - 1)) & 1ull);
            if (!over) {
                if (sel && ((refreshed_slots >> (slot_of[i] - 1)) & 1ull)) sel = false;
                if (probe_of[i] > 0) sel = true;
            }
            ages[i] = sel ? 0 : ages[i] + 1;
        }
    }
}

// The decision of one position without probes, for NPL <= 4: the same selection as `decide`,
// with each lane's cells sorted once. A lane's entries (key, cell, score, unit) are put in the
// selection's order (key descending, cell ascending: a strict total order, so a five-comparator
// network sorts them exactly); the head is in registers and the rest in LDS. A round's winner
// is the lane whose head is the wavefront's largest (the first such lane: the smaller cell), and
// it only writes its head to the round's slot and reads its next entry, instead of rescanning
// its cells. kOne (one unit, M = 1): every slot costs the same, so the budget's running sum is
// a product, and a contiguous logits row is one vector load per lane.
template <int NPL, bool kOne, typename IO, typename IDX>
__device__ void decide_sorted(const RouteArgs& a, int b, int p, uint4* ent, uint4* tab) {
    static_assert(NPL == 1 || NPL == 2 || NPL == 4, "NPL");
    const int lane = lane_id();
    const int N = a.N, M = a.M, K = a.K, R = a.reserved;
    const IO* logits = static_cast<const IO*>(a.logits) + b * a.l_row + p * a.l_pos;
    const bool scale_cost = a.lambda > 0.0f;

    float sc[NPL];
    int unit[NPL], nn[NPL];
    uint32_t key[NPL];
    // kOne: the one unit's cost, loaded with the logits so the position waits for memory once
    const float cost0 = kOne ? a.cost[0] : 0.0f;
    if constexpr (kOne) {
        IO raw[NPL];
        constexpr uint32_t kRun = NPL * sizeof(IO);
        const bool vec = a.width == 1 && N % NPL == 0 &&
                         (reinterpret_cast<uintptr_t>(logits) & (kRun - 1)) == 0;
        if (vec) {  // lanes past the row read zeros (kOob); their cells are masked below
            const rsrc_t r = make_rsrc(logits, uint32_t(N) * sizeof(IO));
            load_run<NPL, IO>(raw, r, lane * NPL < N ? uint32_t(lane) * kRun : kOob);
        } else {
#pragma unroll
            for (int i = 0; i < NPL; ++i)
                raw[i] = logits[int64_t(min(lane * NPL + i, N - 1)) * a.width];
        }
        const float lc = scale_cost ? mul_rn(a.lambda, cost0) : 0.0f;
#pragma unroll
        for (int i = 0; i < NPL; ++i) {
            const int n = lane * NPL + i;
            float best = to_f32(raw[i]);
            if (scale_cost) best = sub_rn(best, lc);
            // masks, not a conditional: the compiler would branch around the key otherwise
            const uint32_t in = 0u - static_cast<uint32_t>(n < N);
            const uint32_t rsv = 0u - static_cast<uint32_t>(n < R);
            sc[i] = n < N ? best : -INFINITY;
            unit[i] = 0;
            key[i] = ((score_key(best) & ~rsv) | (kKeyPosInf & rsv)) & in;
            nn[i] = n;
        }
    } else {
#pragma unroll
        for (int i = 0; i < NPL; ++i) {
            const int n = lane * NPL + i;
            sc[i] = -INFINITY;
            unit[i] = 0;
            key[i] = 0u;
            nn[i] = n;
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
                sc[i] = best;
                unit[i] = arg;
                key[i] = n < R ? kKeyPosInf : score_key(best);
            }
        }
    }
    // the earlier entry first; bitwise, not short-circuit: compares and selects, no branch. Where
    // the entry at i is known to hold the smaller cell (kTie false), equal keys keep their places.
    auto ce = [&](int i, int j, auto tie_c) __attribute__((always_inline)) {
        constexpr bool kTie = decltype(tie_c)::value;
        bool sw = key[i] < key[j];
        if constexpr (kTie) sw = sw | ((key[i] == key[j]) & (nn[i] > nn[j]));
        const uint32_t k = key[i];
        const int c = nn[i], u = unit[i];
        const float v = sc[i];
        key[i] = sw ? key[j] : k;
        key[j] = sw ? k : key[j];
        nn[i] = sw ? nn[j] : c;
        nn[j] = sw ? c : nn[j];
        if constexpr (!kOne) {
            unit[i] = sw ? unit[j] : u;
            unit[j] = sw ? u : unit[j];
        }
        sc[i] = sw ? sc[j] : v;
        sc[j] = sw ? v : sc[j];
    };
    // Cells n = lane*NPL + i start in order of i. The first four comparators of the network
    // compare an entry from {0, 1} with one from {2, 3} (or 0 with 1, 2 with 3), the smaller
    // cell always at the lower place; only the last one can see either order.
    if constexpr (NPL == 2) ce(0, 1, std::false_type{});
    if constexpr (NPL == 4) {
        ce(0, 1, std::false_type{});
        ce(2, 3, std::false_type{});
        ce(0, 2, std::false_type{});
        ce(1, 3, std::false_type{});
        ce(1, 2, std::true_type{});
    }
    // entries 1 .. NPL-1 at mine[0 .. NPL-2], an empty entry (key 0: never the largest) last
    uint4* const mine = ent + lane * NPL;
#pragma unroll
    for (int i = 1; i < NPL; ++i)
        mine[i - 1] = make_uint4(key[i], uint32_t(nn[i]), __float_as_uint(sc[i]), uint32_t(unit[i]));
    mine[NPL - 1] = make_uint4(0u, 0u, 0u, 0u);

    // K rounds: the wavefront's largest head, its first lane; the winner moves to its next entry
    uint4 head = make_uint4(key[0], uint32_t(nn[0]), __float_as_uint(sc[0]), uint32_t(unit[0]));
    int ptr = 0;            // this lane's entries given to slots
    uint32_t srec = 0u;     // per entry (8 bits each): 1 + the slot that took it, 0 if none
    for (int r = 0; r < K; r = uniform(r + 1)) {
        const uint32_t wk = wave_reduce_u32(head.x, [](uint32_t x, uint32_t y) { return x > y ? x : y; }, 0u);
        const int src = __builtin_ctzll(ballot(head.x == wk));
        if (lane == src) {
            tab[r] = head;
            srec |= uint32_t(r + 1) << (8 * ptr);
            ++ptr;
            head = mine[min(ptr, NPL) - 1];
        }
    }
    __builtin_amdgcn_wave_barrier();  // the slot table's writes before its reads (one wavefront)
    const bool is_slot = lane < K;
    const uint4 e = is_slot ? tab[lane] : make_uint4(0u, 0u, 0u, 0u);
    const int my_cell = static_cast<int>(e.y);
    const float my_score = __uint_as_float(e.z);

    // the budget (as decide): the running sum of the slots' costs in double, as the CPU cumsum
    int my_unit = 0;
    float cumulative;
    if constexpr (kOne) {
        // every slot costs ps: the sum over slots 0..lane is (lane + 1) * ps, exact in double
        // (a float times at most 64), as the running sum is
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
    const uint64_t vmask = ballot(ok);

    // the threshold (as decide)
    const bool in_low = ok && my_cell >= R;
    const float low = wave_amin_k(in_low ? ford(my_score) : ford(INFINITY), in_low && my_score != my_score);
    const uint64_t full = K >= kWave ? ~0ull : (1ull << K) - 1ull;
    const bool all_valid = vmask == full;  // then an entry is selected when it was taken
    int32_t hk = ford(-INFINITY);
    bool high_nan = false;
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
        bool sel;
        if (all_valid) {
            sel = i < ptr;
        } else {
            const uint32_t so = (srec >> (8 * i)) & 0xffu;
            sel = so > 0u && ((vmask >> (so - 1u)) & 1ull);
        }
        const bool out = (nn[i] < N) & !sel;
        hk = max(hk, out ? ford(sc[i]) : ford(-INFINITY));
        high_nan = high_nan | (out & (sc[i] != sc[i]));
    }
    const float high = wave_amax_k(hk, high_nan);
    const float th = 0.5f * (low + high);

    if (is_slot) {
        const int64_t o = b * a.o_row + p * a.o_pos + lane;
        store_index<IDX>(a.cells, o, ok ? my_cell : 0);
        store_index<IDX>(a.units, o, ok ? my_unit : 0);
        a.valid[o] = ok ? 1 : 0;
        a.refreshed[o] = 0;
        if (a.slots) a.slots[o] = ok ? my_cell : -1;
    }
    if (lane == 0) {
        a.theta[b * a.th_row + p * a.th_pos] = th;
        if (a.h_max_zero) a.h_max_zero[static_cast<int64_t>(b) * a.P + p] = 0.0f;
    }
}


// The decision of one position without probes for one unit and wide rows (NPL >= 16): the
// selection of decide_select with every key recomputed from the lane's packed logits where a pass
// needs it instead of held in registers (a key and a logit per cell would take two registers per
// cell: at N = 4096 more than one wavefront's share of a SIMD), and the heavy-ties path's taken
// cells in a bit mask. kUni: every lane full, no reserved cells, no cost term (the key of a cell
// is its logit's).
template <int NPL, bool kUni, typename IO, typename IDX>
__device__ void decide_lean_body(const RouteArgs& a, int b, int p, uint4* cand, uint4* tab,
                                 uint64_t* ord) {
    static_assert(NPL >= 16 && NPL <= 64, "NPL");
    constexpr int kW = NPL * static_cast<int>(sizeof(IO)) / 4;  // packed words per lane
    static_assert(kW % 4 == 0, "whole 16-byte loads");
    const int lane = lane_id();
    const int N = a.N, K = a.K, R = a.reserved;
    const IO* logits = static_cast<const IO*>(a.logits) + b * a.l_row + p * a.l_pos;
    const bool scale_cost = a.lambda > 0.0f;
    const float cost0 = a.cost[0];
    const float lc = scale_cost ? mul_rn(a.lambda, cost0) : 0.0f;
    const int n0 = lane * NPL;
    uint32_t w[kW];
    {
        constexpr uint32_t kRun = NPL * sizeof(IO);
        const bool vec = a.width == 1 && N % NPL == 0 &&
                         (reinterpret_cast<uintptr_t>(logits) & 15) == 0;
        if (vec) {  // lanes past the row read zeros (kOob); their cells are masked below
            const rsrc_t r = make_rsrc(logits, uint32_t(N) * sizeof(IO));
            const uint32_t vo = n0 < N ? uint32_t(lane) * kRun : kOob;
#pragma unroll
            for (int c = 0; c < kW / 4; ++c) {
                const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, vo + 16u * c, 0, 0);
                __builtin_memcpy(&w[4 * c], &v, 16);
            }
        } else {
            IO raw[NPL];
#pragma unroll
            for (int i = 0; i < NPL; ++i) raw[i] = logits[int64_t(min(n0 + i, N - 1)) * a.width];
            __builtin_memcpy(w, raw, sizeof(raw));
        }
    }
    auto val = [&](int i) __attribute__((always_inline)) -> float {
        if constexpr (sizeof(IO) == 4) return __uint_as_float(w[i]);
        else return __uint_as_float((i & 1) ? (w[i >> 1] & 0xffff0000u) : (w[i >> 1] << 16));
    };
    auto score = [&](int i) __attribute__((always_inline)) -> float {
        const float v = val(i);
        return scale_cost ? sub_rn(v, lc) : v;
    };
    const int n_in = min(max(N - n0, 0), NPL), n_rsv = min(max(R - n0, 0), NPL);
    auto key = [&](int i) __attribute__((always_inline)) -> uint32_t {
        if constexpr (kUni) {
            return score_key(val(i));
        } else {
            const uint32_t in = 0u - static_cast<uint32_t>(i < n_in);
            const uint32_t rsv = 0u - static_cast<uint32_t>(i < n_rsv);
            return ((score_key(score(i)) & ~rsv) | (kKeyPosInf & rsv)) & in;
        }
    };

    // the words may change at each block of 16 cells (an empty asm): the compiler computes a
    // block's keys within the block instead of all of them up front
    auto fence = [&](int i) __attribute__((always_inline)) {
        if ((i & 15) == 0) {
#pragma unroll
            for (int c = 0; c < kW; ++c) asm volatile("" : "+v"(w[c]));
        }
    };
    // 1. the threshold prefix from the lanes' maxima
    uint32_t hb = 0u;
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
        fence(i);
        hb = umax(hb, key(i));
    }
    const int Kc = K < N ? K + 1 : K;
    const uint32_t top = hb >> 16;
    uint32_t pfx = 0u;
#pragma unroll
    for (int bit = 15; bit >= 0; --bit) {
        const uint32_t c = pfx | (1u << bit);
        pfx = __popcll(ballot(top >= c)) >= Kc ? c : pfx;
    }
    const uint32_t L = pfx > 0u ? pfx << 16 : 1u;  // 1: every real key (a cell past N has key 0)

    // 2. the candidates into LDS, and the largest key below L (the keys computed again)
    uint32_t below = 0u;
    int C = 0;
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
        fence(i);
        const uint32_t k = key(i);
        const bool c = k >= L;
        below = umax(below, c ? 0u : k);
        const uint64_t m = ballot(c);
        if (m != 0u) {  // uniform
            const int at = C + lanes_below(m);
            if (c && at < kWave) {
                const uint32_t n = uint32_t(n0 + i);
                cand[at] = make_uint4(k, n, __float_as_uint(score(i)), 0u);
                ord[at] = (uint64_t(k) << 32) | ~n;  // the selection's order as one integer
            }
            C += __popcll(m);
        }
    }
    int32_t pool;
    bool pool_nan;
    if (C <= kWave) {
        __builtin_amdgcn_wave_barrier();  // the candidates' writes before their reads
        const bool is_c = lane < C;
        const uint4 me = is_c ? cand[lane] : make_uint4(0u, 0xffffffffu, 0u, 0u);
        // 3. each candidate's place in the selection's order (as decide_select)
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
        // Heavy ties: K rounds of a wavefront argmax (as decide_select), the lane's best among
        // its cells not yet taken found by a pass over its keys
        uint64_t taken = 0ull;
        uint32_t bk = 0u;
        int bi = 0;
        float bs = 0.0f;
        auto best = [&]() __attribute__((always_inline)) {
            bk = 0u;
            bi = 0;
            bs = 0.0f;
#pragma unroll
            for (int i = 0; i < NPL; ++i) {
                fence(i);
                const uint32_t k = ((taken >> i) & 1ull) ? 0u : key(i);
                const bool gt = k > bk;
                bk = gt ? k : bk;
                bi = gt ? i : bi;
                bs = gt ? score(i) : bs;
            }
        };
        best();
        for (int r = 0; r < K; r = uniform(r + 1)) {
            const uint32_t wk = wave_reduce_u32(bk, [](uint32_t x, uint32_t y) { return x > y ? x : y; }, 0u);
            const int src = __builtin_ctzll(ballot(bk == wk));
            if (lane == src) {
                tab[r] = make_uint4(bk, uint32_t(n0 + bi), __float_as_uint(bs), 0u);
                taken |= 1ull << bi;
                best();
            }
        }
        pool = ford(-INFINITY);
        pool_nan = false;
#pragma unroll
        for (int i = 0; i < NPL; ++i) {  // every real cell still in the pool
            fence(i);
            const bool out = i < n_in && !((taken >> i) & 1ull);
            const float si = score(i);
            pool = max(pool, out ? ford(si) : ford(-INFINITY));
            pool_nan = pool_nan | (out & (si != si));
        }
    }
    finish_select<true, IDX>(a, b, p, tab, pool, pool_nan, cost0);
}

template <int NPL, typename IO, typename IDX>
__device__ __forceinline__ void decide_lean(const RouteArgs& a, int b, int p, uint4* cand,
                                            uint4* tab, uint64_t* ord) {
    if (a.N == kWave * NPL && a.reserved == 0 && !(a.lambda > 0.0f))
        decide_lean_body<NPL, true, IO, IDX>(a, b, p, cand, tab, ord);
    else
        decide_lean_body<NPL, false, IO, IDX>(a, b, p, cand, tab, ord);
}

// Whole window without probes, one unit, N <= 1024 and K < LP: G = 64 / LP positions a
// wavefront (decide_grouped), four wavefronts a workgroup; a group with more candidates than
// lanes is decided afterwards by the wavefront's one-position selection (NPLF cells a lane).
template <int LP, int CPL, int NPLF, typename IO, typename IDX>
__global__ __launch_bounds__(256) void route_grouped(RouteArgs a) {
    constexpr int G = kWave / LP;
    constexpr int kBytes = grouped_scratch_bytes<LP, CPL>();
    __shared__ __align__(16) unsigned char smem[4][kBytes];
    const int wv = uniform(threadIdx.x / kWave);
    const int q0 = (blockIdx.x * 4 + wv) * G;
    if (q0 >= a.B * a.P) return;
    unsigned char* const sw = smem[wv];
    uint32_t need = decide_grouped<LP, CPL, IO, IDX>(a, q0, sw);
    if (need != 0u) {  // its scratch is the groups' lists, order words and slot tables
        __builtin_amdgcn_wave_barrier();
        const GroupedScratch sm = grouped_scratch<LP, CPL>(sw);
        while (need != 0u) {
            const int g = __builtin_ctz(need);
            need &= need - 1u;
            const int q = q0 + g;
            if constexpr (NPLF >= 16) decide_lean<NPLF, IO, IDX>(a, q / a.P, q % a.P, sm.cand, sm.tab, sm.ord);
            else decide_select<NPLF, true, IO, IDX>(a, q / a.P, q % a.P, sm.cand, sm.tab, sm.ord);
            __builtin_amdgcn_wave_barrier();
        }
    }
}

// Whole window without probes: a wavefront per (row, position), four per workgroup; kOne
// (one unit) is a kernel of its own, so its register budget is not the multi-unit one.
template <int NPL, bool kOne, typename IO, typename IDX>
__global__ __launch_bounds__(256) void route_parallel(RouteArgs a) {
    const int wv = uniform(threadIdx.x / kWave);  // uniform: the position's offsets stay scalar
    const int p = blockIdx.x * (blockDim.x / kWave) + wv;
    const int b = blockIdx.y;
    if (p >= a.P) return;
    __shared__ uint4 cand[4][kWave];
    __shared__ uint4 tab[4][kWave];
    __shared__ uint64_t ord[4][kWave + 4];
    if constexpr (kOne && NPL >= 16)
        decide_lean<NPL, IO, IDX>(a, b, p, cand[wv], tab[wv], ord[wv]);
    else
        decide_select<NPL, kOne, IO, IDX>(a, b, p, cand[wv], tab[wv], ord[wv]);
}

// Whole window without probes, one unit, a workgroup per (row, position) for rows too wide for a
// wavefront's registers (N > 1024): 256 threads of CPT consecutive cells each (thread t holds
// cells t*CPT ..), the selection of decide_select across the workgroup:
//  1. every thread's largest key into LDS; L, the largest 16-bit key prefix that at least Kc of
//     the 256 thread maxima reach (each wavefront computes it from the same 256 values);
//  2. each wavefront compacts its cells with key >= L into its own LDS segment;
//  3. wavefront 0 ranks the candidates (at most 64 in all) and finishes as decide_select; more
//     than 64 (heavy ties) take K rounds of a workgroup argmax (the largest key, the lowest cell:
//     the first wavefront, lane and cell holding it).
template <int CPT, typename IO, typename IDX>
__global__ __launch_bounds__(256) void route_block(RouteArgs a) {
    static_assert(CPT >= 1 && CPT <= 16, "CPT");
    constexpr int kT = 256, kWv = kT / kWave;
    constexpr int kW = (CPT * static_cast<int>(sizeof(IO)) + 3) / 4;  // packed words per thread
    __shared__ uint32_t smax[kT];
    __shared__ uint4 cand[kWv][kWave];
    __shared__ uint64_t ord[kWave + 4];
    __shared__ uint4 tab[kWave];
    __shared__ int wcnt[kWv];
    __shared__ uint32_t wbelow[kWv];
    __shared__ uint4 wbest[kWv];
    __shared__ int32_t wpool[kWv];
    __shared__ int wnan[kWv];
    const int p = blockIdx.x, b = blockIdx.y;
    const int tid = threadIdx.x, lane = lane_id(), wv = uniform(tid / kWave);
    const int N = a.N, K = a.K, R = a.reserved;
    const IO* logits = static_cast<const IO*>(a.logits) + b * a.l_row + p * a.l_pos;
    const bool scale_cost = a.lambda > 0.0f;
    const float cost0 = a.cost[0];
    const float lc = scale_cost ? mul_rn(a.lambda, cost0) : 0.0f;
    const int n0 = tid * CPT;
    uint32_t w[kW];
    {
        constexpr uint32_t kRun = CPT * sizeof(IO);
        const bool vec = kRun % 16 == 0 && a.width == 1 && N % CPT == 0 &&
                         (reinterpret_cast<uintptr_t>(logits) & 15) == 0;
        if (vec) {  // threads past the row read zeros (kOob); their cells are masked below
            const rsrc_t r = make_rsrc(logits, uint32_t(N) * sizeof(IO));
            const uint32_t vo = n0 < N ? uint32_t(tid) * kRun : kOob;
#pragma unroll
            for (int c = 0; c < kW / 4; ++c) {
                const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, vo + 16u * c, 0, 0);
                __builtin_memcpy(&w[4 * c], &v, 16);
            }
        } else {
            IO raw[kW * 4 / sizeof(IO)] = {};
#pragma unroll
            for (int i = 0; i < CPT; ++i) raw[i] = logits[int64_t(min(n0 + i, N - 1)) * a.width];
            __builtin_memcpy(w, raw, kW * 4);
        }
    }
    auto score = [&](int i) __attribute__((always_inline)) -> float {
        float v;
        if constexpr (sizeof(IO) == 4) v = __uint_as_float(w[i]);
        else v = __uint_as_float((i & 1) ? (w[i >> 1] & 0xffff0000u) : (w[i >> 1] << 16));
        return scale_cost ? sub_rn(v, lc) : v;
    };
    const int n_in = min(max(N - n0, 0), CPT), n_rsv = min(max(R - n0, 0), CPT);
    uint32_t key[CPT];
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
        const uint32_t in = 0u - static_cast<uint32_t>(i < n_in);
        const uint32_t rsv = 0u - static_cast<uint32_t>(i < n_rsv);
        key[i] = ((score_key(score(i)) & ~rsv) | (kKeyPosInf & rsv)) & in;
    }

    // 1. the threshold prefix from the threads' maxima
    uint32_t hb = 0u;
#pragma unroll
    for (int i = 0; i < CPT; ++i) hb = umax(hb, key[i]);
    smax[tid] = hb >> 16;
    __syncthreads();
    const int Kc = K < N ? K + 1 : K;
    uint32_t tops[kWv];
#pragma unroll
    for (int j = 0; j < kWv; ++j) tops[j] = smax[lane + kWave * j];
    uint32_t pfx = 0u;
#pragma unroll
    for (int bit = 15; bit >= 0; --bit) {
        const uint32_t c = pfx | (1u << bit);
        int cnt = 0;
#pragma unroll
        for (int j = 0; j < kWv; ++j) cnt += __popcll(ballot(tops[j] >= c));
        pfx = cnt >= Kc ? c : pfx;
    }
    const uint32_t L = pfx > 0u ? pfx << 16 : 1u;

    // 2. each wavefront's candidates into its LDS segment, and its largest key below L
    uint32_t below = 0u;
    int C = 0;
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
        const bool c = key[i] >= L;
        below = umax(below, c ? 0u : key[i]);
        const uint64_t m = ballot(c);
        if (m != 0u) {  // uniform
            const int at = C + lanes_below(m);
            if (c && at < kWave)
                cand[wv][at] = make_uint4(key[i], uint32_t(n0 + i), __float_as_uint(score(i)), 0u);
            C += __popcll(m);
        }
    }
    below = wave_reduce_u32(below, [](uint32_t x, uint32_t y) { return x > y ? x : y; }, 0u);
    if (lane == 0) {
        wcnt[wv] = C;
        wbelow[wv] = below;
    }
    __syncthreads();
    int Ct = 0;
    uint32_t bel = 0u;
#pragma unroll
    for (int j = 0; j < kWv; ++j) {
        Ct += wcnt[j];
        bel = umax(bel, wbelow[j]);
    }
    if (Ct <= kWave) {
        if (wv != 0) return;
        // 3. wavefront 0: candidate `lane` from the segments, its place in the selection's order
        int seg = 0, base = 0, off = 0;  // the segment holding candidate `lane`, its start
#pragma unroll
        for (int j = 0; j + 1 < kWv; ++j) {
            off += wcnt[j];  // the start of segment j + 1 (the starts never decrease)
            const bool past = lane >= off;
            seg = past ? j + 1 : seg;
            base = past ? off : base;
        }
        const bool is_c = lane < Ct;
        const uint4 me = is_c ? cand[seg][lane - base] : make_uint4(0u, 0xffffffffu, 0u, 0u);
        const uint64_t mine = (uint64_t(me.x) << 32) | ~me.y;
        ord[lane] = is_c ? mine : 0u;
        __builtin_amdgcn_wave_barrier();
        int rank = 0;
        for (int j = 0; j < Ct; j = uniform(j + 4)) {
            const uint64_t o0 = ord[j], o1 = ord[j + 1], o2 = ord[j + 2], o3 = ord[j + 3];
            rank += static_cast<int>(o0 > mine) + static_cast<int>(o1 > mine) +
                    static_cast<int>(o2 > mine) + static_cast<int>(o3 > mine);
        }
        if (is_c && rank < K) tab[rank] = me;
        const bool out = is_c && rank >= K;
        const float cs = __uint_as_float(me.z);
        const int32_t pool = max(out ? ford(cs) : ford(-INFINITY),
                                 bel != 0u ? ford(key_score(bel)) : ford(-INFINITY));
        finish_select<true, IDX>(a, b, p, tab, pool, out && cs != cs, cost0);
        return;
    }
    // heavy ties: K rounds of a workgroup argmax, the taken cells in a bit mask
    uint32_t taken = 0u;
    for (int r = 0; r < K; ++r) {
        uint32_t bk = 0u;
        int bi = 0;
        float bs = 0.0f;
#pragma unroll
        for (int i = 0; i < CPT; ++i) {
            const uint32_t k = ((taken >> i) & 1u) ? 0u : key[i];
            const bool gt = k > bk;
            bk = gt ? k : bk;
            bi = gt ? i : bi;
            bs = gt ? score(i) : bs;
        }
        const uint32_t wk = wave_reduce_u32(bk, [](uint32_t x, uint32_t y) { return x > y ? x : y; }, 0u);
        const int src = __builtin_ctzll(ballot(bk == wk));
        if (lane == src) wbest[wv] = make_uint4(wk, uint32_t(n0 + bi), __float_as_uint(bs), 0u);
        __syncthreads();
        int wsel = 0;
        uint32_t kmax = wbest[0].x;
#pragma unroll
        for (int j = 1; j < kWv; ++j) {
            const bool gt = wbest[j].x > kmax;  // equal keys: the earlier wavefront (lower cells)
            kmax = gt ? wbest[j].x : kmax;
            wsel = gt ? j : wsel;
        }
        if (wv == wsel && lane == src) taken |= 1u << bi;
        if (tid == 0) tab[r] = wbest[wsel];
        __syncthreads();
    }
    int32_t pk = ford(-INFINITY);
    bool pn = false;
#pragma unroll
    for (int i = 0; i < CPT; ++i) {  // every real cell still in the pool
        const bool out = i < n_in && !((taken >> i) & 1u);
        const float si = score(i);
        pk = max(pk, out ? ford(si) : ford(-INFINITY));
        pn = pn | (out & (si != si));
    }
    pk = static_cast<int32_t>(wave_reduce_u32(
        static_cast<uint32_t>(pk),
        [](uint32_t x, uint32_t y) { return static_cast<int32_t>(x) > static_cast<int32_t>(y) ? x : y; },
        static_cast<uint32_t>(ford(-INFINITY))));
    const bool wn = ballot(pn) != 0u;
    if (lane == 0) {
        wpool[wv] = pk;
        wnan[wv] = wn ? 1 : 0;
    }
    __syncthreads();
    if (wv != 0) return;
    int32_t pool = wpool[0];
    bool pool_nan = wnan[0] != 0;
#pragma unroll
    for (int j = 1; j < kWv; ++j) {
        pool = max(pool, wpool[j]);
        pool_nan = pool_nan || wnan[j] != 0;
    }
    finish_select<true, IDX>(a, b, p, tab, pool, pool_nan, cost0);
}

// With probes (or the per-position form): one wavefront walks a row's positions in order.
// Window form (a.age0): ages start at age0, a reset at p zeroes them before p reads them, and
// each decision ticks them. Per-position form (a.age): the ages of record a.age_rec, P = 1.
template <int NPL, typename IO, typename IDX>
__global__ __launch_bounds__(64) void route_sequential(RouteArgs a) {
    const int b = blockIdx.x;
    const int lane = lane_id();
    int64_t ages[NPL];
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
        const int n = lane * NPL + i;
        int64_t v = 0;
        if (n < a.N) {
            if (a.age0) v = a.age0[static_cast<int64_t>(b) * a.N + n];
            else if (a.age) v = a.age[b * a.age_row + a.age_rec * a.N + n];
        }
        ages[i] = v;
    }
    for (int p = 0; p < a.P; ++p) {
        if (a.reset && a.reset[static_cast<int64_t>(b) * a.P + p]) {
#pragma unroll
            for (int i = 0; i < NPL; ++i) ages[i] = 0;
        }
        decide<NPL, IO, IDX>(a, b, p, ages, a.P > 1);
    }
}

template <int LP, int CPL, int NPLF, typename IO, typename IDX>
hipError_t launch_grouped(const RouteArgs& a, hipStream_t stream) {
    constexpr int G = kWave / LP;
    const int64_t groups = (int64_t(a.B) * a.P + G - 1) / G;
    hipLaunchKernelGGL((route_grouped<LP, CPL, NPLF, IO, IDX>), dim3(unsigned((groups + 3) / 4)),
                       dim3(256), 0, stream, a);
    return hipGetLastError();
}

template <typename IO, typename IDX>
hipError_t launch_route(const RouteArgs& a, bool sequential, hipStream_t stream) {
    const int npl = (a.N + kWave - 1) / kWave;
    // one unit, N <= 256, K < 32: two positions a wavefront of 32 lanes each. Sixteen lanes of
    // sixteen cells measured slower (about one position in twenty has more candidates than lanes
    // and falls back to the one-position selection, and a quarter of the wavefronts wait for
    // one), and so did one position of 64 lanes above N = 256 (no second position to share the
    // instructions, and the 64-lane sort costs more than the one-position bisection: tbptt's
    // router 20.4 against 17.2 us, bf16's 45.0 against 42.0)
    if (!sequential && a.M == 1 && a.N <= 256 && a.K < 32) {
        const int N = a.N;
        if (N <= 32) return launch_grouped<32, 1, 1, IO, IDX>(a, stream);
        if (N <= 64) return launch_grouped<32, 2, 1, IO, IDX>(a, stream);
        if (N <= 128) return launch_grouped<32, 4, 2, IO, IDX>(a, stream);
        return launch_grouped<32, 8, 4, IO, IDX>(a, stream);
    }
    if (!sequential && a.M == 1 && a.N > 1024) {  // a workgroup per position (N <= 4096)
        hipLaunchKernelGGL((route_block<16, IO, IDX>), dim3(a.P, a.B), dim3(256), 0, stream, a);
        return hipGetLastError();
    }
#define HSN_ROUTE_CASE(V)                                                                      \
    if (npl <= V) {                                                                            \
        if (sequential) {                                                                      \
            hipLaunchKernelGGL((route_sequential<V, IO, IDX>), dim3(a.B), dim3(kWave), 0,      \
                               stream, a);                                                     \
        } else {                                                                               \
            const dim3 grid((a.P + 3) / 4, a.B);                                               \
            if (a.M == 1)                                                                      \
                hipLaunchKernelGGL((route_parallel<V, true, IO, IDX>), grid, dim3(256), 0,     \
                                   stream, a);                                                 \
            else                                                                               \
                hipLaunchKernelGGL((route_parallel<V, false, IO, IDX>), grid, dim3(256), 0,    \
                                   stream, a);                                                 \
        }                                                                                      \
        return hipGetLastError();                                                              \
    }
    HSN_ROUTE_CASE(1)
    HSN_ROUTE_CASE(2)
    HSN_ROUTE_CASE(4)
    HSN_ROUTE_CASE(8)
    HSN_ROUTE_CASE(16)
    HSN_ROUTE_CASE(32)
    HSN_ROUTE_CASE(64)
#undef HSN_ROUTE_CASE
    return hipErrorInvalidValue;
}

hipError_t dispatch_route(const RouteArgs& a, int io_dtype, int index_bits, bool sequential,
                          hipStream_t stream) {
    if (io_dtype == HSN_DTYPE_F32) {
        return index_bits == 64 ? launch_route<float, int64_t>(a, sequential, stream)
                                : launch_route<float, int32_t>(a, sequential, stream);
    }
    return index_bits == 64 ? launch_route<bf16_t, int64_t>(a, sequential, stream)
                            : launch_route<bf16_t, int32_t>(a, sequential, stream);
}

}  // namespace
}  // namespace hsn

#include "abi_util.h"

using namespace hsn;

extern "C" int hsn_win_route(const void* logits, int io_dtype, int64_t width, const float* cost,
                             const int64_t* age0, const uint8_t* reset, void* cells, void* units,
                             int index_bits, uint8_t* valid, float* theta, uint8_t* refreshed,
                             int32_t* slots, float* h_max_zero, int B, int T, int N, int M, int K,
                             int age_max,
                             int probes, float lambda_cost, float cell_overhead,
                             float shared_cost, float limit, int reserved, int reserved_units,
                             void* stream) {
    HSN_ABI_BEGIN
    HSN_REQUIRE(logits && cost && cells && units && valid && theta && refreshed,
                HSN_ERR_INVALID_ARGUMENT, "hsn_win_route: a required pointer is NULL");
    HSN_REQUIRE(B >= 1 && T >= 1 && N >= 1 && M >= 1 && K >= 1, HSN_ERR_INVALID_ARGUMENT,
                "hsn_win_route: dimensions must be >= 1");
    HSN_REQUIRE(K <= N && K <= kWave, HSN_ERR_INVALID_ARGUMENT,
                "hsn_win_route: need K <= N and K <= 64");
    HSN_REQUIRE(N <= 64 * kWave, HSN_ERR_INVALID_ARGUMENT, "hsn_win_route: N above 4096");
    HSN_REQUIRE(width >= M, HSN_ERR_INVALID_ARGUMENT, "hsn_win_route: width < M");
    // the router's own checks (python/hsn/model/router.py:1328-1339)
    HSN_REQUIRE(reserved >= 0 && (reserved == 0 || reserved < K), HSN_ERR_INVALID_ARGUMENT,
                "hsn_win_route: reserved must be 0 or lie in [1, K)");
    HSN_REQUIRE(!reserved_units || reserved > 0, HSN_ERR_INVALID_ARGUMENT,
                "hsn_win_route: reserved_units needs reserved > 0");
    HSN_REQUIRE(index_bits == 32 || index_bits == 64, HSN_ERR_INVALID_ARGUMENT,
                "hsn_win_route: index_bits must be 32 or 64");
    HSN_REQUIRE(io_dtype == HSN_DTYPE_F32 || io_dtype == HSN_DTYPE_BF16,
                HSN_ERR_UNSUPPORTED_DTYPE, "hsn_win_route: logits must be f32 or bf16");
    HSN_REQUIRE(!probes || (age0 && reset), HSN_ERR_INVALID_ARGUMENT,
                "hsn_win_route: probes need age0 and reset");
    HSN_REQUIRE(check_elems({int64_t(B) * T * N * width, int64_t(B) * T * K, int64_t(B) * N}),
                HSN_ERR_SIZE_OVERFLOW, "hsn_win_route: a tensor is too large");
    RouteArgs a{};
    a.logits = logits;
    a.width = width;
    a.l_pos = int64_t(N) * width;
    a.l_row = int64_t(T) * a.l_pos;
    a.cost = cost;
    a.age0 = probes ? age0 : nullptr;
    a.reset = probes ? reset : nullptr;
    a.cells = cells;
    a.units = units;
    a.valid = valid;
    a.refreshed = refreshed;
    a.slots = slots;
    a.o_pos = K;
    a.o_row = int64_t(T) * K;
    a.theta = theta;
    a.th_pos = 1;
    a.th_row = T;
    a.h_max_zero = h_max_zero;
    a.B = B, a.P = T, a.N = N, a.M = M, a.K = K, a.age_max = age_max, a.probes = probes ? 1 : 0;
    a.reserved = reserved, a.fixed_units = reserved_units ? 1 : 0;
    a.lambda = lambda_cost, a.overhead = cell_overhead, a.shared = shared_cost, a.limit = limit;
    HSN_HIP(dispatch_route(a, io_dtype, index_bits, probes != 0, as_stream(stream)));
    HSN_ABI_END
}

extern "C" int hsn_win_select(const void* logits, int io_dtype, int64_t width, const int64_t* age,
                              const float* cost, int64_t* cells, int64_t* units, uint8_t* valid,
                              float* theta, uint8_t* refreshed, int B, int N, int M, int K, int t,
                              int n_out, int n_age, int age_max, int probes, float lambda_cost,
                              float cell_overhead, float shared_cost, float limit, int reserved,
                              int reserved_units, void* stream) {
    HSN_ABI_BEGIN
    HSN_REQUIRE(logits && cost && cells && units && valid && theta && refreshed,
                HSN_ERR_INVALID_ARGUMENT, "hsn_win_select: a required pointer is NULL");
    HSN_REQUIRE(B >= 1 && N >= 1 && M >= 1 && K >= 1, HSN_ERR_INVALID_ARGUMENT,
                "hsn_win_select: dimensions must be >= 1");
    HSN_REQUIRE(K <= N && K <= kWave && N <= 64 * kWave, HSN_ERR_INVALID_ARGUMENT,
                "hsn_win_select: need K <= N, K <= 64, N <= 4096");
    HSN_REQUIRE(width >= M, HSN_ERR_INVALID_ARGUMENT, "hsn_win_select: width < M");
    HSN_REQUIRE(t >= 0 && t < n_out && (!probes || (age && t < n_age)), HSN_ERR_INVALID_ARGUMENT,
                "hsn_win_select: record t outside the tapes (or probes without ages)");
    // the router's own checks (python/hsn/model/router.py:1328-1339)
    HSN_REQUIRE(reserved >= 0 && (reserved == 0 || reserved < K), HSN_ERR_INVALID_ARGUMENT,
                "hsn_win_select: reserved must be 0 or lie in [1, K)");
    HSN_REQUIRE(!reserved_units || reserved > 0, HSN_ERR_INVALID_ARGUMENT,
                "hsn_win_select: reserved_units needs reserved > 0");
    HSN_REQUIRE(io_dtype == HSN_DTYPE_F32 || io_dtype == HSN_DTYPE_BF16,
                HSN_ERR_UNSUPPORTED_DTYPE, "hsn_win_select: logits must be f32 or bf16");
    RouteArgs a{};
    a.logits = logits;
    a.width = width;
    a.l_pos = 0;
    a.l_row = int64_t(N) * width;
    a.cost = cost;
    a.age = probes ? age : nullptr;
    a.age_row = int64_t(n_age) * N;
    a.age_rec = t;
    a.cells = cells;
    a.units = units;
    a.valid = valid;
    a.refreshed = refreshed;
    a.o_row = int64_t(n_out) * K;
    a.o_pos = 0;
    // the record offset rides on the base pointers
    a.cells = cells + int64_t(t) * K;
    a.units = units + int64_t(t) * K;
    a.valid = valid + int64_t(t) * K;
    a.refreshed = refreshed + int64_t(t) * K;
    a.theta = theta + t;
    a.th_row = n_out;
    a.th_pos = 0;
    a.B = B, a.P = 1, a.N = N, a.M = M, a.K = K, a.age_max = age_max, a.probes = probes ? 1 : 0;
    a.reserved = reserved, a.fixed_units = reserved_units ? 1 : 0;
    a.lambda = lambda_cost, a.overhead = cell_overhead, a.shared = shared_cost, a.limit = limit;
    HSN_HIP(dispatch_route(a, io_dtype, 64, probes != 0, as_stream(stream)));
    HSN_ABI_END
}
