// The event-map path of hsn_win_forward and hsn_win_backward (evmap.cuh): argument blocks and
// launches; and the forward that routes its own window (hsn_win_route_forward), whose
// workgroups hand the row's decisions to each other through stamped words in device memory.
#include <mutex>

#include "abi_util.h"
#include "chain_host.h"
#include "evmap.cuh"
// after the sweeps: the router's header turns floating-point contraction off for what follows
#include "route.cuh"

namespace hsn {

void evmap_forward(const void* y, const void* gate_pre, const uint8_t* reset,
                   const int32_t* slots, const float* h0, const float* q0, const int64_t* age0,
                   const int64_t* pos0, void* q_pre, void* q_post, void* h_sel, void* h_old,
                   float* h_max, float* h_T, float* q_T, int64_t* age_T, int64_t* pos_T, int B,
                   int T, int N, int d, int K, hipStream_t st) {
    evmap::FwdEv a{};
    a.y = static_cast<const float*>(y), a.g = static_cast<const float*>(gate_pre);
    a.slots = slots, a.reset = reset, a.h0 = h0, a.q0 = q0, a.age0 = age0, a.pos0 = pos0;
    a.q_pre = static_cast<float*>(q_pre), a.q_post = static_cast<float*>(q_post);
    a.h_sel = static_cast<float*>(h_sel), a.h_old = static_cast<float*>(h_old);
    a.h_max = h_max, a.h_T = h_T, a.q_T = q_T, a.age_T = age_T, a.pos_T = pos_T;
    a.T = T, a.N = N, a.d = d, a.K = K, a.P = (T + evmap::kChunks - 1) / evmap::kChunks;
    a.divn = make_divn(N);
    const size_t lds = evmap::fwd_layout(N).bytes;
    auto k = evmap::fwd<float>;
    HSN_HIP(allow_lds(k, lds));
    hipLaunchKernelGGL(k, sweep_grid(B, d / evmap::kS), dim3(kWave * evmap::kWaves), lds, st, a);
    HSN_HIP(hipGetLastError());
}

void evmap_backward(const void* y, const void* gate_pre, const void* h_old, const int32_t* slots,
                    const uint8_t* reset, const void* d_q_pre, const void* d_q_post,
                    const void* d_h_sel, const float* d_h_T, const float* d_q_T, void* dy,
                    void* dgate, float* d_h0, float* d_q0, int B, int T, int N, int d, int K,
                    hipStream_t st) {
    evmap::BwdEv a{};
    a.y = static_cast<const float*>(y), a.g = static_cast<const float*>(gate_pre);
    a.h_old = static_cast<const float*>(h_old), a.dsel = static_cast<const float*>(d_h_sel);
    a.slots = slots, a.reset = reset;
    a.dq_pre = static_cast<const float*>(d_q_pre), a.dq_post = static_cast<const float*>(d_q_post);
    a.dh_T = d_h_T, a.dq_T = d_q_T;
    a.dy = static_cast<float*>(dy), a.dg = static_cast<float*>(dgate);
    a.dh0 = d_h0, a.dq0 = d_q0;
    a.T = T, a.N = N, a.d = d, a.K = K, a.P = (T + evmap::kChunks - 1) / evmap::kChunks;
    a.divn = make_divn(N);
    const size_t lds = evmap::bwd_layout(N).bytes;
    auto k = evmap::bwd<float>;
    HSN_HIP(allow_lds(k, lds));
    hipLaunchKernelGGL(k, sweep_grid(B, d / evmap::kS), dim3(kWave * evmap::kWaves), lds, st, a);
    HSN_HIP(hipGetLastError());
}

namespace {

// ---- the forward that routes its own window -------------------------------------------------
//
// The workgroups of row b (one a slice of 8 columns, all on one XCD by the grid's layout) split
// the row's positions: slice s decides positions [s R, s R + R), R = ceil(T / slices), a
// wavefront every 8th of them, while its slot rows load. Every decision goes to the row as one
// 64-bit word a slot, (stamp << 16) | (cell + 1), written and read as relaxed agent-scope
// atomics: a word is complete by itself, so a reader needs no fence, only the stamp of this
// launch, which tells the word from an older launch's. The stamp is the device's count of these
// launches (the host's, a kernel argument): each launch has its own, since no graph captures
// one (a replay would repeat its stamp). The row maxima of |h| take the same way back: every
// slice's part of every position is a word (stamp << 32) | bits, and slice s max-reduces its own
// positions' parts and writes them (the host clears these words whenever the stamp's low 32
// bits wrap). Only the device's first stream that calls uses these buffers (the host keeps the
// others on two launches), so launches that share them are ordered.

constexpr int kBoxRows = 256;       // rows, at most (the grid B * slices <= 256)
constexpr int kBoxPositions = 256;  // T, at most (the event maps' bound)
__device__ uint64_t g_slot_box[size_t(kBoxRows) * kBoxPositions * evmap::kK];
__device__ uint64_t g_hmax_box[size_t(kBoxRows) * kBoxPositions];  // [B][T][slices], B slices <= 256
__device__ unsigned int g_exchange_timeouts;

// Polls of one word before the word is taken as it is and the launch counted in
// g_exchange_timeouts (about a second: only a grid whose workgroups of a row are not all
// resident can wait that long).
constexpr int kSpinLimit = 1 << 20;

constexpr int kRouteWaves = evmap::kWaves;
constexpr int kRouteJ = 4;  // consecutive positions a wavefront decides, at most
constexpr int kRouteShare = kRouteWaves * kRouteJ;
// the row's int16 decisions (T K <= 256 * 8) and a workgroup's row-maximum accumulators fit in a
// chunk's maps below cell 0's entry (kConst) and the dummy entry, which hold identity maps
static_assert(kBoxPositions * evmap::kK * 2 <= evmap::kConst * evmap::kEntBytes, "slot table");
static_assert(kBoxPositions * 4 <= evmap::kConst * evmap::kEntBytes, "row maxima");

// The decisions of a wavefront's positions by decide_grouped (LP lanes a position, CPL cells a
// lane; a position with more candidates than lanes by decide_select, NPLF cells a lane), its
// scratch in its first chunk's maps: the scores, lists and order words below the alpha table's
// cell-0 and dummy entries, the slot tables in the beta table.
template <int LP, int CPL, int NPLF>
struct WindowRoute {
    static constexpr bool kOn = true;
    static constexpr int G = kWave / LP;
    static constexpr int kCalls = kRouteJ / G;
    static constexpr uint32_t kTabAt = evmap::kEnt * evmap::kEntBytes;
    static_assert(CPL * kWave * 4 + kWave * 16 + G * (LP + 4) * 8 <= evmap::kConst * evmap::kEntBytes,
                  "scores, lists and order words below cell 0's and the dummy entries");
    static_assert(kTabAt + kWave * 16 <= (evmap::kEnt + evmap::kDummy) * evmap::kEntBytes, "slot tables");
    static_assert(G * (LP + 4) * 8 >= (kWave + 4) * 8, "decide_select's order words");
    const RouteArgs& ra;
    uint64_t launch;  // this launch's stamp
    int share;        // positions a workgroup decides
    int slices;       // workgroups a row
    float raw[kCalls][CPL];

    __device__ __forceinline__ int q_first(int b, int slice, int w, int c) const {
        return b * ra.P + slice * share + kRouteJ * w + G * c;
    }
    __device__ __forceinline__ int q_end(int b, int slice) const {
        return b * ra.P + min(ra.P, (slice + 1) * share);
    }
    __device__ __forceinline__ uint64_t stamp(int) const { return launch; }
    __device__ __forceinline__ void prefetch(int b, int slice, int w) {
#pragma unroll
        for (int c = 0; c < kCalls; ++c)
            load_grouped<LP, CPL, float>(ra, q_first(b, slice, w, c), q_end(b, slice), raw[c]);
    }
    __device__ __forceinline__ void decide(int b, int slice, int w, uint64_t st, unsigned char* scratch) {
        GroupedScratch sm;
        sm.sc = reinterpret_cast<float*>(scratch);
        sm.cand = reinterpret_cast<uint4*>(scratch + CPL * kWave * 4);
        sm.ord = reinterpret_cast<uint64_t*>(sm.cand + kWave);
        sm.tab = reinterpret_cast<uint4*>(scratch + kTabAt);
        const int qe = q_end(b, slice);
#pragma unroll
        for (int c = 0; c < kCalls; ++c) {
            const int q0 = q_first(b, slice, w, c);
            uint32_t need = decide_grouped_from<LP, CPL, float, int32_t>(ra, q0, qe, raw[c], sm, st);
            while (need != 0u) {
                __builtin_amdgcn_wave_barrier();
                const int g = __builtin_ctz(need);
                need &= need - 1u;
                const int q = q0 + g;
                decide_select<NPLF, true, float, int32_t>(ra, q / ra.P, q % ra.P, sm.cand, sm.tab, sm.ord, st);
            }
            __builtin_amdgcn_wave_barrier();
        }
    }
    // the row's T K decisions into LDS as int16 (the cell, -1 where padded): thread t polls
    // words t, t + 512, ... until each carries the stamp; the workgroup's barrier comes before
    // the LDS writes (the table shares the maps with the decisions' scratch)
    __device__ __forceinline__ void gather(int b, uint64_t st, unsigned char* slotv) const {
        const int total = ra.P * ra.K;
        const uint64_t* row = g_slot_box + size_t(b) * total;
        int16_t* out = reinterpret_cast<int16_t*>(slotv);
        constexpr int kThreads = kWave * evmap::kWaves;
        uint64_t v[4];
        uint32_t pending = 0u;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int e = int(threadIdx.x) + kThreads * q;
            v[q] = 0u;
            if (e < total) pending |= 1u << q;
        }
        for (int polls = 0; pending != 0u;) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                if ((pending >> q) & 1u) {
                    v[q] = __hip_atomic_load(row + int(threadIdx.x) + kThreads * q, __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT);
                    if ((v[q] >> 16) == st) pending &= ~(1u << q);
                }
            }
            if (pending == 0u) break;
            if (++polls >= kSpinLimit) {
                atomicAdd(&g_exchange_timeouts, 1u);
                break;
            }
            __builtin_amdgcn_s_sleep(2);
        }
        __syncthreads();
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int e = int(threadIdx.x) + kThreads * q;
            if (e < total) {
                const int c = int(v[q] & 0xffffu) - 1;  // in range even for a word taken as it is
                out[e] = static_cast<int16_t>(c < -1 ? -1 : (c >= ra.N ? ra.N - 1 : c));
            }
        }
    }
    // this slice's part of position t's row maximum, for the slice that decided t
    __device__ __forceinline__ void put_hmax(int b, int t, int slice, uint32_t mx, uint64_t st) const {
        __hip_atomic_store(g_hmax_box + (size_t(b) * ra.P + t) * slices + slice,
                           (st << 32) | uint64_t(mx), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    // the row maxima of this workgroup's positions from every slice's part (max-reduced in LDS
    // at `scratch`, 4 bytes a position)
    __device__ __forceinline__ void finish(int b, int slice, uint64_t st, float* h_max,
                                           unsigned char* scratch) const {
        constexpr int kThreads = kWave * evmap::kWaves;
        const int lo = slice * share;
        const int hi = min(ra.P, lo + share);
        if (h_max && hi > lo) {
            uint32_t* acc = reinterpret_cast<uint32_t*>(scratch);
            for (int i = threadIdx.x; i < hi - lo; i += kThreads) acc[i] = 0u;
            __syncthreads();
            const uint32_t want = static_cast<uint32_t>(st);
            for (int e = threadIdx.x; e < (hi - lo) * slices; e += kThreads) {
                const int t = lo + e / slices;
                const uint64_t* word = g_hmax_box + (size_t(b) * ra.P + t) * slices + e % slices;
                uint64_t v = __hip_atomic_load(word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                for (int polls = 0; uint32_t(v >> 32) != want;) {
                    if (++polls >= kSpinLimit) {
                        atomicAdd(&g_exchange_timeouts, 1u);
                        break;
                    }
                    __builtin_amdgcn_s_sleep(2);
                    v = __hip_atomic_load(word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
                atomicMax(&acc[t - lo], static_cast<uint32_t>(v));
            }
            __syncthreads();
            for (int i = threadIdx.x; i < hi - lo; i += kThreads)
                h_max[size_t(b) * ra.P + lo + i] = __uint_as_float(acc[i]);
        }
    }
};

template <int LP, int CPL, int NPLF>
__global__ __launch_bounds__(kWave* evmap::kWaves) void fwd_routed(evmap::FwdEv a, RouteArgs ra,
                                                                   uint64_t stamp, int share,
                                                                   int slices) {
    WindowRoute<LP, CPL, NPLF> route{ra, stamp, share, slices, {}};
    evmap::fwd_body<float>(a, route);
}

std::mutex g_route_lock;
constexpr int kMaxDevices = 64;
hipStream_t g_route_stream[kMaxDevices] = {};
bool g_route_claimed[kMaxDevices] = {};
int g_route_cus[kMaxDevices] = {};
void* g_route_box[kMaxDevices] = {};   // each device's address of g_slot_box
void* g_route_hmax[kMaxDevices] = {};  // and of g_hmax_box
uint64_t g_route_serial[kMaxDevices] = {};

}  // namespace

bool evmap_routes(int B, int T, int N, int d, int K, const char** why) {
    const char* r = nullptr;
    const int slices = d / evmap::kS;
    if (!evmap_takes(HSN_OP_FORWARD, B, T, N, d, K, 4, &r)) {
    } else if (N > 8 * kWave) r = "the routed forward takes N <= 512";
    else if (int64_t(B) * slices > kBoxRows) r = "the routed forward takes B d / 8 <= 256 workgroups";
    else if ((T + slices - 1) / slices > kRouteShare) r = "the routed forward takes T <= 32 d / 8";
    if (r && why) *why = r;
    return r == nullptr;
}

bool evmap_route_claim(hipStream_t st, int B, int d, bool take, const char** why) {
    int dev = 0;
    HSN_HIP(hipGetDevice(&dev));
    HSN_REQUIRE(dev >= 0 && dev < kMaxDevices, HSN_ERR_BACKEND, "device index above 63");
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    HSN_HIP(hipStreamIsCapturing(st, &cs));
    std::lock_guard<std::mutex> guard(g_route_lock);
    if (!g_route_cus[dev]) {
        HSN_HIP(hipDeviceGetAttribute(&g_route_cus[dev], hipDeviceAttributeMultiprocessorCount, dev));
        // the device's own copy of the slot words (host code never passes the symbol itself)
        void* box = nullptr;
        void* hmax = nullptr;
        HSN_HIP(hipGetSymbolAddress(&box, HIP_SYMBOL(g_slot_box)));
        HSN_HIP(hipGetSymbolAddress(&hmax, HIP_SYMBOL(g_hmax_box)));
        HSN_REQUIRE(box && hmax, HSN_ERR_BACKEND, "no device address for the routed forward's words");
        g_route_box[dev] = box;
        g_route_hmax[dev] = hmax;
    }
    const char* r = nullptr;
    if (cs != hipStreamCaptureStatusNone) r = "the stream is capturing (a graph's replays would repeat a launch's stamp)";
    else if (int64_t(B) * (d / evmap::kS) > g_route_cus[dev]) r = "the grid exceeds the device's compute units (its workgroups must all be resident)";
    else if (g_route_claimed[dev] && g_route_stream[dev] != st) r = "another stream of the device routes its windows in the forward";
    if (r) {
        if (why) *why = r;
        return false;
    }
    if (take) {
        g_route_claimed[dev] = true;
        g_route_stream[dev] = st;
    }
    return true;
}

// The slot words' address evmap_route_claim took for the current device, and the next launch's
// stamp (nonzero in its low 32 bits: where they wrap, the row maxima's words are cleared first,
// on the stream, so that no word of 2^32 launches ago can pass for this launch's).
void* route_launch(hipStream_t st, uint64_t* stamp) {
    int dev = 0;
    HSN_HIP(hipGetDevice(&dev));
    std::lock_guard<std::mutex> guard(g_route_lock);
    HSN_REQUIRE(dev >= 0 && dev < kMaxDevices && g_route_box[dev], HSN_ERR_BACKEND,
                "the routed forward ran before its device was set up");
    uint64_t next = ++g_route_serial[dev];
    if (static_cast<uint32_t>(next) == 0u) {
        HSN_HIP(hipMemsetAsync(g_route_hmax[dev], 0, sizeof(g_hmax_box), st));
        next = ++g_route_serial[dev];
    }
    *stamp = next;
    return g_route_box[dev];
}

void evmap_route_forward(const WindowRouteSpec& rs, const void* y, const void* gate_pre,
                         const uint8_t* reset, const float* h0, const float* q0,
                         const int64_t* age0, const int64_t* pos0, void* q_pre, void* q_post,
                         void* h_sel, void* h_old, float* h_max, float* h_T, float* q_T,
                         int64_t* age_T, int64_t* pos_T, int B, int T, int N, int d, int K,
                         hipStream_t st) {
    evmap::FwdEv a{};
    a.y = static_cast<const float*>(y), a.g = static_cast<const float*>(gate_pre);
    a.slots = nullptr, a.reset = reset, a.h0 = h0, a.q0 = q0, a.age0 = age0, a.pos0 = pos0;
    a.q_pre = static_cast<float*>(q_pre), a.q_post = static_cast<float*>(q_post);
    a.h_sel = static_cast<float*>(h_sel), a.h_old = static_cast<float*>(h_old);
    a.h_max = h_max, a.h_T = h_T, a.q_T = q_T, a.age_T = age_T, a.pos_T = pos_T;
    a.T = T, a.N = N, a.d = d, a.K = K, a.P = (T + evmap::kChunks - 1) / evmap::kChunks;
    a.divn = make_divn(N);

    RouteArgs ra{};
    ra.logits = rs.logits;
    ra.width = rs.width;
    ra.l_pos = int64_t(N) * rs.width;
    ra.l_row = int64_t(T) * ra.l_pos;
    ra.cost = rs.cost;
    ra.cells = rs.cells, ra.units = rs.units, ra.valid = rs.valid, ra.refreshed = rs.refreshed;
    ra.slots = rs.slots;
    ra.o_pos = K, ra.o_row = int64_t(T) * K;
    ra.theta = rs.theta, ra.th_pos = 1, ra.th_row = T;
    ra.h_max_zero = nullptr;
    uint64_t stamp = 0;
    ra.box = static_cast<uint64_t*>(route_launch(st, &stamp));
    ra.B = B, ra.P = T, ra.N = N, ra.M = 1, ra.K = K, ra.age_max = 0, ra.probes = 0;
    ra.reserved = rs.reserved, ra.fixed_units = 0;
    ra.lambda = rs.lambda, ra.overhead = rs.overhead, ra.shared = rs.shared, ra.limit = rs.limit;

    const int slices = d / evmap::kS;
    const int share = (T + slices - 1) / slices;
    const size_t lds = evmap::fwd_layout(N).bytes;
    const dim3 grid = sweep_grid(B, slices), block(kWave * evmap::kWaves);
    auto launch = [&](auto k) {
        HSN_HIP(allow_lds(k, lds));
        hipLaunchKernelGGL(k, grid, block, lds, st, a, ra, stamp, share, slices);
        HSN_HIP(hipGetLastError());
    };
    // the router's layouts (route.hip): two positions of 32 lanes a wavefront up to N = 256, one
    // of 64 lanes up to 512
    if (N <= 32) launch(fwd_routed<32, 1, 1>);
    else if (N <= 64) launch(fwd_routed<32, 2, 1>);
    else if (N <= 128) launch(fwd_routed<32, 4, 2>);
    else if (N <= 256) launch(fwd_routed<32, 8, 4>);
    else if (N <= 512) launch(fwd_routed<64, 8, 8>);
    else HSN_REQUIRE(false, HSN_ERR_INVALID_ARGUMENT, "the routed forward takes N <= 512");
}

unsigned evmap_exchange_timeouts(bool clear) {
    unsigned v = 0;
    HSN_HIP(hipDeviceSynchronize());
    HSN_HIP(hipMemcpyFromSymbol(&v, HIP_SYMBOL(g_exchange_timeouts), sizeof(v), 0, hipMemcpyDeviceToHost));
    if (clear && v) {
        const unsigned zero = 0;
        HSN_HIP(hipMemcpyToSymbol(HIP_SYMBOL(g_exchange_timeouts), &zero, sizeof(zero), 0, hipMemcpyHostToDevice));
    }
    return v;
}

}  // namespace hsn
