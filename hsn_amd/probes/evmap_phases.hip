// Phase timeline of the event-map forward and backward (evmap.cuh) at the ref shape
// (B32 T256 N256 d64 K8 fp32): the kernels built with their phase-stamp hooks on, each
// wavefront recording the real-time counter (100 MHz) at its phase edges. Prints, per phase edge,
// the mean and largest time from the earliest wavefront's start, the spread of each phase's span
// over the wavefronts and of the workgroups' ends, and the back-to-back event durations of the
// uninstrumented launch sequence for comparison (the stamps cost a few instructions a phase).
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <random>
#include <vector>

#include <hip/hip_runtime.h>

#define HSN_EVMAP_STAMPS 1
__device__ unsigned long long* g_evmap_stamps[2];  // [workgroup][wavefront][10] per kernel
#define HSN_EVMAP_STAMPS_BEGIN()       \
    unsigned long long stamp_[10] = {}; \
    stamp_[0] = __builtin_amdgcn_s_memrealtime()
#define HSN_EVMAP_STAMP(i) stamp_[i] = __builtin_amdgcn_s_memrealtime()
#define HSN_EVMAP_NOTE(i, v) stamp_[i] = (v)
#define HSN_EVMAP_STAMPS_END(which)                                                               \
    do {                                                                                          \
        stamp_[7] = __builtin_amdgcn_s_memrealtime();                                             \
        __builtin_amdgcn_s_waitcnt(0);                                                            \
        stamp_[8] = __builtin_amdgcn_s_memrealtime();                                             \
        unsigned long long* const out_ = g_evmap_stamps[which];                                   \
        if (out_ && (threadIdx.x & 63) == 0) {                                                    \
            const size_t wg_ = blockIdx.x + size_t(gridDim.x) * (blockIdx.y + size_t(gridDim.y) * blockIdx.z); \
            unsigned long long* const o_ = out_ + (wg_ * (blockDim.x / 64) + threadIdx.x / 64) * 10; \
            for (int i_ = 0; i_ < 10; ++i_) o_[i_] = stamp_[i_];                                  \
        }                                                                                         \
    } while (0)

#include "../csrc/evmap.hip"

// the library's host helpers that evmap.hip calls (defined elsewhere in the library)
hipError_t hsn::allow_lds_raw(const void* k, size_t lds) {
    return hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, int(lds));
}
bool hsn::evmap_takes(int, int, int, int, int, int, size_t, const char**) { return true; }
void hsn::set_last_error(const std::string&) {}
void hsn::clear_last_error() {}

#define CK(x)                                                                          \
    do {                                                                               \
        const hipError_t e_ = (x);                                                     \
        if (e_ != hipSuccess) {                                                        \
            std::printf("HIP error %s at line %d\n", hipGetErrorString(e_), __LINE__); \
            return 1;                                                                  \
        }                                                                              \
    } while (0)

namespace {

// `edges`: the stamps in the order the kernel reaches them (0..6 at the phase edges, 7 the last
// store issued, 8 every store done, 9 the routed forward's decisions made); in the forward and
// the backward word 9 notes whether the wavefront's chunks hold a reset (`split_by_note`)
void report(const char* what, const std::vector<unsigned long long>& h, const char* const* names,
            const std::vector<int>& edges, bool split_by_note = false) {
    const int kEdges = int(edges.size());
    unsigned long long t0 = ~0ull;
    for (size_t i = 0; i < h.size(); i += 10) t0 = std::min(t0, h[i]);
    const auto us = [&](unsigned long long t) { return double(t - t0) * 0.01; };
    std::printf("%s: time of each phase edge from the first wavefront's start (us)\n", what);
    for (int p = 0; p < kEdges; ++p) {
        double sum = 0, mx = 0;
        size_t n = 0;
        for (size_t i = 0; i < h.size(); i += 10, ++n) {
            sum += us(h[i + edges[p]]);
            mx = std::max(mx, us(h[i + edges[p]]));
        }
        std::printf("  %-28s mean %6.2f  max %6.2f\n", names[p], sum / n, mx);
    }
    std::printf("  span of each phase over the wavefronts (us):\n");
    for (int p = 1; p < kEdges; ++p) {
        std::vector<double> d;
        for (size_t i = 0; i < h.size(); i += 10)
            d.push_back(double(h[i + edges[p]] - h[i + edges[p - 1]]) * 0.01);
        std::sort(d.begin(), d.end());
        std::printf("    %-26s p10 %5.2f  p50 %5.2f  p90 %5.2f  max %5.2f\n", names[p], d[d.size() / 10],
                    d[d.size() / 2], d[d.size() * 9 / 10], d.back());
    }
    if (split_by_note) {  // the wavefronts whose chunks hold a reset against the others
        std::printf("  span of each phase, wavefronts with a reset in their chunks | without (p50 / max us):\n");
        for (int p = 1; p < kEdges; ++p) {
            std::vector<double> d[2];
            for (size_t i = 0; i < h.size(); i += 10)
                d[h[i + 9] != 0 ? 0 : 1].push_back(double(h[i + edges[p]] - h[i + edges[p - 1]]) * 0.01);
            for (auto& v : d) std::sort(v.begin(), v.end());
            if (d[0].empty() || d[1].empty()) break;
            std::printf("    %-26s %5.2f / %5.2f | %5.2f / %5.2f   (%zu | %zu)\n", names[p], d[0][d[0].size() / 2],
                        d[0].back(), d[1][d[1].size() / 2], d[1].back(), d[0].size(), d[1].size());
        }
    }
    const size_t nwg = h.size() / 80;
    std::vector<double> end(nwg, 0.0);
    for (size_t w = 0; w < nwg; ++w)
        for (int v = 0; v < 8; ++v) end[w] = std::max(end[w], us(h[(w * 8 + v) * 10 + 8]));
    std::sort(end.begin(), end.end());
    std::printf("  workgroups' last store done (us): p10 %.2f  p50 %.2f  p90 %.2f  max %.2f\n",
                end[nwg / 10], end[nwg / 2], end[nwg * 9 / 10], end.back());
}

}  // namespace

int main(int argc, char** argv) {
    using namespace hsn;
    // argv[1]: one reset in this many positions (default 256; 0 for none)
    const int reset_every = argc > 1 ? std::atoi(argv[1]) : 256;
    const int B = 32, T = 256, N = 256, d = 64, K = 8;
    const size_t ne = size_t(B) * T * K * d, nq = size_t(B) * T * d, nh = size_t(B) * N * d;
    // the ref workload's distributions: rows N(0, 1), gates N(2, 0.5), start state N(0, 0.1),
    // K distinct cells a position, resets Bernoulli(1/256); cotangents N(0, 1)
    std::mt19937 rng(5);
    std::normal_distribution<float> nd(0.f, 1.f);
    std::uniform_real_distribution<float> ud(0.f, 1.f);
    std::vector<float> y(ne), g(ne), dsel(ne), dq(nq), h0(nh), dhT(nh);
    for (auto& v : y) v = nd(rng);
    for (auto& v : g) v = 2.0f + 0.5f * nd(rng);
    for (auto& v : dsel) v = nd(rng);
    for (auto& v : dq) v = nd(rng);
    for (auto& v : h0) v = 0.1f * nd(rng);
    for (auto& v : dhT) v = nd(rng);
    std::vector<int32_t> slots(size_t(B) * T * K), perm(N);
    for (int i = 0; i < N; ++i) perm[i] = i;
    for (size_t bt = 0; bt < size_t(B) * T; ++bt) {
        std::shuffle(perm.begin(), perm.end(), rng);
        for (int k = 0; k < K; ++k) slots[bt * K + k] = perm[k];
    }
    std::vector<uint8_t> reset(size_t(B) * T);
    for (auto& r : reset) r = reset_every > 0 && ud(rng) < 1.0f / float(reset_every) ? 1 : 0;
    std::printf("resets: Bernoulli(1/%d), %d in the window's %d rows\n", reset_every,
                int(std::count(reset.begin(), reset.end(), uint8_t(1))), B);

    float *dy_, *dg_, *y_, *g_, *ho_, *hs_, *qa_, *qb_, *hm_, *h0_, *q0_, *hT_, *qT_, *ds_, *dqa_,
        *dqb_, *dhT_, *dqT_, *dh0_, *dq0_;
    int32_t* sl_;
    uint8_t* rs_;
    int64_t *a0_, *p0_, *aT_, *pT_;
    for (float** p : {&y_, &g_, &ho_, &hs_, &ds_, &dy_, &dg_}) CK(hipMalloc(p, ne * 4));
    for (float** p : {&qa_, &qb_, &dqa_, &dqb_}) CK(hipMalloc(p, nq * 4));
    for (float** p : {&h0_, &hT_, &dhT_, &dh0_}) CK(hipMalloc(p, nh * 4));
    for (float** p : {&q0_, &qT_, &dqT_, &dq0_}) CK(hipMalloc(p, size_t(B) * d * 4));
    CK(hipMalloc(&hm_, size_t(B) * T * 4));
    CK(hipMalloc(&sl_, slots.size() * 4));
    CK(hipMalloc(&rs_, reset.size()));
    for (int64_t** p : {&a0_, &aT_}) CK(hipMalloc(p, size_t(B) * N * 8));
    for (int64_t** p : {&p0_, &pT_}) CK(hipMalloc(p, size_t(B) * 8));
    CK(hipMemcpy(y_, y.data(), ne * 4, hipMemcpyHostToDevice));
    CK(hipMemcpy(g_, g.data(), ne * 4, hipMemcpyHostToDevice));
    CK(hipMemcpy(ds_, dsel.data(), ne * 4, hipMemcpyHostToDevice));
    CK(hipMemcpy(dqa_, dq.data(), nq * 4, hipMemcpyHostToDevice));
    CK(hipMemcpy(dqb_, dq.data(), nq * 4, hipMemcpyHostToDevice));
    CK(hipMemcpy(h0_, h0.data(), nh * 4, hipMemcpyHostToDevice));
    CK(hipMemcpy(dhT_, dhT.data(), nh * 4, hipMemcpyHostToDevice));
    CK(hipMemcpy(sl_, slots.data(), slots.size() * 4, hipMemcpyHostToDevice));
    CK(hipMemcpy(rs_, reset.data(), reset.size(), hipMemcpyHostToDevice));
    CK(hipMemset(q0_, 0, size_t(B) * d * 4));
    CK(hipMemset(dqT_, 0, size_t(B) * d * 4));
    CK(hipMemset(a0_, 0, size_t(B) * N * 8));
    CK(hipMemset(p0_, 0, size_t(B) * 8));
    CK(hipMemset(hm_, 0, size_t(B) * T * 4));

    const auto forward = [&] {
        evmap_forward(y_, g_, rs_, sl_, h0_, q0_, a0_, p0_, qa_, qb_, hs_, ho_, hm_, hT_, qT_, aT_,
                      pT_, B, T, N, d, K, nullptr);
    };
    const auto backward = [&] {
        evmap_backward(y_, g_, ho_, sl_, rs_, dqa_, dqb_, ds_, dhT_, dqT_, dy_, dg_, dh0_, dq0_, B,
                       T, N, d, K, nullptr);
    };
    const size_t nwg = size_t(B) * (d / evmap::kS), words = nwg * evmap::kWaves * 10;
    unsigned long long *st_f, *st_b;
    CK(hipMalloc(&st_f, words * 8));
    CK(hipMalloc(&st_b, words * 8));
    unsigned long long* none[2] = {nullptr, nullptr};
    CK(hipMemcpyToSymbol(HIP_SYMBOL(g_evmap_stamps), none, sizeof(none)));
    hipEvent_t e0, e1, e2;
    CK(hipEventCreate(&e0));
    CK(hipEventCreate(&e1));
    CK(hipEventCreate(&e2));
    try {
        for (int i = 0; i < 3; ++i) forward(), backward();
        CK(hipDeviceSynchronize());
        // back to back: 20 forwards, then 20 backwards
        float tf = 0, tb = 0;
        CK(hipEventRecord(e0));
        for (int i = 0; i < 20; ++i) forward();
        CK(hipEventRecord(e1));
        for (int i = 0; i < 20; ++i) backward();
        CK(hipEventRecord(e2));
        CK(hipEventSynchronize(e2));
        CK(hipEventElapsedTime(&tf, e0, e1));
        CK(hipEventElapsedTime(&tb, e1, e2));
        std::printf("back-to-back launches (instrumented build): forward %.2f us, backward %.2f us\n",
                    tf * 1e3f / 20, tb * 1e3f / 20);
        unsigned long long* on[2] = {st_f, st_b};
        CK(hipMemcpyToSymbol(HIP_SYMBOL(g_evmap_stamps), on, sizeof(on)));
        forward();
        backward();
        CK(hipDeviceSynchronize());
    } catch (const AbiError& e) {
        std::printf("library error: %s\n", e.message.c_str());
        return 1;
    }
    std::vector<unsigned long long> h(words);
    CK(hipMemcpy(h.data(), st_f, words * 8, hipMemcpyDeviceToHost));
    const char* fwd_names[9] = {"start", "first loads issued", "tables built, compose starts",
                                "phase A barrier passed", "phase B (walk) barrier passed",
                                "replay done", "summary scanned and stored",
                                "last store issued", "every store done"};
    const std::vector<int> in_order = {0, 1, 2, 3, 4, 5, 6, 7, 8};
    report("forward", h, fwd_names, in_order, true);
    CK(hipMemcpy(h.data(), st_b, words * 8, hipMemcpyDeviceToHost));
    const char* bwd_names[9] = {"start", "first loads issued", "summary maps, tables built",
                                "shares written, compose starts", "phase A barrier passed",
                                "phase B (walk) barrier passed", "replay done",
                                "last store issued", "every store done"};
    report("backward", h, bwd_names, in_order, true);

    // the forward that routes its own window (hsn_win_route_forward's one launch): logits N(0, 1)
    std::vector<float> logits(size_t(B) * T * N);
    for (auto& v : logits) v = nd(rng);
    float *lg_, *cost_, *th_;
    int32_t *cells_, *units_, *rslots_;
    uint8_t *valid_, *refr_;
    CK(hipMalloc(&lg_, logits.size() * 4));
    CK(hipMalloc(&cost_, 4));
    CK(hipMalloc(&th_, size_t(B) * T * 4));
    for (int32_t** p : {&cells_, &units_, &rslots_}) CK(hipMalloc(p, size_t(B) * T * K * 4));
    for (uint8_t** p : {&valid_, &refr_}) CK(hipMalloc(p, size_t(B) * T * K));
    CK(hipMemcpy(lg_, logits.data(), logits.size() * 4, hipMemcpyHostToDevice));
    const float c0 = 1.0f / N;
    CK(hipMemcpy(cost_, &c0, 4, hipMemcpyHostToDevice));
    WindowRouteSpec r{};
    r.logits = lg_, r.width = 1, r.cost = cost_, r.cells = cells_, r.units = units_;
    r.valid = valid_, r.theta = th_, r.refreshed = refr_, r.slots = rslots_, r.reserved = 0;
    r.lambda = 0.0f, r.overhead = 0.0f, r.shared = 0.0f, r.limit = 1.00001f;
    const char* why = nullptr;
    if (!evmap_route_claim(nullptr, B, d, true, &why)) {
        std::printf("routed forward not taken: %s\n", why);
        return 0;
    }
    const auto routed = [&] {
        evmap_route_forward(r, y_, g_, rs_, h0_, q0_, a0_, p0_, qa_, qb_, hs_, ho_, hm_, hT_, qT_,
                            aT_, pT_, B, T, N, d, K, nullptr);
    };
    try {
        CK(hipMemcpyToSymbol(HIP_SYMBOL(g_evmap_stamps), none, sizeof(none)));
        for (int i = 0; i < 3; ++i) routed();
        CK(hipDeviceSynchronize());
        float tr = 0;
        CK(hipEventRecord(e0));
        for (int i = 0; i < 20; ++i) routed();
        CK(hipEventRecord(e1));
        CK(hipEventSynchronize(e1));
        CK(hipEventElapsedTime(&tr, e0, e1));
        std::printf("back-to-back launches (instrumented build): routed forward %.2f us\n", tr * 1e3f / 20);
        unsigned long long* on[2] = {st_f, st_b};
        CK(hipMemcpyToSymbol(HIP_SYMBOL(g_evmap_stamps), on, sizeof(on)));
        routed();
        CK(hipDeviceSynchronize());
    } catch (const AbiError& e) {
        std::printf("library error: %s\n", e.message.c_str());
        return 1;
    }
    CK(hipMemcpy(h.data(), st_f, words * 8, hipMemcpyDeviceToHost));
    const char* routed_names[10] = {"start", "first loads issued (logits first)",
                                    "the wavefront's decisions made",
                                    "row's decisions gathered, tables built",
                                    "phase A barrier passed", "phase B (walk) barrier passed",
                                    "replay done", "summary scanned and stored",
                                    "last store issued", "every store done"};
    report("routed forward", h, routed_names, {0, 1, 9, 2, 3, 4, 5, 6, 7, 8});
    unsigned timeouts = 0;
    CK(hipMemcpyFromSymbol(&timeouts, HIP_SYMBOL(g_exchange_timeouts), sizeof(timeouts)));
    std::printf("exchange waits that reached their limit: %u\n", timeouts);
    return 0;
}
