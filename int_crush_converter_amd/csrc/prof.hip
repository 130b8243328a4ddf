// Launch profiler (see prof.hpp).
#include "prof.hpp"

#include <mutex>
#include <vector>

namespace icq {

struct ProfRec {
    hipEvent_t a = nullptr, b = nullptr;
    int tag = 0;
    double flops = 0, bytes = 0;
};

static std::mutex g_mu;
static bool g_on = false;
static std::vector<ProfRec> g_recs;   // events are reused across resets
static size_t g_used = 0;

static thread_local bool t_suppress = false;

bool prof_enabled() { return g_on; }

ProfSuppress::ProfSuppress() : prev_(t_suppress) { t_suppress = true; }
ProfSuppress::~ProfSuppress() { t_suppress = prev_; }

ProfScope::ProfScope(hipStream_t st, int tag, double flops, double bytes) : st_(st) {
    if (!g_on || t_suppress) return;
    std::lock_guard<std::mutex> lk(g_mu);
    if (g_used == g_recs.size()) {
        ProfRec r;
        if (hipEventCreate(&r.a) != hipSuccess || hipEventCreate(&r.b) != hipSuccess) return;
        g_recs.push_back(r);
    }
    idx_ = (int)g_used++;
    ProfRec& r = g_recs[idx_];
    r.tag = tag;
    r.flops = flops;
    r.bytes = bytes;
    (void)hipEventRecord(r.a, st_);
}

ProfScope::~ProfScope() {
    if (idx_ < 0) return;
    (void)hipEventRecord(g_recs[idx_].b, st_);
}

}  // namespace icq

using namespace icq;

extern "C" int ic_profile_enable(int on) {
    std::lock_guard<std::mutex> lk(g_mu);
    g_on = on != 0;
    g_used = 0;
    return IC_OK;
}

extern "C" int ic_profile_read(double* ms, double* flops, double* bytes, int64_t* launches, int ntags) {
    IC_REQUIRE(ms && flops && bytes && launches && ntags >= PT_COUNT, "ic_profile_read: need PT_COUNT slots");
    std::lock_guard<std::mutex> lk(g_mu);
    for (int t = 0; t < ntags; ++t) { ms[t] = 0; flops[t] = 0; bytes[t] = 0; launches[t] = 0; }
    for (size_t i = 0; i < g_used; ++i) {
        ProfRec& r = g_recs[i];
        IC_CHECK_HIP(hipEventSynchronize(r.b));
        float e = 0.0f;
        IC_CHECK_HIP(hipEventElapsedTime(&e, r.a, r.b));
        ms[r.tag] += e;
        flops[r.tag] += r.flops;
        bytes[r.tag] += r.bytes;
        launches[r.tag] += 1;
    }
    return IC_OK;
}
