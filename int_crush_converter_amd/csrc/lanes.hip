// Side streams and event pool of lanes.hpp.
#include "lanes.hpp"

#include <unordered_map>
#include <vector>

namespace icq {

constexpr int LANES_EVENTS = 64;

struct LaneSet {
    hipStream_t a = nullptr, b = nullptr, c = nullptr;
    hipEvent_t ev[LANES_EVENTS] = {};
    int next = 0;
    bool ok = false;
};

// One CU in LANES_RESERVE_EVERY is kept free of the side streams' work, so
// that the critical chain's single-work-group kernels always find a CU.
constexpr int LANES_RESERVE_EVERY = 8;

static LaneSet* lane_set() {
    static thread_local std::unordered_map<int, LaneSet> sets;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return nullptr;
    LaneSet& s = sets[dev];
    if (!s.ok) {
        int ncu = 0;
        if (hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || ncu <= 0)
            return nullptr;
        std::vector<uint32_t> mask((size_t)(ncu + 31) / 32, 0u);
        for (int cu = 0; cu < ncu; ++cu)
            if (cu % LANES_RESERVE_EVERY != 0) mask[cu / 32] |= 1u << (cu % 32);
        if (hipStreamCreateWithFlags(&s.a, hipStreamNonBlocking) != hipSuccess) return nullptr;
        if (hipExtStreamCreateWithCUMask(&s.b, (uint32_t)mask.size(), mask.data()) != hipSuccess) return nullptr;
        if (hipExtStreamCreateWithCUMask(&s.c, (uint32_t)mask.size(), mask.data()) != hipSuccess) return nullptr;
        for (int i = 0; i < LANES_EVENTS; ++i)
            if (hipEventCreateWithFlags(&s.ev[i], hipEventDisableTiming) != hipSuccess) return nullptr;
        s.ok = true;
    }
    return &s;
}

void Lanes::note(hipError_t e) {
    if (e != hipSuccess && err_ == 0) err_ = fail(IC_ERR_HIP, std::string("lanes: ") + hipGetErrorString(e));
}

int Lanes::begin(hipStream_t caller) {
    LaneSet* s = lane_set();
    if (!s) return fail(IC_ERR_HIP, "lanes: cannot create the side streams");
    caller_ = caller;
    a = s->a;
    b = s->b;
    c = s->c;
    hipEvent_t e = mark(caller_);
    wait(a, e);
    wait(b, e);
    wait(c, e);
    return err_;
}

hipEvent_t Lanes::mark(hipStream_t st) {
    LaneSet* s = lane_set();
    if (!s) {
        if (err_ == 0) err_ = fail(IC_ERR_HIP, "lanes: no event pool");
        return nullptr;
    }
    hipEvent_t e = s->ev[s->next];
    s->next = (s->next + 1) % LANES_EVENTS;
    note(hipEventRecord(e, st));
    return e;
}

void Lanes::wait(hipStream_t st, hipEvent_t e) {
    if (e) note(hipStreamWaitEvent(st, e, 0));
}

int Lanes::end() {
    wait(caller_, mark(a));
    wait(caller_, mark(b));
    wait(caller_, mark(c));
    return err_;
}

}  // namespace icq
