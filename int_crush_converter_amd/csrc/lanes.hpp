// Streams for the lookahead schedules of the blocked factorisations: `a`
// carries the critical chain (diagonal blocks, panels, the next block's
// update), `b` and `c` the wide updates that the chain does not wait for.
// All have the default priority and are created once per host thread and
// device; b and c are confined (CU mask) to 7 of every 8 CUs, so the
// chain's single-work-group kernels never wait for a CU behind them.  The
// caller's stream only fences in (begin) and out (end); ordering between
// the three is explicit (events).
#pragma once

#include "common.hpp"

namespace icq {

class Lanes {
public:
    hipStream_t a = nullptr, b = nullptr, c = nullptr;

    // a, b and c start after the work already enqueued on `caller`.
    int begin(hipStream_t caller);
    // Event recorded on s now (from a per-thread pool; an event is reused
    // only after LANES_EVENTS later marks, by which time its waits are
    // enqueued).
    hipEvent_t mark(hipStream_t s);
    // s waits for the work behind event e (no-op for a null event).
    void wait(hipStream_t s, hipEvent_t e);
    // the caller's stream waits for everything enqueued on a, b and c;
    // returns the first error.
    int end();

private:
    hipStream_t caller_ = nullptr;
    int err_ = 0;
    void note(hipError_t e);
};

}  // namespace icq
