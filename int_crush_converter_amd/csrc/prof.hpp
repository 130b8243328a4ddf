// Optional launch profiler: when enabled (ic_profile_enable), instrumented
// launches are bracketed by HIP events on their stream and tagged with a
// phase and the algorithmic flops / bytes they perform.  ic_profile_read()
// synchronises the recorded events and returns per-phase totals.  Disabled,
// a scope costs one branch.
#pragma once

#include "common.hpp"

namespace icq {

enum ProfTag : int {
    PT_GEMM_TRAIL = 0,   // GPTQ / LDLQ lazy trailing update
    PT_GEMM_CHOL = 1,    // potrf panel + SYRK
    PT_GEMM_INV = 2,     // trtri + lauum
    PT_DIAG = 3,         // nb x nb diagonal factor + inverse
    PT_SWEEP = 4,        // GPTQ / LDLQ column sweep
    PT_ROTATE = 5,       // weight rotation
    PT_ROTATE_H = 6,     // two-sided Hessian rotation
    PT_RTN = 7,          // quantise / pack
    PT_GREEDY = 8,       // greedy block kernel + its cross-term GEMMs
    PT_OTHER = 9,
    PT_GEMM_GREEDY = 10, // greedy cross-term GEMMs
    PT_PANEL = 11,       // Cholesky panel solve (fp64 accumulation)
    PT_RTN_SCALES = 12,  // RTN scales / clipping-ratio search
    PT_VERIFY = 13,      // fp64 quantisation error
    PT_PERMUTE = 14,     // PermuQuant moments, sort, error scales, gathers
    PT_PERM_SUM = 15,    // PermuQuant acceptance error: ordered-sum block kernel
    PT_DLR = 16,         // Woodbury inverse: r x r products
    PT_DLR_GEMM = 17,    // Woodbury / dense DLR: the n x n product
    PT_PISO = 18,        // PiSO scale search
    PT_COUNT = 19,
};

bool prof_enabled();

// While alive, ProfScope records nothing on this thread (the allocation-free
// entry points: a recording scope creates HIP events).
class ProfSuppress {
public:
    ProfSuppress();
    ~ProfSuppress();
private:
    bool prev_;
};

class ProfScope {
public:
    ProfScope(hipStream_t st, int tag, double flops, double bytes);
    ~ProfScope();
private:
    hipStream_t st_;
    int idx_ = -1;
};

}  // namespace icq
