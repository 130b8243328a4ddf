// Blocked fp32 Cholesky and triangular inverse of chol.hip, for reuse by
// other kernels' drivers (the orthonormalisation of lowrank.hip).
#pragma once

#include "gemm.hpp"

namespace icq {

// floats of a workspace region for `batch` matrices of order n; the fp64
// Dinv blocks follow it at dinv64_of(dinv, batch, n).
int64_t dinv_floats(int64_t batch, int64_t n);
double* dinv64_of(float* dinv, int64_t batch, int64_t n);

// Lower Cholesky in place of `batch` matrices [n, n] (pitch ld, stride sH);
// info[b] receives the 1-based column of the first non-positive pivot (or
// stays as it was).  The strict upper triangle is left as it was, except in
// the 128 x 128 diagonal blocks (zeroed).
int potrf(float* H, int64_t batch, int64_t n, int64_t ld, int64_t sH, double* dinv64, int* info, hipStream_t st);

// X = L^-1 from potrf's L and fp64 Dinv blocks (rounded to fp32 on the
// diagonal of X): the lower triangle of X is exact, its strict upper
// triangle outside the diagonal blocks is scratch.
int trtri(const float* L, float* X, int64_t batch, int64_t n, int64_t ld, int64_t sH, const double* dinv64,
          hipStream_t st);

}  // namespace icq
