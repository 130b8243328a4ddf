// fp32 MFMA GEMM used by the Hessian inverse and the GPTQ / LDLQ lazy
// trailing updates.  C = alpha * op(A) op(B) + beta * C, row-major.
#pragma once

#include "common.hpp"
#include "prof.hpp"

namespace icq {

enum CMask : int {
    CMASK_FULL = 0,
    CMASK_LOWER = 1,   // only elements i >= j are computed / stored
    CMASK_UPPER = 2,   // only elements i <= j
};

enum KRange : int {
    KR_FULL = 0,
    KR_FROM_MAXIJ = 1,   // k in [max(tile_i0, tile_j0), K): C = X^T X with X lower
    KR_FROM_J = 2,       // k in [tile_j0, K): op(B) lower (B[k][j] = 0 for k < j)
    KR_TO_I = 3,         // k in [0, tile_i0 + BM): op(A) lower (A[i][k] = 0 for k > i)
    KR_FROM_I = 4,       // k in [tile_i0, K): op(A) upper (A[i][k] = 0 for k < i)
};

struct GemmArgs {
    int64_t M, N, K;
    float alpha, beta;
    const float* A; int64_t lda; int64_t sA;   // sA: batch stride (elements)
    const float* B; int64_t ldb; int64_t sB;
    float* C; int64_t ldc; int64_t sC;
    int transA, transB;
    int cmask, krange;
    int64_t batch;
    int tag = PT_OTHER;        // profiler phase
    double algo_flops = 0.0;   // algorithmic flops of the launch (0: 2*M*N*K*batch)
    int kc = 128;              // accumulation chunk along K: a power of two, at least 32
    // 1: C <- (..((C - P_0) - P_1)..) - P_last, chunk by chunk (alpha = -1,
    // beta = 1, op(A) = A), the roundings of consecutive rank-kc updates; C
    // is held in registers through the K loop.  0: C <- alpha * sum + beta * C.
    int chunk_sub = 0;
    // Where the old C is read (same pitch and batch stride as C); null: C.
    // Lets a first update read pristine weights and write a separate buffer.
    const float* Cin = nullptr;
};

// Launches on `st`; returns IC_OK or an error code.  Safe in place (C aliases
// op(B)) when one output tile row spans all of M (M <= 128) and each tile
// only reads the columns it writes, because a tile reads all of its K range
// before its epilogue stores.
int gemm_f32(const GemmArgs& g, hipStream_t st);

}  // namespace icq
