// torch's CPU summation order for fp32 (torch 2.10, AVX-512 build), shared
// by the kernels that must reproduce the reference's CPU sums bit for bit.
#pragma once

#include "common.hpp"

namespace icq {

constexpr int64_t TORCH_GRAIN = 32768;   // at::internal::GRAIN_SIZE
constexpr int COL_VEC = 16;              // columns per vector in torch's outer-sum loop
constexpr int SUM_VEC = 8;               // lanes of the inner-sum vector accumulators
constexpr int SUM_SEQ = 4 * SUM_VEC;     // interleaved sequences of one chunk

__host__ __device__ inline int ceil_log2(int64_t x) {
    int r = 0;
    while ((int64_t(1) << r) < x) ++r;
    return r;
}
// log2 of the cascade's group size for a sequence of L values
__host__ __device__ inline int cascade_lp(int64_t L) {
    const int c = ceil_log2(L) / 4;
    return c > 4 ? c : 4;
}

// Sequential cascade of torch's multi_row_sum over get(0) .. get(L-1):
// accumulator 0 takes groups of S values, each group is added to
// accumulator 1, and every S groups accumulator 1 goes to 2, every S^2
// groups 2 goes to 3; the rest of the values go to 0; the result is
// ((a0 + a1) + a2) + a3.
template <typename Get>
__device__ float cascade_seq(Get get, int64_t L, int lp) {
    const int64_t S = int64_t(1) << lp, mask = S - 1;
    float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
    int64_t i = 0;
    while (i + S <= L) {
        // S >= 16: the values of a group are fetched four at a time
#pragma unroll 4
        for (int64_t j = 0; j < S; ++j, ++i) a0 = a0 + get(i);
        a1 = a1 + a0;
        a0 = 0.0f;
        if ((i & (mask << lp)) == 0) {
            a2 = a2 + a1;
            a1 = 0.0f;
            if ((i & (mask << (2 * lp))) == 0) {
                a3 = a3 + a2;
                a2 = 0.0f;
            }
        }
    }
    for (; i < L; ++i) a0 = a0 + get(i);
    a0 = a0 + a1;
    a0 = a0 + a2;
    a0 = a0 + a3;
    return a0;
}

// cascade_seq for K sequences at once that share their positions:
// get(i, e) fills e[k] with value i of sequence k; out[k] = sequence k's sum.
template <int K, typename Get>
__device__ __forceinline__ void cascade_seq_k(Get get, int64_t L, int lp, float (&out)[K]) {
    const int64_t S = int64_t(1) << lp, mask = S - 1;
    float a0[K], a1[K], a2[K], a3[K];
#pragma unroll
    for (int k = 0; k < K; ++k) a0[k] = a1[k] = a2[k] = a3[k] = 0.0f;
    int64_t i = 0;
    while (i + S <= L) {
        for (int64_t j = 0; j < S; ++j, ++i) {
            float e[K];
            get(i, e);
#pragma unroll
            for (int k = 0; k < K; ++k) a0[k] = a0[k] + e[k];
        }
#pragma unroll
        for (int k = 0; k < K; ++k) {
            a1[k] = a1[k] + a0[k];
            a0[k] = 0.0f;
        }
        if ((i & (mask << lp)) == 0) {
#pragma unroll
            for (int k = 0; k < K; ++k) {
                a2[k] = a2[k] + a1[k];
                a1[k] = 0.0f;
            }
            if ((i & (mask << (2 * lp))) == 0) {
#pragma unroll
                for (int k = 0; k < K; ++k) {
                    a3[k] = a3[k] + a2[k];
                    a2[k] = 0.0f;
                }
            }
        }
    }
    for (; i < L; ++i) {
        float e[K];
        get(i, e);
#pragma unroll
        for (int k = 0; k < K; ++k) a0[k] = a0[k] + e[k];
    }
#pragma unroll
    for (int k = 0; k < K; ++k) {
        float r = a0[k] + a1[k];
        r = r + a2[k];
        out[k] = r + a3[k];
    }
}

// The end of torch's contiguous inner sum of x(0 .. L - 1), L >= SUM_VEC:
// p[s] (s < SUM_SEQ) is the cascade of sequence s (values SUM_SEQ m + s,
// m < L / SUM_SEQ); the leftover vectors, the merge, the leftover scalars
// and the lanes follow here in torch's order.
template <typename X>
__device__ float inner_sum_finish(const float* p, X x, int64_t L) {
    const int64_t vs = L / SUM_VEC, n4 = vs / 4;
    float pl[SUM_VEC];
    for (int l = 0; l < SUM_VEC; ++l) {
        float a = p[l];
        for (int64_t v = 4 * n4; v < vs; ++v) a = a + x(v * SUM_VEC + l);
        a = a + p[SUM_VEC + l];
        a = a + p[2 * SUM_VEC + l];
        a = a + p[3 * SUM_VEC + l];
        pl[l] = a;
    }
    float f = 0.0f;
    for (int64_t e = vs * SUM_VEC; e < L; ++e) f = f + x(e);
    for (int l = 0; l < SUM_VEC; ++l) f = f + pl[l];
    return f;
}

// torch's inner sum of L < SUM_VEC values: its scalar loop, four interleaved
// accumulators.
template <typename X>
__device__ float inner_sum_short(X x, int64_t L) {
    const int64_t n4 = L / 4;
    const int lp = cascade_lp(n4);
    float p[4];
    for (int k = 0; k < 4; ++k) p[k] = cascade_seq([&](int64_t m) { return x(4 * m + k); }, n4, lp);
    for (int64_t i = 4 * n4; i < L; ++i) p[0] = p[0] + x(i);
    return ((p[0] + p[1]) + p[2]) + p[3];
}

// ---------------------------------------------------------------- row_sum
// torch's scalar reduction of L values x(0 .. L - 1) (a strided or short
// row: the diagonal of a matrix, H.diagonal().sum() below the parallel grain
// size): four interleaved sequences x(4 m + k), m < L / 4, each a cascade
// with group size S = 2^cascade_lp(L / 4); the last L mod 4 values go to
// sequence 0; the result is ((p0 + p1) + p2) + p3.  The whole-block values
// of the cascades (S groups of S values each) are independent, so a
// work-group computes them in parallel and then finishes each sequence in
// the cascade's own order.

// The value the cascade's second accumulator holds after block b of a
// sequence get(0 ..): the sum from 0 of its S group sums.
template <typename Get>
__device__ float rs_block(Get get, int64_t b, int lp) {
    const int64_t S = int64_t(1) << lp, i0 = b << (2 * lp);
    float a1 = 0.0f;
    for (int64_t g = 0; g < S; ++g) {
        float a0 = 0.0f;
        for (int64_t j = 0; j < S; ++j) a0 = a0 + get(i0 + g * S + j);
        a1 = a1 + a0;
    }
    return a1;
}

// The cascade of a sequence of L values given its whole-block values
// blk(0 .. L / S^2 - 1): the blocks into the third accumulator (flushed to
// the fourth every S blocks), then the values after the last whole block.
template <typename Blk, typename Get>
__device__ float rs_finish(Blk blk, Get get, int64_t L, int lp) {
    const int64_t S = int64_t(1) << lp;
    const int64_t nb = L >> (2 * lp);
    float a2 = 0.0f, a3 = 0.0f;
    for (int64_t b = 0; b < nb; ++b) {
        a2 = a2 + blk(b);
        if (((b + 1) & (S - 1)) == 0) {
            a3 = a3 + a2;
            a2 = 0.0f;
        }
    }
    int64_t i = nb << (2 * lp);
    float a1 = 0.0f;
    for (; i + S <= L; i += S) {
        float a0 = 0.0f;
        for (int64_t j = 0; j < S; ++j) a0 = a0 + get(i + j);
        a1 = a1 + a0;
    }
    float a0 = 0.0f;
    for (; i < L; ++i) a0 = a0 + get(i);
    a0 = a0 + a1;
    a0 = a0 + a2;
    return a0 + a3;
}

// row_sum of x(0 .. L - 1) by the threads of a work-group (all of them must
// call it); blk: LDS scratch of RS_MAX_BLOCKS floats.  Every thread gets the
// result.
constexpr int RS_MAX_BLOCKS = 256;
template <typename X>
__device__ float row_sum_wg(X x, int64_t L, float* blk, float* part) {
    const int t = threadIdx.x, nt = blockDim.x;
    const int64_t n4 = L / 4;
    const int lp = cascade_lp(n4);
    const int64_t nb = n4 >> (2 * lp);
    const bool blocked = 4 * nb <= RS_MAX_BLOCKS;
    if (blocked) {
        for (int64_t u = t; u < 4 * nb; u += nt) {
            const int k = (int)(u & 3);
            const int64_t b = u >> 2;
            blk[u] = rs_block([&](int64_t m) { return x(4 * m + k); }, b, lp);
        }
    }
    __syncthreads();
    if (t < 4) {
        const int k = t;
        auto get = [&](int64_t m) { return x(4 * m + k); };
        part[k] = blocked ? rs_finish([&](int64_t b) { return blk[4 * b + k]; }, get, n4, lp)
                          : cascade_seq(get, n4, lp);
    }
    __syncthreads();
    float p0 = part[0];
    for (int64_t i = 4 * n4; i < L; ++i) p0 = p0 + x(i);
    const float r = ((p0 + part[1]) + part[2]) + part[3];
    __syncthreads();   // part[] may be reused by the caller
    return r;
}

}  // namespace icq
