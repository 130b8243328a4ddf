// PermuQuant channel reordering on the GPU (converter/permuquant.py:13-211,
// used by converter/pipeline.py:572-615, 728-756, 1085-1087).
//
// The reference computes these steps with torch on the CPU, and two of them
// depend on the order in which torch adds fp32 values:
//   * the channel second moments mean(W^2, dim=0) (permuquant.py:13-23):
//     torch reduces each column with a four-level cascade of accumulators
//     (groups of S = 2^lp rows, lp = max(4, ceil(log2 rows) / 4)); columns
//     past the last whole 16-column vector of its AVX-512 loop take a scalar
//     loop with four interleaved accumulators (rows i = 4m + k);
//   * the acceptance error sum((W - dq)^2) (permuquant.py:72-111): a full
//     reduction that torch splits into one contiguous chunk per CPU thread
//     (ceil(n / threads) elements, at least 32768 per thread); inside a
//     chunk it keeps four interleaved 8-lane vector accumulators (element
//     32 m + 8 k + l goes to accumulator k, lane l), each a four-level
//     cascade, adds the leftover vectors to accumulator 0, merges the four,
//     and sums the leftover scalars and then the 8 lanes; the per-thread
//     results are summed again the same way.
// These orders were measured against torch 2.10 on the CPU bit for bit
// (1 to 16 threads, odd and even sizes).  The kernels below add in exactly
// that order, in parallel over the independent sub-sums of the cascade, so
// the moments, the permutation and the accept / reject decision equal the
// reference's when it runs with the same number of CPU threads.
//
// The permutation itself is a stable descending sort (ties by column
// index, NaN first, -0 equal to +0), a bitonic network on 64-bit keys.
#include <vector>

#include "common.hpp"
#include "prof.hpp"
#include "torchsum.hpp"

namespace icq {

// The value accumulator 1 holds when block b (S groups of S values) is
// done: the sequential sum of its S group sums.
template <typename Get>
__device__ __forceinline__ float cascade_block(Get get, int64_t b, int lp) {
    const int64_t S = int64_t(1) << lp;
    const int64_t i0 = b << (2 * lp);
    float a1 = 0.0f;
    for (int64_t g = 0; g < S; ++g) a1 = a1 + seq_sum(get, i0 + g * S, S);
    return a1;
}

// Sequential sum (from 0) of get(i0) .. get(i0 + n - 1): the values are
// loaded GB at a time before they are added, so their latencies overlap.
constexpr int GB = 16;
template <typename Get>
__device__ __forceinline__ float seq_sum(Get get, int64_t i0, int64_t n) {
    float a = 0.0f;
    int64_t i = 0;
    for (; i + GB <= n; i += GB) {
        float v[GB];
#pragma unroll
        for (int u = 0; u < GB; ++u) v[u] = get(i0 + i + u);
#pragma unroll
        for (int u = 0; u < GB; ++u) a = a + v[u];
    }
    for (; i < n; ++i) a = a + get(i0 + i);
    return a;
}

// The cascade of a sequence of L values from its whole-block values
// blk(0 .. L / S^2 - 1) and the values past the last whole block.
template <typename Blk, typename Get>
__device__ float cascade_finish(Blk blk, Get get, int64_t L, int lp) {
    const int64_t S = int64_t(1) << lp;
    const int64_t nb = L >> (2 * lp);
    float a2 = 0.0f, a3 = 0.0f;
    int64_t b = 0;
    for (; b + GB <= nb; b += GB) {
        float v[GB];
#pragma unroll
        for (int u = 0; u < GB; ++u) v[u] = blk(b + u);
#pragma unroll
        for (int u = 0; u < GB; ++u) {
            a2 = a2 + v[u];
            if (((b + u + 1) & (S - 1)) == 0) {
                a3 = a3 + a2;
                a2 = 0.0f;
            }
        }
    }
    for (; b < nb; ++b) {
        a2 = a2 + blk(b);
        if (((b + 1) & (S - 1)) == 0) {
            a3 = a3 + a2;
            a2 = 0.0f;
        }
    }
    int64_t i = nb << (2 * lp);
    float a1 = 0.0f;
    for (; i + S <= L; i += S) a1 = a1 + seq_sum(get, i, S);
    float a0 = seq_sum(get, i, L - i);
    a0 = a0 + a1;
    a0 = a0 + a2;
    a0 = a0 + a3;
    return a0;
}

// ------------------------------------------------------------ column moments

// Block values of the column cascades: thread (column j, block b).
__global__ void colmom_block_kernel(const float* W, int64_t rows, int64_t cols, int64_t ld, int lp, int64_t nb,
                                    float* B) {
    const int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t b = blockIdx.y;
    if (j >= cols || b >= nb) return;
    const float* col = W + j;
    auto get = [&](int64_t i) { const float w = col[i * ld]; return w * w; };
    B[b * cols + j] = cascade_block(get, b, lp);
}

// mu2[j] = (sum of W[:, j]^2 in torch's order) / rows.  Columns below
// tail_from finish the block cascade; the others take the scalar loop with
// four interleaved accumulators.
__global__ void colmom_finish_kernel(const float* W, int64_t rows, int64_t cols, int64_t ld, int lp, int64_t nb,
                                     const float* B, int64_t tail_from, float* mu2) {
    const int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= cols) return;
    const float* col = W + j;
    auto get = [&](int64_t i) { const float w = col[i * ld]; return w * w; };
    float s;
    if (j < tail_from) {
        auto blk = [&](int64_t b) { return B[b * cols + j]; };
        s = cascade_finish(blk, get, rows, lp);
    } else {
        const int64_t n4 = rows / 4;
        const int lp4 = cascade_lp(n4);
        float p[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            auto gk = [&](int64_t m) { return get(4 * m + k); };
            p[k] = cascade_seq(gk, n4, lp4);
        }
        for (int64_t i = 4 * n4; i < rows; ++i) p[0] = p[0] + get(i);
        s = ((p[0] + p[1]) + p[2]) + p[3];
    }
    mu2[j] = s / (float)rows;
}

// ------------------------------------------------------------ full sums

// Element access of the summed tensor: a plain fp32 array, or the squared
// RTN errors of a (column-permuted) matrix computed on the fly.  Both give
// element k of the logical row-major tensor; at(row, col) is the same for
// matrices, and the block kernel walks (row, col) incrementally.
struct ArraySrc {
    const float* x;
    int64_t cols;      // row length of the logical tensor (a vector: its length)
    __device__ __forceinline__ float at(int64_t r, int64_t c) const { return x[r * cols + c]; }
    __device__ __forceinline__ float operator()(int64_t k) const { return x[k]; }
};

// e = (w - q s)^2, w = W[r][perm[c]] (or W[r][c]), s the scale of its group,
// q = clamp(rhaz(w / s), qmin, qmax): the reference's dequantised error.
struct ErrSrc {
    const float* W;
    int64_t ld, cols, group;
    const int64_t* perm;
    const float* S;      // [rows, ngroups] scales
    int64_t ngroups;
    float qmin, qmax;
    __device__ __forceinline__ float at(int64_t r, int64_t c) const {
        const float w = W[r * ld + (perm ? perm[c] : c)];
        // 32-bit group index (cols < 2^31); one group per row needs none
        const int64_t gi = ngroups == 1 ? 0 : (int64_t)((uint32_t)c / (uint32_t)group);
        const float sc = S[r * ngroups + gi];
        const float q = clampf(rhaz(w / sc), qmin, qmax);
        const float d = w - q * sc;
        return d * d;
    }
    __device__ __forceinline__ float operator()(int64_t k) const { return at(k / cols, k % cols); }
};

// torch's contiguous inner sum of x[0 .. L), sequentially (small L).
template <typename Src>
__device__ float inner_sum_seq(const Src& x, int64_t L) {
    const int64_t vs = L / SUM_VEC;
    if (vs == 0) {
        // scalar loop: four interleaved accumulators
        const int64_t n4 = L / 4;
        const int lp = cascade_lp(n4);
        float p[4];
        for (int k = 0; k < 4; ++k) p[k] = cascade_seq([&](int64_t m) { return x(4 * m + k); }, n4, lp);
        for (int64_t i = 4 * n4; i < L; ++i) p[0] = p[0] + x(i);
        return ((p[0] + p[1]) + p[2]) + p[3];
    }
    const int64_t n4 = vs / 4;
    const int lp = cascade_lp(n4);
    float p[SUM_SEQ];
    for (int s = 0; s < SUM_SEQ; ++s) p[s] = cascade_seq([&](int64_t m) { return x(SUM_SEQ * m + s); }, n4, lp);
    float f = 0.0f;
    for (int l = 0; l < SUM_VEC; ++l) {
        float a = p[l];
        for (int64_t v = 4 * n4; v < vs; ++v) a = a + x(v * SUM_VEC + l);
        a = a + p[SUM_VEC + l];
        a = a + p[2 * SUM_VEC + l];
        a = a + p[3 * SUM_VEC + l];
        p[l] = a;
    }
    for (int64_t e = vs * SUM_VEC; e < L; ++e) f = f + x(e);
    for (int l = 0; l < SUM_VEC; ++l) f = f + p[l];
    return f;
}

struct SumPlan {
    int64_t n, chunk;     // elements, elements per chunk
    int nt, T;            // chunks used, CPU threads (buffer slots)
    bool single;          // one serial reduction, no per-thread buffer
};

static SumPlan sum_plan(int64_t n, int threads) {
    SumPlan p{};
    p.n = n;
    p.T = threads;
    p.single = n < TORCH_GRAIN || threads <= 1;
    if (p.single) {
        p.nt = 1;
        p.chunk = n;
    } else {
        p.nt = (int)std::min<int64_t>(threads, cdiv(n, TORCH_GRAIN));
        p.chunk = cdiv(n, p.nt);
    }
    return p;
}

// Block values of the 32 interleaved sequences of every chunk: thread
// (chunk t, block b, sequence s).  The sequence s of a chunk starting at
// c0 is x[c0 + 32 m + s], m < n4; its elements are visited with a running
// (row, column) of the logical tensor.
template <typename Src>
__global__ void fsum_block_kernel(Src x, SumPlan p, int64_t nbmax, float* B) {
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int t = blockIdx.y;
    const int s = (int)(gid % SUM_SEQ);
    const int64_t b = gid / SUM_SEQ;
    const int64_t c0 = (int64_t)t * p.chunk;
    const int64_t L = std::min(p.n, c0 + p.chunk) - c0;
    if (L <= 0) return;
    const int64_t n4 = (L / SUM_VEC) / 4;
    const int lp = cascade_lp(n4);
    if (b >= (n4 >> (2 * lp))) return;
    // element m of the sequence is k = k0 + 32 m: its (row, column) from the
    // block's first (r0, c0) with a division only when a row ends
    const int64_t k0 = c0 + (b << (2 * lp)) * SUM_SEQ + s;
    const int64_t r0 = k0 / x.cols, cc0 = k0 - r0 * x.cols;
    auto get = [&](int64_t m) {
        int64_t c = cc0 + (m - (b << (2 * lp))) * SUM_SEQ, r = r0;
        if (c >= x.cols) {
            r += c / x.cols;
            c -= (c / x.cols) * x.cols;
        }
        return x.at(r, c);
    };
    B[((int64_t)t * nbmax + b) * SUM_SEQ + s] = cascade_block(get, b, lp);
}

// The same block values with 2^LP times the parallelism: work-group (block
// b, chunk t), thread (sequence s, group g) sums the S = 2^LP values of group
// g in order, and thread (s, 0) adds the S group sums in order, which is
// the sequence of additions cascade_block makes.
template <typename Src, int LP>
__global__ __launch_bounds__(SUM_SEQ << LP) void fsum_group_kernel(Src x, SumPlan p, int64_t nbmax, float* B) {
    constexpr int S = 1 << LP;
    __shared__ float G[S][SUM_SEQ + 1];
    const int s = threadIdx.x % SUM_SEQ, g = threadIdx.x / SUM_SEQ;
    const int t = blockIdx.y;
    const int64_t b = blockIdx.x;
    const int64_t c0 = (int64_t)t * p.chunk;
    const int64_t L = std::min(p.n, c0 + p.chunk) - c0;
    if (L <= 0) return;                                  // uniform in the work-group
    const int64_t n4 = (L / SUM_VEC) / 4;
    if (b >= (n4 >> (2 * LP))) return;                   // uniform in the work-group
    const int64_t m0 = (b << (2 * LP)) + (int64_t)g * S;
    const int64_t k0 = c0 + m0 * SUM_SEQ + s;
    const int64_t r0 = k0 / x.cols, cc0 = k0 - r0 * x.cols;
    auto get = [&](int64_t m) {
        int64_t c = cc0 + (m - m0) * SUM_SEQ, r = r0;
        if (c >= x.cols) {
            r += c / x.cols;
            c -= (c / x.cols) * x.cols;
        }
        return x.at(r, c);
    };
    G[g][s] = seq_sum(get, m0, S);
    __syncthreads();
    if (g == 0) {
        float a1 = 0.0f;
        for (int q = 0; q < S; ++q) a1 = a1 + G[q][s];
        B[((int64_t)t * nbmax + b) * SUM_SEQ + s] = a1;
    }
}

// The cascade's log2 group size shared by every chunk of the plan, or -1.
static int common_lp(const SumPlan& p) {
    int lp = -1;
    for (int t = 0; t < p.nt; ++t) {
        const int64_t c0 = (int64_t)t * p.chunk;
        const int64_t L = std::min(p.n, c0 + p.chunk) - c0;
        if (L <= 0) continue;
        const int l = cascade_lp((L / SUM_VEC) / 4);
        if (lp >= 0 && l != lp) return -1;
        lp = l;
    }
    return lp;
}

// One work-group per chunk: the 32 sequence cascades from the block values,
// then the chunk's leftover vectors, the merge of the four accumulators,
// the leftover scalars and the lanes (thread 0).  Chunk results go to buf
// (0 + result, like torch's per-thread buffer) or, for a single chunk,
// straight to out.
template <typename Src>
__global__ void fsum_finish_kernel(Src x, SumPlan p, int64_t nbmax, const float* B, float* buf, float* out) {
    __shared__ float ps[SUM_SEQ];
    const int t = blockIdx.x;
    const int s = threadIdx.x;
    const int64_t c0 = (int64_t)t * p.chunk;
    const int64_t L = std::min(p.n, c0 + p.chunk) - c0;
    if (L <= 0) return;                                  // uniform in the work-group
    auto xc = [&](int64_t i) { return x(c0 + i); };
    const int64_t vs = L / SUM_VEC;
    if (vs < 64) {
        // a short chunk: the whole inner sum on one thread
        if (s == 0) {
            const float r = inner_sum_seq(xc, L);
            if (p.single) out[0] = 0.0f + r;
            else buf[t] = 0.0f + r;
        }
        return;
    }
    const int64_t n4 = vs / 4;
    const int lp = cascade_lp(n4);
    if (s < SUM_SEQ) {
        auto blk = [&](int64_t b) { return B[((int64_t)t * nbmax + b) * SUM_SEQ + s]; };
        ps[s] = cascade_finish(blk, [&](int64_t m) { return xc(SUM_SEQ * m + s); }, n4, lp);
    }
    __syncthreads();
    if (s == 0) {
        float f = 0.0f;
        float lanes[SUM_VEC];
        for (int l = 0; l < SUM_VEC; ++l) {
            float a = ps[l];
            for (int64_t v = 4 * n4; v < vs; ++v) a = a + xc(v * SUM_VEC + l);
            a = a + ps[SUM_VEC + l];
            a = a + ps[2 * SUM_VEC + l];
            a = a + ps[3 * SUM_VEC + l];
            lanes[l] = a;
        }
        for (int64_t e = vs * SUM_VEC; e < L; ++e) f = f + xc(e);
        for (int l = 0; l < SUM_VEC; ++l) f = f + lanes[l];
        if (p.single) out[0] = 0.0f + f;
        else buf[t] = 0.0f + f;
    }
}

// The per-thread buffer (T slots, unused ones 0) summed like any tensor.
__global__ void fsum_buffer_kernel(const float* buf, int T, float* out) {
    if (threadIdx.x == 0 && blockIdx.x == 0) out[0] = 0.0f + inner_sum_seq(ArraySrc{buf, 1}, T);
}

// Most whole blocks of any chunk (a shorter last chunk can have a smaller
// group size and so more blocks).
static int64_t fsum_nbmax(const SumPlan& p) {
    int64_t most = 0;
    for (int t = 0; t < p.nt; ++t) {
        const int64_t c0 = (int64_t)t * p.chunk;
        const int64_t L = std::min(p.n, c0 + p.chunk) - c0;
        if (L <= 0) continue;
        const int64_t n4 = (L / SUM_VEC) / 4;
        most = std::max(most, n4 >> (2 * cascade_lp(n4)));
    }
    return most;
}

// out[0] = torch.sum(x[0 .. n)) as torch on the CPU with `threads` threads.
// ws: fsum_ws_floats(n, threads) floats.
static int64_t fsum_ws_floats(int64_t n, int threads) {
    const SumPlan p = sum_plan(n, threads);
    return (int64_t)p.nt * std::max<int64_t>(fsum_nbmax(p), 1) * SUM_SEQ + std::max(threads, 1) + 64;
}

template <typename Src>
static int torch_sum(const Src& x, int64_t n, int threads, float* out, float* ws, hipStream_t st) {
    const SumPlan p = sum_plan(n, threads);
    const int64_t nbmax = fsum_nbmax(p);
    float* B = ws;
    float* buf = ws + (int64_t)p.nt * std::max<int64_t>(nbmax, 1) * SUM_SEQ;
    if (!p.single) IC_CHECK_HIP(hipMemsetAsync(buf, 0, (size_t)p.T * sizeof(float), st));
    if (nbmax > 0) {
        const int64_t per = nbmax * SUM_SEQ;
        ProfScope prof_scope(st, PT_PERM_SUM, (double)n, 4.0 * n);
        const int lp = common_lp(p);
        if (lp == 4) {
            hipLaunchKernelGGL((fsum_group_kernel<Src, 4>), dim3((unsigned)nbmax, (unsigned)p.nt), dim3(SUM_SEQ << 4),
                               0, st, x, p, nbmax, B);
        } else if (lp == 5) {
            hipLaunchKernelGGL((fsum_group_kernel<Src, 5>), dim3((unsigned)nbmax, (unsigned)p.nt), dim3(SUM_SEQ << 5),
                               0, st, x, p, nbmax, B);
        } else {
            hipLaunchKernelGGL(fsum_block_kernel<Src>, dim3((unsigned)cdiv(per, 256), (unsigned)p.nt), dim3(256), 0,
                               st, x, p, nbmax, B);
        }
        IC_CHECK_LAUNCH();
    }
    hipLaunchKernelGGL(fsum_finish_kernel<Src>, dim3((unsigned)p.nt), dim3(64), 0, st, x, p,
                       std::max<int64_t>(nbmax, 1), B, buf, out);
    IC_CHECK_LAUNCH();
    if (!p.single) {
        hipLaunchKernelGGL(fsum_buffer_kernel, dim3(1), dim3(64), 0, st, buf, p.T, out);
        IC_CHECK_LAUNCH();
    }
    return IC_OK;
}

// ------------------------------------------------------------ group error

// Symmetric RTN scale of every (row, group) of the (column-permuted)
// matrix: fp16(clamp(amax / div, 1e-5, 65500)), kept as its fp32 value.
// Columns past `cols` in the last group are the reference's zero padding.
__global__ void perm_scales_kernel(const float* W, int64_t cols, int64_t ld, const int64_t* perm, int64_t group,
                                   float div, float* S, int64_t ngroups) {
    const int64_t r = blockIdx.x, g = blockIdx.y;    // rows on x (up to 2^31), groups on y
    const float* row = W + r * ld;
    float m = 0.0f;
    const int64_t j1 = std::min(cols, (g + 1) * group);
    for (int64_t j = g * group + threadIdx.x; j < j1; j += blockDim.x) {
        const int64_t c = perm ? perm[j] : j;
        m = fmaxf(m, fabsf(row[c]));
    }
    m = wave_max(m);
    __shared__ float part[16];
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < (int)(blockDim.x >> 6); ++w) m = fmaxf(m, part[w]);
        S[r * ngroups + g] = f16_bits_to_f32(f32_to_f16_bits(clampf(m / div, 1e-5f, 65500.0f)));
    }
}

// ------------------------------------------------------------ sort

constexpr int SORT_TILE = 2048;           // keys sorted in LDS by one work-group (one pair per thread)
constexpr int SORT_THREADS = 1024;

__device__ __forceinline__ uint64_t desc_key(float v, int64_t i) {
    if (v != v) v = __uint_as_float(0x7fc00000u);        // every NaN first
    if (v == 0.0f) v = 0.0f;                             // -0 == +0
    const uint32_t k = ~float_key(v);
    return ((uint64_t)k << 32) | (uint64_t)(uint32_t)i;
}

__global__ void sort_keys_kernel(const float* v, int64_t n, int64_t P, uint64_t* keys) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < P) keys[i] = i < n ? desc_key(v[i], i) : ~uint64_t(0);
}

__device__ __forceinline__ void cmp_swap(uint64_t& a, uint64_t& b, bool up) {
    if ((a > b) == up) {
        const uint64_t t = a;
        a = b;
        b = t;
    }
}

// Bitonic steps on one tile of `len` keys (a power of 2 <= SORT_TILE) at
// keys + base: either the whole sort up to kmax = len (kfix == 0), or the
// steps j < len of the merge with k = kfix.  Directions use the global
// index, so tiles compose into the global network.
__global__ __launch_bounds__(SORT_THREADS) void sort_tile_kernel(uint64_t* keys, int64_t len, int64_t kfix) {
    __shared__ uint64_t sk[SORT_TILE];
    const int64_t base = (int64_t)blockIdx.x * len;
    for (int64_t i = threadIdx.x; i < len; i += blockDim.x) sk[i] = keys[base + i];
    __syncthreads();
    const int64_t k0 = kfix ? kfix : 2, k1 = kfix ? kfix : len;
    for (int64_t k = k0; k <= k1; k <<= 1) {
        for (int64_t j = std::min(k >> 1, len >> 1); j > 0; j >>= 1) {
            for (int64_t q = threadIdx.x; q < len / 2; q += blockDim.x) {
                const int64_t i = 2 * q - (q & (j - 1));     // i has bit j clear
                const int64_t l = i + j;
                const bool up = ((base + i) & k) == 0;
                uint64_t a = sk[i], b = sk[l];
                cmp_swap(a, b, up);
                sk[i] = a;
                sk[l] = b;
            }
            __syncthreads();
        }
    }
    for (int64_t i = threadIdx.x; i < len; i += blockDim.x) keys[base + i] = sk[i];
}

// One global bitonic step (k, j) with j >= SORT_TILE.
__global__ void sort_step_kernel(uint64_t* keys, int64_t P, int64_t k, int64_t j) {
    const int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (q >= P / 2) return;
    const int64_t i = 2 * q - (q & (j - 1));
    const int64_t l = i + j;
    uint64_t a = keys[i], b = keys[l];
    cmp_swap(a, b, (i & k) == 0);
    keys[i] = a;
    keys[l] = b;
}

__global__ void sort_index_kernel(const uint64_t* keys, int64_t n, int64_t* perm) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) perm[i] = (int64_t)(keys[i] & 0xffffffffu);
}

static int64_t pow2_at_least(int64_t n) {
    int64_t p = 1;
    while (p < n) p <<= 1;
    return p;
}

static int argsort_desc(const float* v, int64_t n, int64_t* perm, uint64_t* keys, hipStream_t st) {
    const int64_t P = std::max<int64_t>(pow2_at_least(n), 2);
    hipLaunchKernelGGL(sort_keys_kernel, dim3((unsigned)cdiv(P, 256)), dim3(256), 0, st, v, n, P, keys);
    IC_CHECK_LAUNCH();
    const int64_t tile = std::min<int64_t>(P, SORT_TILE);
    hipLaunchKernelGGL(sort_tile_kernel, dim3((unsigned)(P / tile)), dim3(SORT_THREADS), 0, st, keys, tile,
                       (int64_t)0);
    IC_CHECK_LAUNCH();
    for (int64_t k = 2 * tile; k <= P; k <<= 1) {
        for (int64_t j = k >> 1; j >= tile; j >>= 1) {
            hipLaunchKernelGGL(sort_step_kernel, dim3((unsigned)cdiv(P / 2, 256)), dim3(256), 0, st, keys, P, k, j);
            IC_CHECK_LAUNCH();
        }
        hipLaunchKernelGGL(sort_tile_kernel, dim3((unsigned)(P / tile)), dim3(SORT_THREADS), 0, st, keys, tile, k);
        IC_CHECK_LAUNCH();
    }
    hipLaunchKernelGGL(sort_index_kernel, dim3((unsigned)cdiv(n, 256)), dim3(256), 0, st, keys, n, perm);
    IC_CHECK_LAUNCH();
    return IC_OK;
}

// ------------------------------------------------------------ gathers

constexpr int ROW_LDS = 16384;     // floats of a row staged in LDS by permute_cols_lds_kernel

// dst[r][j] = src[r][perm[j]] with the row staged in LDS (src_cols <=
// ROW_LDS): coalesced reads and writes, the gather inside LDS.
__global__ __launch_bounds__(1024) void permute_cols_lds_kernel(const float* src, int64_t src_cols, int64_t lds,
                                                                const int64_t* perm, int64_t np, float* dst,
                                                                int64_t ldd) {
    __shared__ float row[ROW_LDS];
    const int64_t r = blockIdx.x;
    for (int64_t j = threadIdx.x; j < src_cols; j += blockDim.x) row[j] = src[r * lds + j];
    __syncthreads();
    for (int64_t j = threadIdx.x; j < np; j += blockDim.x) {
        const int64_t c = perm[j];
        dst[r * ldd + j] = (c >= 0 && c < src_cols) ? row[c] : 0.0f;
    }
}

// dst[r][j] = src[r][perm[j]] for j < np; indices outside [0, src_cols)
// are not read (their outputs are 0).
__global__ void permute_cols_kernel(const float* src, int64_t rows, int64_t src_cols, int64_t lds, const int64_t* perm,
                                    int64_t np, float* dst, int64_t ldd) {
    const int64_t r = blockIdx.x;
    for (int64_t j = (int64_t)blockIdx.y * blockDim.x + threadIdx.x; j < np; j += (int64_t)gridDim.y * blockDim.x) {
        const int64_t c = perm[j];
        dst[r * ldd + j] = (c >= 0 && c < src_cols) ? src[r * lds + c] : 0.0f;
    }
}

// out[i][j] = H[perm[i]][perm[j]] for i, j < np (same index rule).
__global__ void permute_sym_kernel(const float* H, int64_t n, int64_t ldh, const int64_t* perm, int64_t np,
                                   float* out, int64_t ldo) {
    const int64_t i = blockIdx.x;
    const int64_t pi = perm[i];
    const bool ok_i = pi >= 0 && pi < n;
    for (int64_t j = (int64_t)blockIdx.y * blockDim.x + threadIdx.x; j < np; j += (int64_t)gridDim.y * blockDim.x) {
        const int64_t pj = perm[j];
        out[i * ldo + j] = (ok_i && pj >= 0 && pj < n) ? H[pi * ldh + pj] : 0.0f;
    }
}

}  // namespace icq

using namespace icq;

extern "C" int64_t ic_col_moments_workspace_bytes(int64_t rows, int64_t cols) {
    const int64_t nb = rows >> (2 * cascade_lp(rows));
    return (std::max<int64_t>(nb, 1) * cols) * (int64_t)sizeof(float) + 256;
}

extern "C" int ic_col_moments(const float* W, int64_t rows, int64_t cols, int64_t ld, int cpu_vec, float* mu2,
                              void* workspace, void* stream) {
    IC_REQUIRE(W && mu2 && workspace, "ic_col_moments: null pointer");
    IC_REQUIRE(rows >= 1 && cols >= 0 && ld >= cols, "ic_col_moments: bad size");
    IC_REQUIRE(cpu_vec == 8 || cpu_vec == 16, "ic_col_moments: cpu_vec must be 8 or 16");
    if (cols == 0) return IC_OK;
    hipStream_t st = as_stream(stream);
    ProfScope prof_scope(st, PT_PERMUTE, 2.0 * rows * cols, 4.0 * rows * cols);
    const int lp = cascade_lp(rows);
    const int64_t nb = rows >> (2 * lp);
    float* B = reinterpret_cast<float*>(workspace);
    if (nb > 0) {
        hipLaunchKernelGGL(colmom_block_kernel, dim3((unsigned)cdiv(cols, 64), (unsigned)nb), dim3(64), 0, st, W,
                           rows, cols, ld, lp, nb, B);
        IC_CHECK_LAUNCH();
    }
    const int64_t tail_from = cols - cols % cpu_vec;
    hipLaunchKernelGGL(colmom_finish_kernel, dim3((unsigned)cdiv(cols, 64)), dim3(64), 0, st, W, rows, cols, ld, lp,
                       nb, B, tail_from, mu2);
    IC_CHECK_LAUNCH();
    return IC_OK;
}

extern "C" int64_t ic_argsort_workspace_bytes(int64_t n) {
    return std::max<int64_t>(pow2_at_least(n), 2) * (int64_t)sizeof(uint64_t) + 256;
}

extern "C" int ic_argsort_desc(const float* v, int64_t n, int64_t* perm, void* workspace, void* stream) {
    IC_REQUIRE(v && perm && workspace, "ic_argsort_desc: null pointer");
    IC_REQUIRE(n >= 0 && n <= (int64_t(1) << 31), "ic_argsort_desc: n out of range");
    if (n == 0) return IC_OK;
    hipStream_t st = as_stream(stream);
    ProfScope prof_scope(st, PT_PERMUTE, 0.0, 8.0 * n);
    return argsort_desc(v, n, perm, reinterpret_cast<uint64_t*>(workspace), st);
}

extern "C" int64_t ic_group_quant_error_workspace_bytes(int64_t rows, int64_t cols, int64_t group, int bits,
                                                        int threads) {
    const int64_t g = bits == 8 ? cols : std::max<int64_t>(group, 1);
    const int64_t ngroups = std::max<int64_t>(cdiv(cols, g), 1);
    const int64_t n = rows * cols;
    return (rows * ngroups + fsum_ws_floats(n, std::max(threads, 1))) * (int64_t)sizeof(float) + 512;
}

extern "C" int ic_group_quant_error(const float* W, int64_t rows, int64_t cols, int64_t ld, const int64_t* perm,
                                    int64_t group, int bits, int threads, float* out, void* workspace, void* stream) {
    IC_REQUIRE(W && out && workspace, "ic_group_quant_error: null pointer");
    IC_REQUIRE(bits == 4 || bits == 8, "ic_group_quant_error: bits must be 4 or 8");
    IC_REQUIRE(rows >= 0 && cols >= 0 && ld >= cols, "ic_group_quant_error: bad size");
    IC_REQUIRE(bits == 8 || group >= 1, "ic_group_quant_error: group must be >= 1");
    IC_REQUIRE(threads >= 1 && threads <= 4096, "ic_group_quant_error: threads must be in [1, 4096]");
    hipStream_t st = as_stream(stream);
    if (rows == 0 || cols == 0) {
        IC_CHECK_HIP(hipMemsetAsync(out, 0, sizeof(float), st));
        return IC_OK;
    }
    const int64_t n = rows * cols;
    const int64_t g = bits == 8 ? cols : group;
    const int64_t ngroups = cdiv(cols, g);
    float* S = reinterpret_cast<float*>(workspace);
    float* sws = S + rows * ngroups;
    const float div = bits == 8 ? 127.0f : 7.0f;
    const float qmin = bits == 8 ? -128.0f : -8.0f, qmax = bits == 8 ? 127.0f : 7.0f;
    IC_REQUIRE(rows <= 0x7fffffff && cols <= 0x7fffffff && ngroups <= 65535,
               "ic_group_quant_error: too many rows, columns or groups");
    {
        // one group per row: its amax does not depend on the column order
        ProfScope prof_scope(st, PT_PERMUTE, 0.0, 4.0 * n);
        hipLaunchKernelGGL(perm_scales_kernel, dim3((unsigned)rows, (unsigned)ngroups), dim3(256), 0, st, W, cols,
                           ld, ngroups == 1 ? nullptr : perm, g, div, S, ngroups);
        IC_CHECK_LAUNCH();
    }
    const ErrSrc src{W, ld, cols, g, perm, S, ngroups, qmin, qmax};
    return torch_sum(src, n, threads, out, sws, st);
}

extern "C" int ic_torch_sum(const float* x, int64_t n, int threads, float* out, void* workspace, void* stream) {
    IC_REQUIRE(x && out && workspace, "ic_torch_sum: null pointer");
    IC_REQUIRE(n >= 0 && threads >= 1 && threads <= 4096, "ic_torch_sum: bad size");
    hipStream_t st = as_stream(stream);
    if (n == 0) {
        IC_CHECK_HIP(hipMemsetAsync(out, 0, sizeof(float), st));
        return IC_OK;
    }
    // one logical row: the block kernel's running column rarely wraps
    return torch_sum(ArraySrc{x, n}, n, threads, out, reinterpret_cast<float*>(workspace), st);
}

extern "C" int64_t ic_torch_sum_workspace_bytes(int64_t n, int threads) {
    return fsum_ws_floats(n, std::max(threads, 1)) * (int64_t)sizeof(float) + 256;
}

extern "C" int ic_permute_cols(const float* src, int64_t rows, int64_t src_cols, int64_t ld_src, const int64_t* perm,
                               int64_t n_perm, float* dst, int64_t ld_dst, void* stream) {
    IC_REQUIRE(src && perm && dst, "ic_permute_cols: null pointer");
    IC_REQUIRE(rows >= 0 && n_perm >= 0 && ld_src >= src_cols && ld_dst >= n_perm, "ic_permute_cols: bad size");
    IC_REQUIRE(rows <= 0x7fffffff, "ic_permute_cols: too many rows");
    if (rows == 0 || n_perm == 0) return IC_OK;
    hipStream_t st = as_stream(stream);
    ProfScope prof_scope(st, PT_PERMUTE, 0.0, 8.0 * rows * n_perm);
    if (src_cols <= ROW_LDS) {
        hipLaunchKernelGGL(permute_cols_lds_kernel, dim3((unsigned)rows), dim3(1024), 0, st, src, src_cols, ld_src, perm,
                           n_perm, dst, ld_dst);
    } else {
        const unsigned gy = (unsigned)std::min<int64_t>(cdiv(n_perm, 256), 64);
        hipLaunchKernelGGL(permute_cols_kernel, dim3((unsigned)rows, gy), dim3(256), 0, st, src, rows, src_cols,
                           ld_src, perm, n_perm, dst, ld_dst);
    }
    IC_CHECK_LAUNCH();
    return IC_OK;
}

extern "C" int ic_permute_sym(const float* H, int64_t n, int64_t ld, const int64_t* perm, int64_t n_perm, float* out,
                              int64_t ld_out, void* stream) {
    IC_REQUIRE(H && perm && out, "ic_permute_sym: null pointer");
    IC_REQUIRE(n >= 0 && n_perm >= 0 && ld >= n && ld_out >= n_perm, "ic_permute_sym: bad size");
    IC_REQUIRE(n_perm <= 0x7fffffff, "ic_permute_sym: too large");
    if (n_perm == 0) return IC_OK;
    hipStream_t st = as_stream(stream);
    ProfScope prof_scope(st, PT_PERMUTE, 0.0, 8.0 * n_perm * n_perm);
    const unsigned gy = (unsigned)std::min<int64_t>(cdiv(n_perm, 256), 64);
    hipLaunchKernelGGL(permute_sym_kernel, dim3((unsigned)n_perm, gy), dim3(256), 0, st, H, n, ld, perm, n_perm, out,
                       ld_out);
    IC_CHECK_LAUNCH();
    return IC_OK;
}
