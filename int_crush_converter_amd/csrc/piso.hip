// PiSO per-row scale search (converter/piso.py:28-183, the reference's
// PyTorch path).  For each row w of W and the Hessian diagonal h, the
// weighted quantisation error
//   E(s) = sum_d ((w_d - dq(w_d; s))^2 * h_d)
// is evaluated for the scales s_ref * coarse[c] (c < nc); the first minimum
// (torch argmin) picks s_best; then for s_best * fine[f] (f < nf), whose
// first minimum is the result.  Symmetric: s_ref = max(absmax / qmax, 1e-10),
// q = clamp(rhaz(w / s)), dq = q s.  Asymmetric: s_ref = max((max - min) /
// (qmax - qmin), 1e-10), every candidate clamped at 1e-10, zp = clamp(rhaz(
// qmin - min / s)), q = clamp(rhaz(w / s + zp)), dq = (q - zp) s.
//
// The reference sums E over d with torch's CPU inner-sum order (one thread
// per output row of its [rows, candidates, d] tensor); the kernel adds in
// the same order, so the chosen candidate, scale and zero-point are the
// reference's bit for bit.  A work-group takes one row: the row and h are
// staged in LDS, 32 lanes take the 32 interleaved sequences of one
// candidate's sum (up to 4 candidates per lane share the loads), one lane
// per candidate finishes the sum.
#include <algorithm>

#include "prof.hpp"
#include "torchsum.hpp"

namespace icq {
namespace {

constexpr int PISO_THREADS = 1024;
constexpr int PISO_GROUPS = PISO_THREADS / SUM_SEQ;   // candidate groups of 32 lanes
constexpr int PISO_MAXK = 4;                           // candidates per lane
constexpr int PISO_SLOTS = PISO_GROUPS * PISO_MAXK;    // candidates per pass
constexpr int64_t PISO_LDS_COLS = 16384;               // widest row staged in LDS
constexpr int PISO_MAX_CAND = 1024;                    // num_coarse, num_fine limit

struct PisoArgs {
    const float* W;
    int64_t ld, rows, cols;
    const float* h;
    const float* coarse;
    const float* fine;
    int nc, nf;
    float qmin, qmax;
    float* scales;
    int8_t* zp;
};

// round half away from zero: trunc(x + copysign(0.5, x)) is floor(x + 0.5)
// for x >= +0 and ceil(x - 0.5) for x < 0 (the additions round the same
// way); for x = -0 it gives -0 where the reference gives +0, which no later
// step of the error can tell apart
__device__ __forceinline__ float rhaz_t(float x) { return truncf(x + copysignf(0.5f, x)); }

struct Cand {
    float s, y, zp;   // scale, RN(1 / s), zero-point (0 when symmetric)
    bool fast;        // w / s by the Markstein sequence (exact in its domain)
};

// FAST: every candidate of the caller takes the Markstein division
template <bool ASYM, bool FAST = false>
__device__ __forceinline__ float piso_err(float w, float h, const Cand& c, float qmin, float qmax) {
    float t;
    if (FAST || c.fast) {
        const float q0 = w * c.y;
        const float r = __builtin_fmaf(-q0, c.s, w);
        t = __builtin_fmaf(r, c.y, q0);
    } else {
        t = w / c.s;
    }
    if (ASYM) t = t + c.zp;
    const float q = fminf(fmaxf(rhaz_t(t), qmin), qmax);
    const float dq = ASYM ? (q - c.zp) * c.s : q * c.s;
    const float d = w - dq;
    return (d * d) * h;
}

template <bool ASYM>
__device__ __forceinline__ Cand make_cand(float base, float factor, float wmin, float qmin, float qmax,
                                          bool row_ok) {
    Cand c;
    float s = base * factor;
    if (ASYM && s < 1e-10f) s = 1e-10f;   // clamp(min=1e-10); NaN stays NaN
    c.s = s;
    c.y = 1.0f / s;
    c.fast = row_ok && div_b_ok(s);
    c.zp = 0.0f;
    if (ASYM) {
        const float z = qmin - wmin / s;
        c.zp = fminf(fmaxf(rhaz(z), qmin), qmax);
    }
    return c;
}

// torch argmin over v[0 .. n): the first minimum; a NaN is the minimum
__device__ int first_argmin(const float* v, int n) {
    int b = 0;
    float bv = v[0];
    if (bv != bv) return 0;
    for (int i = 1; i < n; ++i) {
        const float x = v[i];
        if (x != x) return i;
        if (x < bv) {
            bv = x;
            b = i;
        }
    }
    return b;
}

// Costs of the candidates base * factor[0 .. n) into cost[]; K candidates per lane.
template <bool ASYM, int K>
__device__ void eval_costs(const float* wv, const float* hv, int64_t L, float base, const float* factor, int n,
                           float wmin, float qmin, float qmax, bool row_ok, float (*part)[SUM_SEQ + 1],
                           float* cost) {
    const int t = threadIdx.x, g = t / SUM_SEQ, s = t % SUM_SEQ;
    const int64_t n4 = L / SUM_VEC / 4;
    const int lp = cascade_lp(n4);
    for (int c0 = 0; c0 < n; c0 += PISO_GROUPS * K) {
        const int cnt = min(PISO_GROUPS * K, n - c0);
        if (L >= SUM_VEC && g * K < cnt) {
            Cand cd[K];
#pragma unroll
            for (int k = 0; k < K; ++k) {
                const int c = min(c0 + g * K + k, n - 1);
                cd[k] = make_cand<ASYM>(base, factor[c], wmin, qmin, qmax, row_ok);
            }
            float out[K];
            bool all_fast = true;
#pragma unroll
            for (int k = 0; k < K; ++k) all_fast = all_fast && cd[k].fast;
            if (all_fast) {
                cascade_seq_k<K>(
                    [&](int64_t m, float (&e)[K]) {
                        const int64_t i = m * SUM_SEQ + s;
                        const float w = wv[i], h = hv[i];
#pragma unroll
                        for (int k = 0; k < K; ++k) e[k] = piso_err<ASYM, true>(w, h, cd[k], qmin, qmax);
                    },
                    n4, lp, out);
            } else {
                cascade_seq_k<K>(
                    [&](int64_t m, float (&e)[K]) {
                        const int64_t i = m * SUM_SEQ + s;
                        const float w = wv[i], h = hv[i];
#pragma unroll
                        for (int k = 0; k < K; ++k) e[k] = piso_err<ASYM>(w, h, cd[k], qmin, qmax);
                    },
                    n4, lp, out);
            }
#pragma unroll
            for (int k = 0; k < K; ++k) part[g * K + k][s] = out[k];
        }
        __syncthreads();
        if (t < cnt) {
            const Cand cd = make_cand<ASYM>(base, factor[c0 + t], wmin, qmin, qmax, row_ok);
            auto x = [&](int64_t i) { return piso_err<ASYM>(wv[i], hv[i], cd, qmin, qmax); };
            cost[c0 + t] = L >= SUM_VEC ? inner_sum_finish(part[t], x, L) : inner_sum_short(x, L);
        }
        __syncthreads();
    }
}

template <bool ASYM, int K>
__device__ float search(const float* wv, const float* hv, int64_t L, float base, const float* factor, int n,
                        float wmin, float qmin, float qmax, bool row_ok, float (*part)[SUM_SEQ + 1], float* cost,
                        float* best, float* best_zp) {
    eval_costs<ASYM, K>(wv, hv, L, base, factor, n, wmin, qmin, qmax, row_ok, part, cost);
    if (threadIdx.x == 0) {
        const int b = first_argmin(cost, n);
        const Cand cd = make_cand<ASYM>(base, factor[b], wmin, qmin, qmax, row_ok);
        *best = cd.s;
        *best_zp = cd.zp;
    }
    __syncthreads();
    return *best;
}

template <bool ASYM, bool STAGE>
__global__ __launch_bounds__(PISO_THREADS) void piso_kernel(PisoArgs a) {
    __shared__ float stage[STAGE ? 2 * PISO_LDS_COLS : 1];
    __shared__ float part[PISO_SLOTS][SUM_SEQ + 1];
    __shared__ float cost[PISO_MAX_CAND];
    __shared__ float red[4][PISO_THREADS / 64];
    __shared__ float best, best_zp;
    const int t = threadIdx.x;
    const int64_t row = blockIdx.x;
    const int64_t L = a.cols;
    const float* wrow = a.W + row * a.ld;
    const float* wv = wrow;
    const float* hv = a.h;
    if (STAGE) {
        for (int64_t i = t; i < L; i += PISO_THREADS) {
            stage[i] = wrow[i];
            stage[PISO_LDS_COLS + i] = a.h[i];
        }
        wv = stage;
        hv = stage + PISO_LDS_COLS;
        __syncthreads();
    }
    // row statistics: min, max, and the extent of the nonzero |w| (the fast
    // division's domain: 2^-60 <= |w| < 2^61 or w == 0)
    float mn = INFINITY, mx = -INFINITY, amin = INFINITY, amax = 0.0f;
    bool nan = false;
    for (int64_t i = t; i < L; i += PISO_THREADS) {
        const float w = wv[i], aw = fabsf(w);
        nan |= w != w;
        mn = fminf(mn, w);
        mx = fmaxf(mx, w);
        amax = fmaxf(amax, aw);
        if (aw != 0.0f) amin = fminf(amin, aw);
    }
    for (int off = 32; off > 0; off >>= 1) {
        mn = fminf(mn, __shfl_xor(mn, off));
        mx = fmaxf(mx, __shfl_xor(mx, off));
        amax = fmaxf(amax, __shfl_xor(amax, off));
        amin = fminf(amin, __shfl_xor(amin, off));
    }
    nan = __any(nan);
    const int lane = t & 63, wave = t >> 6;
    if (lane == 0) {
        red[0][wave] = mn;
        red[1][wave] = mx;
        red[2][wave] = amax;
        red[3][wave] = nan ? 1.0f : amin;   // 1.0 keeps the domain test simple; NaN rows take the IEEE path
    }
    __shared__ int any_nan;
    if (t == 0) any_nan = 0;
    __syncthreads();
    if (lane == 0 && nan) any_nan = 1;
    __syncthreads();
    mn = red[0][0];
    mx = red[1][0];
    amax = red[2][0];
    amin = red[3][0];
    for (int w = 1; w < PISO_THREADS / 64; ++w) {
        mn = fminf(mn, red[0][w]);
        mx = fmaxf(mx, red[1][w]);
        amax = fmaxf(amax, red[2][w]);
        amin = fminf(amin, red[3][w]);
    }
    const bool has_nan = any_nan != 0;
    if (has_nan) {   // torch's amin / amax / abs().amax() propagate NaN
        mn = mx = amax = NAN;
    }
    const bool row_ok = !has_nan && amax < 0x1p61f && (amin == INFINITY || amin >= 0x1p-60f);
    float sref;
    if (ASYM) {
        sref = (mx - mn) / (a.qmax - a.qmin);
    } else {
        sref = amax / a.qmax;
    }
    if (sref < 1e-10f) sref = 1e-10f;   // clamp(min=1e-10); NaN stays NaN
    const float qmin = a.qmin, qmax = a.qmax;
    float sb;
    if (a.nc >= PISO_SLOTS)
        sb = search<ASYM, PISO_MAXK>(wv, hv, L, sref, a.coarse, a.nc, mn, qmin, qmax, row_ok, part, cost, &best,
                                     &best_zp);
    else
        sb = search<ASYM, 1>(wv, hv, L, sref, a.coarse, a.nc, mn, qmin, qmax, row_ok, part, cost, &best, &best_zp);
    if (a.nf >= PISO_SLOTS)
        search<ASYM, PISO_MAXK>(wv, hv, L, sb, a.fine, a.nf, mn, qmin, qmax, row_ok, part, cost, &best, &best_zp);
    else
        search<ASYM, 1>(wv, hv, L, sb, a.fine, a.nf, mn, qmin, qmax, row_ok, part, cost, &best, &best_zp);
    if (t == 0) {
        a.scales[row] = best;
        if (ASYM) a.zp[row] = (int8_t)(int)best_zp;
    }
}

template <bool ASYM, bool STAGE>
static int launch(const PisoArgs& a, hipStream_t st) {
    hipLaunchKernelGGL((piso_kernel<ASYM, STAGE>), dim3((unsigned)a.rows), dim3(PISO_THREADS), 0, st, a);
    IC_CHECK_LAUNCH();
    return IC_OK;
}

}  // namespace
}  // namespace icq

using namespace icq;

extern "C" int ic_piso_scales(const float* W, int64_t rows, int64_t cols, int64_t ld, const float* h, int bits,
                              int asym, const float* coarse, int num_coarse, const float* fine, int num_fine,
                              float* scales, int8_t* zp, void* stream) {
    IC_REQUIRE(W && h && coarse && fine && scales, "ic_piso_scales: null pointer");
    IC_REQUIRE(!asym || zp, "ic_piso_scales: asymmetric search needs zp");
    IC_REQUIRE(bits == 4 || bits == 8, "ic_piso_scales: bits must be 4 or 8");
    IC_REQUIRE(rows >= 0 && cols >= 1 && ld >= cols, "ic_piso_scales: bad shape");
    IC_REQUIRE(rows <= 0x7fffffff, "ic_piso_scales: too many rows");
    IC_REQUIRE(num_coarse >= 1 && num_coarse <= PISO_MAX_CAND && num_fine >= 1 && num_fine <= PISO_MAX_CAND,
               "ic_piso_scales: num_coarse and num_fine must be in [1, 1024]");
    if (rows == 0) return IC_OK;
    hipStream_t st = as_stream(stream);
    PisoArgs a{W, ld, rows, cols, h, coarse, fine, num_coarse, num_fine, bits == 8 ? -128.0f : -8.0f,
               bits == 8 ? 127.0f : 7.0f, scales, zp};
    ProfScope prof(st, PT_PISO, 0.0, 4.0 * (double)rows * cols + 4.0 * cols);
    const bool stage = cols <= PISO_LDS_COLS;
    if (asym) return stage ? launch<true, true>(a, st) : launch<true, false>(a, st);
    return stage ? launch<false, true>(a, st) : launch<false, false>(a, st);
}
