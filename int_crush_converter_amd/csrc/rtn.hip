// Row statistics, RTN scales / zero-points (with clipping-ratio search), RTN
// quantisation fused with INT4 packing, pack/unpack, and the quantisation
// error used for verification.  All bandwidth-bound; one wave owns one row
// for the row-wise reductions, elementwise kernels stream 16 columns per lane.
//
// Bit-exactness: codes and fp16 scales reproduce the fp32 formulas of
// converter/scales.py exactly (IEEE division, no contraction, rhaz with the
// literal +-0.5, round-half-even in the clip search).  The clip search's
// per-row MSE is the reference's (W - dequant).pow(2).mean(dim=-1): fp32
// squares summed in torch's CPU inner-sum order, divided by the row length
// (rows up to 15872 columns; longer rows accumulate in fp64).
#include "common.hpp"
#include "prof.hpp"
#include "torchsum.hpp"

namespace icq {

// NaN-propagating min/max (torch.amin / amax / maximum semantics).
__device__ __forceinline__ float nmax(float a, float b) { return (a != a || a > b) ? a : b; }
__device__ __forceinline__ float nmin(float a, float b) { return (a != a || a < b) ? a : b; }

__device__ __forceinline__ float wave_nmax(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = nmax(v, __shfl_xor(v, o, 64));
    return v;
}
__device__ __forceinline__ float wave_nmin(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = nmin(v, __shfl_xor(v, o, 64));
    return v;
}

struct RowStats { float mn, mx, amax; };

// One wave per row; 16-byte loads when the row start is 16-byte aligned.
__device__ RowStats row_stats_wave(const float* __restrict__ x, int64_t cols) {
    const int lane = threadIdx.x & 63;
    float mn = INFINITY, mx = -INFINITY, am = 0.0f;
    int64_t c = lane;
    if ((reinterpret_cast<uintptr_t>(x) & 15) == 0) {
        const int64_t c4 = cols & ~(int64_t)3;
        int64_t j = 4 * (int64_t)lane;
        // four 16-byte loads in flight per lane (min / max do not depend on order)
        for (; j + 768 < c4; j += 1024) {
            float4 t[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) t[k] = *reinterpret_cast<const float4*>(x + j + 256 * k);
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const float v[4] = {t[k].x, t[k].y, t[k].z, t[k].w};
#pragma unroll
                for (int u = 0; u < 4; ++u) { mn = nmin(mn, v[u]); mx = nmax(mx, v[u]); am = nmax(am, fabsf(v[u])); }
            }
        }
        for (; j < c4; j += 256) {
            const float4 t = *reinterpret_cast<const float4*>(x + j);
            const float v[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
            for (int u = 0; u < 4; ++u) { mn = nmin(mn, v[u]); mx = nmax(mx, v[u]); am = nmax(am, fabsf(v[u])); }
        }
        c = c4 + lane;
    }
    for (; c < cols; c += 64) {
        float v = x[c];
        mn = nmin(mn, v); mx = nmax(mx, v); am = nmax(am, fabsf(v));
    }
    return {wave_nmin(mn), wave_nmax(mx), wave_nmax(am)};
}

__global__ __launch_bounds__(256) void row_stats_kernel(const float* __restrict__ x, int64_t rows, int64_t cols,
                                                        int64_t ld, float* rmin, float* rmax, float* ramax) {
    const int64_t wpb = blockDim.x >> 6;
    for (int64_t r = blockIdx.x * wpb + (threadIdx.x >> 6); r < rows; r += (int64_t)gridDim.x * wpb) {
        RowStats s = row_stats_wave(x + r * ld, cols);
        if ((threadIdx.x & 63) == 0) {
            if (rmin) rmin[r] = s.mn;
            if (rmax) rmax[r] = s.mx;
            if (ramax) ramax[r] = s.amax;
        }
    }
}

__device__ __forceinline__ float clamp_scale(float s) { return clampf(s, 1e-5f, 65500.0f); }

// Zero-point clamp fix of converter/scales.py:184-229 (both masks are taken
// from the incoming scale, then the two corrections apply in order).
__device__ __forceinline__ float fix_asym(float s, float wmin, float wmax, float qmin, float qmax) {
    const float spread = qmax - qmin;
    float zraw = qmin - rhaz(wmin / s);
    bool lo = zraw < qmin, hi = zraw > qmax;
    if (lo) s = nmax(s, clamp_scale(wmax / spread));
    if (hi) s = nmax(s, clamp_scale(-wmin / spread));
    return s;
}

// Candidate scale of one clip ratio (or of the plain formula when !has_ratio).
struct Cand { float s, z; };

// Clipping ratios travel by value in the kernel arguments.
constexpr int MAX_RATIOS = 16;
struct Ratios { float v[MAX_RATIOS]; };

__device__ __forceinline__ Cand rtn_candidate(const RowStats& st, int bits, int asym, bool has_ratio, float ratio) {
    const float qmin = bits == 4 ? -8.0f : -128.0f, qmax = bits == 4 ? 7.0f : 127.0f;
    Cand c;
    if (!asym) {
        const float div = bits == 4 ? 7.0f : 127.0f;
        float a = has_ratio ? st.amax * ratio : st.amax;
        c.s = clamp_scale(a / div);
        c.z = 0.0f;
    } else {
        const float spread = bits == 4 ? 15.0f : 255.0f;
        float range = st.mx - st.mn;
        if (has_ratio) range = range * ratio;
        float s = clamp_scale(range / spread);
        s = fix_asym(s, st.mn, st.mx, qmin, qmax);
        c.s = s;
        c.z = clampf(qmin - rhaz(st.mn / s), qmin, qmax);
    }
    return c;
}

// Squared error of one clip candidate for one value (fp64).  q =
// clamp(round_half_even(w / s [+ z])) with w / s correctly rounded: the
// fast quotient from RN(1/s) when the caller established div_rn's domain
// (FAST), else the IEEE division, as in the reference.
template <bool FAST>
__device__ __forceinline__ double cand_sq_err(float w, const Cand& c, float rs, int asym, float qmin, float qmax) {
    float y = FAST ? div_rn_fast(w, c.s, rs) : w / c.s;
    if (asym) y = y + c.z;
    const float q = clampf_med3(rhte(y), qmin, qmax);
    const float d = asym ? (q - c.z) * c.s : q * c.s;
    const float e = w - d;
    return (double)e * (double)e;
}

// One wave per row: stats, then either the closed form or the clip search.
// CR > 0: the row (cols <= 64 CR) is held in registers for all candidates;
// CR == 0: each candidate re-reads the row (from the caches).
template <int CR>
__global__ __launch_bounds__(256) void rtn_scales_kernel(const float* __restrict__ W, int64_t rows, int64_t cols,
                                                         int64_t ld, int bits, int asym, int n_ratios,
                                                         Ratios rt, uint16_t* __restrict__ scale16, int8_t* __restrict__ zp) {
    const int64_t wpb = blockDim.x >> 6;
    const int lane = threadIdx.x & 63;
    const float qmin = bits == 4 ? -8.0f : -128.0f, qmax = bits == 4 ? 7.0f : 127.0f;
    for (int64_t r = blockIdx.x * wpb + (threadIdx.x >> 6); r < rows; r += (int64_t)gridDim.x * wpb) {
        const float* x = W + r * ld;
        float v[CR > 0 ? CR : 1];
        RowStats st;
        bool row_ok = false;   // every value of the row in div_rn's numerator domain
        if (CR > 0) {
            float mn = INFINITY, mx = -INFINITY, am = 0.0f;
            bool ok = true;
#pragma unroll
            for (int i = 0; i < CR; ++i) {
                const int64_t j = lane + 64 * i;
                v[i] = j < cols ? x[j] : 0.0f;
                if (j < cols) { mn = nmin(mn, v[i]); mx = nmax(mx, v[i]); am = nmax(am, fabsf(v[i])); }
                ok = ok && div_a_ok(v[i]);
            }
            st = {wave_nmin(mn), wave_nmax(mx), wave_nmax(am)};
            row_ok = __builtin_amdgcn_ballot_w64(!ok) == 0;
        } else {
            st = row_stats_wave(x, cols);
        }
        Cand best;
        if (n_ratios == 0) {
            best = rtn_candidate(st, bits, asym, false, 1.0f);
            // zero groups map zero to zero in the INT4 closed form only (scales.py:265-267)
            if (asym && bits == 4 && st.mn == 0.0f && st.mx == 0.0f) best.z = 0.0f;
        } else {
            double best_m = 0.0;
            for (int k = 0; k < n_ratios; ++k) {
                const Cand c = rtn_candidate(st, bits, asym, true, rt.v[k]);
                const float rs = 1.0f / c.s;
                double acc = 0.0;
                if (CR > 0 && row_ok && div_b_ok(c.s)) {
#pragma unroll
                    for (int i = 0; i < CR; ++i)
                        if (lane + 64 * i < cols) acc += cand_sq_err<true>(v[i], c, rs, asym, qmin, qmax);
                } else if (CR > 0) {
#pragma unroll
                    for (int i = 0; i < CR; ++i)
                        if (lane + 64 * i < cols) acc += cand_sq_err<false>(v[i], c, rs, asym, qmin, qmax);
                } else {
                    for (int64_t j = lane; j < cols; j += 64) acc += cand_sq_err<false>(x[j], c, rs, asym, qmin, qmax);
                }
                acc = wave_sum(acc);
                // strict '<' keeps the first ratio on ties; NaN never wins
                if (k == 0 || acc < best_m) { best = c; best_m = acc; }
            }
        }
        if (lane == 0) {
            scale16[r] = f32_to_f16_bits(best.s);
            if (asym && zp) zp[r] = (int8_t)(int)best.z;
        }
    }
}

// fp32 squared error of one clip candidate for one value (the elementwise
// steps of the reference's mse before its sum).
// FAST: the caller checked that the row holds no NaN and every value and the
// scale lie in the fast division's domain, so y is finite and the clamp
// needs no NaN test.
template <bool FAST, bool ASYM>
__device__ __forceinline__ float cand_sq(float w, const Cand& c, float rs, float qmin, float qmax) {
    float y = FAST ? div_rn_fast(w, c.s, rs) : w / c.s;
    if (ASYM) y = y + c.z;
    const float q = FAST ? __builtin_amdgcn_fmed3f(rhte(y), qmin, qmax) : clampf_med3(rhte(y), qmin, qmax);
    const float d = ASYM ? (q - c.z) * c.s : q * c.s;
    const float e = w - d;
    return e * e;
}

// Clip search with the reference's fp32 MSE, one work-group per row: the row
// is staged in LDS (cols <= CLIP_LDS_COLS), its min / max / absmax reduced,
// then thread (candidate k, sequence q) runs the cascade of sequence q
// (values 32 m + q) of candidate k's squared errors, blockDim / 32
// candidates per pass, and one thread per candidate finishes torch's inner
// sum (leftover vectors, merge, leftover scalars, lanes) and divides by the
// row length.  The first minimum (strict <, a NaN never wins) is kept.  The
// work-group has 32 threads per candidate rounded up to whole waves (at most
// 256), so that e.g. 5 candidates take 3 waves, not 4 with 3/8 idle.
constexpr int64_t CLIP_LDS_COLS = 15872;   // the row plus the static arrays within 64 KB of LDS
constexpr int CLIP_PASS = 256 / SUM_SEQ;   // candidates per pass at most

template <bool ASYM>
__global__ __launch_bounds__(256) void rtn_clip_kernel(const float* __restrict__ W, int64_t rows, int64_t cols,
                                                       int64_t ld, int bits, int n_ratios, Ratios rt,
                                                       uint16_t* __restrict__ scale16, int8_t* __restrict__ zp) {
    extern __shared__ float xs[];                   // the row, cols floats
    __shared__ float part[CLIP_PASS][SUM_SEQ];
    __shared__ float mses[MAX_RATIOS];
    __shared__ float red[4][3];
    __shared__ int red_ok[4];
    const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
    const int nt = blockDim.x, nwv = nt >> 6, pass = nt / SUM_SEQ;
    const float qmin = bits == 4 ? -8.0f : -128.0f, qmax = bits == 4 ? 7.0f : 127.0f;
    for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
        const float* x = W + r * ld;
        float mn = INFINITY, mx = -INFINITY, am = 0.0f;
        bool ok = true;
        for (int64_t j = t; j < cols; j += nt) {
            const float v = x[j];
            xs[j] = v;
            mn = nmin(mn, v);
            mx = nmax(mx, v);
            am = nmax(am, fabsf(v));
            ok = ok && div_a_ok(v);
        }
        mn = wave_nmin(mn);
        mx = wave_nmax(mx);
        am = wave_nmax(am);
        const bool wok = __builtin_amdgcn_ballot_w64(!ok) == 0;
        if (lane == 0) {
            red[wv][0] = mn; red[wv][1] = mx; red[wv][2] = am;
            red_ok[wv] = wok;
        }
        __syncthreads();
        RowStats st{red[0][0], red[0][1], red[0][2]};
        bool row_ok = red_ok[0] != 0;
        for (int w = 1; w < nwv; ++w) {
            st.mn = nmin(st.mn, red[w][0]);
            st.mx = nmax(st.mx, red[w][1]);
            st.amax = nmax(st.amax, red[w][2]);
            row_ok = row_ok && red_ok[w] != 0;
        }
        const int64_t n4 = cols / SUM_VEC / 4;
        const int lp = cascade_lp(n4);
        for (int k0 = 0; k0 < n_ratios; k0 += pass) {
            const int kk = t / SUM_SEQ, q = t % SUM_SEQ, k = k0 + kk;
            if (k < n_ratios && cols >= SUM_VEC) {
                const Cand c = rtn_candidate(st, bits, ASYM, true, rt.v[k]);
                const float rs = 1.0f / c.s;
                part[kk][q] = row_ok && div_b_ok(c.s)
                    ? cascade_seq([&](int64_t m) { return cand_sq<true, ASYM>(xs[m * SUM_SEQ + q], c, rs, qmin, qmax); },
                                  n4, lp)
                    : cascade_seq([&](int64_t m) { return cand_sq<false, ASYM>(xs[m * SUM_SEQ + q], c, rs, qmin, qmax); },
                                  n4, lp);
            }
            __syncthreads();
            if (t < pass && k0 + t < n_ratios) {
                const Cand c = rtn_candidate(st, bits, ASYM, true, rt.v[k0 + t]);
                const float rs = 1.0f / c.s;
                auto sq = [&](int64_t i) { return cand_sq<false, ASYM>(xs[i], c, rs, qmin, qmax); };
                const float sum = cols >= SUM_VEC ? inner_sum_finish(part[t], sq, cols) : inner_sum_short(sq, cols);
                mses[k0 + t] = sum / (float)cols;
            }
            __syncthreads();
        }
        if (t == 0) {
            int best = 0;
            float bm = mses[0];
            for (int k = 1; k < n_ratios; ++k)
                if (mses[k] < bm) { bm = mses[k]; best = k; }
            const Cand c = rtn_candidate(st, bits, ASYM, true, rt.v[best]);
            scale16[r] = f32_to_f16_bits(c.s);
            if (ASYM && zp) zp[r] = (int8_t)(int)c.z;
        }
        __syncthreads();   // xs and part are reused by the next row
    }
}

// The same clip search with the row in registers, for rows whose 32
// inner-sum sequences (values 32 m + q, m < n4 = cols / 32) are whole groups
// of 16 of torch's cascade (n4 a multiple of 16 up to 128: 512 .. 4127
// columns with such an n4).  Such a cascade never reaches its third
// accumulator: each group of 16 is summed from zero and added to a1, and
// the sequence's sum is ((0 + a1) + 0) + 0 = a1.  One wave per row: lanes q
// and q + 32 hold the first and second half of sequence q's groups, and
// each lane runs every candidate over its values in one pass (each value is
// fetched once for all candidates).  Group sums stay separate until lane q's
// chain a1 reaches lane q + 32, which continues it over its own groups in
// order.  The lanes' sums meet in LDS, where lane k < K finishes candidate
// k's inner sum (inner_sum_finish: the row's leftover values come from
// global memory) and lane 0 keeps the first strict minimum.  While a wave
// searches one row, the loads of its next row are in flight: each group's
// registers are refilled as soon as the group is summed.  Rows whose
// values or scales leave the fast division's domain take the IEEE division.
constexpr int CLIP_REG_MAX_K = 8;

// Orders one wave's LDS writes before its later LDS reads by other lanes
// (a wave's LDS operations complete in issue order; this keeps the compiler
// from moving them and waits for the writes).  The clip search's LDS slots
// belong to one wave each, so no work-group barrier is needed.
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0)
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}
constexpr int CLIP_VPL = 64;   // values per lane: up to 4 groups of 16

// Group sums of one lane's values for every candidate (fast division);
// after group g is summed, refill(g) may overwrite its 16 registers (the
// next row's loads).
template <int K, bool ASYM, typename Refill>
__device__ __forceinline__ void clip_group_sums(float (&v)[CLIP_VPL], int cnt, const Cand (&c)[K],
                                                const float (&rs)[K], float qmin, float qmax,
                                                float (&gs)[K][CLIP_VPL / 16], Refill refill) {
#pragma unroll
    for (int g = 0; g < CLIP_VPL / 16; ++g) {
        if (g < cnt) {
            float a0[K];
#pragma unroll
            for (int k = 0; k < K; ++k) a0[k] = 0.0f;
#pragma unroll
            for (int j = 0; j < 16; ++j) {
#pragma unroll
                for (int k = 0; k < K; ++k)
                    a0[k] = a0[k] + cand_sq<true, ASYM>(v[16 * g + j], c[k], rs[k], qmin, qmax);
                // one value at a time: the K chains are enough to fill the
                // VALU, and the registers stay few
                __builtin_amdgcn_sched_barrier(0);
            }
#pragma unroll
            for (int k = 0; k < K; ++k) gs[k][g] = a0[k];
            refill(g);
        }
    }
}

template <int K, bool ASYM>
__global__ __launch_bounds__(256, 2) void rtn_clip_reg_kernel(const float* __restrict__ W, int64_t rows, int64_t cols,
                                                           int64_t ld, int bits, Ratios rt, int64_t iters,
                                                           uint16_t* __restrict__ scale16, int8_t* __restrict__ zp) {
    __shared__ float part[4][K][SUM_SEQ];
    __shared__ float mses[4][K];
    const int t = threadIdx.x, lane = t & 63, wv = t >> 6, q = lane & 31, h = lane >> 5;
    const float qmin = bits == 4 ? -8.0f : -128.0f, qmax = bits == 4 ? 7.0f : 127.0f;
    const int ng = (int)(cols / SUM_SEQ / 16);               // groups per sequence
    const int hA = (ng + 1) / 2;                              // groups of the first half
    const int g0 = h * hA, cnt = h ? ng - hA : hA;            // this lane's groups
    const int64_t rest0 = (int64_t)ng * 16 * SUM_SEQ;         // values past the sequences (< 32)
    const int64_t nwv = (int64_t)gridDim.x * 4;
    int64_t r = (int64_t)blockIdx.x * 4 + wv;                 // every wave runs `iters` rounds
    float cur[CLIP_VPL];
    // group g of this lane's values of a row
    auto load_group = [&](int g, int64_t row) {
        const float* x = W + row * ld + q + (int64_t)(16 * (g0 + g)) * SUM_SEQ;
#pragma unroll
        for (int gg = 0; gg < CLIP_VPL / 16; ++gg)
            if (gg == g) {
#pragma unroll
                for (int j = 0; j < 16; ++j) cur[16 * gg + j] = x[j * SUM_SEQ];
            }
    };
    if (r < rows) {
#pragma unroll
        for (int g = 0; g < CLIP_VPL / 16; ++g)
            if (g < cnt) load_group(g, r);
    }
    for (int64_t it = 0; it < iters; ++it, r += nwv) {
        const bool live = r < rows;   // wave-uniform
        const bool more = r + nwv < rows;
        float mn = INFINITY, mx = -INFINITY, am = 0.0f;
        bool bad = false, tiny = false;
        if (live) {
#pragma unroll
            for (int g = 0; g < CLIP_VPL / 16; ++g)
                if (g < cnt) {
#pragma unroll
                    for (int j = 0; j < 16; ++j) {
                        const float u = cur[16 * g + j];
                        mn = fminf(mn, u); mx = fmaxf(mx, u); am = fmaxf(am, fabsf(u));
                        bad = bad || u != u;
                        tiny = tiny || (fabsf(u) < 0x1p-60f && u != 0.0f);
                    }
                }
            if (h == 0 && rest0 + q < cols) {
                const float u = W[r * ld + rest0 + q];
                mn = fminf(mn, u); mx = fmaxf(mx, u); am = fmaxf(am, fabsf(u));
                bad = bad || u != u;
                tiny = tiny || (fabsf(u) < 0x1p-60f && u != 0.0f);
            }
        }
        // the row's stats: minimum, maximum and largest magnitude, NaN if any
        // value is NaN (torch's amin / amax); every value in the fast
        // division's numerator domain iff no NaN, no magnitude in (0, 2^-60)
        // and the largest one below 2^61
        mn = wave_nmin(mn);
        mx = wave_nmax(mx);
        am = wave_nmax(am);
        const bool nan_row = __builtin_amdgcn_ballot_w64(bad) != 0;
        const bool tiny_row = __builtin_amdgcn_ballot_w64(tiny) != 0;
        if (nan_row) mn = mx = am = __builtin_nanf("");
        const RowStats st{mn, mx, am};
        Cand c[K];
        float rs[K];
        bool fast = !nan_row && !tiny_row && am < 0x1p61f;
#pragma unroll
        for (int k = 0; k < K; ++k) {
            c[k] = rtn_candidate(st, bits, ASYM, true, rt.v[k]);
            rs[k] = 1.0f / c[k].s;
            fast = fast && div_b_ok(c[k].s);
        }
        float gs[K][CLIP_VPL / 16];
        // each group's registers take the next row's values once summed
        auto refill = [&](int g) {
            if (more) load_group(g, r + nwv);
        };
        if (live && fast) {
            clip_group_sums<K, ASYM>(cur, cnt, c, rs, qmin, qmax, gs, refill);
        } else if (live) {
            // IEEE division (rare): the values again from memory, one at a time
            const float* x = W + r * ld + q + (int64_t)(16 * g0) * SUM_SEQ;
#pragma unroll
            for (int g = 0; g < CLIP_VPL / 16; ++g)
                if (g < cnt) {
#pragma unroll
                    for (int k = 0; k < K; ++k) {
                        float a0 = 0.0f;
#pragma unroll 1
                        for (int j = 0; j < 16; ++j)
                            a0 = a0 + cand_sq<false, ASYM>(x[(16 * g + j) * SUM_SEQ], c[k], rs[k], qmin, qmax);
                        gs[k][g] = a0;
                    }
                    refill(g);
                }
        }
        // sequence q's chain: lane q over the first groups, then lane q + 32
        // from lane q's value over the rest
#pragma unroll
        for (int k = 0; k < K; ++k) {
            float a1 = 0.0f;
#pragma unroll
            for (int g = 0; g < CLIP_VPL / 16; ++g)
                if (g < cnt) a1 = a1 + gs[k][g];
            const float from_first = __shfl_xor(a1, 32, 64);
            if (h) {
                a1 = from_first;
#pragma unroll
                for (int g = 0; g < CLIP_VPL / 16; ++g)
                    if (g < cnt) a1 = a1 + gs[k][g];
                part[wv][k][q] = a1;
            }
        }
        wave_lds_sync();
        if (live && lane < K) {
            Cand cq = c[0];
            float rq = rs[0];
#pragma unroll
            for (int k = 1; k < K; ++k)
                if (lane == k) { cq = c[k]; rq = rs[k]; }
            const float* xr = W + r * ld;
            auto sq = [&](int64_t i) { return cand_sq<false, ASYM>(xr[i], cq, rq, qmin, qmax); };
            mses[wv][lane] = inner_sum_finish(part[wv][lane], sq, cols) / (float)cols;
        }
        wave_lds_sync();
        if (live && lane == 0) {
            int best = 0;
            float bm = mses[wv][0];
#pragma unroll
            for (int k = 1; k < K; ++k)
                if (mses[wv][k] < bm) { bm = mses[wv][k]; best = k; }
            Cand cb = c[0];
#pragma unroll
            for (int k = 1; k < K; ++k)
                if (best == k) cb = c[k];
            scale16[r] = f32_to_f16_bits(cb.s);
            if (ASYM && zp) zp[r] = (int8_t)(int)cb.z;
        }
        wave_lds_sync();   // part / mses are reused by the next round
    }
}

template <int K, bool ASYM>
static void launch_clip_reg(const float* W, int64_t rows, int64_t cols, int64_t ld, int bits, const Ratios& rt,
                            uint16_t* scale16, int8_t* zp, hipStream_t st) {
    // two rows per wave where the rows allow (the second row's loads overlap
    // the first row's search); four waves per work-group
    const int64_t wgs = std::max<int64_t>(1, std::min<int64_t>(cdiv(rows, 8), 65535));
    const int64_t iters = cdiv(rows, wgs * 4);
    hipLaunchKernelGGL((rtn_clip_reg_kernel<K, ASYM>), dim3((unsigned)wgs), dim3(256), 0, st, W, rows, cols, ld, bits,
                       rt, iters, scale16, zp);
}

template <int K>
static void launch_clip_reg_k(int n_ratios, bool asym, const float* W, int64_t rows, int64_t cols, int64_t ld,
                              int bits, const Ratios& rt, uint16_t* scale16, int8_t* zp, hipStream_t st) {
    if constexpr (K <= CLIP_REG_MAX_K) {
        if (n_ratios == K) {
            if (asym) launch_clip_reg<K, true>(W, rows, cols, ld, bits, rt, scale16, zp, st);
            else launch_clip_reg<K, false>(W, rows, cols, ld, bits, rt, scale16, zp, st);
        } else {
            launch_clip_reg_k<K + 1>(n_ratios, asym, W, rows, cols, ld, bits, rt, scale16, zp, st);
        }
    }
}

__device__ __forceinline__ uint8_t nib(float q) { return (uint8_t)(((int)q) & 0xF); }

// One wave per row, 4 consecutive columns per lane and step: 16-byte W
// loads, 4-byte code stores, 2-byte packed stores (VEC: row pointers and
// pitches aligned for them; else element by element).  The quotient is the
// fast correctly rounded one unless some value of the wave's step lies
// outside div_rn's domain, which takes the IEEE division.
// codes: int8 [rows, ld_q]; packed: uint8 [rows, ld_p] (low nibble = even column).
template <bool VEC>
__global__ __launch_bounds__(256) void rtn_quant_kernel(const float* __restrict__ W, int64_t rows, int64_t cols,
                                                        int64_t ld, int bits, const void* __restrict__ scale,
                                                        int scale_kind, const float* __restrict__ zp,
                                                        int8_t* __restrict__ codes, int64_t ld_q,
                                                        uint8_t* __restrict__ packed, int64_t ld_p) {
    const float qmin = bits == 4 ? -8.0f : -128.0f, qmax = bits == 4 ? 7.0f : 127.0f;
    const int lane = threadIdx.x & 63;
    const int64_t nw = (int64_t)gridDim.x * (blockDim.x >> 6);
    for (int64_t r = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6); r < rows; r += nw) {
        const float s = scale_kind == 0 ? f16_bits_to_f32(reinterpret_cast<const uint16_t*>(scale)[r])
                                        : reinterpret_cast<const float*>(scale)[r];
        const float z = zp ? zp[r] : 0.0f;
        const float rs = 1.0f / s;
        const bool s_ok = div_b_ok(s);
        const float* x = W + r * ld;
        // QU column steps of the wave per pass, all their loads in flight first
        constexpr int QU = 4;
        for (int64_t cb = 4 * (int64_t)lane; cb < cols; cb += 256 * QU) {
          float wq[QU][4];
#pragma unroll
          for (int k = 0; k < QU; ++k) {
            const int64_t c0 = cb + 256 * k;
            if (VEC && c0 + 4 <= cols) {
                const float4 t = *reinterpret_cast<const float4*>(x + c0);
                wq[k][0] = t.x; wq[k][1] = t.y; wq[k][2] = t.z; wq[k][3] = t.w;
            } else {
#pragma unroll
                for (int u = 0; u < 4; ++u) wq[k][u] = c0 + u < cols ? x[c0 + u] : 0.0f;
            }
          }
#pragma unroll
          for (int k = 0; k < QU; ++k) {
            const int64_t c0 = cb + 256 * k;
            const bool full = c0 + 4 <= cols;
            const float* w = wq[k];
            const bool ok = s_ok && div_a_ok(w[0]) && div_a_ok(w[1]) && div_a_ok(w[2]) && div_a_ok(w[3]);
            const bool all_ok = __builtin_amdgcn_ballot_w64(!ok) == 0;
            float q[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                float y = all_ok ? div_rn_fast(w[u], s, rs) : (ok ? div_rn_fast(w[u], s, rs) : w[u] / s);
                if (zp) y = y + z;
                q[u] = c0 + u < cols ? clampf_med3(rhaz_trunc(y), qmin, qmax) : 0.0f;
            }
            if (codes) {
                int8_t* o = codes + r * ld_q + c0;
                if (VEC && full) {
                    *reinterpret_cast<char4*>(o) = make_char4((signed char)(int)q[0], (signed char)(int)q[1],
                                                              (signed char)(int)q[2], (signed char)(int)q[3]);
                } else {
#pragma unroll
                    for (int u = 0; u < 4; ++u)
                        if (c0 + u < cols) o[u] = (int8_t)(int)q[u];
                }
            }
            if (packed) {
                uint8_t* o = packed + r * ld_p + c0 / 2;
                const uint8_t b0 = (uint8_t)(nib(q[0]) | (nib(q[1]) << 4)), b1 = (uint8_t)(nib(q[2]) | (nib(q[3]) << 4));
                if (VEC && full) {
                    *reinterpret_cast<uint16_t*>(o) = (uint16_t)(b0 | (b1 << 8));
                } else if (c0 < cols) {
                    o[0] = b0;
                    if (c0 + 2 < cols) o[1] = b1;
                }
            }
          }
        }
    }
}

// flags: [0] any non-finite, [1] any value < -8, [2] any value > 7
__global__ __launch_bounds__(256) void pack_int4_kernel(const void* __restrict__ src, int kind, int64_t rows,
                                                        int64_t cols, int64_t ld_src, uint8_t* __restrict__ dst,
                                                        int64_t ld_dst, int32_t* flags) {
    const int64_t bpr = cdiv(cols, 2);
    const int64_t total = rows * bpr;
    int nf = 0, lo = 0, hi = 0;
    for (int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; g < total;
         g += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = g / bpr;
        const int64_t c = (g - r * bpr) * 2;
        int v[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            if (c + i < cols) {
                if (kind == 0) {
                    v[i] = reinterpret_cast<const int8_t*>(src)[r * ld_src + c + i];
                } else {
                    float f = reinterpret_cast<const float*>(src)[r * ld_src + c + i];
                    nf |= !isfinite(f);
                    lo |= f < -8.0f;
                    hi |= f > 7.0f;
                    v[i] = isfinite(f) ? (int)f : 0;   // .to(int8) truncates toward zero
                }
                lo |= v[i] < -8;
                hi |= v[i] > 7;
            } else {
                v[i] = 0;
            }
        }
        if (dst) dst[r * ld_dst + c / 2] = (uint8_t)((v[0] & 0xF) | ((v[1] & 0xF) << 4));
    }
    if (__any(nf)) { if ((threadIdx.x & 63) == 0) atomicOr(flags + 0, 1); }
    if (__any(lo)) { if ((threadIdx.x & 63) == 0) atomicOr(flags + 1, 1); }
    if (__any(hi)) { if ((threadIdx.x & 63) == 0) atomicOr(flags + 2, 1); }
}

// Packing of int8 codes, 32 per thread (16-byte loads and stores), for rows
// of whole 32-code units with 16-byte aligned rows.  Per 32-bit word of 4
// codes: nibbles (w & 0x0F0F0F0F) fold into 2 bytes; a code lies in
// [-8, 7] iff its bits 3..7 are equal, i.e. ((w ^ (w << 1)) & 0xF0F0F0F0)
// is zero.  A thread that sees an out-of-range code re-checks its 32 codes
// one by one to set the < -8 / > 7 flags like the scalar kernel.
typedef unsigned int pk_uintx4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ unsigned pack_word_pair(unsigned w0, unsigned w1) {
    const unsigned l0 = w0 & 0x0F0F0F0Fu, l1 = w1 & 0x0F0F0F0Fu;
    const unsigned p0 = l0 | (l0 >> 4), p1 = l1 | (l1 >> 4);
    return (p0 & 0xFFu) | ((p0 >> 8) & 0xFF00u) | ((p1 & 0xFFu) << 16) | ((p1 << 8) & 0xFF000000u);
}

__global__ __launch_bounds__(256) void pack_int4_vec_kernel(const int8_t* __restrict__ src, uint32_t rows,
                                                            uint32_t upr, int64_t ld_src, uint8_t* __restrict__ dst,
                                                            int64_t ld_dst, int32_t* flags) {
    const uint32_t total = rows * upr;
    int lo = 0, hi = 0;
    for (uint32_t u = blockIdx.x * blockDim.x + threadIdx.x; u < total; u += gridDim.x * blockDim.x) {
        const uint32_t r = u / upr, c0 = (u - r * upr) * 32;
        const pk_uintx4* p = reinterpret_cast<const pk_uintx4*>(src + (int64_t)r * ld_src + c0);
        const pk_uintx4 a = p[0], b = p[1];
        unsigned bad = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) bad |= ((a[k] ^ (a[k] << 1)) | (b[k] ^ (b[k] << 1))) & 0xF0F0F0F0u;
        if (bad) {
            const int8_t* q = src + (int64_t)r * ld_src + c0;
            for (int i = 0; i < 32; ++i) {
                lo |= q[i] < -8;
                hi |= q[i] > 7;
            }
        }
        if (dst) {
            pk_uintx4 o;
            o[0] = pack_word_pair(a[0], a[1]);
            o[1] = pack_word_pair(a[2], a[3]);
            o[2] = pack_word_pair(b[0], b[1]);
            o[3] = pack_word_pair(b[2], b[3]);
            *reinterpret_cast<pk_uintx4*>(dst + (int64_t)r * ld_dst + c0 / 2) = o;
        }
    }
    if (__any(lo)) { if ((threadIdx.x & 63) == 0) atomicOr(flags + 1, 1); }
    if (__any(hi)) { if ((threadIdx.x & 63) == 0) atomicOr(flags + 2, 1); }
}

__global__ void unpack_int4_kernel(const uint8_t* __restrict__ src, int64_t rows, int64_t k, int64_t ld_src,
                                   int8_t* __restrict__ dst, int64_t ld_dst) {
    const int64_t total = rows * k;
    for (int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; g < total;
         g += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = g / k, c = g - r * k;
        uint8_t b = src[r * ld_src + c / 2];
        int v = (c & 1) ? (b >> 4) : (b & 0xF);
        dst[r * ld_dst + c] = (int8_t)(v >= 8 ? v - 16 : v);
    }
}

constexpr int QERR_BLOCKS = 1024;

// Work-group b takes rows b, b + gridDim.x, ...; per row the scale and
// zero-point are read once and the thread walks the row 4 elements at a
// time (16-byte W loads, 4-byte code loads) when the row is 16-byte aligned,
// else one element at a time.  Each thread's partial sums run in a fixed
// order, so the result does not depend on timing.
__global__ __launch_bounds__(256) void quant_error_partial(const float* __restrict__ W, int64_t rows, int64_t cols,
                                                           int64_t ld, const int8_t* __restrict__ codes, int64_t ld_q,
                                                           const void* __restrict__ scale, int scale_kind,
                                                           const int8_t* __restrict__ zp, double* part_sum,
                                                           float* part_max) {
    double acc = 0.0;
    float mx = 0.0f;
    const bool vec = (cols % 4 == 0) && (ld % 4 == 0) && (ld_q % 4 == 0) && ((uintptr_t)W % 16 == 0) &&
                     ((uintptr_t)codes % 4 == 0);
    for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
        const float s = scale_kind == 0 ? f16_bits_to_f32(reinterpret_cast<const uint16_t*>(scale)[r])
                                        : reinterpret_cast<const float*>(scale)[r];
        const float z = zp ? (float)zp[r] : 0.0f;
        const float* wr = W + r * ld;
        const int8_t* qr = codes + r * ld_q;
        if (vec) {
            // four column steps per pass, their loads in flight together
            constexpr int EU = 4;
            const int64_t step = 4 * (int64_t)blockDim.x;
            for (int64_t cb = 4 * (int64_t)threadIdx.x; cb < cols; cb += EU * step) {
                float4 wv[EU];
                char4 qv[EU];
#pragma unroll
                for (int k = 0; k < EU; ++k) {
                    const int64_t c = cb + k * step;
                    wv[k] = c < cols ? *reinterpret_cast<const float4*>(wr + c) : float4{0.f, 0.f, 0.f, 0.f};
                    qv[k] = c < cols ? *reinterpret_cast<const char4*>(qr + c) : char4{0, 0, 0, 0};
                }
#pragma unroll
                for (int k = 0; k < EU; ++k) {
                    if (cb + k * step >= cols) continue;
                    const float q[4] = {(float)qv[k].x, (float)qv[k].y, (float)qv[k].z, (float)qv[k].w};
                    const float w[4] = {wv[k].x, wv[k].y, wv[k].z, wv[k].w};
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        const float d = zp ? (q[u] - z) * s : q[u] * s;
                        const float e = w[u] - d;
                        acc += (double)e * (double)e;
                        mx = nmax(mx, fabsf(e));
                    }
                }
            }
        } else {
            for (int64_t c = threadIdx.x; c < cols; c += blockDim.x) {
                const float q = (float)qr[c];
                const float d = zp ? (q - z) * s : q * s;
                const float e = wr[c] - d;
                acc += (double)e * (double)e;
                mx = nmax(mx, fabsf(e));
            }
        }
    }
    __shared__ double ss[4];
    __shared__ float sm[4];
    acc = wave_sum(acc);
    mx = wave_nmax(mx);
    if ((threadIdx.x & 63) == 0) { ss[threadIdx.x >> 6] = acc; sm[threadIdx.x >> 6] = mx; }
    __syncthreads();
    if (threadIdx.x == 0) {
        double a = 0.0;
        float m = 0.0f;
        for (int w = 0; w < (int)(blockDim.x >> 6); ++w) { a += ss[w]; m = nmax(m, sm[w]); }
        part_sum[blockIdx.x] = a;
        part_max[blockIdx.x] = m;
    }
}

// One workgroup: fixed-order tree reduction of the partials (deterministic).
__global__ __launch_bounds__(256) void quant_error_final(const double* part_sum, const float* part_max, int n,
                                                         double* out_sum, float* out_max) {
    double a = 0.0;
    float m = 0.0f;
    for (int i = threadIdx.x; i < n; i += blockDim.x) { a += part_sum[i]; m = nmax(m, part_max[i]); }
    __shared__ double ss[4];
    __shared__ float sm[4];
    a = wave_sum(a);
    m = wave_nmax(m);
    if ((threadIdx.x & 63) == 0) { ss[threadIdx.x >> 6] = a; sm[threadIdx.x >> 6] = m; }
    __syncthreads();
    if (threadIdx.x == 0) {
        *out_sum = (ss[0] + ss[1]) + (ss[2] + ss[3]);
        *out_max = nmax(nmax(sm[0], sm[1]), nmax(sm[2], sm[3]));
    }
}

// flag = 1 when any of the n scales (fp16 bits or fp32) is +-Inf, NaN or 0,
// else 0: the reference's bad-scale test (converter/pipeline.py:938-940).
__global__ __launch_bounds__(1024) void scale_status_kernel(const void* __restrict__ scale, int kind, int64_t n,
                                                           int32_t* flag) {
    int bad = 0;
    for (int64_t i = threadIdx.x; i < n; i += blockDim.x) {
        const float s = kind == 0 ? f16_bits_to_f32(reinterpret_cast<const uint16_t*>(scale)[i])
                                  : reinterpret_cast<const float*>(scale)[i];
        bad |= (!(fabsf(s) <= 3.402823466e38f) || s == 0.0f) ? 1 : 0;   // NaN fails the comparison
    }
    bad = __syncthreads_or(bad);
    if (threadIdx.x == 0) *flag = bad ? 1 : 0;
}

static int rows_grid(int64_t rows, int waves_per_block) {
    return (int)std::max<int64_t>(1, std::min<int64_t>(cdiv(rows, waves_per_block), 65535));
}
static int elem_grid(int64_t work) {
    return (int)std::max<int64_t>(1, std::min<int64_t>(cdiv(work, 256), 256 * 64));
}

}  // namespace icq

using namespace icq;

extern "C" int ic_row_stats(const float* x, int64_t rows, int64_t cols, int64_t ld, float* row_min, float* row_max,
                            float* row_absmax, void* stream) {
    IC_REQUIRE(x && ld >= cols, "ic_row_stats: bad arguments");
    if (rows == 0) return IC_OK;
    hipLaunchKernelGGL(row_stats_kernel, dim3(rows_grid(rows, 4)), dim3(256), 0, as_stream(stream), x, rows, cols,
                       ld, row_min, row_max, row_absmax);
    IC_CHECK_LAUNCH();
    return IC_OK;
}

extern "C" int ic_rtn_scales(const float* W, int64_t rows, int64_t cols, int64_t ld, int bits, int asym,
                             const float* ratios, int n_ratios, uint16_t* scale16, int8_t* zp, void* stream) {
    IC_REQUIRE(W && scale16 && ld >= cols && cols > 0, "ic_rtn_scales: bad arguments");
    IC_REQUIRE(bits == 4 || bits == 8, "ic_rtn_scales: bits must be 4 or 8");
    IC_REQUIRE(!asym || zp, "ic_rtn_scales: asymmetric needs zp output");
    IC_REQUIRE(n_ratios >= 0 && n_ratios <= MAX_RATIOS, "ic_rtn_scales: at most 16 clipping ratios are supported");
    IC_REQUIRE(n_ratios == 0 || ratios, "ic_rtn_scales: null ratios");
    if (rows == 0) return IC_OK;
    Ratios rt;
    for (int i = 0; i < MAX_RATIOS; ++i) rt.v[i] = i < n_ratios ? ratios[i] : 1.0f;
    ProfScope prof_scope(as_stream(stream), PT_RTN_SCALES, 0.0, (double)rows * cols * 4.0 + rows * 3.0);
    if (n_ratios >= 1 && n_ratios <= CLIP_REG_MAX_K && cols >= 16 * SUM_SEQ && cols / SUM_SEQ <= 128 &&
        (cols / SUM_SEQ) % 16 == 0)
        launch_clip_reg_k<1>(n_ratios, asym != 0, W, rows, cols, ld, bits, rt, scale16, zp, as_stream(stream));
    else if (n_ratios > 0 && cols <= CLIP_LDS_COLS) {
        const int threads = (int)std::min<int64_t>(256, cdiv((int64_t)n_ratios * SUM_SEQ, 64) * 64);
        if (asym)
            hipLaunchKernelGGL(rtn_clip_kernel<true>, dim3((unsigned)std::min<int64_t>(rows, 65536)), dim3(threads),
                               cols * sizeof(float), as_stream(stream), W, rows, cols, ld, bits, n_ratios, rt,
                               scale16, zp);
        else
            hipLaunchKernelGGL(rtn_clip_kernel<false>, dim3((unsigned)std::min<int64_t>(rows, 65536)), dim3(threads),
                               cols * sizeof(float), as_stream(stream), W, rows, cols, ld, bits, n_ratios, rt,
                               scale16, zp);
    }
    else if (n_ratios > 0 && cols <= 64 * 64)
        hipLaunchKernelGGL(rtn_scales_kernel<64>, dim3(rows_grid(rows, 4)), dim3(256), 0, as_stream(stream), W, rows,
                           cols, ld, bits, asym, n_ratios, rt, scale16, zp);
    else
        hipLaunchKernelGGL(rtn_scales_kernel<0>, dim3(rows_grid(rows, 4)), dim3(256), 0, as_stream(stream), W, rows,
                           cols, ld, bits, asym, n_ratios, rt, scale16, zp);
    IC_CHECK_LAUNCH();
    return IC_OK;
}

extern "C" int ic_rtn_quantize(const float* W, int64_t rows, int64_t cols, int64_t ld, int bits,
                               const void* scale, int scale_kind, const float* zp, int8_t* codes, int64_t ld_q,
                               uint8_t* packed, int64_t ld_p, void* stream) {
    IC_REQUIRE(W && scale && ld >= cols, "ic_rtn_quantize: bad arguments");
    IC_REQUIRE(scale_kind == 0 || scale_kind == 1, "ic_rtn_quantize: scale_kind must be 0 (f16) or 1 (f32)");
    IC_REQUIRE(bits == 4 || bits == 8, "ic_rtn_quantize: bits must be 4 or 8");
    IC_REQUIRE(!packed || bits == 4, "ic_rtn_quantize: packing needs bits == 4");
    IC_REQUIRE(!codes || ld_q >= cols, "ic_rtn_quantize: bad ld_q");
    IC_REQUIRE(!packed || ld_p >= cdiv(cols, 2), "ic_rtn_quantize: bad ld_p");
    if (rows == 0 || cols == 0) return IC_OK;
    ProfScope prof_scope(as_stream(stream), PT_RTN, 0.0, (double)rows * cols * (4 + (codes ? 1 : 0) + (packed ? 0.5 : 0)));
    const bool vec = ((uintptr_t)W % 16 == 0) && ld % 4 == 0 && (!codes || ((uintptr_t)codes % 4 == 0 && ld_q % 4 == 0)) &&
                     (!packed || ((uintptr_t)packed % 2 == 0 && ld_p % 2 == 0));
    if (vec)
        hipLaunchKernelGGL(rtn_quant_kernel<true>, dim3(rows_grid(rows, 4)), dim3(256), 0, as_stream(stream), W, rows,
                           cols, ld, bits, scale, scale_kind, zp, codes, ld_q, packed, ld_p);
    else
        hipLaunchKernelGGL(rtn_quant_kernel<false>, dim3(rows_grid(rows, 4)), dim3(256), 0, as_stream(stream), W, rows,
                           cols, ld, bits, scale, scale_kind, zp, codes, ld_q, packed, ld_p);
    IC_CHECK_LAUNCH();
    return IC_OK;
}

extern "C" int ic_pack_int4(const void* src, int src_kind, int64_t rows, int64_t cols, int64_t ld_src,
                            uint8_t* dst, int64_t ld_dst, int32_t* flags, void* stream) {
    IC_REQUIRE(src && flags && ld_src >= cols && (!dst || ld_dst >= cdiv(cols, 2)), "ic_pack_int4: bad arguments");
    IC_REQUIRE(src_kind == 0 || src_kind == 1, "ic_pack_int4: src_kind must be 0 (int8) or 1 (f32)");
    hipStream_t st = as_stream(stream);
    IC_CHECK_HIP(hipMemsetAsync(flags, 0, 3 * sizeof(int32_t), st));
    if (rows == 0 || cols == 0) return IC_OK;
    ProfScope prof_scope(st, PT_RTN, 0.0, (double)rows * cols * (src_kind == 0 ? 1.5 : 4.5));
    const bool vec = src_kind == 0 && cols % 32 == 0 && ld_src % 16 == 0 && (uintptr_t)src % 16 == 0 &&
                     (!dst || (ld_dst % 16 == 0 && (uintptr_t)dst % 16 == 0)) && rows * (cols / 32) < (1LL << 31);
    if (vec) {
        const int64_t units = rows * (cols / 32);
        const int grid = (int)std::min<int64_t>(cdiv(units, 256), 4096);
        hipLaunchKernelGGL(pack_int4_vec_kernel, dim3(grid), dim3(256), 0, st, reinterpret_cast<const int8_t*>(src),
                           (uint32_t)rows, (uint32_t)(cols / 32), ld_src, dst, ld_dst, flags);
    } else {
        hipLaunchKernelGGL(pack_int4_kernel, dim3(elem_grid(rows * cdiv(cols, 2))), dim3(256), 0, st, src, src_kind,
                           rows, cols, ld_src, dst, ld_dst, flags);
    }
    IC_CHECK_LAUNCH();
    return IC_OK;
}

extern "C" int ic_unpack_int4(const uint8_t* src, int64_t rows, int64_t k, int64_t ld_src, int8_t* dst,
                              int64_t ld_dst, void* stream) {
    IC_REQUIRE(src && dst && ld_src >= cdiv(k, 2) && ld_dst >= k, "ic_unpack_int4: bad arguments");
    if (rows == 0 || k == 0) return IC_OK;
    hipLaunchKernelGGL(unpack_int4_kernel, dim3(elem_grid(rows * k)), dim3(256), 0, as_stream(stream), src, rows, k,
                       ld_src, dst, ld_dst);
    IC_CHECK_LAUNCH();
    return IC_OK;
}

extern "C" int ic_scale_status(const void* scale, int scale_kind, int64_t n, int32_t* flag, void* stream) {
    IC_REQUIRE(scale && flag, "ic_scale_status: null pointer");
    IC_REQUIRE(scale_kind == 0 || scale_kind == 1, "ic_scale_status: scale_kind must be 0 (f16) or 1 (f32)");
    IC_REQUIRE(n >= 0, "ic_scale_status: negative size");
    hipLaunchKernelGGL(scale_status_kernel, dim3(1), dim3(1024), 0, as_stream(stream), scale, scale_kind, n, flag);
    IC_CHECK_LAUNCH();
    return IC_OK;
}

extern "C" int64_t ic_quant_error_workspace_bytes(void) {
    return QERR_BLOCKS * (int64_t)(sizeof(double) + sizeof(float));
}

extern "C" int ic_quant_error(const float* W, int64_t rows, int64_t cols, int64_t ld, const int8_t* codes,
                              int64_t ld_q, const void* scale, int scale_kind, const int8_t* zp, double* out_sumsq,
                              float* out_maxabs, void* workspace, void* stream) {
    IC_REQUIRE(W && codes && scale && out_sumsq && out_maxabs && workspace, "ic_quant_error: null pointer");
    IC_REQUIRE(ld >= cols && ld_q >= cols, "ic_quant_error: bad leading dimension");
    IC_REQUIRE(scale_kind == 0 || scale_kind == 1, "ic_quant_error: scale_kind must be 0 (f16) or 1 (f32)");
    hipStream_t st = as_stream(stream);
    double* ps = reinterpret_cast<double*>(workspace);
    float* pm = reinterpret_cast<float*>(ps + QERR_BLOCKS);
    ProfScope prof_scope(st, PT_VERIFY, 0.0, (double)rows * cols * 5.0);
    hipLaunchKernelGGL(quant_error_partial, dim3(QERR_BLOCKS), dim3(256), 0, st, W, rows, cols, ld, codes, ld_q,
                       scale, scale_kind, zp, ps, pm);
    IC_CHECK_LAUNCH();
    hipLaunchKernelGGL(quant_error_final, dim3(1), dim3(256), 0, st, ps, pm, QERR_BLOCKS, out_sumsq, out_maxabs);
    IC_CHECK_LAUNCH();
    return IC_OK;
}
