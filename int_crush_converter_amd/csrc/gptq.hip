// GPTQ / LDLQ column sweep and layer driver.
//
// Per block of nb <= 128 columns the reference (converter/rounding.py:37-103,
// converter/ldlq.py:369-417) quantises column j for every row, normalises the
// error by Hinv[j][j] and immediately updates the later columns of the block,
// w_k <- w_k - RN(e_j * Hinv[j][k]); after the block the errors E [M, nb]
// update all later columns at once, W[:, end:] -= E @ Hinv[blk, end:].
//
// Sweep kernel: the nb x nb Hinv block is staged in LDS once per work-group
// of 8 waves; a wave holds 64 / LPR rows of LPR lanes each (LPR = 32 for
// a single matrix, 8 for batched groups).  Lane p of a row slot holds
// columns p + LPR r of its row.  At step j the owners' values are read into
// scalar registers (readlane) and each row slot takes its own, so the LPR
// lanes of a row quantise the same value and the error is uniform per row;
// every
// lane then applies its updates in column order, so every w_k sees exactly
// the reference's sequence of fp32 roundings (bit-exact given the same
// Hinv).  The next Hinv row and the next pivot data are fetched while the
// current column is processed.  A lane owns the codes and errors of its
// columns and stores them at the end.
//
// The lazy trailing update is an fp32-MFMA GEMM (gemm_f32); its summation
// order differs from MKL's sgemm, which is the only non-bit-exact step.
#include <mutex>

#include "gemm.hpp"

namespace icq {

constexpr int SW_NB = 128;     // max columns per sweep block
constexpr int SW_WAVES = 8;
constexpr int SW_THREADS = SW_WAVES * 64;
// Lanes per row: 32 (two rows per wave) when there are few rows, so that
// enough waves share each SIMD to hide the column chain's latency; 8 (eight
// rows per wave) when the launch has many waves per SIMD anyway (batched
// block-diagonal groups), so that the chain's instructions serve more rows.
constexpr int SW_LPR_LATENCY = 32, SW_LPR_THROUGHPUT = 8;
// rows x groups from which the throughput variant (8 rows per wave) is the
// faster one: at 12288 rows its sweeps take 1.49 ms per [12288, 3072] layer
// against 1.98 ms with 2 rows per wave
constexpr int64_t SW_THROUGHPUT_ROWS = 12288;

template <int LPR> constexpr int sw_rows() { return (64 / LPR) * SW_WAVES; }   // rows per work-group

enum SweepMode : int {
    SWEEP_GPTQ = 0,   // per-row scale (+zp), err / Hinv_jj, clamp +-100, NaN -> 0
    SWEEP_LDLQ = 1,   // per-element scale (>= 1e-8), err * (1 / max(Hinv_jj, 1e-8)), no clamp
};

struct SweepArgs {
    float* W; int64_t ldw;          // working weights (block columns start at col0)
    int64_t rows;
    int64_t col0; int nb;
    int64_t gcol;                   // column stride between batched groups
    const float* H; int64_t ldh;    // Hinv block top-left; group stride hg
    int64_t hg;
    const float* s;                 // GPTQ: per-row scale [rows]; LDLQ: per-element [rows, lds]
    int64_t lds;
    const float* zp;                // per-row zero-point (fp32) or null
    float qmin, qmax;
    int8_t* Q; int64_t ldq;         // codes, same column indexing as W
    float* E; int64_t lde; int64_t eg;   // errors [rows, nb] per group (group stride eg)
    int mode;
    // Row sweep only (whole blocks of one matrix): the next block's update by
    // this block's errors, Wn = Cn - E Hinv[blk, next] over 128 columns
    // (pitch ldw), run by the sweep's own work-groups; Hn = Hinv[blk, next]
    // (pitch ldh).  Hn null: no such update.
    const float* Hn = nullptr;
    const float* Cn = nullptr;
    float* Wn = nullptr;
};

__device__ __forceinline__ float rdlanef(float v, int l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

// The value v of lane (k LPR + o) of the wave, for the lane's row slot k.
template <int LPR>
__device__ __forceinline__ float row_owner(float v, int o, int slot) {
    float x = rdlanef(v, o);
#pragma unroll
    for (int k = 1; k < 64 / LPR; ++k) {
        const float y = rdlanef(v, k * LPR + o);
        x = slot == k ? y : x;
    }
    return x;
}

// The column loop of one sweep block for the lane's row slot.  Column
// j = LPR r0 + o lives in register r0 of lane o of each row slot; updates are
// unconditional on registers r >= r0 (the register of column j on lanes <= o
// is already quantised and never read again, so those updates are dead).
//
// EXACT = false: every division takes the fast correctly rounded quotient
// without a per-column test.  It is exact for dividends in [2^-60, 2^61)
// (or 0, and NaN passes through as NaN) and divisors in [2^-30, 2^31).  The
// lane keeps the largest |x| and |x - deq| and the smallest nonzero
// |x - deq| of its columns; a value outside that domain, or a pivot or scale
// outside [2^-30, 2^31) (tested once per block / row), sets `unsafe` and the
// caller redoes the block with EXACT = true, the wave-uniform test of
// div_rn_wave.
template <int MODE, int LPR, bool ZP, bool EXACT>
__device__ __forceinline__ void sweep_cols(float (&w)[SW_NB / LPR], float (&qv)[SW_NB / LPR],
                                           float (&ev)[SW_NB / LPR], const float* sc, const float* scr,
                                           const float* Hs, const float* hjj, const float* dinv, const int* dok,
                                           int nb, int p, int half, float s_row, float s_rrow, bool srow_ok,
                                           float z_row, float qmin, float qmax, bool& unsafe) {
    constexpr int SW_HALF = LPR;
    constexpr int R = SW_NB / LPR;
#pragma unroll
    for (int r = 0; r < R; ++r) qv[r] = ev[r] = 0.0f;
    float h[R];
#pragma unroll
    for (int r = 0; r < R; ++r) h[r] = Hs[r * SW_HALF + p];
    float hd = hjj[0], dvj = dinv[0];
    bool dkj = dok[0] != 0;
    bool bad = false;
    // the fast division's domain, checked once after the block: the largest
    // |dividend| (and |x|, which also covers +-Inf) and the smallest nonzero
    // |dividend| of the lane's columns; NaN passes both paths alike
    float amax = 0.0f, amin = INFINITY;
#pragma unroll
    for (int r0 = 0; r0 < R; ++r0) {
        if (r0 * SW_HALF >= nb) break;
#pragma nounroll
        for (int o = 0; o < SW_HALF; ++o) {
            const int j = r0 * SW_HALF + o;
            if (j >= nb) break;
            const int jn = j + 1 < SW_NB ? j + 1 : j;
            float hn[R];
#pragma unroll
            for (int r = r0; r < R; ++r) hn[r] = Hs[jn * SW_NB + r * SW_HALF + p];
            const float hdn = hjj[jn], dvn = dinv[jn];
            const bool dkn = dok[jn] != 0;
            float q, e;
            if (MODE == SWEEP_GPTQ) {
                // the owner's value of this lane's row
                const float x = row_owner<LPR>(w[r0], o, half);
                float y;
                if (EXACT) {
                    y = div_rn_wave(x, s_row, s_rrow, srow_ok);
                } else {
                    y = div_rn_fast(x, s_row, s_rrow);
                }
                if (ZP) y = y + z_row;
                q = clampf_med3(rhaz_trunc(y), qmin, qmax);
                const float deq = ZP ? (q - z_row) * s_row : q * s_row;
                const float num = x - deq;
                if (EXACT) {
                    e = div_rn_wave(num, hd, dvj, dkj);
                } else {
                    e = div_rn_fast(num, hd, dvj);
                    const float an = fabsf(num);
                    amax = fmaxf(amax, fmaxf(fabsf(x), an));
                    amin = fminf(amin, an == 0.0f ? INFINITY : an);
                }
                e = e != e ? 0.0f : __builtin_amdgcn_fmed3f(e, -100.0f, 100.0f);
            } else {
                // Every lane quantises its own column of register r0 (the
                // owner's is column j) with its own element scale; the
                // owner's error is then broadcast over the row.  The
                // reference's sign-flip correction is inert here: the scales
                // are clamped to >= 1e-8 (or NaN), so the rounded, clamped
                // code has the sign of x or is 0, and it is left out.
                const float x = w[r0], s_el = sc[r0], s_rc = scr[r0];
                float y;
                if (EXACT) {
                    y = div_rn_wave(x, s_el, s_rc, div_b_ok(s_el));
                } else {
                    y = div_rn_fast(x, s_el, s_rc);
                    y = fabsf(x) < 0x1p61f ? y : x * s_rc;
                    bad = bad || !div_b_ok(s_el);
                }
                q = clampf(clampf_med3(rhaz_trunc(y), qmin, qmax), qmin, qmax);
                e = row_owner<LPR>((x - q * s_el) * dvj, o, half);
            }
            const bool own = p == o;
            qv[r0] = own ? q : qv[r0];
            ev[r0] = own ? e : ev[r0];
#pragma unroll
            for (int r = r0; r < R; ++r) w[r] = w[r] - e * h[r];
#pragma unroll
            for (int r = r0; r < R; ++r) h[r] = hn[r];
            hd = hdn;
            dvj = dvn;
            dkj = dkn;
        }
    }
    if (!EXACT && MODE == SWEEP_GPTQ) bad = bad || amax >= 0x1p61f || amin < 0x1p-60f;
    unsafe = unsafe || bad;
}

template <int MODE, int LPR>
__global__ __launch_bounds__(SW_THREADS) void sweep_kernel(SweepArgs a) {
    constexpr int SW_HALF = LPR;
    constexpr int SW_RPW = 64 / LPR;
    constexpr int SW_ROWS = SW_RPW * SW_WAVES;
    constexpr int R = SW_NB / LPR;
    __shared__ float Hs[SW_NB * SW_NB];
    __shared__ float hjj[SW_NB];              // Hinv_jj
    __shared__ float dinv[SW_NB];             // GPTQ: RN(1 / Hinv_jj); LDLQ: 1 / max(Hinv_jj, 1e-8)
    __shared__ int dok[SW_NB];                // GPTQ: Hinv_jj inside the fast-division domain

    const int g = blockIdx.y;
    const int nb = a.nb;
    const int64_t col0 = a.col0 + (int64_t)g * a.gcol;
    const float* H = a.H + (int64_t)g * a.hg;
    const int t = threadIdx.x, lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    {
        // all global loads in flight before the LDS stores
        constexpr int STEP = SW_THREADS / SW_NB, PER = SW_NB / STEP;
        const int c = t & (SW_NB - 1), i0 = t / SW_NB;
        float tmp[PER];
#pragma unroll
        for (int k = 0; k < PER; ++k) {
            const int i = i0 + k * STEP;
            tmp[k] = (i < nb && c < nb) ? H[(int64_t)i * a.ldh + c] : 0.0f;
        }
#pragma unroll
        for (int k = 0; k < PER; ++k) Hs[(i0 + k * STEP) * SW_NB + c] = tmp[k];
    }
    int piv_ok = 1;
    if (t < SW_NB) {
        const int j = t;
        const float hd = j < nb ? H[(int64_t)j * a.ldh + j] : 1.0f;
        float d = hd;
        if (MODE == SWEEP_LDLQ) d = d > 1e-8f ? d : (d != d ? d : 1e-8f);
        hjj[j] = hd;
        dinv[j] = 1.0f / d;
        piv_ok = div_b_ok(d) ? 1 : 0;
        dok[j] = piv_ok;
    }
    // every pivot of the block inside the fast division's domain
    const bool pivots_ok = __syncthreads_and(piv_ok) != 0;
    const int half = lane / SW_HALF, p = lane & (SW_HALF - 1);   // half: the wave's row slot
    const int64_t row0 = (int64_t)blockIdx.x * SW_ROWS + SW_RPW * wave;
    if (row0 >= a.rows) return;                          // all rows of the wave past the end
    const int64_t row = row0 + half;
    const bool rv = row < a.rows;
    const int64_t rrow = rv ? row : row0;                // a row that exists (results not stored)

    float w[R];
    const float* wrow = a.W + rrow * a.ldw + col0;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int c = r * SW_HALF + p;
        w[r] = c < nb ? wrow[c] : 0.0f;
    }
    float s_row = 1.0f, z_row = 0.0f;
    float sc[MODE == SWEEP_LDLQ ? R : 1];
    float scr[MODE == SWEEP_LDLQ ? R : 1];
    if (MODE == SWEEP_GPTQ) {
        s_row = a.s[rrow];
        if (a.zp) z_row = a.zp[rrow];
    } else {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int c = r * SW_HALF + p;
            float v = c < nb ? a.s[rrow * a.lds + col0 + c] : 1.0f;
            v = v > 1e-8f ? v : (v != v ? v : 1e-8f);
            sc[r] = v;
            scr[r] = 1.0f / v;
        }
    }
    const float s_rrow = 1.0f / s_row;
    const bool has_zp = a.zp != nullptr;
    const bool srow_ok = div_b_ok(s_row);

    float qv[R], ev[R];
    float w0[R];
#pragma unroll
    for (int r = 0; r < R; ++r) w0[r] = w[r];
    bool unsafe = MODE == SWEEP_GPTQ && !(srow_ok && pivots_ok);
#define ICQ_COLS(ZP, EXACT) \
    sweep_cols<MODE, LPR, ZP, EXACT>(w, qv, ev, sc, scr, Hs, hjj, dinv, dok, nb, p, half, s_row, s_rrow, srow_ok, \
                                     z_row, a.qmin, a.qmax, unsafe)
    if (has_zp) ICQ_COLS(true, false);
    else ICQ_COLS(false, false);
    // A value outside the fast division's exact domain (none in practice:
    // a weight or residual of magnitude 2^61 or more, a nonzero residual
    // below 2^-60, or a pivot / scale outside [2^-30, 2^31)): the wave runs
    // the block again with the IEEE-exact division test on every column.
    if (__builtin_expect(__builtin_amdgcn_ballot_w64(unsafe) != 0, 0)) {
#pragma unroll
        for (int r = 0; r < R; ++r) w[r] = w0[r];
        if (has_zp) ICQ_COLS(true, true);
        else ICQ_COLS(false, true);
    }
#undef ICQ_COLS
    // codes and errors of the lane's own columns (coalesced per row)
    if (rv) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int c = r * SW_HALF + p;
            if (c < nb) {
                a.Q[row * a.ldq + col0 + c] = (int8_t)(int)qv[r];
                a.E[(int64_t)g * a.eg + row * a.lde + c] = ev[r];
            }
        }
    }
}

// Quad sweep: full 128-column blocks, 4 lanes (a DPP quad) per row, 16 rows
// per wave.  Lane p of a row owns the block
// columns j = 4 m + p (m = 0..31): their weights, codes and errors stay in
// registers.  At column j the owner (p = j mod 4) quantises its weight and
// forms the error, one quad broadcast hands the error to the row's lanes,
// and each lane updates its later columns, w <- w - RN(e Hinv[j][k]) (the
// product rounded, then subtracted, in column order: the reference's
// sequence of roundings).  The column loop is unrolled (the slots are
// registers) and Hinv's next row share and pivot are fetched a column
// ahead.  The other lanes of the quad run the same steps on their own
// columns, results unused, so the common path has no branch.  Division
// uses the fast correctly rounded quotient; a value outside its exact
// domain (as in sweep_cols, plus LDLQ dividends outside [2^-60, 2^61))
// sends the wave's rows through the block once more, one lane per row with
// the row's error output as its working row, with the IEEE-exact test on
// every division (rare).  WV waves share the staged Hinv block; blockIdx.y
// is the column group of a block-diagonal Hessian.
constexpr int SQ_M = SW_NB / 4;   // columns per lane
constexpr int SQ_ROWS = 16;       // rows per wave

// The quad sweep's Hinv block in LDS, packed: row j keeps only the
// 16-column groups g >= j / 16 (the later columns its update reaches), as
// [p][g - j/16] float4s (lane p's four columns 16 g + 4 s + p, s = 0..3):
// 36 KB instead of 64, so four work-groups share a CU.
__host__ __device__ constexpr int qp_row4(int j) {   // float4 offset of row j
    return 4 * (16 * (8 * (j / 16) - (j / 16) * (j / 16 - 1) / 2) + (j % 16) * (8 - j / 16));
}
constexpr int QP_F4 = qp_row4(SW_NB);
static_assert(QP_F4 == 2304, "packed quad-sweep Hinv block");
__device__ __forceinline__ int qp_idx(int j, int c) {   // float index of Hinv[j][c], c >= 16 (j / 16)
    const int m = c >> 2, p = c & 3, g0 = j >> 4;
    return 4 * (qp_row4(j) + p * (8 - g0) + (m >> 2) - g0) + (m & 3);
}

template <int MODE, bool ZP, int WV>
__global__ __launch_bounds__(64 * WV) void sweep4_kernel(SweepArgs a) {
    __shared__ __align__(16) float4 Hq4[QP_F4];          // packed Hinv block (qp_idx)
    __shared__ __align__(16) float4 piv[SW_NB];          // {Hinv_jj, 1 / d_j, d_j in the fast domain, 0}
    const int tid = threadIdx.x, t = tid & 63, p = t & 3;
    const int rw = (tid >> 6) * SQ_ROWS + (t >> 2);      // row within the work-group
    const int g = blockIdx.y;                            // column group (block-diagonal Hessians)
    const int64_t col0 = a.col0 + (int64_t)g * a.gcol;
    const float* Hg = a.H + (int64_t)g * a.hg;
    float* Eg = a.E + (int64_t)g * a.eg;
    {
        // the Hinv block: 32 loads per thread in flight, then their LDS stores
        constexpr int NT = 64 * WV, CH = 32, PER = SW_NB * SW_NB / NT;
#pragma unroll
        for (int k0 = 0; k0 < PER; k0 += CH) {
            float tmp[CH];
#pragma unroll
            for (int k = 0; k < CH; ++k) {
                const int idx = tid + (k0 + k) * NT;
                tmp[k] = Hg[(int64_t)(idx / SW_NB) * a.ldh + (idx % SW_NB)];
            }
#pragma unroll
            for (int k = 0; k < CH; ++k) {
                const int idx = tid + (k0 + k) * NT, i = idx / SW_NB, c = idx % SW_NB;
                if (c >= 16 * (i / 16)) reinterpret_cast<float*>(Hq4)[qp_idx(i, c)] = tmp[k];
            }
        }
        for (int j = tid; j < SW_NB; j += 64 * WV) {
            const float hd = Hg[(int64_t)j * a.ldh + j];
            float d = hd;
            if (MODE == SWEEP_LDLQ) d = d > 1e-8f ? d : (d != d ? d : 1e-8f);
            piv[j] = make_float4(hd, 1.0f / d, div_b_ok(d) ? 1.0f : 0.0f, 0.0f);
        }
    }
    __syncthreads();
    const int64_t row = (int64_t)blockIdx.x * (WV * SQ_ROWS) + rw;
    const bool rv = row < a.rows;
    const int64_t rrow = rv ? row : a.rows - 1;   // a row that exists (results not stored)
    const float* wrow = a.W + rrow * a.ldw + col0;
    float w[SQ_M];
#pragma unroll
    for (int m = 0; m < SQ_M; ++m) w[m] = wrow[4 * m + p];
    float s_row = 1.0f, z_row = 0.0f;
    float sc[MODE == SWEEP_LDLQ ? SQ_M : 1], scr[MODE == SWEEP_LDLQ ? SQ_M : 1];
    if (MODE == SWEEP_GPTQ) {
        s_row = a.s[rrow];
        if (ZP) z_row = a.zp[rrow];
    } else {
#pragma unroll
        for (int m = 0; m < SQ_M; ++m) {
            float v = a.s[rrow * a.lds + col0 + 4 * m + p];
            v = v > 1e-8f ? v : (v != v ? v : 1e-8f);
            sc[m] = v;
            scr[m] = 1.0f / v;
        }
    }
    const float s_rrow = 1.0f / s_row;
    const bool srow_ok = div_b_ok(s_row);
    float qv[SQ_M], ev[SQ_M];
    uint64_t badm = 0;   // LDLQ: lanes with a value outside the fast division's domain
    float amax = 0.0f, amin = INFINITY;   // GPTQ: the dividends' range (amin = 0: a pivot outside)
    float4 pvn = piv[0], hc[SQ_M / 4], hn[SQ_M / 4];
#pragma unroll
    for (int g = 0; g < SQ_M / 4; ++g) hc[g] = Hq4[qp_row4(0) + p * 8 + g];
    auto column = [&](auto J) {
        constexpr int j = decltype(J)::value, m = j / 4, o = j % 4;
        const float4 pv = pvn;
        if constexpr (j + 1 < SW_NB) {
            pvn = piv[j + 1];
#pragma unroll
            for (int g = (j + 1) / 16; g < SQ_M / 4; ++g)
                hn[g] = Hq4[qp_row4(j + 1) + p * (8 - (j + 1) / 16) + g - (j + 1) / 16];
        }
        const float x = w[m];
        float q, e;
        if (MODE == SWEEP_GPTQ) {
            float y = div_rn_fast(x, s_row, s_rrow);
            if (ZP) y = y + z_row;
            q = clampf_med3(rhaz_trunc(y), a.qmin, a.qmax);
            const float deq = ZP ? (q - z_row) * s_row : q * s_row;
            const float num = x - deq;
            e = div_rn_fast(num, pv.x, pv.y);
            const float an = fabsf(num);
            amax = fmaxf(amax, fmaxf(fabsf(x), an));
            amin = fminf(amin, an == 0.0f ? INFINITY : an);
            amin = pv.z == 0.0f ? 0.0f : amin;   // a pivot outside the domain
            __asm__ volatile("" : "+v"(amax), "+v"(amin));   // fold this column in now, not at the end
            e = e != e ? 0.0f : __builtin_amdgcn_fmed3f(e, -100.0f, 100.0f);
        } else {
            const float y = div_rn_fast(x, sc[m], scr[m]);
            const float ax = fabsf(x);
            badm |= __builtin_amdgcn_ballot_w64(!div_b_ok(sc[m]) || ax >= 0x1p61f || (ax < 0x1p-60f && ax != 0.0f));
            __asm__ volatile("" : "+s"(badm));   // fold this column in now, not at the end
            q = clampf(clampf_med3(rhaz_trunc(y), a.qmin, a.qmax), a.qmin, a.qmax);
            e = (x - q * sc[m]) * pv.y;
        }
        const float d = quad_bcast<o>(e);
        if (p == o) {
            qv[m] = q;
            ev[m] = e;
        }
        __asm__ volatile("" : "+v"(qv[m]), "+v"(ev[m]));   // select now: keeps the columns' q, e dead
#pragma unroll
        for (int m2 = m; m2 < SQ_M; ++m2) {
            const float4 h4 = hc[m2 / 4];
            const float hv = m2 % 4 == 0 ? h4.x : m2 % 4 == 1 ? h4.y : m2 % 4 == 2 ? h4.z : h4.w;
            w[m2] = w[m2] - d * hv;
        }
#pragma unroll
        for (int g = 0; g < SQ_M / 4; ++g) hc[g] = hn[g];
        __builtin_amdgcn_sched_barrier(0);   // keep the one-column-ahead loads where they are
    };
    static_for<0, SW_NB>(column);
    const bool bad = MODE == SWEEP_GPTQ ? !srow_ok || amax >= 0x1p61f || amin < 0x1p-60f : false;
    if (__builtin_expect((__builtin_amdgcn_ballot_w64(bad) | badm) != 0, 0)) {
        // the wave's rows again from the block's start, one lane per row,
        // every division IEEE-exact (div_rn tests its domain per value); the
        // row's error output is the working row, and that lane writes the
        // row's codes and errors itself
        __asm__ volatile("" ::: "memory");
        if (rv && p == 0) {
            float* xr = Eg + row * a.lde;
            for (int c = 0; c < SW_NB; ++c) xr[c] = wrow[c];
            for (int j = 0; j < SW_NB; ++j) {
                const float x = xr[j];
                const float4 pv = piv[j];
                float q, e;
                if (MODE == SWEEP_GPTQ) {
                    float y = div_rn(x, s_row, s_rrow, srow_ok);
                    if (ZP) y = y + z_row;
                    q = clampf_med3(rhaz_trunc(y), a.qmin, a.qmax);
                    const float deq = ZP ? (q - z_row) * s_row : q * s_row;
                    e = div_rn(x - deq, pv.x, pv.y, pv.z != 0.0f);
                    e = e != e ? 0.0f : __builtin_amdgcn_fmed3f(e, -100.0f, 100.0f);
                } else {
                    float v = a.s[rrow * a.lds + col0 + j];
                    v = v > 1e-8f ? v : (v != v ? v : 1e-8f);
                    const float y = div_rn(x, v, 1.0f / v, div_b_ok(v));
                    q = clampf(clampf_med3(rhaz_trunc(y), a.qmin, a.qmax), a.qmin, a.qmax);
                    e = (x - q * v) * pv.y;
                }
                a.Q[row * a.ldq + col0 + j] = (int8_t)(int)q;
                xr[j] = e;
                for (int k = j + 1; k < SW_NB; ++k) xr[k] = xr[k] - e * reinterpret_cast<const float*>(Hq4)[qp_idx(j, k)];
            }
        }
        return;
    }
    if (rv) {
#pragma unroll
        for (int m = 0; m < SQ_M; ++m) {
            const int c = 4 * m + p;
            a.Q[row * a.ldq + col0 + c] = (int8_t)(int)qv[m];
            Eg[row * a.lde + c] = ev[m];
        }
    }
}

// Row sweep: full 128-column blocks of one matrix (groups == 1), 16 lanes (a
// DPP row) per row, 4 rows per wave.  Lane p of a row owns the block
// columns j = 16 m + p (m = 0..7): their weights, codes and errors stay in
// registers.  At column j the owner (p = j mod 16) quantises its weight and
// forms the error, one DPP row broadcast (row_newbcast) hands the error to
// the row's lanes, and each lane updates its later columns,
// w <- w - RN(e Hinv[j][k]) (the product rounded, then subtracted, in column
// order: the reference's sequence of roundings).  The column loop is
// unrolled (the slots are registers) and Hinv's next row share and pivot
// are fetched a column ahead.  The other lanes of the row run the same
// steps on their own columns, results unused, so the common path has no
// branch.  Division uses the fast correctly rounded quotient; a value
// outside its exact domain (as in sweep_cols, plus LDLQ dividends outside
// [2^-60, 2^61)) sends the wave's rows through the block once more, one lane
// per row from LDS, with the IEEE-exact test on every division (rare).  WV
// waves share the staged Hinv block.
//
// FUSE: the work-group then applies the next block's update by this block's
// errors to its own rows, W[:, next] = C - E_blk Hinv[blk, next] (the first
// update of the lazy-batch sequence that reaches the next block), on the
// matrix cores: wave w takes rows 16 (w / 4) .. + 15 and columns
// 32 (w % 4) .. + 31, the errors pass through LDS as the A operand, and
// Hinv[blk, next] and C are fetched into registers while the block is swept.
// Every output is formed as gemm_f32 forms it for a single chunk (fresh
// accumulators, one 16x16x4 MFMA step per 4 k in increasing k, then
// -(0 + sum) + C), so the result is that GEMM's bit for bit, without its
// launch.
constexpr int SR_L = 16;             // lanes per row
constexpr int SR_M = SW_NB / SR_L;   // columns per lane
constexpr int SR_ROWS = 64 / SR_L;   // rows per wave

// Lane L's value of v in every lane of its 16-lane DPP row.
template <int L>
__device__ __forceinline__ float row_bcast16(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x150 + L, 0xf, 0xf, false));
}

typedef float f32x4 __attribute__((ext_vector_type(4)));

template <int MODE, bool ZP, int WV, bool FUSE>
__global__ __launch_bounds__(64 * WV) void sweep16_kernel(SweepArgs a) {
    __shared__ __align__(16) float Hq[SW_NB][SR_L][SR_M];   // Hq[j][p][m] = Hinv[j][16 m + p]
    __shared__ __align__(16) float4 piv[SW_NB];          // {Hinv_jj, 1 / d_j, d_j in the fast domain, 0}
    __shared__ float Xr[WV * SR_ROWS][SW_NB + 1];        // exact rerun: weights, then errors
    __shared__ signed char Qr[WV * SR_ROWS][SW_NB];      //              codes
    const int tid = threadIdx.x, t = tid & 63, p = t & (SR_L - 1);
    const int rw = (tid >> 6) * SR_ROWS + t / SR_L;      // row within the work-group
    {
        // the Hinv block: 32 loads per thread in flight (32-bit offsets from
        // the block's corner), then their LDS stores
        constexpr int NT = 64 * WV, CH = 32, ALL = SW_NB * SW_NB;
        const int ldh = (int)a.ldh;   // the block spans < 2^31 elements (launch_sweep checks it)
#pragma unroll 1
        for (int base = 0; base < ALL; base += NT * CH) {
            float tmp[CH];
#pragma unroll
            for (int k = 0; k < CH; ++k) {
                const int idx = base + tid + k * NT;
                tmp[k] = idx < ALL ? a.H[(idx / SW_NB) * ldh + (idx % SW_NB)] : 0.0f;
            }
#pragma unroll
            for (int k = 0; k < CH; ++k) {
                const int idx = base + tid + k * NT, c = idx % SW_NB;
                if (idx < ALL) Hq[idx / SW_NB][c % SR_L][c / SR_L] = tmp[k];
            }
        }
        for (int j = tid; j < SW_NB; j += 64 * WV) {
            const float hd = a.H[(int64_t)j * a.ldh + j];
            float d = hd;
            if (MODE == SWEEP_LDLQ) d = d > 1e-8f ? d : (d != d ? d : 1e-8f);
            piv[j] = make_float4(hd, 1.0f / d, div_b_ok(d) ? 1.0f : 0.0f, 0.0f);
        }
    }
    __syncthreads();
    const int64_t row = (int64_t)blockIdx.x * (WV * SR_ROWS) + rw;
    const bool rv = row < a.rows;
    const int64_t rrow = rv ? row : a.rows - 1;   // a row that exists (results not stored)
    const float* wrow = a.W + rrow * a.ldw + a.col0;
    float w[SR_M];
#pragma unroll
    for (int m = 0; m < SR_M; ++m) w[m] = wrow[SR_L * m + p];
    float s_row = 1.0f, z_row = 0.0f;
    float sc[MODE == SWEEP_LDLQ ? SR_M : 1], scr[MODE == SWEEP_LDLQ ? SR_M : 1];
    if (MODE == SWEEP_GPTQ) {
        s_row = a.s[rrow];
        if (ZP) z_row = a.zp[rrow];
    } else {
#pragma unroll
        for (int m = 0; m < SR_M; ++m) {
            float v = a.s[rrow * a.lds + a.col0 + SR_L * m + p];
            v = v > 1e-8f ? v : (v != v ? v : 1e-8f);
            sc[m] = v;
            scr[m] = 1.0f / v;
        }
    }
    // FUSE: this wave's B operand (Hinv[blk, next], k = 4 s + lane / 16,
    // column 32 (w % 4) + 16 c + lane % 16) and C elements (row
    // 16 (w / 4) + 4 (lane / 16) + v of the work-group, same columns), in
    // flight during the sweep; issued after the sweep's own loads
    const int fw = tid >> 6, frt = fw >> 2, fcol = 32 * (fw & 3) + (t & 15), fk = t >> 4;
    float fb[FUSE ? 2 : 1][FUSE ? SW_NB / 4 : 1], fc[FUSE ? 2 : 1][4];
    if constexpr (FUSE) {
        __builtin_amdgcn_sched_barrier(0);
        const int ldh = (int)a.ldh;   // (SW_NB - 1) ldh + 2 SW_NB < 2^31 (launch_sweep checks it)
#pragma unroll
        for (int s = 0; s < SW_NB / 4; ++s)
#pragma unroll
            for (int c = 0; c < 2; ++c) fb[c][s] = a.Hn[(4 * s + fk) * ldh + fcol + 16 * c];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int64_t r = (int64_t)blockIdx.x * (WV * SR_ROWS) + 16 * frt + 4 * fk + v;
            const float* cr = a.Cn + (r < a.rows ? r : a.rows - 1) * a.ldw + fcol;
            fc[0][v] = cr[0];
            fc[1][v] = cr[16];
        }
        __builtin_amdgcn_sched_barrier(0);
    }
    const float s_rrow = 1.0f / s_row;
    const bool srow_ok = div_b_ok(s_row);
    float qv[SR_M], ev[SR_M];
    uint64_t badm = 0;   // LDLQ: lanes with a value outside the fast division's domain
    float amax = 0.0f, amin = INFINITY;   // GPTQ: the dividends' range (amin = 0: a pivot outside)
    float4 pvn = piv[0], hc[SR_M / 4], hn[SR_M / 4];
    const float4* Hq4 = reinterpret_cast<const float4*>(&Hq[0][p][0]);   // + j * SW_NB / 4
#pragma unroll
    for (int g = 0; g < SR_M / 4; ++g) hc[g] = Hq4[g];
    auto column = [&](auto J) {
        constexpr int j = decltype(J)::value, m = j / SR_L, o = j % SR_L;
        const float4 pv = pvn;
        if constexpr (j + 1 < SW_NB) {
            pvn = piv[j + 1];
#pragma unroll
            for (int g = (j + 1) / (4 * SR_L); g < SR_M / 4; ++g) hn[g] = Hq4[(j + 1) * (SW_NB / 4) + g];
        }
        const float x = w[m];
        float q, e;
        if (MODE == SWEEP_GPTQ) {
            float y = div_rn_fast(x, s_row, s_rrow);
            if (ZP) y = y + z_row;
            q = clampf_med3(rhaz_trunc(y), a.qmin, a.qmax);
            const float deq = ZP ? (q - z_row) * s_row : q * s_row;
            const float num = x - deq;
            e = div_rn_fast(num, pv.x, pv.y);
            const float an = fabsf(num);
            amax = fmaxf(amax, fmaxf(fabsf(x), an));
            amin = fminf(amin, an == 0.0f ? INFINITY : an);
            amin = pv.z == 0.0f ? 0.0f : amin;   // a pivot outside the domain
            __asm__ volatile("" : "+v"(amax), "+v"(amin));   // fold this column in now, not at the end
            e = e != e ? 0.0f : __builtin_amdgcn_fmed3f(e, -100.0f, 100.0f);
        } else {
            const float y = div_rn_fast(x, sc[m], scr[m]);
            const float ax = fabsf(x);
            badm |= __builtin_amdgcn_ballot_w64(!div_b_ok(sc[m]) || ax >= 0x1p61f || (ax < 0x1p-60f && ax != 0.0f));
            __asm__ volatile("" : "+s"(badm));   // fold this column in now, not at the end
            q = clampf(clampf_med3(rhaz_trunc(y), a.qmin, a.qmax), a.qmin, a.qmax);
            e = (x - q * sc[m]) * pv.y;
        }
        const float d = row_bcast16<o>(e);
        if (p == o) {
            qv[m] = q;
            ev[m] = e;
        }
        __asm__ volatile("" : "+v"(qv[m]), "+v"(ev[m]));   // select now: keeps the columns' q, e dead
#pragma unroll
        for (int m2 = m; m2 < SR_M; ++m2) {
            const float4 h4 = hc[m2 / 4];
            const float hv = m2 % 4 == 0 ? h4.x : m2 % 4 == 1 ? h4.y : m2 % 4 == 2 ? h4.z : h4.w;
            w[m2] = w[m2] - d * hv;
        }
#pragma unroll
        for (int g = 0; g < SR_M / 4; ++g) hc[g] = hn[g];
        __builtin_amdgcn_sched_barrier(0);   // keep the one-column-ahead loads where they are
    };
    static_for<0, SW_NB>(column);
    const bool bad = MODE == SWEEP_GPTQ ? !srow_ok || amax >= 0x1p61f || amin < 0x1p-60f : false;
    if (__builtin_expect((__builtin_amdgcn_ballot_w64(bad) | badm) != 0, 0)) {
        // the wave's rows again from the block's start, one lane per row,
        // every division IEEE-exact (div_rn tests its domain per value)
        __asm__ volatile("" ::: "memory");
#pragma unroll
        for (int m = 0; m < SR_M; ++m) Xr[rw][SR_L * m + p] = wrow[SR_L * m + p];
        lds_wave_fence();
        if (p == 0) {
            for (int j = 0; j < SW_NB; ++j) {
                const float x = Xr[rw][j];
                const float4 pv = piv[j];
                float q, e;
                if (MODE == SWEEP_GPTQ) {
                    float y = div_rn(x, s_row, s_rrow, srow_ok);
                    if (ZP) y = y + z_row;
                    q = clampf_med3(rhaz_trunc(y), a.qmin, a.qmax);
                    const float deq = ZP ? (q - z_row) * s_row : q * s_row;
                    e = div_rn(x - deq, pv.x, pv.y, pv.z != 0.0f);
                    e = e != e ? 0.0f : __builtin_amdgcn_fmed3f(e, -100.0f, 100.0f);
                } else {
                    float v = a.s[rrow * a.lds + a.col0 + j];
                    v = v > 1e-8f ? v : (v != v ? v : 1e-8f);
                    const float y = div_rn(x, v, 1.0f / v, div_b_ok(v));
                    q = clampf(clampf_med3(rhaz_trunc(y), a.qmin, a.qmax), a.qmin, a.qmax);
                    e = (x - q * v) * pv.y;
                }
                Qr[rw][j] = (signed char)(int)q;
                Xr[rw][j] = e;
                for (int k = j + 1; k < SW_NB; ++k) Xr[rw][k] = Xr[rw][k] - e * Hq[j][k % SR_L][k / SR_L];
            }
        }
        lds_wave_fence();
#pragma unroll
        for (int m = 0; m < SR_M; ++m) {
            qv[m] = (float)Qr[rw][SR_L * m + p];
            ev[m] = Xr[rw][SR_L * m + p];
        }
    }
    if (rv) {
#pragma unroll
        for (int m = 0; m < SR_M; ++m) {
            const int c = SR_L * m + p;
            a.Q[row * a.ldq + a.col0 + c] = (int8_t)(int)qv[m];
            a.E[row * a.lde + c] = ev[m];
        }
    }
    if constexpr (FUSE) {
        // the errors, row-major in LDS (the rerun rows; a wave rewrites only
        // its own rows, which its rerun has finished with), then every wave's
        // 16 x 32 share of E Hinv[blk, next] with the gemm_f32 operand layout:
        // A[i = lane % 16][k = 4 s + lane / 16], B[k][j = lane % 16],
        // accumulator v at row 4 (lane / 16) + v, column lane % 16
#pragma unroll
        for (int m = 0; m < SR_M; ++m) Xr[rw][SR_L * m + p] = ev[m];
        __syncthreads();
        f32x4 acc0 = {0.0f, 0.0f, 0.0f, 0.0f}, acc1 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int s = 0; s < SW_NB / 4; ++s) {
            const float av = Xr[16 * frt + (t & 15)][4 * s + fk];
            acc0 = __builtin_amdgcn_mfma_f32_16x16x4f32(av, fb[0][s], acc0, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_f32_16x16x4f32(av, fb[1][s], acc1, 0, 0, 0);
        }
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int64_t r = (int64_t)blockIdx.x * (WV * SR_ROWS) + 16 * frt + 4 * fk + v;
            if (r < a.rows) {
                float* wr = a.Wn + r * a.ldw + fcol;
                // gemm_f32's single-chunk epilogue: run = 0 + sum; C <- -run + C
                const float run0 = 0.0f + acc0[v], run1 = 0.0f + acc1[v];
                wr[0] = -run0 + fc[0][v];
                wr[16] = -run1 + fc[1][v];
            }
        }
    }
}

// Waves per work-group of the row sweep for `rows` rows (4 rows per wave,
// one work-group per CU where that covers the rows).
static int row_sweep_waves(int64_t rows) {
    const int64_t need = cdiv(cdiv(rows, SR_ROWS), 256);
    return need <= 4 ? 4 : need <= 8 ? 8 : need <= 12 ? 12 : 16;
}

// Whether the row sweep takes the next block's update (SweepArgs::Hn): whole
// blocks of one matrix, at most 12 waves per work-group (the fetched operands
// take 72 more registers per lane), and 32-bit offsets across the two Hinv
// blocks.
static bool row_sweep_fuses(int64_t rows, int groups, int nb, int64_t ldh) {
    return groups == 1 && nb == SW_NB && row_sweep_waves(rows) <= 12 &&
           (SW_NB - 1) * ldh + 2 * SW_NB < (int64_t(1) << 31);
}

static int launch_sweep(const SweepArgs& a, int groups, hipStream_t st) {
    IC_REQUIRE(a.nb >= 1 && a.nb <= SW_NB, "sweep: block size must be in [1, 128]");
    IC_REQUIRE(!a.Hn || row_sweep_fuses(a.rows, groups, a.nb, a.ldh), "sweep: no fused update for this shape");
    const bool wide = a.rows * groups >= SW_THROUGHPUT_ROWS;
    const int64_t wgs = cdiv(a.rows, wide ? sw_rows<SW_LPR_THROUGHPUT>() : sw_rows<SW_LPR_LATENCY>());
    ProfScope prof_scope(st, PT_SWEEP, (double)groups * a.rows * a.nb * (a.nb - 1.0),
                 (double)groups * (a.rows * a.nb * 9.0 + 4.0 * a.nb * a.nb));
    if (groups > 1 && a.nb == SW_NB) {
        // batched column groups (block-diagonal Hessians): many work-groups per
        // CU over the launch, where the quad sweep's few instructions per
        // row and column count (two work-groups per CU)
        const dim3 g4((unsigned)cdiv(a.rows, 4 * SQ_ROWS), (unsigned)groups);
        const bool zp = a.zp != nullptr;
#define ICQ_SWEEP4(M, Z) hipLaunchKernelGGL((sweep4_kernel<M, Z, 4>), g4, dim3(256), 0, st, a)
        // (LDLQ always sweeps one matrix: ic_ldlq_quantize passes groups = 1)
        IC_REQUIRE(a.mode == SWEEP_GPTQ, "sweep: batched column groups are GPTQ only");
        if (zp) ICQ_SWEEP4(SWEEP_GPTQ, true);
        else ICQ_SWEEP4(SWEEP_GPTQ, false);
#undef ICQ_SWEEP4
        IC_CHECK_LAUNCH();
        return IC_OK;
    }
    if (groups == 1 && a.nb == SW_NB) {
        // whole blocks of one matrix: the row sweep (16 lanes per row), with
        // 4 to 16 waves per work-group sharing the staged Hinv block, as many
        // as one work-group per CU needs to cover the rows
        // the kernel addresses the staged Hinv block with 32-bit offsets
        IC_REQUIRE((SW_NB - 1) * a.ldh + SW_NB < (int64_t(1) << 31), "sweep: Hinv pitch too large");
        const int WVs = row_sweep_waves(a.rows);
        const dim3 g16((unsigned)cdiv(a.rows, WVs * SR_ROWS));
        const bool zp = a.zp != nullptr;
#define ICQ_SWEEP16(M, Z, W, F) hipLaunchKernelGGL((sweep16_kernel<M, Z, W, F>), g16, dim3(64 * W), 0, st, a)
#define ICQ_SWEEP16_WV(M, Z)                                   \
    if (a.Hn) {                                                \
        switch (WVs) {                                         \
            case 4: ICQ_SWEEP16(M, Z, 4, true); break;         \
            case 8: ICQ_SWEEP16(M, Z, 8, true); break;         \
            default: ICQ_SWEEP16(M, Z, 12, true); break;       \
        }                                                      \
    } else {                                                   \
        switch (WVs) {                                         \
            case 4: ICQ_SWEEP16(M, Z, 4, false); break;        \
            case 8: ICQ_SWEEP16(M, Z, 8, false); break;        \
            case 12: ICQ_SWEEP16(M, Z, 12, false); break;      \
            default: ICQ_SWEEP16(M, Z, 16, false); break;      \
        }                                                      \
    }
        if (a.mode == SWEEP_GPTQ) {
            if (zp) ICQ_SWEEP16_WV(SWEEP_GPTQ, true)
            else ICQ_SWEEP16_WV(SWEEP_GPTQ, false)
        } else {
            ICQ_SWEEP16_WV(SWEEP_LDLQ, false)
        }
#undef ICQ_SWEEP16_WV
#undef ICQ_SWEEP16
        IC_CHECK_LAUNCH();
        return IC_OK;
    }
    const dim3 grid((unsigned)wgs, (unsigned)groups);
#define ICQ_SWEEP(M, L) hipLaunchKernelGGL((sweep_kernel<M, L>), grid, dim3(SW_THREADS), 0, st, a)
    if (a.mode == SWEEP_GPTQ) {
        if (wide) ICQ_SWEEP(SWEEP_GPTQ, SW_LPR_THROUGHPUT);
        else ICQ_SWEEP(SWEEP_GPTQ, SW_LPR_LATENCY);
    } else {
        if (wide) ICQ_SWEEP(SWEEP_LDLQ, SW_LPR_THROUGHPUT);
        else ICQ_SWEEP(SWEEP_LDLQ, SW_LPR_LATENCY);
    }
#undef ICQ_SWEEP
    IC_CHECK_LAUNCH();
    return IC_OK;
}

// Per-row GPTQ parameters from row min / max / absmax
// (converter/gptq.py:254-317): fp32 scale, fp32 zero-point, and their
// stored forms (fp16 scale bits, int8 zero-point).
__global__ void gptq_params_kernel(const float* rmin, const float* rmax, const float* ramax, int64_t rows, int bits,
                                   int asym, float* s32, float* z32, uint16_t* s16, int8_t* z8) {
    for (int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; r < rows; r += (int64_t)gridDim.x * blockDim.x) {
        float s, z = 0.0f;
        if (bits == 4 || asym) {
            const float qmin = bits == 4 ? -8.0f : -128.0f, qmax = bits == 4 ? 7.0f : 127.0f;
            const float spread = bits == 4 ? 15.0f : 255.0f;
            const float mn = rmin[r], mx = rmax[r];
            s = clampf((mx - mn) / spread, 1e-5f, 65500.0f);
            const float zraw = qmin - rhaz(mn / s);
            const bool lo = zraw < qmin, hi = zraw > qmax;
            if (lo) { float f = clampf(mx / spread, 1e-5f, 65500.0f); s = (s != s || s > f) ? s : f; }
            if (hi) { float f = clampf(-mn / spread, 1e-5f, 65500.0f); s = (s != s || s > f) ? s : f; }
            z = clampf(qmin - rhaz(mn / s), qmin, qmax);
            if (mn == 0.0f && mx == 0.0f) z = 0.0f;
            if (z8) z8[r] = (int8_t)(int)z;
            if (z32) z32[r] = z;
        } else {
            s = clampf(ramax[r] / 127.0f, 1e-5f, 65500.0f);
        }
        s32[r] = s;
        if (s16) s16[r] = f32_to_f16_bits(s);
    }
}

// Whole-layer sweep for `groups` independent column groups of width gw
// (groups == 1, gw == N: full 2-D Hessian; 3-D: one group per Hessian block).
// Hinv of group g starts at Hinv + g * hg with pitch ldh.  E is scratch of
// groups * rows * min(B,128) floats.
// Two-level lazy update.  Columns are taken in super-blocks of up to
// SUPER columns (one group when groups > 1).  Inside a super-block, the
// errors of the blocks reach the later blocks of the super-block in a
// Fenwick order (layer_sweep); the columns after it receive one update
// with all of its errors at once,
// W[:, end:] -= E_sb @ Hinv[sb, end:], a GEMM with K = SUPER.  Same flops
// as one update per block, with the trailing matrix read and written once
// per super-block instead of once per block.
constexpr int SUPER = 1024;

static int64_t super_cols(int64_t groups, int block) {
    const int64_t b = std::min<int64_t>(std::max(block, 1), SW_NB);
    return groups == 1 ? std::max<int64_t>(b, (SUPER / b) * b) : b;
}

// Win: the weights as given; W: the working weights.  With Win != W, W's
// initial contents are never read: the first block is swept from Win, and
// the first update of every other column (the one after the first block,
// and the trailing one after the first super-block) reads Win and writes W,
// so no copy of the layer is made (W == Win: in place).
static int layer_sweep(const float* Win, float* W, int64_t ldw, int64_t rows, int64_t gw, int64_t groups,
                       const float* Hinv, int64_t ldh, int64_t hg, const float* s, int64_t lds, const float* zp,
                       float qmin, float qmax, int B, int8_t* Q, int64_t ldq, float* E, int mode, hipStream_t st) {
    IC_REQUIRE(B >= 1 && B <= SW_NB, "block size must be in [1, 128]");
    const int64_t SB = super_cols(groups, B);   // error matrix E: [groups][rows][SB]
    // W[:, c0 : c0+nc] -= E[:, e0 : e0+k] @ Hinv[h0 : h0+k, c0 : c0+nc]   (per group)
    // the GEMM subtracts its K range chunk by chunk; with chunks of one block
    // every weight receives the per-block updates W -= E_b Hinv[b, :] of the
    // reference in its order (block sizes 32, 64, 128)
    const int kc = (B == 32 || B == 64 || B == 128) ? B : 128;
    auto update = [&](int64_t e0, int64_t h0, int64_t k, int64_t c0, int64_t nc, bool first) {
        GemmArgs ga{rows, nc, k, -1.0f, 1.0f, E + e0, SB, rows * SB, Hinv + h0 * ldh + c0, ldh, hg,
                    W + c0, ldw, gw, 0, 0, CMASK_FULL, KR_FULL, groups, PT_GEMM_TRAIL};
        ga.kc = kc;
        ga.chunk_sub = 1;   // the reference's per-block updates, one after the other
        if (first && Win != W) ga.Cin = Win + c0;
        return gemm_f32(ga, st);
    };
    for (int64_t sb0 = 0; sb0 < gw; sb0 += SB) {
        const int64_t sbe = std::min<int64_t>(gw, sb0 + SB);
        for (int64_t b0 = sb0, j = 0; b0 < sbe; b0 += B, ++j) {
            const int nb = (int)std::min<int64_t>(B, sbe - b0);
            // the sweep reads W (never writes it); the first block is read from Win
            SweepArgs a{b0 == 0 ? const_cast<float*>(Win) : W, ldw, rows, b0, nb, gw, Hinv + b0 * ldh + b0, ldh,
                        hg, s, lds, zp, qmin, qmax, Q, ldq, E + (b0 - sb0), SB, rows * SB, mode};
            // Fenwick order inside the super-block: after block j, the errors
            // of blocks j - lb + 1 .. j (lb = lowest set bit of j + 1) go to
            // blocks j + 1 .. j + lb.  Every block m receives the errors of
            // blocks 0 .. m - 1 once each, in increasing order (the ranges of
            // the binary digits of m), so its weights see the reference's
            // per-block updates in the reference's order, while the columns
            // rewritten per super-block fall from (n - 1) n / 2 blocks to
            // about n log2(n) / 2.  Blocks before the last one are whole.
            const int64_t lb = (j + 1) & -(j + 1);
            const int64_t c0 = b0 + nb, c1 = std::min<int64_t>(sbe, b0 + nb + (lb - 1) * B + B);
            const int64_t e0 = (j + 1 - lb) * B;
            const bool first = sb0 == 0 && e0 == 0;
            // lb = 1 with a whole next block: the update is this block's errors
            // times Hinv[blk, next] (K = one chunk of 128), which the row sweep
            // applies itself
            const bool fused = lb == 1 && c1 - c0 == SW_NB && row_sweep_fuses(rows, (int)groups, nb, ldh);
            if (fused) {
                a.Hn = Hinv + b0 * ldh + c0;
                a.Cn = (first && Win != W ? Win : W) + c0;
                a.Wn = W + c0;
            }
            int rc = launch_sweep(a, (int)groups, st);
            if (rc) return rc;
            if (c0 < c1 && !fused) {
                rc = update(e0, sb0 + e0, (j + 1) * B - e0, c0, c1 - c0, first);
                if (rc) return rc;
            }
        }
        if (sbe < gw) {
            int rc = update(0, sb0, sbe - sb0, sbe, gw - sbe, sb0 == 0);
            if (rc) return rc;
        }
    }
    return IC_OK;
}

}  // namespace icq

using namespace icq;

extern "C" int ic_gptq_row_params(const float* rmin, const float* rmax, const float* ramax, int64_t rows, int bits,
                                  int asym, float* s32, float* z32, uint16_t* s16, int8_t* z8, void* stream) {
    IC_REQUIRE(s32, "ic_gptq_row_params: null scale output");
    IC_REQUIRE(bits == 4 || bits == 8, "ic_gptq_row_params: bits must be 4 or 8");
    IC_REQUIRE((bits == 8 && !asym) ? ramax != nullptr : (rmin && rmax), "ic_gptq_row_params: missing stats");
    if (rows == 0) return IC_OK;
    int grid = (int)std::min<int64_t>(cdiv(rows, 256), 4096);
    hipLaunchKernelGGL(gptq_params_kernel, dim3(grid), dim3(256), 0, as_stream(stream), rmin, rmax, ramax, rows, bits,
                       asym, s32, z32, s16, z8);
    IC_CHECK_LAUNCH();
    return IC_OK;
}

extern "C" int64_t ic_gptq_workspace_bytes(int64_t rows, int64_t groups, int block) {
    return groups * rows * super_cols(groups, block) * (int64_t)sizeof(float) + 256;
}

extern "C" int ic_gptq_quantize(float* W, int64_t rows, int64_t gw, int64_t groups, const float* Hinv,
                                const float* s32, const float* z32, int bits, int block, int8_t* Q,
                                void* workspace, void* stream) {
    IC_REQUIRE(W && Hinv && s32 && Q && workspace, "ic_gptq_quantize: null pointer");
    IC_REQUIRE(bits == 4 || bits == 8, "ic_gptq_quantize: bits must be 4 or 8");
    IC_REQUIRE(groups >= 1 && gw >= 0 && rows >= 0, "ic_gptq_quantize: bad size");
    if (rows == 0 || gw == 0) return IC_OK;
    const float qmin = bits == 4 ? -8.0f : -128.0f, qmax = bits == 4 ? 7.0f : 127.0f;
    const int64_t N = gw * groups;
    return layer_sweep(W, W, N, rows, gw, groups, Hinv, gw, gw * gw, s32, 0, z32, qmin, qmax, block, Q, N,
                       reinterpret_cast<float*>(workspace), SWEEP_GPTQ, as_stream(stream));
}

extern "C" int ic_gptq_quantize_from(const float* W_in, float* W, int64_t rows, int64_t gw, int64_t groups,
                                     const float* Hinv, const float* s32, const float* z32, int bits, int block,
                                     int8_t* Q, void* workspace, void* stream) {
    IC_REQUIRE(W_in && W && Hinv && s32 && Q && workspace, "ic_gptq_quantize_from: null pointer");
    IC_REQUIRE(bits == 4 || bits == 8, "ic_gptq_quantize_from: bits must be 4 or 8");
    IC_REQUIRE(groups >= 1 && gw >= 0 && rows >= 0, "ic_gptq_quantize_from: bad size");
    if (rows == 0 || gw == 0) return IC_OK;
    const float qmin = bits == 4 ? -8.0f : -128.0f, qmax = bits == 4 ? 7.0f : 127.0f;
    const int64_t N = gw * groups;
    return layer_sweep(W_in, W, N, rows, gw, groups, Hinv, gw, gw * gw, s32, 0, z32, qmin, qmax, block, Q, N,
                       reinterpret_cast<float*>(workspace), SWEEP_GPTQ, as_stream(stream));
}

// ------------------------------------------------ allocation-free GPTQ sweep
// For callers that cannot allocate device memory (HIP graph capture, serving
// loops): the error matrix E of the lazy update lives in a static device
// array of NOALLOC_SCRATCH_BYTES per GPU (held until the process ends),
// whose address is looked up once per device.  In host code `scratch` only
// names the symbol; its device address is the one hipGetSymbolAddress
// returns.  Every call on a GPU shares that GPU's array, so calls that
// overlap on one GPU race.  Nothing in it needs to start at zero: the sweep
// writes every error column a lazy update reads.
constexpr int64_t NOALLOC_SCRATCH_BYTES = int64_t(128) << 20;
constexpr int NOALLOC_MAX_DEVICES = 64;
static __device__ __align__(256) unsigned char scratch[NOALLOC_SCRATCH_BYTES];
static void* g_scratch_ptr[NOALLOC_MAX_DEVICES] = {};
static std::mutex g_scratch_mu;

static int scratch_address(void** out) {
    int dev = -1;
    IC_CHECK_HIP(hipGetDevice(&dev));
    IC_REQUIRE(dev >= 0 && dev < NOALLOC_MAX_DEVICES, "ic_gptq_quantize_noalloc: device index out of range");
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        IC_CHECK_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        IC_REQUIRE(p != nullptr, "ic_gptq_quantize_noalloc: no device address for the scratch array");
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return IC_OK;
}

extern "C" int64_t ic_gptq_noalloc_scratch_bytes(void) { return NOALLOC_SCRATCH_BYTES; }

extern "C" int ic_gptq_quantize_noalloc(float* W, int64_t rows, int64_t gw, int64_t groups, const float* Hinv,
                                        const float* s32, const float* z32, int bits, int block, int8_t* Q,
                                        void* stream) {
    IC_REQUIRE(W && Hinv && s32 && Q, "ic_gptq_quantize_noalloc: null pointer");
    IC_REQUIRE(bits == 4 || bits == 8, "ic_gptq_quantize_noalloc: bits must be 4 or 8");
    IC_REQUIRE(groups >= 1 && gw >= 0 && rows >= 0, "ic_gptq_quantize_noalloc: bad size");
    if (rows == 0 || gw == 0) return IC_OK;
    IC_REQUIRE(block >= 1 && block <= SW_NB, "ic_gptq_quantize_noalloc: block size must be in [1, 128]");
    {
        // groups x rows x super-block columns floats must fit; bounded by
        // division so that no product can overflow
        const int64_t cap = NOALLOC_SCRATCH_BYTES / (int64_t)sizeof(float), sc = super_cols(groups, block);
        IC_REQUIRE(sc >= 1 && rows <= cap / sc && groups <= cap / (rows * sc),
                   "ic_gptq_quantize_noalloc: rows x groups x super-block columns need more than the 128 MiB "
                   "static scratch; use ic_gptq_quantize with a workspace");
    }
    void* ws = nullptr;
    int rc = scratch_address(&ws);
    if (rc) return rc;
    ProfSuppress no_events;   // a recording profiler scope would create HIP events
    const float qmin = bits == 4 ? -8.0f : -128.0f, qmax = bits == 4 ? 7.0f : 127.0f;
    const int64_t N = gw * groups;
    return layer_sweep(W, W, N, rows, gw, groups, Hinv, gw, gw * gw, s32, 0, z32, qmin, qmax, block, Q, N,
                       reinterpret_cast<float*>(ws), SWEEP_GPTQ, as_stream(stream));
}

extern "C" int ic_ldlq_quantize(float* W, int64_t rows, int64_t N, const float* Hinv, const float* scales,
                                int bits, int block, int8_t* Q, void* workspace, void* stream) {
    IC_REQUIRE(W && Hinv && scales && Q && workspace, "ic_ldlq_quantize: null pointer");
    IC_REQUIRE(bits == 4 || bits == 8, "ic_ldlq_quantize: bits must be 4 or 8");
    if (rows == 0 || N == 0) return IC_OK;
    const float qmin = bits == 4 ? -8.0f : -128.0f, qmax = bits == 4 ? 7.0f : 127.0f;
    return layer_sweep(W, W, N, rows, N, 1, Hinv, N, N * N, scales, N, nullptr, qmin, qmax, block, Q, N,
                       reinterpret_cast<float*>(workspace), SWEEP_LDLQ, as_stream(stream));
}
