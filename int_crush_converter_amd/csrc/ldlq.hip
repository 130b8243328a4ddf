// LDLQ helpers (per-element scales, iteration MSE, scale refinement,
// least-squares row scales) and the full-rank greedy coordinate descent.
//
// Greedy (converter/greedy.py:487-541): for every column j, every row picks
// the grid value minimising (e+d)^2 H_jj + 2 (e+d) cross, cross =
// err . H[j, :] - e_j H_jj.  Columns are processed in blocks of 64: one
// fp32-MFMA GEMM gives err @ H[blk, :]^T for the whole block at its start,
// and the changes d_j' of earlier columns of the block are added exactly as
// sum_j' d_j' H[j', j] - the same quantity in exact arithmetic as the
// reference's per-column GEMV (its fp32 rounding differs).
#include "gemm.hpp"
#include "torchsum.hpp"

namespace icq {

constexpr int GB = 64;          // greedy column block
constexpr int GL = 16;          // lanes per row in the greedy block kernel

__device__ __forceinline__ float nclampmin(float x, float lo) { return x != x ? x : (x < lo ? lo : x); }

// s_r = max(absmax_r / div, 1e-5) (no upper clamp, ldlq.py:212); S = broadcast
__global__ void ldlq_init_scales_kernel(const float* ramax, int64_t rows, int64_t cols, float div, float* srow,
                                        float* S) {
    const int64_t total = rows * cols;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = i / cols;
        const float s = nclampmin(ramax[r] / div, 1e-5f);
        S[i] = s;
        if (i - r * cols == 0 && srow) srow[r] = s;
    }
}

// Non-finite scales -> nan_to_num(nan=1e-8, posinf=1e30, neginf=1e-8).clamp(min=1e-8)
__global__ void sanitize_scales_kernel(float* S, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        float v = S[i];
        if (v != v) v = 1e-8f;
        else if (isinf(v)) v = v > 0 ? 1e30f : 1e-8f;
        S[i] = v < 1e-8f ? 1e-8f : v;
    }
}

// partial sums of (W - Q*S)^2 in fp64 (product and difference in fp32)
__global__ __launch_bounds__(256) void ldlq_mse_kernel(const float* W, const int8_t* Q, const float* S, int64_t n,
                                                       double* part) {
    double acc = 0.0;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        float d = W[i] - (float)Q[i] * S[i];
        acc += (double)d * (double)d;
    }
    __shared__ double sh[4];
    acc = wave_sum(acc);
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) part[blockIdx.x] = sh[0] + sh[1] + sh[2] + sh[3];
}

__global__ __launch_bounds__(256) void sum_parts_kernel(const double* part, int n, double* out) {
    double a = 0.0;
    for (int i = threadIdx.x; i < n; i += blockDim.x) a += part[i];
    __shared__ double sh[4];
    a = wave_sum(a);
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = a;
    __syncthreads();
    if (threadIdx.x == 0) *out = (sh[0] + sh[1]) + (sh[2] + sh[3]);
}

// converter/ldlq.py:553-599
__global__ void ldlq_update_kernel(const float* W, const int8_t* Q, const float* cur, const float* flat, int64_t n,
                                   float momentum, float lo, float hi, float* out) {
    const float keep = 1.0f - momentum;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        const float w = W[i], q = (float)Q[i];
        const bool nonzero = q != 0.0f;
        const bool consistent = fabsf(w) > 1e-8f && (w * q) > 0.0f;
        float v = cur[i];
        if (nonzero && consistent) {
            float comp = clampf(fabsf(w) / fabsf(q), lo, hi);
            v = momentum > 0.0f ? momentum * cur[i] + keep * comp : comp;
        } else if (nonzero) {
            v = clampf(flat[i], lo, hi);
        }
        out[i] = v;
    }
}

// Per-row least squares scale clamp(sum(q w) / max(sum(q q), 1e-8), min=1e-5)
// (ldlq.py:227-231, 262-265).  The reference sums the fp32 products
// (Q_float * W, Q_float * Q_float) over each row with torch's CPU inner
// sum (one CPU thread per row when there is more than one row), so the
// sums here follow that order: lane s (< 32) of a row's wave takes
// sequence s of the numerator, lane 32 + s that of the denominator, and one
// lane per sum finishes it (the leftover vectors, the merge, the leftover
// scalars, the lanes).  A wave per row, four rows per work-group.
__global__ __launch_bounds__(256) void ls_scales_kernel(const int8_t* Q, const float* W, int64_t rows, int64_t cols,
                                                        float* out) {
    __shared__ float part[4][2][SUM_SEQ];
    __shared__ float dens[4];
    const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t r0 = (int64_t)blockIdx.x * 4 + wv;
    const bool live = r0 < rows;
    const int64_t r = live ? r0 : rows - 1;
    const int8_t* q = Q + r * cols;
    const float* w = W + r * cols;
    auto xn = [&](int64_t i) { const float qf = (float)q[i]; return qf * w[i]; };
    auto xd = [&](int64_t i) { const float qf = (float)q[i]; return qf * qf; };
    const int which = lane >> 5, s = lane & (SUM_SEQ - 1);
    float sum = 0.0f;
    if (cols >= SUM_VEC) {
        const int64_t n4 = cols / SUM_VEC / 4;
        const int lp = cascade_lp(n4);
        part[wv][which][s] = which == 0 ? cascade_seq([&](int64_t m) { return xn(m * SUM_SEQ + s); }, n4, lp)
                                        : cascade_seq([&](int64_t m) { return xd(m * SUM_SEQ + s); }, n4, lp);
        __syncthreads();
        if (s == 0) sum = which == 0 ? inner_sum_finish(part[wv][0], xn, cols) : inner_sum_finish(part[wv][1], xd, cols);
    } else {
        __syncthreads();
        if (s == 0) sum = which == 0 ? inner_sum_short(xn, cols) : inner_sum_short(xd, cols);
    }
    if (lane == 32) dens[wv] = sum;
    __syncthreads();
    if (lane == 0 && live) {
        float d32 = dens[wv];
        d32 = d32 < 1e-8f ? 1e-8f : d32;
        out[r] = nclampmin(sum / d32, 1e-5f);
    }
}

// err = Q * S - W  (S is per-row here: greedy uses least-squares row scales)
__global__ void greedy_err_kernel(const int8_t* Q, const float* srow, const float* W, int64_t rows, int64_t cols,
                                  float* err, float* Qf) {
    const int64_t total = rows * cols;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const float q = (float)Q[i];
        Qf[i] = q;
        err[i] = q * srow[i / cols] - W[i];
    }
}

// One 64-column block of a greedy pass for GROWS rows.  The block's err,
// codes and cross terms are staged in LDS (all loads in flight at once), so
// the column loop touches no global memory; at the end the new err and codes
// and the changes d (D [rows, 64]) are written back.  C holds, for the
// block's columns, err @ H[:, j] as of the start of the block.
// GL lanes per row: lane l keeps the changes d_j' of the columns
// j' = l (mod GL) and their share of the correction sum, and scans the
// candidates g = qmin + l + GL m in increasing order; the lanes' best
// (cost, g) pairs are then merged, the lower g winning a tie, which is the
// sequential first-minimum scan.  H is the matrix of the cross terms (the
// Hessian, or its low-rank truncation) and hd its exact diagonal H_jj (null:
// the diagonal of H).
constexpr int GROWS = 256 / GL;
constexpr int GSTAGE = GROWS * GB / 256;   // staged elements per thread

// Exchanges inside a 16-lane DPP row (one greedy row): rotations by 8 and 4
// within the row, then quad swaps; after the four steps of a commutative,
// associative merge every lane of the row holds the merge of all 16.
template <int CTRL>
__device__ __forceinline__ float rdpp(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xf, 0xf, true));
}
constexpr int DPP_ROR8 = 0x128, DPP_ROR4 = 0x124, DPP_QXOR2 = 0x4E, DPP_QXOR1 = 0xB1;
static_assert(GL == 16, "the row exchanges assume one greedy row per 16-lane DPP row");

__device__ __forceinline__ float row_sum16(float v) {
    v = v + rdpp<DPP_ROR8>(v);
    v = v + rdpp<DPP_ROR4>(v);
    v = v + rdpp<DPP_QXOR2>(v);
    return v + rdpp<DPP_QXOR1>(v);
}

// Merge (cost, g) pairs: the lower cost, on a tie the lower g (branch-free).
template <int CTRL>
__device__ __forceinline__ void argmin_step(float& best, float& bq) {
    const float ob = rdpp<CTRL>(best), oq = rdpp<CTRL>(bq);
    const bool take = (ob < best) | ((ob == best) & (oq < bq));
    best = take ? ob : best;
    bq = take ? oq : bq;
}

template <int NG>
__global__ __launch_bounds__(256) void greedy_block_kernel(float* err, float* Qf, const float* srow, const float* H,
                                                           int64_t ldh, const float* hd, const float* C,
                                                           int64_t ldc, float* D, int64_t rows, int64_t cols,
                                                           int64_t j0, int nb, float qmin, float qmax) {
    constexpr int HP = GB + 1;                 // pitch of the transposed H tile
    __shared__ float HsT[GB * HP];             // HsT[j][j'] = H[j0 + j'][j0 + j]
    __shared__ float Es[GROWS][GB + 1];
    __shared__ float Qs[GROWS][GB + 1];
    __shared__ float Cs[GROWS][GB + 1];
    __shared__ float hds[GB];
    const int t = threadIdx.x;
    const int64_t r0 = (int64_t)blockIdx.x * GROWS;
    if (t < GB) hds[t] = t < nb ? (hd ? hd[j0 + t] : H[(j0 + t) * ldh + j0 + t]) : 1.0f;
    {
        float e[GSTAGE], q[GSTAGE], c[GSTAGE], h[GB * GB / 256];
#pragma unroll
        for (int k = 0; k < GSTAGE; ++k) {
            const int idx = t + 256 * k, rr = idx / GB, cc = idx % GB;
            const int64_t r = r0 + rr;
            const bool ok = r < rows && cc < nb;
            e[k] = ok ? err[r * cols + j0 + cc] : 0.0f;
            q[k] = ok ? Qf[r * cols + j0 + cc] : 0.0f;
            c[k] = ok ? C[r * ldc + cc] : 0.0f;
        }
#pragma unroll
        for (int k = 0; k < GB * GB / 256; ++k) {
            const int idx = t + 256 * k, a = idx / GB, b = idx % GB;
            h[k] = (a < nb && b < nb) ? H[(j0 + a) * ldh + j0 + b] : 0.0f;
        }
#pragma unroll
        for (int k = 0; k < GSTAGE; ++k) {
            const int idx = t + 256 * k, rr = idx / GB, cc = idx % GB;
            Es[rr][cc] = e[k];
            Qs[rr][cc] = q[k];
            Cs[rr][cc] = c[k];
        }
#pragma unroll
        for (int k = 0; k < GB * GB / 256; ++k) {
            const int idx = t + 256 * k, a = idx / GB, b = idx % GB;
            HsT[b * HP + a] = h[k];
        }
    }
    __syncthreads();
    const int lane = t % GL, rr = t / GL;
    const int64_t r = r0 + rr;
    const float s = r < rows ? srow[r] : 1.0f;
    float dl[GB / GL];
#pragma unroll
    for (int i = 0; i < GB / GL; ++i) dl[i] = 0.0f;
    // operands of column 0; each iteration fetches those of the next column
    float hv[GB / GL];
#pragma unroll
    for (int i = 0; i < GB / GL; ++i) hv[i] = HsT[i * GL + lane];
    float e = Es[rr][0], qo = Qs[rr][0], cc0 = Cs[rr][0], hjj = hds[0];
    for (int jl = 0; jl < nb; ++jl) {
        const int jn = jl + 1 < GB ? jl + 1 : jl;
        float hn[GB / GL];
#pragma unroll
        for (int i = 0; i < GB / GL; ++i) hn[i] = HsT[jn * HP + i * GL + lane];
        const float en = Es[rr][jn], qn = Qs[rr][jn], cn = Cs[rr][jn], hjn = hds[jn];
        // correction: sum over earlier block columns of d_j' * H[j', j]
        // (branch-free; columns j' >= j add +0)
        float part = 0.0f;
#pragma unroll
        for (int i = 0; i < GB / GL; ++i) {
            const float pr = dl[i] * hv[i];
            part = part + (i * GL + lane < jl ? pr : 0.0f);
        }
        part = row_sum16(part);
        const float c = (cc0 + part) - e * hjj;
        float best = 1e30f, bq = qo;
#pragma unroll
        for (int m = 0; m < NG / GL; ++m) {
            const float g = qmin + (float)(m * GL + lane);
            const float ne = e + (g - qo) * s;
            const float cost = ne * ne * hjj + 2.0f * ne * c;
            const bool better = cost < best;
            best = better ? cost : best;
            bq = better ? g : bq;
        }
        argmin_step<DPP_ROR8>(best, bq);
        argmin_step<DPP_ROR4>(best, bq);
        argmin_step<DPP_QXOR2>(best, bq);
        argmin_step<DPP_QXOR1>(best, bq);
        bq = clampf(bq, qmin, qmax);
        const float d = (bq - qo) * s;
        if (lane == 0) {   // column jl is not read again in this block; Cs[.][jl] now keeps d
            Qs[rr][jl] = bq;
            Es[rr][jl] = e + d;
            Cs[rr][jl] = d;
        }
#pragma unroll
        for (int i = 0; i < GB / GL; ++i) dl[i] = i * GL + lane == jl ? d : dl[i];
#pragma unroll
        for (int i = 0; i < GB / GL; ++i) hv[i] = hn[i];
        e = en;
        qo = qn;
        cc0 = cn;
        hjj = hjn;
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < GSTAGE; ++k) {
        const int idx = t + 256 * k, rr2 = idx / GB, c2 = idx % GB;
        const int64_t r2 = r0 + rr2;
        if (r2 < rows && c2 < nb) {
            err[r2 * cols + j0 + c2] = Es[rr2][c2];
            Qf[r2 * cols + j0 + c2] = Qs[rr2][c2];
            D[r2 * GB + c2] = Cs[rr2][c2];
        }
    }
}

__global__ void to_int8_kernel(const float* Qf, int64_t n, float qmin, float qmax, int8_t* Q) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        Q[i] = (int8_t)(int)clampf(Qf[i], qmin, qmax);
}

static int egrid(int64_t n) { return (int)std::max<int64_t>(1, std::min<int64_t>(cdiv(n, 256), 65536)); }

// hd[j] = H[j][j]
__global__ void diag_kernel(const float* H, int64_t n, float* hd) {
    for (int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; j < n; j += (int64_t)gridDim.x * blockDim.x)
        hd[j] = H[j * n + j];
}

// US[i][c] = U[i][c] * s[c]   (n x k, U pitch ldu)
__global__ void scale_cols_kernel(const float* U, int64_t ldu, const float* s, int64_t n, int64_t k, float* US) {
    const int64_t total = n * k;
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (int64_t)gridDim.x * blockDim.x) {
        const int64_t i = idx / k, c = idx - i * k;
        US[idx] = U[i * ldu + c] * s[c];
    }
}

// part[b] = sum over the block's share of err * EH (fp64), EH = err @ H
__global__ void proxy_partial_kernel(const float* err, const float* EH, int64_t n, double* part) {
    __shared__ double red[4];
    double acc = 0.0;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        acc += (double)err[i] * (double)EH[i];
    acc = wave_sum(acc);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) part[blockIdx.x] = red[0] + red[1] + red[2] + red[3];
}

constexpr int PROXY_PARTS = 1024;

// Two-level pass.  Columns go in super-blocks of GSB: one GEMM gives the
// cross terms of a whole super-block, C = err @ Hc[sb, :]^T (K = cols, full
// tiles), and after each 64-column block its changes D update the rest of
// the super-block, C[:, rest] += D @ Hc[blk, rest] (K = 64).  Cross terms of
// later super-blocks come from the updated err.  Same sums as one GEMM per
// block over all of err, in another fp32 order.
constexpr int64_t GSB = 512;
// The cross-term GEMM of a super-block has few 128-tiles (rows / 128 x 4)
// and a long K (= cols): it runs as GSPLIT products over K / GSPLIT each
// (GSPLIT times the tiles, two per CU), summed in order by split_sum_kernel.
constexpr int GSPLIT = 4;

// C[r][c] = ((P_0 + P_1) + P_2) + P_3 for the GSPLIT partial products
// (pitch GSB, stride rows * GSB).
__global__ void split_sum_kernel(const float* __restrict__ P, int64_t rows, int64_t sw, float* __restrict__ C) {
    const int64_t total = rows * sw, stride = rows * GSB;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = i / sw, c = i - r * sw, o = r * GSB + c;
        float v = P[o];
#pragma unroll
        for (int k = 1; k < GSPLIT; ++k) v = v + P[k * stride + o];
        C[o] = v;
    }
}

// part: scratch for the split products (GSPLIT * rows * GSB floats), or null.
static int greedy_pass(float* err, float* Qf, const float* srow, const float* Hc, const float* hd, float* C,
                       float* D, float* part, int64_t rows, int64_t cols, float qmin, float qmax, hipStream_t st) {
    for (int64_t s0 = 0; s0 < cols; s0 += GSB) {
        const int64_t sw = std::min<int64_t>(GSB, cols - s0);
        const int64_t ks = cols / GSPLIT;
        const bool split = part && cols % (GSPLIT * 128) == 0 && cdiv(rows, 128) * cdiv(sw, 128) < 256 &&
                           ks >= 1024;
        int rc;
        if (split) {
            GemmArgs g{rows, sw, ks, 1.0f, 0.0f, err, cols, ks, Hc + s0 * cols, cols, ks, part, GSB, rows * GSB,
                       0, 1, CMASK_FULL, KR_FULL, GSPLIT, PT_GEMM_GREEDY};
            g.algo_flops = 2.0 * rows * sw * cols;
            if ((rc = gemm_f32(g, st))) return rc;
            hipLaunchKernelGGL(split_sum_kernel, dim3(egrid(rows * sw)), dim3(256), 0, st, part, rows, sw, C);
            IC_CHECK_LAUNCH();
        } else {
            GemmArgs g{rows, sw, cols, 1.0f, 0.0f, err, cols, 0, Hc + s0 * cols, cols, 0, C, GSB, 0, 0, 1,
                       CMASK_FULL, KR_FULL, 1, PT_GEMM_GREEDY};
            if ((rc = gemm_f32(g, st))) return rc;
        }
        for (int64_t j0 = s0; j0 < s0 + sw; j0 += GB) {
            const int nb = (int)std::min<int64_t>(GB, s0 + sw - j0);
            {
                ProfScope prof_scope(st, PT_GREEDY, (double)rows * nb * (nb + 4.0 * (qmax - qmin + 1)),
                                     (double)rows * nb * 20);
                if (qmax - qmin + 1.0f == 16.0f)
                    hipLaunchKernelGGL(greedy_block_kernel<16>, dim3((unsigned)cdiv(rows, GROWS)), dim3(256), 0, st,
                                       err, Qf, srow, Hc, cols, hd, C + (j0 - s0), GSB, D, rows, cols, j0, nb, qmin,
                                       qmax);
                else
                    hipLaunchKernelGGL(greedy_block_kernel<256>, dim3((unsigned)cdiv(rows, GROWS)), dim3(256), 0, st,
                                       err, Qf, srow, Hc, cols, hd, C + (j0 - s0), GSB, D, rows, cols, j0, nb, qmin,
                                       qmax);
                IC_CHECK_LAUNCH();
            }
            const int64_t rest = s0 + sw - (j0 + nb);
            if (rest > 0) {
                GemmArgs u{rows, rest, nb, 1.0f, 1.0f, D, GB, 0, Hc + j0 * cols + j0 + nb, cols, 0,
                           C + (j0 + nb - s0), GSB, 0, 0, 0, CMASK_FULL, KR_FULL, 1, PT_GEMM_GREEDY};
                if ((rc = gemm_f32(u, st))) return rc;
            }
        }
    }
    return IC_OK;
}

}  // namespace icq

using namespace icq;

extern "C" int ic_ldlq_init_scales(const float* row_absmax, int64_t rows, int64_t cols, int bits, float* srow,
                                   float* S, void* stream) {
    IC_REQUIRE(row_absmax && S, "ic_ldlq_init_scales: null pointer");
    if (rows * cols == 0) return IC_OK;
    hipLaunchKernelGGL(ldlq_init_scales_kernel, dim3(egrid(rows * cols)), dim3(256), 0, as_stream(stream),
                       row_absmax, rows, cols, bits == 8 ? 127.0f : 7.0f, srow, S);
    IC_CHECK_LAUNCH();
    return IC_OK;
}

extern "C" int ic_sanitize_scales(float* S, int64_t n, void* stream) {
    IC_REQUIRE(S, "ic_sanitize_scales: null pointer");
    if (n == 0) return IC_OK;
    hipLaunchKernelGGL(sanitize_scales_kernel, dim3(egrid(n)), dim3(256), 0, as_stream(stream), S, n);
    IC_CHECK_LAUNCH();
    return IC_OK;
}

extern "C" int ic_ldlq_mse(const float* W, const int8_t* Q, const float* S, int64_t n, double* out_sumsq,
                           void* workspace, void* stream) {
    IC_REQUIRE(W && Q && S && out_sumsq && workspace, "ic_ldlq_mse: null pointer");
    hipStream_t st = as_stream(stream);
    double* part = reinterpret_cast<double*>(workspace);
    hipLaunchKernelGGL(ldlq_mse_kernel, dim3(1024), dim3(256), 0, st, W, Q, S, n, part);
    IC_CHECK_LAUNCH();
    hipLaunchKernelGGL(sum_parts_kernel, dim3(1), dim3(256), 0, st, part, 1024, out_sumsq);
    IC_CHECK_LAUNCH();
    return IC_OK;
}

extern "C" int ic_ldlq_update_scales(const float* W, const int8_t* Q, const float* cur, const float* flat, int64_t n,
                                     float momentum, float lo, float hi, float* out, void* stream) {
    IC_REQUIRE(W && Q && cur && flat && out, "ic_ldlq_update_scales: null pointer");
    if (n == 0) return IC_OK;
    hipLaunchKernelGGL(ldlq_update_kernel, dim3(egrid(n)), dim3(256), 0, as_stream(stream), W, Q, cur, flat, n,
                       momentum, lo, hi, out);
    IC_CHECK_LAUNCH();
    return IC_OK;
}

extern "C" int ic_ls_scales(const int8_t* Q, const float* W, int64_t rows, int64_t cols, float* out, void* stream) {
    IC_REQUIRE(Q && W && out && rows < (1LL << 31), "ic_ls_scales: bad arguments");
    if (rows == 0) return IC_OK;
    hipLaunchKernelGGL(ls_scales_kernel, dim3((unsigned)cdiv(rows, 4)), dim3(256), 0, as_stream(stream), Q, W, rows,
                       cols, out);
    IC_CHECK_LAUNCH();
    return IC_OK;
}

extern "C" int64_t ic_greedy_workspace_bytes(int64_t rows, int64_t cols) {
    return (2 * rows * cols + rows * (GSB + GB) + GSPLIT * rows * GSB) * (int64_t)sizeof(float) + 256;
}

extern "C" int ic_greedy(const float* W, int8_t* Q, const float* srow, const float* H, int64_t rows, int64_t cols,
                         int passes, int bits, void* workspace, void* stream) {
    IC_REQUIRE(W && Q && srow && H && workspace, "ic_greedy: null pointer");
    IC_REQUIRE(bits == 4 || bits == 8, "ic_greedy: bits must be 4 or 8");
    if (rows == 0 || cols == 0 || passes <= 0) return IC_OK;
    hipStream_t st = as_stream(stream);
    const float qmin = bits == 4 ? -8.0f : -128.0f, qmax = bits == 4 ? 7.0f : 127.0f;
    float* err = reinterpret_cast<float*>(workspace);
    float* Qf = err + rows * cols;
    float* cross = Qf + rows * cols;
    hipLaunchKernelGGL(greedy_err_kernel, dim3(egrid(rows * cols)), dim3(256), 0, st, Q, srow, W, rows, cols, err, Qf);
    IC_CHECK_LAUNCH();
    float* part = cross + rows * (GSB + GB);
    for (int p = 0; p < passes; ++p) {
        int rc = greedy_pass(err, Qf, srow, H, nullptr, cross, cross + rows * GSB, part, rows, cols, qmin, qmax, st);
        if (rc) return rc;
    }
    hipLaunchKernelGGL(to_int8_kernel, dim3(egrid(rows * cols)), dim3(256), 0, st, Qf, rows * cols, qmin, qmax, Q);
    IC_CHECK_LAUNCH();
    return IC_OK;
}

extern "C" int64_t ic_greedy_lowrank_workspace_bytes(int64_t rows, int64_t cols, int64_t k) {
    return (3 * rows * cols + rows * (GSB + GB) + cols * cols + cols * std::max<int64_t>(k, 1) + cols +
            GSPLIT * rows * GSB) * (int64_t)sizeof(float) + PROXY_PARTS * (int64_t)sizeof(double) + 1024;
}

extern "C" int ic_greedy_lowrank(const float* W, int8_t* Q, const float* srow, const float* H, const float* U,
                                 int64_t ldu, const float* s, int64_t k, int64_t rows, int64_t cols, int passes,
                                 int bits, int* passes_run, void* workspace, void* stream) {
    IC_REQUIRE(W && Q && srow && H && workspace && (k == 0 || (U && s)), "ic_greedy_lowrank: null pointer");
    IC_REQUIRE(bits == 4 || bits == 8, "ic_greedy_lowrank: bits must be 4 or 8");
    IC_REQUIRE(k >= 0 && k <= cols && ldu >= k, "ic_greedy_lowrank: bad rank");
    if (passes_run) *passes_run = 0;
    if (rows == 0 || cols == 0 || passes <= 0) return IC_OK;
    hipStream_t st = as_stream(stream);
    const float qmin = bits == 4 ? -8.0f : -128.0f, qmax = bits == 4 ? 7.0f : 127.0f;
    float* err = reinterpret_cast<float*>(workspace);
    float* Qf = err + rows * cols;
    float* EH = Qf + rows * cols;
    float* cross = EH + rows * cols;
    float* D = cross + rows * GSB;
    float* Hk = D + rows * GB;
    float* US = Hk + cols * cols;
    float* hd = US + cols * std::max<int64_t>(k, 1);
    float* split_part = hd + cols;
    double* part = reinterpret_cast<double*>(
        (reinterpret_cast<uintptr_t>(split_part + GSPLIT * rows * GSB) + 255) & ~(uintptr_t)255);
    // Hk = U_k diag(s_k) U_k^T
    if (k == 0) {
        IC_CHECK_HIP(hipMemsetAsync(Hk, 0, cols * cols * sizeof(float), st));
    } else {
        hipLaunchKernelGGL(scale_cols_kernel, dim3(egrid(cols * k)), dim3(256), 0, st, U, ldu, s, cols, k, US);
        IC_CHECK_LAUNCH();
        GemmArgs g{cols, cols, k, 1.0f, 0.0f, US, k, 0, U, ldu, 0, Hk, cols, 0, 0, 1, CMASK_FULL, KR_FULL, 1,
                   PT_GEMM_GREEDY};
        int rc = gemm_f32(g, st);
        if (rc) return rc;
    }
    hipLaunchKernelGGL(diag_kernel, dim3(egrid(cols)), dim3(256), 0, st, H, cols, hd);
    IC_CHECK_LAUNCH();
    hipLaunchKernelGGL(greedy_err_kernel, dim3(egrid(rows * cols)), dim3(256), 0, st, Q, srow, W, rows, cols, err, Qf);
    IC_CHECK_LAUNCH();
    double prev = 0.0;
    int done = 0;
    for (int p = 0; p < passes; ++p) {
        int rc = greedy_pass(err, Qf, srow, Hk, hd, cross, D, split_part, rows, cols, qmin, qmax, st);
        if (rc) return rc;
        done = p + 1;
        if (p + 1 == passes) break;   // a stall test after the last pass changes nothing
        // proxy = sum((err @ H) * err) with the full Hessian
        GemmArgs g{rows, cols, cols, 1.0f, 0.0f, err, cols, 0, H, cols, 0, EH, cols, 0, 0, 0, CMASK_FULL, KR_FULL,
                   1, PT_GEMM_GREEDY};
        if ((rc = gemm_f32(g, st))) return rc;
        hipLaunchKernelGGL(proxy_partial_kernel, dim3(PROXY_PARTS), dim3(256), 0, st, err, EH, rows * cols, part);
        IC_CHECK_LAUNCH();
        double parts[PROXY_PARTS];
        IC_CHECK_HIP(hipMemcpyAsync(parts, part, sizeof(parts), hipMemcpyDeviceToHost, st));
        IC_CHECK_HIP(hipStreamSynchronize(st));
        double proxy = 0.0;
        for (int i = 0; i < PROXY_PARTS; ++i) proxy += parts[i];
        if (p > 0 && proxy >= prev * 0.99) break;   // STALL_THRESHOLD (converter/config.py:128)
        prev = proxy;
    }
    if (passes_run) *passes_run = done;
    hipLaunchKernelGGL(to_int8_kernel, dim3(egrid(rows * cols)), dim3(256), 0, st, Qf, rows * cols, qmin, qmax, Q);
    IC_CHECK_LAUNCH();
    return IC_OK;
}
