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

namespace icq {

constexpr int GB = 64;          // greedy column block
constexpr int GL = 4;           // lanes per row in the greedy block kernel

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
// (ldlq.py:227-231, 262-265), fp64 accumulation rounded once to fp32.
__global__ __launch_bounds__(256) void ls_scales_kernel(const int8_t* Q, const float* W, int64_t rows, int64_t cols,
                                                        float* out) {
    const int64_t r = blockIdx.x;
    if (r >= rows) return;
    double num = 0.0, den = 0.0;
    for (int64_t c = threadIdx.x; c < cols; c += blockDim.x) {
        const float q = (float)Q[r * cols + c];
        num += (double)(q * W[r * cols + c]);
        den += (double)(q * q);
    }
    __shared__ double sn[4], sd[4];
    num = wave_sum(num);
    den = wave_sum(den);
    if ((threadIdx.x & 63) == 0) { sn[threadIdx.x >> 6] = num; sd[threadIdx.x >> 6] = den; }
    __syncthreads();
    if (threadIdx.x == 0) {
        float n32 = (float)(sn[0] + sn[1] + sn[2] + sn[3]);
        float d32 = (float)(sd[0] + sd[1] + sd[2] + sd[3]);
        d32 = d32 < 1e-8f ? 1e-8f : d32;
        out[r] = nclampmin(n32 / d32, 1e-5f);
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

// One 64-column block of a greedy pass.  GL lanes per row: lane l keeps the
// changes d_j' of the columns j' = l (mod GL) and their share of the
// correction sum; the candidate scan runs redundantly on all GL lanes.
// H is the matrix of the cross terms (the Hessian, or its low-rank
// truncation) and hd its exact diagonal H_jj (null: the diagonal of H).
__global__ __launch_bounds__(256) void greedy_block_kernel(float* err, float* Qf, const float* srow, const float* H,
                                                           int64_t ldh, const float* hd, const float* cross,
                                                           int64_t rows, int64_t cols, int64_t j0, int nb,
                                                           float qmin, float qmax) {
    __shared__ float Hs[GB * GB];
    const int t = threadIdx.x;
    for (int idx = t; idx < nb * nb; idx += blockDim.x) {
        int a = idx / nb, b = idx - a * nb;
        Hs[a * GB + b] = H[(j0 + a) * ldh + j0 + b];
    }
    __syncthreads();
    const int lane = t % GL;
    const int64_t r = (int64_t)blockIdx.x * (blockDim.x / GL) + t / GL;
    const bool rv = r < rows;
    const float s = rv ? srow[r] : 1.0f;
    float dl[GB / GL];
#pragma unroll
    for (int i = 0; i < GB / GL; ++i) dl[i] = 0.0f;
    for (int jl = 0; jl < nb; ++jl) {
        const int64_t j = j0 + jl;
        // correction: sum over earlier block columns of d_j' * H[j', j]
        float part = 0.0f;
#pragma unroll
        for (int i = 0; i < GB / GL; ++i) {
            const int jp = i * GL + lane;
            if (jp < jl) part = part + dl[i] * Hs[jp * GB + jl];
        }
        part = part + __shfl_xor(part, 1, GL);
        part = part + __shfl_xor(part, 2, GL);
        const float hjj = hd ? hd[j0 + jl] : Hs[jl * GB + jl];
        float e = 0.0f, qo = 0.0f, c = 0.0f;
        if (rv) {
            e = err[r * cols + j];
            qo = Qf[r * cols + j];
            c = (cross[r * GB + jl] + part) - e * hjj;
        }
        float best = 1e30f, bq = qo;
        for (float g = qmin; g <= qmax; g += 1.0f) {
            const float ne = e + (g - qo) * s;
            const float cost = ne * ne * hjj + 2.0f * ne * c;
            if (cost < best) { best = cost; bq = g; }
        }
        bq = clampf(bq, qmin, qmax);
        const float d = (bq - qo) * s;
        if (rv && lane == 0) {
            Qf[r * cols + j] = bq;
            err[r * cols + j] = e + d;
        }
#pragma unroll
        for (int i = 0; i < GB / GL; ++i)
            if (i * GL + lane == jl) dl[i] = d;
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

// One greedy pass over all column blocks: cross terms from Hc (the full
// Hessian or its truncation), exact diagonal hd (null: Hc's).
static int greedy_pass(float* err, float* Qf, const float* srow, const float* Hc, const float* hd, float* cross,
                       int64_t rows, int64_t cols, float qmin, float qmax, hipStream_t st) {
    for (int64_t j0 = 0; j0 < cols; j0 += GB) {
        const int nb = (int)std::min<int64_t>(GB, cols - j0);
        // cross[:, 0:nb] = err @ Hc[j0:j0+nb, :]^T
        GemmArgs g{rows, nb, cols, 1.0f, 0.0f, err, cols, 0, Hc + j0 * cols, cols, 0, cross, GB, 0, 0, 1,
                   CMASK_FULL, KR_FULL, 1, PT_GEMM_GREEDY};
        int rc = gemm_f32(g, st);
        if (rc) return rc;
        const int rpb = 256 / GL;
        ProfScope prof_scope(st, PT_GREEDY, (double)rows * nb * (nb + 4.0 * (qmax - qmin + 1)), (double)rows * nb * 16);
        hipLaunchKernelGGL(greedy_block_kernel, dim3((unsigned)cdiv(rows, rpb)), dim3(256), 0, st, err, Qf, srow,
                           Hc, cols, hd, cross, rows, cols, j0, nb, qmin, qmax);
        IC_CHECK_LAUNCH();
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
    hipLaunchKernelGGL(ls_scales_kernel, dim3((unsigned)rows), dim3(256), 0, as_stream(stream), Q, W, rows, cols, out);
    IC_CHECK_LAUNCH();
    return IC_OK;
}

extern "C" int64_t ic_greedy_workspace_bytes(int64_t rows, int64_t cols) {
    return (2 * rows * cols + rows * GB) * (int64_t)sizeof(float) + 256;
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
    for (int p = 0; p < passes; ++p) {
        int rc = greedy_pass(err, Qf, srow, H, nullptr, cross, rows, cols, qmin, qmax, st);
        if (rc) return rc;
    }
    hipLaunchKernelGGL(to_int8_kernel, dim3(egrid(rows * cols)), dim3(256), 0, st, Qf, rows * cols, qmin, qmax, Q);
    IC_CHECK_LAUNCH();
    return IC_OK;
}

extern "C" int64_t ic_greedy_lowrank_workspace_bytes(int64_t rows, int64_t cols, int64_t k) {
    return (3 * rows * cols + rows * GB + cols * cols + cols * std::max<int64_t>(k, 1) + cols) *
               (int64_t)sizeof(float) + PROXY_PARTS * (int64_t)sizeof(double) + 1024;
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
    float* Hk = cross + rows * GB;
    float* US = Hk + cols * cols;
    float* hd = US + cols * std::max<int64_t>(k, 1);
    double* part = reinterpret_cast<double*>((reinterpret_cast<uintptr_t>(hd + cols) + 255) & ~(uintptr_t)255);
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
        int rc = greedy_pass(err, Qf, srow, Hk, hd, cross, rows, cols, qmin, qmax, st);
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
