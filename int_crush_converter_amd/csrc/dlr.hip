// Diagonal + low-rank Hessians H = diag(D) + U U^T (D [n], U [n, r]).
//
// Damped inverse by the Woodbury identity (converter/dlr.py:70-119):
//   shift = damping * max(mean(D + rowsum(U^2)), 1e-6)       (damping > 0)
//   Dinv  = 1 / max(D + shift, 1e-12),   Z = Dinv[:, None] * U          [n, r]
//   M     = I + U^T Z                                                   [r, r]
//   H^-1  = diag(Dinv) - (Z M^-1) Z^T                                   [n, n]
// M^-1 comes from the blocked Cholesky inverse of chol.hip; the three
// products run on the fp32 MFMA GEMM.  The n x n product is the only large
// one (2 n^2 r flops, 4 n^2 bytes written): everything else is O(n r).
//
// Dense form (converter/dlr.py:122-127): H = U U^T + diag(D).
#include <algorithm>

#include "chol.hpp"

namespace icq {
namespace {

constexpr int DLR_THREADS = 256;
constexpr int DLR_PARTS = 512;         // work-groups of the diagonal-mean reduction
constexpr int DLR_SPLIT_MAX = 64;      // K chunks of the r x r product U^T Z
constexpr int DLR_GEMM_TARGET = 1024;  // work-groups wanted for U^T Z
constexpr int64_t BAND = 128;          // largest Hinv block a sweep stages whole

constexpr float DIAG_MEAN_FLOOR = 1e-6f;   // converter/config.py
constexpr float DLR_DIAG_FLOOR = 1e-12f;   // converter/dlr.py:22

static int egrid(int64_t n) { return (int)std::max<int64_t>(1, std::min<int64_t>(cdiv(n, DLR_THREADS), 4096)); }
static size_t align256(size_t b) { return (b + 255) & ~size_t(255); }

// one wave per row: part[block] = sum over the block's rows of
// D[i] + sum_k U[i][k]^2 (row sums in fp32, the block total in fp64)
__global__ __launch_bounds__(DLR_THREADS) void diag_partial_kernel(const float* __restrict__ D,
                                                                   const float* __restrict__ U, int64_t n, int64_t r,
                                                                   int64_t ldu, double* __restrict__ part) {
    __shared__ double wsum[DLR_THREADS / 64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t waves = (int64_t)gridDim.x * (DLR_THREADS / 64);
    double acc = 0.0;
    for (int64_t i = (int64_t)blockIdx.x * (DLR_THREADS / 64) + wave; i < n; i += waves) {
        const float* u = U + i * ldu;
        float s = 0.0f;
        for (int64_t k = lane; k < r; k += 64) s += u[k] * u[k];
        for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off);
        if (lane == 0) acc += (double)(D[i] + s);
    }
    if (lane == 0) wsum[wave] = acc;
    __syncthreads();
    if (threadIdx.x == 0) {
        double t = 0.0;
        for (int w = 0; w < DLR_THREADS / 64; ++w) t += wsum[w];
        part[blockIdx.x] = t;
    }
}

// shift = fp32(damping) * max(fp32(mean), floor)
__global__ void diag_shift_kernel(const double* __restrict__ part, int parts, int64_t n, float damping,
                                  float* __restrict__ shift) {
    __shared__ double s[64];
    double acc = 0.0;
    for (int i = threadIdx.x; i < parts; i += 64) acc += part[i];
    s[threadIdx.x] = acc;
    __syncthreads();
    if (threadIdx.x == 0) {
        double t = 0.0;
        for (int i = 0; i < 64; ++i) t += s[i];
        const float mean = (float)(t / (double)n);
        *shift = damping * fmaxf(mean, DIAG_MEAN_FLOOR);
    }
}

// Dinv[i] = 1 / max(D[i] + shift, 1e-12); Z[i][k] = Dinv[i] * U[i][k] (pitch r)
__global__ __launch_bounds__(DLR_THREADS) void scale_rows_kernel(const float* __restrict__ D,
                                                                 const float* __restrict__ U, int64_t n, int64_t r,
                                                                 int64_t ldu, const float* __restrict__ shift,
                                                                 float* __restrict__ Dinv, float* __restrict__ Z) {
    const float sh = shift ? *shift : 0.0f;
    const int64_t total = n * r;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < (r ? total : n);
         e += (int64_t)gridDim.x * blockDim.x) {
        const int64_t i = r ? e / r : e, k = r ? e - i * r : 0;
        const float d = shift ? D[i] + sh : D[i];
        const float di = 1.0f / fmaxf(d, DLR_DIAG_FLOOR);
        if (k == 0) Dinv[i] = di;
        if (r) Z[e] = di * U[i * ldu + k];
    }
}

// M[i][j] = (i == j) + sum of the S partial products (fixed order)
__global__ void m_finish_kernel(const float* __restrict__ Gp, int S, int64_t r, float* __restrict__ M,
                                float* __restrict__ Mout) {
    const int64_t rr = r * r;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < rr; e += (int64_t)gridDim.x * blockDim.x) {
        float acc = Gp[e];
        for (int s = 1; s < S; ++s) acc = acc + Gp[s * rr + e];
        const int64_t i = e / r, j = e - i * r;
        const float m = (i == j ? 1.0f : 0.0f) + acc;
        M[e] = m;
        if (Mout) Mout[e] = m;
    }
}

// H[i][i] += v[i]; with `band`, H[i][j] = 0 for 0 < i - j < BAND (the lower
// part of the diagonal blocks a sweep stages, left unwritten by an upper GEMM)
__global__ void diag_add_kernel(float* __restrict__ H, int64_t n, int64_t ldh, const float* __restrict__ v, int band) {
    const int64_t total = band ? n * BAND : n;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += (int64_t)gridDim.x * blockDim.x) {
        const int64_t i = band ? e / BAND : e, d = band ? e - i * BAND : 0;
        if (d == 0) {
            H[i * ldh + i] += v[i];
        } else if (i - d >= 0) {
            H[i * ldh + (i - d)] = 0.0f;
        }
    }
}

// H = 0 (part `cmask`) for r == 0, where no GEMM writes the off-diagonal
__global__ void zero_kernel(float* __restrict__ H, int64_t n, int64_t ldh, int upper) {
    const int64_t total = n * n;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += (int64_t)gridDim.x * blockDim.x) {
        const int64_t i = e / n, j = e - i * n;
        if (!upper || j >= i) H[i * ldh + j] = 0.0f;
    }
}

struct DlrWork {
    double* part;
    float* shift;
    float* Dinv;
    float* Z;     // [n, r]
    float* Gp;    // [S, r, r]
    float* M;     // [r, r]
    float* Y;     // [n, r]
    void* inv_ws;
};

struct Split {
    int S;
    int64_t kc;
};

static Split split_of(int64_t n, int64_t r) {
    const int64_t tiles = std::max<int64_t>(1, cdiv(r, 64) * cdiv(r, 64));
    int64_t S = std::min<int64_t>(DLR_SPLIT_MAX, std::max<int64_t>(1, DLR_GEMM_TARGET / tiles));
    S = std::max<int64_t>(1, std::min<int64_t>(S, cdiv(n, 256)));
    const int64_t kc = std::max<int64_t>(32, cdiv(cdiv(n, S), 32) * 32);
    return {(int)std::max<int64_t>(1, cdiv(n, kc)), kc};
}

static size_t dlr_layout(int64_t n, int64_t r, char* base, DlrWork* w) {
    size_t off = 0;
    auto take = [&](size_t bytes) {
        char* p = base ? base + off : nullptr;
        off += align256(bytes);
        return p;
    };
    const Split sp = split_of(n, r);
    DlrWork t{};
    t.part = (double*)take(DLR_PARTS * sizeof(double));
    t.shift = (float*)take(sizeof(float));
    t.Dinv = (float*)take((size_t)n * 4);
    t.Z = (float*)take((size_t)n * r * 4);
    t.Gp = (float*)take((size_t)sp.S * r * r * 4);
    t.M = (float*)take((size_t)r * r * 4);
    t.Y = (float*)take((size_t)n * r * 4);
    t.inv_ws = take((size_t)ic_hessian_inverse_workspace_bytes(1, r));
    if (w) *w = t;
    return off + 256;
}

}  // namespace
}  // namespace icq

using namespace icq;

extern "C" int64_t ic_woodbury_workspace_bytes(int64_t n, int64_t r) {
    if (n < 0 || r < 0) return 0;
    return (int64_t)dlr_layout(n, r, nullptr, nullptr);
}

extern "C" int ic_woodbury_inverse(const float* D, const float* U, int64_t n, int64_t r, int64_t ldu, float damping,
                                   const float* Minv_in, int upper_only, float* Hinv, int64_t ldh, float* M_out,
                                   int* info, void* workspace, void* stream) {
    IC_REQUIRE(D && Hinv && info && workspace, "ic_woodbury_inverse: null pointer");
    IC_REQUIRE(n >= 0 && r >= 0, "ic_woodbury_inverse: bad size");
    IC_REQUIRE(r == 0 || (U && ldu >= r), "ic_woodbury_inverse: U missing or ldu < r");
    IC_REQUIRE(ldh >= n, "ic_woodbury_inverse: ldh < n");
    IC_REQUIRE(damping >= 0.0f, "ic_woodbury_inverse: damping must be >= 0");
    hipStream_t st = as_stream(stream);
    IC_CHECK_HIP(hipMemsetAsync(info, 0, 2 * sizeof(int), st));
    if (n == 0) return IC_OK;
    DlrWork w;
    dlr_layout(n, r, reinterpret_cast<char*>(workspace), &w);
    const bool damped = damping > 0.0f;
    if (damped) {
        const int parts = (int)std::min<int64_t>(DLR_PARTS, cdiv(n, DLR_THREADS / 64));
        hipLaunchKernelGGL(diag_partial_kernel, dim3(parts), dim3(DLR_THREADS), 0, st, D, U, n, r, ldu, w.part);
        IC_CHECK_LAUNCH();
        hipLaunchKernelGGL(diag_shift_kernel, dim3(1), dim3(64), 0, st, w.part, parts, n, damping, w.shift);
        IC_CHECK_LAUNCH();
    }
    hipLaunchKernelGGL(scale_rows_kernel, dim3(egrid(r ? n * r : n)), dim3(DLR_THREADS), 0, st, D, U, n, r, ldu,
                       damped ? w.shift : nullptr, w.Dinv, w.Z);
    IC_CHECK_LAUNCH();
    int rc;
    if (r == 0) {
        hipLaunchKernelGGL(zero_kernel, dim3(egrid(n * n)), dim3(DLR_THREADS), 0, st, Hinv, n, ldh, upper_only);
        IC_CHECK_LAUNCH();
    } else {
        const float* Minv = Minv_in;
        if (!Minv) {
            // M = I + U^T Z, K = n cut into S chunks (r x r alone is too few tiles)
            const Split sp = split_of(n, r);
            const int64_t rr = r * r;
            if (sp.S > 1) {
                GemmArgs g{r, r, sp.kc, 1.0f, 0.0f, U, ldu, sp.kc * ldu, w.Z, r, sp.kc * r, w.Gp, r, rr, 1, 0,
                           CMASK_FULL, KR_FULL, sp.S - 1, PT_DLR};
                if ((rc = gemm_f32(g, st))) return rc;
            }
            const int64_t k0 = (int64_t)(sp.S - 1) * sp.kc;
            GemmArgs g{r, r, n - k0, 1.0f, 0.0f, U + k0 * ldu, ldu, 0, w.Z + k0 * r, r, 0, w.Gp + (sp.S - 1) * rr,
                       r, 0, 1, 0, CMASK_FULL, KR_FULL, 1, PT_DLR};
            if ((rc = gemm_f32(g, st))) return rc;
            hipLaunchKernelGGL(m_finish_kernel, dim3(egrid(rr)), dim3(DLR_THREADS), 0, st, w.Gp, sp.S, r, w.M, M_out);
            IC_CHECK_LAUNCH();
            // M^-1 in place (Cholesky; info[0] != 0 when a pivot is not positive)
            if ((rc = ic_hessian_inverse(w.M, 1, r, 0.0f, 0, info, w.inv_ws, stream))) return rc;
            Minv = w.M;
        }
        // Y = Z M^-1, then Hinv = -Y Z^T (upper triangle only when asked)
        GemmArgs y{n, r, r, 1.0f, 0.0f, w.Z, r, 0, Minv, r, 0, w.Y, r, 0, 0, 0, CMASK_FULL, KR_FULL, 1, PT_DLR};
        if ((rc = gemm_f32(y, st))) return rc;
        GemmArgs h{n, n, r, -1.0f, 0.0f, w.Y, r, 0, w.Z, r, 0, Hinv, ldh, 0, 0, 1,
                   upper_only ? CMASK_UPPER : CMASK_FULL, KR_FULL, 1, PT_DLR_GEMM,
                   (upper_only ? 1.0 : 2.0) * (double)n * (double)n * (double)r};
        if ((rc = gemm_f32(h, st))) return rc;
    }
    const int band = upper_only ? 1 : 0;
    hipLaunchKernelGGL(diag_add_kernel, dim3(egrid(band ? n * BAND : n)), dim3(DLR_THREADS), 0, st, Hinv, n, ldh,
                       w.Dinv, band);
    IC_CHECK_LAUNCH();
    return IC_OK;
}

extern "C" int ic_dlr_to_dense(const float* D, const float* U, int64_t n, int64_t r, int64_t ldu, float* H,
                               int64_t ldh, void* stream) {
    IC_REQUIRE(D && H, "ic_dlr_to_dense: null pointer");
    IC_REQUIRE(n >= 0 && r >= 0, "ic_dlr_to_dense: bad size");
    IC_REQUIRE(r == 0 || (U && ldu >= r), "ic_dlr_to_dense: U missing or ldu < r");
    IC_REQUIRE(ldh >= n, "ic_dlr_to_dense: ldh < n");
    if (n == 0) return IC_OK;
    hipStream_t st = as_stream(stream);
    if (r == 0) {
        hipLaunchKernelGGL(zero_kernel, dim3(egrid(n * n)), dim3(DLR_THREADS), 0, st, H, n, ldh, 0);
        IC_CHECK_LAUNCH();
    } else {
        GemmArgs g{n, n, r, 1.0f, 0.0f, U, ldu, 0, U, ldu, 0, H, ldh, 0, 0, 1, CMASK_FULL, KR_FULL, 1, PT_DLR_GEMM};
        int rc = gemm_f32(g, st);
        if (rc) return rc;
    }
    hipLaunchKernelGGL(diag_add_kernel, dim3(egrid(n)), dim3(DLR_THREADS), 0, st, H, n, ldh, D, 0);
    IC_CHECK_LAUNCH();
    return IC_OK;
}
