// Damped-Hessian inverse H^-1 = L^-T L^-1 (the reference's
// torch.linalg.cholesky + torch.cholesky_inverse, converter/rounding.py:19-34,
// after the damping of converter/gptq.py:91-121), for one matrix or a batch
// of equal-size diagonal blocks.
//
//  1. damp:   H += fp32(damping) * max(mean(diag H), 1e-6) * I   (per matrix)
//  2. potrf:  blocked right-looking Cholesky, nb = 128.  The nb x nb diagonal
//             block is factored in LDS by one workgroup, which also writes
//             its triangular inverse Dinv_k; the panel is A21 <- A21 Dinv_k^T
//             and the trailing update A22 -= A21 A21^T, both fp32-MFMA GEMMs.
//  3. trtri:  X = L^-1 by right-looking block substitution on L X = I:
//             X[k, :k] <- Dinv_k X[k, :k];  X[k, k] = Dinv_k;
//             X[k+1:, :k+1] -= L[k+1:, k] X[k, :k+1]           (GEMMs)
//  4. lauum:  H^-1 (upper triangle) = X^T X, one GEMM whose tile (I, J)
//             only runs k >= max(I, J) because X is lower triangular.
// Flops: n^3/3 each for 2-4; all but the nb x nb factorisations are MFMA.
#include "gemm.hpp"

namespace icq {

constexpr int NB = 128;

static double dtri(double n) { return n * (n + 1) / 2; }

__global__ void damp_kernel(float* H, int64_t n, int64_t ld, int64_t stride, float damping) {
    float* A = H + (int64_t)blockIdx.x * stride;
    double acc = 0.0;
    for (int64_t i = threadIdx.x; i < n; i += blockDim.x) acc += (double)A[i * ld + i];
    __shared__ double part[4];
    acc = wave_sum(acc);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = acc;
    __syncthreads();
    double tot = 0.0;
    for (int w = 0; w < (int)(blockDim.x >> 6); ++w) tot += part[w];
    float mean = (float)(tot / (double)n);
    mean = mean > 1e-6f ? mean : (mean != mean ? mean : 1e-6f);
    const float delta = damping * mean;
    for (int64_t i = threadIdx.x; i < n; i += blockDim.x) A[i * ld + i] = A[i * ld + i] + delta;
}

// Factor the diagonal block [k0, k0+nb) of matrix blockIdx.x in place (lower,
// upper part of the block set to 0) and write Dinv = L_kk^-1 (lower, upper 0)
// to dinv (pitch NB).  info[b] gets the 1-based column of the first
// non-positive pivot (LAPACK convention) if it is still 0.
//
// 256 threads as a 16 x 16 grid; thread (ty, tx) keeps the 8 x 8 tile at
// rows 8ty.., columns 8tx.. of both L and X = L^-1 in registers.  Column j of
// the Cholesky (and row k of the inverse) is published through LDS once per
// step, double-buffered so one barrier per step suffices.  Rank-1 updates are
// unconditional: factors of rows / columns that must not change are zero.
// A partial block (nb < 128) is padded with the identity.
// 8 consecutive LDS floats (32-byte aligned) as two 16-byte reads.
__device__ __forceinline__ void load8(const float* p, float* v) {
    const float4 a = reinterpret_cast<const float4*>(p)[0];
    const float4 b = reinterpret_cast<const float4*>(p)[1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

__global__ __launch_bounds__(256) void potrf_diag_kernel(float* H, int64_t ld, int64_t stride, int64_t k0, int nb,
                                                         float* dinv, int64_t dstride, int* info) {
    __shared__ __attribute__((aligned(16))) float colL[2][NB];
    __shared__ __attribute__((aligned(16))) float rowX[2][NB];
    const int b = blockIdx.x;
    float* A = H + (int64_t)b * stride + k0 * ld + k0;
    const int t = threadIdx.x;
    const int tx = t & 15, ty = t >> 4;
    const int r0 = ty * 8, c0 = tx * 8;
    float a[8][8];
#pragma unroll
    for (int p = 0; p < 8; ++p)
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const int r = r0 + p, c = c0 + q;
            float v = 0.0f;
            if (c <= r) v = (r < nb) ? A[(int64_t)r * ld + c] : (r == c ? 1.0f : 0.0f);
            a[p][q] = v;
        }
    int bad = 0;
    int buf = 0;
    // ---- Cholesky, right-looking, one column per step
    for (int jb = 0; jb < 16; ++jb) {
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) {
            const int j = jb * 8 + jj;
            if (tx == jb) {
#pragma unroll
                for (int p = 0; p < 8; ++p) colL[buf][r0 + p] = a[p][jj];
            }
            __syncthreads();
            float d = colL[buf][j];
            if (!(d > 0.0f)) {
                if (!bad) bad = j + 1;
                d = 1.0f;
            }
            const float ljj = sqrtf(d);
            const float rinv = 1.0f / ljj;
            float li[8], lc[8];
            load8(&colL[buf][r0], li);
            load8(&colL[buf][c0], lc);
#pragma unroll
            for (int p = 0; p < 8; ++p) li[p] = (r0 + p > j) ? li[p] * rinv : 0.0f;
#pragma unroll
            for (int q = 0; q < 8; ++q) lc[q] = (c0 + q > j) ? lc[q] * rinv : 0.0f;
#pragma unroll
            for (int p = 0; p < 8; ++p)
#pragma unroll
                for (int q = 0; q < 8; ++q) a[p][q] = a[p][q] - li[p] * lc[q];
            if (tx == jb) {
#pragma unroll
                for (int p = 0; p < 8; ++p) {
                    const int r = r0 + p;
                    if (r > j) a[p][jj] = li[p];
                    else if (r == j) a[p][jj] = ljj;
                }
            }
            buf ^= 1;
        }
    }
    // ---- X = L^-1, right-looking on L X = I: row k final = R[k,:] / L[k][k]
    float x[8][8];
#pragma unroll
    for (int p = 0; p < 8; ++p)
#pragma unroll
        for (int q = 0; q < 8; ++q) x[p][q] = (r0 + p == c0 + q) ? 1.0f : 0.0f;
    for (int kb = 0; kb < 16; ++kb) {
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) {
            const int k = kb * 8 + kk;
            if (tx == kb) {
#pragma unroll
                for (int p = 0; p < 8; ++p) colL[buf][r0 + p] = a[p][kk];
            }
            if (ty == kb) {
#pragma unroll
                for (int q = 0; q < 8; ++q) rowX[buf][c0 + q] = x[kk][q];
            }
            __syncthreads();
            const float rk = 1.0f / colL[buf][k];
            float li[8], xk[8];
            load8(&colL[buf][r0], li);
            load8(&rowX[buf][c0], xk);
#pragma unroll
            for (int p = 0; p < 8; ++p) li[p] = (r0 + p > k) ? li[p] : 0.0f;
#pragma unroll
            for (int q = 0; q < 8; ++q) xk[q] = xk[q] * rk;
#pragma unroll
            for (int p = 0; p < 8; ++p)
#pragma unroll
                for (int q = 0; q < 8; ++q) x[p][q] = x[p][q] - li[p] * xk[q];
            if (ty == kb) {
#pragma unroll
                for (int q = 0; q < 8; ++q) x[kk][q] = xk[q];
            }
            buf ^= 1;
        }
    }
    float* D = dinv + (int64_t)b * dstride;
#pragma unroll
    for (int p = 0; p < 8; ++p)
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const int r = r0 + p, c = c0 + q;
            const bool in = r < nb && c < nb;
            if (in) A[(int64_t)r * ld + c] = c <= r ? a[p][q] : 0.0f;
            D[r * NB + c] = (in && c <= r) ? x[p][q] : 0.0f;
        }
    if (t == 0 && bad && info[b] == 0) info[b] = (int)k0 + bad;
}

// Copy Dinv_k into the diagonal block of X (lower, upper zero).
__global__ void put_diag_kernel(float* X, int64_t ld, int64_t stride, int64_t k0, int nb, const float* dinv,
                                int64_t dstride) {
    const int b = blockIdx.y;
    const float* D = dinv + (int64_t)b * dstride;
    float* P = X + (int64_t)b * stride + k0 * ld + k0;
    for (int idx = blockIdx.x * blockDim.x + threadIdx.x; idx < nb * nb; idx += gridDim.x * blockDim.x) {
        int i = idx / nb, j = idx - i * nb;
        P[(int64_t)i * ld + j] = D[i * NB + j];
    }
}

__global__ void fill_kernel(float* p, int64_t n, float v) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        p[i] = v;
}

// Copy the upper triangle onto the lower one (in place), per matrix.
__global__ void mirror_upper_kernel(float* H, int64_t n, int64_t ld, int64_t stride) {
    float* A = H + (int64_t)blockIdx.z * stride;
    const int64_t i = (int64_t)blockIdx.y * 16 + threadIdx.y;
    const int64_t j = (int64_t)blockIdx.x * 16 + threadIdx.x;
    if (i < n && j < n && i > j) A[i * ld + j] = A[j * ld + i];
}

// Transpose the lower triangle into the upper one and zero the lower (in place):
// turns a lower Cholesky factor L into L^T.
__global__ void lower_to_upper_kernel(float* H, int64_t n, int64_t ld, int64_t stride) {
    float* A = H + (int64_t)blockIdx.z * stride;
    const int64_t i = (int64_t)blockIdx.y * 16 + threadIdx.y;
    const int64_t j = (int64_t)blockIdx.x * 16 + threadIdx.x;
    if (i < n && j < n && i < j) {
        A[i * ld + j] = A[j * ld + i];
        A[j * ld + i] = 0.0f;
    }
}

static int fill(float* p, int64_t n, float v, hipStream_t st) {
    if (n <= 0) return IC_OK;
    int grid = (int)std::min<int64_t>(cdiv(n, 256), 65536);
    hipLaunchKernelGGL(fill_kernel, dim3(grid), dim3(256), 0, st, p, n, v);
    IC_CHECK_LAUNCH();
    return IC_OK;
}

static int64_t dinv_floats(int64_t batch, int64_t n) { return batch * cdiv(n, NB) * NB * NB; }

// Lower Cholesky in place of `batch` matrices [n, n] (pitch ld, stride sH);
// dinv receives every Dinv_k (batch x nblk x NB x NB).
static int potrf(float* H, int64_t batch, int64_t n, int64_t ld, int64_t sH, float* dinv, int* info,
                 hipStream_t st) {
    const int64_t nblk = cdiv(n, NB);
    const int64_t dstride = nblk * NB * NB;
    for (int64_t kb = 0; kb < nblk; ++kb) {
        const int64_t k0 = kb * NB;
        const int nb = (int)std::min<int64_t>(NB, n - k0);
        float* Dk = dinv + kb * NB * NB;
        {
            ProfScope prof_scope(st, PT_DIAG, batch * (2.0 / 3.0) * nb * nb * nb, batch * 3.0 * 4 * nb * nb);
            hipLaunchKernelGGL(potrf_diag_kernel, dim3((unsigned)batch), dim3(256), 0, st, H, ld, sH, k0, nb, Dk,
                               dstride, info);
            IC_CHECK_LAUNCH();
        }
        const int64_t m = n - k0 - nb;
        if (m <= 0) break;
        float* A21 = H + (k0 + nb) * ld + k0;
        // panel: A21 <- A21 * Dinv^T (in place: one tile column spans all nb columns)
        GemmArgs p{m, nb, nb, 1.0f, 0.0f, A21, ld, sH, Dk, NB, dstride, A21, ld, sH, 0, 1, CMASK_FULL, KR_FULL, batch,
                   PT_GEMM_CHOL, (double)batch * m * nb * (nb + 1)};
        int rc = gemm_f32(p, st);
        if (rc) return rc;
        // trailing: A22 -= A21 A21^T (lower)
        float* A22 = H + (k0 + nb) * ld + (k0 + nb);
        GemmArgs s{m, m, nb, -1.0f, 1.0f, A21, ld, sH, A21, ld, sH, A22, ld, sH, 0, 1, CMASK_LOWER, KR_FULL, batch,
                   PT_GEMM_CHOL, (double)batch * 2.0 * dtri((double)m) * nb};
        rc = gemm_f32(s, st);
        if (rc) return rc;
    }
    return IC_OK;
}

// X = L^-1 (lower, upper zero) from L (lower, in H) and the Dinv blocks.
static int trtri(const float* L, float* X, int64_t batch, int64_t n, int64_t ld, int64_t sH, const float* dinv,
                 hipStream_t st) {
    const int64_t nblk = cdiv(n, NB);
    const int64_t dstride = nblk * NB * NB;
    int rc = fill(X, batch * sH, 0.0f, st);
    if (rc) return rc;
    for (int64_t kb = 0; kb < nblk; ++kb) {
        const int64_t k0 = kb * NB;
        const int nb = (int)std::min<int64_t>(NB, n - k0);
        const float* Dk = dinv + kb * NB * NB;
        float* Xk = X + k0 * ld;   // row block k
        if (k0 > 0) {
            // X[k, :k] <- Dinv_k X[k, :k]   (in place, M = nb <= 128)
            GemmArgs a{nb, k0, nb, 1.0f, 0.0f, Dk, NB, dstride, Xk, ld, sH, Xk, ld, sH, 0, 0, CMASK_FULL, KR_FULL,
                       batch, PT_GEMM_INV, (double)batch * k0 * nb * (nb + 1)};
            rc = gemm_f32(a, st);
            if (rc) return rc;
        }
        hipLaunchKernelGGL(put_diag_kernel, dim3(16, (unsigned)batch), dim3(256), 0, st, X, ld, sH, k0, nb, dinv + kb * NB * NB,
                           dstride);
        IC_CHECK_LAUNCH();
        const int64_t m = n - k0 - nb;
        if (m <= 0) break;
        // X[k+1:, :k+1] -= L[k+1:, k] X[k, :k+1]
        GemmArgs c{m, k0 + nb, nb, -1.0f, 1.0f, L + (k0 + nb) * ld + k0, ld, sH, Xk, ld, sH, X + (k0 + nb) * ld, ld,
                   sH, 0, 0, CMASK_FULL, KR_FULL, batch, PT_GEMM_INV,
                   (double)batch * m * (2.0 * k0 * nb + (double)nb * (nb + 1))};
        rc = gemm_f32(c, st);
        if (rc) return rc;
    }
    return IC_OK;
}

}  // namespace icq

using namespace icq;

extern "C" int64_t ic_hessian_inverse_workspace_bytes(int64_t batch, int64_t n) {
    return (batch * n * n + dinv_floats(batch, n)) * (int64_t)sizeof(float) + 256;
}

extern "C" int ic_hessian_inverse(float* H, int64_t batch, int64_t n, float damping, int method, int* info,
                                  void* workspace, void* stream) {
    IC_REQUIRE(H && info && workspace, "ic_hessian_inverse: null pointer");
    IC_REQUIRE(n >= 0 && batch >= 0, "ic_hessian_inverse: bad size");
    IC_REQUIRE(method == 0 || method == 1, "ic_hessian_inverse: method must be 0 (hinv) or 1 (cholesky)");
    if (n == 0 || batch == 0) return IC_OK;
    hipStream_t st = as_stream(stream);
    const int64_t ld = n, sH = n * n;
    float* X = reinterpret_cast<float*>(workspace);
    float* dinv = X + batch * sH;
    IC_CHECK_HIP(hipMemsetAsync(info, 0, batch * sizeof(int), st));
    hipLaunchKernelGGL(damp_kernel, dim3((unsigned)batch), dim3(256), 0, st, H, n, ld, sH, damping);
    IC_CHECK_LAUNCH();
    int rc = potrf(H, batch, n, ld, sH, dinv, info, st);
    if (rc) return rc;
    rc = trtri(H, X, batch, n, ld, sH, dinv, st);
    if (rc) return rc;
    // H^-1 (upper triangle incl. diagonal) = X^T X  -> H
    GemmArgs u{n, n, n, 1.0f, 0.0f, X, ld, sH, X, ld, sH, H, ld, sH, 1, 0, CMASK_UPPER, KR_FROM_MAXIJ, batch,
               PT_GEMM_INV, (double)batch * 2.0 * (double)n * (n + 1) * (n + 2) / 6.0};
    rc = gemm_f32(u, st);
    if (rc) return rc;
    dim3 tb(16, 16), tg((unsigned)cdiv(n, 16), (unsigned)cdiv(n, 16), (unsigned)batch);
    hipLaunchKernelGGL(mirror_upper_kernel, tg, tb, 0, st, H, n, ld, sH);
    IC_CHECK_LAUNCH();
    if (method == 1) {
        // upper Cholesky factor of H^-1 (converter/gptq.py:91-110): L2 = chol(H^-1), return L2^T
        rc = potrf(H, batch, n, ld, sH, dinv, info + batch, st);
        if (rc) return rc;
        hipLaunchKernelGGL(lower_to_upper_kernel, tg, tb, 0, st, H, n, ld, sH);
        IC_CHECK_LAUNCH();
    }
    return IC_OK;
}

extern "C" int ic_cholesky(float* H, int64_t batch, int64_t n, int* info, void* workspace, void* stream) {
    IC_REQUIRE(H && info && workspace, "ic_cholesky: null pointer");
    if (n == 0 || batch == 0) return IC_OK;
    hipStream_t st = as_stream(stream);
    IC_CHECK_HIP(hipMemsetAsync(info, 0, batch * sizeof(int), st));
    float* dinv = reinterpret_cast<float*>(workspace) + batch * n * n;
    return potrf(H, batch, n, n, n * n, dinv, info, st);
}
