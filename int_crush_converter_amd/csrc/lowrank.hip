// Low-rank eigendecomposition of a symmetric PSD Hessian for the greedy
// search (converter/greedy.py:293-366, _lowrank_decompose).
//
// The reference calls torch.svd_lowrank(H, q = N/2) (falling back to eigh)
// and keeps the eigenpairs above rank_threshold x the largest.  Only the top
// p = min(N, k_cap + oversampling) pairs can ever be used (the greedy
// refuses k > min(512, 0.3 N)), so this builds them by subspace iteration:
//
//   lam ~ lambda_max(H)                   16 power steps on a seeded vector
//   Q0 = orth(G)                          G: seeded Gaussian [n, p]
//   Q_{i+1} = orth((H + mu I) Q_i)        i < iters, mu = 1e-3 lam
//   T = Q^T H Q  (p x p)   ->   T = V diag(d) V^T  (cyclic Jacobi, fp64)
//   eigenvalues d (descending), eigenvectors Q V
//
// The shift mu keeps (H + mu I) Q of full rank when H is singular (a
// calibration Hessian from few samples) and bounds its condition number by
// ~1e3 without changing the eigenvectors; it slows the separation of an
// eigenvalue above the cut (>= 1e-2 lam) from one below by < 10 %.
// orth() is shifted CholeskyQR3: three passes of Y <- Y chol(Y^T Y + s I)^-T,
// the first with s = 1e-5 tr(Y^T Y), which divides the condition number by
// ~1/sqrt(s) so that the two plain passes see <= ~1e2 and fp32 Gram
// matrices keep them accurate.  Every piece is an fp32-MFMA GEMM or the
// blocked Cholesky / triangular inverse of chol.hip.
//
// The p x p eigenproblem is two-sided cyclic Jacobi in fp64 with the
// round-robin ordering: one launch applies the p/2 disjoint rotations of a
// round to A (Givens from both sides, 2 x 2 blocks, upper half mirrored so
// A stays exactly symmetric) and to V.  Sweeps run until the off-diagonal
// norm is below 1e-12 of the diagonal's, or 40 sweeps.
#include <algorithm>

#include "chol.hpp"

namespace icq {

// ------------------------------------------------------------ helpers

__device__ __forceinline__ uint64_t mix64(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

// Standard normal samples from a counter-based hash (Box-Muller).
__global__ void randn_kernel(float* Y, int64_t n, uint64_t seed) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        const uint64_t h = mix64(seed ^ mix64((uint64_t)i));
        const double u1 = ((double)(h >> 11) + 0.5) * 0x1p-53;
        const double u2 = (double)(mix64(h) >> 11) * 0x1p-53;
        Y[i] = (float)(sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2));
    }
}

// y = H x, one wave per row (fp32 products, fp64 sum)
__global__ void matvec_kernel(const float* H, int64_t n, const float* x, float* y) {
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= n) return;
    const int lane = threadIdx.x & 63;
    double acc = 0.0;
    for (int64_t j = lane; j < n; j += 64) acc += (double)(H[row * n + j] * x[j]);
    acc = wave_sum(acc);
    if (lane == 0) y[row] = (float)acc;
}

// x = y / ||y||, out[0] = rel * ||y||  (one work-group; ||y|| = 0 leaves x)
__global__ void normalize_kernel(const float* y, float* x, int64_t n, double rel, double* out) {
    __shared__ double red[4];
    double acc = 0.0;
    for (int64_t i = threadIdx.x; i < n; i += blockDim.x) acc += (double)y[i] * (double)y[i];
    acc = wave_sum(acc);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
    __syncthreads();
    const double nrm = sqrt(red[0] + red[1] + red[2] + red[3]);
    if (nrm > 0.0)
        for (int64_t i = threadIdx.x; i < n; i += blockDim.x) x[i] = (float)((double)y[i] / nrm);
    if (threadIdx.x == 0) out[0] = rel * nrm;
}

// part[b] = sum of squares over the block's grid-stride share (fp64)
__global__ void sumsq_kernel(const float* x, int64_t n, double* part) {
    __shared__ double red[4];
    double acc = 0.0;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        const double v = x[i];
        acc += v * v;
    }
    acc = wave_sum(acc);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) part[blockIdx.x] = red[0] + red[1] + red[2] + red[3];
}

// T[i][i] -= rel * sqrt(sum part[0..n))  (one work-group; fixed order)
__global__ void sub_frob_diag_kernel(float* T, int64_t p, const double* part, int n, double rel) {
    __shared__ double shift;
    if (threadIdx.x == 0) {
        double acc = 0.0;
        for (int i = 0; i < n; ++i) acc += part[i];
        shift = rel * sqrt(acc);
    }
    __syncthreads();
    for (int64_t i = threadIdx.x; i < p; i += blockDim.x) T[i * p + i] = (float)((double)T[i * p + i] - shift);
}

// Y += mu * Q  (mu read from device memory)
__global__ void axpy_dev_kernel(float* Y, const float* Q, int64_t n, const double* mu) {
    const float m = (float)mu[0];
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        Y[i] = Y[i] + m * Q[i];
}

// G[i][i] += rel * trace(G)  (one work-group)
__global__ void shift_diag_kernel(float* G, int64_t p, float rel) {
    __shared__ float red[4];
    float acc = 0.0f;
    for (int64_t i = threadIdx.x; i < p; i += blockDim.x) acc += G[i * p + i];
    acc = wave_sum(acc);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
    __syncthreads();
    const float s = rel * (red[0] + red[1] + red[2] + red[3]);
    for (int64_t i = threadIdx.x; i < p; i += blockDim.x) G[i * p + i] = G[i * p + i] + s;
}

// Zero the strict upper triangle of a p x p matrix.
__global__ void zero_upper_kernel(float* X, int64_t p) {
    const int64_t n = p * p;
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < n;
         idx += (int64_t)gridDim.x * blockDim.x) {
        const int64_t i = idx / p, j = idx - i * p;
        if (j > i) X[idx] = 0.0f;
    }
}

// A = fp64((T + T^T) / 2), V = I
__global__ void jacobi_init_kernel(const float* T, int64_t p, double* A, double* V) {
    const int64_t n = p * p;
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < n;
         idx += (int64_t)gridDim.x * blockDim.x) {
        const int64_t i = idx / p, j = idx - i * p;
        A[idx] = 0.5 * ((double)T[i * p + j] + (double)T[j * p + i]);
        V[idx] = i == j ? 1.0 : 0.0;
    }
}

// Pair P of round r (round-robin over p indices, p even): index p-1 meets r,
// the others meet by reflection about r.  Returned ordered (a < b).
__device__ __forceinline__ void jpair(int P, int r, int p, int& a, int& b) {
    const int m = p - 1;
    if (P == 0) {
        a = r;
        b = m;
    } else {
        a = (r + P) % m;
        b = (r - P + m) % m;
    }
    if (a > b) {
        const int t = a;
        a = b;
        b = t;
    }
}

// Rotation annihilating A[a][b] (Golub & Van Loan, symmetric Schur 2x2):
// J = [[c, s], [-s, c]] on (a, b), A' = J^T A J; t = tan.
__device__ __forceinline__ void jrot(const double* A, int p, int a, int b, double& c, double& s, double& t) {
    const double apq = A[(int64_t)a * p + b];
    if (apq == 0.0) {
        c = 1.0;
        s = 0.0;
        t = 0.0;
        return;
    }
    const double th = (A[(int64_t)b * p + b] - A[(int64_t)a * p + a]) / (2.0 * apq);
    const double at = fabs(th);
    t = at > 1e150 ? 0.5 / th : (th >= 0.0 ? 1.0 : -1.0) / (at + sqrt(th * th + 1.0));
    c = 1.0 / sqrt(t * t + 1.0);
    s = t * c;
}

// One round: Aout = J^T Ain J, Vout = Vin J.  Threads [0, np^2) handle the
// 2x2 blocks (pair P rows, pair C columns) with P <= C and write the mirror;
// threads [np^2, np^2 + p np) handle a row of V and a pair of its columns.
__global__ void jacobi_round_kernel(const double* Ain, double* Aout, const double* Vin, double* Vout, int p, int r) {
    const int np = p / 2;
    const int64_t nA = (int64_t)np * np;
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx < nA) {
        const int P = (int)(idx / np), C = (int)(idx - (int64_t)P * np);
        if (P > C) return;
        int a, b;
        jpair(P, r, p, a, b);
        double cp, sp, tp;
        jrot(Ain, p, a, b, cp, sp, tp);
        if (P == C) {
            const double apq = Ain[(int64_t)a * p + b];
            Aout[(int64_t)a * p + a] = Ain[(int64_t)a * p + a] - tp * apq;
            Aout[(int64_t)b * p + b] = Ain[(int64_t)b * p + b] + tp * apq;
            Aout[(int64_t)a * p + b] = 0.0;
            Aout[(int64_t)b * p + a] = 0.0;
            return;
        }
        int c2, d;
        jpair(C, r, p, c2, d);
        double cc, sc, tc;
        jrot(Ain, p, c2, d, cc, sc, tc);
        const double x00 = Ain[(int64_t)a * p + c2], x01 = Ain[(int64_t)a * p + d];
        const double x10 = Ain[(int64_t)b * p + c2], x11 = Ain[(int64_t)b * p + d];
        const double y00 = cp * x00 - sp * x10, y01 = cp * x01 - sp * x11;
        const double y10 = sp * x00 + cp * x10, y11 = sp * x01 + cp * x11;
        const double z00 = cc * y00 - sc * y01, z01 = sc * y00 + cc * y01;
        const double z10 = cc * y10 - sc * y11, z11 = sc * y10 + cc * y11;
        Aout[(int64_t)a * p + c2] = z00;
        Aout[(int64_t)a * p + d] = z01;
        Aout[(int64_t)b * p + c2] = z10;
        Aout[(int64_t)b * p + d] = z11;
        Aout[(int64_t)c2 * p + a] = z00;
        Aout[(int64_t)d * p + a] = z01;
        Aout[(int64_t)c2 * p + b] = z10;
        Aout[(int64_t)d * p + b] = z11;
        return;
    }
    const int64_t v = idx - nA;
    if (v >= (int64_t)p * np) return;
    const int row = (int)(v / np), C = (int)(v - (int64_t)row * np);
    int a, b;
    jpair(C, r, p, a, b);
    double c, s, t;
    jrot(Ain, p, a, b, c, s, t);
    const double va = Vin[(int64_t)row * p + a], vb = Vin[(int64_t)row * p + b];
    Vout[(int64_t)row * p + a] = c * va - s * vb;
    Vout[(int64_t)row * p + b] = s * va + c * vb;
}

// part[2 b] = off-diagonal sum of squares, part[2 b + 1] = diagonal's.
__global__ void offdiag_kernel(const double* A, int64_t p, double* part) {
    __shared__ double red[2][4];
    double off = 0.0, dia = 0.0;
    const int64_t n = p * p;
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < n;
         idx += (int64_t)gridDim.x * blockDim.x) {
        const int64_t i = idx / p, j = idx - i * p;
        const double v = A[idx];
        if (i == j) dia += v * v;
        else off += v * v;
    }
    off = wave_sum(off);
    dia = wave_sum(dia);
    if ((threadIdx.x & 63) == 0) {
        red[0][threadIdx.x >> 6] = off;
        red[1][threadIdx.x >> 6] = dia;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        part[2 * blockIdx.x] = red[0][0] + red[0][1] + red[0][2] + red[0][3];
        part[2 * blockIdx.x + 1] = red[1][0] + red[1][1] + red[1][2] + red[1][3];
    }
}

__global__ void finish_pairs_kernel(const double* part, int n, double* out) {
    if (threadIdx.x == 0 && blockIdx.x == 0) {
        double a = 0.0, b = 0.0;
        for (int i = 0; i < n; ++i) {
            a += part[2 * i];
            b += part[2 * i + 1];
        }
        out[0] = a;
        out[1] = b;
    }
}

// Descending order of the diagonal (ties: lower index first): eigenvalue j
// goes to position rank(j); column j of V goes to column rank(j) of Vs.
__global__ void ritz_sort_kernel(const double* A, const double* V, int64_t p, float* evals, float* Vs) {
    for (int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; j < p; j += (int64_t)gridDim.x * blockDim.x) {
        const double dj = A[j * p + j];
        int64_t rank = 0;
        for (int64_t i = 0; i < p; ++i) {
            const double di = A[i * p + i];
            rank += (di > dj || (di == dj && i < j)) ? 1 : 0;
        }
        evals[rank] = (float)dj;
        for (int64_t i = 0; i < p; ++i) Vs[i * p + rank] = (float)V[i * p + j];
    }
}

static int egrid_lr(int64_t n) { return (int)std::max<int64_t>(1, std::min<int64_t>(cdiv(n, 256), 4096)); }

static size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

// Workspace carve-up (every piece 256-byte aligned).
struct LrWork {
    float *Y, *Q, *G, *X, *dinv, *T, *Vs, *x, *y, *Gp;
    double *dinv64, *A0, *A1, *V0, *V1, *part, *scal;
    int* info;
};

constexpr int LR_PARTS = 1024;   // partial sums of the reductions
constexpr int GRAM_SPLIT = 8;    // K chunks of the p x p Gram matrices (K = n)

static size_t lr_layout(int64_t n, int64_t p, char* base, LrWork* w) {
    size_t off = 0;
    auto take = [&](size_t bytes) {
        char* ptr = base ? base + off : nullptr;
        off += align256(bytes);
        return ptr;
    };
    const size_t np4 = (size_t)n * p * 4, pp4 = (size_t)p * p * 4, pp8 = (size_t)p * p * 8;
    LrWork t{};
    t.Y = (float*)take(np4);
    t.Q = (float*)take(np4);
    t.G = (float*)take(pp4);
    t.X = (float*)take(pp4);
    t.T = (float*)take(pp4);
    t.Vs = (float*)take(pp4);
    t.x = (float*)take((size_t)n * 4);
    t.Gp = (float*)take((size_t)GRAM_SPLIT * pp4);
    t.y = (float*)take((size_t)n * 4);
    t.dinv = (float*)take((size_t)dinv_floats(1, p) * 4 + (size_t)dinv_floats(1, p) * 8 + 512);
    t.A0 = (double*)take(pp8);
    t.A1 = (double*)take(pp8);
    t.V0 = (double*)take(pp8);
    t.V1 = (double*)take(pp8);
    t.part = (double*)take((size_t)LR_PARTS * 2 * 8);
    t.scal = (double*)take(8 * 8);
    t.info = (int*)take(64);
    if (base) {
        t.dinv64 = dinv64_of(t.dinv, 1, p);
        *w = t;
    }
    return off + 256;
}

// G[i][j] = sum over the S partials (fixed order), lower triangle
__global__ void sum_partials_kernel(const float* Gp, int S, int64_t pp, float* G) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < pp; i += (int64_t)gridDim.x * blockDim.x) {
        float acc = Gp[i];
        for (int s = 1; s < S; ++s) acc = acc + Gp[s * pp + i];
        G[i] = acc;
    }
}

// G = A^T B (p x p, part `cmask`; A, B [n, p]) with K = n cut into up to
// GRAM_SPLIT chunks of a batched GEMM: the p x p output alone has too few
// tiles to fill the chip.
static int gram(const float* A, const float* B, int64_t n, int64_t p, float* G, const LrWork& w, int cmask,
                hipStream_t st) {
    const int64_t kc = cdiv(cdiv(n, GRAM_SPLIT), 32) * 32;
    const int S = (int)cdiv(n, kc);
    const int64_t pp = p * p;
    int rc;
    if (S > 1) {
        GemmArgs g{p, p, kc, 1.0f, 0.0f, A, p, kc * p, B, p, kc * p, w.Gp, p, pp, 1, 0, cmask, KR_FULL, S - 1,
                   PT_OTHER};
        if ((rc = gemm_f32(g, st))) return rc;
    }
    const int64_t k0 = (S - 1) * kc;
    GemmArgs g{p, p, n - k0, 1.0f, 0.0f, A + k0 * p, p, 0, B + k0 * p, p, 0, w.Gp + (S - 1) * pp, p, 0, 1, 0, cmask,
               KR_FULL, 1, PT_OTHER};
    if ((rc = gemm_f32(g, st))) return rc;
    hipLaunchKernelGGL(sum_partials_kernel, dim3(egrid_lr(pp)), dim3(256), 0, st, w.Gp, S, pp, G);
    IC_CHECK_LAUNCH();
    return IC_OK;
}

// One CholeskyQR pass: Q = Y R^-1 with R^T R = Y^T Y + shift_rel tr(Y^T Y) I.
static int cholqr_pass(const float* Y, float* Q, int64_t n, int64_t p, float shift_rel, const LrWork& w,
                       hipStream_t st) {
    int rc = gram(Y, Y, n, p, w.G, w, CMASK_LOWER, st);
    if (rc) return rc;
    if (shift_rel > 0.0f) {
        hipLaunchKernelGGL(shift_diag_kernel, dim3(1), dim3(256), 0, st, w.G, p, shift_rel);
        IC_CHECK_LAUNCH();
    }
    if ((rc = potrf(w.G, 1, p, p, p * p, w.dinv64, w.info, st))) return rc;
    if ((rc = trtri(w.G, w.X, 1, p, p, p * p, w.dinv64, st))) return rc;
    hipLaunchKernelGGL(zero_upper_kernel, dim3(egrid_lr(p * p)), dim3(256), 0, st, w.X, p);
    IC_CHECK_LAUNCH();
    // Q = Y X^T  (X = L^-1 lower, so op(B) = X^T is upper triangular)
    GemmArgs q{n, p, p, 1.0f, 0.0f, Y, p, 0, w.X, p, 0, Q, p, 0, 0, 1, CMASK_FULL, KR_FULL, 1, PT_OTHER};
    return gemm_f32(q, st);
}

// Shifted CholeskyQR3 of Y (overwritten) into Q; `well_conditioned` (a
// Gaussian start, cond ~ (1 + sqrt(p/n)) / (1 - sqrt(p/n))) skips the
// shifted pass: plain CholeskyQR2.
static int orth(float* Y, float* Q, int64_t n, int64_t p, const LrWork& w, hipStream_t st,
                bool well_conditioned = false) {
    int rc;
    if (well_conditioned) {
        rc = cholqr_pass(Y, Q, n, p, 0.0f, w, st);
        if (!rc) rc = cholqr_pass(Q, Y, n, p, 0.0f, w, st);
        if (!rc) IC_CHECK_HIP(hipMemcpyAsync(Q, Y, (size_t)n * p * sizeof(float), hipMemcpyDeviceToDevice, st));
        return rc;
    }
    rc = cholqr_pass(Y, Q, n, p, 1e-5f, w, st);
    if (!rc) rc = cholqr_pass(Q, Y, n, p, 0.0f, w, st);
    if (!rc) rc = cholqr_pass(Y, Q, n, p, 0.0f, w, st);
    return rc;
}

constexpr int JACOBI_MAX_SWEEPS = 40;

}  // namespace icq

using namespace icq;

extern "C" int64_t ic_lowrank_workspace_bytes(int64_t n, int64_t p) {
    if (n <= 0 || p <= 0) return 256;
    return (int64_t)lr_layout(n, p, nullptr, nullptr);
}

extern "C" int ic_lowrank_eigs(const float* H, int64_t n, int64_t p, int iters, unsigned long long seed,
                               float refuse_rel, float* evals, float* evecs, int* sweeps_out, void* workspace,
                               void* stream) {
    IC_REQUIRE(H && evals && evecs && workspace, "ic_lowrank_eigs: null pointer");
    IC_REQUIRE(n >= 2 && p >= 2 && p <= n && p % 2 == 0, "ic_lowrank_eigs: need 2 <= p <= n, p even");
    IC_REQUIRE(p <= 4096 && iters >= 0 && iters <= 64, "ic_lowrank_eigs: p <= 4096, 0 <= iters <= 64");
    IC_REQUIRE(refuse_rel >= 0.0f, "ic_lowrank_eigs: refuse_rel must be >= 0");
    hipStream_t st = as_stream(stream);
    LrWork w;
    char* base = reinterpret_cast<char*>((reinterpret_cast<uintptr_t>(workspace) + 255) & ~(uintptr_t)255);
    lr_layout(n, p, base, &w);
    IC_CHECK_HIP(hipMemsetAsync(w.info, 0, 2 * sizeof(int), st));
    const int64_t np = n * p;
    // mu = 1e-3 lambda_max estimate (power iteration from a seeded vector)
    constexpr int POWER_STEPS = 16;
    hipLaunchKernelGGL(randn_kernel, dim3(egrid_lr(n)), dim3(256), 0, st, w.y, n, (uint64_t)seed ^ 0x5eedull);
    IC_CHECK_LAUNCH();
    hipLaunchKernelGGL(normalize_kernel, dim3(1), dim3(256), 0, st, w.y, w.x, n, 1e-3, w.scal);
    IC_CHECK_LAUNCH();
    for (int i = 0; i < POWER_STEPS; ++i) {
        hipLaunchKernelGGL(matvec_kernel, dim3((unsigned)cdiv(n, 4)), dim3(256), 0, st, H, n, w.x, w.y);
        IC_CHECK_LAUNCH();
        hipLaunchKernelGGL(normalize_kernel, dim3(1), dim3(256), 0, st, w.y, w.x, n, 1e-3, w.scal);
        IC_CHECK_LAUNCH();
    }
    hipLaunchKernelGGL(randn_kernel, dim3(egrid_lr(np)), dim3(256), 0, st, w.Y, np, (uint64_t)seed);
    IC_CHECK_LAUNCH();
    int rc = orth(w.Y, w.Q, n, p, w, st, /*well_conditioned=*/true);
    if (rc) return rc;
    // the refusal certificate is tried after one and after two steps (the
    // random start's Ritz values sit near the mean eigenvalue; one step of
    // (H + mu I) already lifts them for Hessians of high rank)
    const int test_lo = refuse_rel > 0.0f ? std::min(iters, 1) : -1;
    const int test_hi = refuse_rel > 0.0f ? std::min(iters, 2) : -1;
    for (int it = 0;; ++it) {
        // Y = H Q
        GemmArgs g{n, p, n, 1.0f, 0.0f, H, n, 0, w.Q, p, 0, w.Y, p, 0, 0, 0, CMASK_FULL, KR_FULL, 1, PT_OTHER};
        if ((rc = gemm_f32(g, st))) return rc;
        if (it >= test_lo && it <= test_hi && test_lo >= 0) {
            // Refusal certificate: if T - refuse_rel ||H||_F I is positive definite,
            // every Ritz value exceeds refuse_rel ||H||_F >= refuse_rel lambda_max,
            // and by interlacing so do the p largest eigenvalues of H.
            if ((rc = gram(w.Q, w.Y, n, p, w.T, w, CMASK_LOWER, st))) return rc;
            hipLaunchKernelGGL(sumsq_kernel, dim3(LR_PARTS), dim3(256), 0, st, H, n * n, w.part);
            IC_CHECK_LAUNCH();
            hipLaunchKernelGGL(sub_frob_diag_kernel, dim3(1), dim3(256), 0, st, w.T, p, w.part, LR_PARTS,
                               (double)refuse_rel);
            IC_CHECK_LAUNCH();
            if ((rc = potrf(w.T, 1, p, p, p * p, w.dinv64, w.info + 1, st))) return rc;
            int pd_info = 0;
            IC_CHECK_HIP(hipMemcpyAsync(&pd_info, w.info + 1, sizeof(int), hipMemcpyDeviceToHost, st));
            IC_CHECK_HIP(hipStreamSynchronize(st));
            if (pd_info == 0) {
                if (sweeps_out) *sweeps_out = 0;
                return IC_LOWRANK_REFUSED;
            }
        }
        if (it == iters) break;
        hipLaunchKernelGGL(axpy_dev_kernel, dim3(egrid_lr(np)), dim3(256), 0, st, w.Y, w.Q, np, w.scal);
        IC_CHECK_LAUNCH();
        if ((rc = orth(w.Y, w.Q, n, p, w, st))) return rc;
    }
    // Rayleigh-Ritz: T = Q^T (H Q)
    if ((rc = gram(w.Q, w.Y, n, p, w.T, w, CMASK_FULL, st))) return rc;
    int info = 0;
    IC_CHECK_HIP(hipMemcpyAsync(&info, w.info, sizeof(int), hipMemcpyDeviceToHost, st));
    IC_CHECK_HIP(hipStreamSynchronize(st));
    if (info != 0) return fail(IC_ERR_RANGE, "ic_lowrank_eigs: orthonormalisation lost positive definiteness");
    hipLaunchKernelGGL(jacobi_init_kernel, dim3(egrid_lr(p * p)), dim3(256), 0, st, w.T, p, w.A0, w.V0);
    IC_CHECK_LAUNCH();
    double *A = w.A0, *An = w.A1, *V = w.V0, *Vn = w.V1;
    const int64_t threads = (p / 2) * (p / 2) + p * (p / 2);
    const unsigned blocks = (unsigned)cdiv(threads, 256);
    const int off_blocks = (int)std::min<int64_t>(LR_PARTS, cdiv(p * p, 256));
    int sweeps = 0;
    for (; sweeps < JACOBI_MAX_SWEEPS; ++sweeps) {
        hipLaunchKernelGGL(offdiag_kernel, dim3(off_blocks), dim3(256), 0, st, A, p, w.part);
        IC_CHECK_LAUNCH();
        hipLaunchKernelGGL(finish_pairs_kernel, dim3(1), dim3(64), 0, st, w.part, off_blocks, w.scal + 2);
        IC_CHECK_LAUNCH();
        double od[2];
        IC_CHECK_HIP(hipMemcpyAsync(od, w.scal + 2, sizeof(od), hipMemcpyDeviceToHost, st));
        IC_CHECK_HIP(hipStreamSynchronize(st));
        if (!(od[0] > 1e-24 * od[1])) break;   // converged (or NaN: the caller sees NaN eigenvalues)
        for (int r = 0; r < p - 1; ++r) {
            hipLaunchKernelGGL(jacobi_round_kernel, dim3(blocks), dim3(256), 0, st, A, An, V, Vn, (int)p, r);
            IC_CHECK_LAUNCH();
            std::swap(A, An);
            std::swap(V, Vn);
        }
    }
    if (sweeps_out) *sweeps_out = sweeps;
    hipLaunchKernelGGL(ritz_sort_kernel, dim3((unsigned)cdiv(p, 64)), dim3(64), 0, st, A, V, p, evals, w.Vs);
    IC_CHECK_LAUNCH();
    // eigenvectors of H: Q Vs
    GemmArgs e{n, p, p, 1.0f, 0.0f, w.Q, p, 0, w.Vs, p, 0, evecs, p, 0, 0, 0, CMASK_FULL, KR_FULL, 1, PT_OTHER};
    return gemm_f32(e, st);
}
