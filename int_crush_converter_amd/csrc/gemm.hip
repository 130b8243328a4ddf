// fp32 GEMM on the CDNA4 matrix cores (v_mfma_f32_16x16x4_f32).
//
// Workgroup tile 128x128, K staged 16 at a time through double-buffered LDS;
// 4 waves in a 2x2 arrangement, each owning a 64x64 sub-tile held as 4x4
// MFMA 16x16 accumulators (64 VGPRs).  Per 4-wide k step a wave issues 16
// MFMAs (512 cycles of matrix-core time) against 8 LDS reads, so LDS is far
// from the bound; global traffic per tile step is 16 KB, served by L2.
//
// MFMA 16x16x4 f32 operand layout (lane l of 64):
//   A: A[i = l%16][k = l/16]      B: B[k = l/16][j = l%16]
//   D (4 VGPRs v): D[i = 4*(l/16) + v][j = l%16]
#include "gemm.hpp"

namespace icq {

typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int BM = 128, BN = 128, BK = 16;
constexpr int PITCH = BM + 16;   // LDS row pitch (floats): rows k, k+1.. land 16 banks apart

struct TileRange { int64_t i0, j0, klo, khi; bool skip; };

__device__ __forceinline__ int64_t isqrt_floor(int64_t x) {
    int64_t r = (int64_t)sqrt((double)x);
    while (r * r > x) --r;
    while ((r + 1) * (r + 1) <= x) ++r;
    return r;
}

// Map the linear block id to a tile.  Triangular masks enumerate only tiles
// that touch the kept triangle (square grids); for KR_FROM_MAXIJ the upper
// tiles are enumerated by increasing column block so that long-K tiles start
// first.
__device__ TileRange tile_of(const GemmArgs& g) {
    const int64_t tm = (g.M + BM - 1) / BM, tn = (g.N + BN - 1) / BN;
    const int64_t id = blockIdx.x;
    int64_t ti, tj;
    if (g.cmask == CMASK_LOWER && tm == tn) {
        int64_t r = (isqrt_floor(8 * id + 1) - 1) / 2;   // id -> (r, c), c <= r
        ti = r; tj = id - r * (r + 1) / 2;
    } else if (g.cmask == CMASK_UPPER && tm == tn) {
        int64_t r = (isqrt_floor(8 * id + 1) - 1) / 2;
        tj = r; ti = id - r * (r + 1) / 2;
    } else {
        ti = id / tn; tj = id - ti * tn;
    }
    TileRange t;
    t.i0 = ti * BM; t.j0 = tj * BN;
    t.skip = false;
    if (g.cmask == CMASK_LOWER && t.i0 + BM - 1 < t.j0) t.skip = true;
    if (g.cmask == CMASK_UPPER && t.j0 + BN - 1 < t.i0) t.skip = true;
    t.klo = 0; t.khi = g.K;
    if (g.krange == KR_FROM_MAXIJ) t.klo = t.i0 > t.j0 ? t.i0 : t.j0;
    else if (g.krange == KR_FROM_J) t.klo = t.j0;
    else if (g.krange == KR_TO_I) t.khi = min(g.K, t.i0 + BM);
    t.klo = (t.klo / BK) * BK;
    if (t.klo > g.K) t.klo = g.K;
    return t;
}

// Registers staged from global memory for one K step: 8 floats of A and 8 of B.
struct Stage { float a[8]; float b[8]; };

__device__ __forceinline__ float ldg(const float* p, int64_t r, int64_t c, int64_t ld, int64_t R, int64_t Cc) {
    return (r < R && c < Cc) ? p[r * ld + c] : 0.0f;
}

// op(A) tile [BM x BK] at (i0, k0); op(B) tile [BK x BN] at (k0, j0).
// Thread t covers 2 groups of 4 consecutive elements along the contiguous axis.
__device__ __forceinline__ void load_stage(const GemmArgs& g, const float* A, const float* B, int64_t i0,
                                           int64_t j0, int64_t k0, int64_t khi, Stage& s) {
    const int t = threadIdx.x;
#pragma unroll
    for (int p = 0; p < 2; ++p) {
        const int idx = t + p * 256;   // 0..511
        if (!g.transA) {               // A[i][k]: 128 rows x 4 quads of k
            int r = idx >> 2, kq = (idx & 3) * 4;
#pragma unroll
            for (int c = 0; c < 4; ++c) s.a[p * 4 + c] = ldg(A, i0 + r, k0 + kq + c, g.lda, g.M, khi);
        } else {                       // A[k][i]: 16 k rows x 32 quads of i
            int kr = idx >> 5, iq = (idx & 31) * 4;
#pragma unroll
            for (int c = 0; c < 4; ++c) s.a[p * 4 + c] = ldg(A, k0 + kr, i0 + iq + c, g.lda, khi, g.M);
        }
        if (!g.transB) {               // B[k][j]: 16 k rows x 32 quads of j
            int kr = idx >> 5, jq = (idx & 31) * 4;
#pragma unroll
            for (int c = 0; c < 4; ++c) s.b[p * 4 + c] = ldg(B, k0 + kr, j0 + jq + c, g.ldb, khi, g.N);
        } else {                       // B[j][k]: 128 j rows x 4 quads of k
            int r = idx >> 2, kq = (idx & 3) * 4;
#pragma unroll
            for (int c = 0; c < 4; ++c) s.b[p * 4 + c] = ldg(B, j0 + r, k0 + kq + c, g.ldb, g.N, khi);
        }
    }
}

__device__ __forceinline__ void store_stage(const GemmArgs& g, const Stage& s, float* As, float* Bs) {
    const int t = threadIdx.x;
#pragma unroll
    for (int p = 0; p < 2; ++p) {
        const int idx = t + p * 256;
        if (!g.transA) {
            int r = idx >> 2, kq = (idx & 3) * 4;
#pragma unroll
            for (int c = 0; c < 4; ++c) As[(kq + c) * PITCH + r] = s.a[p * 4 + c];
        } else {
            int kr = idx >> 5, iq = (idx & 31) * 4;
#pragma unroll
            for (int c = 0; c < 4; ++c) As[kr * PITCH + iq + c] = s.a[p * 4 + c];
        }
        if (!g.transB) {
            int kr = idx >> 5, jq = (idx & 31) * 4;
#pragma unroll
            for (int c = 0; c < 4; ++c) Bs[kr * PITCH + jq + c] = s.b[p * 4 + c];
        } else {
            int r = idx >> 2, kq = (idx & 3) * 4;
#pragma unroll
            for (int c = 0; c < 4; ++c) Bs[(kq + c) * PITCH + r] = s.b[p * 4 + c];
        }
    }
}

__global__ __launch_bounds__(256) void gemm_f32_kernel(GemmArgs g) {
    __shared__ float As[2][BK * PITCH];
    __shared__ float Bs[2][BK * PITCH];
    const TileRange tr = tile_of(g);
    if (tr.skip) return;
    const int64_t z = blockIdx.z;
    const float* A = g.A + z * g.sA;
    const float* B = g.B + z * g.sB;
    float* C = g.C + z * g.sC;

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wi = (wave >> 1) * 64, wj = (wave & 1) * 64;
    floatx4 acc[4][4];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b) acc[a][b] = floatx4{0.f, 0.f, 0.f, 0.f};

    Stage st;
    int buf = 0;
    if (tr.klo < tr.khi) {
        load_stage(g, A, B, tr.i0, tr.j0, tr.klo, tr.khi, st);
        store_stage(g, st, As[0], Bs[0]);
    }
    __syncthreads();
    for (int64_t k0 = tr.klo; k0 < tr.khi; k0 += BK) {
        const bool more = k0 + BK < tr.khi;
        if (more) load_stage(g, A, B, tr.i0, tr.j0, k0 + BK, tr.khi, st);
        const float* as = As[buf];
        const float* bs = Bs[buf];
#pragma unroll
        for (int kk = 0; kk < BK; kk += 4) {
            const int kr = kk + (lane >> 4);
            float av[4], bv[4];
#pragma unroll
            for (int a = 0; a < 4; ++a) av[a] = as[kr * PITCH + wi + a * 16 + (lane & 15)];
#pragma unroll
            for (int b = 0; b < 4; ++b) bv[b] = bs[kr * PITCH + wj + b * 16 + (lane & 15)];
#pragma unroll
            for (int a = 0; a < 4; ++a)
#pragma unroll
                for (int b = 0; b < 4; ++b)
                    acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[a], bv[b], acc[a][b], 0, 0, 0);
        }
        if (more) store_stage(g, st, As[buf ^ 1], Bs[buf ^ 1]);
        __syncthreads();
        buf ^= 1;
    }

    // epilogue
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int64_t i = tr.i0 + wi + a * 16 + 4 * (lane >> 4) + v;
                const int64_t j = tr.j0 + wj + b * 16 + (lane & 15);
                if (i >= g.M || j >= g.N) continue;
                if (g.cmask == CMASK_LOWER && i < j) continue;
                if (g.cmask == CMASK_UPPER && i > j) continue;
                float r = g.alpha * acc[a][b][v];
                float* cp = C + i * g.ldc + j;
                if (g.beta != 0.0f) r = r + g.beta * (*cp);
                *cp = r;
            }
}

int gemm_f32(const GemmArgs& g, hipStream_t st) {
    if (g.M <= 0 || g.N <= 0 || g.batch <= 0) return IC_OK;
    const int64_t tm = cdiv(g.M, BM), tn = cdiv(g.N, BN);
    int64_t tiles = tm * tn;
    if ((g.cmask == CMASK_LOWER || g.cmask == CMASK_UPPER) && tm == tn) tiles = tm * (tm + 1) / 2;
    IC_REQUIRE(tiles < (1LL << 31) && g.batch <= 65535, "gemm_f32: problem too large");
    const double fl = g.algo_flops > 0 ? g.algo_flops : 2.0 * g.M * g.N * g.K * g.batch;
    const double by = 4.0 * g.batch * (g.M * g.K + g.K * g.N + g.M * g.N * (g.beta != 0.0f ? 2 : 1));
    ProfScope prof_scope(st, g.tag, fl, by);
    hipLaunchKernelGGL(gemm_f32_kernel, dim3((unsigned)tiles, 1, (unsigned)g.batch), dim3(256), 0, st, g);
    IC_CHECK_LAUNCH();
    return IC_OK;
}

}  // namespace icq

using namespace icq;

extern "C" int ic_sgemm(int transA, int transB, int64_t M, int64_t N, int64_t K, float alpha, const float* A,
                        int64_t lda, const float* B, int64_t ldb, float beta, float* C, int64_t ldc, int cmask,
                        int krange, void* stream) {
    IC_REQUIRE(A && B && C, "ic_sgemm: null pointer");
    IC_REQUIRE(M >= 0 && N >= 0 && K >= 0, "ic_sgemm: negative size");
    IC_REQUIRE(cmask >= 0 && cmask <= 2 && krange >= 0 && krange <= 3, "ic_sgemm: bad mask");
    GemmArgs g{M, N, K, alpha, beta, A, lda, 0, B, ldb, 0, C, ldc, 0, transA, transB, cmask, krange, 1};
    return gemm_f32(g, as_stream(stream));
}
