// fp32 GEMM on the CDNA4 matrix cores (v_mfma_f32_16x16x4_f32).
//
// Workgroup tile 128x128, K staged 32 at a time through LDS; 4 waves in a
// 2x2 arrangement, each owning a 64x64 sub-tile held as 4x4 MFMA 16x16
// accumulators (64 AGPR/VGPRs).  Per stage a wave issues 128 MFMAs (4096
// cycles of matrix-core time) against 64 LDS reads; the next stage's global
// loads are issued right after the LDS write of the current one, so their
// latency hides behind a full stage of MFMAs.  Interior tiles use 16-byte
// global loads; edge tiles take a bounds-checked path.  Work-group ids are
// remapped so that each XCD (ids congruent mod 8) owns a contiguous run of
// tiles that share A rows / B columns in its own L2.
//
// MFMA 16x16x4 f32 operand layout (lane l of 64):
//   A: A[i = l%16][k = l/16]      B: B[k = l/16][j = l%16]
//   D (4 VGPRs v): D[i = 4*(l/16) + v][j = l%16]
#include "gemm.hpp"

namespace icq {

typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int BM = 128, BN = 128, BK = 32;
constexpr int PITCH = BM + 16;   // LDS row pitch (floats): k-rows land 16 banks apart
constexpr int NXCD = 8;

struct TileRange { int64_t i0, j0, klo, khi; bool skip; };

__device__ __forceinline__ int64_t isqrt_floor(int64_t x) {
    int64_t r = (int64_t)sqrt((double)x);
    while (r * r > x) --r;
    while ((r + 1) * (r + 1) <= x) ++r;
    return r;
}

// Linear tile id -> tile.  Triangular masks enumerate only tiles that touch
// the kept triangle (square grids); for KR_FROM_MAXIJ the upper tiles are
// enumerated by increasing column block so that long-K tiles start first.
__device__ TileRange tile_of(const GemmArgs& g, int64_t id) {
    const int64_t tm = (g.M + BM - 1) / BM, tn = (g.N + BN - 1) / BN;
    int64_t ti, tj;
    if (g.cmask == CMASK_LOWER && tm == tn) {
        int64_t r = (isqrt_floor(8 * id + 1) - 1) / 2;   // id -> (r, c), c <= r
        ti = r; tj = id - r * (r + 1) / 2;
    } else if (g.cmask == CMASK_UPPER && tm == tn) {
        int64_t r = (isqrt_floor(8 * id + 1) - 1) / 2;
        tj = r; ti = id - r * (r + 1) / 2;
    } else {
        ti = id / tn; tj = id - ti * tn;
        // K range grows with the tile row: start the long tiles first
        if (g.krange == KR_TO_I) ti = tm - 1 - ti;
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
    else if (g.krange == KR_FROM_I) t.klo = t.i0;
    t.klo = (t.klo / 4) * 4;
    if (t.klo > g.K) t.klo = g.K;
    return t;
}

// Registers staged from global memory for one K stage: 16 floats of A, 16 of B.
struct Stage { float4 a[4]; float4 b[4]; };

__device__ __forceinline__ float ldg(const float* p, int64_t r, int64_t c, int64_t ld, int64_t R, int64_t Cc) {
    return (r < R && c < Cc) ? p[r * ld + c] : 0.0f;
}

// Operand tiles: op(A) [BM x BK] at (i0, k0), op(B) [BK x BN] at (k0, j0).
// "Row-contiguous" layouts (A not transposed, B transposed) are read as
// 128 rows x 8 float4 of k; the others as 32 k-rows x 32 float4.
// Thread t, slot p (0..3): idx = t + 256 p.
__device__ __forceinline__ void rc_coords(int idx, int& r, int& kq) { r = idx >> 3; kq = (idx & 7) * 4; }
__device__ __forceinline__ void kc_coords(int idx, int& kr, int& cq) { kr = idx >> 5; cq = (idx & 31) * 4; }

__device__ __forceinline__ float4 ldg4(const float* p, int64_t r, int64_t c, int64_t ld, int64_t R, int64_t Cc,
                                       bool fast) {
    if (fast) return *reinterpret_cast<const float4*>(p + r * ld + c);
    return make_float4(ldg(p, r, c, ld, R, Cc), ldg(p, r, c + 1, ld, R, Cc), ldg(p, r, c + 2, ld, R, Cc),
                       ldg(p, r, c + 3, ld, R, Cc));
}

__device__ __forceinline__ void load_stage(const GemmArgs& g, const float* A, const float* B, const TileRange& tr,
                                           int64_t k0, bool fast, Stage& s) {
    const int t = threadIdx.x;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        const int idx = t + p * 256;
        int r, q;
        if (!g.transA) { rc_coords(idx, r, q); s.a[p] = ldg4(A, tr.i0 + r, k0 + q, g.lda, g.M, tr.khi, fast); }
        else { kc_coords(idx, r, q); s.a[p] = ldg4(A, k0 + r, tr.i0 + q, g.lda, tr.khi, g.M, fast); }
        if (!g.transB) { kc_coords(idx, r, q); s.b[p] = ldg4(B, k0 + r, tr.j0 + q, g.ldb, tr.khi, g.N, fast); }
        else { rc_coords(idx, r, q); s.b[p] = ldg4(B, tr.j0 + r, k0 + q, g.ldb, g.N, tr.khi, fast); }
    }
}

// LDS holds As[k][i] and Bs[k][j] (k-major, pitch PITCH).
__device__ __forceinline__ void store_stage(const GemmArgs& g, const Stage& s, float* As, float* Bs) {
    const int t = threadIdx.x;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        const int idx = t + p * 256;
        int r, q;
        if (!g.transA) {
            rc_coords(idx, r, q);
            As[(q + 0) * PITCH + r] = s.a[p].x; As[(q + 1) * PITCH + r] = s.a[p].y;
            As[(q + 2) * PITCH + r] = s.a[p].z; As[(q + 3) * PITCH + r] = s.a[p].w;
        } else {
            kc_coords(idx, r, q);
            *reinterpret_cast<float4*>(&As[r * PITCH + q]) = s.a[p];
        }
        if (!g.transB) {
            kc_coords(idx, r, q);
            *reinterpret_cast<float4*>(&Bs[r * PITCH + q]) = s.b[p];
        } else {
            rc_coords(idx, r, q);
            Bs[(q + 0) * PITCH + r] = s.b[p].x; Bs[(q + 1) * PITCH + r] = s.b[p].y;
            Bs[(q + 2) * PITCH + r] = s.b[p].z; Bs[(q + 3) * PITCH + r] = s.b[p].w;
        }
    }
}

__global__ __launch_bounds__(256) void gemm_f32_kernel(GemmArgs g, int64_t ntiles, int remap, int aligned) {
    __shared__ __attribute__((aligned(16))) float As[BK * PITCH];
    __shared__ __attribute__((aligned(16))) float Bs[BK * PITCH];
    int64_t id = blockIdx.x;
    if (remap) {   // XCD-contiguous tile runs
        const int64_t per = (ntiles + NXCD - 1) / NXCD;
        id = (id % NXCD) * per + id / NXCD;
        if (id >= ntiles) return;
    }
    const TileRange tr = tile_of(g, id);
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

    const bool interior = aligned && tr.i0 + BM <= g.M && tr.j0 + BN <= g.N;
    Stage st;
    int64_t k0 = tr.klo;
    if (k0 < tr.khi) load_stage(g, A, B, tr, k0, interior && k0 + BK <= tr.khi, st);
    for (; k0 < tr.khi; k0 += BK) {
        __syncthreads();                       // previous stage's LDS reads are done
        store_stage(g, st, As, Bs);
        __syncthreads();
        const int64_t kn = k0 + BK;
        if (kn < tr.khi) load_stage(g, A, B, tr, kn, interior && kn + BK <= tr.khi, st);
#pragma unroll
        for (int kk = 0; kk < BK; kk += 4) {
            const int kr = kk + (lane >> 4);
            float av[4], bv[4];
#pragma unroll
            for (int a = 0; a < 4; ++a) av[a] = As[kr * PITCH + wi + a * 16 + (lane & 15)];
#pragma unroll
            for (int b = 0; b < 4; ++b) bv[b] = Bs[kr * PITCH + wj + b * 16 + (lane & 15)];
#pragma unroll
            for (int a = 0; a < 4; ++a)
#pragma unroll
                for (int b = 0; b < 4; ++b)
                    acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[a], bv[b], acc[a][b], 0, 0, 0);
        }
    }

    // epilogue: all C loads are issued before any store so their latency overlaps
    float cold[4][4][4];
    if (g.beta != 0.0f) {
#pragma unroll
        for (int a = 0; a < 4; ++a)
#pragma unroll
            for (int b = 0; b < 4; ++b)
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int64_t i = tr.i0 + wi + a * 16 + 4 * (lane >> 4) + v;
                    const int64_t j = tr.j0 + wj + b * 16 + (lane & 15);
                    cold[a][b][v] = (i < g.M && j < g.N) ? C[i * g.ldc + j] : 0.0f;
                }
    }
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
                if (g.beta != 0.0f) r = r + g.beta * cold[a][b][v];
                C[i * g.ldc + j] = r;
            }
}

int gemm_f32(const GemmArgs& g, hipStream_t st) {
    if (g.M <= 0 || g.N <= 0 || g.batch <= 0) return IC_OK;
    const int64_t tm = cdiv(g.M, BM), tn = cdiv(g.N, BN);
    int64_t tiles = tm * tn;
    const bool tri = (g.cmask == CMASK_LOWER || g.cmask == CMASK_UPPER) && tm == tn;
    if (tri) tiles = tm * (tm + 1) / 2;
    IC_REQUIRE(tiles < (1LL << 30) && g.batch <= 65535, "gemm_f32: problem too large");
    // 16-byte loads need 16-byte aligned bases and leading dimensions
    const bool aligned = ((uintptr_t)g.A % 16 == 0) && ((uintptr_t)g.B % 16 == 0) && g.lda % 4 == 0 &&
                         g.ldb % 4 == 0 && g.sA % 4 == 0 && g.sB % 4 == 0;
    // triangular enumerations keep their own (long-K-first) order
    const int remap = (!tri && tiles >= 2 * NXCD) ? 1 : 0;
    const int64_t grid = remap ? cdiv(tiles, NXCD) * NXCD : tiles;
    const double fl = g.algo_flops > 0 ? g.algo_flops : 2.0 * g.M * g.N * g.K * g.batch;
    const double by = 4.0 * g.batch * (g.M * g.K + g.K * g.N + g.M * g.N * (g.beta != 0.0f ? 2 : 1));
    ProfScope prof_scope(st, g.tag, fl, by);
    hipLaunchKernelGGL(gemm_f32_kernel, dim3((unsigned)grid, 1, (unsigned)g.batch), dim3(256), 0, st, g, tiles, remap,
                       (int)aligned);
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
    IC_REQUIRE(cmask >= 0 && cmask <= 2 && krange >= 0 && krange <= 4, "ic_sgemm: bad mask");
    GemmArgs g{M, N, K, alpha, beta, A, lda, 0, B, ldb, 0, C, ldc, 0, transA, transB, cmask, krange, 1};
    return gemm_f32(g, as_stream(stream));
}
