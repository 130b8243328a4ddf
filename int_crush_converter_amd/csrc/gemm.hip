// fp32 GEMM on the CDNA4 matrix cores: the kernels and their host-side
// dispatch (tile size, bounds-check-free instances, XCD remapping).  The
// device code is in gemm_dev.hpp.
#include "gemm_dev.hpp"

namespace icq {
using namespace gk;

// CHUNK_SUB (GemmArgs::chunk_sub; alpha = -1, beta = 1): C is read before the
// K loop and every chunk is subtracted from it; CHUNK_SUM keeps the
// epilogue C <- alpha * sum + beta * C.
// Two work-groups per CU (one wave of each per SIMD) hide each other's
// barriers and LDS staging: the register budget is held to 256 per lane.
// remap bit 0: the XCD-aware tile order (xcd_tile); bit 1: batch entries of
// odd index walk their tiles in reverse.  The hardware deals the work-groups
// of consecutive batch entries to the CUs in the same pattern, so in a launch
// that is resident in one round a CU would otherwise get the same tile
// position, and so the same K range, from every entry.
template <int TA, int TB, bool CHECK, int T, int CHUNK>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void gemm_f32_kernel(GemmArgs g,
                                                                                              int64_t ntiles,
                                                                                              int remap) {
    __shared__ __attribute__((aligned(16))) float lds[2 * Geo<T>::TILE_F];
    TileRange tr;
    const bool mirror = (remap & 2) && (blockIdx.z & 1);
    if (remap & 1) {
        if (!xcd_tile<T>(g, blockIdx.x, tr, mirror)) return;
    } else {
        if ((int64_t)blockIdx.x >= ntiles) return;
        tr = tile_of<T>(g, mirror ? ntiles - 1 - (int64_t)blockIdx.x : (int64_t)blockIdx.x);
    }
    if (tr.skip) return;
    gemm_tile<TA, TB, CHECK, T, CHUNK>(g, tr, blockIdx.z, lds);
}

constexpr int64_t CHIP_CUS = 256;

// Work-groups of gemm_f32_kernel<0, 0, CHECK, T, CHUNK_SUM> resident per CU
// (the instances of one T and CHECK differ little in registers).
template <int T, bool CHECK>
static int resident_per_cu() {
    static const int n = [] {
        int v = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&v, gemm_f32_kernel<0, 0, CHECK, T, CHUNK_SUM>, 256, 0) !=
            hipSuccess)
            v = 1;
        return v > 0 ? v : 1;
    }();
    return n;
}

template <int T>
static int launch_gemm(const GemmArgs& g, bool aligned, hipStream_t st) {
    bool tri;
    const int64_t tiles = tile_count<T>(g, tri);
    const int64_t tm = cdiv(g.M, T), tn = cdiv(g.N, T);
    IC_REQUIRE(tiles < (1LL << 30) && g.batch <= 65535, "gemm_f32: problem too large");
    // triangular enumerations keep their own (long-K-first) order; other
    // grids with at least NXCD tile rows use the XCD row assignment
    const int xcd = (!tri && tm >= NXCD) ? 1 : 0;
    const int64_t grid = xcd ? cdiv(tm, NXCD) * tn * NXCD : tiles;
    IC_REQUIRE(grid < (1LL << 23), "gemm_f32: problem too large");
    const dim3 gd((unsigned)grid, 1, (unsigned)g.batch);
    // whole tiles and whole K stages everywhere: the kernel without bounds checks
    const bool exact = aligned && g.M % T == 0 && g.N % T == 0 && g.K % BK == 0;
    // batched rectangular launches whose K range depends on the tile position
    // and that are resident in one round: odd batch entries in reverse, so
    // that every CU gets long and short tiles alike
    int remap = xcd;
    if (g.batch > 1 && !tri && g.krange != KR_FULL) {
        const int per_cu = exact ? resident_per_cu<T, false>() : resident_per_cu<T, true>();
        if (grid * g.batch <= (int64_t)per_cu * CHIP_CUS) remap |= 2;
    }
    // exact rank-kc update sequences subtract chunk by chunk; everything else
    // sums the chunks and applies alpha, beta once.  With one chunk (K <= kc)
    // the two are the same: fl(-P + C) = fl(C - P), and the sum form keeps C
    // out of the registers of the K loop.
    const bool sub = g.chunk_sub != 0 && g.K > g.kc;
#define ICQ_GEMM_LAUNCH(TA, TB, CH)                                                                                    \
    do {                                                                                                              \
        if (exact) hipLaunchKernelGGL((gemm_f32_kernel<TA, TB, false, T, CH>), gd, dim3(256), 0, st, g, tiles, remap);  \
        else hipLaunchKernelGGL((gemm_f32_kernel<TA, TB, true, T, CH>), gd, dim3(256), 0, st, g, tiles, remap);         \
    } while (0)
    if (!g.transA && !g.transB) {
        if (sub) ICQ_GEMM_LAUNCH(0, 0, CHUNK_SUB);
        else ICQ_GEMM_LAUNCH(0, 0, CHUNK_SUM);
    } else if (!g.transA) {
        if (sub) ICQ_GEMM_LAUNCH(0, 1, CHUNK_SUB);
        else ICQ_GEMM_LAUNCH(0, 1, CHUNK_SUM);
    } else if (!g.transB) {
        ICQ_GEMM_LAUNCH(1, 0, CHUNK_SUM);
    } else {
        ICQ_GEMM_LAUNCH(1, 1, CHUNK_SUM);
    }
#undef ICQ_GEMM_LAUNCH
    IC_CHECK_LAUNCH();
    return IC_OK;
}

// Launches with fewer 128-tiles than the chip has CUs run 64-tiles, and so
// do short-K launches (rank-128 updates) with up to two 128-tiles per CU:
// there the 128-tile's few long stages leave the tail of the launch on a
// fraction of the chip.
constexpr int64_t SMALL_TILE_LIMIT = 256;
// Tiles whose K range depends on their position (the inverse's merges, K
// from the tile column or up to the tile row, and its X^T X, K from max(tile
// row, tile column)): when the longest 128-tile, sharing its CU with a
// second work-group, outlasts the average 128-tile work per CU, the launch
// is bound by that one tile, and 64-tiles cut it to a quarter (same chunks
// of K, same order of accumulation, so the same results).
static bool long_tile_bound(const GemmArgs& g) {
    if (g.krange == KR_FULL) return false;
    const int64_t tm = cdiv(g.M, 128), tn = cdiv(g.N, 128);
    double total = 0.0, longest = 0.0;   // K stages
    for (int64_t ti = 0; ti < tm; ++ti)
        for (int64_t tj = 0; tj < tn; ++tj) {
            const int64_t i0 = ti * 128, j0 = tj * 128;
            if (g.cmask == CMASK_LOWER && i0 + 127 < j0) continue;
            if (g.cmask == CMASK_UPPER && j0 + 127 < i0) continue;
            int64_t klo = 0, khi = g.K;
            if (g.krange == KR_FROM_MAXIJ) klo = std::max(i0, j0);
            else if (g.krange == KR_FROM_J) klo = j0;
            else if (g.krange == KR_TO_I) khi = std::min(g.K, i0 + 128);
            else if (g.krange == KR_FROM_I) klo = i0;
            klo = std::min((klo / 4) * 4, g.K);
            const double st = (double)cdiv(std::max<int64_t>(0, khi - klo), BK);
            total += st;
            longest = std::max(longest, st);
        }
    return 2.0 * longest > total * g.batch / CHIP_CUS;
}
constexpr int64_t SHORT_K = 256, SHORT_K_TILE_LIMIT = 1024;

int gemm_f32(const GemmArgs& g, hipStream_t st) {
    if (g.M <= 0 || g.N <= 0 || g.batch <= 0) return IC_OK;
    IC_REQUIRE(g.kc >= BK && g.kc <= 4096 && (g.kc & (g.kc - 1)) == 0, "gemm_f32: kc must be a power of two >= 32");
    IC_REQUIRE(!g.chunk_sub || (g.alpha == -1.0f && g.beta == 1.0f && !g.transA),
               "gemm_f32: chunk-by-chunk subtraction needs alpha = -1, beta = 1 and op(A) = A");
    // 16-byte loads need 16-byte aligned bases and leading dimensions
    const bool aligned = ((uintptr_t)g.A % 16 == 0) && ((uintptr_t)g.B % 16 == 0) && g.lda % 4 == 0 &&
                         g.ldb % 4 == 0 && g.sA % 4 == 0 && g.sB % 4 == 0;
    const double fl = g.algo_flops > 0 ? g.algo_flops : 2.0 * g.M * g.N * g.K * g.batch;
    const double by = 4.0 * g.batch * (g.M * g.K + g.K * g.N + g.M * g.N * (g.beta != 0.0f ? 2 : 1));
    ProfScope prof_scope(st, g.tag, fl, by);
    bool tri;
    const int64_t t128 = tile_count<128>(g, tri) * g.batch;
    if (t128 < SMALL_TILE_LIMIT || (g.K <= SHORT_K && t128 < SHORT_K_TILE_LIMIT)) return launch_gemm<64>(g, aligned, st);
    if (long_tile_bound(g)) return launch_gemm<64>(g, aligned, st);
    // Triangular grids with the whole K per tile (the Cholesky's SYRK, the
    // Gram products): 64-tiles measured faster at every trailing size of
    // the headline layer (5.31 -> 5.04 ms of SYRK per layer; 300 128-tiles
    // 148 -> 100 us, 3916 1194 -> 1170 us)
    if (tri && g.krange == KR_FULL) return launch_gemm<64>(g, aligned, st);
    return launch_gemm<128>(g, aligned, st);
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
    // C - A op(B) subtracts one 128-wide chunk of K at a time, the sequence
    // of the reference's per-block updates
    g.chunk_sub = (alpha == -1.0f && beta == 1.0f && !transA) ? 1 : 0;
    return gemm_f32(g, as_stream(stream));
}
