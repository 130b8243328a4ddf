// fp32 GEMM on the CDNA4 matrix cores (v_mfma_f32_16x16x4_f32).
//
// Workgroup tile T x T (T = 128, or 64 for launches with fewer 128-tiles
// than CUs), K staged 32 at a time through LDS; 4 waves in a 2x2
// arrangement, each owning a T/2 x T/2 sub-tile held as F x F MFMA 16x16
// accumulators (F = T / 32).  For T = 128 a wave issues 128 MFMAs per stage
// (4096 cycles of matrix-core time) against 64 LDS reads; the next stage's
// global loads are issued before the current stage's MFMAs so their latency
// hides behind them.  The 64 tile has a quarter of the matrix work per
// stage, so a small launch (e.g. a rank-128 update of a few column blocks)
// spreads over four times as many CUs and its latency falls accordingly.  Work-group ids are remapped so that each XCD (ids congruent mod 8)
// owns a balanced set of tile rows and runs 8x8 blocks of tiles at a time,
// which share A rows / B columns in its L2.
//
// Each operand is staged in LDS in its memory order, so every global load
// and LDS store is a 16-byte vector: a row-major operand tile (A, or B^T)
// as T rows x 32 k at pitch 36 floats, a k-major one (A^T, or B) as 32 k
// rows x T at pitch T + 16.  Both pitches make the MFMA operand reads (16
// consecutive rows or columns per k) free of bank conflicts.  The transposes
// are template parameters, and problems made of whole tiles and whole K
// stages run a kernel instance without bounds checks.
//
// MFMA 16x16x4 f32 operand layout (lane l of 64):
//   A: A[i = l%16][k = l/16]      B: B[k = l/16][j = l%16]
//   D (4 VGPRs v): D[i = 4*(l/16) + v][j = l%16]
//
// This header holds the device code (tile geometry, operand staging, MFMA
// stages, the tile body), in namespace icq::gk: gemm.hip's kernels use it,
// and so do kernels that run GEMM tiles beside other work in one launch.
#pragma once

#include "gemm.hpp"

namespace icq {
namespace gk {

typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int BK = 32;
constexpr int PR = BK + 4;        // pitch of a row-major operand tile [T][32]
constexpr int NXCD = 8;
// Accumulation chunk: every kc values of k (aligned to absolute multiples of
// kc, GemmArgs::kc) a fresh set of accumulators is summed, then folded into the running
// result.  A single fp32 accumulator over a long K range gathers rounding
// error in proportion to K; chunking keeps it near kc + K / kc, like a
// blocked CPU BLAS.  With alpha = -1, beta = 1 the running result starts
// as C and each chunk's product is subtracted from it as soon as it is
// complete: C <- (..((C - P_0) - P_1)..) - P_last, the sequence of roundings of
// consecutive rank-kc updates (the GPTQ / LDLQ lazy updates of the
// reference, one per block of kc columns: bit-exact with them when the
// chunk products are).
enum ChunkMode : int { CHUNK_SUM = 1, CHUNK_SUB = 2 };

// Tile geometry for tile size T (the output tile is T x T).
template <int T>
struct Geo {
    static constexpr int F = T / 32;            // MFMA fragments per wave and dimension
    static constexpr int WS = T / 2;             // wave sub-tile
    static constexpr int PKM = T + 16;           // pitch of a k-major operand tile [32][T]
    static constexpr int SLOTS = T / 32;         // float4 per thread and operand per stage
    static constexpr int KROWS = 1024 / T;       // k rows one slot of a k-major tile covers
    static constexpr int TILE_F = T * PR > BK * PKM ? T * PR : BK * PKM;   // floats per operand tile
};

struct TileRange { int64_t i0, j0, klo, khi; bool skip; };

__device__ __forceinline__ int64_t isqrt_floor(int64_t x) {
    int64_t r = (int64_t)sqrt((double)x);
    while (r * r > x) --r;
    while ((r + 1) * (r + 1) <= x) ++r;
    return r;
}

// The tile (ti, tj) with its K range.
template <int T>
__device__ __forceinline__ TileRange tile_range(const GemmArgs& g, int64_t ti, int64_t tj) {
    TileRange t;
    t.i0 = ti * T; t.j0 = tj * T;
    t.skip = false;
    if (g.cmask == CMASK_LOWER && t.i0 + T - 1 < t.j0) t.skip = true;
    if (g.cmask == CMASK_UPPER && t.j0 + T - 1 < t.i0) t.skip = true;
    t.klo = 0; t.khi = g.K;
    if (g.krange == KR_FROM_MAXIJ) t.klo = t.i0 > t.j0 ? t.i0 : t.j0;
    else if (g.krange == KR_FROM_J) t.klo = t.j0;
    else if (g.krange == KR_TO_I) t.khi = min(g.K, t.i0 + T);
    else if (g.krange == KR_FROM_I) t.klo = t.i0;
    t.klo = (t.klo / 4) * 4;
    if (t.klo > g.K) t.klo = g.K;
    return t;
}

// Linear tile id -> tile.  Triangular masks enumerate only tiles that touch
// the kept triangle (square grids); for KR_FROM_MAXIJ the upper tiles are
// enumerated by increasing column block so that long-K tiles start first.
template <int T>
__device__ TileRange tile_of(const GemmArgs& g, int64_t id) {
    const int64_t tm = (g.M + T - 1) / T, tn = (g.N + T - 1) / T;
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
    return tile_range<T>(g, ti, tj);
}

// Work-group b -> tile for rectangular grids with at least NXCD tile rows.
// The hardware deals work-groups to the XCDs round-robin (b mod NXCD), then
// to the 4 shader engines of the XCD round-robin (its l-th group to engine
// l mod 4); only inside an engine does a group take whichever CU frees
// first.  XCD x owns the tile rows of a snake order (round q hands rows
// NXCD q .. NXCD q + 7 to XCDs 0..7, reversed in odd rounds), which
// balances per-row work that grows or shrinks with the row.  Inside the
// XCD, uniform or column-dependent work walks groups of NXCD rows column by
// column (the 64 tiles an XCD runs at once form an 8x8 block, 16 operand
// panels in its L2); row-dependent work (KR_TO_I, KR_FROM_I) walks rows
// one after another, longest first, so that every engine gets every 4th
// tile of every row.  False: no tile.
// mirror: the XCD's sequence of tiles reversed (batch entries of odd index,
// see gemm_f32_kernel).
template <int T>
__device__ __forceinline__ bool xcd_tile(const GemmArgs& g, int64_t b, TileRange& t, bool mirror = false) {
    const int64_t tm = (g.M + T - 1) / T, tn = (g.N + T - 1) / T;
    const int x = (int)(b % NXCD);
    int64_t l = b / NXCD;
    const int64_t full = tm / NXCD, rem = tm - full * NXCD;
    const int lastpos = (full & 1) ? (NXCD - 1 - x) : x;
    const int64_t nr = full + (lastpos < rem ? 1 : 0);   // tile rows of XCD x
    if (l >= nr * tn) return false;
    if (mirror) l = nr * tn - 1 - l;
    int64_t q, tj;                                       // q: round = row index within XCD x
    if (g.krange == KR_TO_I || g.krange == KR_FROM_I) {
        q = l / tn;
        tj = l - q * tn;
        if (g.krange == KR_TO_I) q = nr - 1 - q;         // K grows with the row: last rows first
    } else {
        const int64_t g0 = (l / (NXCD * tn)) * NXCD;    // first row (of XCD x) of l's group
        const int64_t G = min((int64_t)NXCD, nr - g0);
        const int64_t w = l - g0 * tn;
        tj = w / G;
        q = g0 + (w - tj * G);
    }
    const int64_t ti = q * NXCD + ((q & 1) ? (NXCD - 1 - x) : x);
    t = tile_range<T>(g, ti, tj);
    return true;
}

// One operand's share of a stage: SLOTS float4 per thread (kept in named
// registers so that no unrolled index can push them to scratch; T = 64
// uses the first two).
struct Quad { floatx4 v0, v1, v2, v3; };

template <int S>
__device__ __forceinline__ floatx4& qslot(Quad& q) {
    static_assert(S >= 0 && S < 4, "slot");
    if constexpr (S == 0) return q.v0;
    else if constexpr (S == 1) return q.v1;
    else if constexpr (S == 2) return q.v2;
    else return q.v3;
}
template <int S>
__device__ __forceinline__ const floatx4& qslot(const Quad& q) {
    if constexpr (S == 0) return q.v0;
    else if constexpr (S == 1) return q.v1;
    else if constexpr (S == 2) return q.v2;
    else return q.v3;
}

// A row-major tile (ROWMAJ: element (r, k) at p[r * ld + k]) is read as T
// rows x 8 float4 of k; a k-major one (element (k, c) at p[k * ld + c]) as 32
// k-rows x T/4 float4.  Thread t, slot s: idx = t + 256 s.
template <bool ROWMAJ, int T>
struct OperandLoader {
    using G = Geo<T>;
    const float* p;     // this thread's slot-0 element at the current stage
    int64_t step;       // pointer advance per stage
    int64_t slot;       // pointer distance between slots
    int r, c;           // slot-0 coordinates in the tile: (row, k) or (k, col)

    __device__ __forceinline__ void init(const float* base, int64_t ld, int64_t m0, int64_t k0) {
        const int t = threadIdx.x;
        if (ROWMAJ) {
            r = t >> 3; c = (t & 7) * 4;
            p = base + (m0 + r) * ld + k0 + c;
            step = BK; slot = 32 * ld;
        } else {
            r = t / (T / 4); c = (t % (T / 4)) * 4;
            p = base + (k0 + r) * ld + m0 + c;
            step = (int64_t)BK * ld; slot = G::KROWS * ld;
        }
    }
    __device__ __forceinline__ void load_fast(Quad& q) const {
        q.v0 = *reinterpret_cast<const floatx4*>(p);
        q.v1 = *reinterpret_cast<const floatx4*>(p + slot);
        if constexpr (G::SLOTS == 4) {
            q.v2 = *reinterpret_cast<const floatx4*>(p + 2 * slot);
            q.v3 = *reinterpret_cast<const floatx4*>(p + 3 * slot);
        }
    }
    // Element (m, k) exists when m < mlim and k < klim; m0 / k0 are the
    // tile's / stage's origins.
    __device__ __forceinline__ floatx4 get_checked(int s, int64_t m0, int64_t k0, int64_t mlim, int64_t klim,
                                                  int64_t ld, const float* base) const {
        float e[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            int64_t m, k;
            if (ROWMAJ) { m = m0 + r + 32 * s; k = k0 + c + u; }
            else { k = k0 + r + G::KROWS * s; m = m0 + c + u; }
            e[u] = (m < mlim && k < klim) ? base[ROWMAJ ? m * ld + k : k * ld + m] : 0.0f;
        }
        return floatx4{e[0], e[1], e[2], e[3]};
    }
    __device__ __forceinline__ void load_checked(Quad& q, int64_t m0, int64_t k0, int64_t mlim, int64_t klim,
                                                 int64_t ld, const float* base) const {
        q.v0 = get_checked(0, m0, k0, mlim, klim, ld, base);
        q.v1 = get_checked(1, m0, k0, mlim, klim, ld, base);
        if constexpr (G::SLOTS == 4) {
            q.v2 = get_checked(2, m0, k0, mlim, klim, ld, base);
            q.v3 = get_checked(3, m0, k0, mlim, klim, ld, base);
        }
    }
    __device__ __forceinline__ floatx4* at(float* tile, int s) const {
        return ROWMAJ ? reinterpret_cast<floatx4*>(&tile[(r + 32 * s) * PR + c])
                      : reinterpret_cast<floatx4*>(&tile[(r + G::KROWS * s) * G::PKM + c]);
    }
    __device__ __forceinline__ void store_lds(const Quad& q, float* tile) const {
        *at(tile, 0) = q.v0;
        *at(tile, 1) = q.v1;
        if constexpr (G::SLOTS == 4) {
            *at(tile, 2) = q.v2;
            *at(tile, 3) = q.v3;
        }
    }
};

// LDS offset of operand element (m, k) of a tile: row-major tiles are
// m-major at pitch PR, k-major tiles k-major at pitch PKM.
template <bool ROWMAJ, int T>
__device__ __forceinline__ int lds_at(int m, int k) { return ROWMAJ ? m * PR + k : k * Geo<T>::PKM + m; }

// F-wide vector of floats (F = 4: 16 bytes, F = 2: 8 bytes).
template <int F> struct VecF;
template <> struct VecF<4> { typedef float type __attribute__((ext_vector_type(4))); };
template <> struct VecF<2> { typedef float type __attribute__((ext_vector_type(2))); };

// One BK stage of a wave's WS x WS sub-tile; MFMA step s of a group of 16 k
// feeds k = 4 s + l / 16 from lane l.  When both operands are staged k-major
// (A^T B: the LAUUM), each permutes its rows (A) or columns (B) inside the
// wave's sub-tile - fragment a / b at MFMA row / column m is row F m + a /
// column F m + b - so one F-wide LDS read gives a lane all F fragments of
// one step (WIDE).  Otherwise each fragment value is one 4-byte read, which
// measured faster there.
//   row of accumulator (a, v) at lane l:  wi + 16 a + 4 (l/16) + v,  WIDE: wi + F (4 (l/16) + v) + a
//   column of (b) at lane l:              wj + 16 b + l%16,          WIDE: wj + F (l%16) + b
template <int TA, int TB, int T>
__device__ __forceinline__ void mma_stage(const float* As, const float* Bs, int wi, int wj, int lane,
                                          floatx4 (&acc)[Geo<T>::F][Geo<T>::F]) {
    constexpr int F = Geo<T>::F, PKM = Geo<T>::PKM;
    constexpr bool AR = TA == 0, BR = TB == 1;   // row-major staging
    constexpr bool WIDE = !AR && !BR;
    typedef typename VecF<F>::type vecf;
    const int m = lane & 15, g = lane >> 4;
#pragma unroll
    for (int kq = 0; kq < BK; kq += 16) {
        floatx4 af[F], bf[F];   // af[a][s], bf[b][s]
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const int k = kq + 4 * s + g;
            if (WIDE) {
                const vecf ta = *reinterpret_cast<const vecf*>(&As[k * PKM + wi + F * m]);
                const vecf tb = *reinterpret_cast<const vecf*>(&Bs[k * PKM + wj + F * m]);
#pragma unroll
                for (int x = 0; x < F; ++x) {
                    af[x][s] = ta[x];
                    bf[x][s] = tb[x];
                }
            } else {
#pragma unroll
                for (int x = 0; x < F; ++x) {
                    af[x][s] = As[lds_at<AR, T>(wi + 16 * x + m, k)];
                    bf[x][s] = Bs[lds_at<BR, T>(wj + 16 * x + m, k)];
                }
            }
        }
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int a = 0; a < F; ++a)
#pragma unroll
                for (int b = 0; b < F; ++b)
                    acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[a][s], bf[b][s], acc[a][b], 0, 0, 0);
    }
}

template <int TA, int TB, bool CHECK, int T, int CHUNK>
__device__ __forceinline__ void main_loop(const GemmArgs& g, const float* A, const float* B, const TileRange& tr,
                                          float* lds, floatx4 (&acc)[Geo<T>::F][Geo<T>::F],
                                          floatx4 (&run)[Geo<T>::F][Geo<T>::F]) {
    constexpr int F = Geo<T>::F;
    constexpr bool AR = TA == 0, BR = TB == 1;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wi = (wave >> 1) * Geo<T>::WS, wj = (wave & 1) * Geo<T>::WS;
    OperandLoader<AR, T> la;
    OperandLoader<BR, T> lb;
    la.init(A, g.lda, tr.i0, tr.klo);
    lb.init(B, g.ldb, tr.j0, tr.klo);
    Quad va, vb;
    float* As = lds;
    float* Bs = lds + Geo<T>::TILE_F;
#define ICQ_LOAD_STAGE(K0)                                                 \
    do {                                                                   \
        if (CHECK) {                                                       \
            la.load_checked(va, tr.i0, (K0), g.M, tr.khi, g.lda, A);       \
            lb.load_checked(vb, tr.j0, (K0), g.N, tr.khi, g.ldb, B);       \
        } else {                                                           \
            la.load_fast(va);                                              \
            lb.load_fast(vb);                                              \
        }                                                                  \
        la.p += la.step;                                                   \
        lb.p += lb.step;                                                   \
    } while (0)
    int64_t k0 = tr.klo;
    if (k0 >= tr.khi) return;
    ICQ_LOAD_STAGE(k0);
    for (; k0 < tr.khi; k0 += BK) {
        __syncthreads();                       // previous stage's LDS reads are done
        la.store_lds(va, As);
        lb.store_lds(vb, Bs);
        __syncthreads();
        if (k0 + BK < tr.khi) ICQ_LOAD_STAGE(k0 + BK);
        mma_stage<TA, TB, T>(As, Bs, wi, wj, lane, acc);
        if ((((k0 + BK) & (g.kc - 1)) == 0) || k0 + BK >= tr.khi) {
            // end of a chunk (or of the K range): fold it into the running result
#pragma unroll
            for (int a = 0; a < F; ++a)
#pragma unroll
                for (int b = 0; b < F; ++b) {
                    run[a][b] = CHUNK == CHUNK_SUB ? run[a][b] - acc[a][b] : run[a][b] + acc[a][b];
                    acc[a][b] = floatx4{0.f, 0.f, 0.f, 0.f};
                }
        }
    }
#undef ICQ_LOAD_STAGE
}

// One output tile `tr` of batch entry z, by the work-group's first four
// waves (threads 0..255); lds: 2 * Geo<T>::TILE_F floats of LDS.
template <int TA, int TB, bool CHECK, int T, int CHUNK>
__device__ __forceinline__ void gemm_tile(const GemmArgs& g, const TileRange& tr, int64_t z, float* lds) {
    constexpr int F = Geo<T>::F;
    const float* A = g.A + z * g.sA;
    const float* B = g.B + z * g.sB;
    float* C = g.C + z * g.sC;

    constexpr bool WIDE = TA == 1 && TB == 0;
    typedef typename VecF<F>::type vecf;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wi = (wave >> 1) * Geo<T>::WS, wj = (wave & 1) * Geo<T>::WS;
    const int g4 = 4 * (lane >> 4), m = lane & 15;
    // element (a, b, v) of the accumulators is C[row(a, v)][col(b)] (see mma_stage)
    auto row_of = [&](int a, int v) -> int64_t { return tr.i0 + (WIDE ? wi + F * (g4 + v) + a : wi + 16 * a + g4 + v); };
    auto col_of = [&](int b) -> int64_t { return tr.j0 + (WIDE ? wj + F * m + b : wj + 16 * b + m); };
    const bool full = !CHECK && g.cmask == CMASK_FULL;

    floatx4 acc[F][F], run[F][F];
    // the C tile's addresses for the loads before the K loop come from a copy
    // of the base pointer the compiler cannot identify with C, so that they are
    // recomputed for the stores instead of being held through the loop
    const float* Cl = g.Cin ? g.Cin + z * g.sC : C;
    if (CHUNK == CHUNK_SUB) asm volatile("" : "+s"(Cl));
#pragma unroll
    for (int a = 0; a < F; ++a)
#pragma unroll
        for (int b = 0; b < F; ++b) {
            acc[a][b] = floatx4{0.f, 0.f, 0.f, 0.f};
            if (CHUNK == CHUNK_SUB) {
                // the running result starts as C (elements past the matrix: 0, never stored)
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int64_t i = row_of(a, v), j = col_of(b);
                    run[a][b][v] = (full || (i < g.M && j < g.N)) ? Cl[i * g.ldc + j] : 0.0f;
                }
            } else {
                run[a][b] = floatx4{0.f, 0.f, 0.f, 0.f};
            }
        }

    main_loop<TA, TB, CHECK, T, CHUNK>(g, A, B, tr, lds, acc, run);
    // the epilogue below stores alpha * acc + beta * C
    const float alpha = CHUNK == CHUNK_SUB ? 1.0f : g.alpha;
    const float beta = CHUNK == CHUNK_SUB ? 0.0f : g.beta;
#pragma unroll
    for (int a = 0; a < F; ++a)
#pragma unroll
        for (int b = 0; b < F; ++b) acc[a][b] = run[a][b];
    const float* Cr = g.Cin ? g.Cin + z * g.sC : C;   // the old C of the epilogue
    const bool cvec = (((uintptr_t)C) % (4 * F) == 0) && (((uintptr_t)Cr) % (4 * F) == 0) && (g.ldc % F == 0);
    if (WIDE && full && cvec) {
        // the lane's F columns F m .. F m + F - 1 are adjacent: F-wide loads and stores
        const int64_t j0 = col_of(0);
        vecf cold[F][4];
        if (beta != 0.0f) {
#pragma unroll
            for (int a = 0; a < F; ++a)
#pragma unroll
                for (int v = 0; v < 4; ++v)
                    cold[a][v] = *reinterpret_cast<const vecf*>(&Cr[row_of(a, v) * g.ldc + j0]);
        }
#pragma unroll
        for (int a = 0; a < F; ++a)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                vecf r;
#pragma unroll
                for (int b = 0; b < F; ++b) {
                    r[b] = alpha * acc[a][b][v];
                    if (beta != 0.0f) r[b] = r[b] + beta * cold[a][v][b];
                }
                *reinterpret_cast<vecf*>(&C[row_of(a, v) * g.ldc + j0]) = r;
            }
        return;
    }
    // general epilogue: all C loads are issued before any store so their latency overlaps
    float cold[F][F][4];
    if (beta != 0.0f) {
#pragma unroll
        for (int a = 0; a < F; ++a)
#pragma unroll
            for (int b = 0; b < F; ++b)
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int64_t i = row_of(a, v), j = col_of(b);
                    cold[a][b][v] = (full || (i < g.M && j < g.N)) ? Cr[i * g.ldc + j] : 0.0f;
                }
    }
#pragma unroll
    for (int a = 0; a < F; ++a)
#pragma unroll
        for (int b = 0; b < F; ++b)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int64_t i = row_of(a, v), j = col_of(b);
                if (!full) {
                    if (i >= g.M || j >= g.N) continue;
                    if (g.cmask == CMASK_LOWER && i < j) continue;
                    if (g.cmask == CMASK_UPPER && i > j) continue;
                }
                float r = alpha * acc[a][b][v];
                if (beta != 0.0f) r = r + beta * cold[a][b][v];
                C[i * g.ldc + j] = r;
            }
}

// Tiles of size T for a launch (triangular grids count only the kept triangle).
template <int T>
inline int64_t tile_count(const GemmArgs& g, bool& tri) {
    const int64_t tm = cdiv(g.M, T), tn = cdiv(g.N, T);
    tri = (g.cmask == CMASK_LOWER || g.cmask == CMASK_UPPER) && tm == tn;
    return tri ? tm * (tm + 1) / 2 : tm * tn;
}

}  // namespace gk
}  // namespace icq
