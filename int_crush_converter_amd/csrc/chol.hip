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
//  3. trtri:  X = L^-1: diagonal blocks Dinv_k, then adjacent diagonal
//             inverses merged level by level, X21 = -X22 (L21 X11)  (GEMMs)
//  4. lauum:  H^-1 (upper triangle) = X^T X, one GEMM whose tile (I, J)
//             only runs k >= max(I, J) because X is lower triangular.
// Flops: n^3/3 each for 2-4; all but the nb x nb factorisations are MFMA.
#include <utility>
#include <vector>

#include "chol.hpp"
#include "gemm_dev.hpp"
#include "torchsum.hpp"

namespace icq {

constexpr int NB = 128;

static double dtri(double n) { return n * (n + 1) / 2; }

// One work-group of 256 per matrix: H += damping * max(mean(diag H), 1e-6) * I
// with the mean computed as the reference computes H.diagonal().mean() on
// the CPU (converter/gptq.py:104, 118; ldlq.py:83, 169, 207): torch's fp32
// scalar row_sum of the strided diagonal, then one IEEE division by n.  (At
// n >= 32768 torch splits a full reduction over its CPU threads, so this is
// its one-thread order there.)  The diagonal is staged in LDS first, so
// every load is in flight at once.
constexpr int DAMP_LDS = 16384;
__global__ __launch_bounds__(256) void damp_kernel(float* H, int64_t n, int64_t ld, int64_t stride, float damping) {
    float* A = H + (int64_t)blockIdx.x * stride;
    __shared__ float dg[DAMP_LDS];
    __shared__ float blk[RS_MAX_BLOCKS];
    __shared__ float part[4];
    const bool staged = n <= DAMP_LDS;
    if (staged) {
        for (int64_t i0 = threadIdx.x; i0 < n; i0 += 8 * (int64_t)blockDim.x) {
            float v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int64_t i = i0 + u * (int64_t)blockDim.x;
                v[u] = i < n ? A[i * ld + i] : 0.0f;
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int64_t i = i0 + u * (int64_t)blockDim.x;
                if (i < n) dg[i] = v[u];
            }
        }
    }
    __syncthreads();
    const float sum = row_sum_wg([&](int64_t i) { return staged ? dg[i] : A[i * ld + i]; }, n, blk, part);
    float mean = sum / (float)n;
    mean = mean > 1e-6f ? mean : (mean != mean ? mean : 1e-6f);
    const float delta = damping * mean;
    if (staged) {
        // the diagonal is in LDS: stores only, none waits for a load
        for (int64_t i = threadIdx.x; i < n; i += blockDim.x) A[i * ld + i] = dg[i] + delta;
        return;
    }
    for (int64_t i0 = threadIdx.x; i0 < n; i0 += 8 * (int64_t)blockDim.x) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int64_t i = i0 + u * (int64_t)blockDim.x;
            v[u] = i < n ? A[i * ld + i] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int64_t i = i0 + u * (int64_t)blockDim.x;
            if (i < n) A[i * ld + i] = v[u] + delta;
        }
    }
}

// Factor the diagonal block [k0, k0+nb) of matrix blockIdx.x in place (lower,
// upper part of the block set to 0) and write Dinv = L_kk^-1 (lower, upper 0)
// to dinv64 (fp64, pitch NB).  info[b] gets the
// 1-based column of the first non-positive pivot (LAPACK convention) if it
// is still 0.  A partial block (nb < 128) is padded with the identity.
//
// The arithmetic is fp64 (inputs and outputs fp32 / fp64): the diagonal
// blocks and their inverses feed every later step, and an fp64 factor keeps
// the whole inverse at the accuracy of the reference's LAPACK fp32 path.
//
// The block is processed in 16 panels of 8 columns by 8 waves.  Both the
// block A and R (X = L^-1 under construction, started as I) live in MFMA
// accumulators: the 36 lower 16x16 tiles of each are dealt to waves 1..7
// round-robin in column-major order (so one tile column spreads over
// several waves).  Wave 0 owns no tile: it runs the serial part, the
// column-by-column factorisation of each panel and the forward substitution
// for the rows of X, while the other waves apply the rank-8 updates on the
// matrix cores (v_mfma_f64_16x16x4_f64).  Look-ahead keeps the factorisation
// off the MFMA path; iteration it has two phases:
//   U: wave 0 factors panel it (from the published tile column, two rows
//      per lane, pivots and the panel's rows broadcast by readlane); the
//      others apply panel it - 1's update A -= L L^T to every live tile
//      outside the next tile column (which got it in phase A of it - 1) and
//      panel it - 2's update R -= L X to R, then publish rows of R of panel
//      it - 1 (now final up to their own diagonal block);
//   A: the owners of the tile column holding panel it + 1 apply panel it's
//      update to it and publish it for wave 0; waves 0 and 1 turn the
//      published rows of R into the rows of X of panel it - 1 (forward
//      substitution with that panel's 8x8 diagonal block, a column per
//      lane) and store them to Dinv / Dinv64 (whole rows: coalesced).
// Every element receives its updates in panel order with the same fp64
// operations, so the result does not depend on the schedule.  Elements that
// are already final (or above the diagonal) may receive updates; they are
// never read again.  At the end the block writes the image of L row by row.
//
// MFMA 16x16x4 f64 operand layout (lane l of 64; D differs from the f32
// variant's 4*(l/16) + v):
//   A: A[i = l%16][k = l/16]      B: B[k = l/16][j = l%16]
//   D (4 doubles v): D[i = l/16 + 4*v][j = l%16]
typedef double ddoublex4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ double rdlane(double v, int l) {
    const int64_t b = __double_as_longlong(v);
    const int lo = __builtin_amdgcn_readlane((int)(b & 0xffffffff), l);
    const int hi = __builtin_amdgcn_readlane((int)(b >> 32), l);
    return __longlong_as_double(((int64_t)hi << 32) | (uint32_t)lo);
}

constexpr int DIAG_WAVES = 8;            // wave 0: factorisation; 1..7: tiles
constexpr int DIAG_TILES = 36;           // lower 16x16 tiles of the 8x8 tile grid
constexpr int DSLOTS = 6;                // tiles per MFMA wave (at most)

// Lower tile `id` in column-major order over the lower triangle: tile column
// and tile row.  Wave W (1..7) owns the tiles id = W - 1 + 7 s.
constexpr int cm_col(int id) {
    int J = 0;
    while (id >= 8 - J) { id -= 8 - J; ++J; }
    return J;
}
constexpr int cm_row(int id) {
    int J = 0;
    while (id >= 8 - J) { id -= 8 - J; ++J; }
    return J + id;
}
constexpr int tile_id(int W, int s) { return W - 1 + 7 * s; }

// Slot S of wave W as compile-time constants, and a loop over a wave's
// slots that hands each one to f as a type (so every tile coordinate is a
// constant and the accumulators are indexed statically).
template <int W, int S>
struct DiagSlot {
    static constexpr int s = S;
    static constexpr bool ok = tile_id(W, S) < DIAG_TILES;
    static constexpr int I = ok ? cm_row(tile_id(W, S)) : 0;
    static constexpr int J = ok ? cm_col(tile_id(W, S)) : 0;
};
template <int W, typename F, int... S>
__device__ __forceinline__ void each_slot_impl(F&& f, std::integer_sequence<int, S...>) {
    (f(DiagSlot<W, S>{}), ...);
}
template <int W, typename F>
__device__ __forceinline__ void each_slot(F&& f) {
    each_slot_impl<W>(f, std::make_integer_sequence<int, DSLOTS>{});
}

// Panel-local k (0..7) is stored at kperm(k), so that the two k values a
// lane feeds to the two MFMA steps of a panel, lr and lr + 4, are adjacent.
__device__ __forceinline__ constexpr int kperm(int k) { return (k & 3) * 2 + (k >> 2); }

// Rows of 8 doubles are padded to DP = 9, so that a wave's 64 row-wise
// accesses spread over the LDS banks (a 64-byte pitch would put them on 4).
// Arrays indexed by a row of the block have a spare row NB, where accesses
// for rows past the block are clamped (so they need no branch).
constexpr int DP = 9, RP = 17;
constexpr int PLBUF = 3;   // L panels in use: it (phase A), it - 1 (A update), it - 2 (R update)

struct DiagShared {
    double pRaw[NB + 1][RP];       // the tile column of A holding the next panel (row NB stays 0)
    double pL[PLBUF][NB + 1][DP];  // final L columns of the last three panels, at kperm
    double dL[2][8][8];            // the 8x8 diagonal blocks of L of the last two panels
    double rinv[2][8];             // and their pivots' reciprocal square roots
    double rowR[8][NB];            // rows of R of the panel whose X rows are due
    double rowXt[NB][DP];          // final rows of X = L^-1 of that panel, transposed, at kperm
    float Lfin[NB + 1][NB + 1];    // L as it is finalised (on and below the diagonal)
};

// The phases of the diagonal-block kernel hand data to each other only
// through LDS, so they are separated by lds_barrier() (common.hpp), which
// does not wait for the global stores of the Dinv rows.

// Rows 8 p .. 8 p + 7 of X = L^-1, column q: forward substitution with panel
// p's 8x8 diagonal block of L from the published rows of R; the result goes
// to rowXt (for the R updates) and to Dinv64 (whole rows: coalesced over the
// lanes).  Phase A splits the columns over waves 0 and 1.
__device__ __forceinline__ void x_rows(DiagShared& sh, int p, int q, int nb, double* D64) {
    const int x0 = p * 8, xb = p & 1;
    double x[8], l[8][8], ri[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        x[c] = sh.rowR[c][q];
        ri[c] = sh.rinv[xb][c];
#pragma unroll
        for (int c2 = 0; c2 < c; ++c2) l[c][c2] = sh.dL[xb][c][c2];
    }
#pragma unroll
    for (int c = 0; c < 8; ++c) {
#pragma unroll
        for (int c2 = 0; c2 < c; ++c2) x[c] = fma(-l[c][c2], x[c2], x[c]);
        x[c] = q <= x0 + 7 ? x[c] * ri[c] : 0.0;
    }
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        sh.rowXt[q][kperm(c)] = x[c];
        const int row = x0 + c;
        D64[row * NB + q] = (row < nb && q < nb) ? x[c] : 0.0;
    }
}

// Panel it (columns j0 .. j0 + 7, rows j0 .. 127) on wave 0, two rows per
// lane: rows j0 + lane and (TWO: it < 8) j0 + 64 + lane.  From it = 8 on
// the second set lies past the block and is skipped.  Pivots and the
// panel's rows are broadcast by readlane.
template <bool TWO>
__device__ __forceinline__ void factor_panel(DiagShared& sh, int it, int lane, int& bad) {
    const int j0 = it * 8, co = (it & 1) * 8, pb = it % PLBUF, db = it & 1;
    // rows past the block read the zero row NB
    const int ra = j0 + lane, rb = j0 + lane + 64;
    const int rac = ra < NB ? ra : NB, rbc = rb < NB ? rb : NB;
    double va[8], vb[8], rinvv[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        va[c] = sh.pRaw[rac][co + c];
        vb[c] = TWO ? sh.pRaw[rbc][co + c] : 0.0;
    }
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        double d = rdlane(va[c], c);
        if (!(d > 0.0)) {
            if (!bad) bad = j0 + c + 1;
            d = 1.0;
        }
        // 1/sqrt(d) from the hardware estimate and two Newton steps
        // (relative error far below fp32's), then sqrt(d) = d / sqrt(d)
        double rinv = __builtin_amdgcn_rsq(d);
        rinv = rinv * fma(-0.5 * d * rinv, rinv, 1.5);
        rinv = rinv * fma(-0.5 * d * rinv, rinv, 1.5);
        const double ljj = d * rinv;
        va[c] = lane > c ? va[c] * rinv : (lane == c ? ljj : 0.0);
        if (TWO) vb[c] = vb[c] * rinv;
        rinvv[c] = rinv;
#pragma unroll
        for (int c2 = c + 1; c2 < 8; ++c2) {
            const double lk = rdlane(va[c], c2);
            va[c2] = fma(-va[c], lk, va[c2]);
            if (TWO) vb[c2] = fma(-vb[c], lk, vb[c2]);
        }
    }
    // the panel's L columns (fp64 MFMA operands), its 8x8 diagonal block and
    // pivots for the rows of X, and the fp32 image of L (rows past the block
    // go to the spare row NB).  Rows of pL above the panel keep older values:
    // they only reach elements that are final already, which are never read
    // again.
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        sh.pL[pb][rac][kperm(c)] = va[c];
        sh.Lfin[rac][j0 + c] = (float)va[c];
        if (TWO) {
            sh.pL[pb][rbc][kperm(c)] = vb[c];
            sh.Lfin[rbc][j0 + c] = (float)vb[c];
        }
    }
    if (lane < 8) {
#pragma unroll
        for (int c = 0; c < 8; ++c) sh.dL[db][lane][c] = va[c];
    }
    if (lane == 0) {
#pragma unroll
        for (int c = 0; c < 8; ++c) sh.rinv[db][c] = rinvv[c];
    }
}

// Wave 0: phase U factors panel it, phase A finishes columns 0..63 of the
// rows of X of panel it - 1.  Two barriers per iteration, matching
// diag_tile_wave.
__device__ __forceinline__ void diag_factor_wave(DiagShared& sh, int nb, double* D64, int lane, int& bad) {
    for (int it = 0; it <= 16; ++it) {
        if (it < 8) factor_panel<true>(sh, it, lane, bad);
        else if (it < 16) factor_panel<false>(sh, it, lane, bad);
        lds_barrier();
        if (it >= 1) x_rows(sh, it - 1, lane, nb, D64);
        lds_barrier();
    }
}

// Operands of a rank-8 update from an L panel (or the X rows) in LDS:
// op[r][ks] = P[16 r + lj][2 lr + ks] (panel columns 4 ks + lr, at kperm).
__device__ __forceinline__ void load_op(const double (*P)[DP], int r, int lr, int lj, double (&op)[2]) {
    op[0] = P[r * 16 + lj][2 * lr];
    op[1] = P[r * 16 + lj][2 * lr + 1];
}

// Waves 1..7: the tiles of A and R.  Every tile coordinate is a compile-time
// constant, so accumulators are indexed statically.
template <int W>
__device__ __forceinline__ void diag_tile_wave(DiagShared& sh, const float* A, int64_t ld, int nb, double* D64,
                                               int lane) {
    const int lr = lane >> 4, lj = lane & 15;   // accumulator v holds row lr + 4 v, column lj
    ddoublex4 accA[DSLOTS], accX[DSLOTS];
    // all loads in flight at once: addresses are clamped into the block (no
    // branch) and values outside it replaced
    float raw[DSLOTS][4];
    each_slot<W>([&](auto t) {
        using T = decltype(t);
        if constexpr (T::ok) {
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int i = T::I * 16 + lr + 4 * v, j = T::J * 16 + lj;
                const int ic = i < nb ? i : nb - 1, jc = j < nb ? j : nb - 1;
                raw[T::s][v] = A[(int64_t)ic * ld + jc];
            }
        }
    });
    each_slot<W>([&](auto t) {
        using T = decltype(t);
        if constexpr (T::ok) {
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int i = T::I * 16 + lr + 4 * v, j = T::J * 16 + lj;
                const double pad = (i == j) ? 1.0 : 0.0;
                accA[T::s][v] = j > i ? 0.0 : (i < nb ? (double)raw[T::s][v] : pad);
                accX[T::s][v] = pad;
            }
        }
    });
    // tile column 0 for panel 0
    each_slot<W>([&](auto t) {
        using T = decltype(t);
        if constexpr (T::ok && T::J == 0) {
#pragma unroll
            for (int v = 0; v < 4; ++v) sh.pRaw[T::I * 16 + lr + 4 * v][lj] = accA[T::s][v];
        }
    });
    __syncthreads();
    for (int it = 0; it <= 16; ++it) {
        // ---- phase U
        if (it >= 1) {
            // panel p = it - 1: A -= L_p L_p^T on live tiles outside tile
            // column it >> 1 (updated in phase A of iteration p)
            const int p = it - 1, skipJ = it >> 1, lim = 8 * p + 8;
            const double (*P)[DP] = sh.pL[p % PLBUF];
            double op[8][2];
#pragma unroll
            for (int r = 0; r < 8; ++r) load_op(P, r, lr, lj, op[r]);
            each_slot<W>([&](auto t) {
                using T = decltype(t);
                if constexpr (T::ok) {
                    if (T::J != skipJ && T::J * 16 + 15 >= lim) {
#pragma unroll
                        for (int ks = 0; ks < 2; ++ks)
                            accA[T::s] = __builtin_amdgcn_mfma_f64_16x16x4f64(-op[T::I][ks], op[T::J][ks], accA[T::s],
                                                                              0, 0, 0);
                    }
                }
            });
        }
        if (it >= 2) {
            // panel q = it - 2: R -= L_q X_q for rows below the panel and
            // columns up to its end
            const int q = it - 2, x0 = 8 * q;
            const double (*P)[DP] = sh.pL[q % PLBUF];
            double opM[8][2], opX[8][2];
#pragma unroll
            for (int r = 0; r < 8; ++r) {
                load_op(P, r, lr, lj, opM[r]);
                load_op(sh.rowXt, r, lr, lj, opX[r]);
            }
            each_slot<W>([&](auto t) {
                using T = decltype(t);
                if constexpr (T::ok) {
                    if (T::I * 16 + 15 >= x0 + 8 && T::J * 16 <= x0 + 7) {
#pragma unroll
                        for (int ks = 0; ks < 2; ++ks)
                            accX[T::s] = __builtin_amdgcn_mfma_f64_16x16x4f64(-opM[T::I][ks], opX[T::J][ks],
                                                                              accX[T::s], 0, 0, 0);
                    }
                }
            });
        }
        if (it >= 1) {
            // rows x0..x0+7 of R (panel it - 1) for wave 0's substitution
            const int Jx = (it - 1) >> 1, cx = ((it - 1) & 1) * 8;
            each_slot<W>([&](auto t) {
                using T = decltype(t);
                if constexpr (T::ok) {
                    if (T::I == Jx) {
                        if (cx == 0) {
                            sh.rowR[lr][T::J * 16 + lj] = accX[T::s][0];
                            sh.rowR[lr + 4][T::J * 16 + lj] = accX[T::s][1];
                        } else {
                            sh.rowR[lr][T::J * 16 + lj] = accX[T::s][2];
                            sh.rowR[lr + 4][T::J * 16 + lj] = accX[T::s][3];
                        }
                    }
                }
            });
        }
        lds_barrier();
        // ---- phase A: panel it's update of the tile column holding panel it + 1, published
        if (it <= 14) {
            const int Jn = (it + 1) >> 1;
            const double (*P)[DP] = sh.pL[it % PLBUF];
            double opn[2];
            load_op(P, Jn, lr, lj, opn);
            each_slot<W>([&](auto t) {
                using T = decltype(t);
                if constexpr (T::ok) {
                    if (T::J == Jn) {
                        double opi[2];
                        load_op(P, T::I, lr, lj, opi);
#pragma unroll
                        for (int ks = 0; ks < 2; ++ks)
                            accA[T::s] = __builtin_amdgcn_mfma_f64_16x16x4f64(-opi[ks], opn[ks], accA[T::s], 0, 0, 0);
#pragma unroll
                        for (int v = 0; v < 4; ++v) sh.pRaw[T::I * 16 + lr + 4 * v][lj] = accA[T::s][v];
                    }
                }
            });
        }
        // columns 64..127 of the rows of X of panel it - 1 (wave 0 does 0..63)
        if (W == 1 && it >= 1) x_rows(sh, it - 1, 64 + lane, nb, D64);
        lds_barrier();
    }
}

// The diagonal block of matrix b, by a work-group of DIAG_WAVES waves.
__device__ __forceinline__ void diag_block(DiagShared& sh, int b, float* H, int64_t ld, int64_t stride, int64_t k0,
                                           int nb, double* dinv64, int64_t dstride, int* info) {
    float* A = H + (int64_t)b * stride + k0 * ld + k0;
    double* D64 = dinv64 + (int64_t)b * dstride;
    const int lane = threadIdx.x & 63;
    // uniform in the wave; every wave runs 1 + 2 * 17 barriers
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // the spare row of pRaw starts at 0; the first barrier orders this
    if (threadIdx.x < RP) sh.pRaw[NB][threadIdx.x] = 0.0;
    int bad = 0;
    switch (wave) {
        case 0: __syncthreads(); diag_factor_wave(sh, nb, D64, lane, bad); break;
        case 1: diag_tile_wave<1>(sh, A, ld, nb, D64, lane); break;
        case 2: diag_tile_wave<2>(sh, A, ld, nb, D64, lane); break;
        case 3: diag_tile_wave<3>(sh, A, ld, nb, D64, lane); break;
        case 4: diag_tile_wave<4>(sh, A, ld, nb, D64, lane); break;
        case 5: diag_tile_wave<5>(sh, A, ld, nb, D64, lane); break;
        case 6: diag_tile_wave<6>(sh, A, ld, nb, D64, lane); break;
        default: diag_tile_wave<7>(sh, A, ld, nb, D64, lane); break;
    }
    __syncthreads();
    // write L, row-coalesced: Lfin holds every element on and below the
    // diagonal (panel p writes rows 8 p .. 127 of its columns); the upper
    // triangle is 0.  Eight LDS reads in flight per batch of stores.
    constexpr int PER_THREAD = NB * NB / (DIAG_WAVES * 64);
#pragma unroll 8
    for (int u = 0; u < PER_THREAD; ++u) {
        const int idx = (int)threadIdx.x + u * DIAG_WAVES * 64, i = idx >> 7, j = idx & (NB - 1);
        const float v = j <= i ? sh.Lfin[i][j] : 0.0f;
        if (i < nb && j < nb) A[(int64_t)i * ld + j] = v;
    }
    if (threadIdx.x == 0 && bad && info[b] == 0) info[b] = (int)k0 + bad;
}

__global__ __launch_bounds__(DIAG_WAVES * 64) void potrf_diag_kernel(float* H, int64_t ld, int64_t stride, int64_t k0,
                                                                    int nb, double* dinv64, int64_t dstride,
                                                                    int* info) {
    __shared__ __attribute__((aligned(16))) DiagShared sh;
    diag_block(sh, blockIdx.x, H, ld, stride, k0, nb, dinv64, dstride, info);
}

// The diagonal block of matrix blockIdx.z (work-group 0) beside the
// previous block's update of the rest of its super-block: work-group
// t >= 1 runs tile t - 1 (REST_T x REST_T) of the GEMM g (batch entry
// blockIdx.z) on its first four waves, in the LDS the diagonal block uses;
// the other waves end at once (a barrier waits only for the waves still
// running).  The two touch disjoint columns.  One launch instead of two,
// and the update runs while the diagonal block's serial chain does.  The
// launch holds one work-group per CU (the diagonal block's LDS), where
// 128-tiles (a quarter as many as 64-tiles) finish the update sooner.
constexpr int REST_T = 128;
static_assert(2 * gk::Geo<REST_T>::TILE_F * sizeof(float) <= sizeof(DiagShared), "GEMM tile staging fits");
__global__ __launch_bounds__(DIAG_WAVES * 64) void potrf_diag_rest_kernel(float* H, int64_t ld, int64_t stride,
                                                                         int64_t k0, int nb, double* dinv64,
                                                                         int64_t dstride, int* info, GemmArgs g) {
    __shared__ __attribute__((aligned(16))) DiagShared sh;
    if (blockIdx.x == 0) {
        diag_block(sh, blockIdx.z, H, ld, stride, k0, nb, dinv64, dstride, info);
        return;
    }
    if (threadIdx.x >= 256) return;
    const gk::TileRange tr = gk::tile_of<REST_T>(g, blockIdx.x - 1);
    if (tr.skip) return;
    gk::gemm_tile<0, 1, true, REST_T, gk::CHUNK_SUM>(g, tr, blockIdx.z, reinterpret_cast<float*>(&sh));
}

// Panel solve A21 <- A21 * Dinv^T for the m rows below a diagonal block, in
// place, with fp64 products and accumulation (fp32 in and out).  Multiplying
// by an explicit inverse is where a blocked fp32 Cholesky loses most
// accuracy; this step is ~1 % of the factorisation's flops, so it runs on
// the fp64 matrix cores (v_mfma_f64_16x16x4_f64).
// Work-group: 64 rows, wave w owning the 16-row strip 16 w .. 16 w + 15 as 8
// accumulator tiles of 16 columns.  k is staged 32 at a time; a column tile
// J only takes the k-steps with k <= 16 J + 15 (Dinv is lower triangular).
constexpr int PR = 64, PK = 32;
constexpr int PA = PK + 1;   // As pitch (floats)
constexpr int PD = PK + 2;   // Ds pitch (doubles)

__global__ __launch_bounds__(256) void panel64_kernel(float* A21, int64_t m, int nb, int64_t ld, int64_t stride,
                                                      const double* dinv64, int64_t dstride) {
    __shared__ float As[PR * PA];
    __shared__ double Ds[NB * PD];
    const int b = blockIdx.y;
    float* P = A21 + (int64_t)b * stride;
    const double* D64 = dinv64 + (int64_t)b * dstride;
    const int64_t r0 = (int64_t)blockIdx.x * PR;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int li = lane & 15, lk = lane >> 4;
    ddoublex4 acc[8];
#pragma unroll
    for (int J = 0; J < 8; ++J) acc[J] = ddoublex4{0.0, 0.0, 0.0, 0.0};
    // the next chunk's global loads are issued before the current chunk's
    // MFMAs, so that only the first chunk waits for memory
    constexpr int NA = PR * PK / 256, ND = NB * PK / 256;
    float av[NA];
    double dv[ND];
    auto load_chunk = [&](int kc) {
#pragma unroll
        for (int u = 0; u < NA; ++u) {
            const int idx = t + u * 256, r = idx / PK, k = idx % PK;
            const int64_t row = r0 + r;
            av[u] = (row < m && kc + k < nb) ? P[row * ld + kc + k] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < ND; ++u) {
            const int idx = t + u * 256, j = idx / PK, k = idx % PK;
            dv[u] = D64[j * NB + kc + k];
        }
    };
    load_chunk(0);
    for (int kc = 0; kc < nb; kc += PK) {
        __syncthreads();
#pragma unroll
        for (int u = 0; u < NA; ++u) {
            const int idx = t + u * 256;
            As[(idx / PK) * PA + idx % PK] = av[u];
        }
#pragma unroll
        for (int u = 0; u < ND; ++u) {
            const int idx = t + u * 256;
            Ds[(idx / PK) * PD + idx % PK] = dv[u];
        }
        __syncthreads();
        if (kc + PK < nb) load_chunk(kc + PK);
#pragma unroll
        for (int ks = 0; ks < PK / 4; ++ks) {
            const int k = ks * 4 + lk;
            const double a = (double)As[(wave * 16 + li) * PA + k];
#pragma unroll
            for (int J = 0; J < 8; ++J) {
                if (J * 16 + 15 < kc + ks * 4) continue;   // Dinv[j][k] = 0 for k > j
                const double bb = Ds[(J * 16 + li) * PD + k];
                acc[J] = __builtin_amdgcn_mfma_f64_16x16x4f64(a, bb, acc[J], 0, 0, 0);
            }
        }
    }
#pragma unroll
    for (int J = 0; J < 8; ++J)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int64_t row = r0 + wave * 16 + lk + 4 * v;
            const int col = J * 16 + li;
            if (row < m && col < nb) P[row * ld + col] = (float)acc[J][v];
        }
}

// Copy the upper triangle onto the lower one (in place), per matrix, in
// 32 x 32 tiles through LDS: both the upper source tile and the lower target
// tile are read and written along rows.  Grid (tiles, tiles, batch), block
// (32, 8); work-groups above the diagonal exit.
__global__ void mirror_upper_tiled_kernel(float* H, int64_t n, int64_t ld, int64_t stride) {
    const int ti = blockIdx.y, tj = blockIdx.x;   // target tile: rows ti, columns tj (ti >= tj)
    if (ti < tj) return;
    __shared__ float S[32][33];
    float* A = H + (int64_t)blockIdx.z * stride;
    const int tx = threadIdx.x, ty = threadIdx.y;
    for (int r = ty; r < 32; r += 8) {   // source: rows tj, columns ti (upper)
        const int64_t i = (int64_t)tj * 32 + r, j = (int64_t)ti * 32 + tx;
        if (i < n && j < n) S[r][tx] = A[i * ld + j];
    }
    __syncthreads();
    for (int r = ty; r < 32; r += 8) {
        const int64_t i = (int64_t)ti * 32 + r, j = (int64_t)tj * 32 + tx;
        if (i < n && j < n && i > j) A[i * ld + j] = S[tx][r];
    }
}

static int mirror_upper(float* H, int64_t batch, int64_t n, int64_t ld, int64_t stride, hipStream_t st) {
    IC_REQUIRE(batch <= 65535 && cdiv(n, 32) < 65536, "mirror_upper: too large");
    const dim3 tg((unsigned)cdiv(n, 32), (unsigned)cdiv(n, 32), (unsigned)batch);
    hipLaunchKernelGGL(mirror_upper_tiled_kernel, tg, dim3(32, 8), 0, st, H, n, ld, stride);
    IC_CHECK_LAUNCH();
    return IC_OK;
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

int64_t dinv_floats(int64_t batch, int64_t n) { return batch * cdiv(n, NB) * NB * NB; }

// fp64 copy of the Dinv blocks: after the fp32 ones, 256-byte aligned.
double* dinv64_of(float* dinv, int64_t batch, int64_t n) {
    const uintptr_t p = reinterpret_cast<uintptr_t>(dinv + dinv_floats(batch, n));
    return reinterpret_cast<double*>((p + 255) & ~(uintptr_t)255);
}

// Lower Cholesky in place of `batch` matrices [n, n] (pitch ld, stride sH);
// dinv64 receives every Dinv_k (batch x nblk x NB x NB, fp64).
//
// Two-level right-looking: columns are taken in super-blocks of up to
// SUPER_NB columns.  After each block's panel, only the rest of the
// super-block's columns are updated (rank-NB); after the super-block, the
// trailing matrix beyond it gets one SYRK with K = SUPER_NB.  Same flops as
// one SYRK per block, with the trailing matrix read and written once per
// super-block.
//
// Look-ahead inside a super-block: block k's update is split into the next
// block column (before the next diagonal block) and the rest of the
// super-block, which runs in the next diagonal block's launch
// (potrf_diag_rest_kernel).  The next block column's update follows that
// launch, so every element receives the same rank-NB updates in the same
// order as with one update per block (bit-identical results).
constexpr int64_t SUPER_NB = 1024;

int potrf(float* H, int64_t batch, int64_t n, int64_t ld, int64_t sH, double* dinv64, int* info, hipStream_t st) {
    const int64_t nblk = cdiv(n, NB);
    const int64_t dstride = nblk * NB * NB;
    IC_REQUIRE(batch <= 65535, "potrf: batch too large");
    bool rest_pending = false;   // `rest`: the previous block's update of the rest of its super-block
    GemmArgs rest{};
    int64_t rest_tiles = 0;
    for (int64_t s0 = 0; s0 < n; s0 += SUPER_NB) {
        const int64_t s1 = std::min<int64_t>(n, s0 + SUPER_NB);
        for (int64_t k0 = s0; k0 < s1; k0 += NB) {
            const int64_t kb = k0 / NB;
            const int nb = (int)std::min<int64_t>(NB, n - k0);
            double* Dk64 = dinv64 + kb * NB * NB;
            {
                double fl = batch * (2.0 / 3.0) * nb * nb * nb, by = batch * 3.0 * 4 * nb * nb;
                if (rest_pending) fl += rest.algo_flops, by += 4.0 * batch * (2.0 * rest.M * rest.K + 2.0 * rest.M * rest.N);
                ProfScope prof_scope(st, PT_DIAG, fl, by);
                if (rest_pending)
                    hipLaunchKernelGGL(potrf_diag_rest_kernel, dim3((unsigned)(1 + rest_tiles), 1, (unsigned)batch),
                                       dim3(DIAG_WAVES * 64), 0, st, H, ld, sH, k0, nb, Dk64, dstride, info, rest);
                else
                    hipLaunchKernelGGL(potrf_diag_kernel, dim3((unsigned)batch), dim3(DIAG_WAVES * 64), 0, st, H, ld,
                                       sH, k0, nb, Dk64, dstride, info);
                IC_CHECK_LAUNCH();
                rest_pending = false;
            }
            const int64_t k1 = k0 + nb;
            const int64_t m = n - k1;
            if (m <= 0) break;
            float* A21 = H + k1 * ld + k0;
            {
                // panel: A21 <- A21 * Dinv^T (fp64 accumulation, in place)
                ProfScope prof_scope(st, PT_PANEL, (double)batch * m * nb * (nb + 1), (double)batch * m * nb * 8.0);
                hipLaunchKernelGGL(panel64_kernel, dim3((unsigned)cdiv(m, PR), (unsigned)batch), dim3(256), 0, st,
                                   A21, m, nb, ld, sH, Dk64, dstride);
                IC_CHECK_LAUNCH();
            }
            // rest of the super-block: A[k1:, k1:s1] -= A21 A21[:s1-k1]^T (lower in its top square), the
            // next block column now, the others in the next diagonal block's launch
            const int64_t w = s1 - k1;
            if (w > 0) {
                const int64_t la = std::min<int64_t>(NB, w);
                GemmArgs g{m, la, nb, -1.0f, 1.0f, A21, ld, sH, A21, ld, sH, H + k1 * ld + k1, ld, sH, 0, 1,
                           CMASK_LOWER, KR_FULL, batch, PT_GEMM_CHOL,
                           (double)batch * 2.0 * (dtri((double)la) + (double)(m - la) * la) * nb};
                g.chunk_sub = 1;   // a sequence of rank-128 updates, like LAPACK's blocked potrf
                int rc = gemm_f32(g, st);
                if (rc) return rc;
                if (w > la) {
                    // one chunk (K = nb <= kc): C - P in the sum form, as gemm_f32 runs it
                    const float* A2 = A21 + la * ld;
                    rest = GemmArgs{m - la, w - la, nb, -1.0f, 1.0f, A2, ld, sH, A2, ld, sH,
                                    H + (k1 + la) * ld + k1 + la, ld, sH, 0, 1, CMASK_LOWER, KR_FULL, batch,
                                    PT_GEMM_CHOL,
                                    (double)batch * 2.0 * (dtri((double)(w - la)) + (double)(m - w) * (w - la)) * nb};
                    bool tri;
                    rest_tiles = gk::tile_count<REST_T>(rest, tri);
                    IC_REQUIRE(rest_tiles < (1LL << 30), "potrf: problem too large");
                    rest_pending = true;
                }
            }
        }
        // beyond the super-block: A[s1:, s1:] -= L[s1:, s0:s1] L[s1:, s0:s1]^T (lower)
        const int64_t m = n - s1;
        if (m > 0) {
            const float* P = H + s1 * ld + s0;
            const int64_t k = s1 - s0;
            GemmArgs g{m, m, k, -1.0f, 1.0f, P, ld, sH, P, ld, sH, H + s1 * ld + s1, ld, sH, 0, 1, CMASK_LOWER,
                       KR_FULL, batch, PT_GEMM_CHOL, (double)batch * 2.0 * dtri((double)m) * k};
            g.chunk_sub = 1;
            int rc = gemm_f32(g, st);
            if (rc) return rc;
        }
    }
    return IC_OK;
}

// X = L^-1 (lower triangle and the 128x128 diagonal blocks exact; the rest
// of the upper triangle is scratch) from L (lower, in H) and the Dinv
// blocks.  The diagonal blocks of X are the Dinv_k; then adjacent diagonal
// inverses are merged level by level,
//     [L11 0; L21 L22]^-1 = [X11 0; X21 X22],   X21 = -X22 (L21 X11),
// with T (or T^T when the halves differ in size) parked in the unused
// upper block of the merged square.  All pairs of one level that have the same shape run as one
// batched GEMM, so the whole inverse takes ~2 log2(n/128) launches of
// large-K GEMMs instead of 2 n/128 rank-128 updates.
__global__ void put_diag_all_kernel(float* X, int64_t n, int64_t ld, int64_t stride, const double* dinv64,
                                    int64_t dstride) {
    const int64_t k0 = (int64_t)blockIdx.x * NB;
    const int b = blockIdx.y;
    const double* D = dinv64 + (int64_t)b * dstride + (int64_t)blockIdx.x * NB * NB;
    float* P = X + (int64_t)b * stride + k0 * ld + k0;
    const int nb = (int)std::min<int64_t>(NB, n - k0);
    if (nb == NB && ld % 4 == 0 && (reinterpret_cast<uintptr_t>(P) & 15) == 0) {
        // whole block, 16-byte rows: 32 float4 per row, each from 4 doubles
        for (int idx = threadIdx.x; idx < NB * NB / 4; idx += blockDim.x) {
            const int i = idx >> 5, j4 = (idx & 31) * 4;
            const double2 a = *reinterpret_cast<const double2*>(&D[i * NB + j4]);
            const double2 c = *reinterpret_cast<const double2*>(&D[i * NB + j4 + 2]);
            *reinterpret_cast<float4*>(&P[(int64_t)i * ld + j4]) =
                make_float4((float)a.x, (float)a.y, (float)c.x, (float)c.y);
        }
        return;
    }
    for (int idx = threadIdx.x; idx < nb * nb; idx += blockDim.x) {
        const int i = idx / nb, j = idx - i * nb;
        P[(int64_t)i * ld + j] = (float)D[i * NB + j];
    }
}

static int merge_pairs(const float* L, float* X, int64_t ld, int64_t r0, int64_t n1, int64_t n2, int64_t count,
                       int64_t pstride, int64_t batch, int64_t sH, hipStream_t st) {
    // per (pair, matrix): strides differ only when both are > 1; then loop over matrices
    const bool pairs_batched = count > 1;
    const int64_t gb = pairs_batched ? count : batch;
    const int64_t gs = pairs_batched ? pstride : sH;
    const int64_t outer = pairs_batched ? batch : 1;
    for (int64_t m = 0; m < outer; ++m) {
        const int64_t off = pairs_batched ? m * sH : 0;
        const float* X11 = X + off + r0 * ld + r0;
        const float* L21 = L + off + (r0 + n1) * ld + r0;
        const float* X22 = X + off + (r0 + n1) * ld + (r0 + n1);
        float* X21 = X + off + (r0 + n1) * ld + r0;
        int rc;
        if (n2 <= n1 && n2 % NB == 0) {
            // T = L21 X11 (n2 x n1) in the upper triangle of the merged square:
            // rows r0 .. r0+n2, columns r0+n2 .. r0+n2+n1 (strictly above the
            // diagonal blocks, since n2 is a whole number of blocks; X11 is
            // read only on and below its diagonal blocks)
            float* T = X + off + r0 * ld + (r0 + n2);
            GemmArgs t{n2, n1, n1, 1.0f, 0.0f, L21, ld, gs, X11, ld, gs, T, ld, gs, 0, 0, CMASK_FULL, KR_FROM_J, gb,
                       PT_GEMM_INV, (double)gb * n2 * n1 * (n1 + 1)};
            if ((rc = gemm_f32(t, st))) return rc;
            // X21 = -X22 T; k <= i (X22 lower)
            GemmArgs x{n2, n1, n2, -1.0f, 0.0f, X22, ld, gs, T, ld, gs, X21, ld, gs, 0, 0, CMASK_FULL, KR_TO_I, gb,
                       PT_GEMM_INV, (double)gb * n1 * n2 * (n2 + 1)};
            if ((rc = gemm_f32(x, st))) return rc;
        } else {
            // T^T[a][b] = sum_k X11[k][a] L21[b][k], k >= a (X11 lower), stored n1 x n2
            float* U = X + off + r0 * ld + (r0 + n1);
            GemmArgs t{n1, n2, n1, 1.0f, 0.0f, X11, ld, gs, L21, ld, gs, U, ld, gs, 1, 1, CMASK_FULL, KR_FROM_I, gb,
                       PT_GEMM_INV, (double)gb * n2 * n1 * (n1 + 1)};
            if ((rc = gemm_f32(t, st))) return rc;
            // X21 = -X22 T, k <= i (X22 lower)
            GemmArgs x{n2, n1, n2, -1.0f, 0.0f, X22, ld, gs, U, ld, gs, X21, ld, gs, 0, 1, CMASK_FULL, KR_TO_I, gb,
                       PT_GEMM_INV, (double)gb * n1 * n2 * (n2 + 1)};
            if ((rc = gemm_f32(x, st))) return rc;
        }
    }
    return IC_OK;
}

int trtri(const float* L, float* X, int64_t batch, int64_t n, int64_t ld, int64_t sH, const double* dinv64,
          hipStream_t st) {
    const int64_t nblk = cdiv(n, NB);
    const int64_t dstride = nblk * NB * NB;
    hipLaunchKernelGGL(put_diag_all_kernel, dim3((unsigned)nblk, (unsigned)batch), dim3(256), 0, st, X, n, ld, sH,
                       dinv64, dstride);
    IC_CHECK_LAUNCH();
    // segments of rows [start, start + len); merged pairwise per level
    std::vector<int64_t> seg;
    for (int64_t k = 0; k < nblk; ++k) seg.push_back(k * NB);
    seg.push_back(n);
    while (seg.size() > 2) {
        const int64_t nseg = (int64_t)seg.size() - 1;
        const int64_t npair = nseg / 2;
        std::vector<int64_t> next;
        // pairs with the shape of the first one and uniform spacing run together
        int64_t p = 0;
        while (p < npair) {
            const int64_t r0 = seg[2 * p], n1 = seg[2 * p + 1] - r0, n2 = seg[2 * p + 2] - seg[2 * p + 1];
            int64_t q = p + 1;
            while (q < npair && seg[2 * q + 1] - seg[2 * q] == n1 && seg[2 * q + 2] - seg[2 * q + 1] == n2 &&
                   seg[2 * q] - seg[2 * q - 2] == n1 + n2)
                ++q;
            int rc = merge_pairs(L, X, ld, r0, n1, n2, q - p, (n1 + n2) * (ld + 1), batch, sH, st);
            if (rc) return rc;
            p = q;
        }
        for (int64_t i = 0; i < npair; ++i) next.push_back(seg[2 * i]);
        if (nseg % 2) next.push_back(seg[nseg - 1]);
        next.push_back(n);
        seg.swap(next);
    }
    return IC_OK;
}

}  // namespace icq

using namespace icq;

extern "C" int64_t ic_hessian_inverse_workspace_bytes(int64_t batch, int64_t n) {
    return (batch * n * n + dinv_floats(batch, n)) * (int64_t)sizeof(float) +
           dinv_floats(batch, n) * (int64_t)sizeof(double) + 256;
}

extern "C" int ic_hessian_inverse(float* H, int64_t batch, int64_t n, float damping, int method, int* info,
                                  void* workspace, void* stream) {
    IC_REQUIRE(H && info && workspace, "ic_hessian_inverse: null pointer");
    IC_REQUIRE(n >= 0 && batch >= 0, "ic_hessian_inverse: bad size");
    IC_REQUIRE(method >= 0 && method <= 2,
               "ic_hessian_inverse: method must be 0 (hinv), 1 (cholesky) or 2 (hinv, upper triangle)");
    if (n == 0 || batch == 0) return IC_OK;
    hipStream_t st = as_stream(stream);
    const int64_t ld = n, sH = n * n;
    float* X = reinterpret_cast<float*>(workspace);
    float* dinv = X + batch * sH;
    double* dinv64 = dinv64_of(dinv, batch, n);
    IC_CHECK_HIP(hipMemsetAsync(info, 0, batch * sizeof(int), st));
    hipLaunchKernelGGL(damp_kernel, dim3((unsigned)batch), dim3(256), 0, st, H, n, ld, sH, damping);
    IC_CHECK_LAUNCH();
    int rc = potrf(H, batch, n, ld, sH, dinv64, info, st);
    if (rc) return rc;
    rc = trtri(H, X, batch, n, ld, sH, dinv64, st);
    if (rc) return rc;
    // H^-1 (upper triangle incl. diagonal) = X^T X  -> H
    GemmArgs u{n, n, n, 1.0f, 0.0f, X, ld, sH, X, ld, sH, H, ld, sH, 1, 0, CMASK_UPPER, KR_FROM_MAXIJ, batch,
               PT_GEMM_INV, (double)batch * 2.0 * (double)n * (n + 1) * (n + 2) / 6.0};
    rc = gemm_f32(u, st);
    if (rc) return rc;
    dim3 tb(16, 16), tg((unsigned)cdiv(n, 16), (unsigned)cdiv(n, 16), (unsigned)batch);
    if (method == 2) return IC_OK;   // the lower part keeps L: finite, never read by such callers
    if ((rc = mirror_upper(H, batch, n, ld, sH, st))) return rc;
    if (method == 1) {
        // upper Cholesky factor of H^-1 (converter/gptq.py:91-110): L2 = chol(H^-1), return L2^T
        rc = potrf(H, batch, n, ld, sH, dinv64, info + batch, st);
        if (rc) return rc;
        hipLaunchKernelGGL(lower_to_upper_kernel, tg, tb, 0, st, H, n, ld, sH);
        IC_CHECK_LAUNCH();
    }
    return IC_OK;
}

extern "C" int ic_damp_hessian(float* H, int64_t batch, int64_t n, float damping, void* stream) {
    IC_REQUIRE(H || batch == 0 || n == 0, "ic_damp_hessian: null pointer");
    IC_REQUIRE(n >= 0 && batch >= 0 && batch < (1LL << 31), "ic_damp_hessian: bad size");
    if (n == 0 || batch == 0) return IC_OK;
    hipLaunchKernelGGL(damp_kernel, dim3((unsigned)batch), dim3(256), 0, as_stream(stream), H, n, n, n * n, damping);
    IC_CHECK_LAUNCH();
    return IC_OK;
}

extern "C" int ic_gram_tn(const float* W, int64_t M, int64_t N, int64_t ldw, float alpha, float* C, void* stream) {
    IC_REQUIRE(W && C, "ic_gram_tn: null pointer");
    IC_REQUIRE(M >= 0 && N >= 0 && ldw >= N, "ic_gram_tn: bad size");
    if (N == 0) return IC_OK;
    hipStream_t st = as_stream(stream);
    // C[i][j] and C[j][i] are the same products summed in the same order:
    // the upper triangle on the matrix cores, then mirrored
    GemmArgs g{N, N, M, alpha, 0.0f, W, ldw, 0, W, ldw, 0, C, N, 0, 1, 0, CMASK_UPPER, KR_FULL, 1, PT_OTHER,
               (double)N * (N + 1) * M};
    int rc = gemm_f32(g, st);
    if (rc) return rc;
    return mirror_upper(C, 1, N, N, N * N, st);
}

extern "C" int ic_cholesky(float* H, int64_t batch, int64_t n, int* info, void* workspace, void* stream) {
    IC_REQUIRE(H && info && workspace, "ic_cholesky: null pointer");
    if (n == 0 || batch == 0) return IC_OK;
    hipStream_t st = as_stream(stream);
    IC_CHECK_HIP(hipMemsetAsync(info, 0, batch * sizeof(int), st));
    float* dinv = reinterpret_cast<float*>(workspace) + batch * n * n;
    double* dinv64 = dinv64_of(dinv, batch, n);
    return potrf(H, batch, n, n, n * n, dinv64, info, st);
}
