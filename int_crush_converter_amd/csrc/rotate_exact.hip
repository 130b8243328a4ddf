// Group-wise Hadamard rotation in the reference's own summation order.
//
// converter/rotation.py:82-92 rotates weights as `x @ H.T` and :237-248 the
// Hessian as einsum("kp,nkl,le->npe", R, H, R), which torch contracts left
// to right: T = R^T H_blk first, then T R.  On the CPU each of these is an
// fp32 GEMM in which every output is ONE fused multiply-add chain over the
// contraction index in increasing order, starting from zero (checked against
// the reference for R = 2 .. 256, 2-D and 3-D Hessians; R = 512 is two
// 256-long chains whose results are added).  For the regular Hadamard the
// products are exact (entries +-2^-k), so only the order of the additions
// decides the rounding - and a fast Walsh-Hadamard transform (rotate.hip)
// associates them differently.
//
// A K = 1 fp32 MFMA (v_mfma_f32_16x16x1_4b_f32) computes D = fma(A, B, C)
// element by element, correctly rounded with denormals kept, so a chain of
// them over k IS the sequential fma chain, at the matrix-core rate (twice
// the VALU fma rate).  Lane layout of that instruction (block b = v / 4 of
// the 16 accumulator registers v):
//     A: lane 16 b + i supplies A[b][i];   B: lane 16 b + j supplies B[b][j];
//     D[b][i][j] sits in register v = 4 b + i % 4 of lane 16 (i / 4) + j.
//
//  rows (weights, and the right product of the Hessian):
//      Y[r][j] = sum_k X[r][k] Hd[k][j]  -  blocks b = 4 row tiles of 16,
//      A = X (lane <-> row, staged in LDS), B = Hd[k][j] built in registers.
//  cols (the Hessian's left product):
//      T[p][l] = sum_k Hd[k][p] H[k][l]  -  blocks b = 4 column tiles of 16,
//      A = Hd[k][p] in registers, B = H rows (lane <-> column, from LDS).
//
// Hd[k][j] = m * (-1)^s(k, j) with, for the regular matrix of size 4^n,
// m = 2^-n and s = the number of base-4 digits where k_d + j_d = 3, i.e.
// popcount(t & (t >> 1) & 0x55..) with t = k ^ j; for the Sylvester matrix
// of size 2^n, m = fp32(1/sqrt(2^n)) and s = popcount(k & j).  Both split
// over k = 16 k_hi + k_lo, j = 16 j_hi + j_lo: s = s(k_lo, j_lo) + s(k_hi,
// j_hi).  A lane keeps the 16 values m (-1)^s(k_lo, j_lo) of its own j_lo and
// flips their sign bit with the wave-uniform s(k_hi, j_hi).
#include <algorithm>
#include <cmath>
#include <cstring>

#include "common.hpp"
#include "prof.hpp"

namespace icq {

typedef float f32x16 __attribute__((ext_vector_type(16)));

template <bool REG>
__host__ __device__ __forceinline__ uint32_t hd_sign(uint32_t k, uint32_t j) {
    if (REG) {
        const uint32_t t = k ^ j;
        return (uint32_t)__builtin_popcount(t & (t >> 1) & 0x55555555u) & 1u;
    }
    return (uint32_t)__builtin_popcount(k & j) & 1u;
}

__device__ __forceinline__ f32x16 mfma_k1(float a, float b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_16x16x1f32(a, b, c, 0, 0, 0);
}

// Four consecutive source elements as fp32: one 16-byte (f32) or 8-byte
// (bf16 / f16) load when `vec` and in bounds, else element by element with
// zeros beyond `cols`.
template <int DT>
__device__ __forceinline__ void load4(const void* src, int64_t off, int64_t c, int64_t cols, bool vec, float (&v)[4]) {
    if (vec && c + 3 < cols) {
        if (DT == IC_DTYPE_F32) {
            const float4 t = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(src) + off);
            v[0] = t.x; v[1] = t.y; v[2] = t.z; v[3] = t.w;
        } else {
            const uint2 t = *reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(src) + off);
            const uint32_t u[2] = {t.x, t.y};
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                if (DT == IC_DTYPE_BF16) {
                    v[2 * h] = __uint_as_float(u[h] << 16);
                    v[2 * h + 1] = __uint_as_float(u[h] & 0xffff0000u);
                } else {
                    v[2 * h] = f16_bits_to_f32((uint16_t)(u[h] & 0xffffu));
                    v[2 * h + 1] = f16_bits_to_f32((uint16_t)(u[h] >> 16));
                }
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = (c + i < cols) ? load_as_f32(src, DT, off + i) : 0.0f;
    }
}

__device__ __forceinline__ void flush_zeroed(unsigned cnt, unsigned long long* nz) {
    if (!nz) return;
    const unsigned long long c = wave_sum((unsigned long long)cnt);
    if ((threadIdx.x & 63) == 0 && c) atomicAdd(nz, c);
}

// ------------------------------------------------------------------ rows

constexpr int XR_ROWS = 64;            // rows per tile (4 row tiles of 16 per MFMA)
constexpr int XR_SLICE = 256;          // output columns per work-group: 4 waves x 4 tiles x 16
constexpr int XR_LD = XR_SLICE + 4;    // LDS pitch: lanes 4 banks apart, 16-byte reads conflict-free

// Work-group y takes output columns [s0, s0 + 256) of every 64-row tile
// blockIdx.x, blockIdx.x + gridDim.x, ...; a tile's input columns are staged
// in LDS (for R <= 256 the slice holds whole groups and its input is the same
// 256 columns; R = 512 stages the group's inputs in two chunks of 256 whose
// chains are added at the end), and the next tile's global loads are in
// flight while the current one runs on the matrix cores.
//
// Signs.  Tile c (0..3) of wave w covers in-group columns 16 (U + c) .. + 15
// with U a multiple of 4 (R >= 64; for R = 32 its in-group block is c & 1,
// for R = 16 it is 0).  For k = 16 kh + q the entry's sign is
//     s(q, lane & 15)  ^  s(kh & 3, c)  ^  s(kh >> 2, U >> 2)
// (both Hadamard kinds factor over these digit / bit groups).  The first is
// the lane's B register, the second is known at compile time (kh and c are
// unrolled) and picks the register holding the negated value, the third is
// wave-uniform and flips the sign of A, which all four tiles share: no
// per-MFMA sign arithmetic.  TRI (one matrix, rows == n_tri): only blocks
// (bi, bj) of size R with bj <= bi are needed; the work-group walks the row
// tiles from the first that reaches block row s0 / R.
template <int R, int DT, bool TRI>
__global__ __launch_bounds__(256, 2) void rot_rows_exact_kernel(const void* __restrict__ src, int64_t rows, int64_t cols,
                                                               int64_t ld_src, float* __restrict__ dst,
                                                               int64_t cols_pad, int64_t ld_dst, int64_t n_tri,
                                                               uint32_t mag_bits, float zero_above,
                                                               unsigned long long* __restrict__ nz, int vec) {
    constexpr bool REG = (R & 0x55555555) == R;
    constexpr int KL = R < XR_SLICE ? R : XR_SLICE;        // k steps per chunk
    constexpr int NCH = R > XR_SLICE ? R / XR_SLICE : 1;   // chunks
    __shared__ __align__(16) float xs[XR_ROWS * XR_LD];
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int64_t s0 = (int64_t)blockIdx.y * XR_SLICE;
    const int64_t ntile = cdiv(rows, XR_ROWS);
    const int64_t kb = R > XR_SLICE ? (s0 / R) * R : s0;   // first input column of chunk 0
    // the first slice of a group counts its outliers (every input once)
    const bool count = zero_above > 0.0f && (R <= XR_SLICE || s0 % R == 0);
    // TRI (one matrix, rows == n_tri): the row tiles that reach block row s0 / R
    const int64_t rt0 = TRI ? std::max<int64_t>(0, ((s0 / R) * R - (XR_ROWS - 1) + XR_ROWS - 1) / XR_ROWS) : 0;
    int64_t rt = rt0 + blockIdx.x;
    if (rt >= ntile) return;

    float bp[16], bn[16];   // m (-1)^s(q, lane & 15) and its negation
#pragma unroll
    for (int q = 0; q < 16; ++q) {
        bp[q] = __uint_as_float(mag_bits | (hd_sign<REG>((uint32_t)q, (uint32_t)(lane & 15)) << 31));
        bn[q] = -bp[q];
    }
    // U >> 2 of the wave's tiles (uniform)
    const uint32_t uhi = R >= 512 ? (uint32_t)((s0 % R) >> 6) + (uint32_t)w
                         : R == 256 ? (uint32_t)w : R == 128 ? (uint32_t)(w & 1) : 0u;
    int acol[4];   // the first LDS column of tile c's group
#pragma unroll
    for (int c = 0; c < 4; ++c) acol[c] = R <= XR_SLICE ? ((64 * w + 16 * c) / R) * R : 0;

    float v[16][4];
    auto gload = [&](int64_t t, int ch) {
        const int64_t c0 = kb + (int64_t)ch * XR_SLICE, r0 = t * XR_ROWS;
#pragma unroll
        for (int it = 0; it < 16; ++it) {
            const int u = it * 256 + tid, rr = u >> 6, cq = (u & 63) * 4;
            const int64_t r = r0 + rr, c = c0 + cq;
            if (r < rows) load4<DT>(src, r * ld_src + c, c, cols, (vec & 1) != 0, v[it]);
            else v[it][0] = v[it][1] = v[it][2] = v[it][3] = 0.0f;
        }
    };
    gload(rt, 0);
    f32x16 acc[4], part[4];
    unsigned cnt = 0;
    int ch = 0;
    const float* xrow = &xs[lane * XR_LD];
    for (;;) {
        __syncthreads();   // every wave is done with the previous item's LDS
#pragma unroll
        for (int it = 0; it < 16; ++it) {
            if (zero_above > 0.0f) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const bool out = fabsf(v[it][i]) > zero_above;
                    cnt += (out && count) ? 1u : 0u;
                    v[it][i] = out ? 0.0f : v[it][i];
                }
            }
            const int u = it * 256 + tid, rr = u >> 6, cq = (u & 63) * 4;
            *reinterpret_cast<float4*>(&xs[rr * XR_LD + cq]) = make_float4(v[it][0], v[it][1], v[it][2], v[it][3]);
        }
        __syncthreads();
        // the next item's loads fly while this one runs
        int64_t nrt = rt;
        int nch = ch + 1;
        if (nch == NCH) {
            nch = 0;
            nrt = rt + gridDim.x;
        }
        const bool more = nrt < ntile;
        if (more) gload(nrt, nch);
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[c] = f32x16{};
        // steps t = 4 kh + q4 of four k each; each step's A values are read
        // from LDS one step ahead, so the read is in flight during the
        // previous step's MFMAs
        float4 a4n[4];
        auto read_a = [&](int t, float4 (&a4)[4]) {
            if constexpr (R >= 64) {
                a4[0] = *reinterpret_cast<const float4*>(xrow + acol[0] + 4 * t);
            } else {
#pragma unroll
                for (int c = 0; c < 4; ++c) a4[c] = *reinterpret_cast<const float4*>(xrow + acol[c] + 4 * t);
            }
        };
        read_a(0, a4n);
        auto step = [&](auto TT) {
            constexpr int t = decltype(TT)::value, kh = t / 4, q4 = t % 4;
            float4 a4[4];
#pragma unroll
            for (int c = 0; c < 4; ++c) a4[c] = a4n[c];
            if constexpr (t + 1 < KL / 4) read_a(t + 1, a4n);
            __builtin_amdgcn_sched_barrier(0);   // keep the next read ahead of these MFMAs
            if constexpr (R >= 64) {
                if constexpr (R >= 128) {
                    const uint32_t gs = hd_sign<REG>((uint32_t)(ch * (XR_SLICE / 16) + kh) >> 2, uhi) << 31;
                    a4[0].x = __uint_as_float(__float_as_uint(a4[0].x) ^ gs);
                    a4[0].y = __uint_as_float(__float_as_uint(a4[0].y) ^ gs);
                    a4[0].z = __uint_as_float(__float_as_uint(a4[0].z) ^ gs);
                    a4[0].w = __uint_as_float(__float_as_uint(a4[0].w) ^ gs);
                }
                a4[1] = a4[2] = a4[3] = a4[0];
            }
#pragma unroll
            for (int qq = 0; qq < 4; ++qq) {
                const int q = 4 * q4 + qq;
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const int jc = R >= 64 ? c : R == 32 ? (c & 1) : 0;
                    const bool neg = hd_sign<REG>((uint32_t)(kh & 3), (uint32_t)jc) != 0;
                    const float a = qq == 0 ? a4[c].x : qq == 1 ? a4[c].y : qq == 2 ? a4[c].z : a4[c].w;
                    acc[c] = mfma_k1(a, neg ? bn[q] : bp[q], acc[c]);
                }
            }
        };
        static_for<0, KL / 4>(step);
        if constexpr (NCH > 1) {
            if (ch == 0) {
#pragma unroll
                for (int c = 0; c < 4; ++c) part[c] = acc[c];
            }
        }
        if (ch == NCH - 1) {
            // the output tile goes through LDS (its input is no longer
            // needed) so that whole rows leave in 16-byte stores
            __syncthreads();
#pragma unroll
            for (int c = 0; c < 4; ++c)
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    float y = acc[c][e];
                    if constexpr (NCH > 1) y = part[c][e] + y;
                    xs[(16 * (e >> 2) + 4 * (lane >> 4) + (e & 3)) * XR_LD + 64 * w + 16 * c + (lane & 15)] = y;
                }
            __syncthreads();
            const int64_t r0 = rt * XR_ROWS;
#pragma unroll
            for (int it = 0; it < 16; ++it) {
                const int u = it * 256 + tid, rr = u >> 6, cq = (u & 63) * 4;
                const int64_t r = r0 + rr, col = s0 + cq;   // cols_pad is a multiple of 16
                if (r >= rows || col >= cols_pad) continue;
                const float4 y = *reinterpret_cast<const float4*>(&xs[rr * XR_LD + cq]);
                float* o = dst + r * ld_dst + col;
                if (vec & 2) {
                    *reinterpret_cast<float4*>(o) = y;
                } else {
                    o[0] = y.x; o[1] = y.y; o[2] = y.z; o[3] = y.w;
                }
            }
        }
        if (!more) break;
        rt = nrt;
        ch = nch;
    }
    if (count) flush_zeroed(cnt, nz);
}

// Rows out of place, one wave per output slice (R = 64, 128, 256; rows whose
// width is a whole number of groups, aligned for vector loads): work items
// are (256-column slice, 64-row tile) pairs, one round of work-groups takes
// them in turn, and wave w owns the item's output columns 64 w .. + 63, all
// inside one group.  Each lane reads its own row's four values of a step
// straight from memory (the four waves of a work-group share the rows
// through the caches), several steps ahead in registers - the next item's
// first steps while this one's last run; the products leave straight from
// the accumulators.  No LDS and no barrier: the waves of a SIMD drift apart,
// so one wave's loads and stores overlap another's matrix-core work.  In
// place (the Hessian's right product) takes the row kernel above, whose
// tile is read whole before it is written.  Signs, chains and results are
// the row kernel's (the same MFMA sequence per output).
constexpr int XW_PF = 8;   // steps (4 k each) of A in flight

// Four consecutive source elements of a row as they are stored (one 16-byte
// load for f32, one 8-byte load for 16-bit types), and their fp32 values;
// the conversion happens where the values are used, so a load never waits.
template <int DT>
struct Raw4 {
    static constexpr bool F32 = DT == IC_DTYPE_F32;
    uint32_t u[F32 ? 4 : 2];
    __device__ __forceinline__ void load(const void* src, int64_t off) {
        if constexpr (F32) {
            const uint4 t = *reinterpret_cast<const uint4*>(reinterpret_cast<const float*>(src) + off);
            u[0] = t.x; u[1] = t.y; u[2] = t.z; u[3] = t.w;
        } else {
            const uint2 t = *reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(src) + off);
            u[0] = t.x; u[1] = t.y;
        }
    }
    __device__ __forceinline__ float get(int i) const {
        if constexpr (F32) return __uint_as_float(u[i]);
        const uint32_t h = i & 1 ? u[i >> 1] >> 16 : u[i >> 1] & 0xffffu;
        if constexpr (DT == IC_DTYPE_BF16) return __uint_as_float(h << 16);
        return f16_bits_to_f32((uint16_t)h);
    }
};

template <int R, int DT, bool ZA>
__global__ __launch_bounds__(256, 2) void rot_rows_wave_kernel(const void* __restrict__ src, int64_t rows,
                                                              int64_t cols, int64_t ld_src, float* __restrict__ dst,
                                                              int64_t cols_pad, int64_t ld_dst, uint32_t mag_bits,
                                                              float zero_above, unsigned long long* __restrict__ nz,
                                                              int vec) {
    static_assert(R == 64 || R == 128 || R == 256, "one group per 64-column slice");
    constexpr bool REG = (R & 0x55555555) == R;
    constexpr int T = R / 4;   // steps per chain
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    // items: (column slice y, row tile rt), the row tiles of a slice
    // consecutive; work-group i takes items i, i + gridDim.x, ...
    const int64_t ntile = cdiv(rows, XR_ROWS), nitems = ntile * cdiv(cols_pad, XR_SLICE);
    int64_t item = blockIdx.x;
    if (item >= nitems) return;
    int64_t y = item / ntile, rt = item - y * ntile;

    float bp[16], bn[16];   // m (-1)^s(q, lane & 15) and its negation
#pragma unroll
    for (int q = 0; q < 16; ++q) {
        bp[q] = __uint_as_float(mag_bits | (hd_sign<REG>((uint32_t)q, (uint32_t)(lane & 15)) << 31));
        bn[q] = -bp[q];
    }
    unsigned cnt = 0;
    // the wave's columns of slice y: output c0 .. c0 + 63 (inside one group
    // when active: cols_pad is a multiple of R >= 64), inputs from g0
    auto slice_c0 = [&](int64_t yy) { return yy * XR_SLICE + 64 * w; };
    // offset of (this lane's row of tile t, the group's first column); rows
    // past the matrix read its last row (their products are never stored)
    auto row_off = [&](int64_t yy, int64_t tile) {
        const int64_t c = slice_c0(yy);
        return std::min<int64_t>(tile * XR_ROWS + lane, rows - 1) * ld_src + (c < cols_pad ? (c / R) * R : 0);
    };
    Raw4<DT> a[XW_PF];
    auto load_step = [&](int slot, int64_t off, int t) { a[slot].load(src, off + 4 * t); };
    int64_t off = row_off(y, rt);
    if (slice_c0(y) < cols_pad) {
#pragma unroll
        for (int t = 0; t < XW_PF; ++t) load_step(t, off, t);
    }
    for (;;) {
        const int64_t c0 = slice_c0(y);
        const bool active = c0 < cols_pad;               // wave-uniform
        const int64_t g0 = (c0 / R) * R;
        const uint32_t uhi = (uint32_t)((c0 - g0) >> 6); // U >> 2 of its four tiles
        // outliers this lane counts: the group's first slice, its own row
        const unsigned mine = (ZA && active && c0 == g0 && rt * XR_ROWS + lane < rows) ? 1u : 0u;
        const bool more = item + gridDim.x < nitems;
        const int64_t ny = (item + gridDim.x) / ntile, nrt = (item + gridDim.x) - ny * ntile;
        const bool nact = more && slice_c0(ny) < cols_pad;
        const int64_t noff = nact ? row_off(ny, nrt) : off;
        f32x16 acc[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[c] = f32x16{};
        auto step = [&](auto TT) {
            constexpr int t = decltype(TT)::value, kh = t / 4, q4 = t % 4, slot = t % XW_PF;
            float x[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) x[i] = a[slot].get(i);
            if constexpr (ZA) {
                // outliers become 0
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float m = fabsf(x[i]);
                    cnt += m > zero_above ? mine : 0u;
                    x[i] = m > zero_above ? 0.0f : x[i];
                }
                asm volatile("" : "+v"(cnt));   // count now: the compares' masks die here
            }
            // refill the slot: a later step of this item, or the next item's
            if constexpr (t + XW_PF < T) {
                if (active) load_step(slot, off, t + XW_PF);
            } else {
                if (nact) load_step(slot, noff, t + XW_PF - T);
            }
            if constexpr (R >= 128) {
                const uint32_t gs = hd_sign<REG>((uint32_t)kh >> 2, uhi) << 31;
#pragma unroll
                for (int i = 0; i < 4; ++i) x[i] = __uint_as_float(__float_as_uint(x[i]) ^ gs);
            }
            // the step's four A values in four registers before its MFMAs, so
            // that no A register is rewritten while an MFMA still reads it
            asm volatile("" : "+v"(x[0]), "+v"(x[1]), "+v"(x[2]), "+v"(x[3]));
#pragma unroll
            for (int qq = 0; qq < 4; ++qq) {
                const int q = 4 * q4 + qq;
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const bool neg = hd_sign<REG>((uint32_t)(kh & 3), (uint32_t)c) != 0;
                    acc[c] = mfma_k1(x[qq], neg ? bn[q] : bp[q], acc[c]);
                }
            }
        };
        static_for<0, T>(step);
        if (active) {
            const int64_t rb = rt * XR_ROWS + 4 * (lane >> 4);
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                float* o = dst + c0 + 16 * c + (lane & 15);
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const int64_t r = rb + 16 * (v >> 2) + (v & 3);
                    if (r < rows) o[r * ld_dst] = acc[c][v];
                }
            }
        }
        if (!more) break;
        item += gridDim.x;
        y = ny;
        rt = nrt;
        off = noff;
    }
    if (ZA) flush_zeroed(cnt, nz);
}

// Work-groups of a 256-thread kernel without dynamic LDS that fit the
// current device at once (0 when the runtime cannot say).
static int64_t resident_wgs(const void* kernel) {
    int dev = 0, per_cu = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, 256, 0) != hipSuccess) return 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    return (int64_t)per_cu * cus;
}

// One round of work-groups (as many as are resident at once, each taking
// whole items in turn), so no partial second round idles the chip; fewer
// than two rounds' worth of items run one per work-group.
template <int R, int DT, bool ZA>
static void launch_rows_wave(const void* src, int64_t rows, int64_t cols, int64_t ld_src, float* dst,
                             int64_t cols_pad, int64_t ld_dst, uint32_t mb, float zero_above,
                             unsigned long long* nz, int vec, hipStream_t st) {
    const void* k = reinterpret_cast<const void*>(&rot_rows_wave_kernel<R, DT, ZA>);
    static int64_t cap = 0;   // the same on every device this library runs on (one GPU model)
    if (cap <= 0) cap = resident_wgs(k);
    const int64_t n = cdiv(rows, XR_ROWS) * cdiv(cols_pad, XR_SLICE), c = cap > 0 ? cap : 512;
    // below two rounds of items, one item per work-group balances best
    const int64_t per = n >= 2 * c ? cdiv(n, c) : 1;
    const int64_t grid = std::max<int64_t>(1, cdiv(n, per));
    hipLaunchKernelGGL((rot_rows_wave_kernel<R, DT, ZA>), dim3((unsigned)grid), dim3(256), 0, st, src, rows, cols,
                       ld_src, dst, cols_pad, ld_dst, mb, zero_above, nz, vec);
}

// ------------------------------------------------------------------ columns

constexpr int XC_ROWS = 256;   // T rows per work-group: 4 waves x 4 tiles x 16
constexpr int XC_COLS = 64;    // columns per tile: 4 blocks of 16

// Work-group (x, y, z): T rows [r0, r0 + 256) (r0 = 256 y) of matrix z, for
// the 64-column tiles x, x + gridDim.x, ...; R <= 256, so the rows hold whole
// groups.  The next tile's loads are in flight while the current one runs.
// In place is safe: a tile's region is read whole before it is written, and
// no other work-group touches it.  Signs as in the row kernel, with the roles
// of A (the Hadamard entries, per lane p) and B (the data, shared by the
// four tiles: the uniform part of the sign flips it).
template <int R, bool TRI>
__global__ __launch_bounds__(256, 2) void rot_cols_exact_kernel(const float* __restrict__ src, float* __restrict__ dst,
                                                               int64_t n, int64_t ld, int64_t bstride,
                                                               uint32_t mag_bits, int vec) {
    constexpr bool REG = (R & 0x55555555) == R;
    __shared__ __align__(16) float hs[XC_ROWS * XC_COLS];
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int64_t r0 = (int64_t)blockIdx.y * XC_ROWS;
    const int64_t ntile = cdiv(n, XC_COLS);
    const float* S = src + (int64_t)blockIdx.z * bstride;
    float* D = dst + (int64_t)blockIdx.z * bstride;
    // TRI: the column tiles that start at or before the last block column
    // of these rows' block rows
    const int64_t ncap = TRI ? std::min<int64_t>(ntile, cdiv(((r0 + XC_ROWS - 1) / R + 1) * R, XC_COLS)) : ntile;
    int64_t lt = blockIdx.x;
    if (lt >= ncap) return;

    float ap[16], an[16];   // m (-1)^s(q, lane & 15) and its negation
#pragma unroll
    for (int q = 0; q < 16; ++q) {
        ap[q] = __uint_as_float(mag_bits | (hd_sign<REG>((uint32_t)q, (uint32_t)(lane & 15)) << 31));
        an[q] = -ap[q];
    }
    const uint32_t uhi = R == 256 ? (uint32_t)w : 0u;   // U >> 2 of the wave's tiles
    int brow[4];   // the first LDS row of tile c's group
#pragma unroll
    for (int c = 0; c < 4; ++c) brow[c] = ((64 * w + 16 * c) / R) * R;

    float v[16][4];
    auto gload = [&](int64_t t) {
        const int64_t l0 = t * XC_COLS;
#pragma unroll
        for (int it = 0; it < 16; ++it) {
            const int u = it * 256 + tid, rr = u >> 4, cq = (u & 15) * 4;
            const int64_t r = r0 + rr, c = l0 + cq;
            if (r < n) load4<IC_DTYPE_F32>(S, r * ld + c, c, n, (vec & 1) != 0, v[it]);
            else v[it][0] = v[it][1] = v[it][2] = v[it][3] = 0.0f;
        }
    };
    gload(lt);
    f32x16 acc[4];
    for (;;) {
        __syncthreads();   // every wave is done with the previous tile's LDS
#pragma unroll
        for (int it = 0; it < 16; ++it) {
            const int u = it * 256 + tid, rr = u >> 4, cq = (u & 15) * 4;
            *reinterpret_cast<float4*>(&hs[rr * XC_COLS + cq]) = make_float4(v[it][0], v[it][1], v[it][2], v[it][3]);
        }
        __syncthreads();
        const int64_t nlt = lt + gridDim.x;
        const bool more = nlt < ncap;
        if (more) gload(nlt);
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[c] = f32x16{};
        // steps t = 16 kh + q of one k each; B is read from LDS one step ahead
        float bnx[4];
        auto read_b = [&](int t, float (&b)[4]) {
            if constexpr (R >= 64) {
                b[0] = hs[(brow[0] + t) * XC_COLS + lane];
            } else {
#pragma unroll
                for (int c = 0; c < 4; ++c) b[c] = hs[(brow[c] + t) * XC_COLS + lane];
            }
        };
        read_b(0, bnx);
        auto step = [&](auto TT) {
            constexpr int t = decltype(TT)::value, kh = t / 16, q = t % 16;
            float b[4];
#pragma unroll
            for (int c = 0; c < 4; ++c) b[c] = bnx[c];
            if constexpr (t + 1 < R) read_b(t + 1, bnx);
            __builtin_amdgcn_sched_barrier(0);   // keep the next read ahead of these MFMAs
            if constexpr (R >= 64) {
                if constexpr (R == 256) {
                    const uint32_t gs = hd_sign<REG>((uint32_t)kh >> 2, uhi) << 31;
                    b[0] = __uint_as_float(__float_as_uint(b[0]) ^ gs);
                }
                b[1] = b[2] = b[3] = b[0];
            }
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const int pc = R >= 64 ? c : 0;
                const bool neg = hd_sign<REG>((uint32_t)(kh & 3), (uint32_t)pc) != 0;
                acc[c] = mfma_k1(neg ? an[q] : ap[q], b[c], acc[c]);
            }
        };
        static_for<0, R>(step);
        // the output tile through LDS: rows of 64 columns in 16-byte stores
        __syncthreads();
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int e = 0; e < 16; ++e)
                hs[(64 * w + 16 * c + 4 * (lane >> 4) + (e & 3)) * XC_COLS + 16 * (e >> 2) + (lane & 15)] = acc[c][e];
        __syncthreads();
        const int64_t l0 = lt * XC_COLS;
#pragma unroll
        for (int it = 0; it < 16; ++it) {
            const int u = it * 256 + tid, rr = u >> 4, cq = (u & 15) * 4;
            const int64_t r = r0 + rr, col = l0 + cq;
            if (r >= n || col >= n) continue;
            const float4 y = *reinterpret_cast<const float4*>(&hs[rr * XC_COLS + cq]);
            float* o = D + r * ld + col;
            if ((vec & 2) && col + 3 < n) {
                *reinterpret_cast<float4*>(o) = y;
            } else {
                o[0] = y.x;
                if (col + 1 < n) o[1] = y.y;
                if (col + 2 < n) o[2] = y.z;
                if (col + 3 < n) o[3] = y.w;
            }
        }
        if (!more) break;
        lt = nlt;
    }
}

// ------------------------------------------------------------------ small R (2, 4, 8): VALU fma chains

// One thread per (row, group): reads the group's R inputs, writes its R
// outputs (so in place is safe and every input is counted once).
template <int R, int DT>
__global__ __launch_bounds__(256) void rot_rows_small_kernel(const void* __restrict__ src, int64_t rows, int64_t cols,
                                                             int64_t ld_src, float* dst, int64_t groups,
                                                             int64_t ld_dst, float mag, float zero_above,
                                                             unsigned long long* __restrict__ nz) {
    constexpr bool REG = (R & 0x55555555) == R;
    unsigned cnt = 0;
    for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < rows * groups;
         t += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = t / groups, g = t % groups;
        float x[R];
#pragma unroll
        for (int k = 0; k < R; ++k) {
            const int64_t c = g * R + k;
            float v = c < cols ? load_as_f32(src, DT, r * ld_src + c) : 0.0f;
            if (zero_above > 0.0f && fabsf(v) > zero_above) { v = 0.0f; ++cnt; }
            x[k] = v;
        }
#pragma unroll
        for (int j = 0; j < R; ++j) {
            float y = 0.0f;
#pragma unroll
            for (int k = 0; k < R; ++k) y = __builtin_fmaf(x[k], hd_sign<REG>(k, j) ? -mag : mag, y);
            dst[r * ld_dst + g * R + j] = y;
        }
    }
    if (zero_above > 0.0f) flush_zeroed(cnt, nz);
}

// One thread per (matrix, group, column): T[g R + p][l] = sum_k Hd[k][p] H[g R + k][l].
template <int R>
__global__ __launch_bounds__(256) void rot_cols_small_kernel(const float* __restrict__ src, float* dst, int64_t batch,
                                                             int64_t n, int64_t ld, int64_t bstride, float mag) {
    constexpr bool REG = (R & 0x55555555) == R;
    const int64_t per = (n / R) * n;
    for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < batch * per;
         t += (int64_t)gridDim.x * blockDim.x) {
        const int64_t b = t / per, g = (t % per) / n, l = t % n;
        const float* S = src + b * bstride;
        float* D = dst + b * bstride;
        float x[R];
#pragma unroll
        for (int k = 0; k < R; ++k) x[k] = S[(g * R + k) * ld + l];
#pragma unroll
        for (int p = 0; p < R; ++p) {
            float y = 0.0f;
#pragma unroll
            for (int k = 0; k < R; ++k) y = __builtin_fmaf(hd_sign<REG>(k, p) ? -mag : mag, x[k], y);
            D[(g * R + p) * ld + l] = y;
        }
    }
}

static bool pow2(int64_t n) { return n > 0 && (n & (n - 1)) == 0; }
static bool pow4(int64_t n) { return pow2(n) && (n & 0x55555555) == n; }

// fp32 magnitude of the entries: 2^-log4(R) (regular) or fp32(1/sqrt(R)).
static float hd_mag(int rot) {
    if (pow4(rot)) {
        float m = 1.0f;
        for (int r = rot; r > 1; r >>= 2) m *= 0.5f;
        return m;
    }
    return (float)(1.0 / std::sqrt((double)rot));
}

// work-groups a launch aims at (four per CU: two resident, two queued)
constexpr int64_t XR_WGS = 1024;

static int small_grid(int64_t work) {
    return (int)std::max<int64_t>(1, std::min<int64_t>(cdiv(work, 256), 256 * 32));
}

static int rows_exact(const void* src, int dt, int64_t rows, int64_t cols, int64_t ld_src, float* dst,
                      int64_t cols_pad, int64_t ld_dst, int rot, float zero_above, unsigned long long* nz,
                      int64_t n_tri, hipStream_t st, int tag) {
    const float mag = hd_mag(rot);
    if (rot <= 8) {
        const int64_t groups = cols_pad / rot;
        const int grid = small_grid(rows * groups);
        ProfScope prof_scope(st, tag, 2.0 * rot * rows * cols_pad, 4.0 * rows * cols_pad + (dt ? 2.0 : 4.0) * rows * cols);
#define ICQ_SMALL(RR, D) hipLaunchKernelGGL((rot_rows_small_kernel<RR, D>), dim3(grid), dim3(256), 0, st, src, rows, \
                                            cols, ld_src, dst, groups, ld_dst, mag, zero_above, nz)
#define ICQ_SMALL_DT(RR) do { if (dt == IC_DTYPE_F32) ICQ_SMALL(RR, IC_DTYPE_F32); \
                              else if (dt == IC_DTYPE_BF16) ICQ_SMALL(RR, IC_DTYPE_BF16); \
                              else ICQ_SMALL(RR, IC_DTYPE_F16); } while (0)
        if (rot == 2) ICQ_SMALL_DT(2);
        else if (rot == 4) ICQ_SMALL_DT(4);
        else ICQ_SMALL_DT(8);
#undef ICQ_SMALL_DT
#undef ICQ_SMALL
        IC_CHECK_LAUNCH();
        return IC_OK;
    }
    const size_t esz = dt == IC_DTYPE_F32 ? 4 : 2;
    // bit 0: 16-byte (8-byte for 16-bit types) source loads; bit 1: 16-byte stores
    const int vec = (((uintptr_t)src % (4 * esz) == 0) && ((ld_src * esz) % (4 * esz) == 0) ? 1 : 0) |
                    (((uintptr_t)dst % 16 == 0) && (ld_dst % 4 == 0) ? 2 : 0);
    const bool tri = n_tri > 0;
    IC_REQUIRE(!tri || n_tri % XR_ROWS == 0, "rotate_exact: the triangle needs n % 64 == 0");
    IC_REQUIRE(cdiv(rows, XR_ROWS) < (1LL << 31) && cdiv(cols_pad, XR_SLICE) <= 65535, "rotate_exact: too large");
    // a few tiles per work-group, so that each one's loads overlap the previous one's MFMAs
    const int64_t ntile = cdiv(rows, XR_ROWS), slices = cdiv(cols_pad, XR_SLICE);
    const int64_t per = tri ? 4 : std::max<int64_t>(1, std::min<int64_t>(8, ntile * slices / XR_WGS));
    dim3 grid((unsigned)cdiv(ntile, per), (unsigned)slices);
    ProfScope prof_scope(st, tag, 2.0 * rot * rows * cols_pad * (tri ? 0.5 : 1.0),
                         4.0 * rows * cols_pad * (tri ? 0.5 : 1.0) + (double)esz * rows * cols * (tri ? 0.5 : 1.0));
    uint32_t mb;
    std::memcpy(&mb, &mag, 4);
#define ICQ_XR(RR, D, T) hipLaunchKernelGGL((rot_rows_exact_kernel<RR, D, T>), grid, dim3(256), 0, st, src, rows, \
                                            cols, ld_src, dst, cols_pad, ld_dst, n_tri, mb, zero_above, nz, vec)
#define ICQ_XR_DT(RR) do { if (tri) ICQ_XR(RR, IC_DTYPE_F32, true); \
                           else if (dt == IC_DTYPE_F32) ICQ_XR(RR, IC_DTYPE_F32, false); \
                           else if (dt == IC_DTYPE_BF16) ICQ_XR(RR, IC_DTYPE_BF16, false); \
                           else ICQ_XR(RR, IC_DTYPE_F16, false); } while (0)
    // rot_rows_wave_kernel's domain: out of place, whole groups, vector loads
    const bool wave = !tri && src != (const void*)dst && (vec & 1) && cols == cols_pad;
#define ICQ_XW(RR, D, Z) launch_rows_wave<RR, D, Z>(src, rows, cols, ld_src, dst, cols_pad, ld_dst, mb, zero_above, \
                                                    nz, vec, st)
#define ICQ_XW_Z(RR, D) do { if (zero_above > 0.0f) ICQ_XW(RR, D, true); else ICQ_XW(RR, D, false); } while (0)
#define ICQ_XW_DT(RR) do { if (dt == IC_DTYPE_F32) ICQ_XW_Z(RR, IC_DTYPE_F32); \
                           else if (dt == IC_DTYPE_BF16) ICQ_XW_Z(RR, IC_DTYPE_BF16); \
                           else ICQ_XW_Z(RR, IC_DTYPE_F16); } while (0)
    switch (rot) {
        case 16: ICQ_XR_DT(16); break;
        case 32: ICQ_XR_DT(32); break;
        case 64: if (wave) ICQ_XW_DT(64); else ICQ_XR_DT(64); break;
        case 128: if (wave) ICQ_XW_DT(128); else ICQ_XR_DT(128); break;
        case 256: if (wave) ICQ_XW_DT(256); else ICQ_XR_DT(256); break;
        default: ICQ_XR_DT(512); break;
    }
#undef ICQ_XW_DT
#undef ICQ_XW_Z
#undef ICQ_XW
#undef ICQ_XR_DT
#undef ICQ_XR
    IC_CHECK_LAUNCH();
    return IC_OK;
}

}  // namespace icq

using namespace icq;

extern "C" int ic_rotate_rows_exact(const void* src, int src_dtype, int64_t rows, int64_t cols, int64_t ld_src,
                                    float* dst, int64_t cols_pad, int64_t ld_dst, int rot, float zero_above,
                                    unsigned long long* n_zeroed, void* stream) {
    IC_REQUIRE(src && dst, "ic_rotate_rows_exact: null pointer");
    IC_REQUIRE(src_dtype >= 0 && src_dtype <= 2, "ic_rotate_rows_exact: bad dtype");
    IC_REQUIRE(rot >= 1 && rot <= 512 && pow2(rot), "ic_rotate_rows_exact: rot must be a power of 2 <= 512");
    IC_REQUIRE(rows >= 0 && cols >= 0 && cols_pad == cdiv(cols, rot) * rot, "ic_rotate_rows_exact: cols_pad mismatch");
    IC_REQUIRE(ld_src >= cols && ld_dst >= cols_pad, "ic_rotate_rows_exact: bad leading dimension");
    IC_REQUIRE(src != (const void*)dst || (src_dtype == IC_DTYPE_F32 && ld_src == ld_dst && rot <= 256),
               "ic_rotate_rows_exact: in place needs f32, equal ld and rot <= 256");
    if (rot == 1)
        return ic_rotate_rows(src, src_dtype, rows, cols, ld_src, dst, cols_pad, ld_dst, 1, zero_above, n_zeroed,
                              stream);
    if (rows == 0 || cols_pad == 0) return IC_OK;
    return rows_exact(src, src_dtype, rows, cols, ld_src, dst, cols_pad, ld_dst, rot, zero_above, n_zeroed, 0,
                      as_stream(stream), PT_ROTATE);
}

extern "C" int ic_rotate_hessian_exact(const float* src, float* H, int64_t batch, int64_t n, int64_t ld, int rot,
                                       int lower_only, void* stream) {
    IC_REQUIRE(src && H, "ic_rotate_hessian_exact: null pointer");
    IC_REQUIRE(rot == 1 || (pow4(rot) && rot <= 256), "ic_rotate_hessian_exact: rot must be 1, 4, 16, 64 or 256");
    IC_REQUIRE(batch >= 0 && n >= 0 && n % rot == 0 && ld >= n, "ic_rotate_hessian_exact: n must be a multiple of rot");
    IC_REQUIRE(!lower_only || batch == 1, "ic_rotate_hessian_exact: lower_only needs batch == 1");
    IC_REQUIRE(batch <= 65535, "ic_rotate_hessian_exact: batch too large");
    if (batch == 0 || n == 0) return IC_OK;
    hipStream_t st = as_stream(stream);
    if (rot == 1) {
        if (src != H)
            IC_CHECK_HIP(hipMemcpy2DAsync(H, ld * sizeof(float), src, ld * sizeof(float), n * sizeof(float),
                                          batch * n, hipMemcpyDeviceToDevice, st));
        return IC_OK;
    }
    const float mag = hd_mag(rot);
    const bool tri = lower_only && rot >= 16 && n % XR_ROWS == 0;   // else the full matrix (a superset)
    // left product: H <- R^T src (column pass; src -> H, or in place)
    if (rot == 4) {
        ProfScope prof_scope(st, PT_ROTATE_H, 2.0 * rot * batch * n * n, 8.0 * batch * n * n);
        hipLaunchKernelGGL((rot_cols_small_kernel<4>), dim3(small_grid(batch * (n / 4) * n)), dim3(256), 0, st, src,
                           H, batch, n, ld, n * ld, mag);
        IC_CHECK_LAUNCH();
    } else {
        IC_REQUIRE(cdiv(n, XC_COLS) < (1LL << 31) && cdiv(n, XC_ROWS) <= 65535, "ic_rotate_hessian_exact: too large");
        const int vec = (((uintptr_t)src % 16 == 0) && (ld % 4 == 0) ? 1 : 0) |
                        (((uintptr_t)H % 16 == 0) && (ld % 4 == 0) ? 2 : 0);
        uint32_t mb;
        std::memcpy(&mb, &mag, 4);
        const int64_t ntile = cdiv(n, XC_COLS), nrow = cdiv(n, XC_ROWS);
        const int64_t per = tri ? 4 : std::max<int64_t>(1, std::min<int64_t>(8, ntile * nrow * batch / XR_WGS));
        dim3 grid((unsigned)cdiv(ntile, per), (unsigned)nrow, (unsigned)batch);
        ProfScope prof_scope(st, PT_ROTATE_H, 2.0 * rot * batch * n * n * (tri ? 0.5 : 1.0),
                             8.0 * batch * n * n * (tri ? 0.5 : 1.0));
#define ICQ_XC(RR) do { if (tri) hipLaunchKernelGGL((rot_cols_exact_kernel<RR, true>), grid, dim3(256), 0, st, src, H, \
                                                    n, ld, n * ld, mb, vec); \
                        else hipLaunchKernelGGL((rot_cols_exact_kernel<RR, false>), grid, dim3(256), 0, st, src, H, \
                                                n, ld, n * ld, mb, vec); } while (0)
        if (rot == 16) ICQ_XC(16);
        else if (rot == 64) ICQ_XC(64);
        else ICQ_XC(256);
#undef ICQ_XC
        IC_CHECK_LAUNCH();
    }
    // right product: H <- H R (row pass, in place); batch * n rows of pitch ld
    return rows_exact(H, IC_DTYPE_F32, batch * n, n, ld, H, n, ld, rot, 0.0f, nullptr, tri ? n : 0, st,
                      PT_ROTATE_H);
}
