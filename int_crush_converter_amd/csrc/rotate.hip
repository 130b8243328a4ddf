// Group-wise Hadamard rotation (ConvRot) as a fast Walsh-Hadamard transform.
//
// Regular Hadamard of size 4^k is (H4/2)^{kron k}; applying it to a group of
// 4^k values is k radix-4 stages, one per base-4 digit of the index:
//     y_d = S/2 - x_{3-d},   S = (x_0 + x_1) + (x_2 + x_3).
// Sylvester (other powers of 2) is radix-2 +-1 stages followed by one scale
// by fp32(1/sqrt(n)).  Both replace the dense `x @ H.T` of
// converter/rotation.py:82-125 with 2 log4(n) flops per element instead of 2n.
//
// Register kernel (rot 4/16/64/256): each lane owns 16 consecutive columns
// (base-4 digits 0 and 1 of the in-group index live in registers), digit 2
// spans the 4 lanes of a quad and digit 3 the 16 lanes of a row of 16, both
// exchanged with cross-lane shuffles.  A wave therefore streams 64x16
// contiguous elements per step: coalesced 64-byte-per-lane loads and stores.
//
// LDS kernel (any power of 2 up to 4096, and the column pass of R^T H R):
// a [rot x TC] tile is staged in LDS and transformed stage by stage.
#include "common.hpp"
#include "prof.hpp"

namespace icq {

// s * 0.5 is exact, so fma(s, 0.5, -x) is the reference's RN(S/2 - x).
__device__ __forceinline__ void bfly4(float& a, float& b, float& c, float& d) {
    const float s = (a + b) + (c + d);
    const float na = __builtin_fmaf(s, 0.5f, -d), nb = __builtin_fmaf(s, 0.5f, -c);
    const float nc = __builtin_fmaf(s, 0.5f, -b), nd = __builtin_fmaf(s, 0.5f, -a);
    a = na; b = nb; c = nc; d = nd;
}

// One radix-4 stage across the 4 lanes of a quad (the digit value is the
// lane's position in the quad; the partner of digit d is 3 - d = d ^ 3).
// DPP quad permutations keep the exchange in the VALU.
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xf, 0xf, true));
}
constexpr int QP_XOR1 = 0xB1;   // quad_perm(1,0,3,2)
constexpr int QP_XOR2 = 0x4E;   // quad_perm(2,3,0,1)
constexpr int QP_XOR3 = 0x1B;   // quad_perm(3,2,1,0)

__device__ __forceinline__ float bfly4_quad(float v) {
    const float a = v + dpp<QP_XOR1>(v);            // (x0 + x1) or (x2 + x3)
    const float s = a + dpp<QP_XOR2>(a);            // (x0 + x1) + (x2 + x3)
    return __builtin_fmaf(s, 0.5f, -dpp<QP_XOR3>(v));
}

// Outlier sanitising on load (converter/pipeline.py:527-537): |w| > zero_above
// (when zero_above > 0) becomes 0 before rotation; the count goes to *nz.
__device__ __forceinline__ float sanitize(float v, float zero_above, unsigned& cnt) {
    if (zero_above > 0.0f && fabsf(v) > zero_above) { ++cnt; return 0.0f; }
    return v;
}

// Same, for a lane's whole register block: the outlier count is taken per
// wave from the comparison masks (one scalar popcount per element).
template <int K>
__device__ __forceinline__ void sanitize_block(float (&v)[K], float zero_above, unsigned& cnt) {
    if (!(zero_above > 0.0f)) return;
    unsigned wc = 0;
#pragma unroll
    for (int i = 0; i < K; ++i) {
        const bool out = fabsf(v[i]) > zero_above;
        wc += (unsigned)__popcll(__ballot(out));
        v[i] = out ? 0.0f : v[i];
    }
    if ((threadIdx.x & 63) == 0) cnt += wc;   // counted once per wave
}

__device__ __forceinline__ void flush_count(unsigned cnt, unsigned long long* nz) {
    if (!nz) return;
    unsigned long long c = wave_sum((unsigned long long)cnt);
    if ((threadIdx.x & 63) == 0 && c) atomicAdd(nz, c);
}

typedef float floatx4_t __attribute__((ext_vector_type(4)));
typedef unsigned int uintx4_t __attribute__((ext_vector_type(4)));

// 16 consecutive source elements -> fp32 (FAST: 16-byte loads, no bounds).
template <int DT, bool FAST>
__device__ __forceinline__ void load16(const void* src, int64_t base, int64_t c0, int64_t cols, float (&v)[16]) {
    if (FAST) {
        if (DT == IC_DTYPE_F32) {
            const floatx4_t* p = reinterpret_cast<const floatx4_t*>(reinterpret_cast<const float*>(src) + base);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const floatx4_t t = p[i];
                v[4 * i] = t[0]; v[4 * i + 1] = t[1]; v[4 * i + 2] = t[2]; v[4 * i + 3] = t[3];
            }
        } else {
            const uintx4_t* p = reinterpret_cast<const uintx4_t*>(reinterpret_cast<const uint16_t*>(src) + base);
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const uintx4_t t = p[i];
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    if (DT == IC_DTYPE_BF16) {
                        v[8 * i + 2 * k] = __uint_as_float(t[k] << 16);
                        v[8 * i + 2 * k + 1] = __uint_as_float(t[k] & 0xffff0000u);
                    } else {
                        v[8 * i + 2 * k] = f16_bits_to_f32((uint16_t)(t[k] & 0xffffu));
                        v[8 * i + 2 * k + 1] = f16_bits_to_f32((uint16_t)(t[k] >> 16));
                    }
                }
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) v[i] = (c0 + i < cols) ? load_as_f32(src, DT, base + i) : 0.0f;
    }
}

// Rotation of groups of ROT in {4, 16, 64, 256} columns, entirely in
// registers and DPP.  FAST: 16-byte aligned rows made of whole 16-column
// chunks (no bounds checks); DT: the source dtype.  A lane holds NCH chunks of 16 consecutive columns:
// base-4 digits 0 and 1 of the in-group index are the register index inside
// a chunk; for ROT >= 64 digit 2 is the lane's position in its quad; for
// ROT = 256 digit 3 is the chunk (the quad's lane j holds columns
// 16 j + 64 m, m < 4, of its 256-column group).  Item = one thread's
// chunks; threads 4q .. 4q+3 cover one 64- (or 256-) column group.
template <int ROT, int DT, bool FAST>
__global__ __launch_bounds__(256) void rotate_rows_reg(
    const void* __restrict__ src, int64_t rows, int64_t cols, int64_t ld_src,
    float* __restrict__ dst, int64_t cols_pad, int64_t ld_dst, float zero_above,
    unsigned long long* nz) {
    constexpr int NCH = ROT == 256 ? 4 : 1;
    unsigned cnt = 0;
    // per row: units of 16 columns per thread (256 per quad for ROT = 256)
    const uint32_t upr = (uint32_t)(ROT == 256 ? cols_pad / 256 : cols_pad / 16);
    const uint32_t total = (uint32_t)rows * upr * (ROT == 256 ? 4u : 1u);   // threads' items
    const uint32_t stride = gridDim.x * blockDim.x;
    for (uint32_t g = blockIdx.x * blockDim.x + threadIdx.x; g < total; g += stride) {
        uint32_t r, c0;
        if (ROT == 256) {
            const uint32_t u = g >> 2;
            r = u / upr;
            c0 = (u - r * upr) * 256 + 16 * (g & 3);
        } else {
            r = g / upr;
            c0 = (g - r * upr) * 16;
        }
        float v[NCH][16];
#pragma unroll
        for (int m = 0; m < NCH; ++m) {
            const int64_t cm = (int64_t)c0 + 64 * m;
            load16<DT, FAST>(src, (int64_t)r * ld_src + cm, cm, cols, v[m]);
            sanitize_block(v[m], zero_above, cnt);
            // digit 0 (stride 1), digit 1 (stride 4)
#pragma unroll
            for (int a = 0; a < 4; ++a) bfly4(v[m][4 * a], v[m][4 * a + 1], v[m][4 * a + 2], v[m][4 * a + 3]);
            if (ROT >= 16) {
#pragma unroll
                for (int b = 0; b < 4; ++b) bfly4(v[m][b], v[m][b + 4], v[m][b + 8], v[m][b + 12]);
            }
            // digit 2 (the quad)
            if (ROT >= 64) {
#pragma unroll
                for (int i = 0; i < 16; ++i) v[m][i] = bfly4_quad(v[m][i]);
            }
        }
        // digit 3 (the chunks)
        if (ROT == 256) {
#pragma unroll
            for (int i = 0; i < 16; ++i) bfly4(v[0][i], v[1 % NCH][i], v[2 % NCH][i], v[3 % NCH][i]);
        }
#pragma unroll
        for (int m = 0; m < NCH; ++m) {
            float* o = dst + (int64_t)r * ld_dst + c0 + 64 * m;
            if (FAST) {
                floatx4_t* q = reinterpret_cast<floatx4_t*>(o);
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    q[i] = floatx4_t{v[m][4 * i], v[m][4 * i + 1], v[m][4 * i + 2], v[m][4 * i + 3]};
            } else {
#pragma unroll
                for (int i = 0; i < 16; ++i) o[i] = v[m][i];
            }
        }
    }
    flush_count(cnt, nz);
}

// Rotation of 256-column groups with fully coalesced accesses (rows made of
// whole 16-byte aligned groups).  A wave takes four (row, group) items at
// a time, one per 16-lane row of the wave: lane p (< 16) of a row holds the
// in-group columns 64 i + 4 p + e (i, e < 4), so every load and store
// instruction moves 16 contiguous lanes x 16 bytes (fp32) or 8 bytes
// (bf16 / fp16) per item.  The base-4 digits of the in-group index are e
// (digit 0, in registers), p & 3 (digit 1, the quad: DPP quad permutes),
// p >> 2 (digit 2, the 16-lane row: DPP mirrors composed with quad
// permutes) and i (digit 3, in registers); the stages run in that order,
// with the same additions as rotate_rows_reg, whose results they equal.
template <int CTRL1, int CTRL2>
__device__ __forceinline__ float dpp2(float v) {
    return dpp<CTRL2>(dpp<CTRL1>(v));
}
constexpr int ROW_MIRROR = 0x140, ROW_HALF_MIRROR = 0x141;

// One radix-4 stage across lanes p ^ 4, p ^ 8, p ^ 12 of a 16-lane row:
// p ^ 7 (half mirror) then ^ 3 gives p ^ 4; p ^ 15 (mirror) then ^ 7 gives
// p ^ 8; p ^ 15 then ^ 3 gives p ^ 12.
__device__ __forceinline__ float bfly4_row(float v) {
    const float a = v + dpp2<ROW_HALF_MIRROR, QP_XOR3>(v);
    const float s = a + dpp2<ROW_MIRROR, ROW_HALF_MIRROR>(a);
    return __builtin_fmaf(s, 0.5f, -dpp2<ROW_MIRROR, QP_XOR3>(v));
}

template <int DT>
__device__ __forceinline__ void load4(const void* src, int64_t off, float (&v)[4]) {
    if (DT == IC_DTYPE_F32) {
        const floatx4_t t = *reinterpret_cast<const floatx4_t*>(reinterpret_cast<const float*>(src) + off);
        v[0] = t[0]; v[1] = t[1]; v[2] = t[2]; v[3] = t[3];
    } else {
        typedef unsigned int uintx2_t __attribute__((ext_vector_type(2)));
        const uintx2_t t = *reinterpret_cast<const uintx2_t*>(reinterpret_cast<const uint16_t*>(src) + off);
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            if (DT == IC_DTYPE_BF16) {
                v[2 * k] = __uint_as_float(t[k] << 16);
                v[2 * k + 1] = __uint_as_float(t[k] & 0xffff0000u);
            } else {
                v[2 * k] = f16_bits_to_f32((uint16_t)(t[k] & 0xffffu));
                v[2 * k + 1] = f16_bits_to_f32((uint16_t)(t[k] >> 16));
            }
        }
    }
}

template <int DT>
__global__ __launch_bounds__(256) void rotate256_coal(const void* __restrict__ src, int64_t rows, int64_t groups,
                                                      int64_t ld_src, float* __restrict__ dst, int64_t ld_dst,
                                                      float zero_above, unsigned long long* nz) {
    unsigned cnt = 0;
    const int lane = threadIdx.x & 63, p = lane & 15, u = lane >> 4;
    const int64_t items = rows * groups;
    const int64_t nwave = (int64_t)gridDim.x * 4;
    // every lane of a wave runs the same number of iterations (the DPP
    // exchanges need the whole row of 16 lanes): items past the end are
    // clamped to the last one and not stored
    for (int64_t w0 = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * 4; w0 < items; w0 += nwave * 4) {
        const bool live = w0 + u < items;
        const int64_t it = live ? w0 + u : items - 1;
        const int64_t r = it / groups, g = it - r * groups;
        const int64_t so = r * ld_src + g * 256 + 4 * p, doff = r * ld_dst + g * 256 + 4 * p;
        float v[4][4];
#pragma unroll
        for (int i = 0; i < 4; ++i) load4<DT>(src, so + 64 * i, v[i]);
        if (zero_above > 0.0f) {
            // outliers zeroed; counted once per wave, clamped items excluded
            unsigned wc = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const bool out = fabsf(v[i][e]) > zero_above;
                    wc += (unsigned)__popcll(__ballot(out && live));
                    v[i][e] = out ? 0.0f : v[i][e];
                }
            if (lane == 0) cnt += wc;
        }
        // digit 0
#pragma unroll
        for (int i = 0; i < 4; ++i) bfly4(v[i][0], v[i][1], v[i][2], v[i][3]);
        // digit 1 (the quad), digit 2 (the row of 16)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e) v[i][e] = bfly4_quad(v[i][e]);
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e) v[i][e] = bfly4_row(v[i][e]);
        // digit 3
#pragma unroll
        for (int e = 0; e < 4; ++e) bfly4(v[0][e], v[1][e], v[2][e], v[3][e]);
        if (live) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
                *reinterpret_cast<floatx4_t*>(dst + doff + 64 * i) = floatx4_t{v[i][0], v[i][1], v[i][2], v[i][3]};
        }
    }
    flush_count(cnt, nz);
}

// Column pass of R^T H R for groups of 256 rows: in place on fp32 [n, n]
// matrices.  Work-group: one 256-row group x 64 columns; thread (c, q)
// (c = t % 64 the column, q = t / 64 the wave) loads rows 64 q .. 64 q + 63 of
// its column (a wave reads 64 consecutive floats of a row per load), applies
// digits 0-2 of the row index in registers, and hands digit 3 (the wave)
// through LDS: after one exchange thread (c, q) finishes rows 16 q + i +
// 64 m (i < 16, m < 4).  Same stages, in the same order, as the row kernel.
constexpr int CP_COLS = 64;
constexpr int CP_PITCH = CP_COLS + 1;

__global__ __launch_bounds__(256) void rotate_cols256_kernel(float* __restrict__ H, int64_t n, int64_t ld,
                                                             int64_t bstride) {
    __shared__ float tile[256 * CP_PITCH];
    float* P = H + (int64_t)blockIdx.z * bstride + (int64_t)blockIdx.y * 256 * ld + (int64_t)blockIdx.x * CP_COLS;
    const int t = threadIdx.x, c = t & 63, q = t >> 6;
    const bool cv = (int64_t)blockIdx.x * CP_COLS + c < n;
    float v[64];
#pragma unroll
    for (int i = 0; i < 64; ++i) v[i] = cv ? P[(int64_t)(64 * q + i) * ld + c] : 0.0f;
    // digit 0 (stride 1), digit 1 (stride 4), digit 2 (stride 16)
#pragma unroll
    for (int a = 0; a < 16; ++a) bfly4(v[4 * a], v[4 * a + 1], v[4 * a + 2], v[4 * a + 3]);
#pragma unroll
    for (int h = 0; h < 4; ++h)
#pragma unroll
        for (int b = 0; b < 4; ++b) bfly4(v[16 * h + b], v[16 * h + b + 4], v[16 * h + b + 8], v[16 * h + b + 12]);
#pragma unroll
    for (int b = 0; b < 16; ++b) bfly4(v[b], v[b + 16], v[b + 32], v[b + 48]);
#pragma unroll
    for (int i = 0; i < 64; ++i) tile[(64 * q + i) * CP_PITCH + c] = v[i];
    __syncthreads();
    // digit 3 (stride 64): rows r, r+64, r+128, r+192 for r = 16 q + i
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int r = 16 * q + i;
        float x0 = tile[r * CP_PITCH + c], x1 = tile[(r + 64) * CP_PITCH + c];
        float x2 = tile[(r + 128) * CP_PITCH + c], x3 = tile[(r + 192) * CP_PITCH + c];
        bfly4(x0, x1, x2, x3);
        if (cv) {
            P[(int64_t)r * ld + c] = x0;
            P[(int64_t)(r + 64) * ld + c] = x1;
            P[(int64_t)(r + 128) * ld + c] = x2;
            P[(int64_t)(r + 192) * ld + c] = x3;
        }
    }
}

// Convert + zero-pad copy into fp32 (used before the LDS kernel).
__global__ void convert_pad_kernel(const void* __restrict__ src, int dtype, int64_t rows, int64_t cols,
                                   int64_t ld_src, float* __restrict__ dst, int64_t cols_pad, int64_t ld_dst,
                                   float zero_above, unsigned long long* nz) {
    const int64_t total = rows * cols_pad;
    unsigned cnt = 0;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        int64_t r = i / cols_pad, c = i - r * cols_pad;
        dst[r * ld_dst + c] = c < cols ? sanitize(load_as_f32(src, dtype, r * ld_src + c), zero_above, cnt) : 0.0f;
    }
    flush_count(cnt, nz);
}

// In-place transform of tiles [rot along axis A] x [tc along axis B] of an
// fp32 array.  Element (a, b) of tile (ta, tb) of batch z lives at
//   p + z*bstride + (ta*rot + a)*sa + (tb*tc + b)*sb.
// Grid: x = tiles along B, y = tiles along A (groups), z = batch.
// Loads go in the order that is contiguous in memory (sa==1 or sb==1).
__global__ __launch_bounds__(256) void rotate_lds_kernel(
    float* __restrict__ p, int rot, int tc, int64_t nb_valid, int64_t sa, int64_t sb, int64_t bstride,
    int regular, float scale) {
    extern __shared__ float tile[];  // [rot][tc + 1]
    const int pitch = tc + 1;
    float* base = p + (int64_t)blockIdx.z * bstride + (int64_t)blockIdx.y * rot * sa +
                  (int64_t)blockIdx.x * tc * sb;
    const int bvalid = (int)min<int64_t>(tc, nb_valid - (int64_t)blockIdx.x * tc);
    const int n = rot * tc;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        int a, b;
        if (sa == 1) { b = i / rot; a = i - b * rot; } else { a = i / tc; b = i - a * tc; }
        tile[a * pitch + b] = b < bvalid ? base[(int64_t)a * sa + (int64_t)b * sb] : 0.0f;
    }
    __syncthreads();
    if (regular) {
        for (int st = 1; st < rot; st *= 4) {
            const int nq = (rot / 4) * tc;
            for (int i = threadIdx.x; i < nq; i += blockDim.x) {
                int b = i % tc, q = i / tc;
                int hi = q / st, lo = q - hi * st;
                int a0 = hi * st * 4 + lo;
                float x0 = tile[a0 * pitch + b], x1 = tile[(a0 + st) * pitch + b];
                float x2 = tile[(a0 + 2 * st) * pitch + b], x3 = tile[(a0 + 3 * st) * pitch + b];
                bfly4(x0, x1, x2, x3);
                tile[a0 * pitch + b] = x0; tile[(a0 + st) * pitch + b] = x1;
                tile[(a0 + 2 * st) * pitch + b] = x2; tile[(a0 + 3 * st) * pitch + b] = x3;
            }
            __syncthreads();
        }
    } else {
        for (int st = 1; st < rot; st *= 2) {
            const int nq = (rot / 2) * tc;
            for (int i = threadIdx.x; i < nq; i += blockDim.x) {
                int b = i % tc, q = i / tc;
                int hi = q / st, lo = q - hi * st;
                int a0 = hi * st * 2 + lo;
                float x0 = tile[a0 * pitch + b], x1 = tile[(a0 + st) * pitch + b];
                tile[a0 * pitch + b] = x0 + x1;
                tile[(a0 + st) * pitch + b] = x0 - x1;
            }
            __syncthreads();
        }
    }
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        int a, b;
        if (sa == 1) { b = i / rot; a = i - b * rot; } else { a = i / tc; b = i - a * tc; }
        if (b < bvalid) {
            float v = tile[a * pitch + b];
            base[(int64_t)a * sa + (int64_t)b * sb] = regular ? v : v * scale;
        }
    }
}

static bool is_pow2(int64_t n) { return n > 0 && (n & (n - 1)) == 0; }
static bool is_pow4(int64_t n) { return n >= 4 && is_pow2(n) && (n & 0x55555555) == n; }

static int grid_for(int64_t work, int threads) {
    int64_t b = cdiv(work, threads);
    return (int)std::min<int64_t>(std::max<int64_t>(b, 1), 256 * 64);
}

static int launch_lds(float* p, int rot, int64_t groups, int64_t nb, int64_t sa, int64_t sb, int64_t batch,
                      int64_t bstride, hipStream_t st) {
    int tc = (int)std::max<int64_t>(1, std::min<int64_t>(32, 8192 / rot));
    size_t lds = (size_t)rot * (tc + 1) * sizeof(float);
    int regular = is_pow4(rot) ? 1 : 0;
    float scale = regular ? 1.0f : (float)(1.0 / std::sqrt((double)rot));
    dim3 grid((unsigned)cdiv(nb, tc), (unsigned)groups, (unsigned)batch);
    ProfScope prof_scope(st, PT_ROTATE_H, 2.0 * batch * groups * rot * nb * std::log2((double)rot),
                 8.0 * batch * groups * rot * nb);
    hipLaunchKernelGGL(rotate_lds_kernel, grid, dim3(256), lds, st, p, rot, tc, nb, sa, sb, bstride,
                       regular, scale);
    IC_CHECK_LAUNCH();
    return IC_OK;
}

}  // namespace icq

using namespace icq;

// Row rotation; `tag` is the profiler phase (weights or the Hessian's row pass).
static int rotate_rows(const void* src, int src_dtype, int64_t rows, int64_t cols, int64_t ld_src, float* dst,
                       int64_t cols_pad, int64_t ld_dst, int rot, float zero_above, unsigned long long* n_zeroed,
                       void* stream, int tag) {
    IC_REQUIRE(src && dst, "ic_rotate_rows: null pointer");
    IC_REQUIRE(src_dtype >= 0 && src_dtype <= 2, "ic_rotate_rows: bad dtype");
    IC_REQUIRE(rot >= 1 && rot <= 4096 && is_pow2(rot), "ic_rotate_rows: rot must be a power of 2 <= 4096");
    IC_REQUIRE(cols_pad == cdiv(cols, rot) * rot, "ic_rotate_rows: cols_pad mismatch");
    IC_REQUIRE(ld_src >= cols && ld_dst >= cols_pad, "ic_rotate_rows: bad leading dimension");
    IC_REQUIRE(src != (const void*)dst || (src_dtype == IC_DTYPE_F32 && ld_src == ld_dst),
               "ic_rotate_rows: in-place needs f32 and equal ld");
    if (rows == 0 || cols_pad == 0) return IC_OK;
    hipStream_t st = as_stream(stream);
    {
        const size_t esz = src_dtype == IC_DTYPE_F32 ? 4 : 2;
        const bool coal = rot == 256 && cols == cols_pad && ((uintptr_t)src % 16 == 0) &&
                          ((ld_src * esz) % 16 == 0) && ((uintptr_t)dst % 16 == 0) && (ld_dst % 4 == 0);
        if (coal) {
            const int64_t groups = cols / 256, items = rows * groups;
            const int grid = (int)std::max<int64_t>(1, std::min<int64_t>(cdiv(items, 16), 4096));
            ProfScope prof_scope(st, tag, 8.0 * rows * cols_pad, (double)rows * cols * esz + 4.0 * rows * cols_pad);
            if (src_dtype == IC_DTYPE_F32)
                hipLaunchKernelGGL(rotate256_coal<IC_DTYPE_F32>, dim3(grid), dim3(256), 0, st, src, rows, groups,
                                   ld_src, dst, ld_dst, zero_above, n_zeroed);
            else if (src_dtype == IC_DTYPE_BF16)
                hipLaunchKernelGGL(rotate256_coal<IC_DTYPE_BF16>, dim3(grid), dim3(256), 0, st, src, rows, groups,
                                   ld_src, dst, ld_dst, zero_above, n_zeroed);
            else
                hipLaunchKernelGGL(rotate256_coal<IC_DTYPE_F16>, dim3(grid), dim3(256), 0, st, src, rows, groups,
                                   ld_src, dst, ld_dst, zero_above, n_zeroed);
            IC_CHECK_LAUNCH();
            return IC_OK;
        }
    }
    if (rot >= 4 && rot <= 256 && is_pow4(rot) && cols_pad % 16 == 0 && rows * (cols_pad / 16) < (1LL << 31)) {
        size_t esz = src_dtype == IC_DTYPE_F32 ? 4 : 2;
        bool vec_ok = ((uintptr_t)src % 16 == 0) && ((ld_src * esz) % 16 == 0) && ((uintptr_t)dst % 16 == 0) &&
                      (ld_dst % 4 == 0);
        int64_t chunks = rows * (cols_pad / 16);   // one 16-column chunk per thread and pass
        // rot 256: a few items per thread (8 work-groups of 256 per CU)
        int grid = rot == 256 ? (int)std::min<int64_t>(grid_for(chunks / 4, 256), 2048) : grid_for(chunks, 256);
        int stages = rot == 4 ? 1 : rot == 16 ? 2 : rot == 64 ? 3 : 4;
        ProfScope prof_scope(st, tag, 2.0 * stages * rows * cols_pad,
                     (double)rows * cols * esz + 4.0 * rows * cols_pad);
        const bool fast = vec_ok && cols % 16 == 0;
#define ICQ_ROT_LAUNCH(R, D, F)                                                                               \
    hipLaunchKernelGGL((rotate_rows_reg<R, D, F>), dim3(grid), dim3(256), 0, st, src, rows, cols, ld_src, dst, \
                       cols_pad, ld_dst, zero_above, n_zeroed)
#define ICQ_ROT_DT(R)                                                                                          \
    do {                                                                                                       \
        if (src_dtype == IC_DTYPE_F32) { if (fast) ICQ_ROT_LAUNCH(R, IC_DTYPE_F32, true); else ICQ_ROT_LAUNCH(R, IC_DTYPE_F32, false); } \
        else if (src_dtype == IC_DTYPE_BF16) { if (fast) ICQ_ROT_LAUNCH(R, IC_DTYPE_BF16, true); else ICQ_ROT_LAUNCH(R, IC_DTYPE_BF16, false); } \
        else { if (fast) ICQ_ROT_LAUNCH(R, IC_DTYPE_F16, true); else ICQ_ROT_LAUNCH(R, IC_DTYPE_F16, false); } \
    } while (0)
        switch (rot) {
            case 4: ICQ_ROT_DT(4); break;
            case 16: ICQ_ROT_DT(16); break;
            case 64: ICQ_ROT_DT(64); break;
            default: ICQ_ROT_DT(256); break;
        }
#undef ICQ_ROT_DT
#undef ICQ_ROT_LAUNCH
        IC_CHECK_LAUNCH();
        return IC_OK;
    }
    // generic: convert/pad into dst, then transform in place in LDS
    if (!(src == (const void*)dst && cols == cols_pad && zero_above <= 0.0f)) {
        hipLaunchKernelGGL(convert_pad_kernel, dim3(grid_for(rows * cols_pad, 256)), dim3(256), 0, st, src,
                           src_dtype, rows, cols, ld_src, dst, cols_pad, ld_dst, zero_above, n_zeroed);
        IC_CHECK_LAUNCH();
    }
    if (rot == 1) return IC_OK;
    // axis A = columns (stride 1), axis B = rows (stride ld_dst); grid.z kept 1
    return launch_lds(dst, rot, cols_pad / rot, rows, 1, ld_dst, 1, 0, st);
}

extern "C" int ic_rotate_rows(const void* src, int src_dtype, int64_t rows, int64_t cols, int64_t ld_src,
                              float* dst, int64_t cols_pad, int64_t ld_dst, int rot, float zero_above,
                              unsigned long long* n_zeroed, void* stream) {
    return rotate_rows(src, src_dtype, rows, cols, ld_src, dst, cols_pad, ld_dst, rot, zero_above, n_zeroed,
                       stream, PT_ROTATE);
}

extern "C" int ic_rotate_hessian(const float* src, float* H, int64_t batch, int64_t n, int64_t ld, int rot,
                                 void* stream) {
    IC_REQUIRE(src && H, "ic_rotate_hessian: null pointer");
    IC_REQUIRE(rot >= 1 && rot <= 4096 && is_pow2(rot), "ic_rotate_hessian: rot must be a power of 2 <= 4096");
    IC_REQUIRE(n % rot == 0 && ld >= n, "ic_rotate_hessian: n must be a multiple of rot");
    if (batch == 0 || n == 0) return IC_OK;
    hipStream_t st = as_stream(stream);
    if (rot == 1) {
        if (src != H)
            IC_CHECK_HIP(hipMemcpy2DAsync(H, ld * sizeof(float), src, ld * sizeof(float), n * sizeof(float),
                                          batch * n, hipMemcpyDeviceToDevice, st));
        return IC_OK;
    }
    // rows: H <- src R (the copy out of src is this pass); the batch is
    // batch*n consecutive rows of pitch ld
    int rc = rotate_rows(src, IC_DTYPE_F32, batch * n, n, ld, H, n, ld, rot, 0.0f, nullptr, stream, PT_ROTATE_H);
    if (rc) return rc;
    // columns: H <- R^T H
    if (rot == 256) {
        ProfScope prof_scope(st, PT_ROTATE_H, 2.0 * 4 * batch * n * n, 8.0 * batch * n * n);
        dim3 grid((unsigned)cdiv(n, CP_COLS), (unsigned)(n / 256), (unsigned)batch);
        hipLaunchKernelGGL(rotate_cols256_kernel, grid, dim3(256), 0, st, H, n, ld, n * ld);
        IC_CHECK_LAUNCH();
        return IC_OK;
    }
    // axis A = rows (stride ld), axis B = columns (stride 1)
    return launch_lds(H, rot, n / rot, n, ld, 1, batch, n * ld, st);
}
