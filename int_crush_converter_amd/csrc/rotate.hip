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

__device__ __forceinline__ void bfly4(float& a, float& b, float& c, float& d) {
    float s = (a + b) + (c + d);
    float h = s * 0.5f;
    float na = h - d, nb = h - c, nc = h - b, nd = h - a;
    a = na; b = nb; c = nc; d = nd;
}

// One radix-4 stage across the 4 lanes selected by xor masks m1, m2 (partner
// of digit value d is 3-d = d ^ 3, i.e. xor (m1|m2)).
template <int M1, int M2>
__device__ __forceinline__ float bfly4_x(float v) {
    float a = v + __shfl_xor(v, M1, 64);
    float s = a + __shfl_xor(a, M2, 64);
    float p = __shfl_xor(v, M1 | M2, 64);
    return s * 0.5f - p;
}

// Outlier sanitising on load (converter/pipeline.py:527-537): |w| > zero_above
// (when zero_above > 0) becomes 0 before rotation; the count goes to *nz.
__device__ __forceinline__ float sanitize(float v, float zero_above, unsigned& cnt) {
    if (zero_above > 0.0f && fabsf(v) > zero_above) { ++cnt; return 0.0f; }
    return v;
}

__device__ __forceinline__ void flush_count(unsigned cnt, unsigned long long* nz) {
    if (!nz) return;
    unsigned long long c = wave_sum((unsigned long long)cnt);
    if ((threadIdx.x & 63) == 0 && c) atomicAdd(nz, c);
}

template <int ROT>
__global__ __launch_bounds__(256) void rotate_rows_reg(
    const void* __restrict__ src, int dtype, int64_t rows, int64_t cols, int64_t ld_src,
    float* __restrict__ dst, int64_t cols_pad, int64_t ld_dst, int vec_ok, float zero_above,
    unsigned long long* nz) {
    unsigned cnt = 0;
    const int64_t cpr = cols_pad >> 4;  // 16-column chunks per row
    const int64_t total = rows * cpr;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; g < total; g += stride) {
        const int64_t r = g / cpr;
        const int64_t c0 = (g - r * cpr) << 4;
        float v[16];
        const int64_t base = r * ld_src + c0;
        if (vec_ok && c0 + 16 <= cols) {
            if (dtype == IC_DTYPE_F32) {
                const float4* p = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(src) + base);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    float4 t = p[i];
                    v[4 * i] = t.x; v[4 * i + 1] = t.y; v[4 * i + 2] = t.z; v[4 * i + 3] = t.w;
                }
            } else {
                const uint4* p = reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(src) + base);
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    uint4 t = p[i];
                    uint32_t w[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        uint16_t lo = (uint16_t)(w[k] & 0xffffu), hi = (uint16_t)(w[k] >> 16);
                        if (dtype == IC_DTYPE_BF16) {
                            v[8 * i + 2 * k] = __uint_as_float(uint32_t(lo) << 16);
                            v[8 * i + 2 * k + 1] = __uint_as_float(uint32_t(hi) << 16);
                        } else {
                            v[8 * i + 2 * k] = f16_bits_to_f32(lo);
                            v[8 * i + 2 * k + 1] = f16_bits_to_f32(hi);
                        }
                    }
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < 16; ++i)
                v[i] = (c0 + i < cols) ? load_as_f32(src, dtype, base + i) : 0.0f;
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) v[i] = sanitize(v[i], zero_above, cnt);
        // digit 0 (stride 1)
#pragma unroll
        for (int a = 0; a < 4; ++a) bfly4(v[4 * a], v[4 * a + 1], v[4 * a + 2], v[4 * a + 3]);
        if (ROT >= 16) {
#pragma unroll
            for (int b = 0; b < 4; ++b) bfly4(v[b], v[b + 4], v[b + 8], v[b + 12]);
        }
        if (ROT >= 64) {
#pragma unroll
            for (int i = 0; i < 16; ++i) v[i] = bfly4_x<1, 2>(v[i]);
        }
        if (ROT >= 256) {
#pragma unroll
            for (int i = 0; i < 16; ++i) v[i] = bfly4_x<4, 8>(v[i]);
        }
        float* o = dst + r * ld_dst + c0;
        if (vec_ok) {
            float4* q = reinterpret_cast<float4*>(o);
#pragma unroll
            for (int i = 0; i < 4; ++i) q[i] = make_float4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
        } else {
#pragma unroll
            for (int i = 0; i < 16; ++i) o[i] = v[i];
        }
    }
    flush_count(cnt, nz);
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

extern "C" int ic_rotate_rows(const void* src, int src_dtype, int64_t rows, int64_t cols, int64_t ld_src,
                              float* dst, int64_t cols_pad, int64_t ld_dst, int rot, float zero_above,
                              unsigned long long* n_zeroed, void* stream) {
    IC_REQUIRE(src && dst, "ic_rotate_rows: null pointer");
    IC_REQUIRE(src_dtype >= 0 && src_dtype <= 2, "ic_rotate_rows: bad dtype");
    IC_REQUIRE(rot >= 1 && rot <= 4096 && is_pow2(rot), "ic_rotate_rows: rot must be a power of 2 <= 4096");
    IC_REQUIRE(cols_pad == cdiv(cols, rot) * rot, "ic_rotate_rows: cols_pad mismatch");
    IC_REQUIRE(ld_src >= cols && ld_dst >= cols_pad, "ic_rotate_rows: bad leading dimension");
    IC_REQUIRE(src != (const void*)dst || (src_dtype == IC_DTYPE_F32 && ld_src == ld_dst),
               "ic_rotate_rows: in-place needs f32 and equal ld");
    if (rows == 0 || cols_pad == 0) return IC_OK;
    hipStream_t st = as_stream(stream);
    if (rot >= 4 && rot <= 256 && is_pow4(rot) && cols_pad % 16 == 0) {
        size_t esz = src_dtype == IC_DTYPE_F32 ? 4 : 2;
        bool vec_ok = ((uintptr_t)src % 16 == 0) && ((ld_src * esz) % 16 == 0) && ((uintptr_t)dst % 16 == 0) &&
                      (ld_dst % 4 == 0);
        int64_t chunks = rows * (cols_pad / 16);
        int grid = grid_for(chunks, 256);
        int stages = rot == 4 ? 1 : rot == 16 ? 2 : rot == 64 ? 3 : 4;
        ProfScope prof_scope(st, src == (const void*)dst ? PT_ROTATE_H : PT_ROTATE, 2.0 * stages * rows * cols_pad,
                     (double)rows * cols * esz + 4.0 * rows * cols_pad);
        switch (rot) {
            case 4: hipLaunchKernelGGL(rotate_rows_reg<4>, dim3(grid), dim3(256), 0, st, src, src_dtype, rows, cols, ld_src, dst, cols_pad, ld_dst, (int)vec_ok, zero_above, n_zeroed); break;
            case 16: hipLaunchKernelGGL(rotate_rows_reg<16>, dim3(grid), dim3(256), 0, st, src, src_dtype, rows, cols, ld_src, dst, cols_pad, ld_dst, (int)vec_ok, zero_above, n_zeroed); break;
            case 64: hipLaunchKernelGGL(rotate_rows_reg<64>, dim3(grid), dim3(256), 0, st, src, src_dtype, rows, cols, ld_src, dst, cols_pad, ld_dst, (int)vec_ok, zero_above, n_zeroed); break;
            default: hipLaunchKernelGGL(rotate_rows_reg<256>, dim3(grid), dim3(256), 0, st, src, src_dtype, rows, cols, ld_src, dst, cols_pad, ld_dst, (int)vec_ok, zero_above, n_zeroed); break;
        }
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

extern "C" int ic_rotate_hessian(float* H, int64_t batch, int64_t n, int64_t ld, int rot, void* stream) {
    IC_REQUIRE(H, "ic_rotate_hessian: null pointer");
    IC_REQUIRE(rot >= 1 && rot <= 4096 && is_pow2(rot), "ic_rotate_hessian: rot must be a power of 2 <= 4096");
    IC_REQUIRE(n % rot == 0 && ld >= n, "ic_rotate_hessian: n must be a multiple of rot");
    if (batch == 0 || n == 0 || rot == 1) return IC_OK;
    hipStream_t st = as_stream(stream);
    // rows: H <- H R; the batch is batch*n consecutive rows of pitch ld
    int rc = ic_rotate_rows(H, IC_DTYPE_F32, batch * n, n, ld, H, n, ld, rot, 0.0f, nullptr, stream);
    if (rc) return rc;
    // columns: H <- R^T H; axis A = rows (stride ld), axis B = columns (stride 1)
    return launch_lds(H, rot, n / rot, n, ld, 1, batch, n * ld, st);
}
