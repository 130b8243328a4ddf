// Shared device/host helpers for the gfx950 kernels of the quantization path.
//
// Numerics contract: every file is compiled with -ffp-contract=off and
// IEEE-correct fp32 division, so a*b+c is two roundings unless a kernel asks
// for __builtin_fmaf explicitly, and x/y is the correctly rounded quotient.
// The bit-exact parts of the path (RTN codes, the in-block GPTQ/LDLQ sweep,
// packing) rely on this to reproduce the reference's fp32 roundings.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <hip/hip_bf16.h>
#include <stdint.h>
#include <type_traits>
#include <string>

#include "../../include/ic_abi.h"

namespace icq {

// ------------------------------------------------------------ error state

void set_error(const std::string& msg);
int fail(int code, const std::string& msg);

#define IC_CHECK_HIP(expr)                                                        \
    do {                                                                          \
        hipError_t e_ = (expr);                                                   \
        if (e_ != hipSuccess)                                                     \
            return ::icq::fail(IC_ERR_HIP, std::string(#expr " failed: ") +       \
                                               hipGetErrorString(e_));            \
    } while (0)

#define IC_CHECK_LAUNCH() IC_CHECK_HIP(hipGetLastError())

#define IC_REQUIRE(cond, msg)                                                     \
    do {                                                                          \
        if (!(cond)) return ::icq::fail(IC_ERR_ARG, msg);                         \
    } while (0)

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

__host__ __device__ inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// ------------------------------------------------------------ element access

__device__ __forceinline__ float load_as_f32(const void* p, int dtype, int64_t i) {
    if (dtype == IC_DTYPE_F32) return reinterpret_cast<const float*>(p)[i];
    uint16_t h = reinterpret_cast<const uint16_t*>(p)[i];
    if (dtype == IC_DTYPE_BF16) return __uint_as_float(uint32_t(h) << 16);
    return __half2float(__ushort_as_half(h));
}

// Round half away from zero exactly as floor(x + 0.5) / ceil(x - 0.5) in fp32.
// The +-0.5 is an fp32 addition (rounded), e.g. 0.49999997f -> 1.
__device__ __forceinline__ float rhaz(float x) {
    return x >= 0.0f ? floorf(x + 0.5f) : ceilf(x - 0.5f);
}

// Correctly rounded a / b from a precomputed y = RN(1/b) (an IEEE division):
// q0 = RN(a*y), r = a - b*q0 exactly (FMA), q = RN(q0 + r*y).  Markstein's
// theorem gives q == RN(a/b) when no intermediate over- or underflows, which
// holds for b in [2^-30, 2^31) and |a| in [2^-60, 2^61) (or a == 0, where
// only the sign of a zero result may differ).  Verified on the CPU against
// IEEE division on ~1e9 operand pairs of that domain.  Outside it, or when
// b_ok is false, the plain IEEE division is used.
__device__ __forceinline__ bool div_b_ok(float b) {
    return b >= 0x1p-30f && b < 0x1p31f;
}
// `needed` = false marks a lane whose result is discarded: it skips the
// domain test so that it cannot force the slow path on the wave.
__device__ __forceinline__ float div_rn(float a, float b, float y, bool b_ok, bool needed = true) {
    const float aa = fabsf(a);
    const bool ok = !needed || (b_ok && ((aa >= 0x1p-60f && aa < 0x1p61f) || aa == 0.0f));
    if (__builtin_expect(!ok, 0)) return a / b;
    const float q0 = a * y;
    const float r = __builtin_fmaf(-q0, b, a);
    return __builtin_fmaf(r, y, q0);
}

// div_rn for code where the domain test must not branch per lane: the fast
// path runs for every lane, and only if some lane of the wave is outside
// its domain (a wave-uniform test) do those lanes take the IEEE division.
// Same result as div_rn.
__device__ __forceinline__ float div_rn_wave(float a, float b, float y, bool b_ok) {
    const float q0 = a * y;
    const float r = __builtin_fmaf(-q0, b, a);
    float q = __builtin_fmaf(r, y, q0);
    const float aa = fabsf(a);
    const bool ok = b_ok && ((aa >= 0x1p-60f && aa < 0x1p61f) || aa == 0.0f);
    if (__builtin_expect(__builtin_amdgcn_ballot_w64(!ok) != 0, 0)) q = ok ? q : a / b;
    return q;
}

// The fast quotient alone, for callers that established the domain of
// div_rn beforehand (b_ok, and every a in [2^-60, 2^61) or 0).
__device__ __forceinline__ float div_rn_fast(float a, float b, float y) {
    const float q0 = a * y;
    const float r = __builtin_fmaf(-q0, b, a);
    return __builtin_fmaf(r, y, q0);
}

// |a| in the numerator domain of div_rn: [2^-60, 2^61) or 0.
__device__ __forceinline__ bool div_a_ok(float a) {
    const float aa = fabsf(a);
    return (aa >= 0x1p-60f && aa < 0x1p61f) || aa == 0.0f;
}

// rhaz with fewer operations: trunc(x + copysign(0.5, x)).  For x >= 0
// this is floor(x + 0.5) (x + 0.5 > 0); for x < 0 ceil(x - 0.5).  The one
// difference is x = -0.0, which gives -0.0 instead of +0.0: an equal code
// (same int8, same products and sums), so no result can tell them apart.
__device__ __forceinline__ float rhaz_trunc(float x) {
    return truncf(x + __builtin_copysignf(0.5f, x));
}

// Work-group barrier for waves that hand data to each other only through
// LDS: each waits for its own LDS operations and no more (__syncthreads()
// also waits for outstanding global memory operations, e.g. loads issued
// early to hide their latency, or stores that only later kernels read).
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Orders a wave's own LDS accesses (exchanges between its lanes), with no
// work-group barrier.
__device__ __forceinline__ void lds_wave_fence() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// f(std::integral_constant<int, i>) for i = I .. N-1: a loop whose index
// is a compile-time constant in the body (register-array slots).
template <int I, int N, typename F>
__device__ __forceinline__ void static_for(F& f) {
    if constexpr (I < N) {
        f(std::integral_constant<int, I>{});
        static_for<I + 1, N>(f);
    }
}

// Lane P's value of v in every lane of its DPP quad (lanes 4k .. 4k+3).
template <int P>
__device__ __forceinline__ float quad_bcast(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), P * 0x55, 0xf, 0xf, false));
}

// clampf as a median of three (NaN still propagates).
__device__ __forceinline__ float clampf_med3(float x, float lo, float hi) {
    return x != x ? x : __builtin_amdgcn_fmed3f(x, lo, hi);
}

// Round half to even (torch.round).
__device__ __forceinline__ float rhte(float x) { return rintf(x); }

__device__ __forceinline__ float clampf(float x, float lo, float hi) {
    // torch.clamp(x, lo, hi) = min(max(x, lo), hi); NaN propagates.
    return x != x ? x : fminf(fmaxf(x, lo), hi);
}

// fp32 -> fp16 with round-to-nearest-even (matches tensor.to(torch.float16)).
__device__ __forceinline__ uint16_t f32_to_f16_bits(float x) {
    return __half_as_ushort(__float2half_rn(x));
}
__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) {
    return __half2float(__ushort_as_half(h));
}

// Total-order key of an fp32 value so that unsigned comparisons order floats.
__device__ __forceinline__ uint32_t float_key(float x) {
    uint32_t u = __float_as_uint(x);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float key_float(uint32_t k) {
    uint32_t u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
    return __uint_as_float(u);
}

// ------------------------------------------------------------ wave reductions

template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}
__device__ __forceinline__ float wave_min(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fminf(v, __shfl_xor(v, o, 64));
    return v;
}

}  // namespace icq
