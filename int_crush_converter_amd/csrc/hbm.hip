// Streaming kernels that measure the HBM ceiling of the box the library runs
// on (bench.py --hbm-ceiling): the bandwidth the path's HBM-bound kernels
// are compared with.  Every access is a 16-byte vector, consecutive lanes
// touch consecutive 16-byte words, and each thread keeps four loads in
// flight per grid-stride step.
#include "common.hpp"

namespace icq {
namespace {

typedef float f4 __attribute__((ext_vector_type(4)));
typedef unsigned int u4 __attribute__((ext_vector_type(4)));
constexpr int HU = 4;   // 16-byte loads in flight per thread and step

// kind 0: dst = src (copy); 1: read src (a data-dependent store of one value
// that never happens keeps the loads); 2: write dst; 3: bf16 src -> fp32 dst
// (16 bytes read, 32 written per lane and element group)
template <int KIND>
__global__ __launch_bounds__(256) void stream_kernel(const u4* __restrict__ s, f4* __restrict__ d, int64_t n,
                                                     float* sink) {
    const int64_t stride = (int64_t)gridDim.x * 256 * HU;
    float acc = 0.0f;
    for (int64_t i = (int64_t)blockIdx.x * 256 * HU + threadIdx.x; i < n; i += stride) {
        u4 v[HU];
        if (KIND != 2) {
#pragma unroll
            for (int u = 0; u < HU; ++u) v[u] = i + 256 * u < n ? s[i + 256 * u] : u4{0, 0, 0, 0};
        }
#pragma unroll
        for (int u = 0; u < HU; ++u) {
            const int64_t k = i + 256 * u;
            if (k >= n) continue;
            if (KIND == 0) {
                d[k] = f4{__uint_as_float(v[u][0]), __uint_as_float(v[u][1]), __uint_as_float(v[u][2]),
                          __uint_as_float(v[u][3])};
            } else if (KIND == 1) {
                acc += __uint_as_float(v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3]);
            } else if (KIND == 2) {
                d[k] = f4{1.0f, 2.0f, 3.0f, (float)k};
            } else {
                f4 a, b;
#pragma unroll
                for (int q = 0; q < 2; ++q) {
                    a[2 * q] = __uint_as_float(v[u][q] << 16);
                    a[2 * q + 1] = __uint_as_float(v[u][q] & 0xffff0000u);
                    b[2 * q] = __uint_as_float(v[u][q + 2] << 16);
                    b[2 * q + 1] = __uint_as_float(v[u][q + 2] & 0xffff0000u);
                }
                d[2 * k] = a;
                d[2 * k + 1] = b;
            }
        }
    }
    if (KIND == 1 && acc == 1.2345e-31f) sink[0] = acc;
}

}  // namespace
}  // namespace icq

using namespace icq;

// bytes: the source size (kinds 0, 1, 3) or the destination size (kind 2),
// a multiple of 16; kind 3's destination holds 2 x bytes.
extern "C" int ic_hbm_stream(int kind, const void* src, void* dst, int64_t bytes, void* stream) {
    IC_REQUIRE(kind >= 0 && kind <= 3, "ic_hbm_stream: kind must be 0..3");
    IC_REQUIRE(bytes >= 0 && bytes % 16 == 0, "ic_hbm_stream: bytes must be a multiple of 16");
    IC_REQUIRE((kind == 2 || src) && (kind == 1 || dst) && (kind != 1 || dst),
               "ic_hbm_stream: null pointer");
    if (bytes == 0) return IC_OK;
    const int64_t n = bytes / 16;
    const int grid = 8192;
    hipStream_t st = as_stream(stream);
    const u4* s = reinterpret_cast<const u4*>(src);
    f4* d = reinterpret_cast<f4*>(dst);
    float* sink = reinterpret_cast<float*>(dst);
    switch (kind) {
        case 0: hipLaunchKernelGGL(stream_kernel<0>, dim3(grid), dim3(256), 0, st, s, d, n, sink); break;
        case 1: hipLaunchKernelGGL(stream_kernel<1>, dim3(grid), dim3(256), 0, st, s, d, n, sink); break;
        case 2: hipLaunchKernelGGL(stream_kernel<2>, dim3(grid), dim3(256), 0, st, s, d, n, sink); break;
        default: hipLaunchKernelGGL(stream_kernel<3>, dim3(grid), dim3(256), 0, st, s, d, n, sink); break;
    }
    IC_CHECK_LAUNCH();
    return IC_OK;
}
