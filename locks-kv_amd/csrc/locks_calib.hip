// Measurement helper: a plain streaming read, the practical HBM read ceiling
// for a launch that moves a given number of bytes on this part.  Benchmarks
// time it beside a kernel to separate the layout/compute cost from what any
// read of the same size achieves (fixed launch ramp + ~6.5 TB/s asymptote).
#include "locks_common.h"
#include "locks_hip.h"

namespace locks {

__global__ __launch_bounds__(256) void calib_read_kernel(const uint4* __restrict__ p, long n,
                                                         uint32_t* __restrict__ sink) {
    uint4 a = {0u, 0u, 0u, 0u};
    for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n; i += (long)gridDim.x * 256) {
        const uint4 w = p[i];
        a.x ^= w.x; a.y += w.y; a.z ^= w.z; a.w += w.w;
    }
    // data-dependent store keeps the loads; practically never taken
    if ((a.x ^ a.y ^ a.z ^ a.w) == 0x9e3779b9u) sink[0] = a.x;
}

}  // namespace locks

using namespace locks;

extern "C" int32_t locks_calib_read(const void* src, int64_t bytes, uint32_t* sink, void* stream) {
    LOCKS_REQUIRE(src && sink && bytes >= 16 && bytes % 16 == 0,
                  "locks_calib_read: need 16-byte multiples and non-null pointers");
    hipLaunchKernelGGL(calib_read_kernel, dim3(2048), dim3(256), 0, (hipStream_t)stream,
                       static_cast<const uint4*>(src), (long)(bytes / 16), sink);
    return check_launch("calib_read_kernel");
}
