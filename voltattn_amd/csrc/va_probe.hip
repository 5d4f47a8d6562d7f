// va_probe.hip — empirical HBM read ceiling (the MBU denominator).
// Reference: read_kernel + probe_ceiling, src/voltattn.cu:64-78, 935-957
// (a 256 MiB float4 grid-stride read). On MI355X a buffer that small would be
// served largely from the 256 MB Infinity Cache, so the caller sizes it at
// >= 4 GiB; the kernel reads it with 128-bit loads, UNROLL independent loads
// per lane in flight, and folds the values into a register that is written out
// only on an impossible value so the loads cannot be eliminated.
#include "va_device.hpp"
#include "va_kernels.hpp"

namespace va {

template <int UNROLL>
__global__ __launch_bounds__(256) void hbm_read_probe(const u32x4* __restrict__ src,
                                                      size_t n16, float* __restrict__ sink) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    uint32_t acc = 0;
    for (; i + (UNROLL - 1) * stride < n16; i += UNROLL * stride) {
        u32x4 v[UNROLL];
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) v[u] = __builtin_nontemporal_load(src + i + u * stride);
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    for (; i < n16; i += stride) {
        const u32x4 v = __builtin_nontemporal_load(src + i);
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    if (acc == 0x9E3779B9u) sink[0] = (float)acc;
}

hipError_t launch_probe(const void* src, size_t bytes, float* sink, int grid, int unroll,
                        hipStream_t stream) {
    const u32x4* p = static_cast<const u32x4*>(src);
    const size_t n16 = bytes / 16;
    switch (unroll) {
        case 4:  hipLaunchKernelGGL(hbm_read_probe<4>, dim3(grid), dim3(256), 0, stream, p, n16, sink); break;
        case 8:  hipLaunchKernelGGL(hbm_read_probe<8>, dim3(grid), dim3(256), 0, stream, p, n16, sink); break;
        default: hipLaunchKernelGGL(hbm_read_probe<2>, dim3(grid), dim3(256), 0, stream, p, n16, sink); break;
    }
    return hipGetLastError();
}

// Launch floor: the period of back-to-back launches of a kernel that does no
// work (its one store sits behind a flag the host never sets), i.e. the fixed
// cost every decode step pays before and after its work-groups run.
__global__ __launch_bounds__(256) void launch_floor_probe(float* sink, int flag) {
    if (flag == 0x5EED && blockIdx.x == 0 && threadIdx.x == 0) sink[0] = 1.f;
}

hipError_t launch_empty(int grid, float* sink, hipStream_t stream) {
    hipLaunchKernelGGL(launch_floor_probe, dim3(grid), dim3(256), 0, stream, sink, 0);
    return hipGetLastError();
}

} // namespace va
