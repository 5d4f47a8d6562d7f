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

// Chunked form: each work-group streams one contiguous chunk of whole tiles
// (tile = 256 lanes x 16 B x UNROLL, one raw buffer resource per tile), the
// access shape of a decode split, with UNROLL non-temporal 16-byte loads per
// lane in flight. On MI355X 32 KB in flight per CU (one 4-wave group per CU,
// UNROLL = 8) reads ~7.3 TB/s, where the grid-stride form above tops out near
// 6.8 TB/s, so the ceiling is the best of both.
template <int UNROLL>
__global__ __launch_bounds__(256) void hbm_read_chunks(const uint8_t* __restrict__ src,
                                                       size_t tiles_per_group, float* __restrict__ sink) {
    constexpr uint32_t TILE = 256u * 16u * UNROLL;
    const uint8_t* base = src + (size_t)blockIdx.x * tiles_per_group * TILE;
    const uint32_t lane_off = threadIdx.x * 16u;
    uint32_t acc = 0;
    for (size_t k = 0; k < tiles_per_group; ++k) {
        const __amdgpu_buffer_rsrc_t r = make_rsrc(base + k * TILE, TILE);
        u32x4 v[UNROLL];
#pragma unroll
        for (int u = 0; u < UNROLL; ++u)
            v[u] = __builtin_amdgcn_raw_buffer_load_b128(r, lane_off + (uint32_t)u * 4096u, 0, VA_LOAD_AUX);
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    if (acc == 0x9E3779B9u) sink[0] = (float)acc;
}

hipError_t launch_probe_chunks(const void* src, size_t bytes, float* sink, int grid, int unroll,
                               hipStream_t stream, size_t* bytes_read) {
    const size_t tile = (size_t)4096 * (unroll == 8 ? 8 : 4);
    const size_t per = grid > 0 ? bytes / tile / (size_t)grid : 0;
    *bytes_read = per * (size_t)grid * tile;
    if (per == 0) return hipErrorInvalidValue;
    const uint8_t* p = static_cast<const uint8_t*>(src);
    if (unroll == 8) hipLaunchKernelGGL(hbm_read_chunks<8>, dim3(grid), dim3(256), 0, stream, p, per, sink);
    else hipLaunchKernelGGL(hbm_read_chunks<4>, dim3(grid), dim3(256), 0, stream, p, per, sink);
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
