// va_probe.hip — empirical HBM read ceiling (the MBU denominator).
// Reference: read_kernel + probe_ceiling, src/voltattn.cu:64-78, 935-957
// (a 256 MiB float4 grid-stride read). On MI355X a buffer that small would be
// served largely from the 256 MB Infinity Cache, so the caller sizes it at
// >= 4 GiB; the kernels read it with 128-bit loads, UNROLL independent loads
// per lane in flight.
//
// Every probe launch writes a digest per work-group: the XOR of every 16-byte
// word the group loaded and the number of 16-byte loads it issued. The digest
// is stored unconditionally, so no load can be eliminated, and a host that
// knows the buffer's contents can check that a form reads exactly the bytes it
// is credited with (va_probe_digest).
#include "va_device.hpp"
#include "va_kernels.hpp"

namespace va {

// Wave-wide XOR and sum: rotations inside each 16-lane DPP row, then the
// gfx950 row swaps (v_permlane16_swap / v_permlane32_swap) across rows; every
// lane gets the result.
template <bool XOR>
__device__ __forceinline__ uint32_t wave_fold(uint32_t x) {
    auto op = [](uint32_t a, uint32_t b) { return XOR ? a ^ b : a + b; };
    x = op(x, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, dpp_row_ror(8), 0xF, 0xF, false));
    x = op(x, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, dpp_row_ror(4), 0xF, 0xF, false));
    x = op(x, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, dpp_row_ror(2), 0xF, 0xF, false));
    x = op(x, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, dpp_row_ror(1), 0xF, 0xF, false));
    unsigned a = x, b = x;
    permlane16_swap(a, b);
    x = op(a, b);
    a = x;
    b = x;
    permlane32_swap(a, b);
    return op(a, b);
}

// Fold the work-group's (xor, count) into its digest slot
// dig[blockIdx.x] = {x, y, z, w, loads, 0, 0, 0}: wave folds, one LDS entry per
// wave, one 32-byte store by thread 0. (LDS atomics from every lane measured
// ~10 us per launch here: the compiler serialises them lane by lane.)
__device__ __forceinline__ void store_digest(const u32x4& acc, uint32_t loads, uint32_t* dig) {
    __shared__ uint32_t s_d[4][5];
    const uint32_t d0 = wave_fold<true>(acc.x), d1 = wave_fold<true>(acc.y);
    const uint32_t d2 = wave_fold<true>(acc.z), d3 = wave_fold<true>(acc.w);
    const uint32_t n = wave_fold<false>(loads);
    const int w = (int)(threadIdx.x >> 6);
    if ((threadIdx.x & 63) == 0) {
        s_d[w][0] = d0; s_d[w][1] = d1; s_d[w][2] = d2; s_d[w][3] = d3; s_d[w][4] = n;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        u32x4 x = {0u, 0u, 0u, 0u};
        uint32_t c = 0;
        for (int i = 0; i < (int)(blockDim.x >> 6); ++i) {
            x ^= u32x4{s_d[i][0], s_d[i][1], s_d[i][2], s_d[i][3]};
            c += s_d[i][4];
        }
        u32x4* out = reinterpret_cast<u32x4*>(dig + (size_t)blockIdx.x * PROBE_DIGEST_WORDS);
        out[0] = x;
        out[1] = u32x4{c, 0u, 0u, 0u};
    }
}

// Grid-stride form (the reference's read_kernel shape): thread i reads words
// i, i + stride, ... of the n16 16-byte words.
template <int UNROLL>
__global__ __launch_bounds__(256) void hbm_read_probe(const u32x4* __restrict__ src,
                                                      size_t n16, uint32_t* __restrict__ dig) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    u32x4 acc = {0u, 0u, 0u, 0u};
    uint32_t loads = 0;
    for (; i + (UNROLL - 1) * stride < n16; i += UNROLL * stride) {
        u32x4 v[UNROLL];
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) v[u] = __builtin_nontemporal_load(src + i + u * stride);
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) acc ^= v[u];
        loads += UNROLL;
    }
    for (; i < n16; i += stride) {
        acc ^= __builtin_nontemporal_load(src + i);
        ++loads;
    }
    store_digest(acc, loads, dig);
}

hipError_t launch_probe(const void* src, size_t bytes, uint32_t* dig, int grid, int unroll,
                        hipStream_t stream) {
    const u32x4* p = static_cast<const u32x4*>(src);
    const size_t n16 = bytes / 16;
    switch (unroll) {
        case 4:  hipLaunchKernelGGL(hbm_read_probe<4>, dim3(grid), dim3(256), 0, stream, p, n16, dig); break;
        case 8:  hipLaunchKernelGGL(hbm_read_probe<8>, dim3(grid), dim3(256), 0, stream, p, n16, dig); break;
        default: hipLaunchKernelGGL(hbm_read_probe<2>, dim3(grid), dim3(256), 0, stream, p, n16, dig); break;
    }
    return hipGetLastError();
}

// Chunked form: work-group g streams its own contiguous chunk
// [g*per, min(bytes, (g+1)*per)) (per a multiple of 16 bytes) in tiles of
// 256 lanes x 16 B x UNROLL, with UNROLL non-temporal 16-byte loads per lane
// in flight: the access shape of a decode split. One raw buffer resource
// covers the chunk, so loads of the last, partial tile that fall past its end
// return zeros without a memory access and are not counted. On MI355X one
// 4-wave group per CU with UNROLL = 8 (32 KB in flight per CU) reads ~7.3 TB/s,
// where the grid-stride form above tops out near 6.8 TB/s.
template <int UNROLL>
__global__ __launch_bounds__(256) void hbm_read_chunks(const uint8_t* __restrict__ src, size_t bytes,
                                                       uint32_t per, uint32_t* __restrict__ dig) {
    constexpr uint32_t TILE = 256u * 16u * UNROLL;
    const size_t start = (size_t)blockIdx.x * per;
    const uint32_t mine = start >= bytes ? 0u : (uint32_t)min((size_t)per, bytes - start);
    const __amdgpu_buffer_rsrc_t r = make_rsrc(src + (start < bytes ? start : 0), mine);
    const uint32_t lane_off = threadIdx.x * 16u;
    const uint32_t ntiles = (mine + TILE - 1) / TILE;
    u32x4 acc = {0u, 0u, 0u, 0u};
    uint32_t loads = 0;
    for (uint32_t k = 0; k < ntiles; ++k) {
        // the whole offset is in the VGPR operand, which the range check covers
        const uint32_t off = k * TILE + lane_off;
        u32x4 v[UNROLL];
#pragma unroll
        for (int u = 0; u < UNROLL; ++u)
            v[u] = __builtin_amdgcn_raw_buffer_load_b128(r, off + (uint32_t)u * 4096u, 0, VA_LOAD_AUX);
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
            acc ^= v[u];
            loads += off + (uint32_t)u * 4096u < mine ? 1u : 0u;
        }
    }
    store_digest(acc, loads, dig);
}

// Bytes per work-group of the chunked form over `bytes` with `grid` groups:
// ceil(bytes / grid) rounded up to 16.
size_t probe_chunk_bytes(size_t bytes, int grid) {
    if (grid <= 0) return 0;
    const size_t per = (bytes + (size_t)grid - 1) / (size_t)grid;
    return (per + 15) & ~(size_t)15;
}

hipError_t launch_probe_chunks(const void* src, size_t bytes, uint32_t* dig, int grid, int unroll,
                               hipStream_t stream) {
    const size_t per = probe_chunk_bytes(bytes, grid);
    if (per == 0 || per > 0x7FFFFFFFu || bytes % 16) return hipErrorInvalidValue;
    const uint8_t* p = static_cast<const uint8_t*>(src);
    if (unroll == 8) hipLaunchKernelGGL(hbm_read_chunks<8>, dim3(grid), dim3(256), 0, stream, p, bytes, (uint32_t)per, dig);
    else hipLaunchKernelGGL(hbm_read_chunks<4>, dim3(grid), dim3(256), 0, stream, p, bytes, (uint32_t)per, dig);
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
