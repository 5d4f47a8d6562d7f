// va_quant.hip — device-side producers of the decode path's inputs:
//   * quantize_groups / append_groups: the symmetric per-group quantizer +
//     packer (over fp32 rows, or over fp16 rows written into a paged cache at
//     given positions: the cache write path), bit-exact
//     with the reference's host quantize() (src/voltattn.cu:705-745) for
//     G in {32, 64}: amax in fp32, s = amax/lim (IEEE division), the fp16
//     scale rounded to nearest even, codes clamp(rint(x / float(scale))), with
//     a non-finite quotient giving code 0 as x86-64 lrint + int truncation does;
//   * dequantize_groups: the inverse, packed codes and fp16 scales back to
//     fp32 values, bit-exact with the reference's dq() (src/voltattn.cu:747-767);
//   * f32_to_f16: round-to-nearest-even conversion of fp32 arrays (the
//     reference's __float2half over the f16-format K/V, src/voltattn.cu:866-868);
//   * fill_normal: seeded N(0,1) bench data, Philox4x32-10 (Salmon et al.,
//     SC'11) counters through the Box-Muller transform.
#include "va_device.hpp"
#include "va_kernels.hpp"

namespace va {

template <int BITS> struct QLim;
template <> struct QLim<8> { static constexpr int value = 127; };
template <> struct QLim<4> { static constexpr int value = 7; };
template <> struct QLim<3> { static constexpr int value = 3; };

// Quantize and pack one group of G values (fp32 in registers) to `dst`
// (G*BITS/8 bytes, 4-byte aligned) and its fp16 scale to `*scale`.
template <int BITS, int G>
__device__ __forceinline__ void quant_group(const float (&xv)[G], uint8_t* dst, uint16_t* scale) {
    constexpr int lim = QLim<BITS>::value;
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < G; ++i) amax = fmaxf(amax, __builtin_fabsf(xv[i]));
    const float s = amax > 0.f ? amax / (float)lim : 1.f;
    const uint16_t sb = f2h_rne(s);
    const float sh = h2f(sb);
    int code[G];
#pragma unroll
    for (int i = 0; i < G; ++i) {
        const float t = xv[i] / sh;
        int v = __builtin_isfinite(t) ? (int)__builtin_rintf(t) : 0;
        v = v < -lim ? -lim : (v > lim ? lim : v);
        code[i] = v;
    }
    *scale = sb;
    uint32_t* d32 = reinterpret_cast<uint32_t*>(dst);
    if constexpr (BITS == 8) {
#pragma unroll
        for (int k = 0; k < G / 4; ++k) {
            uint32_t w = 0;
#pragma unroll
            for (int b = 0; b < 4; ++b) w |= (uint32_t)(uint8_t)(int8_t)code[4 * k + b] << (8 * b);
            d32[k] = w;
        }
    } else if constexpr (BITS == 4) {             // element i: byte i/2, low nibble when i even
#pragma unroll
        for (int k = 0; k < G / 8; ++k) {
            uint32_t w = 0;
#pragma unroll
            for (int i = 0; i < 8; ++i) w |= (uint32_t)(code[8 * k + i] + 8) << (4 * i);
            d32[k] = w;
        }
    } else {                                       // element i: bits [3i, 3i+3), little endian
        constexpr int NW = 3 * G / 32;
        uint32_t w[NW];
#pragma unroll
        for (int k = 0; k < NW; ++k) w[k] = 0;
#pragma unroll
        for (int i = 0; i < G; ++i) {
            const uint32_t c = (uint32_t)(code[i] + 4);
            const int b = 3 * i;
            w[b / 32] |= c << (b % 32);
            if (b % 32 > 29) w[b / 32 + 1] |= c >> (32 - b % 32);
        }
#pragma unroll
        for (int k = 0; k < NW; ++k) d32[k] = w[k];
    }
}

// One thread per quantization group of G consecutive elements. Groups are
// contiguous: group r*(D/G) + g starts at element (r*(D/G) + g) * G.
template <int BITS, int G>
__global__ __launch_bounds__(256) void quantize_groups(const float* __restrict__ x, size_t ngroups,
                                                       uint8_t* __restrict__ packed,
                                                       uint16_t* __restrict__ scales) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t gi = (size_t)blockIdx.x * blockDim.x + threadIdx.x; gi < ngroups; gi += stride) {
        const f32x4* xp = reinterpret_cast<const f32x4*>(x + gi * G);
        float xv[G];
#pragma unroll
        for (int c = 0; c < G / 4; ++c) {
            const f32x4 w = xp[c];
            xv[4 * c] = w.x; xv[4 * c + 1] = w.y; xv[4 * c + 2] = w.z; xv[4 * c + 3] = w.w;
        }
        quant_group<BITS, G>(xv, packed + gi * (G * BITS / 8), scales + gi);
    }
}

// Inverse of the packer, one thread per group: value = float(scale) * code.
// The reference's dq() forms the same product in double; an fp16 scale times a
// code of at most 7 bits is exact in fp32 (non-finite scales give the same
// inf/NaN), so the results are equal bit for bit. Code layouts as in
// quant_group: q8 int8, q4 nibble + 8 (low nibble first), q3 3-bit fields + 4.
template <int BITS, int G>
__global__ __launch_bounds__(256) void dequantize_groups(const uint8_t* __restrict__ packed,
                                                         const uint16_t* __restrict__ scales,
                                                         size_t ngroups, float* __restrict__ out) {
    constexpr int NW = G * BITS / 32;              // packed words per group
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t gi = (size_t)blockIdx.x * blockDim.x + threadIdx.x; gi < ngroups; gi += stride) {
        const uint32_t* src = reinterpret_cast<const uint32_t*>(packed + gi * (G * BITS / 8));
        uint32_t w[NW];
#pragma unroll
        for (int k = 0; k < NW; ++k) w[k] = src[k];
        const float s = h2f(scales[gi]);
        float v[G];
#pragma unroll
        for (int i = 0; i < G; ++i) {
            int c;
            if constexpr (BITS == 8) {
                c = (int)(int8_t)(uint8_t)(w[i / 4] >> (8 * (i % 4)));
            } else if constexpr (BITS == 4) {
                c = (int)((w[i / 8] >> (4 * (i % 8))) & 15u) - 8;
            } else {
                const int b = 3 * i;
                uint32_t f = w[b / 32] >> (b % 32);
                if (b % 32 > 29) f |= w[b / 32 + 1] << (32 - b % 32);
                c = (int)(f & 7u) - 4;
            }
            v[i] = s * (float)c;
        }
        f32x4* dst = reinterpret_cast<f32x4*>(out + gi * G);
#pragma unroll
        for (int k = 0; k < G / 4; ++k) dst[k] = f32x4{v[4 * k], v[4 * k + 1], v[4 * k + 2], v[4 * k + 3]};
    }
}

// Destination row of (sequence b, KV head hk, position p) in a page pool
// [num_pages][hkv][page_rows][...], or -1 when the position lies past the
// block table or on a page id outside the pool (such rows are not written).
__device__ __forceinline__ long long paged_row(const AppendArgs& a, int b, int hk, int p) {
    if (p < 0) return -1;
    const int pi = p / a.page_rows;
    if (pi >= a.max_pages) return -1;
    const int page = a.block_table[(size_t)b * a.max_pages + pi];
    if (page < 0 || page >= a.num_pages) return -1;
    return ((long long)page * a.hkv + hk) * a.page_rows + (p - pi * a.page_rows);
}

// Quantize-and-append: one thread per (b, hk, r, group) of the new rows
// x[b][hk][r][D] (fp16), written at position start[b] + r.
template <int BITS, int G>
__global__ __launch_bounds__(256) void append_groups(AppendArgs a, size_t ngroups) {
    const int NG = a.D / G;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t gi = (size_t)blockIdx.x * blockDim.x + threadIdx.x; gi < ngroups; gi += stride) {
        const int g = (int)(gi % NG);
        size_t rest = gi / NG;
        const int r = (int)(rest % a.n);
        rest /= a.n;
        const int hk = (int)(rest % a.hkv);
        const int b  = (int)(rest / a.hkv);
        const long long row = paged_row(a, b, hk, a.start[b] + r);
        if (row < 0) continue;
        const u32x4* xp = reinterpret_cast<const u32x4*>(a.x + gi * G);   // G fp16 values
        float xv[G];
#pragma unroll
        for (int c = 0; c < G / 8; ++c) {
            const u32x4 w = xp[c];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                xv[8 * c + 2 * k]     = h2f_lo(w[k]);
                xv[8 * c + 2 * k + 1] = h2f_hi(w[k]);
            }
        }
        quant_group<BITS, G>(xv, a.pages + (size_t)row * (a.D * BITS / 8) + (size_t)g * (G * BITS / 8),
                             a.scales + (size_t)row * NG + g);
    }
}

// f16 append: one thread per 8 values (16 bytes) of the new rows.
__global__ __launch_bounds__(256) void append_f16(AppendArgs a, size_t nchunks) {
    const int CPR = a.D / 8;                       // 16-byte chunks per row
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t ci = (size_t)blockIdx.x * blockDim.x + threadIdx.x; ci < nchunks; ci += stride) {
        const int c = (int)(ci % CPR);
        size_t rest = ci / CPR;
        const int r = (int)(rest % a.n);
        rest /= a.n;
        const int hk = (int)(rest % a.hkv);
        const int b  = (int)(rest / a.hkv);
        const long long row = paged_row(a, b, hk, a.start[b] + r);
        if (row < 0) continue;
        const u32x4 w = reinterpret_cast<const u32x4*>(a.x)[ci];
        reinterpret_cast<u32x4*>(a.pages + (size_t)row * (a.D * 2))[c] = w;
    }
}

__global__ __launch_bounds__(256) void f32_to_f16_kernel(const float* __restrict__ x, size_t n,
                                                         uint16_t* __restrict__ out) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        out[i] = f2h_rne(x[i]);
}

// Philox4x32-10 block: counter (c0..c3), key (k0, k1).
__device__ __forceinline__ u32x4 philox4x32_10(u32x4 c, uint32_t k0, uint32_t k1) {
    constexpr uint32_t M0 = 0xD2511F53u, M1 = 0xCD9E8D57u;
    constexpr uint32_t W0 = 0x9E3779B9u, W1 = 0xBB67AE85u;
#pragma unroll
    for (int r = 0; r < 10; ++r) {
        const uint32_t hi0 = __umulhi(M0, c.x), lo0 = M0 * c.x;
        const uint32_t hi1 = __umulhi(M1, c.z), lo1 = M1 * c.z;
        c = u32x4{hi1 ^ c.y ^ k0, lo1, hi0 ^ c.w ^ k1, lo0};
        k0 += W0;
        k1 += W1;
    }
    return c;
}

__global__ __launch_bounds__(256) void fill_normal_kernel(float* __restrict__ x, size_t n,
                                                          uint32_t k0, uint32_t k1) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    const size_t nblk = (n + 3) / 4;
    for (size_t b = (size_t)blockIdx.x * blockDim.x + threadIdx.x; b < nblk; b += stride) {
        const u32x4 r = philox4x32_10(u32x4{(uint32_t)b, (uint32_t)(b >> 32), 0u, 0u}, k0, k1);
        float z[4];
#pragma unroll
        for (int p = 0; p < 2; ++p) {
            const uint32_t a = p ? r.z : r.x, c = p ? r.w : r.y;
            const float u1 = (float)((a >> 8) + 1u) * 5.9604644775390625e-8f;  // (0, 1]
            const float u2 = (float)(c >> 8) * 5.9604644775390625e-8f;         // [0, 1)
            const float rad = sqrtf(-2.f * logf(u1));
            float sn, cs;
            sincosf(6.28318530717958648f * u2, &sn, &cs);
            z[2 * p] = rad * cs;
            z[2 * p + 1] = rad * sn;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (4 * b + i < n) x[4 * b + i] = z[i];
    }
}

static unsigned grid_for(size_t work) {
    const size_t blocks = (work + 255) / 256;
    return (unsigned)(blocks < 16384 ? (blocks ? blocks : 1) : 16384);
}

hipError_t launch_quantize(int bits, int G, const float* x, size_t rows, int D, uint8_t* packed,
                           uint16_t* scales, hipStream_t stream) {
    const size_t ngroups = rows * (size_t)(D / G);
    const dim3 grid(grid_for(ngroups)), block(256);
#define VA_QLAUNCH(B, GG) hipLaunchKernelGGL((quantize_groups<B, GG>), grid, block, 0, stream, x, ngroups, packed, scales)
    if (G == 32) {
        if (bits == 8) VA_QLAUNCH(8, 32); else if (bits == 4) VA_QLAUNCH(4, 32); else VA_QLAUNCH(3, 32);
    } else {
        if (bits == 8) VA_QLAUNCH(8, 64); else if (bits == 4) VA_QLAUNCH(4, 64); else VA_QLAUNCH(3, 64);
    }
#undef VA_QLAUNCH
    return hipGetLastError();
}

hipError_t launch_dequantize(int bits, int G, const uint8_t* packed, const uint16_t* scales, size_t rows,
                             int D, float* out, hipStream_t stream) {
    const size_t ngroups = rows * (size_t)(D / G);
    const dim3 grid(grid_for(ngroups)), block(256);
#define VA_DLAUNCH(B, GG) hipLaunchKernelGGL((dequantize_groups<B, GG>), grid, block, 0, stream, packed, scales, ngroups, out)
    if (G == 32) {
        if (bits == 8) VA_DLAUNCH(8, 32); else if (bits == 4) VA_DLAUNCH(4, 32); else VA_DLAUNCH(3, 32);
    } else {
        if (bits == 8) VA_DLAUNCH(8, 64); else if (bits == 4) VA_DLAUNCH(4, 64); else VA_DLAUNCH(3, 64);
    }
#undef VA_DLAUNCH
    return hipGetLastError();
}

hipError_t launch_append(int bits, int G, const AppendArgs& a, hipStream_t stream) {
    const size_t rows = (size_t)a.B * a.hkv * a.n;
    if (bits == 16) {
        const size_t nch = rows * (size_t)(a.D / 8);
        hipLaunchKernelGGL(append_f16, dim3(grid_for(nch)), dim3(256), 0, stream, a, nch);
        return hipGetLastError();
    }
    const size_t ngroups = rows * (size_t)(a.D / G);
    const dim3 grid(grid_for(ngroups)), block(256);
#define VA_ALAUNCH(B, GG) hipLaunchKernelGGL((append_groups<B, GG>), grid, block, 0, stream, a, ngroups)
    if (G == 32) {
        if (bits == 8) VA_ALAUNCH(8, 32); else if (bits == 4) VA_ALAUNCH(4, 32); else VA_ALAUNCH(3, 32);
    } else {
        if (bits == 8) VA_ALAUNCH(8, 64); else if (bits == 4) VA_ALAUNCH(4, 64); else VA_ALAUNCH(3, 64);
    }
#undef VA_ALAUNCH
    return hipGetLastError();
}

hipError_t launch_f32_to_f16(const float* x, size_t n, uint16_t* out, hipStream_t stream) {
    hipLaunchKernelGGL(f32_to_f16_kernel, dim3(grid_for(n)), dim3(256), 0, stream, x, n, out);
    return hipGetLastError();
}

hipError_t launch_fill_normal(float* x, size_t n, uint64_t seed, hipStream_t stream) {
    hipLaunchKernelGGL(fill_normal_kernel, dim3(grid_for((n + 3) / 4)), dim3(256), 0, stream, x, n,
                       (uint32_t)seed, (uint32_t)(seed >> 32));
    return hipGetLastError();
}

} // namespace va
