// va_merge.hip — second pass of the split-L decode: per head, the S partials
// (m, l, o[D]) written by the decode kernels are merged by log-sum-exp and the
// normalised output is rounded to fp16 (reference combine, src/voltattn.cu:651-672).
// m is in log2 units (the decode kernels work with exp2), so the weights are
// exp2(m_s - max_s m_s). Empty splits carry l = 0 and o = 0 and drop out; a
// head whose merged l is 0 (no positions: a paged sequence of length 0) gets a
// zero output, as in the fused merge, and a non-finite l (an input the decode
// kernel flagged with l = NaN) gives NaN.
//
// The pass is latency-bound (a few hundred KB in total), so it is laid out for
// one round of independent loads: a work-group owns 32 output columns of one
// head and its 8 wave-halves split the S partials between them; every thread
// loads (m_s, l_s, o_s[d]) for up to MERGE_PT splits at once, folds them with a
// running maximum, and the 8 split groups are combined through LDS.
#include "va_device.hpp"
#include "va_kernels.hpp"

namespace va {

constexpr int MERGE_DC = 32;   // output columns per work-group
constexpr int MERGE_SG = 8;    // split groups per work-group (256 = 32 x 8 threads)
constexpr int MERGE_PT = 8;    // splits per thread per load round
constexpr float MERGE_FLOOR = -3.0e38f;   // below any partial's m (>= -1e30)

__global__ __launch_bounds__(256) void lse_merge(const float* __restrict__ ws,
                                                 uint16_t* __restrict__ out, int S, int D) {
    __shared__ float s_acc[MERGE_SG][MERGE_DC];
    __shared__ float s_l[MERGE_SG];
    __shared__ float s_m[4];

    const int nbd = D / MERGE_DC;
    const int h   = blockIdx.x / nbd;
    const int d   = (blockIdx.x - h * nbd) * MERGE_DC + (int)(threadIdx.x % MERGE_DC);
    const int sg  = (int)(threadIdx.x / MERGE_DC);
    const size_t stride = (size_t)(D + 2);
    const float* base = ws + (size_t)h * S * stride;

    float mt = MERGE_FLOOR, acc = 0.f, lacc = 0.f;
    for (int s0 = sg; s0 < S; s0 += MERGE_SG * MERGE_PT) {
        float mv[MERGE_PT], lv[MERGE_PT], ov[MERGE_PT];
#pragma unroll
        for (int i = 0; i < MERGE_PT; ++i) {
            const int s = s0 + MERGE_SG * i;
            const bool ok = s < S;
            const float* slot = base + (size_t)(ok ? s : 0) * stride;
            mv[i] = ok ? slot[0] : MERGE_FLOOR;
            lv[i] = ok ? slot[1] : 0.f;
            ov[i] = ok ? slot[2 + d] : 0.f;
        }
        float mr = mt;
#pragma unroll
        for (int i = 0; i < MERGE_PT; ++i) mr = fmaxf(mr, mv[i]);
        const float c = fast_exp2(mt - mr);
        acc *= c;
        lacc *= c;
#pragma unroll
        for (int i = 0; i < MERGE_PT; ++i) {
            const float w = fast_exp2(mv[i] - mr);
            acc  = __builtin_fmaf(w, ov[i], acc);
            lacc = __builtin_fmaf(w, lv[i], lacc);
        }
        mt = mr;
    }
    // Combine the split groups: common maximum, then sums through LDS.
    const float wm = wave_max(mt);
    if ((threadIdx.x & 63) == 0) s_m[threadIdx.x >> 6] = wm;
    __syncthreads();
    const float M = fmaxf(fmaxf(s_m[0], s_m[1]), fmaxf(s_m[2], s_m[3]));
    const float f = fast_exp2(mt - M);
    s_acc[sg][threadIdx.x % MERGE_DC] = acc * f;
    if (threadIdx.x % MERGE_DC == 0) s_l[sg] = lacc * f;
    __syncthreads();
    if (sg == 0) {
        float o = 0.f, l = 0.f;
#pragma unroll
        for (int g = 0; g < MERGE_SG; ++g) {
            o += s_acc[g][threadIdx.x];
            l += s_l[g];
        }
        out[(size_t)h * D + d] = f2h_rne(l == 0.f ? 0.f : o / l);
    }
}

hipError_t launch_merge(const float* ws, uint16_t* out, int H, int D, int S, hipStream_t stream) {
    hipLaunchKernelGGL(lse_merge, dim3((unsigned)(H * (D / MERGE_DC))), dim3(256), 0, stream, ws,
                       out, S, D);
    return hipGetLastError();
}

} // namespace va
