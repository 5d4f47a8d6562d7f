// va_merge.hip — second pass of the split-L decode: per head, the S partials
// (m, l, o[D]) written by the decode kernels are merged by log-sum-exp and the
// normalised output is rounded to fp16 (reference combine, src/voltattn.cu:651-672).
// m is in log2 units (the decode kernels work with exp2), so the weights are
// exp2(m_s - max_s m_s). Empty splits carry l = 0 and o = 0 and drop out.
#include "va_device.hpp"
#include "va_kernels.hpp"

namespace va {

__global__ __launch_bounds__(128) void lse_merge(const float* __restrict__ ws,
                                                 uint16_t* __restrict__ out, int S, int D) {
    const int h = blockIdx.x;
    const int t = (int)threadIdx.x;
    const float* base = ws + (size_t)h * S * (D + 2);
    float M = -__builtin_inff();
    for (int s = 0; s < S; ++s) M = fmaxf(M, base[(size_t)s * (D + 2)]);
    float lsum = 0.f, acc = 0.f;
    for (int s = 0; s < S; ++s) {
        const float* slot = base + (size_t)s * (D + 2);
        const float w = fast_exp2(slot[0] - M);
        lsum = __builtin_fmaf(w, slot[1], lsum);
        if (t < D) acc = __builtin_fmaf(w, slot[2 + t], acc);
    }
    if (t < D) out[(size_t)h * D + t] = f2h_rne(acc / lsum);
}

hipError_t launch_merge(const float* ws, uint16_t* out, int H, int D, int S, hipStream_t stream) {
    hipLaunchKernelGGL(lse_merge, dim3((unsigned)H), dim3(128), 0, stream, ws, out, S, D);
    return hipGetLastError();
}

} // namespace va
