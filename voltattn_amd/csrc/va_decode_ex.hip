// va_decode_ex.hip — the grouped-query and paged launches of the tiled decode
// kernel (va_tiled.hpp). The reference has neither (README.md:205-206 lists
// GQA and paged KV as missing); the row format, quantization and arithmetic
// are the reference path's.
//
// Every launch uses 4-wave work-groups. The query slots a work-group carries
// (QG, the query heads that share one unpacked K/V row) are capped per kind by
// the register budget of its o accumulators (QG x EPL fp32 per lane): f16 and
// q8 up to 8, q4 up to 4, q3 up to 2; larger GQA groups run as several
// sub-groups over the same rows. The tile depth U shrinks as QG grows so the
// two register stages of K/V loads still fit.
#include "va_tiled.hpp"

namespace va {

constexpr int EX_WAVES = 4;

int max_query_slots(int kind) {
    switch (kind) {
        case KF16: return 8;
        case KQ8:  return 8;
        case KQ4:  return 4;
        default:   return 2;
    }
}

// Rows per lane per tile (U) for (kind, QG).
template <int KIND, int QG> struct ExDepth;
template <int QG> struct ExDepth<KF16, QG> { static constexpr int U = QG <= 2 ? 8 : 4; };
template <int QG> struct ExDepth<KQ8, QG>  { static constexpr int U = QG <= 4 ? 4 : 2; };
template <int QG> struct ExDepth<KQ4, QG>  { static constexpr int U = QG <= 2 ? 4 : 2; };
template <int QG> struct ExDepth<KQ3, QG>  { static constexpr int U = 2; };

// The largest work-group tile over the QG variants of a kind: split lengths
// are multiples of it, so every variant starts its splits on a tile boundary.
template <int KIND, int D>
static int max_tile() {
    constexpr int PPW = Tile<KIND, D>::PPW;
    constexpr int u = ExDepth<KIND, 1>::U;
    return PPW * u * EX_WAVES;
}

int tile_positions_ex(int kind, int D) {
    switch (kind) {
        case KF16: return D == 128 ? max_tile<KF16, 128>() : max_tile<KF16, 64>();
        case KQ8:  return D == 128 ? max_tile<KQ8, 128>()  : max_tile<KQ8, 64>();
        case KQ4:  return D == 128 ? max_tile<KQ4, 128>()  : max_tile<KQ4, 64>();
        default:   return D == 128 ? max_tile<KQ3, 128>()  : max_tile<KQ3, 64>();
    }
}

template <int KIND, int D, int G, int QG, bool PAGED>
static hipError_t launch_ex(int groups, const DecodeArgs& a, hipStream_t st) {
    constexpr int U = ExDepth<KIND, QG>::U;
    hipLaunchKernelGGL((decode_tiled<KIND, D, G, U, EX_WAVES, QG, PAGED>),
                       dim3((unsigned)(groups * a.S)), dim3(EX_WAVES * 64), 0, st, a);
    return hipGetLastError();
}

template <int KIND, int D, int G, bool PAGED>
static hipError_t launch_qg(int qg, int groups, const DecodeArgs& a, hipStream_t st) {
    switch (qg) {
        case 1:
            if constexpr (PAGED) return launch_ex<KIND, D, G, 1, true>(groups, a, st);
            else return hipErrorInvalidValue;       // QG = 1 contiguous: va_decode.hip
        case 2: return launch_ex<KIND, D, G, 2, PAGED>(groups, a, st);
        case 4:
            if constexpr (KIND != KQ3) return launch_ex<KIND, D, G, 4, PAGED>(groups, a, st);
            else return hipErrorInvalidValue;
        case 8:
            if constexpr (KIND == KF16 || KIND == KQ8) return launch_ex<KIND, D, G, 8, PAGED>(groups, a, st);
            else return hipErrorInvalidValue;
        default: return hipErrorInvalidValue;
    }
}

template <int KIND, int D, int G>
static hipError_t launch_p(int qg, bool paged, int groups, const DecodeArgs& a, hipStream_t st) {
    return paged ? launch_qg<KIND, D, G, true>(qg, groups, a, st)
                 : launch_qg<KIND, D, G, false>(qg, groups, a, st);
}

template <int KIND, int D>
static hipError_t launch_dg(int G, int qg, bool paged, int groups, const DecodeArgs& a, hipStream_t st) {
    if constexpr (KIND == KF16) return launch_p<KIND, D, 64>(qg, paged, groups, a, st);
    else return G == 32 ? launch_p<KIND, D, 32>(qg, paged, groups, a, st)
                        : launch_p<KIND, D, 64>(qg, paged, groups, a, st);
}

template <int KIND>
static hipError_t launch_k(int D, int G, int qg, bool paged, int groups, const DecodeArgs& a,
                           hipStream_t st) {
    return D == 128 ? launch_dg<KIND, 128>(G, qg, paged, groups, a, st)
                    : launch_dg<KIND, 64>(G, qg, paged, groups, a, st);
}

hipError_t launch_decode_ex(int kind, int D, int G, int qg, bool paged, int groups,
                            const DecodeArgs& a, hipStream_t stream) {
    // malformed arguments never reach a kernel
    if (groups < 1 || a.S < 1 || a.chunk < 1 || a.hkv < 1 || a.qgroup < 1 || a.nsub < 1 ||
        qg < 1 || (long long)qg * a.nsub < a.qgroup || groups % (a.hkv * a.nsub) != 0)
        return hipErrorInvalidValue;
    if (paged && (!a.block_table || !a.seq_lens || a.max_pages < 1 || a.num_pages < 1 ||
                  a.page_shift < 6 || a.chunk % (1 << 6) != 0))
        return hipErrorInvalidValue;
    switch (kind) {
        case KF16: return launch_k<KF16>(D, G, qg, paged, groups, a, stream);
        case KQ8:  return launch_k<KQ8>(D, G, qg, paged, groups, a, stream);
        case KQ4:  return launch_k<KQ4>(D, G, qg, paged, groups, a, stream);
        case KQ3:  return launch_k<KQ3>(D, G, qg, paged, groups, a, stream);
        default:   return hipErrorInvalidValue;
    }
}

} // namespace va
