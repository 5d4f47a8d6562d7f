// va_decode_ex.hip — the grouped-query and paged launches of the tiled decode
// kernel (va_tiled.hpp). The reference has neither (README.md:205-206 lists
// GQA and paged KV as missing); the row format, quantization and arithmetic
// are the reference path's.
//
// The query slots a work-group carries (QG, the query heads that share one
// unpacked K/V row) are capped per kind (max_query_slots); larger GQA groups
// run as several sub-groups over the same rows, a group that is not a multiple
// of QG masks the spare slots. Grouped work-groups are 8 waves (two per SIMD)
// where that fits in 256 VGPRs, else 4; the tile depth U shrinks as QG grows
// so the two register stages of K/V loads still fit.
#include "va_phased.hpp"
#include "va_mfma.hpp"

#include <algorithm>

namespace va {

// Launch shape of the grouped/paged kernels (VA_EX_MODE):
//   0: 4-wave work-groups, one per CU;
//   1: 4-wave work-groups, two per CU where two waves per SIMD fit in 256 VGPRs;
//   2: 8-wave work-groups (two waves per SIMD from one group) where they fit,
//      else as 0.
// Two waves per SIMD hide the latency of the longer per-row chains of several
// query heads; one wider group keeps the split count (and so the merge) as in 0.
#ifndef VA_EX_MODE
#define VA_EX_MODE 2
#endif

// Matrix-core form (va_mfma.hpp) for q8 and q4 rows, and q3 rows at D = 128, with
// two or more query slots:
// MFMA_WAVES waves per work-group, 32-row wave tiles. A build with
// VA_GQA_MFMA=0 runs the vector-ALU form of va_tiled.hpp for them instead (the
// comparison variant the tests build; the product is built with the default).
#ifndef VA_MFMA_WAVES
#define VA_MFMA_WAVES 8
#endif
#ifndef VA_GQA_MFMA
#define VA_GQA_MFMA 1
#endif
constexpr int MFMA_WAVES = VA_MFMA_WAVES;
constexpr int MFMA_TILE  = 32 * MFMA_WAVES;
constexpr bool MFMA_ON   = VA_GQA_MFMA != 0;

static bool mfma_kind(int kind, int D) { return (kind == KQ8 || kind == KQ4 || (kind == KQ3 && D == 128)) && MFMA_ON; }
static bool mfma_form(int kind, int D, int qg) { return mfma_kind(kind, D) && qg >= 2; }
template <int KIND, int D> constexpr bool mfma_kind_c = (KIND == KQ8 || KIND == KQ4 || (KIND == KQ3 && D == 128)) && MFMA_ON;

// Query slots per work-group, per kind: the largest QG whose 8-wave form (two
// waves per SIMD) fits in 256 VGPRs. Measured on MI355X (Hq/Hkv = 32/8, 64/8,
// 28/4 at L = 16K-64K): QG = 4 at two waves per SIMD beats QG = 8 at one for
// f16 and q8 (groups of 8 run as two sub-groups, 12-38% faster), and q4 is
// fastest at QG = 2 (QG = 4 spills at two waves per SIMD). The matrix-core
// form carries 4 slots for q4, and for q3 at D = 128, too. A build with
// VA_EX_QMAX = 1|2|4 lowers the cap (a tuning variant).
#ifndef VA_EX_QMAX
#define VA_EX_QMAX 0
#endif
int max_query_slots(int kind, int D) {
    constexpr int cap = VA_EX_QMAX;
    const int q = (kind == KF16 || kind == KQ8 || mfma_kind(kind, D)) ? 4 : 2;
    return (cap == 1 || cap == 2 || cap == 4) ? std::min(q, cap) : q;
}

// Rows per lane per tile (U), waves per work-group and work-groups per CU
// (MINB) for (kind, QG). FIT: two waves per SIMD fit in 256 VGPRs without
// spilling at the shallower depth U2 (measured with the compiler's register
// report), and the 8-wave LDS reduction fits (QG <= 4).
template <int KIND, int QG> struct ExBase;
template <int QG> struct ExBase<KF16, QG> { static constexpr int U = QG <= 2 ? 8 : 4, U2 = QG <= 2 ? 8 : 4; static constexpr bool FIT = QG == 2 || QG == 4; };
template <int QG> struct ExBase<KQ8, QG>  { static constexpr int U = QG <= 4 ? 4 : 2, U2 = QG <= 2 ? 4 : 2; static constexpr bool FIT = QG == 2 || QG == 4; };
template <int QG> struct ExBase<KQ4, QG>  { static constexpr int U = QG <= 2 ? 4 : 2, U2 = 2; static constexpr bool FIT = QG == 2; };
template <int QG> struct ExBase<KQ3, QG>  { static constexpr int U = 2, U2 = 1; static constexpr bool FIT = QG == 2; };

template <int KIND, int QG> struct ExCfg {
    using B = ExBase<KIND, QG>;
    static constexpr bool two = B::FIT && VA_EX_MODE != 0;
    static constexpr int U     = two ? B::U2 : B::U;
    static constexpr int WAVES = two && VA_EX_MODE == 2 ? 8 : 4;
    static constexpr int MINB  = two && VA_EX_MODE == 1 ? 2 : 1;
};

template <int KIND>
static int minb_of(int qg) {
    switch (qg) {
        case 1: return ExCfg<KIND, 1>::MINB;
        case 2: return ExCfg<KIND, 2>::MINB;
        default: return ExCfg<KIND, 4>::MINB;
    }
}

int ex_groups_per_cu(int kind, int D, int qg) {
    if (mfma_form(kind, D, qg)) return 1;
    switch (kind) {
        case KF16: return minb_of<KF16>(qg);
        case KQ8:  return minb_of<KQ8>(qg);
        case KQ4:  return minb_of<KQ4>(qg);
        default:   return minb_of<KQ3>(qg);
    }
}

// Rows per lane actually used: a wave tile (PPW * U rows) must fit in the
// smallest page (64 rows), e.g. q4 at D = 64 reads 32 rows per wave load.
template <int KIND, int D, int QG>
constexpr int ex_unroll() {
    return ExCfg<KIND, QG>::U < 64 / Tile<KIND, D>::PPW ? ExCfg<KIND, QG>::U : 64 / Tile<KIND, D>::PPW;
}

template <int KIND, int D, int QG>
constexpr int ex_tile() {
    return Tile<KIND, D>::PPW * ex_unroll<KIND, D, QG>() * ExCfg<KIND, QG>::WAVES;
}

// The largest work-group tile over the QG variants of a kind (all are powers
// of two): split lengths are multiples of it, so every variant starts its
// splits on a tile boundary.
template <int KIND, int D>
static int max_tile() {
    return std::max(std::max(ex_tile<KIND, D, 1>(), ex_tile<KIND, D, 2>()), ex_tile<KIND, D, 4>());
}

int tile_positions_ex(int kind, int D) {
    switch (kind) {
        case KF16: return D == 128 ? max_tile<KF16, 128>() : max_tile<KF16, 64>();
        case KQ8:  return std::max(MFMA_TILE, D == 128 ? max_tile<KQ8, 128>() : max_tile<KQ8, 64>());
        case KQ4:  return std::max(MFMA_TILE, D == 128 ? max_tile<KQ4, 128>() : max_tile<KQ4, 64>());
        default:   return D == 128 ? std::max(MFMA_ON ? MFMA_TILE : 1, max_tile<KQ3, 128>()) : max_tile<KQ3, 64>();
    }
}

// Grouped-query f16 over contiguous K/V: the two-phase kernel (va_phased.hpp)
// with QG query slots, one 8-wave group per CU (U = 4: 32 KB per stage);
// VA_EX_PHASED = 0 keeps it on decode_tiled. Interleaved A/B on MI355X, Hq 32 /
// Hkv 8, D 128, against decode_tiled: L 65536 48.40 -> 45.49 us, 16384 19.19 ->
// 17.71, 4096 11.94 -> 11.58; 4-wave groups lost at short L (their merge of
// four query slots runs on half the waves: 4096 11.89 -> 12.18).
#ifndef VA_EX_PHASED
#define VA_EX_PHASED 1
#endif
#ifndef VA_EX_PH_WAVES
#define VA_EX_PH_WAVES 8
#endif
#ifndef VA_EX_PH_U
#define VA_EX_PH_U 4
#endif

// Paged f16 and q8 with one query slot per KV head: the two-phase kernel's
// paged form (4 waves, U = 4) when a page holds a whole work-group tile and
// splits start on one; other page sizes stay on decode_tiled. Interleaved A/B on
// MI355X, B 1, Hq = Hkv = 32, D 128, L 16384, against decode_tiled: f16 pages of
// 256 42.60 -> 40.67 us, pages of 64 43.59 -> 41.03; q8 pages of 256 25.46 ->
// 24.58 (page ids read a stage ahead), 4096 10.18 -> 10.21.
#ifndef VA_EX_PHASED_PAGED
#define VA_EX_PHASED_PAGED 1
#endif
#ifndef VA_EX_PHASED_PAGED_Q8
#define VA_EX_PHASED_PAGED_Q8 1
#endif

template <int KIND, int D, int G, int QG, bool PAGED>
static hipError_t launch_ex(int groups, const DecodeArgs& a, hipStream_t st) {
    constexpr int PTB = Tile<KIND, D>::PPW * 4 * 4;   // the paged form's work-group tile (a power of two)
    if constexpr (VA_EX_PHASED_PAGED && QG == 1 && PAGED && (KIND == KF16 || (VA_EX_PHASED_PAGED_Q8 && KIND == KQ8))) {
        if ((1 << a.page_shift) >= PTB && a.chunk % PTB == 0) {
            hipLaunchKernelGGL((decode_phased<KIND, D, G, 4, 4, 1, true>), dim3((unsigned)(groups * a.S)), dim3(256),
                               0, st, VA_TILED_ARGS(a));
            return hipGetLastError();
        }
    }
    if constexpr (VA_EX_PHASED && KIND == KF16 && !PAGED && QG >= 2) {
        hipLaunchKernelGGL((decode_phased<KIND, D, G, VA_EX_PH_U, VA_EX_PH_WAVES, QG>), dim3((unsigned)(groups * a.S)),
                           dim3(VA_EX_PH_WAVES * 64), 0, st, VA_TILED_ARGS(a));
        return hipGetLastError();
    } else if constexpr (mfma_kind_c<KIND, D> && QG >= 2) {
        hipLaunchKernelGGL((decode_mfma<KIND, D, G, MFMA_WAVES, QG, PAGED>),
                           dim3((unsigned)(groups * a.S)), dim3(MFMA_WAVES * 64), 0, st, a);
        return hipGetLastError();
    } else if constexpr ((KIND == KQ4 || KIND == KQ3) && QG > 2) {
        return hipErrorInvalidValue;                 // matrix-core form only
    } else {
        using Cfg = ExCfg<KIND, QG>;
        constexpr int U = ex_unroll<KIND, D, QG>();
        static_assert(Tile<KIND, D>::PPW * U <= 64, "a wave tile must fit the smallest page");
        hipLaunchKernelGGL((decode_tiled<KIND, D, G, U, Cfg::WAVES, QG, PAGED, Cfg::MINB>),
                           dim3((unsigned)(groups * a.S)), dim3(Cfg::WAVES * 64), 0, st, VA_TILED_ARGS(a));
        return hipGetLastError();
    }
}

template <int KIND, int D, int G, bool PAGED>
static hipError_t launch_qg(int qg, int groups, const DecodeArgs& a, hipStream_t st) {
    switch (qg) {
        case 1:
            if constexpr (PAGED) return launch_ex<KIND, D, G, 1, true>(groups, a, st);
            else return hipErrorInvalidValue;       // QG = 1 contiguous: va_decode.hip
        case 2: return launch_ex<KIND, D, G, 2, PAGED>(groups, a, st);
        case 4:
            if constexpr (KIND == KF16 || KIND == KQ8 || KIND == KQ4 || (KIND == KQ3 && D == 128))
                return launch_ex<KIND, D, G, 4, PAGED>(groups, a, st);
            else return hipErrorInvalidValue;
        default: return hipErrorInvalidValue;          // above max_query_slots(kind, D)
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

hipError_t lost_merges_ex(unsigned* n) { return read_lost_merges(n); }
hipError_t clear_tagged_ex(int slot, hipStream_t stream) { return launch_clear_tagged(slot, stream); }

} // namespace va
