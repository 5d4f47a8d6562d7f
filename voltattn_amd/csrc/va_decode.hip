// va_decode.hip — the reference-shape decode launches (one sequence, one
// query head per K/V head, contiguous K/V): the tiled ("+") kernels of
// va_tiled.hpp at QG = 1, and the naive one-position-per-wave kernels.
//
// Naive kernels (f16, q8, q4): one wave64 per position, D/64 elements per
// lane, a 6-step cross-lane sum and an exact per-position online-softmax
// update — the attribution control of the reference's attn_f16/q8/q4
// (src/voltattn.cu:122-320).
#include "va_phased.hpp"

#include <algorithm>

namespace va {

constexpr int WAVES = 4;                 // waves per work-group of the naive kernels

// ------------------------------------------------------- naive (w1) kernel --
// One wave64 per position: lane owns dims [lane*P, lane*P+P), P = D/64.
template <int KIND, int D, int G>
__global__ __launch_bounds__(256) void decode_w1(DecodeArgs a) {
    constexpr int P = D / 64;
    constexpr bool QUANT = KIND != KF16;
    constexpr int NG = D / G;
    constexpr int ROWB = RowBytes<KIND, D>::value;

    __shared__ float s_o[WAVES][D];
    __shared__ float s_l[WAVES];
    __shared__ float s_m[WAVES];

    const int wg   = blockIdx.x;
    const int h    = wg / a.S;
    const int s    = wg - h * a.S;
    const unsigned epoch = read_epoch<1>(a, h);
    const Route rt{h, s, 1, h};
    const int wave = (int)(threadIdx.x >> 6);
    const int lane = (int)(threadIdx.x & 63);
    const int g    = (lane * P) / G;
    const int j0   = s * a.chunk;
    const int j1   = min(a.L, j0 + a.chunk);

    float qv[P];
#pragma unroll
    for (int p = 0; p < P; ++p) qv[p] = h2f(a.q[(size_t)h * D + lane * P + p]) * a.qscale;

    float m = M_INIT, l = 0.f, o[P];
#pragma unroll
    for (int p = 0; p < P; ++p) o[p] = 0.f;

    for (int j = j0 + wave; j < j1; j += WAVES) {
        const size_t row = (size_t)h * a.L + j;
        const uint8_t* kr = a.k + row * ROWB;
        const uint8_t* vr = a.v + row * ROWB;
        float kf[P], vf[P];
        if constexpr (KIND == KF16) {
            const uint16_t* kh = reinterpret_cast<const uint16_t*>(kr) + lane * P;
            const uint16_t* vh = reinterpret_cast<const uint16_t*>(vr) + lane * P;
#pragma unroll
            for (int p = 0; p < P; ++p) { kf[p] = h2f(kh[p]); vf[p] = h2f(vh[p]); }
        } else if constexpr (KIND == KQ8) {
            const int8_t* kb = reinterpret_cast<const int8_t*>(kr) + lane * P;
            const int8_t* vb = reinterpret_cast<const int8_t*>(vr) + lane * P;
#pragma unroll
            for (int p = 0; p < P; ++p) { kf[p] = (float)kb[p]; vf[p] = (float)vb[p]; }
        } else {                                   // q4: element e in byte e/2, low nibble first
#pragma unroll
            for (int p = 0; p < P; ++p) {
                const int e = lane * P + p;
                const uint32_t kb = kr[e >> 1], vb = vr[e >> 1];
                const int sh = (e & 1) * 4;
                kf[p] = (float)((int)((kb >> sh) & 0xFu) - 8);
                vf[p] = (float)((int)((vb >> sh) & 0xFu) - 8);
            }
        }
        float acc = 0.f;
#pragma unroll
        for (int p = 0; p < P; ++p) acc = __builtin_fmaf(qv[p], kf[p], acc);
        float vs = 1.f;
        if constexpr (QUANT) {
            acc *= h2f(a.sk[row * NG + g]);
            vs = h2f(a.sv[row * NG + g]);
        }
        acc = wave_sum(acc);
        const float mn = fmaxf(m, acc);
        const float c  = fast_exp2(m - mn);
        const float e  = fast_exp2(acc - mn);
        l = l * c + e;
        m = mn;
        const float ev = e * vs;
#pragma unroll
        for (int p = 0; p < P; ++p) o[p] = __builtin_fmaf(o[p], c, ev * vf[p]);
    }

#pragma unroll
    for (int p = 0; p < P; ++p) s_o[wave][lane * P + p] = o[p];
    if (lane == 0) { s_m[wave] = m; s_l[wave] = l; }
    __syncthreads();
    const int t = (int)threadIdx.x;
    float M[1] = {0.f}, acc[1] = {0.f}, ls[1] = {0.f};
    if (t < D) {
        M[0] = s_m[0];
#pragma unroll
        for (int w = 1; w < WAVES; ++w) M[0] = fmaxf(M[0], s_m[w]);
#pragma unroll
        for (int w = 0; w < WAVES; ++w) {
            const float f = fast_exp2(s_m[w] - M[0]);
            acc[0] = __builtin_fmaf(f, s_o[w][t], acc[0]);
            ls[0]  = __builtin_fmaf(f, s_l[w], ls[0]);
        }
    }
    finish_partial<D, WAVES * 64, 1>(a, rt, M, ls, acc, epoch);
}

// ---------------------------------------------------------------- dispatch --
// Tiled configuration per kind: waves per group and tile depth (UnrollSet a or
// b), measured at H=32 D=128 over L = 4K..64K on MI355X, one group per CU.
// The configuration is fixed at compile time (VA_<KIND>_WAVES = 4|8,
// VA_<KIND>_DEEP = 0|1 build variants); only the configured kernel of each
// kind is built. f16 in 4-wave groups (the waves interleaved by load, as every
// contiguous 4-wave group) against 8-wave groups: L 4096 13.65 -> 13.26 us,
// 16384 41.71 -> 40.97, 65536 155.3 -> 153.0.
#ifndef VA_F16_WAVES
#define VA_F16_WAVES 4               // 4 waves x 4 rows
#endif
#ifndef VA_F16_DEEP
#define VA_F16_DEEP 0
#endif
#ifndef VA_Q8_WAVES
#define VA_Q8_WAVES 4                // 4 waves x 4 rows
#endif
#ifndef VA_Q8_DEEP
#define VA_Q8_DEEP 1
#endif
#ifndef VA_Q4_WAVES
#define VA_Q4_WAVES 4                // 4 waves x 2 rows
#endif
#ifndef VA_Q4_DEEP
#define VA_Q4_DEEP 0                 // 2 rows: L 4096 7.88 -> 7.58 us, 65536 49.0 -> 46.8 against 4
#endif
#ifndef VA_Q3_WAVES
#define VA_Q3_WAVES 8                // 8 waves x 2 rows
#endif
#ifndef VA_Q3_DEEP
#define VA_Q3_DEEP 0
#endif

// Two-phase kernel (va_phased.hpp) per kind: VA_<KIND>_PHASED = 1 selects it
// for the reference-shape launches, with VA_<KIND>_PU rows per lane per tile
// of one tensor and VA_<KIND>_PWAVES waves per group. Interleaved A/B on one
// MI355X, H=32 D=128 G=32, against the single-pass tiled kernel: q8+ L 16384
// 24.36 -> 23.46 us, 65536 85.17 -> 80.65, 4096 9.19 -> 9.21; f16+ L 16384
// 41.12 -> 40.54, 4096 13.24 -> 12.88. The codecs with more vector-ALU work
// per byte lose with it (q4+ 65536 46.07 -> 50.00, q3+ 262144 150.1 -> 187.6
// at 4 waves, 182.6 at 8), so they keep the tiled kernel.
#ifndef VA_F16_PHASED
#define VA_F16_PHASED 1
#endif
#ifndef VA_Q8_PHASED
#define VA_Q8_PHASED 1
#endif
#ifndef VA_Q4_PHASED
#define VA_Q4_PHASED 0
#endif
#ifndef VA_Q3_PHASED
#define VA_Q3_PHASED 0
#endif
#ifndef VA_F16_PU
#define VA_F16_PU 4
#endif
#ifndef VA_Q8_PU
#define VA_Q8_PU 4
#endif
#ifndef VA_Q4_PU
#define VA_Q4_PU 4
#endif
#ifndef VA_Q3_PU
#define VA_Q3_PU 4
#endif
#ifndef VA_F16_PWAVES
#define VA_F16_PWAVES 4
#endif
#ifndef VA_Q8_PWAVES
#define VA_Q8_PWAVES 4
#endif
#ifndef VA_Q4_PWAVES
#define VA_Q4_PWAVES 4
#endif
#ifndef VA_Q3_PWAVES
#define VA_Q3_PWAVES 4
#endif

template <int KIND> struct TiledCfg;
template <> struct TiledCfg<KF16> {
    static constexpr int waves = VA_F16_WAVES; static constexpr bool deep = VA_F16_DEEP;
    static constexpr bool phased = VA_F16_PHASED; static constexpr int pu = VA_F16_PU; static constexpr int pwaves = VA_F16_PWAVES;
};
template <> struct TiledCfg<KQ8> {
    static constexpr int waves = VA_Q8_WAVES; static constexpr bool deep = VA_Q8_DEEP;
    static constexpr bool phased = VA_Q8_PHASED; static constexpr int pu = VA_Q8_PU; static constexpr int pwaves = VA_Q8_PWAVES;
};
template <> struct TiledCfg<KQ4> {
    static constexpr int waves = VA_Q4_WAVES; static constexpr bool deep = VA_Q4_DEEP;
    static constexpr bool phased = VA_Q4_PHASED; static constexpr int pu = VA_Q4_PU; static constexpr int pwaves = VA_Q4_PWAVES;
};
template <> struct TiledCfg<KQ3> {
    static constexpr int waves = VA_Q3_WAVES; static constexpr bool deep = VA_Q3_DEEP;
    static constexpr bool phased = VA_Q3_PHASED; static constexpr int pu = VA_Q3_PU; static constexpr int pwaves = VA_Q3_PWAVES;
};
template <int KIND> struct TiledShape {
    static_assert(TiledCfg<KIND>::waves == 4 || TiledCfg<KIND>::waves == 8, "4 or 8 waves per group");
    static constexpr bool phased = TiledCfg<KIND>::phased;
    static constexpr int waves = phased ? TiledCfg<KIND>::pwaves : TiledCfg<KIND>::waves;
    static constexpr int U = phased ? TiledCfg<KIND>::pu
                                    : TiledCfg<KIND>::deep ? UnrollSet<KIND>::b : UnrollSet<KIND>::a;
};

template <int KIND, int D>
static int tiled_positions() {
    return Tile<KIND, D>::PPW * TiledShape<KIND>::U * TiledShape<KIND>::waves;
}

int tile_positions(int kind, bool tiled, int D) {
    if (!tiled) return WAVES;
    switch (kind) {
        case KF16: return D == 128 ? tiled_positions<KF16, 128>() : tiled_positions<KF16, 64>();
        case KQ8:  return D == 128 ? tiled_positions<KQ8, 128>()  : tiled_positions<KQ8, 64>();
        case KQ4:  return D == 128 ? tiled_positions<KQ4, 128>()  : tiled_positions<KQ4, 64>();
        default:   return D == 128 ? tiled_positions<KQ3, 128>()  : tiled_positions<KQ3, 64>();
    }
}

// Tiled kinds: one work-group per CU. A second group per CU (twice the
// splits) measured slower on MI355X with every configured shape (f16+ at
// L 16384: 42.91 against 40.97 us; q8+ and q4+ at S = 16, 32, 64 too).
int groups_per_cu(int kind, bool tiled) {
    (void)kind;
    return tiled ? 1 : 8;                 // naive: one position per wave, 32 waves per CU
}

template <int KIND, int D, int G>
static hipError_t launch_one(bool tiled, int H, const DecodeArgs& a, hipStream_t st) {
    const dim3 grid((unsigned)(H * a.S));
    if (tiled) {
        using T = TiledShape<KIND>;
        if constexpr (T::phased)
            hipLaunchKernelGGL((decode_phased<KIND, D, G, T::U, T::waves>), grid, dim3(T::waves * 64), 0, st,
                               VA_TILED_ARGS(a));
        else
            hipLaunchKernelGGL((decode_tiled<KIND, D, G, T::U, T::waves, 1, false>), grid, dim3(T::waves * 64), 0, st,
                               VA_TILED_ARGS(a));
    } else {
        if constexpr (KIND == KQ3) return hipErrorInvalidValue;
        else hipLaunchKernelGGL((decode_w1<KIND, D, G>), grid, dim3(256), 0, st, a);
    }
    return hipGetLastError();
}

template <int KIND, int D>
static hipError_t launch_g(bool tiled, int H, int G, const DecodeArgs& a, hipStream_t st) {
    if constexpr (KIND == KF16) return launch_one<KIND, D, 64>(tiled, H, a, st);
    else return G == 32 ? launch_one<KIND, D, 32>(tiled, H, a, st)
                        : launch_one<KIND, D, 64>(tiled, H, a, st);
}

template <int KIND>
static hipError_t launch_d(bool tiled, int H, int D, int G, const DecodeArgs& a, hipStream_t st) {
    return D == 128 ? launch_g<KIND, 128>(tiled, H, G, a, st) : launch_g<KIND, 64>(tiled, H, G, a, st);
}

hipError_t launch_decode(int kind, bool tiled, int H, int D, int G, const DecodeArgs& a,
                         hipStream_t stream) {
    if (H < 1 || a.S < 1 || a.chunk < 1 || a.hkv != H || a.qgroup != 1 || a.nsub != 1)
        return hipErrorInvalidValue;             // malformed arguments never reach a kernel
    switch (kind) {
        case KF16: return launch_d<KF16>(tiled, H, D, G, a, stream);
        case KQ8:  return launch_d<KQ8>(tiled, H, D, G, a, stream);
        case KQ4:  return launch_d<KQ4>(tiled, H, D, G, a, stream);
        case KQ3:  return launch_d<KQ3>(tiled, H, D, G, a, stream);
        default:   return hipErrorInvalidValue;
    }
}

hipError_t lost_merges_decode(unsigned* n) { return read_lost_merges(n); }
hipError_t clear_tagged_decode(int slot, hipStream_t stream) { return launch_clear_tagged(slot, stream); }

} // namespace va
