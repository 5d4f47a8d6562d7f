// va_codec.hpp — lane layouts and lane codecs of the tiled decode kernels.
//
// Layout: a position row of ROWB compressed bytes is read by LP lanes, each
// taking LB = 16 contiguous bytes (12 for q3) with one buffer load, so one
// wave-wide load covers PPW = 64/LP consecutive rows (1 KiB; 768 B for q3).
//
// Codecs: a lane owns EPL consecutive elements of a row. Each row is unpacked
// once, with bit operations only (no per-element convert), into NP fp16 pairs
// that every query head sharing the row consumes (grouped-query attention
// reuses one unpack for several heads):
//   * K (`unpack_k`, `dot`): exact signed values 2^r v as fp16, through the
//     "magic" construction below, against the fp16 q slice with
//     v_dot2_f32_f16 (products of two normal fp16 values are exact in fp32;
//     measured on MI355X, the result is within 1 fp32 ulp of |p0| + |p1| on a
//     zero accumulator and within 16 ulps of |p0| + |p1| + |acc| chained on a
//     nonzero one). q is unscaled for f16, q8 and q4 and pre-scaled per
//     element by a power of two for q3. `dot` returns the raw sum; the caller
//     applies the group scale and qs = log2(e)/sqrt(D) (QReg::qs, uniform
//     over the wave).
//   * V (`unpack_v`, `axpy_v`, `fix_v`): the unsigned stored code c = v + OFF
//     as an fp16 subnormal c 2^(r-24) (the masked bits alone, exponent field
//     0: no magic and no subtract), accumulated by v_fma_mix_f32,
//     o_e += ev * c_e 2^(r_e-24), with an fp16 operand and fp32 accumulation
//     (P.V stays fp32; v_fma_mix_f32 with an fp32 weight and an fp16 code,
//     subnormal or normal, is one correctly rounded fma: bit-identical to the
//     host's fmaf in 2^19 random cases on MI355X). The offset is removed in bulk:
//     the caller sums ev over a window of rows (S; at most 16 per lane) and
//     `fix_v` adds S * voff(e) = -OFF 2^(r_e-24) S to each accumulator, so the
//     running sums never drift more than one window's worth from the signed
//     sums. fin(e) = 2^(24-r_e) rescales o_e once at the end; the caller folds
//     it into the last fix, o_e = fma(o_e, fin(e), S * voff(e) * fin(e)), which
//     is fin(e) * (o_e + S * voff(e)) rounded once, as fix then rescale
//     (fin(e) and voff(e) * fin(e) = -OFF are powers of two or small integers,
//     so S * voff(e) * fin(e) is exact).
// The magic construction (K): OR-ing a code n (< 2^10 / 2^r) shifted left by r
// into the mantissa of 1024.0 (0x6400) gives 1024 + 2^r n exactly; one packed
// fp16 subtract of 1024 + 2^r * offset then leaves 2^r * v. The magic constant
// lives in a VGPR (`magic()`, made once per kernel) so mask-and-insert is one
// v_and_or_b32 (a gfx9 VOP3 reads one scalar constant; mask and magic cannot
// both be literals). A subnormal K operand is not used: v_dot2_f32_f16 sums
// two products with a subnormal operand less precisely (measured up to 320
// fp32 ulps of |p0| + |p1| on MI355X).
//
// Interface: QReg (one query head's slice in codec form, with qs),
// load_q<LP>(QReg&, q slice, qs) (LP: lanes per row), magic(), unpack_k(w, magic, p[NP]), dot(p, QReg) -> raw q.k,
// unpack_v(w, p[NP]), axpy_v(p, ev, o), VFIX / voff(e) (bulk offset removal),
// fin(e) (per-element rescale once at the end).
#pragma once
#include "va_device.hpp"

#include <utility>

namespace va {

template <int KIND, int D> struct Tile {
    static constexpr int ROWB = RowBytes<KIND, D>::value;   // bytes per row
    static constexpr int LB   = KIND == KQ3 ? 12 : 16;      // bytes per lane per row
    static constexpr int LP   = ROWB / LB;                  // lanes per row
    static constexpr int PPW  = 64 / LP;                    // rows per wave load
    static constexpr int EPL  = D / LP;                     // elements per lane
    static_assert(ROWB % LB == 0 && 64 % LP == 0 && LP <= 16, "lane split");
};

// Rows per lane per tile and tensor (U). Each kind is instantiated for two
// depths; the dispatch picks one per kind.
template <int KIND> struct UnrollSet;
template <> struct UnrollSet<KF16> { static constexpr int a = 4, b = 8; };
template <> struct UnrollSet<KQ8>  { static constexpr int a = 2, b = 4; };
template <> struct UnrollSet<KQ4>  { static constexpr int a = 2, b = 4; };
template <> struct UnrollSet<KQ3>  { static constexpr int a = 2, b = 4; };

template <int KIND> struct LaneLoad { using type = u32x4; };
template <> struct LaneLoad<KQ3> { using type = u32x3; };

template <int KIND>
__device__ __forceinline__ typename LaneLoad<KIND>::type
lane_load(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    if constexpr (KIND == KQ3) return ld96(r, voff, soff);
    else return ld128(r, voff, soff);
}

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ h2 as_h2(uint32_t x) { return __builtin_bit_cast(h2, x); }
__device__ __forceinline__ h2 hh(float a, float b) { return h2{(_Float16)a, (_Float16)b}; }

// x times the fp16 in the low / high half of w, as one v_fma_mix_f32 (the
// half is converted inside the instruction; exact, like v_cvt_f32_f16 and a
// multiply, except that a zero product is +0).
__device__ __forceinline__ float mul_lo_h(float x, uint32_t w) { return __builtin_fmaf(x, (float)as_h2(w).x, 0.f); }
__device__ __forceinline__ float mul_hi_h(float x, uint32_t w) { return __builtin_fmaf(x, (float)as_h2(w).y, 0.f); }

#define VA_VGPR_CONST(dst, imm) asm volatile("v_mov_b32 %0, " #imm : "=v"(dst))

// Load a lane's q slice (EPL fp16 values, 16-byte aligned) as raw dwords.
template <int EPL>
__device__ __forceinline__ void load_q_words(uint32_t (&qw)[EPL / 2], const uint16_t* qh) {
#pragma unroll
    for (int c = 0; c < EPL / 8; ++c) {
        const u32x4 w = reinterpret_cast<const u32x4*>(qh)[c];
        qw[4 * c] = w.x; qw[4 * c + 1] = w.y; qw[4 * c + 2] = w.z; qw[4 * c + 3] = w.w;
    }
}

template <int KIND> struct Codec;

// v_dot2_f32_f16 with a zero accumulator in the instruction (VOP3 inline 0);
// written as asm because the compiler otherwise rewrites the builtin to the
// tied-accumulator form and spends a v_mov_b32 on the zero.
__device__ __forceinline__ float fdot2_z(h2 a, h2 b) {
    float r;
    asm("v_dot2_f32_f16 %0, %1, %2, 0" : "=v"(r) : "v"(a), "v"(b));
    return r;
}

// Pairs (2k, 2k+1) as consecutive elements: the f16 and q8 layouts.
template <int NP>
__device__ __forceinline__ float dot_pairs(const h2 (&p)[NP], const h2 (&q)[NP]) {
    float a = fdot2_z(p[0], q[0]);
#pragma unroll
    for (int k = 1; k < NP; ++k) a = __builtin_amdgcn_fdot2(p[k], q[k], a, false);
    return a;
}
template <int NP>
__device__ __forceinline__ void axpy_pairs(const h2 (&p)[NP], float ev, float* o) {
#pragma unroll
    for (int k = 0; k < NP; ++k) {
        o[2 * k]     = __builtin_fmaf(ev, (float)p[k].x, o[2 * k]);
        o[2 * k + 1] = __builtin_fmaf(ev, (float)p[k].y, o[2 * k + 1]);
    }
}

// f16: 8 halves per lane, element 2k+j in half j of dword k.
template <> struct Codec<KF16> {
    static constexpr int EPL = 8, NP = 4;
    struct QReg { h2 q[NP]; float qs; };
    template <int LP>
    __device__ static void load_q(QReg& r, const uint16_t* qh, float qs) {
        uint32_t qw[4];
        load_q_words<8>(qw, qh);
#pragma unroll
        for (int i = 0; i < 4; ++i) r.q[i] = as_h2(qw[i]);
        r.qs = qs;
    }
    __device__ static uint32_t magic() { return 0u; }
    __device__ static void unpack_k(const u32x4& w, uint32_t, h2 (&p)[NP]) {
#pragma unroll
        for (int i = 0; i < 4; ++i) p[i] = as_h2(w[i]);
    }
    __device__ static float dot(const h2 (&p)[NP], const QReg& r) { return dot_pairs<NP>(p, r.q); }
    static constexpr bool VFIX = false;       // stored values are the values
    __device__ static constexpr float voff(int) { return 0.f; }
    __device__ static void unpack_v(const u32x4& w, h2 (&p)[NP]) { unpack_k(w, 0u, p); }
    __device__ static void axpy_v(const h2 (&p)[NP], float ev, float* o) { axpy_pairs<NP>(p, ev, o); }
    __device__ static constexpr float fin(int) { return 1.f; }
};

// q8: 16 int8 per lane, element 4i+b in byte b of dword i. xor 0x80 makes the
// bytes u = v + 128; v_perm_b32 places bytes (b0, b1) / (b2, b3) under the
// 0x64 magic byte: fp16 pair (1024 + u, 1024 + u'), minus 1152 -> (v, v') for
// K, and under zero bytes (selector 0x0C) for V: subnormal (u 2^-24, u' 2^-24),
// OFF = 128. Pair k holds elements (2k, 2k+1).
template <> struct Codec<KQ8> {
    static constexpr int EPL = 16, NP = 8;
    struct QReg { h2 q[NP]; float qs; };
    template <int LP>
    __device__ static void load_q(QReg& r, const uint16_t* qh, float qs) {
        uint32_t qw[8];
        load_q_words<16>(qw, qh);
#pragma unroll
        for (int i = 0; i < 8; ++i) r.q[i] = as_h2(qw[i]);
        r.qs = qs;
    }
    __device__ static uint32_t magic() { uint32_t m; VA_VGPR_CONST(m, 0x64646464); return m; }
    __device__ static void unpack_k(const u32x4& w, uint32_t magic, h2 (&p)[NP]) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t u = w[i] ^ 0x80808080u;
            p[2 * i]     = as_h2(__builtin_amdgcn_perm(magic, u, 0x04010400u)) - hh(1152.f, 1152.f);
            p[2 * i + 1] = as_h2(__builtin_amdgcn_perm(magic, u, 0x04030402u)) - hh(1152.f, 1152.f);
        }
    }
    __device__ static float dot(const h2 (&p)[NP], const QReg& r) { return dot_pairs<NP>(p, r.q); }
    static constexpr bool VFIX = true;
    __device__ static constexpr float voff(int) { return -128.f / 16777216.f; }
    __device__ static void unpack_v(const u32x4& w, h2 (&p)[NP]) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t u = w[i] ^ 0x80808080u;
            p[2 * i]     = as_h2(__builtin_amdgcn_perm(u, u, 0x0C010C00u));
            p[2 * i + 1] = as_h2(__builtin_amdgcn_perm(u, u, 0x0C030C02u));
        }
    }
    __device__ static void axpy_v(const h2 (&p)[NP], float ev, float* o) { axpy_pairs<NP>(p, ev, o); }
    __device__ static constexpr float fin(int) { return 16777216.f; }
};

// q4: 32 nibbles per lane; element 8i+j sits in nibble j of dword i. Masking
// nibbles (0, 4) / (1, 5) in place and (2, 6) / (3, 7) after a shift by 8 under
// the 1024.0 magic gives the exact pairs
//   P0 = (e0, e4) = v,  P1 = (e1, e5) = 16v,  P2 = (e2, e6) = v,  P3 = (e3, e7) = 16v;
// the 16v pairs accumulate separately (scaled by 1/16 once) for K. For V the
// same masks alone give subnormals c 2^-24 (P0, P2) and 16c 2^-24 (P1, P3),
// OFF = 8. Pair 4i+c is Pc of dword i.
template <> struct Codec<KQ4> {
    static constexpr int EPL = 32, NP = 16;
    struct QReg { h2 q[NP]; float qs; };     // q[4i+c] pairs the elements of P_c of dword i
    template <int LP>
    __device__ static void load_q(QReg& r, const uint16_t* qh, float qs) {
        uint32_t qw[16];
        load_q_words<32>(qw, qh);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            // halves of elements 8i..8i+7: qw[4i] = (e0, e1), +1 = (e2, e3), +2 = (e4, e5), +3 = (e6, e7)
            r.q[4 * i + 0] = as_h2(__builtin_amdgcn_perm(qw[4 * i + 2], qw[4 * i], 0x05040100u));      // (e0, e4)
            r.q[4 * i + 1] = as_h2(__builtin_amdgcn_perm(qw[4 * i + 2], qw[4 * i], 0x07060302u));      // (e1, e5)
            r.q[4 * i + 2] = as_h2(__builtin_amdgcn_perm(qw[4 * i + 3], qw[4 * i + 1], 0x05040100u));  // (e2, e6)
            r.q[4 * i + 3] = as_h2(__builtin_amdgcn_perm(qw[4 * i + 3], qw[4 * i + 1], 0x07060302u));  // (e3, e7)
        }
        r.qs = qs;
    }
    __device__ static uint32_t magic() { uint32_t m; VA_VGPR_CONST(m, 0x64006400); return m; }
    __device__ static void unpack_k(const u32x4& w, uint32_t magic, h2 (&p)[NP]) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t x = w[i], x8 = w[i] >> 8;
            p[4 * i + 0] = as_h2((x & 0x000F000Fu) | magic) - hh(1032.f, 1032.f);
            p[4 * i + 1] = as_h2((x & 0x00F000F0u) | magic) - hh(1152.f, 1152.f);
            p[4 * i + 2] = as_h2((x8 & 0x000F000Fu) | magic) - hh(1032.f, 1032.f);
            p[4 * i + 3] = as_h2((x8 & 0x00F000F0u) | magic) - hh(1152.f, 1152.f);
        }
    }
    __device__ static float dot(const h2 (&p)[NP], const QReg& r) {
        float a1 = fdot2_z(p[0], r.q[0]), a16 = fdot2_z(p[1], r.q[1]);
        a1  = __builtin_amdgcn_fdot2(p[2], r.q[2], a1, false);
        a16 = __builtin_amdgcn_fdot2(p[3], r.q[3], a16, false);
#pragma unroll
        for (int i = 1; i < 4; ++i) {
            a1  = __builtin_amdgcn_fdot2(p[4 * i + 0], r.q[4 * i + 0], a1, false);
            a16 = __builtin_amdgcn_fdot2(p[4 * i + 1], r.q[4 * i + 1], a16, false);
            a1  = __builtin_amdgcn_fdot2(p[4 * i + 2], r.q[4 * i + 2], a1, false);
            a16 = __builtin_amdgcn_fdot2(p[4 * i + 3], r.q[4 * i + 3], a16, false);
        }
        return __builtin_fmaf(a16, 0.0625f, a1);
    }
    static constexpr bool VFIX = true;
    // element 8i+j: nibble j; j = 1, 3, 5, 7 sit 4 bits up in their half (16c)
    __device__ static constexpr float voff(int e) { return (e & 1) ? -128.f / 16777216.f : -8.f / 16777216.f; }
    __device__ static void unpack_v(const u32x4& w, h2 (&p)[NP]) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t x = w[i], x8 = w[i] >> 8;
            p[4 * i + 0] = as_h2(x & 0x000F000Fu);
            p[4 * i + 1] = as_h2(x & 0x00F000F0u);
            p[4 * i + 2] = as_h2(x8 & 0x000F000Fu);
            p[4 * i + 3] = as_h2(x8 & 0x00F000F0u);
        }
    }
    __device__ static void axpy_v(const h2 (&p)[NP], float ev, float* o) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                o[8 * i + c]     = __builtin_fmaf(ev, (float)p[4 * i + c].x, o[8 * i + c]);
                o[8 * i + c + 4] = __builtin_fmaf(ev, (float)p[4 * i + c].y, o[8 * i + c + 4]);
            }
        }
    }
    __device__ static constexpr float fin(int e) { return (e & 1) ? 1048576.f : 16777216.f; }
};

// q3: 32 3-bit fields per lane, element e at bits [3e, 3e+3) of the lane's
// 96-bit little-endian word (v + 4). Eight 32-bit windows of that word (one
// alignbit/shift each) hold two pairs apiece: a field at bit r of the low half
// and one at bit 16 + r' of the high half, r, r' <= 7. The 16 pairs:
//   window s = 0, 6, 12, 36, 42, 48: (a, a+6) at (0, 18) and (a+1, a+7) at (3, 21), a = s/3
//   window s = 68, 74:               (a, a+4) at (4, 16) and (a+1, a+5) at (7, 19), a = (s+4)/3
// For K a pair becomes (2^r v, 2^r' v') exactly and goes through
// v_dot2_f32_f16 against an fp16 q pair pre-scaled per element by 2^(k - r):
// each product 2^r v * q 2^(k - r) = q v 2^k is exact in fp32, and the head's
// power of two k (max |q| * 2^k in [2^14, 2^15) over the whole head, so qs is
// the same in every lane) keeps every scaled q that matters normal; 2^-k is
// folded into qs. For V the masked window alone is the subnormal pair
// (c 2^(r-24), c' 2^(r'-24)), OFF = 4, and fin(e) = 2^(24-r).
struct Q3Pair { int a, b, s, r, rp; };
__device__ constexpr Q3Pair kQ3Pairs[16] = {
    {0, 6, 0, 0, 2},    {1, 7, 0, 3, 5},    {2, 8, 6, 0, 2},    {3, 9, 6, 3, 5},
    {4, 10, 12, 0, 2},  {5, 11, 12, 3, 5},  {12, 18, 36, 0, 2}, {13, 19, 36, 3, 5},
    {14, 20, 42, 0, 2}, {15, 21, 42, 3, 5}, {16, 22, 48, 0, 2}, {17, 23, 48, 3, 5},
    {24, 28, 68, 4, 0}, {25, 29, 68, 7, 3}, {26, 30, 74, 4, 0}, {27, 31, 74, 7, 3},
};
__device__ constexpr int q3_shift(int e) {          // r of element e in its pair
    for (int i = 0; i < 16; ++i) {
        if (kQ3Pairs[i].a == e) return kQ3Pairs[i].r;
        if (kQ3Pairs[i].b == e) return kQ3Pairs[i].rp;
    }
    return 0;
}

template <> struct Codec<KQ3> {
    static constexpr int EPL = 32, NP = 16;
    struct QReg { h2 q[NP]; float qs; };     // q[i] = (q_a 2^(k - r), q_b 2^(k - r')) of pair i
    // The funnel shifts are asm so that both pairs of a window share one
    // instruction: with the builtin, the compiler narrows a pair whose masked
    // bits all come from one dword to a separate shift (one extra op per
    // window, measured in the q3 loop).
    __device__ static uint32_t funnel(uint32_t hi, uint32_t lo, int s) {
        uint32_t r;
        asm("v_alignbit_b32 %0, %1, %2, %3" : "=v"(r) : "v"(hi), "v"(lo), "i"(s));
        return r;
    }
    __device__ static uint32_t window(const u32x3& w, int s) {
        if (s == 0) return w.x;
        if (s < 32) return funnel(w.y, w.x, s);
        if (s == 32) return w.y;
        if (s < 64) return funnel(w.z, w.y, s - 32);
        return w.z >> (s - 64);
    }
    template <int I>
    __device__ static h2 pair(const u32x3& w, uint32_t magic) {
        constexpr Q3Pair P = kQ3Pairs[I];
        constexpr uint32_t mask = (7u << P.r) | (7u << (16 + P.rp));
        return as_h2((window(w, P.s) & mask) | magic) -
               hh(1024.f + 4.f * (float)(1 << P.r), 1024.f + 4.f * (float)(1 << P.rp));
    }
    template <int I>
    __device__ static h2 vpair(const u32x3& w) {
        constexpr Q3Pair P = kQ3Pairs[I];
        constexpr uint32_t mask = (7u << P.r) | (7u << (16 + P.rp));
        return as_h2(window(w, P.s) & mask);
    }
    // The LP lanes of a row (aligned lane groups) hold the slices of one head.
    template <int LP>
    __device__ static void load_q(QReg& r, const uint16_t* qh, float qs) {
        uint32_t qw[16];
        load_q_words<32>(qw, qh);
        float x[32], mx = 0.f;
#pragma unroll
        for (int e = 0; e < 32; ++e) {
            x[e] = (e & 1) ? h2f_hi(qw[e / 2]) : h2f_lo(qw[e / 2]);
            mx = fmaxf(mx, __builtin_fabsf(x[e]));
        }
        mx = group_max<LP>(mx);                       // over the head
        // k: max |q| * 2^k in [2^14, 2^15) (frexp exponent e: mx = m 2^e, m in [0.5, 1));
        // an all-zero head keeps k = 0
        const int k = mx > 0.f ? 15 - __builtin_amdgcn_frexp_expf(mx) : 0;
#pragma unroll
        for (int i = 0; i < NP; ++i)
            r.q[i] = hh(__builtin_ldexpf(x[kQ3Pairs[i].a], k - kQ3Pairs[i].r),
                        __builtin_ldexpf(x[kQ3Pairs[i].b], k - kQ3Pairs[i].rp));
        r.qs = __builtin_ldexpf(qs, -k);
    }
    __device__ static uint32_t magic() { uint32_t m; VA_VGPR_CONST(m, 0x64006400); return m; }
    template <int... I>
    __device__ static void unpack_all(const u32x3& w, uint32_t magic, h2 (&p)[NP],
                                      std::integer_sequence<int, I...>) {
        ((p[I] = pair<I>(w, magic)), ...);
    }
    template <int... I>
    __device__ static void unpack_all_v(const u32x3& w, h2 (&p)[NP], std::integer_sequence<int, I...>) {
        ((p[I] = vpair<I>(w)), ...);
    }
    __device__ static void unpack_k(const u32x3& w, uint32_t magic, h2 (&p)[NP]) {
        unpack_all(w, magic, p, std::make_integer_sequence<int, NP>{});
    }
    __device__ static float dot(const h2 (&p)[NP], const QReg& r) { return dot_pairs<NP>(p, r.q); }
    static constexpr bool VFIX = true;
    __device__ static constexpr float voff(int e) { return -4.f * (float)(1 << q3_shift(e)) / 16777216.f; }
    __device__ static void unpack_v(const u32x3& w, h2 (&p)[NP]) {
        unpack_all_v(w, p, std::make_integer_sequence<int, NP>{});
    }
    __device__ static void axpy_v(const h2 (&p)[NP], float ev, float* o) {
#pragma unroll
        for (int i = 0; i < NP; ++i) {
            o[kQ3Pairs[i].a] = __builtin_fmaf(ev, (float)p[i].x, o[kQ3Pairs[i].a]);
            o[kQ3Pairs[i].b] = __builtin_fmaf(ev, (float)p[i].y, o[kQ3Pairs[i].b]);
        }
    }
    __device__ static constexpr float fin(int e) { return 16777216.f / (float)(1 << q3_shift(e)); }
};

} // namespace va
