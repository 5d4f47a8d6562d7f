// va_device.hpp — gfx950 device helpers shared by the decode, merge, probe and
// quantize kernels. CDNA4 only: wave64, raw buffer loads, DPP row ops.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace va {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float    f32x4 __attribute__((ext_vector_type(4)));

// Payload kinds. f16 / q8 / q4 / q3 are the reference's storage formats
// (src/voltattn.cu:676-692); "+" vs naive is a kernel choice, not a kind.
enum Kind : int { KF16 = 0, KQ8 = 1, KQ4 = 2, KQ3 = 3 };

template <int KIND> struct KindBits;
template <> struct KindBits<KF16> { static constexpr int num = 16; };
template <> struct KindBits<KQ8>  { static constexpr int num = 8; };
template <> struct KindBits<KQ4>  { static constexpr int num = 4; };
template <> struct KindBits<KQ3>  { static constexpr int num = 3; };

// Bytes of one D-element row of a kind.
template <int KIND, int D> struct RowBytes {
    static constexpr int value = D * KindBits<KIND>::num / 8;
};

// ------------------------------------------------------------ buffer loads --
// Raw buffer resource: base, no stride, `bytes` records. A load whose offset
// lies at or beyond `bytes` returns zeros without touching memory, which is
// how partial tiles at the end of a split are handled.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                             0x00020000);
}

// Cache policy bits of the streaming K/V loads (gfx950 CPol: 1 = sc0,
// 2 = nt, 16 = sc1). The K/V stream is read once, so it is loaded
// non-temporal (nt): measured ~12% faster than the default policy.
#ifndef VA_LOAD_AUX
#define VA_LOAD_AUX 2
#endif

// `soff` must be wave-uniform; it is pinned to an SGPR with readfirstlane so
// the compiler never wraps the load in a per-lane (waterfall) loop.
__device__ __forceinline__ uint32_t sgpr(uint32_t x) {
    return (uint32_t)__builtin_amdgcn_readfirstlane((int)x);
}
__device__ __forceinline__ u32x4 ld128(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, voff, sgpr(soff), VA_LOAD_AUX);
}
__device__ __forceinline__ u32x3 ld96(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b96(r, voff, sgpr(soff), VA_LOAD_AUX);
}
__device__ __forceinline__ uint32_t ld32(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, voff, sgpr(soff), 0);
}
__device__ __forceinline__ uint32_t ld16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, voff, sgpr(soff), 0);
}

// ------------------------------------------------- device-coherent access --
// Relaxed device-scope atomic stores/loads compile to global_store/load with
// sc1: the store is written through to the device coherence point and the
// load is served from it, so another work-group on any XCD sees the data
// without an L2 writeback or invalidate (which a device-scope fence would do).
__device__ __forceinline__ void store_dev(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_dev(const float* p) {
    return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_dev(unsigned* p, unsigned v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned load_dev(const unsigned* p) {
    return __hip_atomic_load(const_cast<unsigned*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// 64-bit forms: a relaxed atomic access is single-copy atomic, so a 32-bit
// value and a 32-bit tag stored together are always observed together.
__device__ __forceinline__ void store_dev(uint64_t* p, uint64_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t load_dev(const uint64_t* p) {
    return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Wait until every memory operation this wave issued has completed (for the
// sc1 stores above: reached the coherence point).
__device__ __forceinline__ void wait_all_mem() { __builtin_amdgcn_s_waitcnt(0); }

// ------------------------------------------------------------------ scalars --
__device__ __forceinline__ int uniform(int x) { return __builtin_amdgcn_readfirstlane(x); }
__device__ __forceinline__ size_t uniform64(size_t x) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)x);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(x >> 32));
    return ((size_t)hi << 32) | lo;
}
__device__ __forceinline__ float uniformf(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, x)));
}

// 2^x on the VALU transcendental unit (v_exp_f32). exp2(-inf) = 0.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ float h2f(uint32_t bits16) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}
__device__ __forceinline__ float h2f_lo(uint32_t w) { return h2f(w & 0xFFFFu); }
__device__ __forceinline__ float h2f_hi(uint32_t w) { return h2f(w >> 16); }
// Two consecutive fp16 values (lo, hi halves of v) at p, 4-byte aligned.
__device__ __forceinline__ void store_u32(uint16_t* p, uint32_t v) {
    *reinterpret_cast<uint32_t*>(p) = v;
}
__device__ __forceinline__ uint16_t f2h_rne(float x) {
    return __builtin_bit_cast(uint16_t, (_Float16)x);   // v_cvt_f16_f32, RNE mode
}

// --------------------------------------------------------------- DPP / swizzle --
// dpp_ctrl encodings (GCN3+ DPP): quad_perm, row rotate right, row mirrors.
constexpr int DPP_QP_XOR1 = 0xB1;       // quad_perm [1,0,3,2]
constexpr int DPP_QP_XOR2 = 0x4E;       // quad_perm [2,3,0,1]
constexpr int DPP_ROW_HALF_MIRROR = 0x141;
constexpr int DPP_ROW_MIRROR = 0x140;
constexpr int dpp_row_ror(int n) { return 0x120 + n; }   // n in 1..15

// All rows and banks enabled; bound_ctrl set, so a lane whose source is out
// of range reads 0 (the "old" operand is 0 as well, so the result is the same
// either way). With bound_ctrl set the compiler folds the move into the
// consuming add/max as one DPP instruction instead of a v_mov_b32_dpp plus a
// v_mov_b32 of the old value.
template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x),
                                                                 CTRL, 0xF, 0xF, true));
}

// Sum over aligned groups of N consecutive lanes (N in 1,2,4,8,16); every lane
// of the group receives the group total. Butterfly inside a DPP row: xor 1,
// xor 2, then half-row and full-row mirrors (each mirror pairs sub-blocks whose
// members already hold equal partial sums).
template <int N>
__device__ __forceinline__ float group_sum(float x) {
    static_assert(N == 1 || N == 2 || N == 4 || N == 8 || N == 16, "group size");
    if constexpr (N >= 2)  x += dpp<DPP_QP_XOR1>(x);
    if constexpr (N >= 4)  x += dpp<DPP_QP_XOR2>(x);
    if constexpr (N >= 8)  x += dpp<DPP_ROW_HALF_MIRROR>(x);
    if constexpr (N >= 16) x += dpp<DPP_ROW_MIRROR>(x);
    return x;
}

// ds_swizzle bit-mask mode: lane i reads lane ((i & and) | or) ^ xor within 32.
template <int XOR_MASK>
__device__ __forceinline__ float swz_xor(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, x),
                                                                 0x1F | (XOR_MASK << 10)));
}
__device__ __forceinline__ float lane_xor32(float x) {
    const int src = ((int)__lane_id() ^ 32) << 2;
    return __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(src, __builtin_bit_cast(int, x)));
}

// x combined over the four 16-lane rows (lanes l, l^16, l^32, l^48), in
// every lane, with gfx950's v_permlane16_swap / v_permlane32_swap (VALU, no LDS
// round trip). With both operands holding v, permlane16_swap leaves rows
// {v0, v0, v2, v2} and {v1, v1, v3, v3}, permlane32_swap halves {lo, lo} and
// {hi, hi} (probed on MI355X). Every lane gets (v0 (+) v1) (+) (v2 (+) v3), bit
// for bit the same. The swaps are written as inline asm on two read-write
// operands: this compiler's builtins lose the second result when both results
// feed one instruction. The s_nop before covers the VALU-write -> permlane-read
// wait states the compiler inserts for the builtin; the one after is spare.
__device__ __forceinline__ void permlane16_swap(unsigned& a, unsigned& b) {
    asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ void permlane32_swap(unsigned& a, unsigned& b) {
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ float rows_sum(float x) {
    unsigned a = __builtin_bit_cast(unsigned, x), b = a;
    permlane16_swap(a, b);
    x = __builtin_bit_cast(float, a) + __builtin_bit_cast(float, b);
    a = __builtin_bit_cast(unsigned, x);
    b = a;
    permlane32_swap(a, b);
    return __builtin_bit_cast(float, a) + __builtin_bit_cast(float, b);
}
__device__ __forceinline__ float rows_max(float x) {
    unsigned a = __builtin_bit_cast(unsigned, x), b = a;
    permlane16_swap(a, b);
    x = fmaxf(__builtin_bit_cast(float, a), __builtin_bit_cast(float, b));
    a = __builtin_bit_cast(unsigned, x);
    b = a;
    permlane32_swap(a, b);
    return fmaxf(__builtin_bit_cast(float, a), __builtin_bit_cast(float, b));
}

// Max over aligned groups of N consecutive lanes (N in 1,2,4,8,16), in every
// lane of the group; same butterfly as group_sum.
template <int N>
__device__ __forceinline__ float group_max(float x) {
    static_assert(N == 1 || N == 2 || N == 4 || N == 8 || N == 16, "group size");
    if constexpr (N >= 2)  x = fmaxf(x, dpp<DPP_QP_XOR1>(x));
    if constexpr (N >= 4)  x = fmaxf(x, dpp<DPP_QP_XOR2>(x));
    if constexpr (N >= 8)  x = fmaxf(x, dpp<DPP_ROW_HALF_MIRROR>(x));
    if constexpr (N >= 16) x = fmaxf(x, dpp<DPP_ROW_MIRROR>(x));
    return x;
}

// Full-wave max and sum (all 64 lanes receive the result).
__device__ __forceinline__ float wave_max(float x) {
    x = fmaxf(x, dpp<DPP_QP_XOR1>(x));
    x = fmaxf(x, dpp<DPP_QP_XOR2>(x));
    x = fmaxf(x, dpp<DPP_ROW_HALF_MIRROR>(x));
    x = fmaxf(x, dpp<DPP_ROW_MIRROR>(x));
    return rows_max(x);
}
__device__ __forceinline__ float wave_sum(float x) {
    return rows_sum(group_sum<16>(x));
}

// Sum / max over the 64/PW lanes of a wave that share lane % PW (PW in 1, 2,
// 4, 8, 16): DPP row rotations by PW, 2PW, .., 8 inside each 16-lane row, then
// the row swaps. Every lane receives its class's result; the sum's rounding
// order differs between the lanes of a class, but is fixed for each lane.
template <int PW>
__device__ __forceinline__ float column_sum(float x) {
    static_assert(PW == 1 || PW == 2 || PW == 4 || PW == 8 || PW == 16, "lane class");
    if constexpr (PW <= 1) x += dpp<dpp_row_ror(1)>(x);
    if constexpr (PW <= 2) x += dpp<dpp_row_ror(2)>(x);
    if constexpr (PW <= 4) x += dpp<dpp_row_ror(4)>(x);
    if constexpr (PW <= 8) x += dpp<dpp_row_ror(8)>(x);
    return rows_sum(x);
}
template <int PW>
__device__ __forceinline__ float column_max(float x) {
    static_assert(PW == 1 || PW == 2 || PW == 4 || PW == 8 || PW == 16, "lane class");
    if constexpr (PW <= 1) x = fmaxf(x, dpp<dpp_row_ror(1)>(x));
    if constexpr (PW <= 2) x = fmaxf(x, dpp<dpp_row_ror(2)>(x));
    if constexpr (PW <= 4) x = fmaxf(x, dpp<dpp_row_ror(4)>(x));
    if constexpr (PW <= 8) x = fmaxf(x, dpp<dpp_row_ror(8)>(x));
    return rows_max(x);
}

} // namespace va
