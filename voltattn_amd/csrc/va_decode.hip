// va_decode.hip — fused dequant + split-L decode attention for gfx950.
//
// One work-group (4 wave64) per (head h, split s) computes a log-sum-exp
// partial (m, l, o[D]) over positions [s*chunk, min(L, (s+1)*chunk)) of head h
// (flash-decoding; reference src/voltattn.cu:80-120, 122-649). A second pass
// (va_merge.hip) merges the S partials of each head.
//
// Tiled ("+") kernels. A position row of ROWB compressed bytes is read by LP
// lanes, each taking LB = 16 contiguous bytes (12 for q3) with one buffer
// load, so one wave-wide load instruction covers PPW = 64/LP consecutive rows
// (1 KiB; 768 B for q3) with no gaps. Each lane dequantizes its EPL elements in
// registers (bit ops, one convert and one FMA per element), the partial dot is
// summed over the LP lanes with DPP row ops, and the online softmax runs in
// fp32 in log2 units (q is pre-scaled by log2(e)/sqrt(D), exponentials are
// v_exp_f32). Per wave and iteration U rows per lane are in flight for K and
// V, and the next tile is prefetched into registers while the current one is
// computed. The fp16 group scales of a wave's tile are fetched with one
// coalesced load per tensor and staged once in LDS as (k, v) pairs.
//
// The running maximum is shared by the whole wave and is raised lazily: a
// rescale (one cross-lane max and a multiply of l and o) happens only when a
// new score exceeds it by more than RESCALE_SLACK (log2 units), so weights
// stay <= 2^RESCALE_SLACK and most tiles skip the rescale entirely. (o, l, m)
// always describe the same normalised value, so the result is unchanged.
//
// Codes become exact fp16 values two at a time with bit operations and feed
// v_dot2_f32_f16 / v_fma_mix_f32 directly (see the lane codecs), so no
// separate convert or offset correction runs per element.
//
// Naive kernels (f16, q8, q4): one wave64 per position, D/64 elements per
// lane, a 6-step cross-lane sum and an exact per-position online-softmax
// update — the attribution control of the reference's attn_f16/q8/q4
// (src/voltattn.cu:122-320).
#include "va_device.hpp"
#include "va_kernels.hpp"

#include <algorithm>
#include <cstdlib>
#include <utility>

namespace va {

constexpr int WAVES = 4;                 // waves per work-group
constexpr float RESCALE_SLACK = 8.0f;    // log2 units: weights stay <= 256
constexpr float M_INIT = -1e30f;         // finite "no score yet" maximum

// Ticket lines and partial store of the fused merge (zero-initialised with
// the code object; layout in va_kernels.hpp).
__device__ __align__(256) unsigned g_tickets[TICKET_SLOTS * TICKET_MAXH * TICKET_STRIDE];
__device__ __align__(256) uint64_t g_parts[(size_t)TICKET_SLOTS * PART_CAP * PART_STRIDE];

constexpr int POLL_MAX    = 1 << 12;     // bound on re-reads of one in-flight word

__device__ __forceinline__ uint64_t tagged(float v, uint32_t tag) {
    return ((uint64_t)tag << 32) | __builtin_bit_cast(uint32_t, v);
}
__device__ __forceinline__ bool tag_ok(uint64_t w, uint32_t tag) { return (uint32_t)(w >> 32) == tag; }
__device__ __forceinline__ float tag_val(uint64_t w) { return __builtin_bit_cast(float, (uint32_t)w); }

// 16 bytes (two tagged words) from the device coherence point (sc1, as the
// relaxed agent-scope loads above). The compiler tracks these like any buffer
// load, so a round of them is in flight at once.
__device__ __forceinline__ u32x4 ld128_dev(__amdgpu_buffer_rsrc_t r, uint32_t voff) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, voff, 0, 16 /* sc1 */);
}

// The call epoch of head h on this call's ticket slot; read at kernel start
// (the merge of this call advances it only after every group has arrived).
__device__ __forceinline__ unsigned read_epoch(const DecodeArgs& a, int h) {
    if (a.ticket_slot < 0) return 0u;
    return load_dev(g_tickets + ((size_t)a.ticket_slot * TICKET_MAXH + h) * TICKET_STRIDE + 1);
}

// End of a work-group (head h, split s) of NT threads: thread t < D holds
// o[t] = acc of the group's partial (m, l, o), and each such thread also holds
// m and l.
//
// Two-pass form (ticket_slot < 0): the partial goes to ws for the merge pass.
//
// Fused form: every value of the partial is stored as one 64-bit word
// (tag << 32 | fp32 bits), tag = (epoch << 9 | h << 1 | 1), unique per head
// and call and never zero; a partial is PART_STRIDE words: m, l, o[0..D).
// Thread NT-1 (which stores nothing, so its wait covers only its own atomic)
// takes the head's ticket without waiting for the stores to complete; the
// group that completes the ticket merges. It keeps its own partial in LDS and
// reads the others with 16-byte coherent loads, each carrying two words; a
// word whose tag is stale belongs to a group that has already arrived and
// issued its stores, so it is re-read (bounded) until it lands.
//
// The merge spreads the loads over all NT/64 waves, so each wave issues only
// 1 + ceil(S / (NT/64)) loads (coherent loads are serviced one instruction at
// a time): lane j of every wave reads split j's (m, l); wave w folds splits
// j = w, w + NW, ... in increasing order into lane-pair columns (2i, 2i+1)
// with split j's weight read by readlane; the NW wave sums are added in wave
// order through LDS. The order is fixed, so the result does not depend on
// arrival order. Needs S <= 64.
template <int D, int NT>
__device__ void finish_partial(const DecodeArgs& a, int h, int s, float M, float ls, float acc,
                               unsigned epoch) {
    constexpr int NW = NT / 64;
    constexpr int R  = 4;                       // o-pair loads per wave per round
    constexpr uint32_t PB = PART_STRIDE * 8;    // bytes per partial (16-byte multiple)
    static_assert(PB % 16 == 0 && D + 2 <= PART_STRIDE, "partial layout");
    const int t = (int)threadIdx.x;
    if (a.ticket_slot < 0) {
        if (t < D) {
            float* slot = a.ws + ((size_t)h * a.S + s) * (D + 2);
            store_dev(slot + 2 + t, acc);
            if (t == 0) {
                store_dev(slot, M);
                store_dev(slot + 1, ls);
            }
        }
        return;
    }
    __shared__ int   s_last, s_bad;
    __shared__ float s_own[D + 2];              // o[0..D), m, l of this group
    __shared__ float s_fold[NW][D];
    unsigned* ticket = g_tickets + ((size_t)a.ticket_slot * TICKET_MAXH + h) * TICKET_STRIDE;
    if (t == NT - 1)
        s_last = __hip_atomic_fetch_add(ticket, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                 (unsigned)(a.S - 1);
    const uint32_t tag = (epoch << 9) | ((uint32_t)h << 1) | 1u;
    uint64_t* part = g_parts + ((size_t)a.ticket_slot * PART_CAP + (size_t)h * a.S) * PART_STRIDE;
    if (t < D) {
        uint64_t* mine = part + (size_t)s * PART_STRIDE;
        store_dev(mine + 2 + t, tagged(acc, tag));
        s_own[t] = acc;
        if (t == 0) {
            store_dev(mine, tagged(M, tag));
            store_dev(mine + 1, tagged(ls, tag));
            s_own[D] = M;
            s_own[D + 1] = ls;
            s_bad = 0;
        }
    }
    __syncthreads();
    if (!s_last) return;

    const int w    = uniform(t >> 6);
    const int lane = t & 63;
    const int dp   = min(lane, D / 2 - 1);     // o pair of this lane: dims 2dp, 2dp + 1
    const __amdgpu_buffer_rsrc_t rp = make_rsrc(part, (uint32_t)a.S * PB);
    bool good;

    // (m, l) of split `lane` (words 0, 1 of its partial).
    const int jl = min(lane, a.S - 1);
    u32x4 ml = ld128_dev(rp, (uint32_t)jl * PB);
    // First round of this wave's o pairs, issued together with (m, l).
    u32x4 op[R];
    auto load_round = [&](int j0) {
#pragma unroll
        for (int i = 0; i < R; ++i) {
            const int j = j0 + NW * i;           // wave-uniform: no load past the last split
            if (j < a.S) op[i] = ld128_dev(rp, (uint32_t)j * PB + 16u + (uint32_t)dp * 16u);
        }
    };
    load_round(w);
    // Selection is branch-free and the rare re-read loop is wave-uniform (all
    // lanes run it, stale lanes take the new value), so no loaded value has to
    // survive a divergent branch.
    // The words are taken out of the vector right after each load (the
    // compiler mis-tracked a 16-byte value carried through the re-read loop).
    const bool in_s = lane < a.S, own = lane == s;
    uint32_t mv = ml.x, mt = ml.y, lv = ml.z, lt = ml.w;
    for (int k = 0; k < POLL_MAX; ++k) {          // rare: stores still in flight
        const bool need = in_s && !own && !(mt == tag && lt == tag);
        if (__builtin_amdgcn_ballot_w64(need) == 0) break;
        __builtin_amdgcn_s_sleep(2);
        const u32x4 re = ld128_dev(rp, (uint32_t)jl * PB);
        const uint32_t rmv = re.x, rmt = re.y, rlv = re.z, rlt = re.w;
        mv = need ? rmv : mv;
        mt = need ? rmt : mt;
        lv = need ? rlv : lv;
        lt = need ? rlt : lt;
    }
    good = !in_s || own || (mt == tag && lt == tag);
    const float own_m = s_own[D], own_l = s_own[D + 1];
    const float mj = !in_s ? -__builtin_inff() : own ? own_m : __builtin_bit_cast(float, mv);
    const float lj = !in_s ? 0.f : own ? own_l : __builtin_bit_cast(float, lv);
    const float mx   = wave_max(mj);
    const float wj   = fast_exp2(mj - mx);      // weight of split `lane` (0 past S)
    const float lsum = wave_sum(wj * lj);
    float o0 = 0.f, o1 = 0.f;
    for (int j0 = w; j0 < a.S; j0 += NW * R) {
        if (j0 != w) load_round(j0);
#pragma unroll
        for (int i = 0; i < R; ++i) {
            const int j = j0 + NW * i;           // wave-uniform
            if (j >= a.S) break;
            float v0, v1;
            if (j == s) {                        // wave-uniform
                v0 = s_own[2 * dp];
                v1 = s_own[2 * dp + 1];
            } else {
                uint32_t a0 = op[i].x, t0 = op[i].y, a1 = op[i].z, t1 = op[i].w;
                for (int k = 0; k < POLL_MAX; ++k) {
                    const bool need = !(t0 == tag && t1 == tag);
                    if (__builtin_amdgcn_ballot_w64(need) == 0) break;
                    __builtin_amdgcn_s_sleep(2);
                    const u32x4 re = ld128_dev(rp, (uint32_t)j * PB + 16u + (uint32_t)dp * 16u);
                    const uint32_t ra0 = re.x, rt0 = re.y, ra1 = re.z, rt1 = re.w;
                    a0 = need ? ra0 : a0;
                    t0 = need ? rt0 : t0;
                    a1 = need ? ra1 : a1;
                    t1 = need ? rt1 : t1;
                }
                good = good && t0 == tag && t1 == tag;
                v0 = __builtin_bit_cast(float, a0);
                v1 = __builtin_bit_cast(float, a1);
            }
            const float f = __builtin_bit_cast(float,
                __builtin_amdgcn_readlane(__builtin_bit_cast(int, wj), j));
            o0 = __builtin_fmaf(f, v0, o0);
            o1 = __builtin_fmaf(f, v1, o1);
        }
    }
    if (lane < D / 2) {
        s_fold[w][2 * lane]     = o0;
        s_fold[w][2 * lane + 1] = o1;
    }
    // A lost partial (never observed within the poll bound) shows as NaN.
    if (__builtin_amdgcn_ballot_w64(!good) != 0 && lane == 0) s_bad = 1;
    __syncthreads();
    if (t < D) {
        float o = 0.f;
#pragma unroll
        for (int v = 0; v < NW; ++v) o += s_fold[v][t];
        a.out[(size_t)h * D + t] = s_bad ? (uint16_t)0x7E00u : f2h_rne(o / lsum);
    }
    if (t == 0) {                            // every arrival is in: reset for the slot's next call
        store_dev(ticket, 0u);
        store_dev(ticket + 1, epoch + 1u);
    }
}

// --------------------------------------------------------------- layouts ----
template <int KIND, int D> struct Tile {
    static constexpr int ROWB = RowBytes<KIND, D>::value;   // bytes per row
    static constexpr int LB   = KIND == KQ3 ? 12 : 16;      // bytes per lane per row
    static constexpr int LP   = ROWB / LB;                  // lanes per row
    static constexpr int PPW  = 64 / LP;                    // rows per wave load
    static constexpr int EPL  = D / LP;                     // elements per lane
    static_assert(ROWB % LB == 0 && 64 % LP == 0 && LP <= 16, "lane split");
};

// Rows per lane per tile and tensor (U). Each kind is instantiated for two
// depths; the dispatch below picks one per kind.
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

// ------------------------------------------------------------ lane codecs --
// A lane owns EPL consecutive elements of a row. Every codec turns the stored
// codes into exact fp16 values two at a time (bit ops only), so the arithmetic
// sees exactly the dequantized integers:
//   * K: v_dot2_f32_f16 against the unscaled fp16 q (f16, q8, q4: products of
//     two fp16 values are exact in fp32), or v_fma_mix_f32 against fp32 q (q3);
//   * V: v_fma_mix_f32, o_e += ev * code_e with an fp16 operand and fp32
//     accumulation (P.V stays fp32).
// The fp16 "magic" construction: OR-ing a code n (< 2^10 / 2^r) shifted left by
// r into the mantissa of 1024.0 (0x6400) gives 1024 + 2^r n exactly; one packed
// fp16 subtract of 1024 + 2^r * offset then leaves 2^r * v. The magic constant
// lives in a VGPR so mask-and-insert is one v_and_or_b32 (a gfx9 VOP3 reads one
// scalar constant; mask and magic cannot both be literals).
//
// Interface: QReg (the lane's q in codec form), load_q(QReg&, q slice, qs) with
// qs = log2(e)/sqrt(D), dot(w, QReg) -> q.k in log2 units, axpy(w, ev, o, QReg),
// finish(o) (per-element fix-up once at the end).
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ h2 as_h2(uint32_t x) { return __builtin_bit_cast(h2, x); }
__device__ __forceinline__ h2 hh(float a, float b) { return h2{(_Float16)a, (_Float16)b}; }

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

// f16: 8 halves per lane, element 2i+j in half j of dword i.
template <> struct Codec<KF16> {
    static constexpr int EPL = 8;
    struct QReg { h2 q[4]; float qs; };
    __device__ static void load_q(QReg& r, const uint16_t* qh, float qs) {
        uint32_t qw[4];
        load_q_words<8>(qw, qh);
#pragma unroll
        for (int i = 0; i < 4; ++i) r.q[i] = as_h2(qw[i]);
        r.qs = qs;
    }
    __device__ static float dot(const u32x4& w, const QReg& r) {
        float a = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) a = __builtin_amdgcn_fdot2(as_h2(w[i]), r.q[i], a, false);
        return a * r.qs;
    }
    __device__ static void axpy(const u32x4& w, float ev, float* o, const QReg&) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const h2 v = as_h2(w[i]);
            o[2 * i]     = __builtin_fmaf(ev, (float)v.x, o[2 * i]);
            o[2 * i + 1] = __builtin_fmaf(ev, (float)v.y, o[2 * i + 1]);
        }
    }
    __device__ static void finish(float*) {}
};

// q8: 16 int8 per lane, element 4i+b in byte b of dword i. xor 0x80 makes the
// bytes u = v + 128; v_perm_b32 places bytes (b0, b1) / (b2, b3) under the
// 0x64 magic byte: fp16 pair (1024 + u, 1024 + u'), minus 1152 -> (v, v').
template <> struct Codec<KQ8> {
    static constexpr int EPL = 16;
    struct QReg { h2 q[8]; float qs; uint32_t magic; };
    __device__ static void pairs(uint32_t w, uint32_t magic, h2& p01, h2& p23) {
        const uint32_t u = w ^ 0x80808080u;
        p01 = as_h2(__builtin_amdgcn_perm(magic, u, 0x04010400u)) - hh(1152.f, 1152.f);
        p23 = as_h2(__builtin_amdgcn_perm(magic, u, 0x04030402u)) - hh(1152.f, 1152.f);
    }
    __device__ static void load_q(QReg& r, const uint16_t* qh, float qs) {
        uint32_t qw[8];
        load_q_words<16>(qw, qh);
#pragma unroll
        for (int i = 0; i < 8; ++i) r.q[i] = as_h2(qw[i]);
        r.qs = qs;
        VA_VGPR_CONST(r.magic, 0x64646464);
    }
    __device__ static float dot(const u32x4& w, const QReg& r) {
        float a = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            h2 p01, p23;
            pairs(w[i], r.magic, p01, p23);
            a = __builtin_amdgcn_fdot2(p01, r.q[2 * i], a, false);
            a = __builtin_amdgcn_fdot2(p23, r.q[2 * i + 1], a, false);
        }
        return a * r.qs;
    }
    __device__ static void axpy(const u32x4& w, float ev, float* o, const QReg& r) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            h2 p01, p23;
            pairs(w[i], r.magic, p01, p23);
            o[4 * i + 0] = __builtin_fmaf(ev, (float)p01.x, o[4 * i + 0]);
            o[4 * i + 1] = __builtin_fmaf(ev, (float)p01.y, o[4 * i + 1]);
            o[4 * i + 2] = __builtin_fmaf(ev, (float)p23.x, o[4 * i + 2]);
            o[4 * i + 3] = __builtin_fmaf(ev, (float)p23.y, o[4 * i + 3]);
        }
    }
    __device__ static void finish(float*) {}
};

// q4: 32 nibbles per lane; element 8i+j sits in nibble j of dword i. Masking
// nibbles (0, 4) / (1, 5) in place and (2, 6) / (3, 7) after a shift by 8 under
// the 1024.0 magic gives the exact pairs
//   P0 = (e0, e4) = v,  P1 = (e1, e5) = 16v,  P2 = (e2, e6) = v,  P3 = (e3, e7) = 16v;
// the 16v pairs accumulate separately (scaled by 1/16 once) for K and use
// ev/16 for V.
template <> struct Codec<KQ4> {
    static constexpr int EPL = 32;
    struct QReg { h2 q0[4], q1[4], q2[4], q3[4]; float qs; uint32_t magic; };
    __device__ static void pairs(uint32_t w, uint32_t magic, h2& p0, h2& p1, h2& p2, h2& p3) {
        const uint32_t w8 = w >> 8;
        p0 = as_h2((w & 0x000F000Fu) | magic) - hh(1032.f, 1032.f);
        p1 = as_h2((w & 0x00F000F0u) | magic) - hh(1152.f, 1152.f);
        p2 = as_h2((w8 & 0x000F000Fu) | magic) - hh(1032.f, 1032.f);
        p3 = as_h2((w8 & 0x00F000F0u) | magic) - hh(1152.f, 1152.f);
    }
    __device__ static void load_q(QReg& r, const uint16_t* qh, float qs) {
        uint32_t qw[16];
        load_q_words<32>(qw, qh);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            // halves of elements 8i..8i+7: qw[4i] = (e0, e1), +1 = (e2, e3), +2 = (e4, e5), +3 = (e6, e7)
            r.q0[i] = as_h2(__builtin_amdgcn_perm(qw[4 * i + 2], qw[4 * i], 0x05040100u));      // (e0, e4)
            r.q1[i] = as_h2(__builtin_amdgcn_perm(qw[4 * i + 2], qw[4 * i], 0x07060302u));      // (e1, e5)
            r.q2[i] = as_h2(__builtin_amdgcn_perm(qw[4 * i + 3], qw[4 * i + 1], 0x05040100u));  // (e2, e6)
            r.q3[i] = as_h2(__builtin_amdgcn_perm(qw[4 * i + 3], qw[4 * i + 1], 0x07060302u));  // (e3, e7)
        }
        r.qs = qs;
        VA_VGPR_CONST(r.magic, 0x64006400);
    }
    __device__ static float dot(const u32x4& w, const QReg& r) {
        float a1 = 0.f, a16 = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            h2 p0, p1, p2, p3;
            pairs(w[i], r.magic, p0, p1, p2, p3);
            a1  = __builtin_amdgcn_fdot2(p0, r.q0[i], a1, false);
            a16 = __builtin_amdgcn_fdot2(p1, r.q1[i], a16, false);
            a1  = __builtin_amdgcn_fdot2(p2, r.q2[i], a1, false);
            a16 = __builtin_amdgcn_fdot2(p3, r.q3[i], a16, false);
        }
        return __builtin_fmaf(a16, 0.0625f, a1) * r.qs;
    }
    __device__ static void axpy(const u32x4& w, float ev, float* o, const QReg& r) {
        const float ev16 = ev * 0.0625f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            h2 p0, p1, p2, p3;
            pairs(w[i], r.magic, p0, p1, p2, p3);
            o[8 * i + 0] = __builtin_fmaf(ev,   (float)p0.x, o[8 * i + 0]);
            o[8 * i + 4] = __builtin_fmaf(ev,   (float)p0.y, o[8 * i + 4]);
            o[8 * i + 1] = __builtin_fmaf(ev16, (float)p1.x, o[8 * i + 1]);
            o[8 * i + 5] = __builtin_fmaf(ev16, (float)p1.y, o[8 * i + 5]);
            o[8 * i + 2] = __builtin_fmaf(ev,   (float)p2.x, o[8 * i + 2]);
            o[8 * i + 6] = __builtin_fmaf(ev,   (float)p2.y, o[8 * i + 6]);
            o[8 * i + 3] = __builtin_fmaf(ev16, (float)p3.x, o[8 * i + 3]);
            o[8 * i + 7] = __builtin_fmaf(ev16, (float)p3.y, o[8 * i + 7]);
        }
    }
    __device__ static void finish(float*) {}
};

// q3: 32 3-bit fields per lane, element e at bits [3e, 3e+3) of the lane's
// 96-bit little-endian word (v + 4). Eight 32-bit windows of that word (one
// alignbit/shift each) hold two pairs apiece: a field at bit r of the low half
// and one at bit 16 + r' of the high half, r, r' <= 7. The 16 pairs:
//   window s = 0, 6, 12, 36, 42, 48: (a, a+6) at (0, 18) and (a+1, a+7) at (3, 21), a = s/3
//   window s = 68, 74:               (a, a+4) at (4, 16) and (a+1, a+5) at (7, 19), a = (s+4)/3
// A pair becomes (2^r v, 2^r' v') exactly; K uses fp32 q pre-scaled by 2^-r,
// V accumulates 2^r v and finish() scales o_e by 2^-r once.
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
    static constexpr int EPL = 32;
    struct QReg { float q[32]; uint32_t magic; };
    __device__ static uint32_t window(const u32x3& w, int s) {
        if (s == 0) return w.x;
        if (s < 32) return __builtin_amdgcn_alignbit(w.y, w.x, s);
        if (s == 32) return w.y;
        if (s < 64) return __builtin_amdgcn_alignbit(w.z, w.y, s - 32);
        return w.z >> (s - 64);
    }
    template <int I>
    __device__ static h2 pair(const u32x3& w, uint32_t magic) {
        constexpr Q3Pair P = kQ3Pairs[I];
        constexpr uint32_t mask = (7u << P.r) | (7u << (16 + P.rp));
        return as_h2((window(w, P.s) & mask) | magic) -
               hh(1024.f + 4.f * (float)(1 << P.r), 1024.f + 4.f * (float)(1 << P.rp));
    }
    __device__ static void load_q(QReg& r, const uint16_t* qh, float qs) {
        uint32_t qw[16];
        load_q_words<32>(qw, qh);
#pragma unroll
        for (int e = 0; e < 32; ++e) {
            const float x = (e & 1) ? h2f_hi(qw[e / 2]) : h2f_lo(qw[e / 2]);
            r.q[e] = x * qs * (1.0f / (float)(1 << q3_shift(e)));
        }
        VA_VGPR_CONST(r.magic, 0x64006400);
    }
    template <int I>
    __device__ static void dot_pair(const u32x3& w, const QReg& r, float& a) {
        const h2 p = pair<I>(w, r.magic);
        a = __builtin_fmaf((float)p.x, r.q[kQ3Pairs[I].a], a);
        a = __builtin_fmaf((float)p.y, r.q[kQ3Pairs[I].b], a);
    }
    template <int I>
    __device__ static void axpy_pair(const u32x3& w, float ev, float* o, const QReg& r) {
        const h2 p = pair<I>(w, r.magic);
        o[kQ3Pairs[I].a] = __builtin_fmaf(ev, (float)p.x, o[kQ3Pairs[I].a]);
        o[kQ3Pairs[I].b] = __builtin_fmaf(ev, (float)p.y, o[kQ3Pairs[I].b]);
    }
    template <int... I>
    __device__ static float dot_all(const u32x3& w, const QReg& r, std::integer_sequence<int, I...>) {
        float a0 = 0.f, a1 = 0.f;
        ((I % 2 ? dot_pair<I>(w, r, a1) : dot_pair<I>(w, r, a0)), ...);
        return a0 + a1;
    }
    template <int... I>
    __device__ static void axpy_all(const u32x3& w, float ev, float* o, const QReg& r,
                                    std::integer_sequence<int, I...>) {
        (axpy_pair<I>(w, ev, o, r), ...);
    }
    __device__ static float dot(const u32x3& w, const QReg& r) {
        return dot_all(w, r, std::make_integer_sequence<int, 16>{});
    }
    __device__ static void axpy(const u32x3& w, float ev, float* o, const QReg& r) {
        axpy_all(w, ev, o, r, std::make_integer_sequence<int, 16>{});
    }
    __device__ static void finish(float* o) {
#pragma unroll
        for (int e = 0; e < 32; ++e) o[e] *= 1.0f / (float)(1 << q3_shift(e));
    }
};

// -------------------------------------------------------- tiled ("+") kernel --
template <int KIND, int D, int G, int U, int WAVES>
__global__ __launch_bounds__(WAVES * 64) void decode_tiled(DecodeArgs a) {
    using T = Tile<KIND, D>;
    using C = Codec<KIND>;
    using LoadT = typename LaneLoad<KIND>::type;
    constexpr int ROWB = T::ROWB, LB = T::LB, LP = T::LP, PPW = T::PPW, EPL = T::EPL;
    static_assert(EPL == C::EPL, "codec width");
    constexpr bool QUANT = KIND != KF16;
    constexpr int NG  = D / G;                   // scale groups per row
    constexpr int TW  = PPW * U;                 // rows per wave per iteration
    constexpr int TB  = TW * WAVES;              // rows per work-group per iteration
    constexpr int SCN = QUANT ? TW * NG : 1;     // (k, v) scale pairs per wave tile
    constexpr int SCE = !QUANT ? 1 : NG >= 2 ? SCN / 2 : SCN;  // scale dwords/halves per tensor
    constexpr int SCR = (SCE + 63) / 64;         // scale loads per lane per tensor
    static_assert(!QUANT || G % EPL == 0, "a lane's elements share one scale group");
    static_assert(SCE % 64 == 0 || SCR == 1, "scale entries fill whole wave loads");

    __shared__ uint32_t s_scale[WAVES][SCN];
    __shared__ float    s_red[WAVES * 4][D + 1];
    __shared__ float    s_l[WAVES * 4];
    __shared__ float    s_m[WAVES];

    const int wg   = blockIdx.x;
    const int h    = wg / a.S;
    const int s    = wg - h * a.S;
    const unsigned epoch = read_epoch(a, h);
    const int wave = uniform((int)(threadIdx.x >> 6));
    const int lane = (int)(threadIdx.x & 63);
    const int sl   = lane % LP;                  // lane within its row
    const int pw   = lane / LP;                  // row slot within a wave load
    const int g    = (sl * EPL) / G;             // scale group of this lane

    const int j0 = s * a.chunk;
    const int n  = min(a.L - j0, a.chunk);       // rows of this split (<= 0: empty)

    float m = M_INIT, l = 0.f;
    float o[EPL];
#pragma unroll
    for (int e = 0; e < EPL; ++e) o[e] = 0.f;

    if (n > 0) {
        const size_t row0 = (size_t)h * a.L + j0;
        const __amdgpu_buffer_rsrc_t rk = make_rsrc(a.k + row0 * ROWB, (uint32_t)n * ROWB);
        const __amdgpu_buffer_rsrc_t rv = make_rsrc(a.v + row0 * ROWB, (uint32_t)n * ROWB);
        __amdgpu_buffer_rsrc_t rsk = rk, rsv = rv;
        if constexpr (QUANT) {
            rsk = make_rsrc(a.sk + row0 * NG, (uint32_t)n * NG * 2);
            rsv = make_rsrc(a.sv + row0 * NG, (uint32_t)n * NG * 2);
        }

        const uint32_t lane_off = (uint32_t)(pw * ROWB + sl * LB);
        const int niter = (n + TB - 1) / TB;

        // Two register stages (A, B) alternate: while one tile is computed the
        // next one is already in flight, and no register copy ever waits on it.
        LoadT ka[U], va_[U], kb[U], vb[U];
        uint32_t ska[SCR], sva[SCR], skb[SCR], svb[SCR];

        // Issue order is pinned (scales, then K, then V) so the prologue and the
        // loop leave the same pending-load sequence and the waits stay partial.
        auto load_tile = [&](int it, LoadT* kk, LoadT* vv, uint32_t* sk, uint32_t* sv) {
            const uint32_t tpos = sgpr((uint32_t)(it * TB + wave * TW));   // wave-uniform
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (QUANT) {            // lanes past SCE repeat the last entry (unused)
#pragma unroll
                for (int r = 0; r < SCR; ++r) {
                    const uint32_t sidx = (uint32_t)min(lane + 64 * r, SCE - 1);
                    if constexpr (NG >= 2) {
                        sk[r] = ld32(rsk, sidx * 4, tpos * NG * 2);
                        sv[r] = ld32(rsv, sidx * 4, tpos * NG * 2);
                    } else {
                        sk[r] = ld16(rsk, sidx * 2, tpos * 2);
                        sv[r] = ld16(rsv, sidx * 2, tpos * 2);
                    }
                }
            }
#pragma unroll
            for (int u = 0; u < U; ++u)
                kk[u] = lane_load<KIND>(rk, lane_off + (uint32_t)(u * PPW * ROWB), tpos * ROWB);
#pragma unroll
            for (int u = 0; u < U; ++u)
                vv[u] = lane_load<KIND>(rv, lane_off + (uint32_t)(u * PPW * ROWB), tpos * ROWB);
            __builtin_amdgcn_sched_barrier(0);
        };

        // The first tile is issued before q is read, so the two latencies overlap.
        load_tile(0, ka, va_, ska, sva);

        // q slice of this lane (dims [sl*EPL, sl*EPL + EPL)) in codec form.
        typename C::QReg qr;
        C::load_q(qr, a.q + (size_t)h * D + sl * EPL, a.qscale);

        auto stage_scales = [&](const uint32_t* sk, const uint32_t* sv) {  // (k | v << 16) pairs
            if constexpr (QUANT) {
#pragma unroll
                for (int r = 0; r < SCR; ++r) {
                    const int e = lane + 64 * r;
                    if (e < SCE) {
                        if constexpr (NG >= 2) {
                            s_scale[wave][2 * e]     = __builtin_amdgcn_perm(sv[r], sk[r], 0x05040100u);
                            s_scale[wave][2 * e + 1] = __builtin_amdgcn_perm(sv[r], sk[r], 0x07060302u);
                        } else {
                            s_scale[wave][e] = (sk[r] & 0xFFFFu) | (sv[r] << 16);
                        }
                    }
                }
            }
        };

        auto compute_tile = [&](int it, const LoadT* kk, const LoadT* vv) {
            const int rem = uniform(n - it * TB - wave * TW);   // valid rows of this wave tile
            float sc[U];
            uint32_t pair[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int slot = u * PPW + pw;
                float d = C::dot(kk[u], qr);
                pair[u] = 0;
                if constexpr (QUANT) {
                    pair[u] = s_scale[wave][slot * NG + g];
                    d *= h2f_lo(pair[u]);
                }
                d = group_sum<LP>(d);
                sc[u] = slot < rem ? d : -__builtin_inff();
            }
            float tmax = sc[0];
#pragma unroll
            for (int u = 1; u < U; ++u) tmax = fmaxf(tmax, sc[u]);
            if (__builtin_amdgcn_ballot_w64(tmax > m + RESCALE_SLACK)) {
                const float mn = uniformf(wave_max(fmaxf(m, tmax)));
                const float c  = fast_exp2(m - mn);
                l *= c;
#pragma unroll
                for (int e = 0; e < EPL; ++e) o[e] *= c;
                m = mn;
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const float p = fast_exp2(sc[u] - m);
                l += p;
                float ev = p;
                if constexpr (QUANT) ev = p * h2f_hi(pair[u]);
                C::axpy(vv[u], ev, o, qr);
            }
        };

        // Tiles are processed in pairs. Loads past the end of the split return
        // zeros without memory traffic and their scores are masked, so the
        // prefetch after the last tile and the empty tile that completes an
        // odd count add no traffic and leave (m, l, o) unchanged.
        const int npair = (niter + 1) / 2;
        for (int ip = 0; ip < npair; ++ip) {
            const int it = 2 * ip;
            stage_scales(ska, sva);
            load_tile(it + 1, kb, vb, skb, svb);
            compute_tile(it, ka, va_);
            stage_scales(skb, svb);
            load_tile(it + 2, ka, va_, ska, sva);
            compute_tile(it + 1, kb, vb);
        }
        C::finish(o);
    }

    // ---- work-group merge: slots of a DPP row first, then rows/waves via LDS.
#pragma unroll
    for (int off = LP; off < 16; off *= 2) {
        if (off == 1) { l += dpp<dpp_row_ror(1)>(l); for (int e = 0; e < EPL; ++e) o[e] += dpp<dpp_row_ror(1)>(o[e]); }
        if (off == 2) { l += dpp<dpp_row_ror(2)>(l); for (int e = 0; e < EPL; ++e) o[e] += dpp<dpp_row_ror(2)>(o[e]); }
        if (off == 4) { l += dpp<dpp_row_ror(4)>(l); for (int e = 0; e < EPL; ++e) o[e] += dpp<dpp_row_ror(4)>(o[e]); }
        if (off == 8) { l += dpp<dpp_row_ror(8)>(l); for (int e = 0; e < EPL; ++e) o[e] += dpp<dpp_row_ror(8)>(o[e]); }
    }
    const int row = lane >> 4;
    if ((lane & 15) < LP) {                       // one slot per 16-lane row holds the row sum
#pragma unroll
        for (int e = 0; e < EPL; ++e) s_red[wave * 4 + row][sl * EPL + e] = o[e];
        if (sl == 0) s_l[wave * 4 + row] = l;
    }
    if (lane == 0) s_m[wave] = m;
    __syncthreads();
    const int t = (int)threadIdx.x;
    float M = 0.f, acc = 0.f, ls = 0.f;
    if (t < D) {
        M = s_m[0];
#pragma unroll
        for (int w = 1; w < WAVES; ++w) M = fmaxf(M, s_m[w]);
        float f[WAVES];
#pragma unroll
        for (int w = 0; w < WAVES; ++w) f[w] = fast_exp2(s_m[w] - M);
#pragma unroll
        for (int r = 0; r < WAVES * 4; ++r) acc = __builtin_fmaf(f[r / 4], s_red[r][t], acc);
#pragma unroll
        for (int r = 0; r < WAVES * 4; ++r) ls = __builtin_fmaf(f[r / 4], s_l[r], ls);
    }
    finish_partial<D, WAVES * 64>(a, h, s, M, ls, acc, epoch);
}

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
    const unsigned epoch = read_epoch(a, h);
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
    float M = 0.f, acc = 0.f, ls = 0.f;
    if (t < D) {
        M = s_m[0];
#pragma unroll
        for (int w = 1; w < WAVES; ++w) M = fmaxf(M, s_m[w]);
#pragma unroll
        for (int w = 0; w < WAVES; ++w) {
            const float f = fast_exp2(s_m[w] - M);
            acc = __builtin_fmaf(f, s_o[w][t], acc);
            ls  = __builtin_fmaf(f, s_l[w], ls);
        }
    }
    finish_partial<D, WAVES * 64>(a, h, s, M, ls, acc, epoch);
}

// ---------------------------------------------------------------- dispatch --
// Tiled configuration per kind: waves per group and tile depth (UnrollSet a or
// b), measured at H=32 D=128 over L = 4K..64K on MI355X. Every default keeps
// the same bytes in flight per CU (8 waves x depth a); fewer, deeper groups
// mean fewer partials to merge and a shorter dispatch. VA_WAVES=4|8 and
// VA_UNROLL=a|b in the environment override the defaults (tuning switches,
// read once).
struct TiledCfg { int waves; bool deep; };

static TiledCfg default_cfg(int kind) {
    switch (kind) {
        case KF16: return {8, false};    // 8 waves x 4 rows
        case KQ8:  return {4, true};     // 4 waves x 4 rows
        case KQ4:  return {4, true};     // 4 waves x 4 rows
        default:   return {4, false};    // q3: 4 waves x 2 rows, two groups per CU
    }
}

static TiledCfg tiled_cfg(int kind) {
    static const int w = [] { const char* e = std::getenv("VA_WAVES");  return e ? e[0] : 0; }();
    static const int u = [] { const char* e = std::getenv("VA_UNROLL"); return e ? e[0] : 0; }();
    TiledCfg c = default_cfg(kind);
    if (w == '4' || w == '8') c.waves = w - '0';
    if (u == 'a' || u == 'b') c.deep = u == 'b';
    return c;
}

template <int KIND> static int unroll_of(bool deep) { return deep ? UnrollSet<KIND>::b : UnrollSet<KIND>::a; }

template <int KIND, int D>
static int tiled_positions(const TiledCfg& c) {
    return Tile<KIND, D>::PPW * unroll_of<KIND>(c.deep) * c.waves;
}

template <int KIND>
static int tiled_groups(const TiledCfg& c) {
    return std::max(1, 8 * UnrollSet<KIND>::a / (c.waves * unroll_of<KIND>(c.deep)));
}

int tile_positions(int kind, bool tiled, int D) {
    if (!tiled) return WAVES;
    const TiledCfg c = tiled_cfg(kind);
    switch (kind) {
        case KF16: return D == 128 ? tiled_positions<KF16, 128>(c) : tiled_positions<KF16, 64>(c);
        case KQ8:  return D == 128 ? tiled_positions<KQ8, 128>(c)  : tiled_positions<KQ8, 64>(c);
        case KQ4:  return D == 128 ? tiled_positions<KQ4, 128>(c)  : tiled_positions<KQ4, 64>(c);
        default:   return D == 128 ? tiled_positions<KQ3, 128>(c)  : tiled_positions<KQ3, 64>(c);
    }
}

int groups_per_cu(int kind, bool tiled) {
    if (!tiled) return 8;                 // naive: one position per wave, 32 waves per CU
    const TiledCfg c = tiled_cfg(kind);
    switch (kind) {
        case KF16: return tiled_groups<KF16>(c);
        case KQ8:  return tiled_groups<KQ8>(c);
        case KQ4:  return tiled_groups<KQ4>(c);
        default:   return tiled_groups<KQ3>(c);
    }
}

template <int KIND, int D, int G>
static hipError_t launch_one(bool tiled, int H, const DecodeArgs& a, hipStream_t st) {
    const dim3 grid((unsigned)(H * a.S)), block(256), block8(512);
    if (tiled) {
        constexpr int UA = UnrollSet<KIND>::a, UB = UnrollSet<KIND>::b;
        const TiledCfg c = tiled_cfg(KIND);
        if (c.waves == 8) {
            if (c.deep) hipLaunchKernelGGL((decode_tiled<KIND, D, G, UB, 8>), grid, block8, 0, st, a);
            else        hipLaunchKernelGGL((decode_tiled<KIND, D, G, UA, 8>), grid, block8, 0, st, a);
        } else {
            if (c.deep) hipLaunchKernelGGL((decode_tiled<KIND, D, G, UB, 4>), grid, block, 0, st, a);
            else        hipLaunchKernelGGL((decode_tiled<KIND, D, G, UA, 4>), grid, block, 0, st, a);
        }
    } else {
        if constexpr (KIND == KQ3) return hipErrorInvalidValue;
        else hipLaunchKernelGGL((decode_w1<KIND, D, G>), grid, block, 0, st, a);
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
    switch (kind) {
        case KF16: return launch_d<KF16>(tiled, H, D, G, a, stream);
        case KQ8:  return launch_d<KQ8>(tiled, H, D, G, a, stream);
        case KQ4:  return launch_d<KQ4>(tiled, H, D, G, a, stream);
        case KQ3:  return launch_d<KQ3>(tiled, H, D, G, a, stream);
        default:   return hipErrorInvalidValue;
    }
}

} // namespace va
