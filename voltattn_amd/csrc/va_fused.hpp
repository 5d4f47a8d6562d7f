// va_fused.hpp — end of a split-L work-group: the partial (m, l, o[D]) of each
// of its query heads, and the fused second pass (the last work-group of a
// merge group merges all of its partials, so one decode step is one kernel).
//
// The ticket lines and the partial store are file-static device arrays, so
// every translation unit that includes this header (one code object each)
// owns its own set of TICKET_SLOTS slots; the host binds a slot to each stream
// that calls (va_slots.hpp).
#pragma once
#include "va_device.hpp"
#include "va_kernels.hpp"

namespace va {

// Ticket lines and partial store of the fused merge (zero-initialised with
// the code object; layout in va_kernels.hpp).
static __device__ __align__(256) unsigned g_tickets[TICKET_SLOTS * TICKET_MAXH * TICKET_STRIDE];
static __device__ __align__(256) uint64_t g_parts[(size_t)TICKET_SLOTS * PART_CAP * PART_STRIDE];
// Plain fp32 partials of the counted protocol (their own store, so a stale
// word of one protocol is never read by the other).
static __device__ __align__(256) float g_partf[(size_t)TICKET_SLOTS * PART_CAP * PARTF_STRIDE];

constexpr int POLL_MAX = 1 << 12;   // bound on re-reads of one in-flight word

// Test builds only (a comparison library, never the product): every fused
// merge waits for something that never comes, a tag no partial carries or one
// more count than there are groups, so it gives up after its bounded wait,
// stores NaN and counts the loss; every kernel still exits normally.
#ifndef VA_TEST_LOSE_MERGES
#define VA_TEST_LOSE_MERGES 0
#endif

// Merges of this code object that gave up waiting for a partial (NaN output);
// read by the host through read_lost_merges().
static __device__ unsigned g_lost_merges;

static inline hipError_t read_lost_merges(unsigned* n) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(g_lost_merges));
    if (e != hipSuccess) return e;
    return hipMemcpy(n, p, sizeof(unsigned), hipMemcpyDeviceToHost);
}

__device__ __forceinline__ void count_lost_merge() {
    __hip_atomic_fetch_add(&g_lost_merges, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Tag of this call's partial words (va_kernels.hpp, TAG_EPOCH_BITS).
__device__ __forceinline__ uint32_t part_tag(unsigned epoch, int S) {
    return ((epoch & ((1u << TAG_EPOCH_BITS) - 1u)) << 7) | (uint32_t)S;
}

// Zero one slot's tagged partials (tag 0 is never current); a grid-stride
// fill kernel rather than a memset, so it may sit in a captured graph.
static __global__ __launch_bounds__(256) void clear_tagged_slot(int slot) {
    constexpr size_t N = (size_t)PART_CAP * PART_STRIDE;
    uint64_t* p = g_parts + (size_t)slot * N;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < N; i += (size_t)gridDim.x * 256) p[i] = 0;
}
static inline hipError_t launch_clear_tagged(int slot, hipStream_t stream) {
    if (slot < 0 || slot >= TICKET_SLOTS) return hipErrorInvalidValue;
    hipLaunchKernelGGL(clear_tagged_slot, dim3(256), dim3(256), 0, stream, slot);
    return hipGetLastError();
}

__device__ __forceinline__ uint64_t tagged(float v, uint32_t tag) {
    return ((uint64_t)tag << 32) | __builtin_bit_cast(uint32_t, v);
}

// 16 bytes (two tagged words, or four plain floats) from the device coherence
// point (sc1, as the relaxed agent-scope loads of va_device.hpp). The compiler
// tracks these like any buffer load, so a round of them is in flight at once.
__device__ __forceinline__ u32x4 ld128_dev(__amdgpu_buffer_rsrc_t r, uint32_t voff) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, voff, 0, 16 /* sc1 */);
}

// The call epoch of merge group mg on this call's ticket slot (the tagged
// protocol's tags); read at kernel start (the merge of this call advances it
// only after every group arrived). Only the tagged protocol (one query slot)
// uses it: with several slots nothing is read, so no coherent load sits in
// front of the work-group's first tile.
template <int QG>
__device__ __forceinline__ unsigned read_epoch(const DecodeArgs& a, int mg) {
    if constexpr (QG > 1) return 0u;
    if (a.ticket_slot < 0) return 0u;
    return load_dev(g_tickets + ((size_t)a.ticket_slot * TICKET_MAXH + mg) * TICKET_STRIDE + 1);
}

// Where a work-group's partials go. A merge group is the set of S splits of
// one (sequence, KV head, query sub-group); it owns QG query slots, of which
// the first nq are real query heads, with global (batch-flattened) indexes
// oh0, oh0 + 1, ...
struct Route {
    int mg;    // merge group = blockIdx.x / S
    int s;     // split
    int nq;    // valid query slots
    int oh0;   // global index of query slot 0: rows of q, out and ws
};

// Work-group of NT threads; thread t < D holds acc[q] = o[t] of query slot q's
// partial, and M[q], ls[q] (slots >= nq are ignored).
//
// Two-pass form (ticket_slot < 0): the partials go to ws[(oh0+q)*S + s].
//
// Fused form, two protocols (measured on MI355X): with one query slot per
// work-group the partials are tagged, so the merging work-group never waits
// for another group's stores to complete (finish_tagged); with several slots
// the merge reads QG*S partials and its bytes dominate, so the partials are
// plain fp32 (half the bytes) behind a count of completed stores
// (finish_counted): 0.9-1.8 us less per grouped step at Hq 32 / Hkv 8,
// L 65536, and 0.1-0.4 us more per one-slot step.

// Tagged protocol: every value of a partial is stored as one 64-bit word
// (tag << 32 | fp32 bits), tag = part_tag(epoch, S), never zero and, among the
// words ever stored at that address, current only for this call
// (va_kernels.hpp, TAG_EPOCH_BITS); a partial is PART_STRIDE words: m, l,
// o[0..D), and partial (q, s) of merge group mg sits at (mg*QG + q)*S + s.
// Thread NT-1 (which stores nothing, so its wait covers only its own atomic)
// takes the group's ticket without waiting for the stores to complete; the
// work-group that completes the ticket merges. It reads every partial, its
// own included, with 16-byte coherent loads, each carrying two words; a word
// whose tag is stale belongs to a group that has already arrived and issued
// its stores, so it is re-read (bounded) until it lands.
//
// A lone merging wave issues one instruction every few cycles, so the merge is
// written for few instructions per wave. Wave w of the NW = NT/64 waves owns
// the PW = D/2/NW o-pair columns [w*PW, (w+1)*PW) of the output: lane (jj, c)
// of its i-th load pair reads split j = i*SPI + jj (SPI = 64/PW splits per
// instruction): the (m, l) words and the o pair of column w*PW + c. Each lane
// weights its own splits (exp2(m_j - M), M the maximum over all splits); the
// lanes of a column are summed by a fixed butterfly (DPP row rotations, then
// the row swaps of rows_sum), which also sums l, and the wave stores its own
// columns: no LDS and no barrier after the ticket. Up to RB*SPI splits are
// held at once; more are folded in batches with the running maximum
// rescaled. The order is fixed, so the result does not depend on arrival
// order. A merged l of zero (no positions) gives a zero output; a non-finite
// one (an invalid input that the kernel flagged with l = NaN) gives NaN.
// Needs S <= 64.
template <int D, int NT, int QG>
__device__ void finish_tagged(const DecodeArgs& a, const Route& rt, const float (&M)[QG],
                              const float (&ls)[QG], const float (&acc)[QG], unsigned epoch) {
    static_assert(QG == 1, "the tagged protocol merges one query slot per work-group");
    constexpr int NW = NT / 64;
    constexpr int PW = D / 2 / NW;              // o pairs (columns) per wave
    constexpr int SPI = 64 / PW;                // splits per load instruction
    constexpr int RB = 4;                       // load pairs per batch
    constexpr uint32_t PB = PART_STRIDE * 8;    // bytes per partial (16-byte multiple)
    static_assert(PB % 16 == 0 && D + 2 <= PART_STRIDE, "partial layout");
    static_assert(PW >= 1 && PW <= 16 && (PW & (PW - 1)) == 0 && D / 2 == PW * NW, "columns per wave");
    const int t = (int)threadIdx.x;
    const int S = a.S, s = rt.s;
    __shared__ int s_last;
    unsigned* ticket = g_tickets + ((size_t)a.ticket_slot * TICKET_MAXH + rt.mg) * TICKET_STRIDE;
    if (t == NT - 1)
        s_last = __hip_atomic_fetch_add(ticket, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                 (unsigned)(S - 1);
    const uint32_t tag = part_tag(epoch, S);
    const uint32_t want = VA_TEST_LOSE_MERGES ? tag ^ 0x80000000u : tag;   // the merger's expected tag
    uint64_t* base = g_parts + ((size_t)a.ticket_slot * PART_CAP + (size_t)rt.mg * S) * PART_STRIDE;
    if (t < D && rt.nq > 0) {
        uint64_t* mine = base + (size_t)s * PART_STRIDE;
        store_dev(mine + 2 + t, tagged(acc[0], tag));
        if (t == 0) {
            store_dev(mine, tagged(M[0], tag));
            store_dev(mine + 1, tagged(ls[0], tag));
        }
    }
    __syncthreads();
    if (!s_last) return;

    const int w    = uniform(t >> 6);
    const int lane = t & 63;
    const int c    = w * PW + (lane % PW);      // this lane's o pair: dims 2c, 2c + 1
    const int jj   = lane / PW;                 // split within a load instruction
    const int ninst = (S + SPI - 1) / SPI;      // load pairs per wave (wave-uniform)
    const __amdgpu_buffer_rsrc_t rp = make_rsrc(base, (uint32_t)S * PB);
    float mx = 0.f, o0 = 0.f, o1 = 0.f, lw = 0.f;
    uint32_t stale = 0;
    for (int b0 = 0; b0 < ninst; b0 += RB) {     // one batch up to S = RB*SPI
        // The words are taken out of each 16-byte vector right after its load
        // (carrying the vectors through the re-read loop was mis-compiled).
        uint32_t mv[RB], mt[RB], lv[RB], lt[RB], a0[RB], t0[RB], a1[RB], t1[RB];
        auto load = [&]() {
#pragma unroll
            for (int i = 0; i < RB; ++i) {
                if (b0 + i < ninst) {           // wave-uniform
                    // lanes past S re-read split S-1 (weight 0)
                    const uint32_t off = (uint32_t)min((b0 + i) * SPI + jj, S - 1) * PB;
                    const u32x4 x = ld128_dev(rp, off);
                    mv[i] = x.x; mt[i] = x.y; lv[i] = x.z; lt[i] = x.w;
                    const u32x4 y = ld128_dev(rp, off + 16u + (uint32_t)c * 16u);
                    a0[i] = y.x; t0[i] = y.y; a1[i] = y.z; t1[i] = y.w;
                }
            }
        };
        auto stale_words = [&]() {
            uint32_t x = 0;
#pragma unroll
            for (int i = 0; i < RB; ++i)
                if (b0 + i < ninst) x |= (mt[i] ^ want) | (lt[i] ^ want) | (t0[i] ^ want) | (t1[i] ^ want);
            return x;
        };
        load();
        uint32_t st = stale_words();
        // Rare: a partial's stores still in flight. The loop is wave-uniform
        // and re-reads the whole batch (current words stay current).
        for (int k = 0; k < POLL_MAX; ++k) {
            if (__builtin_amdgcn_ballot_w64(st != 0) == 0) break;
            __builtin_amdgcn_s_sleep(2);
            load();
            st = stale_words();
        }
        stale |= st;
        float mi[RB];
        float bm = -__builtin_inff();
#pragma unroll
        for (int i = 0; i < RB; ++i) {
            if (b0 + i < ninst) {
                mi[i] = (b0 + i) * SPI + jj < S ? __builtin_bit_cast(float, mv[i]) : -__builtin_inff();
                bm = fmaxf(bm, mi[i]);
            }
        }
        bm = column_max<PW>(bm);                 // over every split of the batch
        if (b0 == 0) {
            mx = bm;
        } else {
            const float mn = fmaxf(mx, bm);
            const float r = fast_exp2(mx - mn);
            o0 *= r;
            o1 *= r;
            lw *= r;
            mx = mn;
        }
#pragma unroll
        for (int i = 0; i < RB; ++i) {
            if (b0 + i < ninst) {
                const float f = fast_exp2(mi[i] - mx);       // 0 past S
                o0 = __builtin_fmaf(f, __builtin_bit_cast(float, a0[i]), o0);
                o1 = __builtin_fmaf(f, __builtin_bit_cast(float, a1[i]), o1);
                lw = __builtin_fmaf(f, __builtin_bit_cast(float, lv[i]), lw);
            }
        }
    }
    o0 = column_sum<PW>(o0);
    o1 = column_sum<PW>(o1);
    lw = column_sum<PW>(lw);
    // A lost partial (never observed within the poll bound) shows as NaN in the
    // columns of every wave that saw it. Every wave reads every split's (m, l),
    // so a partial that never landed is seen by wave 0, which counts the merge
    // once for the host (va_merge_faults).
    const bool bad = __builtin_amdgcn_ballot_w64(stale != 0) != 0;
    if (lane < PW && rt.nq > 0) {
        // v_rcp_f32 (1 ulp): the fp16 result is rounded from o * r
        const float r = lw == 0.f ? 0.f : __builtin_amdgcn_rcpf(lw);
        const uint32_t h = bad ? 0x7E007E00u : ((uint32_t)f2h_rne(o0 * r) | ((uint32_t)f2h_rne(o1 * r) << 16));
        store_u32(a.out + (size_t)rt.oh0 * D + 2 * c, h);
    }
    // Every arrival is in: reset the slot for its next call (which runs after
    // this kernel, so no other wave needs to have finished).
    if (t == 0) {
        if (bad) count_lost_merge();
        store_dev(ticket, 0u);
        store_dev(ticket + 1, epoch + 1u);
    }
}

// Counted protocol: every work-group stores its partials as plain fp32 (o[0..D),
// m, l; PSF floats each, partial (q, s) of merge group mg at (mg*QG + q)*S + s)
// with device-coherent stores while thread NT-1 takes the merge group's ticket
// (word 0 of the group's ticket line), so the stores' round trip overlaps the
// ticket's. Every thread then waits until its stores (or the atomic) have
// completed, and after the barrier a work-group that did not complete the
// ticket counts itself in word 2 of the line. The work-group that completes the
// ticket merges from its own partials in LDS (its stores go unused), after
// waiting (bounded) until the other S-1 have counted: it waits only for groups
// that have already taken their ticket, so every wait ends.
//
// The merge spreads the loads over all NT/64 waves and runs the query slots
// side by side: WQ = NW/QG waves per slot; lane j of each of them reads split
// j's (m, l), and sub-wave sw folds splits j = sw, sw + WQ, ... into
// 4-dimension columns. Each 16-byte load instruction carries SPL = 256/D
// splits (one per D/4-lane block), each block weighted by its split's weight
// (readlane); the blocks are summed at the end by lane swaps, the WQ sub-wave
// sums in order through LDS. The order is fixed, so the result does not depend
// on arrival order. A merged l of zero (no positions)
// gives a zero output; a non-finite one (an invalid input that the kernel
// flagged with l = NaN) gives NaN, and so does a count that never completes
// within the poll bound. Needs S <= 64.
template <int D, int NT, int QG>
__device__ void finish_counted(const DecodeArgs& a, const Route& rt, const float (&M)[QG],
                               const float (&ls)[QG], const float (&acc)[QG]) {
    constexpr int NW = NT / 64;
    constexpr int PSF = D + 4;                   // floats per partial: o[D], m, l, 2 spare (16-byte rows)
    constexpr uint32_t PB = PSF * 4;
    static_assert(PSF <= PARTF_STRIDE, "partial store");
    const int t = (int)threadIdx.x;
    const int S = a.S, s = rt.s;
    constexpr int WQ = NW / QG;
    static_assert(NW >= QG && NW % QG == 0, "whole waves per query slot");
    __shared__ int   s_last, s_bad;
    __shared__ float s_own[QG][D + 2];
    __shared__ float s_fold[QG][WQ][D];
    __shared__ float s_lsum[QG];
    unsigned* line = g_tickets + ((size_t)a.ticket_slot * TICKET_MAXH + rt.mg) * TICKET_STRIDE;
    float* base = g_partf + (size_t)a.ticket_slot * PART_CAP * PARTF_STRIDE + (size_t)rt.mg * QG * S * PSF;
    if (t < D) {
#pragma unroll
        for (int q = 0; q < QG; ++q) {
            if (q >= rt.nq) break;
            float* mine = base + ((size_t)q * S + s) * PSF;
            store_dev(mine + t, acc[q]);
            if (t == 0) {
                store_dev(mine + D, M[q]);
                store_dev(mine + D + 1, ls[q]);
            }
        }
    }
    if (t == NT - 1)
        s_last = __hip_atomic_fetch_add(line, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                 (unsigned)(S - 1);
    // The stores are written through to the device coherence point (sc1): once
    // each thread has seen its own complete, the count may go up.
    wait_all_mem();
    __syncthreads();
    if (!s_last) {
        if (t == 0) __hip_atomic_fetch_add(line + 2, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
    }
    if (t < D) {
#pragma unroll
        for (int q = 0; q < QG; ++q) {
            if (q >= rt.nq) break;
            s_own[q][t] = acc[q];
            if (t == 0) {
                s_own[q][D] = M[q];
                s_own[q][D + 1] = ls[q];
            }
        }
    }
    if (t == 0) {                                // the other S - 1 partials stored?
        const unsigned need = (unsigned)(S - 1 + VA_TEST_LOSE_MERGES);
        unsigned n = load_dev(line + 2);
        for (int k = 0; k < POLL_MAX && n < need; ++k) {
            __builtin_amdgcn_s_sleep(2);
            n = load_dev(line + 2);
        }
        s_bad = n < need;
        if (s_bad) count_lost_merge();
    }
    __syncthreads();                             // the partial loads below are served from the coherence point (sc1)

    const int w    = uniform(t >> 6);
    const int lane = t & 63;
    const int qw   = w / WQ, sw = w - (w / WQ) * WQ;
    // Each load instruction carries SPL splits: lane = sub * NQD + dq reads the
    // 4 dimensions 4dq .. 4dq + 3 of split sw + WQ * (SPL * i + sub).
    constexpr int NQD = D / 4, SPL = 64 / NQD;
    constexpr int RI  = QG > 1 ? 8 : 2;          // load instructions per wave per batch
    const int dq  = lane % NQD, sub = lane / NQD;
    const int jl  = min(lane, S - 1);
    const bool in_s = lane < S, own = lane == s;
    if (qw < rt.nq) {                            // wave-uniform
        const __amdgpu_buffer_rsrc_t rp = make_rsrc(base + (size_t)qw * S * PSF, (uint32_t)S * PB);
        const int nsw = (S - sw + WQ - 1) / WQ;  // splits folded by this wave
        const int ni  = (nsw + SPL - 1) / SPL;   // load instructions
        // The words are taken out of each 16-byte vector right after its load
        // (an array of the vectors carried across the loop is mis-compiled).
        uint32_t op[RI][4];
        auto load_batch = [&](int b0) {
#pragma unroll
            for (int i = 0; i < RI; ++i) {
                if (b0 + i < ni) {               // wave-uniform
                    const int k = SPL * (b0 + i) + sub;
                    const int j = sw + WQ * min(k, nsw - 1);   // lanes past the last split reread it (weight 0)
                    const u32x4 x = ld128_dev(rp, (uint32_t)j * PB + (uint32_t)dq * 16u);
                    op[i][0] = x.x; op[i][1] = x.y; op[i][2] = x.z; op[i][3] = x.w;
                }
            }
        };
        const uint32_t mlv = __builtin_amdgcn_raw_buffer_load_b32(rp, (uint32_t)jl * PB + D * 4, 0, 16);
        const uint32_t llv = __builtin_amdgcn_raw_buffer_load_b32(rp, (uint32_t)jl * PB + D * 4 + 4, 0, 16);
        load_batch(0);
        asm volatile("" ::: "memory");
        const float own_m = s_own[qw][D], own_l = s_own[qw][D + 1];
        const float mj = !in_s ? -__builtin_inff() : own ? own_m : __builtin_bit_cast(float, mlv);
        const float lj = !in_s ? 0.f : own ? own_l : __builtin_bit_cast(float, llv);
        const float mx = wave_max(mj);
        const float wj = fast_exp2(mj - mx);    // weight of split `lane` (0 past S)
        const float lsum = wave_sum(wj * lj);
        float o4[4] = {0.f, 0.f, 0.f, 0.f};
        for (int b0 = 0; b0 < ni; b0 += RI) {
            if (b0 != 0) load_batch(b0);
#pragma unroll
            for (int i = 0; i < RI; ++i) {
                if (b0 + i >= ni) break;         // wave-uniform
                // weight of this lane's split: readlane per sub-block, then select
                float f = 0.f;
                bool mine = false;
#pragma unroll
                for (int r = 0; r < SPL; ++r) {
                    const int k = SPL * (b0 + i) + r;
                    const int j = sw + WQ * min(k, nsw - 1);
                    const float fr = k < nsw ? __builtin_bit_cast(float,
                        __builtin_amdgcn_readlane(__builtin_bit_cast(int, wj), j)) : 0.f;
                    f = sub == r ? fr : f;
                    mine = sub == r ? (k < nsw && j == s) : mine;
                }
                float v[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) v[e] = __builtin_bit_cast(float, op[i][e]);
                if (__builtin_amdgcn_ballot_w64(mine) != 0) {   // this group's own split: from LDS
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float ov = s_own[qw][4 * dq + e];
                        v[e] = mine ? ov : v[e];
                    }
                }
#pragma unroll
                for (int e = 0; e < 4; ++e) o4[e] = __builtin_fmaf(f, v[e], o4[e]);
            }
        }
        // sub-block sums in a fixed order: (s0 + s1) for SPL = 2, rows_sum for SPL = 4
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            if constexpr (SPL == 4) {
                o4[e] = rows_sum(o4[e]);
            } else {
                unsigned x = __builtin_bit_cast(unsigned, o4[e]), y = x;
                permlane32_swap(x, y);
                o4[e] = __builtin_bit_cast(float, x) + __builtin_bit_cast(float, y);
            }
        }
        if (lane < NQD) {
#pragma unroll
            for (int e = 0; e < 4; ++e) s_fold[qw][sw][4 * lane + e] = o4[e];
        }
        if (sw == 0 && lane == 0) s_lsum[qw] = lsum;
    }
    __syncthreads();
    if (t < D) {
#pragma unroll
        for (int q = 0; q < QG; ++q) {
            if (q >= rt.nq) break;
            float o = 0.f;
#pragma unroll
            for (int v = 0; v < WQ; ++v) o += s_fold[q][v][t];
            const float r = s_lsum[q] == 0.f ? 0.f : o / s_lsum[q];
            a.out[(size_t)(rt.oh0 + q) * D + t] = s_bad ? (uint16_t)0x7E00u : f2h_rne(r);
        }
    }
    if (t == 0) {                                // reset for the slot's next call
        store_dev(line, 0u);                     // every ticket of this call is taken
        // The S - 1 counts waited for are taken back rather than the word
        // zeroed: after a poll that gave up (NaN output), a count still on its
        // way then brings the word back to 0 instead of into the next call.
        __hip_atomic_fetch_sub(line + 2, (unsigned)(S - 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

template <int D, int NT, int QG>
__device__ void finish_partial(const DecodeArgs& a, const Route& rt, const float (&M)[QG],
                               const float (&ls)[QG], const float (&acc)[QG], unsigned epoch) {
    const int t = (int)threadIdx.x;
    const int S = a.S, s = rt.s;
    if (a.ticket_slot < 0) {
        if (t < D) {
#pragma unroll
            for (int q = 0; q < QG; ++q) {
                if (q >= rt.nq) break;
                float* slot = a.ws + ((size_t)(rt.oh0 + q) * S + s) * (D + 2);
                store_dev(slot + 2 + t, acc[q]);
                if (t == 0) {
                    store_dev(slot, M[q]);
                    store_dev(slot + 1, ls[q]);
                }
            }
        }
        return;
    }
    if constexpr (QG == 1) finish_tagged<D, NT, QG>(a, rt, M, ls, acc, epoch);
    else finish_counted<D, NT, QG>(a, rt, M, ls, acc);
}

} // namespace va
