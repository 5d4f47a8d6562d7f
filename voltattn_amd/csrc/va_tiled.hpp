// va_tiled.hpp — the tiled ("+") split-L decode kernel, shared by the
// reference-shape launches (va_decode.hip) and the grouped-query / paged
// launches (va_decode_ex.hip).
//
// One work-group of WAVES wave64 per (merge group, split) computes log-sum-exp
// partials (m, l, o[D]) over positions [s*chunk, min(L, (s+1)*chunk)) of one
// KV head, for QG query heads that share it (flash-decoding; reference
// src/voltattn.cu:80-120, 364-649, which has QG = 1 and contiguous K/V).
// Each lane takes LB = 16 contiguous bytes (12 for q3) of a row with one
// buffer load, so one wave-wide load instruction covers PPW = 64/LP rows with
// no gaps; each row is unpacked once into fp16 pairs (va_codec.hpp) and used
// by all QG query heads, the partial dot is summed over the LP lanes with DPP
// row ops, and the online softmax runs in fp32 in log2 units: scores stay raw
// (q.k times the group scale) and qs = log2(e)/sqrt(D) enters through the
// exponent's fma, exp2(score * qs - m) on v_exp_f32. Per wave and
// iteration U rows per lane are in flight for K and V, and the next tile is
// prefetched into registers while the current one is computed. The fp16 group
// scales of a wave's tile are fetched with one coalesced load per tensor and
// staged once in LDS as (k, v) pairs.
//
// The running maximum of each query head is shared by the whole wave and is
// raised lazily: a rescale (one cross-lane max and a multiply of l and o)
// happens only when a new score exceeds it by more than RESCALE_SLACK (log2
// units), so weights stay <= 2^RESCALE_SLACK and most tiles skip the rescale
// entirely. (o, l, m) always describe the same normalised value, so the
// result is unchanged.
//
// Contiguous form (PAGED = false): K/V rows of KV head hk are [hk][L][row];
// each work-group builds raw buffer resources covering exactly its split, so a
// load at or past the split end returns 0 with no memory access (partial
// tiles, and the prefetch beyond the last tile).
//
// Paged form: rows of sequence b live in pages of 2^page_shift rows, page p
// holding [hkv][page_rows][row] of the pool; position j of sequence b is row
// j mod page_rows of page block_table[b][j / page_rows]. Page sizes are
// multiples of the wave tile TW and splits start on work-group tiles, so every
// wave tile lies in one page; each wave tile gets its own buffer resources,
// clamped to the split (no access past it, so the prefetch beyond the last
// tile reads nothing, as in the contiguous form) and empty for a page id
// outside the pool (which also marks the output NaN). The page ids of a split
// are staged in LDS once.
#pragma once
#include "va_codec.hpp"
#include "va_fused.hpp"

#include <type_traits>

namespace va {

constexpr float RESCALE_SLACK = 8.0f;    // log2 units: weights stay <= 256
constexpr float M_INIT = -1e30f;         // finite "no score yet" maximum

// log2(e) / sqrt(D), as the host computes it (double, then rounded to float).
template <int D>
__device__ constexpr float qscale_of() {
    static_assert(D == 64 || D == 128, "head dimension");
    return (float)(1.4426950408889634074 / (D == 128 ? 11.313708498984760390 : 8.0));
}

// What the first tile needs comes first as plain scalars (14 dwords: k, v,
// sk, sv, L, S, chunk, slot, q), so the hardware preloads them into SGPRs
// before the wave starts (kernel argument preload) and the first loads issue
// without waiting for a kernarg fetch; dst (`out` for the fused merge, slot
// >= 0; `ws` for the two-pass form) and `rest` (grouped-query and paged
// fields) are read from the kernarg segment when needed.
// The last offset fix and the codec's rescale of one accumulator, one fma with
// compile-time constants: fma(o, fin(e), S * voff(e) * fin(e)) is exactly
// fix_v() followed by o *= fin(e) (va_codec.hpp).
template <class C, int E>
__device__ __forceinline__ void fix_finish_one(float& o, float s) {
    constexpr float f = C::fin(E);
    if constexpr (C::VFIX) {
        constexpr float k = C::voff(E) * C::fin(E);
        o = __builtin_fmaf(o, f, s * k);
    } else {
        o *= f;
    }
}
template <class C, int... E>
__device__ __forceinline__ void fix_finish(float* o, float s, std::integer_sequence<int, E...>) {
    (fix_finish_one<C, E>(o[E], s), ...);
}

// End of a split-L work-group: the per-lane state of every wave (m[q] wave-
// uniform, in log2 units; l[q] and o[q][EPL] over the lane's rows, l repeated
// on the LP lanes of a row) is folded into one partial (M, l, o[D]) per query
// slot — the slots of a DPP row first, then rows and waves via LDS — and
// handed to finish_partial. A paged tile with a bad page id in any wave
// (`bad`) marks every partial of the group (l = NaN).
template <int D, int LP, int EPL, int WAVES, int QG, bool PAGED>
__device__ __forceinline__ void group_finish(const DecodeArgs& a, const Route& rt, const float (&m)[QG],
                                             float (&l)[QG], float (&o)[QG][EPL], bool bad, unsigned epoch) {
    __shared__ float s_red[QG][WAVES * 4][D + 1];
    __shared__ float s_l[QG][WAVES];
    __shared__ float s_m[QG][WAVES];
    const int wave = uniform((int)(threadIdx.x >> 6));
    const int lane = (int)(threadIdx.x & 63);
    const int sl   = lane % LP;
#pragma unroll
    for (int q = 0; q < QG; ++q) {
#pragma unroll
        for (int off = LP; off < 16; off *= 2) {
            if (off == 1) { l[q] += dpp<dpp_row_ror(1)>(l[q]); for (int e = 0; e < EPL; ++e) o[q][e] += dpp<dpp_row_ror(1)>(o[q][e]); }
            if (off == 2) { l[q] += dpp<dpp_row_ror(2)>(l[q]); for (int e = 0; e < EPL; ++e) o[q][e] += dpp<dpp_row_ror(2)>(o[q][e]); }
            if (off == 4) { l[q] += dpp<dpp_row_ror(4)>(l[q]); for (int e = 0; e < EPL; ++e) o[q][e] += dpp<dpp_row_ror(4)>(o[q][e]); }
            if (off == 8) { l[q] += dpp<dpp_row_ror(8)>(l[q]); for (int e = 0; e < EPL; ++e) o[q][e] += dpp<dpp_row_ror(8)>(o[q][e]); }
        }
        // The sums are used only by the lanes that write them out; computed
        // here in every lane, each add stays one DPP instruction (sunk into
        // the write-out branch it would be a DPP move plus an add).
        asm volatile("" : "+v"(l[q]));
#pragma unroll
        for (int e = 0; e < EPL; ++e) asm volatile("" : "+v"(o[q][e]));
    }
    const int row = lane >> 4;
    if ((lane & 15) < LP) {                       // one slot per 16-lane row holds the row sum
#pragma unroll
        for (int q = 0; q < QG; ++q) {
#pragma unroll
            for (int e = 0; e < EPL; ++e) s_red[q][wave * 4 + row][sl * EPL + e] = o[q][e];
        }
    }
    // l: every lane holds its row's sum; the rows are summed in the wave (row
    // swaps), so the fold below takes one l per wave.
    float lw[QG];
#pragma unroll
    for (int q = 0; q < QG; ++q) lw[q] = rows_sum(l[q]);
    if (lane == 0) {
#pragma unroll
        for (int q = 0; q < QG; ++q) {
            s_m[q][wave] = m[q];
            s_l[q][wave] = lw[q];
        }
    }
    // A bad tile in any wave marks every partial of the group (l = NaN).
    bool any_bad = false;
    if constexpr (PAGED) any_bad = __syncthreads_or(bad);
    else __syncthreads();
    const int t = (int)threadIdx.x;
    float M[QG], acc[QG], ls[QG];
    if constexpr (QG < 4) {
        // threads t < D fold every query slot of dimension t (measured faster
        // than the all-thread fold below up to two slots)
#pragma unroll
        for (int q = 0; q < QG; ++q) {
            M[q] = 0.f;
            acc[q] = 0.f;
            ls[q] = 0.f;
            if (t < D) {
                M[q] = s_m[q][0];
#pragma unroll
                for (int w = 1; w < WAVES; ++w) M[q] = fmaxf(M[q], s_m[q][w]);
                float f[WAVES];
#pragma unroll
                for (int w = 0; w < WAVES; ++w) f[w] = fast_exp2(s_m[q][w] - M[q]);
#pragma unroll
                for (int r = 0; r < WAVES * 4; ++r) acc[q] = __builtin_fmaf(f[r / 4], s_red[q][r][t], acc[q]);
#pragma unroll
                for (int w = 0; w < WAVES; ++w) ls[q] = __builtin_fmaf(f[w], s_l[q][w], ls[q]);
                if (any_bad) ls[q] = __builtin_nanf("");
            }
        }
    } else {
        // four query slots: every thread folds (query slot, dimension) pairs
        __shared__ float s_acc[QG][D];
        __shared__ float s_mf[QG], s_lf[QG];
        for (int i = t; i < QG * D; i += WAVES * 64) {
            const int q = i / D, d = i - (i / D) * D;
            float m = s_m[q][0];
#pragma unroll
            for (int w = 1; w < WAVES; ++w) m = fmaxf(m, s_m[q][w]);
            float f[WAVES];
#pragma unroll
            for (int w = 0; w < WAVES; ++w) f[w] = fast_exp2(s_m[q][w] - m);
            float sacc = 0.f, sl = 0.f;
#pragma unroll
            for (int r = 0; r < WAVES * 4; ++r) sacc = __builtin_fmaf(f[r / 4], s_red[q][r][d], sacc);
            s_acc[q][d] = sacc;
            if (d == 0) {
#pragma unroll
                for (int w = 0; w < WAVES; ++w) sl = __builtin_fmaf(f[w], s_l[q][w], sl);
                s_mf[q] = m;
                s_lf[q] = any_bad ? __builtin_nanf("") : sl;
            }
        }
        __syncthreads();
#pragma unroll
        for (int q = 0; q < QG; ++q) {
            M[q] = s_mf[q];
            ls[q] = s_lf[q];
            acc[q] = t < D ? s_acc[q][t] : 0.f;
        }
    }
    finish_partial<D, WAVES * 64, QG>(a, rt, M, ls, acc, epoch);
}

template <int KIND, int D, int G, int U, int WAVES, int QG, bool PAGED, int MINB = 1>
__global__ __launch_bounds__(WAVES * 64, MINB) void decode_tiled(
    const uint8_t* k, const uint8_t* v, const uint16_t* sk, const uint16_t* sv,
    int L_, int S_, int chunk_, int slot_, const uint16_t* q, void* dst, DecodeArgs rest) {
    DecodeArgs a = rest;
    a.k = k; a.v = v; a.sk = sk; a.sv = sv; a.q = q;
    a.out = static_cast<uint16_t*>(dst);
    a.ws = static_cast<float*>(dst);
    a.L = L_; a.S = S_; a.chunk = chunk_; a.ticket_slot = slot_;
    a.qscale = qscale_of<D>();
    using T = Tile<KIND, D>;
    using C = Codec<KIND>;
    using LoadT = typename LaneLoad<KIND>::type;
    constexpr int ROWB = T::ROWB, LB = T::LB, LP = T::LP, PPW = T::PPW, EPL = T::EPL, NP = C::NP;
    static_assert(EPL == C::EPL, "codec width");
    constexpr bool QUANT = KIND != KF16;
    constexpr int NG  = D / G;                   // scale groups per row
    constexpr int TW  = PPW * U;                 // rows per wave per iteration
    constexpr int TB  = TW * WAVES;              // rows per work-group per iteration
    constexpr int SCN = QUANT ? TW * NG : 1;     // (k, v) scale pairs per wave tile
    constexpr int SCE = !QUANT ? 1 : NG >= 2 ? SCN / 2 : SCN;  // scale dwords/halves per tensor
    constexpr int SCR = (SCE + 63) / 64;         // scale loads per lane per tensor
    // Rows of a work-group tile. Contiguous 4-wave groups interleave the waves
    // by load instruction: load u of wave w reads rows u*PPW*WAVES + w*PPW ..
    // + PPW, so the group's u-th loads cover WAVES*PPW consecutive rows
    // (measured on MI355X, H=32 D=128: q8+ L 16384 24.85 -> 24.49 us, 65536
    // 85.8 -> 85.0, q4+ 16384 16.30 -> 16.04). 8-wave groups keep each wave's
    // TW rows together (interleaved, f16+ at 16384 took 47.5 against 41.8 us),
    // and so does the paged form (a wave tile lies in one page).
    // RS = rows between a wave's loads, WS = rows between waves.
    constexpr bool IL = !PAGED && WAVES == 4;
    constexpr int RS = IL ? PPW * WAVES : PPW;
    constexpr int WS = IL ? PPW : TW;
    constexpr int SPG = NG >= 2 ? PPW * NG / 2 : PPW;  // scale entries of one load's rows
    static_assert(!QUANT || G % EPL == 0, "a lane's elements share one scale group");
    static_assert(SCE % 64 == 0 || SCR == 1, "scale entries fill whole wave loads");

    __shared__ uint32_t s_scale[WAVES][SCN];
    __shared__ int      s_page[PAGED ? MAX_SPLIT_PAGES : 1];

    // ---- work-group -> (sequence b, KV head hk, query sub-group, split s)
    Route rt;
    rt.mg = (int)blockIdx.x / a.S;
    rt.s  = (int)blockIdx.x - rt.mg * a.S;
    int b = 0, hk = rt.mg, sub = 0;
    if constexpr (QG > 1 || PAGED) {
        sub = rt.mg % a.nsub;
        const int r = rt.mg / a.nsub;
        hk = r % a.hkv;
        b  = r / a.hkv;
    }
    if constexpr (QG == 1 && !PAGED) {           // the reference's shape: head = merge group
        rt.nq  = 1;
        rt.oh0 = rt.mg;
    } else {
        rt.nq  = min(QG, a.qgroup - sub * QG);
        rt.oh0 = (b * a.hkv + hk) * a.qgroup + sub * QG;
    }
    const int s = rt.s;
    const unsigned epoch = read_epoch<QG>(a, rt.mg);
    const int wave = uniform((int)(threadIdx.x >> 6));
    const int lane = (int)(threadIdx.x & 63);
    const int sl   = lane % LP;                  // lane within its row
    const int pw   = lane / LP;                  // row slot within a wave load
    const int grp  = (sl * EPL) / G;             // scale group of this lane

    int L = a.L;
    bool bad = false;                            // invalid input: the output becomes NaN
    if constexpr (PAGED) {
        const int cap = min(a.L, min(a.S * a.chunk, a.max_pages << a.page_shift));
        L = a.seq_lens[b];
        if (L > cap || L < 0) { bad = true; L = L < 0 ? 0 : cap; }   // outside [0, max_seq_len]: NaN output
    }
    const int j0 = s * a.chunk;
    const int n  = min(L - j0, a.chunk);         // rows of this split (<= 0: empty)

    float m[QG], l[QG];
    float o[QG][EPL];
#pragma unroll
    for (int q = 0; q < QG; ++q) {
        m[q] = M_INIT;
        l[q] = 0.f;
#pragma unroll
        for (int e = 0; e < EPL; ++e) o[q][e] = 0.f;
    }

    if (n > 0) {
        const uint32_t lane_off = (uint32_t)(pw * ROWB + sl * LB);
        const int niter = (n + TB - 1) / TB;

        // Contiguous form: resources over the split, tile offsets in soffset
        // (the paged form builds per-tile resources and leaves these empty).
        const size_t   row0  = PAGED ? 0 : (size_t)hk * a.L + j0;
        const uint32_t nsplt = PAGED ? 0u : (uint32_t)n;
        const __amdgpu_buffer_rsrc_t rk = make_rsrc(a.k + row0 * ROWB, nsplt * ROWB);
        const __amdgpu_buffer_rsrc_t rv = make_rsrc(a.v + row0 * ROWB, nsplt * ROWB);
        const __amdgpu_buffer_rsrc_t rsk = QUANT ? make_rsrc(a.sk + row0 * NG, nsplt * NG * 2) : rk;
        const __amdgpu_buffer_rsrc_t rsv = QUANT ? make_rsrc(a.sv + row0 * NG, nsplt * NG * 2) : rv;
        int p0 = 0;
        if constexpr (PAGED) {
            // Stage the split's page ids (its positions span pages p0 .. p1).
            p0 = j0 >> a.page_shift;
            const int np = ((j0 + n - 1) >> a.page_shift) - p0 + 1;
            const int32_t* tab = a.block_table + (size_t)b * a.max_pages + p0;
            for (int i = (int)threadIdx.x; i < np; i += WAVES * 64) s_page[i] = tab[i];
            __syncthreads();
        }

        // Two register stages (A, B) alternate: while one tile is computed the
        // next one is already in flight, and no register copy ever waits on it.
        LoadT ka[U], va_[U], kb[U], vb[U];
        uint32_t ska[SCR], sva[SCR], skb[SCR], svb[SCR];

        // Issue order is pinned (scales, then K, then V) so the prologue and the
        // loop leave the same pending-load sequence and the waits stay partial.
        auto load_tile = [&](int it, LoadT* kk, LoadT* vv, uint32_t* sk, uint32_t* sv) {
            const int t0 = it * TB + wave * WS;                 // wave's first row in the split
            __amdgpu_buffer_rsrc_t tk = rk, tv = rv, tsk = rsk, tsv = rsv;
            uint32_t soff = (uint32_t)t0;
            if constexpr (PAGED) {
                // Each wave tile lies in one page (TW divides the page size).
                const int pos  = j0 + t0;                       // position in the sequence
                const int rows = max(0, min(TW, n - t0));       // rows of this tile inside the split
                int page = 0;
                if (rows > 0) page = uniform(s_page[(pos >> a.page_shift) - p0]);
                const bool ok = page >= 0 && page < a.num_pages;
                bad = bad || (rows > 0 && !ok);
                const uint32_t nrow = ok ? (uint32_t)rows : 0u;
                const size_t row = ((size_t)(ok ? page : 0) * a.hkv + hk) * ((size_t)1 << a.page_shift) +
                                   (size_t)(pos & ((1 << a.page_shift) - 1));
                tk = make_rsrc(a.k + row * ROWB, nrow * ROWB);
                tv = make_rsrc(a.v + row * ROWB, nrow * ROWB);
                if constexpr (QUANT) {
                    tsk = make_rsrc(a.sk + row * NG, nrow * NG * 2);
                    tsv = make_rsrc(a.sv + row * NG, nrow * NG * 2);
                }
                soff = 0;
            }
            const uint32_t tpos = sgpr(soff);                   // wave-uniform
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (QUANT) {            // lanes past SCE repeat the last entry (unused)
#pragma unroll
                for (int r = 0; r < SCR; ++r) {
                    const uint32_t sidx = (uint32_t)min(lane + 64 * r, SCE - 1);
                    // entry sidx belongs to the rows of load sidx / SPG
                    const uint32_t gap = (sidx / SPG) * (uint32_t)(RS - PPW) * NG * 2;   // bytes
                    if constexpr (NG >= 2) {
                        sk[r] = ld32(tsk, sidx * 4 + gap, tpos * NG * 2);
                        sv[r] = ld32(tsv, sidx * 4 + gap, tpos * NG * 2);
                    } else {
                        sk[r] = ld16(tsk, sidx * 2 + gap, tpos * 2);
                        sv[r] = ld16(tsv, sidx * 2 + gap, tpos * 2);
                    }
                }
            }
#pragma unroll
            for (int u = 0; u < U; ++u)
                kk[u] = lane_load<KIND>(tk, lane_off + (uint32_t)(u * RS * ROWB), tpos * ROWB);
#pragma unroll
            for (int u = 0; u < U; ++u)
                vv[u] = lane_load<KIND>(tv, lane_off + (uint32_t)(u * RS * ROWB), tpos * ROWB);
            __builtin_amdgcn_sched_barrier(0);
        };

        // The first tile is issued before q is read, so the two latencies overlap.
        load_tile(0, ka, va_, ska, sva);

        // q slices of this lane (dims [sl*EPL, sl*EPL + EPL)) in codec form;
        // query slots past nq read query slot 0 (their results are dropped).
        typename C::QReg qr[QG];
#pragma unroll
        for (int q = 0; q < QG; ++q)
            C::template load_q<LP>(qr[q], a.q + (size_t)(rt.oh0 + (q < rt.nq ? q : 0)) * D + sl * EPL, a.qscale);
        const uint32_t magic = C::magic();

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

        // V offset window: S[q] sums the weights ev since the last fix_v, which
        // removes the stored codes' offset from the accumulators in bulk once
        // per tile pair (2U rows per lane), so the sums never drift more than a
        // pair's worth from the signed ones. (An fp32 emulation of the
        // accumulation error against the exact sum: the same as signed
        // accumulation for windows up to 32 rows, q8 / q4 / q3 alike. Fixing
        // every other pair instead measured slower on MI355X: the conditional
        // splits the loop body.)
        float S[QG], thr[QG];
#pragma unroll
        for (int q = 0; q < QG; ++q) {
            S[q] = 0.f;
            thr[q] = (m[q] + RESCALE_SLACK) / qr[q].qs;
        }
        auto fix_v = [&]() {
            if constexpr (C::VFIX) {
#pragma unroll
                for (int q = 0; q < QG; ++q) {
#pragma unroll
                    for (int e = 0; e < EPL; ++e) o[q][e] = __builtin_fmaf(S[q], C::voff(e), o[q][e]);
                    S[q] = 0.f;
                }
            }
        };

        // Scores stay raw (q.k times the group scale); qs is applied inside the
        // exponent's fma and to the tile maximum.
        auto compute_tile = [&](auto masked, int it, const LoadT* kk, const LoadT* vv) {
            constexpr bool MASK = decltype(masked)::value;
            float sc[QG][U];
            uint32_t pair[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int slot = u * PPW + pw;
                h2 pk[NP];
                C::unpack_k(kk[u], magic, pk);
                pair[u] = 0;
                if constexpr (QUANT) pair[u] = s_scale[wave][slot * NG + grp];
#pragma unroll
                for (int q = 0; q < QG; ++q) {
                    float d = C::dot(pk, qr[q]);
                    if constexpr (QUANT) d = mul_lo_h(d, pair[u]);     // x k scale
                    sc[q][u] = group_sum<LP>(d);
                }
            }
            // Rows past the split end score -inf (the masked form of the loop).
            if constexpr (MASK) {
                const int rem = uniform(n - it * TB - wave * WS);   // rows of the split from the wave's first
#pragma unroll
                for (int u = 0; u < U; ++u)
#pragma unroll
                    for (int q = 0; q < QG; ++q)
                        sc[q][u] = u * RS + pw < rem ? sc[q][u] : -__builtin_inff();
            }
#pragma unroll
            for (int q = 0; q < QG; ++q) {
                float tmax = sc[q][0];
#pragma unroll
                for (int u = 1; u < U; ++u) tmax = fmaxf(tmax, sc[q][u]);
                // raw scores against thr = (m + RESCALE_SLACK) / qs (wave-uniform,
                // updated with m); a rounding difference at the threshold only
                // moves a rescale, which is optional
                if (__builtin_amdgcn_ballot_w64(tmax > thr[q])) {
                    tmax *= qr[q].qs;                                  // log2 units
                    const float mn = uniformf(wave_max(fmaxf(m[q], tmax)));
                    const float c  = fast_exp2(m[q] - mn);
                    l[q] *= c;
                    S[q] *= c;
#pragma unroll
                    for (int e = 0; e < EPL; ++e) o[q][e] *= c;
                    m[q] = mn;
                    thr[q] = (mn + RESCALE_SLACK) / qr[q].qs;
                }
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                h2 pv[NP];
                C::unpack_v(vv[u], pv);
#pragma unroll
                for (int q = 0; q < QG; ++q) {
                    const float p = fast_exp2(__builtin_fmaf(sc[q][u], qr[q].qs, -m[q]));
                    l[q] += p;
                    float ev = p;
                    if constexpr (QUANT) ev = mul_hi_h(p, pair[u]);    // x v scale
                    if constexpr (C::VFIX) S[q] += ev;
                    C::axpy_v(pv, ev, o[q]);
                }
            }
        };

        // Tiles are processed in pairs, and an odd last tile after the loop (its
        // loads are the last pair's prefetch; niter is uniform over the
        // work-group). Loads past the end of the split return zeros without
        // memory traffic, so the prefetch after the last tile adds no traffic.
        // (An exit inside the loop instead measured 1.5 us slower for the paged
        // one-slot form, and skipping the last prefetch with a uniform test made
        // q4+ at H=32 L=16384 1.7 us slower: both change how the loop body is
        // scheduled.)
        // f16 rows in 8-wave groups: the older wave of each SIMD pair wins issue
        // and runs ahead, and the younger one finishes alone with half the loads
        // in flight. On long splits a barrier per tile pair keeps the waves
        // together (measured on MI355X, H=32 D=128: L=65536 165.7 -> 161.3 us);
        // below 16 tiles per group it costs more than it saves (L=4096 +0.35 us).
        const bool lockstep = KIND == KF16 && WAVES == 8 && QG == 1 && !PAGED && niter >= 16;
        // Only the last work-group tile of a split can hold rows past its end
        // (rem < TW for some wave), so only that tile runs the masked form; the
        // pair loop covers tiles 0 .. 2P-1, all full.
        const int P = (niter - 1) / 2;
        // One tile pair: tile it from the A stage, tile it+1 from B, the next
        // pair's first tile prefetched into A.
#define VA_PAIR_STEP(it_)                                                     \
        do {                                                                  \
            const int it = (it_);                                             \
            if (lockstep) __builtin_amdgcn_s_barrier();   /* niter is uniform over the group */ \
            stage_scales(ska, sva);                                           \
            load_tile(it + 1, kb, vb, skb, svb);                              \
            compute_tile(std::false_type{}, it, ka, va_);                     \
            stage_scales(skb, svb);                                           \
            load_tile(it + 2, ka, va_, ska, sva);                             \
            compute_tile(std::false_type{}, it + 1, kb, vb);                  \
        } while (0)
        // Kinds with a V offset and 2U < 16 rows per lane per pair take
        // FIXP = 16 / 2U pairs per loop iteration and one offset fix after them:
        // the window stays <= 16 rows per lane with no branch in the loop body.
        constexpr int FIXP = C::VFIX && 2 * U < 16 ? 16 / (2 * U) : 1;
        int ip = 0;
        if constexpr (FIXP > 1) {
            for (; ip + FIXP <= P; ip += FIXP) {
#pragma unroll
                for (int k = 0; k < FIXP; ++k) VA_PAIR_STEP(2 * (ip + k));
                fix_v();
            }
        }
        for (; ip < P; ++ip) {
            VA_PAIR_STEP(2 * ip);
            fix_v();
        }
#undef VA_PAIR_STEP
        // tail: tile 2P is in the A stage; it is the last one, or one full tile
        // and then the last
        if (niter - 2 * P == 2) {
            stage_scales(ska, sva);
            load_tile(2 * P + 1, kb, vb, skb, svb);
            compute_tile(std::false_type{}, 2 * P, ka, va_);
            stage_scales(skb, svb);
            compute_tile(std::true_type{}, 2 * P + 1, kb, vb);
        } else {
            stage_scales(ska, sva);
            compute_tile(std::true_type{}, 2 * P, ka, va_);
        }
#pragma unroll
        for (int q = 0; q < QG; ++q) fix_finish<C>(o[q], S[q], std::make_integer_sequence<int, EPL>{});
    }

    group_finish<D, LP, EPL, WAVES, QG, PAGED>(a, rt, m, l, o, bad, epoch);
}

} // namespace va
