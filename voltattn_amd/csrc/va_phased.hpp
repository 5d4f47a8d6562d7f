// va_phased.hpp — the two-phase split-L decode kernel: over contiguous K/V,
// the reference shape (one query head per K/V head, QG = 1) and grouped-query
// decode of one sequence (QG query heads of a K/V head per work-group); over a
// paged batch (PAGED), one query head per work-group. The same partials,
// splits, codecs and merge as decode_tiled<..., QG, PAGED> (va_tiled.hpp), with
// the K and V rows of a split read in separate phases. The paged form needs
// pages of at least one work-group tile (TB rows, a power of two) and splits
// that start on a tile, so that every tile lies in one page; the host checks
// both.
//
// A work-group walks its split in rounds of up to RT work-group tiles. Each
// round first streams the K rows of its positions (with the K scales): every
// row's raw score (q.k times the group scale) for each of the QG query heads
// goes to the wave's slice of LDS, and the wave keeps each head's maximum. Then
// it streams the V rows of the same positions (with the V scales): each lane
// reads back its row's scores and accumulates p = exp2(score * qs - m) against
// the row, m being the exact maximum of the wave's scores so far for that head
// (one rescale of l and o per round, where it rises). Reference:
// src/voltattn.cu:364-649 (one pass over the positions that reads K and V
// together, an online softmax per position).
//
// Why two phases: a work-group that reads one stream at a time keeps half as
// many DRAM streams open as one that reads K and V side by side. A read-only
// kernel with the decode grid (one 4-wave group per CU, 16 KB per register
// stage, two stages) measured on MI355X: 268 MB in 38.7 us as K-then-V phases
// against 40.2 us as interleaved K and V loads at the same depth (40.6 us at
// the 32 KB stages of the interleaved decode loop); 142.6 MB in 21.8 against
// 21.9 (22.1) us.
//
// Each lane loads LB = 16 bytes (12 for q3) of a row per load, U loads per
// tile of one tensor; the loads of a 4-wave group interleave by instruction
// (load u of wave w reads rows u*PPW*WAVES + w*PPW ..), as in decode_tiled,
// and an 8-wave group keeps each wave's TW rows together.
// Two register stages alternate over the stage sequence K tiles 0..T-1, V
// tiles 0..T-1 of round 0, then round 1, ...: the next stage's loads are in
// flight while the current one is computed, across the phase change too.
// Loads past the end of the split return zeros without memory traffic, which
// covers the last, partial tile.
#pragma once
#include "va_tiled.hpp"

namespace va {

// Positions per round of a work-group at QG = 1 (32 KB of scores in LDS); a
// round at QG > 1 holds 8192/QG positions, so its scores take the same 32 KB.
constexpr int PHASED_ROUND_ROWS = 8192;

template <int KIND, int D, int G, int U, int WAVES, int QG = 1, bool PAGED = false>
__global__ __launch_bounds__(WAVES * 64, 1) void decode_phased(
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
    constexpr int TW  = PPW * U;                 // rows per wave per tile
    constexpr int TB  = TW * WAVES;              // rows per work-group tile
    constexpr int RT  = PHASED_ROUND_ROWS / QG / TB;   // work-group tiles per round
    static_assert(RT >= 1 && RT * TB * QG == PHASED_ROUND_ROWS, "whole tiles per round");
    constexpr int SCN = QUANT ? TW * NG : 1;     // scale entries of one tensor per wave tile
    constexpr int SCE = !QUANT ? 1 : NG >= 2 ? SCN / 2 : SCN;  // scale dwords (NG >= 2) or halves per wave tile
    constexpr int SCR = (SCE + 63) / 64;         // scale loads per lane
    constexpr bool IL = WAVES == 4;              // interleaved waves (as decode_tiled's contiguous 4-wave form)
    constexpr int RS = IL ? PPW * WAVES : PPW;   // rows between a wave's loads
    constexpr int WS = IL ? PPW : TW;            // rows between waves
    constexpr int SPG = NG >= 2 ? PPW * NG / 2 : PPW;  // scale entries of one load's rows
    static_assert(!QUANT || G % EPL == 0, "a lane's elements share one scale group");
    static_assert(SCE % 64 == 0 || SCR == 1, "scale entries fill whole wave loads");
    static_assert(!PAGED || QG == 1, "the paged form carries one query slot");
    static_assert(!PAGED || (TB & (TB - 1)) == 0, "paged tiles must not straddle pages");

    __shared__ uint32_t s_sc[WAVES][SCN];        // scale entries of the wave's current tile (low halves)
    __shared__ float s_score[WAVES][QG][RT * TW];  // raw scores of the wave's rows in the round
    __shared__ int s_page[PAGED ? MAX_SPLIT_PAGES : 1];

    // work-group -> (KV head hk, query sub-group, split s)
    Route rt;
    rt.mg  = (int)blockIdx.x / a.S;
    rt.s   = (int)blockIdx.x - rt.mg * a.S;
    int hk = rt.mg, b = 0;
    if constexpr (PAGED) {                       // sequence b, KV head hk, one query head
        const int sub = rt.mg % a.nsub;
        const int r   = rt.mg / a.nsub;
        hk = r % a.hkv;
        b  = r / a.hkv;
        rt.nq  = 1;
        rt.oh0 = (b * a.hkv + hk) * a.qgroup + sub;
    } else if constexpr (QG == 1) {              // the reference's shape: head = merge group
        rt.nq  = 1;
        rt.oh0 = rt.mg;
    } else {                                     // one sequence: merge group = (hk, sub-group)
        const int sub = rt.mg % a.nsub;
        hk = (rt.mg / a.nsub) % a.hkv;
        rt.nq  = min(QG, a.qgroup - sub * QG);
        rt.oh0 = hk * a.qgroup + sub * QG;
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
        const int ntile = (n + TB - 1) / TB;     // work-group tiles of the split
        const int nst   = 2 * ntile;             // stages: a K and a V pass over every tile
        // Contiguous form: resources over the split, tile offsets in soffset. The
        // paged form builds resources per work-group tile (each lies in one
        // page: the host launches it only for pages of at least TB rows and
        // splits that start on a work-group tile).
        const size_t   row0  = PAGED ? 0 : (size_t)hk * a.L + j0;
        const uint32_t nsplt = PAGED ? 0u : (uint32_t)n;
        const __amdgpu_buffer_rsrc_t rk = make_rsrc(a.k + row0 * ROWB, nsplt * ROWB);
        const __amdgpu_buffer_rsrc_t rv = make_rsrc(a.v + row0 * ROWB, nsplt * ROWB);
        const __amdgpu_buffer_rsrc_t rsk = QUANT ? make_rsrc(a.sk + row0 * NG, nsplt * NG * 2) : rk;
        const __amdgpu_buffer_rsrc_t rsv = QUANT ? make_rsrc(a.sv + row0 * NG, nsplt * NG * 2) : rv;
        int p0 = 0;
        int pnext = 0;                           // page id of the next stage to load (paged form)
        if constexpr (PAGED) {
            // Stage the split's page ids (its positions span pages p0 .. p1).
            p0 = j0 >> a.page_shift;
            const int np = ((j0 + n - 1) >> a.page_shift) - p0 + 1;
            const int32_t* tab = a.block_table + (size_t)b * a.max_pages + p0;
            for (int i = (int)threadIdx.x; i < np; i += WAVES * 64) s_page[i] = tab[i];
            __syncthreads();
            pnext = s_page[0];                   // stage 0: the split's first tile
        }

        // Stage i -> (tile of the split, phase, tile within the round). Rounds
        // before the last hold RT tiles.
        struct StageAt { int tile; bool vph; int t; int tr; };
        auto stage_at = [&](int i) {
            StageAt x;
            const int r  = i / (2 * RT);
            const int w  = i - r * 2 * RT;
            x.tr   = min(RT, ntile - r * RT);    // tiles of this round
            x.vph  = w >= x.tr;
            x.t    = x.vph ? w - x.tr : w;
            x.tile = r * RT + x.t;
            return x;
        };

        LoadT xa[U], xb[U];
        uint32_t sa[SCR], sb[SCR];

        // Issue order pinned (scales, then rows), as in decode_tiled, so every
        // wait stays partial.
        auto load_stage = [&](int i, LoadT* xx, uint32_t* ss) {
            const StageAt st = stage_at(i);
            __amdgpu_buffer_rsrc_t tx = st.vph ? rv : rk;
            __amdgpu_buffer_rsrc_t ts = st.vph ? rsv : rsk;
            uint32_t t0 = (uint32_t)(st.tile * TB + wave * WS);
            if constexpr (PAGED) {
                // the work-group tile's rows in its page, every descriptor field
                // scalar (a field in a VGPR would make each load a loop over lanes)
                const int wt   = st.tile * TB;                      // tile's first row in the split
                const int pos  = j0 + wt;                           // position in the sequence
                const int rows = min(TB, n - wt);                   // >= 1: the tile is inside the split
                // quantized kinds (two resources per stage) take the page id read
                // one stage ahead; f16 reads it here (measured faster for each)
                const int page = QUANT ? uniform(pnext) : uniform(s_page[(pos >> a.page_shift) - p0]);
                const bool ok  = page >= 0 && page < a.num_pages;
                bad = bad || !ok;
                const uint32_t nrow = sgpr(ok ? (uint32_t)rows : 0u);
                const size_t row = uniform64(((size_t)(ok ? page : 0) * a.hkv + hk) * ((size_t)1 << a.page_shift) +
                                             (size_t)(pos & ((1 << a.page_shift) - 1)));
                tx = make_rsrc((st.vph ? a.v : a.k) + row * ROWB, nrow * ROWB);
                if constexpr (QUANT) ts = make_rsrc((st.vph ? a.sv : a.sk) + row * NG, nrow * NG * 2);
                t0 = (uint32_t)(wave * WS);
            }
            const uint32_t tpos = sgpr(t0);
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (QUANT) {               // lanes past SCE repeat the last entry (unused)
#pragma unroll
                for (int r = 0; r < SCR; ++r) {
                    const uint32_t sidx = (uint32_t)min(lane + 64 * r, SCE - 1);
                    const uint32_t gap = (sidx / SPG) * (uint32_t)(RS - PPW) * NG * 2;   // bytes
                    if constexpr (NG >= 2) ss[r] = ld32(ts, sidx * 4 + gap, tpos * NG * 2);
                    else ss[r] = ld16(ts, sidx * 2 + gap, tpos * 2);
                }
            }
#pragma unroll
            for (int u = 0; u < U; ++u)
                xx[u] = lane_load<KIND>(tx, lane_off + (uint32_t)(u * RS * ROWB), tpos * ROWB);
            if constexpr (PAGED && QUANT) {
                // the next stage's page id, read now so that it has arrived by its issue
                const int in = min(i + 1, nst - 1);
                pnext = s_page[((j0 + stage_at(in).tile * TB) >> a.page_shift) - p0];
            }
            __builtin_amdgcn_sched_barrier(0);
        };

        load_stage(0, xa, sa);

        // q slices of this lane (dims [sl*EPL, sl*EPL + EPL)); query slots past
        // nq read query slot 0 (their results are dropped)
        typename C::QReg qr[QG];
#pragma unroll
        for (int q = 0; q < QG; ++q)
            C::template load_q<LP>(qr[q], a.q + (size_t)(rt.oh0 + (q < rt.nq ? q : 0)) * D + sl * EPL, a.qscale);
        const uint32_t magic = C::magic();

        auto stage_scales = [&](const uint32_t* ss) {
            if constexpr (QUANT) {
#pragma unroll
                for (int r = 0; r < SCR; ++r) {
                    const int e = lane + 64 * r;
                    if (e < SCE) {               // entry i in the low half of s_sc[wave][i]
                        if constexpr (NG >= 2) {
                            s_sc[wave][2 * e]     = ss[r];
                            s_sc[wave][2 * e + 1] = ss[r] >> 16;
                        } else {
                            s_sc[wave][e] = ss[r];
                        }
                    }
                }
            }
        };

        // V offset window (va_tiled.hpp): vsum sums the weights ev since the
        // last fix_v, which removes the stored codes' offset in bulk.
        float vsum[QG];
#pragma unroll
        for (int q = 0; q < QG; ++q) vsum[q] = 0.f;
        auto fix_v = [&]() {
            if constexpr (C::VFIX) {
#pragma unroll
                for (int q = 0; q < QG; ++q) {
#pragma unroll
                    for (int e = 0; e < EPL; ++e) o[q][e] = __builtin_fmaf(vsum[q], C::voff(e), o[q][e]);
                    vsum[q] = 0.f;
                }
            }
        };

        float lmax[QG];                          // this lane's largest raw score of the round, per slot
#pragma unroll
        for (int q = 0; q < QG; ++q) lmax[q] = -__builtin_inff();

        // K phase of one tile: raw scores to LDS; rows past the split's end
        // (the last tile only) score -inf.
        auto score_tile = [&](auto masked, const StageAt& st, const LoadT* kk) {
            constexpr bool MASK = decltype(masked)::value;
            const int rem = MASK ? uniform(n - st.tile * TB - wave * WS) : 0;   // rows from the wave's first
            uint32_t scl[U];                     // the rows' K scales, read before any score is stored
#pragma unroll
            for (int u = 0; u < U; ++u) scl[u] = QUANT ? s_sc[wave][(u * PPW + pw) * NG + grp] : 0u;
            float sc[QG][U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                h2 pk[NP];
                C::unpack_k(kk[u], magic, pk);  // once for every query slot
#pragma unroll
                for (int q = 0; q < QG; ++q) {
                    float d = C::dot(pk, qr[q]);
                    if constexpr (QUANT) d = mul_lo_h(d, scl[u]);
                    sc[q][u] = group_sum<LP>(d);
                    if constexpr (MASK) sc[q][u] = u * RS + pw < rem ? sc[q][u] : -__builtin_inff();
                    lmax[q] = fmaxf(lmax[q], sc[q][u]);
                }
            }
            // one lane per row stores its scores: one branch per tile, so the
            // rows above stay in one block and their chains interleave
            if (sl == 0) {
#pragma unroll
                for (int q = 0; q < QG; ++q)
#pragma unroll
                    for (int u = 0; u < U; ++u) s_score[wave][q][st.t * TW + u * PPW + pw] = sc[q][u];
            }
            if (st.t == st.tr - 1) {             // the round's maxima; rescale where one rose
#pragma unroll
                for (int q = 0; q < QG; ++q) {
                    const float mn = fmaxf(m[q], uniformf(wave_max(lmax[q])) * qr[q].qs);
                    if (mn > m[q]) {
                        const float c = fast_exp2(m[q] - mn);
                        l[q] *= c;
                        vsum[q] *= c;
#pragma unroll
                        for (int e = 0; e < EPL; ++e) o[q][e] *= c;
                        m[q] = mn;
                    }
                    lmax[q] = -__builtin_inff();
                }
            }
        };
        // V phase of one tile.
        auto value_tile = [&](const StageAt& st, const LoadT* vv) {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int slot = u * PPW + pw;
                h2 pv[NP];
                C::unpack_v(vv[u], pv);         // once for every query slot
                uint32_t vsc = 0;
                if constexpr (QUANT) vsc = s_sc[wave][slot * NG + grp];
#pragma unroll
                for (int q = 0; q < QG; ++q) {
                    const float sc = s_score[wave][q][st.t * TW + slot];
                    const float p = fast_exp2(__builtin_fmaf(sc, qr[q].qs, -m[q]));
                    l[q] += p;
                    float ev = p;
                    if constexpr (QUANT) ev = mul_lo_h(p, vsc);
                    if constexpr (C::VFIX) vsum[q] += ev;
                    C::axpy_v(pv, ev, o[q]);
                }
            }
        };
        auto compute = [&](int i, const LoadT* xx) {
            const StageAt st = stage_at(i);
            if (st.vph) {
                value_tile(st, xx);
            } else if (st.tile == ntile - 1) {
                score_tile(std::true_type{}, st, xx);
            } else {
                score_tile(std::false_type{}, st, xx);
            }
        };

        // nst is even: the stages run in (A, B) pairs with no tail. The last pair
        // issues no prefetch, so no load is pending on the stage registers after
        // the loop (interleaved A/B on MI355X, H=32 D=128: q8+ L 16384 23.41 ->
        // 23.29 us, 65536 80.47 -> 80.16; f16+ unchanged).
        int i = 0;
        for (; i + 2 < nst; i += 2) {
            stage_scales(sa);
            load_stage(i + 1, xb, sb);
            compute(i, xa);
            stage_scales(sb);
            load_stage(i + 2, xa, sa);
            compute(i + 1, xb);
            if (stage_at(i + 1).vph) fix_v();    // <= 2U rows per lane since the last fix
        }
        stage_scales(sa);
        load_stage(i + 1, xb, sb);
        compute(i, xa);
        stage_scales(sb);
        compute(i + 1, xb);
        fix_v();
#pragma unroll
        for (int q = 0; q < QG; ++q) fix_finish<C>(o[q], vsum[q], std::make_integer_sequence<int, EPL>{});
    }

    group_finish<D, LP, EPL, WAVES, QG, PAGED>(a, rt, m, l, o, bad, epoch);
}

} // namespace va
