// va_mfma.hpp — grouped-query decode on the matrix cores (gfx950 MFMA).
//
// Same partials as decode_tiled (va_tiled.hpp), for q8 and q4 rows and q3 rows at
// D = 128, with q.K and P.V on the matrix cores instead of per-lane dot/axpy chains
// (the VALU form spends ~28 vector instructions per position at four query
// heads; here the matrix core does the multiply-adds and the VALU keeps the
// unpack, the softmax and the operand set-up).
//
// MFMA lane layouts (probed on MI355X): for 16x16x32 f16, lane l holds
// A[l%16][8(l/16)+e] and B[8(l/16)+e][l%16] (e = 0..7); for 16x16x64 i8,
// A[l%16][16(l/16)+e] and B[16(l/16)+e][l%16] (e = 0..15, byte order); both
// return D[4(l/16)+v][l%16] (v = 0..3). Below, quarter g = l/16 and column
// n = l%16.
//
// q.K — two 16-row blocks of positions per 32-row wave tile, k = dimensions,
// on v_mfma_i32_16x16x64_i8 (exact integer products and sums).
//   A = the K codes of 16 rows as unsigned or signed bytes: q8's int8 codes as
//       loaded, q4's nibbles and q3's 3-bit fields spread to bytes n = v + 8 /
//       v + 4 (the offset's -8 or -4 times the column sum of q is the int32
//       accumulator's start value).
//   B = q as three balanced int8 digits of round(q * 2^sh) (sh per column puts
//       max |q| in [2^21, 2^22)), with the scale groups stacked as columns:
//       column n = cg*QP + cq (QP = 16/NG column slots per group) holds query
//       slot cq restricted to the dimensions of scale group cg (zero
//       elsewhere). Each digit's dot with the codes is exact in int32; the
//       three are recombined in fp32 with one rounding, so each output column
//       is the partial dot of one (query, group); the per-position group scales
//       are applied afterwards in fp32 and the NG columns of a query are summed
//       with DPP row rotations (every replica gets the same bits).
// P.V — k = positions, 32 per f16 MFMA (the two q.K blocks).
//   A = P * s_v with the same stacked rows: row n = (cg, cq) carries
//       p[cq][pos] * s_v[pos][cg]. Lane (g, n) already holds the scores of
//       exactly the positions of its k slots (16c + 4g + v), so no data moves.
//       The fp32 value is split into fp16 hi + lo (RNE), two MFMAs, so P.V
//       keeps ~22 significant bits (MFMA keeps fp16 subnormals; probed).
//   B = V codes transposed: the wave's V tile is staged in LDS row-major and
//       read with ds_read_b64_tr_b8 (within 16 lanes, lane i receives byte i of
//       each 16-byte row formed by the chunks of lanes 2e and 2e+1), giving each
//       lane 8 positions of one column.
//   Output row (cg, cq), column d is useful when d lies in scale group cg;
//   each (query, dimension) is produced by exactly one lane and accumulator.
// Softmax: log2 units (q pre-scaled by log2(e)/sqrt(D) in fp32 after the dot),
// lazy running maximum per query slot as in decode_tiled (RESCALE_SLACK).
//
// Work split, loads and the merge are decode_tiled's: one work-group per
// (merge group, split), per-wave 32-row tiles double-buffered in registers,
// buffer resources bounded by the split (or per tile for paged caches), and
// finish_partial for the partials / fused merge.
#pragma once
#include "va_codec.hpp"
#include "va_fused.hpp"
#include "va_tiled.hpp"

namespace va {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef int i32x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) i32x2 lds_i32x2;

typedef int i32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4 mfma_16x16x32(const f16x8& a, const f16x8& b, const f32x4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
// int8 x int8 -> int32, k = 64: lane l holds A[l%16][16(l/16)+e] and
// B[16(l/16)+e][l%16] (e = 0..15, byte order; probed) and receives
// D[4(l/16)+v][l%16].
__device__ __forceinline__ i32x4 mfma_i8(const u32x4& a, const u32x4& b, const i32x4& c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(i32x4, a), __builtin_bit_cast(i32x4, b), c, 0, 0, 0);
}

__device__ __forceinline__ u32x2 ld64(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b64(r, voff, sgpr(soff), VA_LOAD_AUX);
}

// 8 bytes of q4 codes (two dwords, byte order) -> the 8 low nibbles as exact fp16
// v = n - 8, and the 8 high nibbles as exact fp16 16v (masked in place under the
// 1024.0 magic: 1024 + 16n - 1152).
__device__ __forceinline__ void q4_to_f16x8(uint32_t w0, uint32_t w1, uint32_t magic, f16x8& lo, f16x8& hi) {
    const h2 blo = hh(1032.f, 1032.f), bhi = hh(1152.f, 1152.f);
    const uint32_t l0 = w0 & 0x0F0F0F0Fu, l1 = w1 & 0x0F0F0F0Fu;
    const uint32_t u0 = w0 & 0xF0F0F0F0u, u1 = w1 & 0xF0F0F0F0u;
    const h2 a0 = as_h2(__builtin_amdgcn_perm(magic, l0, 0x04010400u)) - blo;
    const h2 a1 = as_h2(__builtin_amdgcn_perm(magic, l0, 0x04030402u)) - blo;
    const h2 a2 = as_h2(__builtin_amdgcn_perm(magic, l1, 0x04010400u)) - blo;
    const h2 a3 = as_h2(__builtin_amdgcn_perm(magic, l1, 0x04030402u)) - blo;
    const h2 b0 = as_h2(__builtin_amdgcn_perm(magic, u0, 0x04010400u)) - bhi;
    const h2 b1 = as_h2(__builtin_amdgcn_perm(magic, u0, 0x04030402u)) - bhi;
    const h2 b2 = as_h2(__builtin_amdgcn_perm(magic, u1, 0x04010400u)) - bhi;
    const h2 b3 = as_h2(__builtin_amdgcn_perm(magic, u1, 0x04030402u)) - bhi;
    lo = f16x8{a0.x, a0.y, a1.x, a1.y, a2.x, a2.y, a3.x, a3.y};
    hi = f16x8{b0.x, b0.y, b1.x, b1.y, b2.x, b2.y, b3.x, b3.y};
}

// 8 int8 codes (two dwords, byte order) -> 8 exact fp16 values in the same order.
__device__ __forceinline__ f16x8 q8_to_f16x8(uint32_t w0, uint32_t w1, uint32_t magic) {
    const uint32_t u0 = w0 ^ 0x80808080u, u1 = w1 ^ 0x80808080u;
    const h2 bias = hh(1152.f, 1152.f);
    const h2 p0 = as_h2(__builtin_amdgcn_perm(magic, u0, 0x04010400u)) - bias;
    const h2 p1 = as_h2(__builtin_amdgcn_perm(magic, u0, 0x04030402u)) - bias;
    const h2 p2 = as_h2(__builtin_amdgcn_perm(magic, u1, 0x04010400u)) - bias;
    const h2 p3 = as_h2(__builtin_amdgcn_perm(magic, u1, 0x04030402u)) - bias;
    return f16x8{p0.x, p0.y, p1.x, p1.y, p2.x, p2.y, p3.x, p3.y};
}

// 8 q3 codes n = v + 4 (two dwords of bytes, byte order) -> 8 exact fp16 values v.
__device__ __forceinline__ f16x8 q3b_to_f16x8(uint32_t w0, uint32_t w1, uint32_t magic) {
    const h2 bias = hh(1028.f, 1028.f);
    const h2 p0 = as_h2(__builtin_amdgcn_perm(magic, w0, 0x04010400u)) - bias;
    const h2 p1 = as_h2(__builtin_amdgcn_perm(magic, w0, 0x04030402u)) - bias;
    const h2 p2 = as_h2(__builtin_amdgcn_perm(magic, w1, 0x04010400u)) - bias;
    const h2 p3 = as_h2(__builtin_amdgcn_perm(magic, w1, 0x04030402u)) - bias;
    return f16x8{p0.x, p0.y, p1.x, p1.y, p2.x, p2.y, p3.x, p3.y};
}

// Four 3-bit codes in bits 0..11 of x (code i at bit 3i) -> one code per byte:
// the upper pair moves up by 10 (to bits 16 and 19), then every odd code by 5.
__device__ __forceinline__ uint32_t q3_spread4(uint32_t x) {
    const uint32_t t = (x | (x << 10)) & 0x003F003Fu;
    return (t | (t << 5)) & 0x07070707u;
}

// The 32 codes of a 12-byte q3 chunk (code e at bits [3e, 3e + 3) of the
// little-endian 96-bit word) -> 32 bytes in code order, byte e = code e.
__device__ __forceinline__ void q3_to_bytes(const u32x4& w, uint32_t (&b)[8]) {
    b[0] = q3_spread4(__builtin_amdgcn_ubfe(w.x, 0, 12));
    b[1] = q3_spread4(__builtin_amdgcn_ubfe(w.x, 12, 12));
    b[2] = q3_spread4(__builtin_amdgcn_alignbit(w.y, w.x, 24) & 0xFFFu);
    b[3] = q3_spread4(__builtin_amdgcn_ubfe(w.y, 4, 12));
    b[4] = q3_spread4(__builtin_amdgcn_ubfe(w.y, 16, 12));
    b[5] = q3_spread4(__builtin_amdgcn_alignbit(w.z, w.y, 28) & 0xFFFu);
    b[6] = q3_spread4(__builtin_amdgcn_ubfe(w.z, 8, 12));
    b[7] = q3_spread4(w.z >> 20);
}

template <int KIND, int D, int G, int WAVES, int QG, bool PAGED>
__global__ __launch_bounds__(WAVES * 64, 1) void decode_mfma(DecodeArgs a) {
    static_assert(KIND == KQ8 || KIND == KQ4 || (KIND == KQ3 && D == 128),
                  "matrix-core form: q8 and q4 rows, and q3 rows at D = 128");
    constexpr bool Q4  = KIND == KQ4;
    constexpr bool Q3  = KIND == KQ3;
    constexpr int ROWB = Q3 ? 3 * D / 8 : Q4 ? D / 2 : D;   // bytes per row in memory
    constexpr int VRB  = Q3 ? D : ROWB;          // bytes per staged V row (q3: a byte per code)
    constexpr int NG   = D / G;                  // scale groups per row (1, 2, 4)
    constexpr int QP   = 16 / NG;                // column slots per scale group
    static_assert(QG >= 1 && QG <= QP, "query slots per work-group");
    constexpr int TW   = 32;                     // rows per wave tile (two 16-row blocks)
    constexpr int TB   = TW * WAVES;
    constexpr int DQ   = ROWB / 4;               // row bytes per lane quarter (A operand)
    constexpr int KL   = Q3 ? 1 : DQ >= 16 ? DQ / 16 : 1;   // K loads per block per lane (16 B; q4 at D = 64: 8 B; q3: 12 B)
    constexpr int NJ   = D / 64;                 // q.K MFMAs (k = 64) per block and digit
    constexpr int NB   = D / 16;                 // P.V column blocks (16 dimensions each)
    constexpr int NC   = VRB / 16;               // 16-byte column chunks of a staged V row
    constexpr int VCH  = Q3 ? 12 : 16;           // bytes per V load per lane (q3: a quarter row)
    constexpr int VL   = TW * ROWB / (64 * VCH); // V loads per lane per tile
    constexpr int VSTR = VRB + 16;               // LDS row stride of the staged V tile
    constexpr int VROWS = TW + 4;                // rows 16..31 sit 4 slots further
    constexpr int SCE  = NG >= 2 ? TW * NG / 2 : TW;   // scale words (dwords, or halves at NG = 1)
    static_assert(VL >= 1 && SCE <= 64 && (Q4 ? NC * 2 == NB : (NC == NB && (Q3 || NJ == KL))), "tile shape");

    __shared__ __align__(16) uint8_t  s_v[WAVES][VROWS * VSTR];
    __shared__ __align__(16) uint32_t s_sc[WAVES][NG][TW];   // (k | v << 16) scale pairs
    __shared__ float s_red[QG][WAVES][D];
    __shared__ float s_l[QG][WAVES];
    __shared__ float s_m[QG][WAVES];
    __shared__ float s_acc[QG][D];
    __shared__ float s_mf[QG], s_lf[QG];
    __shared__ int   s_page[PAGED ? MAX_SPLIT_PAGES : 1];
    __shared__ int   s_prog[WAVES];                         // tile pair each wave is on (issue priority)

    // ---- work-group -> (sequence b, KV head hk, query sub-group, split s)
    Route rt;
    rt.mg = (int)blockIdx.x / a.S;
    rt.s  = (int)blockIdx.x - rt.mg * a.S;
    const int sub = rt.mg % a.nsub;
    const int hk  = (rt.mg / a.nsub) % a.hkv;
    const int b   = (rt.mg / a.nsub) / a.hkv;
    rt.nq  = min(QG, a.qgroup - sub * QG);
    rt.oh0 = (b * a.hkv + hk) * a.qgroup + sub * QG;
    const int s = rt.s;
    const unsigned epoch = read_epoch<QG>(a, rt.mg);
    const int wave = uniform((int)(threadIdx.x >> 6));
    const int lane = (int)(threadIdx.x & 63);
    const int g    = lane >> 4;                  // quarter
    const int col  = lane & 15;                  // column / row-in-block
    const int cg   = col / QP;                   // scale group of this column
    const int cq   = col % QP;                   // query slot of this column

    int L = a.L;
    bool bad = false;
    if constexpr (PAGED) {
        const int cap = min(a.L, min(a.S * a.chunk, a.max_pages << a.page_shift));
        L = a.seq_lens[b];
        if (L > cap || L < 0) { bad = true; L = L < 0 ? 0 : cap; }   // outside [0, max_seq_len]: NaN output
    }
    const int j0 = s * a.chunk;
    const int n  = min(L - j0, a.chunk);

    // Per lane, for its column (cg, cq): running max mq and weight sum lsum of
    // query slot cq, and the row exponent ex (the P.V operands and the o row of
    // this column carry an exact factor 2^ex, |ex| <= 100).
    float mq = M_INIT, ex = 0.f, lsum = 0.f;
    f32x4 o[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) o[nb] = f32x4{0.f, 0.f, 0.f, 0.f};

    if (n > 0) {
        const int niter = (n + TB - 1) / TB;
        const size_t   row0  = PAGED ? 0 : (size_t)hk * a.L + j0;
        const uint32_t nsplt = PAGED ? 0u : (uint32_t)n;
        const __amdgpu_buffer_rsrc_t rk  = make_rsrc(a.k + row0 * ROWB, nsplt * ROWB);
        const __amdgpu_buffer_rsrc_t rv  = make_rsrc(a.v + row0 * ROWB, nsplt * ROWB);
        const __amdgpu_buffer_rsrc_t rsk = make_rsrc(a.sk + row0 * NG, nsplt * NG * 2);
        const __amdgpu_buffer_rsrc_t rsv = make_rsrc(a.sv + row0 * NG, nsplt * NG * 2);
        int p0 = 0;
        if constexpr (PAGED) {
            p0 = j0 >> a.page_shift;
            const int np = ((j0 + n - 1) >> a.page_shift) - p0 + 1;
            const int32_t* tab = a.block_table + (size_t)b * a.max_pages + p0;
            for (int i = (int)threadIdx.x; i < np; i += WAVES * 64) s_page[i] = tab[i];
            __syncthreads();
        }

        const uint32_t koff = (uint32_t)(col * ROWB + g * DQ);     // K: row n, quarter g
        const uint32_t soff_l = (uint32_t)min(lane, SCE - 1) * (NG >= 2 ? 4u : 2u);

        u32x4 ka[2][KL], kb[2][KL], va_[VL], vb[VL];
        uint32_t ska, sva, skb, svb;

        auto load_tile = [&](int it, u32x4 (&kk)[2][KL], u32x4* vv, uint32_t& sk, uint32_t& sv) {
            const int t0 = it * TB + wave * TW;
            __amdgpu_buffer_rsrc_t tk = rk, tv = rv, tsk = rsk, tsv = rsv;
            uint32_t soff = (uint32_t)t0;
            if constexpr (PAGED) {
                const int pos  = j0 + t0;
                const int rows = max(0, min(TW, n - t0));
                int page = 0;
                if (rows > 0) page = uniform(s_page[(pos >> a.page_shift) - p0]);
                const bool ok = page >= 0 && page < a.num_pages;
                bad = bad || (rows > 0 && !ok);
                const uint32_t nrow = ok ? (uint32_t)rows : 0u;
                const size_t row = ((size_t)(ok ? page : 0) * a.hkv + hk) * ((size_t)1 << a.page_shift) +
                                   (size_t)(pos & ((1 << a.page_shift) - 1));
                tk  = make_rsrc(a.k + row * ROWB, nrow * ROWB);
                tv  = make_rsrc(a.v + row * ROWB, nrow * ROWB);
                tsk = make_rsrc(a.sk + row * NG, nrow * NG * 2);
                tsv = make_rsrc(a.sv + row * NG, nrow * NG * 2);
                soff = 0;
            }
            const uint32_t tpos = sgpr(soff);
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (NG >= 2) {
                sk = ld32(tsk, soff_l, tpos * NG * 2);
                sv = ld32(tsv, soff_l, tpos * NG * 2);
            } else {
                sk = ld16(tsk, soff_l, tpos * 2);
                sv = ld16(tsv, soff_l, tpos * 2);
            }
#pragma unroll
            for (int c = 0; c < 2; ++c)
#pragma unroll
                for (int i = 0; i < KL; ++i) {
                    if constexpr (Q3) {
                        const u32x3 w = ld96(tk, koff + (uint32_t)(c * 16 * ROWB), tpos * ROWB);
                        kk[c][i] = u32x4{w.x, w.y, w.z, 0u};
                    } else if constexpr (DQ >= 16) {
                        kk[c][i] = ld128(tk, koff + (uint32_t)(c * 16 * ROWB + 16 * i), tpos * ROWB);
                    } else {
                        const u32x2 h = ld64(tk, koff + (uint32_t)(c * 16 * ROWB), tpos * ROWB);
                        kk[c][i] = u32x4{h.x, h.y, 0u, 0u};
                    }
                }
#pragma unroll
            for (int i = 0; i < VL; ++i) {
                if constexpr (Q3) {
                    const u32x3 w = ld96(tv, (uint32_t)(12 * (64 * i + lane)), tpos * ROWB);
                    vv[i] = u32x4{w.x, w.y, w.z, 0u};
                } else {
                    vv[i] = ld128(tv, (uint32_t)(16 * (64 * i + lane)), tpos * ROWB);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        };

        // This lane's q words are loaded ahead of tile 0: vector loads complete
        // in order, so the digit arithmetic below then overlaps the tile's
        // latency instead of waiting for it. (Words are taken out of each vector
        // right after its load.)
        constexpr int EPQ = D / 4;                // dimensions of a lane quarter
        uint32_t qwd[EPQ / 2];
        {
            const _Float16* qrow = reinterpret_cast<const _Float16*>(a.q) + (size_t)(rt.oh0 + (cq < rt.nq ? cq : 0)) * D;
#pragma unroll
            for (int i = 0; i < EPQ / 8; ++i) {
                const u32x4 w = *reinterpret_cast<const u32x4*>(qrow + g * EPQ + 8 * i);
                qwd[4 * i] = w.x; qwd[4 * i + 1] = w.y; qwd[4 * i + 2] = w.z; qwd[4 * i + 3] = w.w;
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        load_tile(0, ka, va_, ska, sva);

        // q^T operand of the q.K products: column (cg, cq); k slots of quarter g
        // for MFMA j are dimensions g*DQ + 16j + e, zero outside group cg and for
        // unused slots. q is exact as three balanced int8 digits of the integer
        // round(q * 2^sh), sh per column putting max|q| in [2^21, 2^22) (every
        // fp16 element within 2^-11 of the maximum is exact; below, the error is
        // under 2^-23 of it), so each digit's dot with the int8 codes is exact
        // in int32.
        u32x4 qd[3][NJ];
        float cf;                                 // qscale * 2^-sh of this column
        int   qoff[3] = {0, 0, 0};                // q4: -8 * (column sum of each digit)
        {
            const int e0 = g * EPQ;               // they all lie in scale group e0 / G
            const bool use = cq < rt.nq && e0 / G == cg;
            float qe[EPQ];
            float lmax = 0.f;
#pragma unroll
            for (int i = 0; i < EPQ / 8; ++i) {
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const uint32_t wd = qwd[4 * i + (e >> 1)];
                    const uint32_t h = (e & 1) ? (wd >> 16) : (wd & 0xFFFFu);
                    qe[8 * i + e] = use ? h2f(h) : 0.f;
                    lmax = fmaxf(lmax, fabsf(qe[8 * i + e]));
                }
            }
            const float cmax = rows_max(lmax);          // column maximum over the quarters
            int sh = 0;
            if (cmax > 0.f) sh = 22 - ((int)((__builtin_bit_cast(uint32_t, cmax) >> 23) & 0xFF) - 126);
            const float up = __builtin_bit_cast(float, (uint32_t)(127 + sh) << 23);
            cf = a.qscale * __builtin_bit_cast(float, (uint32_t)(127 - sh) << 23);
            float dsum[3] = {0.f, 0.f, 0.f};
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                uint32_t bq[3][4] = {};
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    // k slot e of MFMA j: q8 dimension 16j + e of the quarter; q4 the
                    // nibble order of the A operand (low nibbles, then high nibbles)
                    const int de = !Q4 ? 16 * j + e : (D == 128 ? 2 * e + j : (e < 8 ? 2 * e : 2 * (e - 8) + 1));
                    const int qi = (int)__builtin_rintf(qe[de] * up);        // |qi| < 2^22
                    const int d0 = (qi << 24) >> 24;
                    const int r1 = (qi - d0) >> 8;
                    const int d1 = (r1 << 24) >> 24;
                    const int d2 = (r1 - d1) >> 8;                           // |d2| <= 64
                    bq[0][e >> 2] |= (uint32_t)(d0 & 0xFF) << (8 * (e & 3));
                    bq[1][e >> 2] |= (uint32_t)(d1 & 0xFF) << (8 * (e & 3));
                    bq[2][e >> 2] |= (uint32_t)(d2 & 0xFF) << (8 * (e & 3));
                    dsum[0] += (float)d0;
                    dsum[1] += (float)d1;
                    dsum[2] += (float)d2;
                }
#pragma unroll
                for (int k = 0; k < 3; ++k) qd[k][j] = u32x4{bq[k][0], bq[k][1], bq[k][2], bq[k][3]};
            }
            if constexpr (Q4 || Q3) {             // codes enter as n = v + 8 (q4), v + 4 (q3)
#pragma unroll
                for (int k = 0; k < 3; ++k) {
                    const float cs = rows_sum(dsum[k]);
                    qoff[k] = (Q4 ? -8 : -4) * (int)cs;
                }
            }
        }
        const uint32_t magic = [] { uint32_t m; VA_VGPR_CONST(m, 0x64646464); return m; }();

        // tr8 source row of this lane: tr row e = col/2 is position 16(e/4) + 4g + e%4,
        // half (col & 1) of a 16-byte column chunk.
        const int te   = col >> 1;
        const int tpos_row = 16 * (te >> 2) + 4 * g + (te & 3);
        const uint32_t vrd = (uint32_t)((tpos_row + 4 * (te >> 2)) * VSTR + 8 * (col & 1));
        uint8_t* const sv_w = &s_v[wave][0];

        // Multiply accumulator rows by the per-column factor f of their column:
        // accumulator row 4g + v is stacked row (column) 4g + v.
        auto scale_rows = [&](f32x4 (&acc_o)[NB], float f) {
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const float fv = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute((4 * g + v) << 2, __builtin_bit_cast(int, f)));
#pragma unroll
                for (int nb = 0; nb < NB; ++nb) acc_o[nb][v] *= fv;
            }
        };

        auto compute_tile = [&](int it, const u32x4 (&kk)[2][KL], const u32x4* vv, uint32_t sk, uint32_t sv) {
            const int rem = uniform(n - (it * TB + wave * TW));
            // V tile -> LDS (row-major, rows 16..31 shifted by 4 slots)
#pragma unroll
            for (int i = 0; i < VL; ++i) {
                const int chunk = 64 * i + lane;
                if constexpr (Q3) {               // a quarter row of codes -> 32 bytes
                    const int row = chunk >> 2, qtr = chunk & 3;
                    uint32_t bt[8];
                    q3_to_bytes(vv[i], bt);
                    uint8_t* dst = sv_w + (row + 4 * (row >> 4)) * VSTR + 32 * qtr;
                    *reinterpret_cast<u32x4*>(dst)      = u32x4{bt[0], bt[1], bt[2], bt[3]};
                    *reinterpret_cast<u32x4*>(dst + 16) = u32x4{bt[4], bt[5], bt[6], bt[7]};
                } else {
                    const int row = chunk / (ROWB / 16), c16 = chunk % (ROWB / 16);
                    *reinterpret_cast<u32x4*>(sv_w + (row + 4 * (row >> 4)) * VSTR + 16 * c16) = vv[i];
                }
            }
            // scales -> LDS as (k | v << 16) pairs, [group][row]
            if (lane < SCE) {
                if constexpr (NG >= 2) {
                    const int f = 2 * lane;
                    s_sc[wave][f % NG][f / NG]             = __builtin_amdgcn_perm(sv, sk, 0x05040100u);
                    s_sc[wave][(f + 1) % NG][(f + 1) / NG] = __builtin_amdgcn_perm(sv, sk, 0x07060302u);
                } else {
                    s_sc[wave][0][lane] = (sk & 0xFFFFu) | (sv << 16);
                }
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            // q.K: two 16-row blocks; per digit, NJ int8 MFMAs straight on the codes
            i32x4 acc[3][2];
#pragma unroll
            for (int k = 0; k < 3; ++k)
#pragma unroll
                for (int c = 0; c < 2; ++c) acc[k][c] = i32x4{qoff[k], qoff[k], qoff[k], qoff[k]};
            uint32_t kb3[2][8];                   // q3: the codes of each block as bytes
            if constexpr (Q3) {
#pragma unroll
                for (int c = 0; c < 2; ++c) q3_to_bytes(kk[c][0], kb3[c]);
            }
#pragma unroll
            for (int j = 0; j < NJ; ++j)
#pragma unroll
                for (int c = 0; c < 2; ++c) {
                    u32x4 kop;                    // A operand: int8 codes of 16 k slots
                    if constexpr (Q3) {
                        kop = u32x4{kb3[c][4 * j], kb3[c][4 * j + 1], kb3[c][4 * j + 2], kb3[c][4 * j + 3]};
                    } else if constexpr (!Q4) {
                        kop = kk[c][j];
                    } else if constexpr (D == 128) {
                        kop = j == 0 ? (kk[c][0] & 0x0F0F0F0Fu) : ((kk[c][0] >> 4) & 0x0F0F0F0Fu);
                    } else {
                        const uint32_t w0 = kk[c][0].x, w1 = kk[c][0].y;
                        kop = u32x4{w0 & 0x0F0F0F0Fu, w1 & 0x0F0F0F0Fu, (w0 >> 4) & 0x0F0F0F0Fu, (w1 >> 4) & 0x0F0F0F0Fu};
                    }
#pragma unroll
                    for (int k = 0; k < 3; ++k) acc[k][c] = mfma_i8(kop, qd[k][j], acc[k][c]);
                }
            // V^T operands of the P.V products (independent of the softmax, so their
            // LDS reads and unpack overlap the q.K MFMAs)
            f16x8 vf[NB];
#pragma unroll
            for (int c16 = 0; c16 < NC; ++c16) {
                const i32x2 t = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_i32x2*)(sv_w + vrd + 16 * c16));
                if constexpr (Q3) vf[c16] = q3b_to_f16x8((uint32_t)t[0], (uint32_t)t[1], magic);
                else if constexpr (!Q4) vf[c16] = q8_to_f16x8((uint32_t)t[0], (uint32_t)t[1], magic);
                else q4_to_f16x8((uint32_t)t[0], (uint32_t)t[1], magic, vf[2 * c16], vf[2 * c16 + 1]);
            }
            // scale pairs of this lane's 8 positions (16c + 4g + v), group cg
            const u32x4 sc0 = *reinterpret_cast<const u32x4*>(&s_sc[wave][cg][4 * g]);
            const u32x4 sc1 = *reinterpret_cast<const u32x4*>(&s_sc[wave][cg][16 + 4 * g]);
            float x[8];
#pragma unroll
            for (int c = 0; c < 2; ++c)
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    // digits recombined: 2^16 acc2 + (2^8 acc1 + acc0), one rounding
                    const float t = __builtin_fmaf((float)acc[2][c][v], 65536.f, (float)(acc[1][c][v] * 256 + acc[0][c][v]));
                    x[4 * c + v] = t * (h2f_lo(c ? sc1[v] : sc0[v]) * cf);
                }
            // sum the NG group columns of each query slot (row rotations by QP, 2QP)
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                if constexpr (NG == 4) { x[e] += dpp<dpp_row_ror(8)>(x[e]); x[e] += dpp<dpp_row_ror(4)>(x[e]); }
                if constexpr (NG == 2) { x[e] += dpp<dpp_row_ror(8)>(x[e]); }
            }
            if (rem < TW) {                       // partial tile: rows at or past rem are masked
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    if (16 * (e >> 2) + 4 * g + (e & 3) >= rem) x[e] = -__builtin_inff();
            }
            float tmax = x[0];
#pragma unroll
            for (int e = 1; e < 8; ++e) tmax = fmaxf(tmax, x[e]);
            const bool raise = __builtin_amdgcn_ballot_w64(tmax > mq + RESCALE_SLACK) != 0;
            if (raise) {
                // new maximum of each query slot: over its NG columns and the 4 quarters
                float mx = fmaxf(mq, tmax);
                if constexpr (NG == 4) { mx = fmaxf(mx, dpp<dpp_row_ror(8)>(mx)); mx = fmaxf(mx, dpp<dpp_row_ror(4)>(mx)); }
                if constexpr (NG == 2) { mx = fmaxf(mx, dpp<dpp_row_ror(8)>(mx)); }
                mx = rows_max(mx);
                const float c = fast_exp2(mq - mx);
                mq = mx;
                lsum *= c;
                scale_rows(o, c);
            }
            // weights p and the operand values p * s_v * 2^ex (2^ex: exact scaling)
            const float fe = __builtin_bit_cast(float, (uint32_t)(127 + (int)ex) << 23);
            float xv[8], xmax = 0.f;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float p = fast_exp2(x[e] - mq);
                lsum += p;
                const uint32_t pr = e < 4 ? sc0[e] : sc1[e - 4];
                xv[e] = (p * h2f_hi(pr)) * fe;
                xmax = fmaxf(xmax, xv[e]);
            }
            // Row exponent: keep operands <= 2^15 (fp16 range), and after a new
            // maximum re-centre them near 2^14 so the lo halves stay normal.
            if (raise || __builtin_amdgcn_ballot_w64(xmax > 32768.f)) {
                const float mc = rows_max(xmax);                // max of the row (column) over quarters
                int dl = 0;
                if (mc > 0.f) dl = 14 - ((int)((__builtin_bit_cast(uint32_t, mc) >> 23) & 0xFF) - 126);
                dl = max(-100 - (int)ex, min(100 - (int)ex, dl));
                const float f = __builtin_bit_cast(float, (uint32_t)(127 + dl) << 23);
                ex += (float)dl;
#pragma unroll
                for (int e = 0; e < 8; ++e) xv[e] *= f;
                scale_rows(o, f);
            }
            // fp16 hi + lo (both RNE), k slot e = 4c + v
            f16x8 ahi, alo;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const _Float16 hi = (_Float16)xv[e];
                ahi[e] = hi;
                alo[e] = (_Float16)(xv[e] - (float)hi);
            }
            // P.V over NB column blocks
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
                o[nb] = mfma_16x16x32(ahi, vf[nb], o[nb]);
                o[nb] = mfma_16x16x32(alo, vf[nb], o[nb]);
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        };

        // Tiles in pairs; an odd count leaves after its last tile (niter is
        // uniform over the work-group; the prefetch past the split reads nothing).
        //
        // q4 and q3 rows keep both waves of a SIMD (waves w and w ^ 4 under the
        // dispatcher's round-robin placement) busy on the vector ALU, and the
        // older one wins issue: it runs ahead, and the other finishes alone with
        // half the loads in flight. Each wave posts its tile pair in LDS and
        // takes issue priority while it trails its partner. The entries are
        // not cleared first: the partner's entry may still hold what an earlier
        // work-group on this CU left there, which only sets one pair's
        // priority, never a result (clearing both entries before the loop
        // measured ~1 us slower for grouped q4+ and q3+ at L 65536).
        // Measured on MI355X, Hq 32 / Hkv 8, 7 interleaved rounds: L 65536 q4+
        // 24.5 -> 24.3 us, q3+ 28.6 -> 28.3 us; paged B 8 x 16384 q4+ 45.6 ->
        // 43.5 us. q8 rows lose ~0.2 us with it and keep free issue.
        constexpr bool PRIO = WAVES == 8 && (KIND == KQ4 || KIND == KQ3);
        const int npair = (niter + 1) / 2;
        for (int ip = 0; ip < npair; ++ip) {
            const int it = 2 * ip;
            if constexpr (PRIO) {
                __hip_atomic_store(&s_prog[wave], ip + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
                const int other = uniform(__hip_atomic_load(&s_prog[wave ^ 4], __ATOMIC_RELAXED,
                                                            __HIP_MEMORY_SCOPE_WORKGROUP));
                if (other > ip + 1) __builtin_amdgcn_s_setprio(2);
                else __builtin_amdgcn_s_setprio(0);
            }
            load_tile(it + 1, kb, vb, skb, svb);
            compute_tile(it, ka, va_, ska, sva);
            if (it + 1 >= niter) break;
            load_tile(it + 2, ka, va_, ska, sva);
            compute_tile(it + 1, kb, vb, skb, svb);
        }
        if constexpr (PRIO) __builtin_amdgcn_s_setprio(0);
    }

    // ---- work-group merge. Per query slot q: lsum of column q summed over the
    // 4 quarters (every group column of q holds the same sum), m = mq; o row
    // (cg', q) drops its row factor 2^ex (an exact power of two).
    const float lt = rows_sum(lsum);
    if (lane < QG) {
        s_l[lane][wave] = lt;
        s_m[lane][wave] = mq;
    }
    // Row (grp, cq) of this lane's accumulators holds its useful dimensions in
    // the JB column blocks of scale group grp (grp depends on the quarter g):
    // the blocks are picked by selects, not branches.
    constexpr int JB = G / 16;                       // column blocks per scale group
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        const int r = 4 * g + v;                     // stacked row (r / QP, r % QP)
        const int grp = r / QP, cq_r = QP == 4 ? v : r % QP;
        const float er = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(r << 2, __builtin_bit_cast(int, ex)));
        const float f  = __builtin_bit_cast(float, (uint32_t)(127 - (int)er) << 23);
        if (cq_r < QG) {
#pragma unroll
            for (int j = 0; j < JB; ++j) {
                float val = o[j][v];
#pragma unroll
                for (int gg = 1; gg < NG; ++gg) val = grp == gg ? o[gg * JB + j][v] : val;
                // q8: block nb is dimensions 16nb + col; q4: byte column 16(nb/2) + col,
                // low nibble (even dimension) or high nibble (odd, accumulated as 16v)
                const int nb = grp * JB + j;
                const int d = !Q4 ? 16 * nb + col : 2 * (16 * (nb >> 1) + col) + (j & 1);
                s_red[cq_r][wave][d] = val * ((Q4 && (j & 1)) ? f * 0.0625f : f);
            }
        }
    }
    bool any_bad = false;
    if constexpr (PAGED) any_bad = __syncthreads_or(bad);
    else __syncthreads();
    // fold the WAVES partials of each (query slot, dimension), one per thread
    const int t = (int)threadIdx.x;
    static_assert(QG * D <= WAVES * 64, "one thread per (query slot, dimension)");
    if (t < QG * D) {
        const int q = t / D, d = t - (t / D) * D;
        float m = s_m[q][0];
#pragma unroll
        for (int w = 1; w < WAVES; ++w) m = fmaxf(m, s_m[q][w]);
        float sacc = 0.f, sl = 0.f;
#pragma unroll
        for (int w = 0; w < WAVES; ++w) {
            const float f = fast_exp2(s_m[q][w] - m);
            sacc = __builtin_fmaf(f, s_red[q][w][d], sacc);
            sl   = __builtin_fmaf(f, s_l[q][w], sl);
        }
        s_acc[q][d] = sacc;
        if (d == 0) {
            s_mf[q] = m;
            s_lf[q] = any_bad ? __builtin_nanf("") : sl;
        }
    }
    __syncthreads();
    float M[QG], acc[QG], ls[QG];
#pragma unroll
    for (int q = 0; q < QG; ++q) {
        M[q] = s_mf[q];
        ls[q] = s_lf[q];
        acc[q] = t < D ? s_acc[q][t] : 0.f;
    }
    finish_partial<D, WAVES * 64, QG>(a, rt, M, ls, acc, epoch);
}

} // namespace va
