// oracle.cpp — CPU restatement of kamilch1k/voltattn's decode-attention path.
// TEST INFRASTRUCTURE ONLY: the checker for the HIP product, never part of it.
// Citations are src/voltattn.cu:line ("va.cu") in the reference.
//
// Build: oracle/Makefile (g++ -O2 -ffp-contract=off, no -march: the x87-free
// SSE float arithmetic of the reference's GCC 11 host build, no FMA).
#include "oracle.hpp"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <thread>

namespace oracle {

// ---------------------------------------------------------------- binary16 --
// IEEE 754-2008 binary16: 1 sign, 5 exponent (bias 15), 10 fraction bits.
// Written from the standard; matches CUDA's documented __float2half (RNE).
uint16_t f32_to_f16(float x) {
    uint32_t u;
    std::memcpy(&u, &x, 4);
    const uint32_t sign = (u >> 16) & 0x8000u;
    const uint32_t e32  = (u >> 23) & 0xFFu;
    const uint32_t m32  = u & 0x7FFFFFu;
    if (e32 == 0xFFu)                       // inf or NaN (NaN stays quiet NaN)
        return (uint16_t)(sign | 0x7C00u | (m32 ? (0x200u | (m32 >> 13)) : 0u));
    const int e16 = (int)e32 - 127 + 15;
    if (e16 >= 31) return (uint16_t)(sign | 0x7C00u);   // |x| >= 2^16: overflow
    if (e16 >= 1) {                                     // normal result
        uint32_t r = ((uint32_t)e16 << 10) | (m32 >> 13);
        const uint32_t rem = m32 & 0x1FFFu;
        if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) ++r; // carry may reach inf
        return (uint16_t)(sign | r);
    }
    // subnormal or zero result: value = full * 2^(e32-150), unit 2^-24
    if (e32 == 0) return (uint16_t)sign;                // |x| < 2^-126
    const uint32_t full  = m32 | 0x800000u;
    const int      shift = 126 - (int)e32;              // >= 14
    if (shift > 24) return (uint16_t)sign;              // < 2^-25 (ties at 2^-25 go to 0)
    uint32_t r = full >> shift;
    const uint32_t rem  = full & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (r & 1u))) ++r;   // may become the min normal
    return (uint16_t)(sign | r);
}

float f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e    = (h >> 10) & 0x1Fu;
    const uint32_t m    = h & 0x3FFu;
    uint32_t u;
    if (e == 0) {
        if (m == 0) u = sign;
        else {                               // subnormal: m * 2^-24
            const float v = (float)m * 5.9604644775390625e-8f;
            std::memcpy(&u, &v, 4);
            u |= sign;
        }
    } else if (e == 31) {
        u = sign | 0x7F800000u | (m << 13);
    } else {
        u = sign | ((e - 15 + 127) << 23) | (m << 13);
    }
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

// ----------------------------------------------------------------- mt19937 --
// Matsumoto & Nishimura (1998), the parameters fixed by [rand.predef] for
// std::mt19937: w=32 n=624 m=397 r=31 a=0x9908b0df u=11 d=0xffffffff s=7
// b=0x9d2c5680 t=15 c=0xefc60000 l=18 f=1812433253.
Mt19937::Mt19937(uint32_t seed) {
    mt_[0] = seed;
    for (int i = 1; i < 624; ++i)
        mt_[i] = 1812433253u * (mt_[i - 1] ^ (mt_[i - 1] >> 30)) + (uint32_t)i;
    idx_ = 624;
}

void Mt19937::twist() {
    for (int i = 0; i < 624; ++i) {
        const uint32_t y = (mt_[i] & 0x80000000u) | (mt_[(i + 1) % 624] & 0x7FFFFFFFu);
        mt_[i] = mt_[(i + 397) % 624] ^ (y >> 1) ^ ((y & 1u) ? 0x9908B0DFu : 0u);
    }
    idx_ = 0;
}

uint32_t Mt19937::next() {
    if (idx_ >= 624) twist();
    uint32_t y = mt_[idx_++];
    y ^= y >> 11;
    y ^= (y << 7) & 0x9D2C5680u;
    y ^= (y << 15) & 0xEFC60000u;
    y ^= y >> 18;
    return y;
}

// ------------------------------------------------------- normal (polar) -----
// libstdc++ (GCC 11.4, the reference's host toolchain) draws
// std::normal_distribution<float> with Marsaglia's polar method, keeping the
// second variate of each accepted pair for the next call. Its uniforms come
// from generate_canonical<float, 24>, which for a 32-bit engine takes one
// engine output u and returns float(u) / 2^32 (float(u) rounded to nearest;
// a result that rounds up to 1 is replaced by the largest float below 1).
// The candidate coordinates are formed as float(double(2.0f*U) - 1.0), the
// radius r2 = x*x + y*y in float, accepted when 0 < r2 <= 1, and the factor
// sqrt(-2*log(r2)/r2) in float arithmetic (logf, sqrtf).
static float canonical_f32(Mt19937& g) {
    const float sum = (float)g.next();
    float r = sum / 4294967296.0f;
    if (r >= 1.0f) r = std::nextafter(1.0f, 0.0f);
    return r;
}

float NormalPolar::next(Mt19937& g) {
    float ret;
    if (have_saved_) {
        have_saved_ = false;
        ret = saved_;
    } else {
        float x, y, r2;
        do {
            x  = (float)((double)(2.0f * canonical_f32(g)) - 1.0);
            y  = (float)((double)(2.0f * canonical_f32(g)) - 1.0);
            r2 = x * x + y * y;
        } while (r2 > 1.0f || r2 == 0.0f);
        const float mult = std::sqrt(-2.0f * std::log(r2) / r2);
        saved_      = x * mult;
        have_saved_ = true;
        ret         = y * mult;
    }
    return ret * 1.0f + 0.0f; // stddev 1, mean 0
}

uint32_t selftest_seed(int H, int L, int D, int S) {
    return 0xC0FFEEu ^ (uint32_t)(H * 131 + L * 7 + D + S);   // va.cu:922
}

CaseDraw draw_case(int H, int L, int D, uint32_t seed) {      // va.cu:839-846
    Mt19937 g(seed);
    NormalPolar nd;
    const size_t n = (size_t)H * L * D;
    CaseDraw c;
    c.kx.resize(n);
    c.vx.resize(n);
    c.q.resize((size_t)H * D);
    for (auto& v : c.kx) v = nd.next(g);
    for (auto& v : c.vx) v = nd.next(g);
    for (auto& v : c.q)  v = f32_to_f16(nd.next(g));
    return c;
}

// ------------------------------------------------------------------ formats --
size_t packed_bytes(int bits, size_t n) {                     // va.cu:692
    switch (bits) {
        case 16: return n * 2;
        case 8:  return n;
        case 4:  return n / 2;
        case 3:  return n * 3 / 8;
        default: return 0;
    }
}

int qlimit(int bits) { return bits == 8 ? 127 : bits == 4 ? 7 : 3; }   // va.cu:711

// x86-64 lrint semantics as the reference's GCC build sees them: round to
// nearest even under the default MXCSR mode; a quotient that is not finite or
// exceeds the long range yields 0x8000000000000000, and the int conversion at
// va.cu:725 keeps its low 32 bits, i.e. 0.
static int lrint_to_int(float t) {
    if (!std::isfinite(t) || std::fabs(t) >= 9.2233720368547758e18f) return 0;
    const long lv = std::lrint(t);
    return (int)(int32_t)(uint32_t)(uint64_t)lv;
}

// Symmetric per-group quantizer + packer: va.cu:705-745 with GROUP -> G.
//   amax = max |x| over the group (fp32); s = amax > 0 ? amax/lim : 1;
//   the fp16 scale is s rounded to nearest even; codes are
//   clamp(lrint(x / float(scale)), -lim, lim).
Quantized quantize(const float* x, size_t rows, int D, int G, int bits) {
    const int    ng  = D / G;
    const int    lim = qlimit(bits);
    const size_t n   = rows * (size_t)D;
    Quantized r;
    r.scale.resize(rows * ng);
    r.data.assign(packed_bytes(bits, n), 0);
    for (size_t rowg = 0; rowg < rows * ng; ++rowg) {
        const size_t base = (rowg / ng) * D + (rowg % ng) * G;
        float amax = 0.f;
        for (int i = 0; i < G; ++i) amax = std::max(amax, std::fabs(x[base + i]));
        const float s = amax > 0.f ? amax / (float)lim : 1.f;
        r.scale[rowg] = f32_to_f16(s);
        const float sh = f16_to_f32(r.scale[rowg]);
        for (int i = 0; i < G; ++i) {
            int v = lrint_to_int(x[base + i] / sh);
            v = std::max(-lim, std::min(lim, v));
            const size_t e = base + i;
            if (bits == 8) {
                r.data[e] = (uint8_t)(int8_t)v;
            } else if (bits == 4) {
                uint8_t& b = r.data[e / 2];
                const uint8_t nib = (uint8_t)(v + 8);
                b = (e % 2 == 0) ? (uint8_t)((b & 0xF0) | nib) : (uint8_t)((b & 0x0F) | (nib << 4));
            } else {
                const size_t   bit  = 3 * e;
                const uint32_t code = (uint32_t)(v + 4) << (bit & 7);
                r.data[bit >> 3] |= (uint8_t)code;
                if ((bit & 7) > 5) r.data[(bit >> 3) + 1] |= (uint8_t)(code >> 8);
            }
        }
    }
    return r;
}

int code_at(const uint8_t* data, size_t idx, int bits) {
    if (bits == 8) return (int)(int8_t)data[idx];
    if (bits == 4) {
        const uint8_t b = data[idx / 2];
        return (int)((idx % 2 == 0) ? (b & 0xF) : (b >> 4)) - 8;
    }
    const size_t bit = 3 * idx;                                 // va.cu:757-762
    uint32_t w = data[bit >> 3];
    if ((bit & 7) > 5) w |= (uint32_t)data[(bit >> 3) + 1] << 8;
    return (int)((w >> (bit & 7)) & 7u) - 4;
}

double dequant(const Quantized& z, size_t idx, int D, int G, int bits) { // va.cu:747-767
    const size_t rowg = (idx / D) * (D / G) + (idx % D) / G;
    const double s = (double)f16_to_f32(z.scale[rowg]);
    return s * code_at(z.data.data(), idx, bits);
}

// --------------------------------------------------------------- attention --
// va.cu:769-794: per head, scores in double, exp(score - max), normalised.
static void reference_heads(const float* kd, const float* vd, const uint16_t* q,
                            int h0, int h1, int L, int D, float* out) {
    std::vector<double> sc(L), od(D), qd(D);
    const double rs = std::sqrt((double)D);
    for (int h = h0; h < h1; ++h) {
        for (int d = 0; d < D; ++d) qd[d] = (double)f16_to_f32(q[(size_t)h * D + d]);
        double mx = -1e300;
        for (int j = 0; j < L; ++j) {
            const float* kr = kd + ((size_t)h * L + j) * D;
            double acc = 0.0;
            for (int d = 0; d < D; ++d) acc += qd[d] * kr[d];
            sc[j] = acc / rs;
            mx = std::max(mx, sc[j]);
        }
        double Z = 0.0;
        std::fill(od.begin(), od.end(), 0.0);
        for (int j = 0; j < L; ++j) {
            const double p = std::exp(sc[j] - mx);
            Z += p;
            const float* vr = vd + ((size_t)h * L + j) * D;
            for (int d = 0; d < D; ++d) od[d] += p * vr[d];
        }
        for (int d = 0; d < D; ++d) out[(size_t)h * D + d] = (float)(od[d] / Z);
    }
}

std::vector<float> reference(const float* kd, const float* vd, const uint16_t* q,
                             int H, int L, int D) {
    std::vector<float> out((size_t)H * D);
    reference_heads(kd, vd, q, 0, H, L, D, out.data());
    return out;
}

std::vector<float> split_attention(const float* kd, const float* vd, const uint16_t* q,
                                   int H, int L, int D, int S,
                                   double* lse_out, double* avg_out) {
    std::vector<float> out((size_t)H * D);
    const int chunk = (L + S - 1) / S;                          // va.cu:804
    const double rs = std::sqrt((double)D);
    std::vector<double> lse(S), avg((size_t)S * D), qd(D), sc;
    for (int h = 0; h < H; ++h) {
        for (int d = 0; d < D; ++d) qd[d] = (double)f16_to_f32(q[(size_t)h * D + d]);
        for (int s = 0; s < S; ++s) {
            const int j0 = std::min(L, s * chunk), j1 = std::min(L, j0 + chunk);
            double* a = &avg[(size_t)s * D];
            std::fill(a, a + D, 0.0);
            if (j1 <= j0) { lse[s] = -INFINITY; continue; }
            sc.assign(j1 - j0, 0.0);
            double m = -1e300;
            for (int j = j0; j < j1; ++j) {
                const float* kr = kd + ((size_t)h * L + j) * D;
                double acc = 0.0;
                for (int d = 0; d < D; ++d) acc += qd[d] * kr[d];
                sc[j - j0] = acc / rs;
                m = std::max(m, sc[j - j0]);
            }
            double l = 0.0;
            for (int j = j0; j < j1; ++j) {
                const double p = std::exp(sc[j - j0] - m);
                l += p;
                const float* vr = vd + ((size_t)h * L + j) * D;
                for (int d = 0; d < D; ++d) a[d] += p * vr[d];
            }
            for (int d = 0; d < D; ++d) a[d] /= l;
            lse[s] = m + std::log(l);
        }
        // log-sum-exp merge of the split partials (va.cu:651-672)
        double M = -INFINITY;
        for (int s = 0; s < S; ++s) M = std::max(M, lse[s]);
        double Z = 0.0;
        std::vector<double> od(D, 0.0);
        for (int s = 0; s < S; ++s) {
            if (lse[s] == -INFINITY) continue;
            const double w = std::exp(lse[s] - M);
            Z += w;
            for (int d = 0; d < D; ++d) od[d] += w * avg[(size_t)s * D + d];
        }
        for (int d = 0; d < D; ++d) out[(size_t)h * D + d] = (float)(od[d] / Z);
        if (lse_out) for (int s = 0; s < S; ++s) lse_out[(size_t)h * S + s] = lse[s];
        if (avg_out) std::copy(avg.begin(), avg.end(), avg_out + (size_t)h * S * D);
    }
    return out;
}

CaseData make_case(int bits, int H, int L, int D, int G, uint32_t seed) {
    CaseData c;
    c.H = H; c.L = L; c.D = D; c.G = G; c.bits = bits;
    CaseDraw dr = draw_case(H, L, D, seed);
    const size_t n = (size_t)H * L * D;
    c.q = dr.q;
    c.kd.resize(n);
    c.vd.resize(n);
    if (bits == 16) {                                           // va.cu:851-853, 866-868
        c.kpay.resize(2 * n);
        c.vpay.resize(2 * n);
        for (size_t i = 0; i < n; ++i) {
            const uint16_t kh = f32_to_f16(dr.kx[i]), vh = f32_to_f16(dr.vx[i]);
            std::memcpy(&c.kpay[2 * i], &kh, 2);
            std::memcpy(&c.vpay[2 * i], &vh, 2);
            c.kd[i] = f16_to_f32(kh);
            c.vd[i] = f16_to_f32(vh);
        }
    } else {                                                    // va.cu:855-859
        const size_t rows = (size_t)H * L;
        Quantized zk = quantize(dr.kx.data(), rows, D, G, bits);
        Quantized zv = quantize(dr.vx.data(), rows, D, G, bits);
        for (size_t i = 0; i < n; ++i) {
            c.kd[i] = (float)dequant(zk, i, D, G, bits);
            c.vd[i] = (float)dequant(zv, i, D, G, bits);
        }
        c.kpay   = std::move(zk.data);
        c.vpay   = std::move(zv.data);
        c.kscale = std::move(zk.scale);
        c.vscale = std::move(zv.scale);
    }
    c.ref = reference(c.kd.data(), c.vd.data(), c.q.data(), H, L, D);
    return c;
}

} // namespace oracle

// ------------------------------------------------------------------ C API --
// Flat entry points for ctypes (tests/, bench.py cpu_baseline, smoke()).
using namespace oracle;

extern "C" {

uint16_t oracle_f32_to_f16(float x) { return f32_to_f16(x); }
float    oracle_f16_to_f32(uint16_t h) { return f16_to_f32(h); }

void oracle_f32_to_f16_array(const float* x, size_t n, uint16_t* out) {
    for (size_t i = 0; i < n; ++i) out[i] = f32_to_f16(x[i]);
}

// n-th output (1-based) of an engine seeded with `seed`.
uint32_t oracle_mt_nth(uint32_t seed, size_t n) {
    Mt19937 g(seed);
    uint32_t v = 0;
    for (size_t i = 0; i < n; ++i) v = g.next();
    return v;
}

void oracle_mt_stream(uint32_t seed, size_t n, uint32_t* out) {
    Mt19937 g(seed);
    for (size_t i = 0; i < n; ++i) out[i] = g.next();
}

void oracle_normal_stream(uint32_t seed, size_t n, float* out) {
    Mt19937 g(seed);
    NormalPolar nd;
    for (size_t i = 0; i < n; ++i) out[i] = nd.next(g);
}

uint32_t oracle_selftest_seed(int H, int L, int D, int S) { return selftest_seed(H, L, D, S); }

void oracle_draw(uint32_t seed, int H, int L, int D, float* kx, float* vx, uint16_t* q) {
    CaseDraw c = draw_case(H, L, D, seed);
    if (kx) std::copy(c.kx.begin(), c.kx.end(), kx);
    if (vx) std::copy(c.vx.begin(), c.vx.end(), vx);
    if (q)  std::copy(c.q.begin(), c.q.end(), q);
}

size_t oracle_packed_bytes(int bits, size_t n) { return packed_bytes(bits, n); }

int oracle_quantize(const float* x, size_t rows, int D, int G, int bits,
                    uint8_t* data, uint16_t* scale) {
    if (!(bits == 8 || bits == 4 || bits == 3) || G <= 0 || D % G) return -1;
    Quantized z = quantize(x, rows, D, G, bits);
    std::copy(z.data.begin(), z.data.end(), data);
    std::copy(z.scale.begin(), z.scale.end(), scale);
    return 0;
}

int oracle_codes(const uint8_t* data, size_t n, int bits, int32_t* out) {
    if (!(bits == 8 || bits == 4 || bits == 3)) return -1;
    for (size_t i = 0; i < n; ++i) out[i] = code_at(data, i, bits);
    return 0;
}

int oracle_dequant(const uint8_t* data, const uint16_t* scale, size_t rows, int D, int G,
                   int bits, float* out) {
    if (!(bits == 8 || bits == 4 || bits == 3) || G <= 0 || D % G) return -1;
    const size_t n = rows * (size_t)D;
    for (size_t i = 0; i < n; ++i) {
        const size_t rowg = (i / D) * (D / G) + (i % D) / G;
        out[i] = (float)((double)f16_to_f32(scale[rowg]) * code_at(data, i, bits));
    }
    return 0;
}

int oracle_reference(const float* kd, const float* vd, const uint16_t* q,
                     int H, int L, int D, float* out) {
    if (H <= 0 || L <= 0 || D <= 0) return -1;
    reference_heads(kd, vd, q, 0, H, L, D, out);
    return 0;
}

// Heads split over `threads` std::threads (the bench's multi-core CPU line).
int oracle_reference_mt(const float* kd, const float* vd, const uint16_t* q,
                        int H, int L, int D, int threads, float* out) {
    if (H <= 0 || L <= 0 || D <= 0 || threads <= 0) return -1;
    threads = std::min(threads, H);
    std::vector<std::thread> pool;
    for (int t = 0; t < threads; ++t) {
        const int h0 = (int)((long)H * t / threads), h1 = (int)((long)H * (t + 1) / threads);
        pool.emplace_back(reference_heads, kd, vd, q, h0, h1, L, D, out);
    }
    for (auto& th : pool) th.join();
    return 0;
}

int oracle_split_attention(const float* kd, const float* vd, const uint16_t* q,
                           int H, int L, int D, int S, float* out,
                           double* lse, double* avg) {
    if (H <= 0 || L <= 0 || D <= 0 || S <= 0) return -1;
    std::vector<float> r = split_attention(kd, vd, q, H, L, D, S, lse, avg);
    std::copy(r.begin(), r.end(), out);
    return 0;
}

// One selftest-style case. Any output pointer may be null. Sizes: kd/vd
// H*L*D floats; q H*D halves; kpay/vpay packed_bytes(bits, H*L*D) bytes
// (2*H*L*D for bits 16); ksc/vsc H*L*D/G halves (untouched for bits 16);
// ref H*D floats.
int oracle_make_case(int bits, int H, int L, int D, int G, uint32_t seed,
                     float* kd, float* vd, uint16_t* q, uint8_t* kpay, uint8_t* vpay,
                     uint16_t* ksc, uint16_t* vsc, float* ref) {
    if (!(bits == 16 || bits == 8 || bits == 4 || bits == 3)) return -1;
    if (H <= 0 || L <= 0 || D <= 0 || G <= 0 || D % G || D % 8) return -1;
    CaseData c = make_case(bits, H, L, D, G, seed);
    if (kd)  std::copy(c.kd.begin(), c.kd.end(), kd);
    if (vd)  std::copy(c.vd.begin(), c.vd.end(), vd);
    if (q)   std::copy(c.q.begin(), c.q.end(), q);
    if (kpay) std::copy(c.kpay.begin(), c.kpay.end(), kpay);
    if (vpay) std::copy(c.vpay.begin(), c.vpay.end(), vpay);
    if (ksc && bits != 16) std::copy(c.kscale.begin(), c.kscale.end(), ksc);
    if (vsc && bits != 16) std::copy(c.vscale.begin(), c.vscale.end(), vsc);
    if (ref) std::copy(c.ref.begin(), c.ref.end(), ref);
    return 0;
}

} // extern "C"
