// oracle.hpp — CPU restatement of kamilch1k/voltattn's decode-attention path.
//
// TEST INFRASTRUCTURE ONLY. This library is the checker for the HIP product in
// voltattn_amd/: only tests/, __graft_entry__.smoke() and bench.py's
// cpu_baseline leg and after-timing output check may link, load or call it,
// as the checker. Nothing in the product path uses
// it, and the product must never fall back to it.
//
// What it restates (citations are src/voltattn.cu:line in the reference):
//   * the seeded input draw of the selftest (run_case, va.cu:838-846): one
//     std::mt19937 and one std::normal_distribution<float>, drawing K, then V,
//     then q (rounded to fp16);
//   * IEEE-754 binary16 round-to-nearest-even conversion (the reference's
//     __float2half / __half2float, va.cu:722-723, 846, 852-853);
//   * the symmetric per-group quantizer and packer (quantize, va.cu:705-745),
//     generalised over the group size G in {32, 64} (the reference fixes 64,
//     va.cu:60);
//   * the exact dequantizer (dq, va.cu:747-767);
//   * the double-precision reference attention (reference, va.cu:769-794);
//   * the split-L partial + log-sum-exp merge algebra (va.cu:80-120, 651-672),
//     in double, so the merge can be checked against the unsplit reference.
//
// Pins (where each function is checked, see tests/):
//   mt19937          — C++ standard known answer (10000th output 4123659995)
//                      and stream equality with libstdc++ (tests/golden/).
//   normal_polar     — stream equality with libstdc++ normal_distribution<float>
//                      (GCC 11.4, the reference's host toolchain).
//   f32_to_f16       — numpy float16 RNE conversion over edge cases.
//   quantize/dequant — closed-form invariants, hand-made ties, layout
//                      round-trips, and (end to end with reference()) the
//                      reference's own logged selftest maxerr values
//                      (results/v100-fhhl-16gb-run3.txt:4-45).
//   reference        — scipy softmax in float64; identical-row and
//                      dominant-row closed forms.
//   split_attention  — equality with reference() for every split count.
#pragma once
#include <cstddef>
#include <cstdint>
#include <vector>

namespace oracle {

// ---- IEEE binary16 ---------------------------------------------------------
uint16_t f32_to_f16(float x);   // round to nearest, ties to even
float    f16_to_f32(uint16_t h); // exact

// ---- RNG: restatement of std::mt19937 + libstdc++ normal_distribution<float>
class Mt19937 {
public:
    explicit Mt19937(uint32_t seed = 5489u);
    uint32_t next();
private:
    void twist();
    uint32_t mt_[624];
    int idx_;
};

class NormalPolar { // mean 0, stddev 1
public:
    float next(Mt19937& g);
private:
    bool  have_saved_ = false;
    float saved_ = 0.f;
};

// Seed of selftest case (H, L, D, S): va.cu:922.
uint32_t selftest_seed(int H, int L, int D, int S);

// Draws of run_case (va.cu:839-846): kx[n], then vx[n], then q[H*D] as fp16.
struct CaseDraw {
    std::vector<float>    kx, vx;
    std::vector<uint16_t> q; // fp16 bits
};
CaseDraw draw_case(int H, int L, int D, uint32_t seed);

// ---- formats ----------------------------------------------------------------
// bits: 16 (fp16, no scales), 8, 4, 3. Packed layouts (va.cu:694-745):
//   8: int8 per element;
//   4: element e -> byte e/2, low nibble when e is even, stored as v+8;
//   3: element e -> bits [3e, 3e+3) of a little-endian bit stream
//      (8 elements per 3-byte granule), stored as v+4.
// Scales: fp16 bits, index (row)*(D/G) + g, row = h*L + j.
size_t packed_bytes(int bits, size_t n);
int    qlimit(int bits); // 127, 7, 3

struct Quantized {
    std::vector<uint8_t>  data;   // packed payload
    std::vector<uint16_t> scale;  // fp16 bits, [rows][D/G]
};
Quantized quantize(const float* x, size_t rows, int D, int G, int bits);
// Exact dequantized value of element idx (double(float(scale)) * v).
double dequant(const Quantized& z, size_t idx, int D, int G, int bits);
// Decoded integer code of element idx (before scaling).
int    code_at(const uint8_t* data, size_t idx, int bits);

// ---- attention ----------------------------------------------------------------
// reference(): va.cu:769-794. kd, vd: float[H*L*D]; q: fp16 bits [H*D].
std::vector<float> reference(const float* kd, const float* vd, const uint16_t* q,
                             int H, int L, int D);
// Same maths computed as S split partials (chunk = ceil(L/S), va.cu:804) merged
// by log-sum-exp (va.cu:651-672), in double. Returns out[H*D] and, when the
// pointers are non-null, per-(h,s) log-sum-exp (natural log; -inf when empty)
// and normalised split outputs o_s/l_s (zero when empty).
std::vector<float> split_attention(const float* kd, const float* vd, const uint16_t* q,
                                   int H, int L, int D, int S,
                                   double* lse_out, double* avg_out);

// Build the exact inputs of one selftest-style case for a format.
// Returns the dequantized float K/V the reference consumes (kd, vd) and the
// device-format buffers (payload bytes and scales; for bits==16 the payload
// is fp16 bits of kx/vx and there are no scales).
struct CaseData {
    int H = 0, L = 0, D = 0, G = 0, bits = 0;
    std::vector<float>    kd, vd;
    std::vector<uint16_t> q;
    std::vector<uint8_t>  kpay, vpay;
    std::vector<uint16_t> kscale, vscale;
    std::vector<float>    ref;
};
CaseData make_case(int bits, int H, int L, int D, int G, uint32_t seed);

} // namespace oracle
