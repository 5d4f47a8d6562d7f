// va_kernels.hpp — internal (C++) interface between the C-ABI layer
// (va_runtime.hip) and the kernel translation units. Not part of the ABI.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

namespace va {

// Arguments of the split-L decode pass (one work-group per (head, split)).
struct DecodeArgs {
    const uint8_t*  k;      // payload [H][L][row bytes]
    const uint8_t*  v;
    const uint16_t* sk;     // fp16 scales [H][L][D/G] (quantized kinds)
    const uint16_t* sv;
    const uint16_t* q;      // fp16 [H][D]
    float*          ws;     // [H*S][D+2]: (m, l, o[D]) per split, m in log2 units
                            // (two-pass form only)
    uint16_t*       out;    // fp16 [H][D], written by the fused merge
    int   L, S, chunk;
    float qscale;           // log2(e) / sqrt(D)
    int   ticket_slot;      // >= 0: fused merge on this ticket slot; < 0: partials to ws
};

// Fused second pass: per-(slot, head) ticket lines in static device memory
// (zero at load): word 0 counts the arrivals of the head's work-groups, word 1
// is the head's call epoch, advanced by the merging work-group. Calls rotate
// over TICKET_SLOTS slots, so up to that many decode calls may be in flight on
// one device at once. Each line is 256 bytes: atomics to one line serialize at
// the memory side, and the S arrivals of every head land together.
// The partials of a fused call live in library memory (PART_CAP partials of
// PART_STRIDE 64-bit words per slot), not in the caller's ws. Calls with more
// than TICKET_MAXH heads or more than PART_CAP partials use the two-pass form.
constexpr int TICKET_SLOTS  = 16;
constexpr int TICKET_MAXH   = 256;
constexpr int TICKET_STRIDE = 64;   // uint32 per ticket line (256 bytes)
constexpr int PART_CAP      = 1024; // partials (H*S) per slot
constexpr int PART_STRIDE   = 130;  // 64-bit words per partial: m, l, o[D], D <= 128

// kind: 0 f16, 1 q8, 2 q4, 3 q3. tiled: the "+" kernels; otherwise the naive
// one-position-per-wave kernels (f16, q8, q4 only).
hipError_t launch_decode(int kind, bool tiled, int H, int D, int G,
                         const DecodeArgs& a, hipStream_t stream);

// Work-groups per CU the split rule aims for (tiled kernels: the configured
// groups per CU of the kind; naive kernels: 8).
int groups_per_cu(int kind, bool tiled);

// Positions one work-group of the tiled kernel covers per loop iteration;
// split lengths that are multiples of it leave no partial tile.
int tile_positions(int kind, bool tiled, int D);

// Second pass: log-sum-exp merge of the S partials of every head, fp16 out.
hipError_t launch_merge(const float* ws, uint16_t* out, int H, int D, int S,
                        hipStream_t stream);

// Read-bandwidth probe kernel over `bytes` (multiple of 16) at `src`.
hipError_t launch_probe(const void* src, size_t bytes, float* sink, int grid,
                        int unroll, hipStream_t stream);

// Bit-exact quantizer (bits 8/4/3) over rows of D fp32 values.
hipError_t launch_quantize(int bits, int G, const float* x, size_t rows, int D,
                           uint8_t* packed, uint16_t* scales, hipStream_t stream);

// fp32 -> fp16 (round to nearest even) over n values.
hipError_t launch_f32_to_f16(const float* x, size_t n, uint16_t* out, hipStream_t stream);

// Seeded N(0,1) fill (Philox4x32-10 + Box-Muller), n values.
hipError_t launch_fill_normal(float* x, size_t n, uint64_t seed, hipStream_t stream);

} // namespace va
