// va_kernels.hpp — internal (C++) interface between the C-ABI layer
// (va_runtime.hip) and the kernel translation units. Not part of the ABI.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

namespace va {

// Arguments of the split-L decode pass: one work-group per (merge group,
// split), a merge group being one (sequence b, KV head hk, query sub-group).
// The reference's shape is B = 1, hkv = H, qgroup = 1, contiguous K/V.
struct DecodeArgs {
    const uint8_t*  k;      // payload: contiguous [hkv][L][row bytes], or the page pool
    const uint8_t*  v;      //   [num_pages][hkv][page_rows][row bytes]
    const uint16_t* sk;     // fp16 scales, same layouts with D/G per row (quantized kinds)
    const uint16_t* sv;
    const uint16_t* q;      // fp16 [B][hkv*qgroup][D]
    float*          ws;     // [B*hkv*qgroup][S][D+2]: (m, l, o[D]) per split, m in log2 units
                            // (two-pass form only)
    uint16_t*       out;    // fp16 [B][hkv*qgroup][D], written by the fused merge
    int   L, S, chunk;      // L: positions (paged form: max_seq_len); chunk: positions per split
    float qscale;           // log2(e) / sqrt(D)
    int   ticket_slot;      // >= 0: fused merge on this ticket slot; < 0: partials to ws
    // grouped-query attention: query head (b, hk*qgroup + i) reads KV head hk
    int   hkv;              // KV heads per sequence
    int   qgroup;           // query heads per KV head
    int   nsub;             // query sub-groups per KV head (ceil(qgroup / QG))
    // paged form (block table over a page pool)
    const int32_t* block_table;   // [B][max_pages] page ids
    const int32_t* seq_lens;      // [B] positions per sequence
    int   max_pages;        // block-table row length
    int   page_shift;       // log2(page_rows)
    int   num_pages;        // pages in the pool (ids outside [0, num_pages) are rejected)
};

// Launch of the tiled decode kernel: the leading scalar arguments (preloaded
// into SGPRs) followed by the rest of the DecodeArgs.
#define VA_TILED_ARGS(a) (a).k, (a).v, (a).sk, (a).sv, (a).L, (a).S, (a).chunk, (a).ticket_slot, (a).q, \
    ((a).ticket_slot >= 0 ? static_cast<void*>((a).out) : static_cast<void*>((a).ws)), (a)

// Fused second pass: per-(slot, merge group) ticket lines in static device
// memory (zero at load): word 0 counts the arrivals of the group's
// work-groups, word 1 is the group's call epoch (tagged protocol), advanced by
// the merging work-group, word 2 counts the groups whose partials are stored
// (counted protocol). A slot belongs to one stream (or one captured stream of
// a graph) at a time (va_slots.hpp), so calls that may overlap never share
// one; when a device's TICKET_SLOTS are all bound, further streams use the
// two-pass form. Each line is 256 bytes:
// atomics to one line serialize at the memory side, and the S arrivals of every
// group land together. The partials of a fused call live in library memory
// (PART_CAP partials per slot: PART_STRIDE 64-bit words tagged, PARTF_STRIDE
// floats plain), not in the caller's ws.
// Calls with more than TICKET_MAXH merge groups, more than PART_CAP partials or
// more than 64 splits use the two-pass form.
constexpr int TICKET_SLOTS  = 16;
constexpr int TICKET_MAXH   = 1024;
constexpr int TICKET_STRIDE = 64;   // uint32 per ticket line (256 bytes)
constexpr int PART_CAP      = 2048; // partials (merge groups x QG x S) per slot
constexpr int PART_STRIDE   = 130;  // 64-bit words per partial: m, l, o[D], D <= 128
constexpr int PARTF_STRIDE  = 132;  // floats per plain partial: o[D], m, l (16-byte rows), D <= 128

// Tags of the one-slot merge's partial words: (epoch mod 2^TAG_EPOCH_BITS) << 7
// | S, S in [1, 64], so a tag is never 0 (the cleared state). Within one S the
// word address fixes the merge group and split, so a word written under
// another S never matches; a word of the same group and split written
// 2^TAG_EPOCH_BITS of the group's calls earlier would, which the host rules
// out by clearing a slot's store (clear_tagged_*) when it changes owner and
// after every SLOT_CLEAR_CALLS eager calls on it. A captured graph's slot is
// replayed with the split counts of its capture, so every word it reads was
// written by the previous call of the same group and S.
constexpr int TAG_EPOCH_BITS = 25;
constexpr unsigned long long SLOT_CLEAR_CALLS = 1ull << (TAG_EPOCH_BITS - 1);

// Page ids of one split of the paged kernels are staged in LDS: a split may
// span at most this many pages.
constexpr int MAX_SPLIT_PAGES = 1024;

// kind: 0 f16, 1 q8, 2 q4, 3 q3. tiled: the "+" kernels; otherwise the naive
// one-position-per-wave kernels (f16, q8, q4 only).
hipError_t launch_decode(int kind, bool tiled, int H, int D, int G,
                         const DecodeArgs& a, hipStream_t stream);

// Grouped-query and paged forms of the tiled kernels (va_decode_ex.hip).
// groups = merge groups (B * hkv * nsub); qg = query slots per work-group
// (max_query_slots(kind, D) at most); paged selects the block-table form.
hipError_t launch_decode_ex(int kind, int D, int G, int qg, bool paged, int groups,
                            const DecodeArgs& a, hipStream_t stream);

// Largest query-slot count (QG) a work-group of the kind carries, and the
// work-group tile (positions per iteration) of the grouped/paged kernels.
int max_query_slots(int kind, int D);
int tile_positions_ex(int kind, int D);
// Work-groups per CU the grouped/paged launch of (kind, QG) is built for.
int ex_groups_per_cu(int kind, int D, int qg);

// Work-groups per CU the split rule aims for (tiled kernels: the configured
// groups per CU of the kind; naive kernels: 8).
int groups_per_cu(int kind, bool tiled);

// Positions one work-group of the tiled kernel covers per loop iteration;
// split lengths that are multiples of it leave no partial tile.
int tile_positions(int kind, bool tiled, int D);

// Host side: the count of fused merges that gave up waiting for a partial
// (poll bound exhausted; the output was set to NaN) in the code object of the
// reference-shape kernels (va_decode.hip) and of the grouped/paged kernels
// (va_decode_ex.hip). The counters only grow.
hipError_t lost_merges_decode(unsigned* n);
hipError_t lost_merges_ex(unsigned* n);

// Zero the tagged partial store of ticket slot `slot` in the code object of the
// reference-shape kernels (va_decode.hip) and of the grouped/paged kernels
// (va_decode_ex.hip), on `stream`.
hipError_t clear_tagged_decode(int slot, hipStream_t stream);
hipError_t clear_tagged_ex(int slot, hipStream_t stream);

// Second pass: log-sum-exp merge of the S partials of every head, fp16 out.
hipError_t launch_merge(const float* ws, uint16_t* out, int H, int D, int S,
                        hipStream_t stream);

// Read-bandwidth probes. Each launch writes one digest per work-group to
// dig[g * PROBE_DIGEST_WORDS ..]: the XOR of every 16-byte word the group
// loaded (4 words), then the number of 16-byte loads it issued.
constexpr int PROBE_DIGEST_WORDS = 8;

// Grid-stride probe over `bytes` (multiple of 16) at `src`.
hipError_t launch_probe(const void* src, size_t bytes, uint32_t* dig, int grid,
                        int unroll, hipStream_t stream);

// Chunked probe: `grid` work-groups, group g streaming the contiguous chunk
// [g*per, min(bytes, (g+1)*per)) with per = probe_chunk_bytes(bytes, grid),
// unroll 4 or 8 loads per lane in flight; covers exactly `bytes` (a multiple
// of 16, per < 2^31).
size_t probe_chunk_bytes(size_t bytes, int grid);
hipError_t launch_probe_chunks(const void* src, size_t bytes, uint32_t* dig, int grid, int unroll,
                               hipStream_t stream);

// Empty kernel of `grid` 256-thread groups (the launch-floor probe).
hipError_t launch_empty(int grid, float* sink, hipStream_t stream);

// Bit-exact quantizer (bits 8/4/3) over rows of D fp32 values.
hipError_t launch_quantize(int bits, int G, const float* x, size_t rows, int D,
                           uint8_t* packed, uint16_t* scales, hipStream_t stream);

// Inverse of the quantizer: packed codes + fp16 scales of rows x D elements to
// fp32 (bits 8/4/3, G 32/64), bit-exact with the reference's dq().
hipError_t launch_dequantize(int bits, int G, const uint8_t* packed, const uint16_t* scales, size_t rows,
                             int D, float* out, hipStream_t stream);

// Quantize-and-append of n new fp16 rows per (sequence, KV head) into a page
// pool [num_pages][hkv][page_rows][row bytes] (+ fp16 scales [...][D/G]).
struct AppendArgs {
    const uint16_t* x;            // [B][hkv][n][D] fp16
    const int32_t*  start;        // [B]: position of row 0 of each sequence
    const int32_t*  block_table;  // [B][max_pages]
    uint8_t*        pages;
    uint16_t*       scales;
    int B, hkv, n, D;
    int page_rows, max_pages, num_pages;
};
hipError_t launch_append(int bits, int G, const AppendArgs& a, hipStream_t stream);

// fp32 -> fp16 (round to nearest even) over n values.
hipError_t launch_f32_to_f16(const float* x, size_t n, uint16_t* out, hipStream_t stream);

// Seeded N(0,1) fill (Philox4x32-10 + Box-Muller), n values.
hipError_t launch_fill_normal(float* x, size_t n, uint64_t seed, hipStream_t stream);

} // namespace va
