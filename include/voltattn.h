/* voltattn.h — C ABI of the MI355X (gfx950) fused dequant + decode-attention
 * library libvoltattn_hip.so.
 *
 * The reference (kamilch1k/voltattn) has no plugin or FFI layer: its path sits
 * behind the file-static C++ function
 *     void launch(Fmt f, const DeviceBufs& b, int H, int L, int D, int S)
 * (src/voltattn.cu:803-835), fed by host-side format code and a CUDA runtime
 * used directly. This header is that boundary as a C ABI: plain pointers,
 * sizes and int status codes, no HIP or torch types. Every entry point names
 * the reference interface it replaces.
 *
 * Conventions
 *   - Every function returns VA_OK (0) or a VA_E* code; va_last_error() gives
 *     the calling thread's message for the last failure.
 *   - "Device pointer" means memory from va_malloc (or any HIP device
 *     allocation). The caller owns every buffer, as in the reference.
 *   - `stream` is a hipStream_t passed as void*; NULL is the default stream.
 *     Launch functions are asynchronous, like the reference's launch().
 *   - Layouts (src/voltattn.cu:92-93, 676-745):
 *       K, V payload  [H][L][row]  row = 2*D bytes (f16), D (q8), D/2 (q4), 3*D/8 (q3)
 *         q8: int8 per element; q4: element e in byte e/2, low nibble first,
 *         stored v+8; q3: element e at bits [3e, 3e+3) of a little-endian
 *         stream (8 elements per 3-byte granule), stored v+4;
 *       scales        [H][L][D/G]  fp16 bits (quantized formats only)
 *       q, out        [H][D]       fp16 bits
 *       ws            va_ws_bytes(H, D, S) bytes; fully overwritten each call.
 */
#ifndef VOLTATTN_H
#define VOLTATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define VA_ABI_VERSION 4

/* Status codes. */
enum {
    VA_OK       = 0,
    VA_EINVAL   = 1,  /* bad argument: format, shape, group size, split count */
    VA_EALIGN   = 2,  /* pointer alignment the kernels require is not met */
    VA_ENULL    = 3,  /* a required pointer is NULL */
    VA_ERANGE   = 4,  /* shape exceeds the 32-bit buffer addressing of a head */
    VA_EHIP     = 5,  /* HIP runtime or launch error */
    VA_ENODEV   = 6,  /* no usable gfx950 device */
    VA_ELOST    = 7,  /* a fused merge gave up waiting for a partial (va_merge_faults) */
    VA_EBUSY    = 8   /* va_decode_noalloc: the device's workspace is bound to another stream */
};

/* Formats: the reference's enum class Fmt {F16, F16M, Q8, Q8M, Q4, Q4M, Q3M}
 * (src/voltattn.cu:676). The "+" formats select the tiled multi-position
 * kernels; the others the naive one-position-per-wave kernels. The type is an
 * int in C and C++ alike: under C++ it is given that underlying type, so a
 * caller's out-of-range value is still a valid va_fmt that the entry points
 * reject with VA_EINVAL (rather than undefined behaviour). */
#ifdef __cplusplus
#define VA_ENUM_BASE : int
#else
#define VA_ENUM_BASE
#endif
typedef enum VA_ENUM_BASE {
    VA_F16  = 0,   /* f16   naive  (attn_f16,     src/voltattn.cu:122-187) */
    VA_F16P = 1,   /* f16+  tiled  (attn_f16_mlp, src/voltattn.cu:364-423) */
    VA_Q8   = 2,   /* q8    naive  (attn_q8,      src/voltattn.cu:189-252) */
    VA_Q8P  = 3,   /* q8+   tiled  (attn_q8_mlp,  src/voltattn.cu:425-490) */
    VA_Q4   = 4,   /* q4    naive  (attn_q4,      src/voltattn.cu:254-320) */
    VA_Q4P  = 5,   /* q4+   tiled  (attn_q4_mlp,  src/voltattn.cu:492-561) */
    VA_Q3P  = 6    /* q3+   tiled  (attn_q3_mlp,  src/voltattn.cu:563-649) */
} va_fmt;

/* Device buffers of one decode step: the reference's struct DeviceBufs
 * {K, V, scK, scV, q, out, ws} (src/voltattn.cu:796-801).
 * Alignment: k, v 16 bytes (4 for q3); sk, sv 4 bytes (2 when D/G == 1);
 * q 16 bytes; out 2 bytes; ws 4 bytes. sk/sv are ignored for f16 formats. */
typedef struct {
    const void*     k;
    const void*     v;
    const uint16_t* sk;
    const uint16_t* sv;
    const uint16_t* q;
    uint16_t*       out;
    float*          ws;
} va_bufs;

/* One decode step: per head softmax(q.K^T / sqrt(D)) V over L positions,
 * split into S chunks of ceil(L/S) positions, partials merged by log-sum-exp,
 * fp16 output. Replaces launch() (src/voltattn.cu:803-835), adding the group
 * size G (the reference fixes GROUP = 64, src/voltattn.cu:60).
 * Valid: D in {64,128}; G in {32,64} with G <= D (ignored for f16 formats);
 * H >= 1; L >= 1; S >= 1. Asynchronous on `stream`.
 * The merge normally runs inside the decode kernel on a ticket slot of
 * library memory bound to `stream` (one slot per stream, and one per stream
 * and capture sequence while a graph is captured; 16 per device). Calls on
 * different streams may run concurrently; replays of one captured graph must
 * be ordered after each other (as every launch of one executable graph is).
 * When all 16 slots are bound, a call may take over the slot of an eager
 * stream that has finished its work; slots of captured graphs are kept until
 * va_graph_destroy or va_capture_release. With H > 1024,
 * S > 64, H*S > 2048, no slot to be had, or the per-thread default stream
 * (hipStreamPerThread, one handle naming a stream per host thread), the
 * partials go to ws and a separate merge kernel follows. */
int va_decode(va_fmt fmt, const va_bufs* b, int H, int L, int D, int G, int S, void* stream);

/* va_decode without a workspace argument, for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). No counterpart in the reference. b->ws is ignored: the two-pass
 * form's partials go to a workspace of library device memory (4 MiB per
 * device, held until the process ends), so H*S*(D+2) must not exceed
 * VA_NOALLOC_MAX_FLOATS (VA_ERANGE otherwise). Allocates nothing; same
 * kernels and outputs as va_decode. The fused merge (va_decode) uses no
 * workspace; the two-pass form binds the device's workspace to the calling
 * stream (or stream and capture sequence; for hipStreamPerThread, the calling
 * thread) as ticket slots are bound: another owner's two-pass call returns
 * VA_EBUSY, unless the owner is an eager stream that has finished its work
 * (the binding then moves). Calls never share the workspace while they may
 * overlap. va_stream_release / va_capture_release free the binding. */
#define VA_NOALLOC_MAX_FLOATS 1048576
int va_decode_noalloc(va_fmt fmt, const va_bufs* b, int H, int L, int D, int G, int S, void* stream);

/* Release what `stream` holds on the current device: its fused-merge ticket
 * slot and its binding of the allocation-free workspace (for
 * hipStreamPerThread, the calling thread's), after waiting for the stream's
 * work. For streams the library did not create (va_stream_destroy releases
 * its own), before they are destroyed or when they stop decoding. No
 * counterpart in the reference, which launches on the default stream only. */
int va_stream_release(void* stream);

/* Release the ticket slots and workspace binding of a graph capture sequence
 * (the id hipStreamGetCaptureInfo reported while capturing), after waiting for
 * the device: for graphs captured outside va_graph_begin/end (which
 * va_graph_destroy releases), once they will not be replayed again. No
 * counterpart in the reference. */
int va_capture_release(unsigned long long capture_id);

/* Fused merges on the current device that gave up waiting for a partial
 * (bounded poll exhausted; the affected outputs were set to NaN) since the
 * previous call. Synchronizes `stream` first. Returns VA_ELOST with *count > 0
 * if there were any, else VA_OK with *count = 0. No counterpart in the
 * reference, whose merge is a separate kernel. */
int va_merge_faults(void* stream, unsigned* count);

/* First pass only: writes the S partials (m, l, o[D]) per head into b->ws
 * (the attention kernels of launch(), src/voltattn.cu:813-833). `out` unused. */
int va_decode_splits(va_fmt fmt, const va_bufs* b, int H, int L, int D, int G, int S,
                     void* stream);

/* Second pass only: log-sum-exp merge of S partials per head into fp16 out
 * (combine, src/voltattn.cu:651-672). */
int va_merge(const float* ws, uint16_t* out, int H, int D, int S, void* stream);

/* Workspace bytes for (H, D, S): H*S*(D+2) floats, the reference's
 * cudaMalloc(&b.ws, H*S*(D+2)*4) (src/voltattn.cu:888). */
size_t va_ws_bytes(int H, int D, int S);

/* Payload bytes of K (or V) for a format: the reference's qbytes() / n*2
 * (src/voltattn.cu:692, 990-991). 0 for an invalid format. */
size_t va_payload_bytes(va_fmt fmt, int H, int L, int D);

/* Scale bytes of K (or V): H*L*(D/G)*2, 0 for f16 formats
 * (src/voltattn.cu:880-881, 991). */
size_t va_scale_bytes(va_fmt fmt, int H, int L, int D, int G);

/* Positions per split the library would use for (L, S): ceil(L/S), the
 * reference's chunk (src/voltattn.cu:804). */
int va_split_chunk(int L, int S);

/* A split count that fills the device for (fmt, H, L, D): the reference's
 * S = max(1, min(2*SMs/H, ceil(L/512))) (src/voltattn.cu:1026) re-derived
 * for 256 CUs and the tiled kernels' work-group tile. */
int va_pick_splits(va_fmt fmt, int H, int L, int D, int* S);

/* Printable format name, "f16", "f16+", ... (fmt_name, src/voltattn.cu:677-687). */
const char* va_fmt_name(va_fmt fmt);

/* Device-side symmetric per-group quantizer + packer, bit-exact with the
 * reference's host quantize() (src/voltattn.cu:705-745) for G in {32,64}.
 * x: device fp32 [rows][D]; packed: rows*D*bits/8 bytes (4-byte aligned);
 * scales: rows*(D/G) fp16. bits in {8,4,3}. */
int va_quantize(int bits, int G, const float* x, size_t rows, int D, void* packed,
                uint16_t* scales, void* stream);

/* Device-side inverse of va_quantize: packed codes (rows*D*bits/8 bytes,
 * 4-byte aligned) and fp16 scales (rows*(D/G)) to fp32 values out[rows][D]
 * (16-byte aligned), bit-exact with the reference's host dq()
 * (src/voltattn.cu:747-767): float(scale) * code, exact in fp32. bits in
 * {8,4,3}, G in {32,64}. */
int va_dequantize(int bits, int G, const void* packed, const uint16_t* scales, size_t rows, int D,
                  float* out, void* stream);

/* Device-side fp32 -> fp16 round-to-nearest-even over n values (the
 * reference's __float2half loops, src/voltattn.cu:866-868, 1000-1002). */
int va_f32_to_f16(const float* x, size_t n, uint16_t* out, void* stream);

/* Seeded N(0,1) fill of n fp32 values on the device (bench data; the
 * reference's fill_fast, src/voltattn.cu:959-965, fills on the host). */
int va_fill_normal(float* x, size_t n, uint64_t seed, void* stream);

/* Empirical HBM read ceiling: best GB/s over `reps` timed reads of a
 * `bytes`-sized device buffer, taking the best of several launch shapes: a
 * grid-stride read (the reference's form, probe_ceiling + read_kernel,
 * src/voltattn.cu:64-78, 935-957) and a chunked read (each work-group streams
 * one contiguous chunk, the shape of a decode split; buffers of 16 MiB and up). */
int va_probe_read(size_t bytes, int reps, double* best_gbps);

/* One launch of a read-probe form of va_probe_read over the caller's device
 * buffer, with a digest of what it read: xor4 = the XOR of every 16-byte word
 * loaded (as four little-endian uint32), *loads = the 16-byte loads issued,
 * *bytes_read = the bytes va_probe_read credits the form with (all of
 * `bytes`, for both forms). form 0: the grid-stride read (read_kernel's shape,
 * src/voltattn.cu:69-78): `grid` groups of 256 threads, unroll 2, 4 or 8 loads
 * in flight per lane; form 1: the chunked read: `grid` groups of 256 threads,
 * each streaming one contiguous chunk, unroll 4 or 8. bytes: a positive
 * multiple of 16; src 16-byte aligned. Synchronous. A form that skipped,
 * repeated or over-counted bytes does not reproduce the XOR and load count of
 * the same bytes computed on the host. */
int va_probe_digest(const void* src, size_t bytes, int form, int grid, int unroll, uint32_t* xor4,
                    uint64_t* loads, size_t* bytes_read);

/* Size-matched read ceiling of one decode step of `bytes`: the chunked read of
 * va_probe_read over exactly `bytes` per launch with one or two 4-wave groups
 * per CU (the decode grid), `launches` launches back to back on one stream
 * between two events, rotating over copies that together span >= min_set
 * bytes (so the Infinity Cache cannot serve them), each shape after at least
 * 50 ms of untimed launches (the clocks leave their idle level); the best
 * mean over the chunked shapes. Returns microseconds per launch and bytes /
 * that time in GB/s: what any kernel that reads that many bytes per launch
 * pays, launch gap, ramp and tail included. No counterpart in the reference
 * (its probe reads one fixed 256 MiB buffer, src/voltattn.cu:935-957). */
int va_probe_read_sized(size_t bytes, size_t min_set, int launches, double* us_per_launch,
                        double* gbps);

/* Launch floor: microseconds per launch of an empty kernel with one 256-thread
 * work-group per CU (the decode step's grid at H*S = CUs), `launches` of them
 * back to back on a private stream after a warm-up: an upper bound on the
 * launch cost a decode step pays outside its own work (part of it overlaps a
 * running kernel). No counterpart in the reference (its bench reports only the
 * read ceiling); a measurement aid like va_probe_read. */
int va_probe_launch(int launches, double* us_per_launch);

/* ---- grouped-query attention, batches and paged caches ----
 * No counterpart in the reference, which decodes one sequence with one query
 * head per K/V head from a contiguous cache (its README.md:205-206 lists GQA
 * and paged KV as missing). The row formats, quantizer and arithmetic are the
 * reference path's; only the tiled formats (f16+, q8+, q4+, q3+) run here,
 * the naive ones return VA_EINVAL. Query head i of a sequence attends KV head
 * i / (Hq / Hkv) (consecutive query heads share a KV head). */

/* One sequence, Hq query heads over Hkv KV heads (Hq % Hkv == 0): b->q and
 * b->out are [Hq][D]; k, v, sk, sv are the contiguous [Hkv][L][...] layouts of
 * va_decode; ws holds va_ws_bytes(Hq, D, S). Each K/V row is unpacked once for
 * all query heads that share it. Hq == Hkv is exactly va_decode. S = 0 picks
 * the split count (va_pick_splits_gqa). */
int va_decode_gqa(va_fmt fmt, const va_bufs* b, int Hq, int Hkv, int L, int D, int G, int S,
                  void* stream);
int va_pick_splits_gqa(va_fmt fmt, int Hq, int Hkv, int L, int D, int* S);

/* Shape of a batch decoded from a page pool. Page p of the pool holds
 * [Hkv][page_rows][row] payload bytes (row as for va_decode) and
 * [Hkv][page_rows][D/G] fp16 scales; position j of sequence b is row
 * j % page_rows of page block_table[b][j / page_rows]. A contiguous cache
 * [Hkv][Lcap][row] per sequence is the case page_rows = Lcap (a power of two)
 * with block_table[b] = {b}. */
typedef struct {
    int B;             /* sequences in the batch */
    int Hq, Hkv;       /* query and KV heads per sequence, Hq % Hkv == 0 */
    int D, G;          /* D in {64,128}; G in {32,64} (ignored for f16 formats) */
    int page_rows;     /* positions per page: a power of two >= 64 */
    int max_pages;     /* block-table row length (pages per sequence at most) */
    int num_pages;     /* pages in the pool; ids outside [0, num_pages) are rejected */
    int max_seq_len;   /* >= every seq_lens[b]: sizes the splits */
} va_paged_shape;

/* Device buffers of a paged batch. Alignment as va_bufs (k, v 16 bytes, 4 for
 * q3; sk, sv 4 bytes; q 16 bytes); block_table and seq_lens 4 bytes. */
typedef struct {
    const void*     k;             /* K page pool */
    const void*     v;             /* V page pool */
    const uint16_t* sk;            /* K scale pool (quantized formats) */
    const uint16_t* sv;            /* V scale pool */
    const int32_t*  block_table;   /* [B][max_pages] page ids */
    const int32_t*  seq_lens;      /* [B] positions per sequence (0 .. max_seq_len) */
    const uint16_t* q;             /* [B][Hq][D] fp16 */
    uint16_t*       out;           /* [B][Hq][D] fp16 */
    float*          ws;            /* va_ws_bytes(B * Hq, D, S) bytes */
} va_paged_bufs;

/* One decode step of every sequence of the batch: per (sequence, query head)
 * softmax(q.K^T / sqrt(D)) V over that sequence's seq_lens[b] positions.
 * Splits are S ranges of ceil(max_seq_len / S) positions (rounded up to the
 * kernel tile); a sequence shorter than max_seq_len leaves its later splits
 * empty. A sequence of length 0 gives a zero output; a length above
 * max_seq_len, or a page id outside the pool on one of its positions, gives
 * NaN for that sequence's heads. S = 0 picks the split count
 * (va_pick_splits_paged). Asynchronous on `stream`. */
int va_decode_paged(va_fmt fmt, const va_paged_bufs* b, const va_paged_shape* shape, int S,
                    void* stream);
int va_pick_splits_paged(va_fmt fmt, const va_paged_shape* shape, int* S);

/* Payload bytes and scale bytes of one page (0 for invalid arguments). */
size_t va_page_bytes(va_fmt fmt, int Hkv, int page_rows, int D);
size_t va_page_scale_bytes(va_fmt fmt, int Hkv, int page_rows, int D, int G);

/* The cache write path: quantize-and-append n new rows per (sequence, KV
 * head). x is fp16 [B][Hkv][n][D] (16-byte aligned); row r of sequence b is
 * written at position start[b] + r of the page pool `pages` (+ `scales`,
 * quantized formats), laid out as in va_paged_shape (page_rows may be any
 * value >= 1 here). Quantized formats apply the reference's quantizer
 * (quantize(), src/voltattn.cu:705-745) to the fp16 values, bit-exact with
 * va_quantize on the same values; f16 formats copy. Rows whose position lies
 * past max_pages * page_rows, or on a page id outside [0, num_pages), are not
 * written. The fields Hq and max_seq_len of `shape` are unused. */
int va_append_kv(va_fmt fmt, const uint16_t* x, int n, const int32_t* start,
                 const int32_t* block_table, const va_paged_shape* shape, void* pages,
                 uint16_t* scales, void* stream);

/* ---- runtime shims (the reference calls the CUDA runtime directly:
 *      cudaMalloc/cudaMemcpy/cudaFree/cudaEvent*, src/voltattn.cu:863-895, 936-955,
 *      cudaGetDeviceProperties, src/voltattn.cu:968-971) ---- */
typedef struct {
    char   name[256];
    char   arch[64];          /* e.g. "gfx950:sramecc+:xnack-" */
    int    compute_units;
    int    clock_khz;
    int    mem_clock_khz;
    int    mem_bus_bits;
    size_t total_mem;
    size_t l2_bytes;
} va_device_info_t;

int va_device_count(int* n);
int va_set_device(int dev);
int va_device_info(va_device_info_t* info);
int va_malloc(void** p, size_t bytes);
int va_free(void* p);
int va_memcpy_h2d(void* dst, const void* src, size_t bytes);
int va_memcpy_d2h(void* dst, const void* src, size_t bytes);
int va_memcpy_d2d(void* dst, const void* src, size_t bytes, void* stream);
int va_memset(void* p, int value, size_t bytes);
int va_sync(void);
int va_stream_create(void** stream);
/* Waits for the stream's work, frees the fused-merge ticket slot bound to it
 * (va_decode), then destroys it. */
int va_stream_destroy(void* stream);
int va_stream_sync(void* stream);
int va_event_create(void** ev);
int va_event_destroy(void* ev);
int va_event_record(void* ev, void* stream);
int va_event_sync(void* ev);
int va_event_elapsed_ms(void* start, void* stop, float* ms);

/* HIP graph capture of a launch sequence on a (non-default) stream: the
 * reference launches every step from the host; a serving loop would replay
 * captured decode steps instead. va_graph_end instantiates the captured work;
 * va_graph_launch replays it on `stream`; replays of one graph must be ordered
 * after each other. va_graph_destroy waits for the device and frees the
 * ticket slots the capture bound (va_decode). No memset nodes are captured by
 * any entry point of this library. */
int va_graph_begin(void* stream);
int va_graph_end(void* stream, void** graph_exec);
int va_graph_launch(void* graph_exec, void* stream);
int va_graph_destroy(void* graph_exec);

/* Message of the calling thread's last failure ("" if none). */
const char* va_last_error(void);

/* VA_ABI_VERSION of the loaded library. */
int va_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* VOLTATTN_H */
