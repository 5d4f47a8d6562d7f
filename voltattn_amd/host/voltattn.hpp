// voltattn.hpp — C++ host mirror of kamilch1k/voltattn's interface over the
// C ABI (include/voltattn.h). Header-only; link libvoltattn_hip.so.
//
//   voltattn::Fmt         enum class Fmt {F16, F16M, Q8, Q8M, Q4, Q4M, Q3M}  (src/voltattn.cu:676)
//   voltattn::DeviceBufs  struct DeviceBufs {K, V, scK, scV, q, out, ws}      (src/voltattn.cu:796-801)
//   voltattn::launch      launch(f, b, H, L, D, S) (+ group size G)           (src/voltattn.cu:803-835)
//   voltattn::launch_splits / merge   the two passes of launch() on their own
//                         (src/voltattn.cu:813-833 and combine, 651-672)
//   voltattn::pick_splits the reference's split rule (src/voltattn.cu:1026)
//   voltattn::quantize    device quantize() (src/voltattn.cu:705-745)
//   voltattn::dequantize  device dq() over whole rows (src/voltattn.cu:747-767)
//
// Beyond the reference (its README.md:205-206 lists GQA and paged KV as
// missing): launch_gqa, launch_paged, append_kv, and the Stream / Graph
// helpers for replaying captured decode steps.
//
// Errors throw voltattn::Error (status code + message), where the reference
// exits through CUDA_CHECK (src/voltattn.cu:49-58).
#pragma once
#include "voltattn.h"

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <utility>

namespace voltattn {

enum class Fmt : int {
    F16 = VA_F16, F16M = VA_F16P, Q8 = VA_Q8, Q8M = VA_Q8P, Q4 = VA_Q4, Q4M = VA_Q4P, Q3M = VA_Q3P
};
inline constexpr Fmt kAllFormats[] = {Fmt::F16, Fmt::F16M, Fmt::Q8, Fmt::Q8M, Fmt::Q4, Fmt::Q4M, Fmt::Q3M};

inline const char* fmt_name(Fmt f) { return va_fmt_name(static_cast<va_fmt>(f)); }
inline bool is_f16(Fmt f) { return f == Fmt::F16 || f == Fmt::F16M; }
inline int qbits(Fmt f) {
    switch (f) {
        case Fmt::F16: case Fmt::F16M: return 16;
        case Fmt::Q8:  case Fmt::Q8M:  return 8;
        case Fmt::Q4:  case Fmt::Q4M:  return 4;
        default:                       return 3;
    }
}

class Error : public std::runtime_error {
public:
    Error(int code, const std::string& msg)
        : std::runtime_error("voltattn error " + std::to_string(code) + ": " + msg), code_(code) {}
    int code() const { return code_; }
private:
    int code_;
};

inline void check(int rc) {
    if (rc != VA_OK) throw Error(rc, va_last_error());
}

struct DeviceBufs {
    void*     K   = nullptr;
    void*     V   = nullptr;
    void*     scK = nullptr;
    void*     scV = nullptr;
    uint16_t* q   = nullptr;
    uint16_t* out = nullptr;
    float*    ws  = nullptr;
};

inline va_bufs to_c(const DeviceBufs& b) {
    return va_bufs{b.K, b.V, static_cast<const uint16_t*>(b.scK), static_cast<const uint16_t*>(b.scV),
                   b.q, b.out, b.ws};
}

// One decode step (attention pass + log-sum-exp merge), asynchronous.
inline void launch(Fmt f, const DeviceBufs& b, int H, int L, int D, int S, int G = 64,
                   void* stream = nullptr) {
    const va_bufs cb = to_c(b);
    check(va_decode(static_cast<va_fmt>(f), &cb, H, L, D, G, S, stream));
}

// The two passes of launch() on their own: partials into b.ws, then the merge.
inline void launch_splits(Fmt f, const DeviceBufs& b, int H, int L, int D, int S, int G = 64,
                          void* stream = nullptr) {
    const va_bufs cb = to_c(b);
    check(va_decode_splits(static_cast<va_fmt>(f), &cb, H, L, D, G, S, stream));
}
inline void merge(const float* ws, uint16_t* out, int H, int D, int S, void* stream = nullptr) {
    check(va_merge(ws, out, H, D, S, stream));
}

// launch() without a workspace (b.ws ignored), for callers that cannot
// allocate; throws Error with code VA_EBUSY while another stream or graph
// holds the device's workspace (see va_decode_noalloc).
inline void launch_noalloc(Fmt f, const DeviceBufs& b, int H, int L, int D, int S, int G = 64,
                           void* stream = nullptr) {
    const va_bufs cb = to_c(b);
    check(va_decode_noalloc(static_cast<va_fmt>(f), &cb, H, L, D, G, S, stream));
}

// Give back the merge slot and workspace binding of a stream the caller keeps
// (or of the calling thread's per-thread default stream), or of a graph
// capture sequence captured outside Graph.
inline void release_stream(void* stream) { check(va_stream_release(stream)); }
inline void release_capture(unsigned long long capture_id) { check(va_capture_release(capture_id)); }

// Fused merges that gave up waiting for a partial since the last call (the
// affected outputs are NaN); synchronises `stream`.
inline unsigned merge_faults(void* stream = nullptr) {
    unsigned n = 0;
    const int rc = va_merge_faults(stream, &n);
    if (rc != VA_OK && rc != VA_ELOST) check(rc);
    return n;
}

// Measurement aids: the read ceiling (GB/s), the size-matched ceiling of one
// decode step of `bytes` (us per launch, GB/s), one digest-checked probe
// launch, and the empty-kernel launch floor (us).
inline double probe_read(size_t bytes, int reps = 5) {
    double g = 0.0;
    check(va_probe_read(bytes, reps, &g));
    return g;
}
inline std::pair<double, double> probe_read_sized(size_t bytes, size_t min_set, int launches = 20) {
    double us = 0.0, g = 0.0;
    check(va_probe_read_sized(bytes, min_set, launches, &us, &g));
    return {us, g};
}
struct ProbeDigest {
    uint32_t xor4[4] = {0, 0, 0, 0};
    uint64_t loads = 0;
    size_t bytes_read = 0;
};
inline ProbeDigest probe_digest(const void* src, size_t bytes, int form, int grid, int unroll) {
    ProbeDigest d;
    check(va_probe_digest(src, bytes, form, grid, unroll, d.xor4, &d.loads, &d.bytes_read));
    return d;
}
inline double probe_launch(int launches = 2000) {
    double us = 0.0;
    check(va_probe_launch(launches, &us));
    return us;
}

inline size_t ws_bytes(int H, int D, int S) { return va_ws_bytes(H, D, S); }
inline size_t payload_bytes(Fmt f, int H, int L, int D) {
    return va_payload_bytes(static_cast<va_fmt>(f), H, L, D);
}
inline size_t scale_bytes(Fmt f, int H, int L, int D, int G = 64) {
    return va_scale_bytes(static_cast<va_fmt>(f), H, L, D, G);
}
inline int pick_splits(Fmt f, int H, int L, int D) {
    int S = 0;
    check(va_pick_splits(static_cast<va_fmt>(f), H, L, D, &S));
    return S;
}

// Grouped-query decode of one sequence: Hq query heads over Hkv KV heads
// (query head i reads KV head i / (Hq / Hkv)); b.q and b.out are [Hq][D],
// b.ws holds ws_bytes(Hq, D, S). S = 0 picks the split count.
inline void launch_gqa(Fmt f, const DeviceBufs& b, int Hq, int Hkv, int L, int D, int S = 0,
                       int G = 64, void* stream = nullptr) {
    const va_bufs cb = to_c(b);
    check(va_decode_gqa(static_cast<va_fmt>(f), &cb, Hq, Hkv, L, D, G, S, stream));
}
inline int pick_splits_gqa(Fmt f, int Hq, int Hkv, int L, int D) {
    int S = 0;
    check(va_pick_splits_gqa(static_cast<va_fmt>(f), Hq, Hkv, L, D, &S));
    return S;
}

// A batch decoded from a page pool (va_paged_shape documents the layout).
using PagedShape = va_paged_shape;

struct PagedBufs {
    void*          K           = nullptr;   // K page pool
    void*          V           = nullptr;   // V page pool
    void*          scK         = nullptr;   // K scale pool (quantized formats)
    void*          scV         = nullptr;   // V scale pool
    const int32_t* block_table = nullptr;   // [B][max_pages]
    const int32_t* seq_lens    = nullptr;   // [B]
    uint16_t*      q           = nullptr;   // [B][Hq][D]
    uint16_t*      out         = nullptr;   // [B][Hq][D]
    float*         ws          = nullptr;   // ws_bytes(B * Hq, D, S)
};

inline va_paged_bufs to_c(const PagedBufs& b) {
    return va_paged_bufs{b.K, b.V, static_cast<const uint16_t*>(b.scK), static_cast<const uint16_t*>(b.scV),
                         b.block_table, b.seq_lens, b.q, b.out, b.ws};
}

inline void launch_paged(Fmt f, const PagedBufs& b, const PagedShape& shape, int S = 0,
                         void* stream = nullptr) {
    const va_paged_bufs cb = to_c(b);
    check(va_decode_paged(static_cast<va_fmt>(f), &cb, &shape, S, stream));
}
inline int pick_splits_paged(Fmt f, const PagedShape& shape) {
    int S = 0;
    check(va_pick_splits_paged(static_cast<va_fmt>(f), &shape, &S));
    return S;
}
inline size_t page_bytes(Fmt f, int Hkv, int page_rows, int D) {
    return va_page_bytes(static_cast<va_fmt>(f), Hkv, page_rows, D);
}
inline size_t page_scale_bytes(Fmt f, int Hkv, int page_rows, int D, int G = 64) {
    return va_page_scale_bytes(static_cast<va_fmt>(f), Hkv, page_rows, D, G);
}

// The cache write path: quantize (or copy, f16 formats) n fp16 rows per
// (sequence, KV head) of x [B][Hkv][n][D] into the page pool at positions
// start[b] .. start[b] + n - 1.
inline void append_kv(Fmt f, const uint16_t* x, int n, const int32_t* start, const int32_t* block_table,
                      const PagedShape& shape, void* pages, uint16_t* scales, void* stream = nullptr) {
    check(va_append_kv(static_cast<va_fmt>(f), x, n, start, block_table, &shape, pages, scales, stream));
}

// Device quantize() of fp32 rows [rows][D] into packed codes and fp16 scales.
inline void quantize(int bits, int G, const float* x, size_t rows, int D, void* packed, uint16_t* scales,
                     void* stream = nullptr) {
    check(va_quantize(bits, G, x, rows, D, packed, scales, stream));
}

// Device dq() of packed codes + fp16 scales back to fp32 rows [rows][D].
inline void dequantize(int bits, int G, const void* packed, const uint16_t* scales, size_t rows, int D,
                       float* out, void* stream = nullptr) {
    check(va_dequantize(bits, G, packed, scales, rows, D, out, stream));
}

// RAII device allocation.
class DeviceBuffer {
public:
    DeviceBuffer() = default;
    explicit DeviceBuffer(size_t bytes) : bytes_(bytes) { check(va_malloc(&p_, bytes)); }
    ~DeviceBuffer() { if (p_) (void)va_free(p_); }
    DeviceBuffer(DeviceBuffer&& o) noexcept : p_(std::exchange(o.p_, nullptr)), bytes_(o.bytes_) {}
    DeviceBuffer& operator=(DeviceBuffer&& o) noexcept {
        if (this != &o) {
            if (p_) (void)va_free(p_);
            p_ = std::exchange(o.p_, nullptr);
            bytes_ = o.bytes_;
        }
        return *this;
    }
    DeviceBuffer(const DeviceBuffer&) = delete;
    DeviceBuffer& operator=(const DeviceBuffer&) = delete;

    void* get() const { return p_; }
    template <class T> T* as() const { return static_cast<T*>(p_); }
    size_t bytes() const { return bytes_; }
    void upload(const void* src, size_t n) { check(va_memcpy_h2d(p_, src, n)); }
    void download(void* dst, size_t n) const { check(va_memcpy_d2h(dst, p_, n)); }

private:
    void*  p_ = nullptr;
    size_t bytes_ = 0;
};

class Event {
public:
    Event() { check(va_event_create(&e_)); }
    ~Event() { if (e_) (void)va_event_destroy(e_); }
    Event(const Event&) = delete;
    Event& operator=(const Event&) = delete;
    void record(void* stream = nullptr) { check(va_event_record(e_, stream)); }
    void sync() { check(va_event_sync(e_)); }
    float ms_since(const Event& start) const {
        float ms = 0.f;
        check(va_event_elapsed_ms(start.e_, e_, &ms));
        return ms;
    }
private:
    void* e_ = nullptr;
};

// RAII stream at the default priority.
class Stream {
public:
    Stream() { check(va_stream_create(&s_)); }
    ~Stream() { if (s_) (void)va_stream_destroy(s_); }
    Stream(const Stream&) = delete;
    Stream& operator=(const Stream&) = delete;
    void* get() const { return s_; }
    void sync() { check(va_stream_sync(s_)); }
private:
    void* s_ = nullptr;
};

// A captured launch sequence, replayed with launch(): begin(stream), the
// launches on that stream, end().
class Graph {
public:
    Graph() = default;
    ~Graph() { if (g_) (void)va_graph_destroy(g_); }
    Graph(const Graph&) = delete;
    Graph& operator=(const Graph&) = delete;
    void begin(void* stream) { check(va_graph_begin(stream)); s_ = stream; }
    void end() {
        if (g_) { (void)va_graph_destroy(g_); g_ = nullptr; }
        check(va_graph_end(s_, &g_));
    }
    void launch(void* stream) const { check(va_graph_launch(g_, stream)); }
private:
    void* g_ = nullptr;
    void* s_ = nullptr;
};

} // namespace voltattn
