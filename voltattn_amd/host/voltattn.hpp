// voltattn.hpp — C++ host mirror of kamilch1k/voltattn's interface over the
// C ABI (include/voltattn.h). Header-only; link libvoltattn_hip.so.
//
//   voltattn::Fmt         enum class Fmt {F16, F16M, Q8, Q8M, Q4, Q4M, Q3M}  (src/voltattn.cu:676)
//   voltattn::DeviceBufs  struct DeviceBufs {K, V, scK, scV, q, out, ws}      (src/voltattn.cu:796-801)
//   voltattn::launch      launch(f, b, H, L, D, S) (+ group size G)           (src/voltattn.cu:803-835)
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

} // namespace voltattn
