// va_slots.hpp — assignment of the fused merge's ticket slots to streams.
// Host-only C++ (no HIP types), so the logic is exercised on the CPU by
// tests/cpp/test_slots.cpp.
//
// A decode call that merges inside its kernel owns one ticket slot (counters
// and partial store in static device memory) for the duration of the kernel.
// Kernels on one stream run one after another, so every call issued on the
// same stream may use the same slot; calls on different streams may overlap
// and must not share one. A slot is therefore bound to a stream the first time
// the stream calls, and kept:
//
//   * an eager stream (not capturing) gets its own slot;
//   * a stream capturing a graph gets a slot of its own per capture sequence:
//     the graph's replays keep using it (every launch of one executable graph
//     is ordered behind the previous launch of the same graph), and no eager
//     stream or other graph ever shares it;
//   * once every slot of the device is bound, acquire() returns -1 and the call
//     uses the two-pass form (partials in the caller's ws, separate merge
//     kernel), which shares no library state.
//
// A binding lasts until release(): the library's own stream and graph
// destructors (va_stream_destroy, va_graph_destroy) first wait for the work
// that may use the slot, then release it. Streams created elsewhere (torch's,
// hipStreamCreate) keep their slot for the life of the process; such a handle
// that is destroyed and reused by a new stream keeps the slot too, which is
// safe as long as the new stream's first call is ordered after the old
// stream's last one.
#pragma once
#include <stdint.h>

#include <mutex>

namespace va {

template <int SLOTS, int DEVICES = 64>
class SlotTable {
public:
    // Slot of (device, stream) outside capture (capture == 0) or inside the
    // capture sequence `capture` (non-zero id); -1 when none is free or the
    // device index is out of range.
    int acquire(int device, uintptr_t stream, unsigned long long capture) {
        if (device < 0 || device >= DEVICES) return -1;
        std::lock_guard<std::mutex> lock(mu_);
        Entry* e = e_[device];
        for (int i = 0; i < SLOTS; ++i)
            if (e[i].used && e[i].stream == stream && e[i].capture == capture) return i;
        for (int i = 0; i < SLOTS; ++i) {
            if (!e[i].used) {
                e[i].used = true;
                e[i].stream = stream;
                e[i].capture = capture;
                return i;
            }
        }
        return -1;
    }

    // Drop the binding of (device, stream, capture) if there is one.
    void release(int device, uintptr_t stream, unsigned long long capture) {
        if (device < 0 || device >= DEVICES) return;
        std::lock_guard<std::mutex> lock(mu_);
        for (int i = 0; i < SLOTS; ++i) {
            Entry& x = e_[device][i];
            if (x.used && x.stream == stream && x.capture == capture) x = Entry{};
        }
    }

    // Drop every binding of a capture sequence (all its streams, any device).
    void release_capture(unsigned long long capture) {
        if (capture == 0) return;
        std::lock_guard<std::mutex> lock(mu_);
        for (int d = 0; d < DEVICES; ++d)
            for (int i = 0; i < SLOTS; ++i)
                if (e_[d][i].used && e_[d][i].capture == capture) e_[d][i] = Entry{};
    }

    // Bound slots of a device (for tests and diagnostics).
    int bound(int device) {
        if (device < 0 || device >= DEVICES) return 0;
        std::lock_guard<std::mutex> lock(mu_);
        int n = 0;
        for (int i = 0; i < SLOTS; ++i) n += e_[device][i].used ? 1 : 0;
        return n;
    }

private:
    struct Entry {
        uintptr_t stream = 0;
        unsigned long long capture = 0;
        bool used = false;
    };
    std::mutex mu_;
    Entry e_[DEVICES][SLOTS];
};

} // namespace va
