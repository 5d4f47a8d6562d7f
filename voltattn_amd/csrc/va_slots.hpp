// va_slots.hpp — assignment of library device state that must not be shared by
// work that may overlap: the fused merge's ticket slots (counters and partial
// store in static device memory) and the allocation-free entry point's
// workspace. Host-only C++ (no HIP types), so the logic is exercised on the CPU
// by tests/cpp/test_slots.cpp.
//
// A decode call that merges inside its kernel owns one ticket slot for the
// duration of the kernel. Kernels on one stream run one after another, so every
// call issued on the same stream may use the same slot; calls on different
// streams may overlap and must not share one. A slot is therefore bound to an
// owner the first time the owner calls, and kept:
//
//   * an eager stream (not capturing) is an owner;
//   * a stream capturing a graph is an owner per capture sequence: the graph's
//     replays keep using its slot (every launch of one executable graph is
//     ordered behind the previous launch of the same graph), and no eager
//     stream or other graph ever shares it;
//   * once every slot of the device is bound, a caller may take over a binding
//     of an eager stream that is idle (its work has completed, as the
//     caller's `idle` predicate reports) and has no call between acquire()
//     and done(); otherwise acquire() returns -1 and the caller falls back to
//     what shares no library state (the two-pass form).
//
// acquire() marks the binding pending until the caller has enqueued its launch
// and calls done(): a take-over never happens between the two, so a stream
// that was idle when asked cannot receive a launch on a slot that has just been
// handed to another stream. Bindings of capture sequences are never taken
// over (their replays may come at any time); release() and release_capture()
// drop bindings explicitly (the library's stream and graph destructors, and
// its release entry points, call them after waiting for the owner's work).
// A stream handle that is destroyed and reused by a new stream keeps the old
// binding, which is safe as long as the new stream's first call is ordered
// after the old stream's last one.
#pragma once
#include <stdint.h>

#include <mutex>

namespace va {

template <int SLOTS, int DEVICES = 64>
class SlotTable {
public:
    // Slot of (device, stream) outside capture (capture == 0) or inside the
    // capture sequence `capture` (non-zero id), marked pending; -1 when none
    // is free or can be taken over, or the device index is out of range.
    // idle(stream) is asked, under the table's lock, only for eager owners of
    // other bindings and only when no slot is free.
    template <class Idle>
    int acquire(int device, uintptr_t stream, unsigned long long capture, Idle&& idle) {
        if (device < 0 || device >= DEVICES) return -1;
        std::lock_guard<std::mutex> lock(mu_);
        Entry* e = e_[device];
        for (int i = 0; i < SLOTS; ++i)
            if (e[i].used && e[i].stream == stream && e[i].capture == capture) return take(e[i], i);
        for (int i = 0; i < SLOTS; ++i)
            if (!e[i].used) return bind(e[i], i, stream, capture);
        for (int i = 0; i < SLOTS; ++i)
            if (e[i].capture == 0 && e[i].pending == 0 && idle(e[i].stream))
                return bind(e[i], i, stream, capture);
        return -1;
    }
    int acquire(int device, uintptr_t stream, unsigned long long capture) {
        return acquire(device, stream, capture, [](uintptr_t) { return false; });
    }

    // The call of (stream, capture) that acquired `slot` has enqueued its
    // work (or given up).
    void done(int device, int slot, uintptr_t stream, unsigned long long capture) {
        if (device < 0 || device >= DEVICES || slot < 0 || slot >= SLOTS) return;
        std::lock_guard<std::mutex> lock(mu_);
        Entry& x = e_[device][slot];
        if (x.used && x.stream == stream && x.capture == capture && x.pending > 0) --x.pending;
    }

    // Slot bound to (device, stream, capture), or -1; binds nothing.
    int find(int device, uintptr_t stream, unsigned long long capture) {
        if (device < 0 || device >= DEVICES) return -1;
        std::lock_guard<std::mutex> lock(mu_);
        for (int i = 0; i < SLOTS; ++i) {
            const Entry& x = e_[device][i];
            if (x.used && x.stream == stream && x.capture == capture) return i;
        }
        return -1;
    }

    // Drop the binding of (device, stream, capture) if there is one; returns
    // its slot or -1.
    int release(int device, uintptr_t stream, unsigned long long capture) {
        if (device < 0 || device >= DEVICES) return -1;
        std::lock_guard<std::mutex> lock(mu_);
        for (int i = 0; i < SLOTS; ++i) {
            Entry& x = e_[device][i];
            if (x.used && x.stream == stream && x.capture == capture) {
                drop(x);
                return i;
            }
        }
        return -1;
    }

    // Drop every binding of a capture sequence (all its streams, any device);
    // dropped(device, slot) is called for each, under the table's lock.
    template <class Dropped>
    void release_capture(unsigned long long capture, Dropped&& dropped) {
        if (capture == 0) return;
        std::lock_guard<std::mutex> lock(mu_);
        for (int d = 0; d < DEVICES; ++d)
            for (int i = 0; i < SLOTS; ++i)
                if (e_[d][i].used && e_[d][i].capture == capture) {
                    drop(e_[d][i]);
                    dropped(d, i);
                }
    }
    void release_capture(unsigned long long capture) {
        release_capture(capture, [](int, int) {});
    }

    // Bound slots of a device (for tests and diagnostics).
    int bound(int device) {
        if (device < 0 || device >= DEVICES) return 0;
        std::lock_guard<std::mutex> lock(mu_);
        int n = 0;
        for (int i = 0; i < SLOTS; ++i) n += e_[device][i].used ? 1 : 0;
        return n;
    }

    // Calls counted on a binding since its counter was last reset (count()
    // adds one and returns the new value; reset_count() starts over).
    unsigned long long count(int device, int slot) {
        if (device < 0 || device >= DEVICES || slot < 0 || slot >= SLOTS) return 0;
        std::lock_guard<std::mutex> lock(mu_);
        return ++e_[device][slot].calls;
    }
    void reset_count(int device, int slot) {
        if (device < 0 || device >= DEVICES || slot < 0 || slot >= SLOTS) return;
        std::lock_guard<std::mutex> lock(mu_);
        e_[device][slot].calls = 0;
    }

private:
    struct Entry {
        uintptr_t stream = 0;
        unsigned long long capture = 0;
        unsigned long long calls = 0;   // survives a take-over: it counts the slot's device state
        int pending = 0;
        bool used = false;
    };
    static int take(Entry& x, int i) {
        ++x.pending;
        return i;
    }
    static void drop(Entry& x) {
        const unsigned long long calls = x.calls;
        x = Entry{};
        x.calls = calls;
    }
    static int bind(Entry& x, int i, uintptr_t stream, unsigned long long capture) {
        drop(x);
        x.used = true;
        x.stream = stream;
        x.capture = capture;
        x.pending = 1;
        return i;
    }
    std::mutex mu_;
    Entry e_[DEVICES][SLOTS];
};

} // namespace va
