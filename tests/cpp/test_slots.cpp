// CPU test of the fused merge's ticket-slot binding (voltattn_amd/csrc/va_slots.hpp):
// built with g++ and run by tests/test_slots.py. Prints "slots: ok" on success.
#include "va_slots.hpp"

#include <atomic>
#include <cstdio>
#include <cstdlib>
#include <set>
#include <thread>
#include <vector>

#define CHECK(c)                                                          \
    do {                                                                  \
        if (!(c)) {                                                       \
            std::fprintf(stderr, "%s:%d: check failed: %s\n", __FILE__, __LINE__, #c); \
            std::exit(1);                                                 \
        }                                                                 \
    } while (0)

int main() {
    constexpr int N = 16;
    {
        va::SlotTable<N, 4> t;
        // one slot per eager stream, stable across calls
        const int a = t.acquire(0, 0x1000, 0), b = t.acquire(0, 0x2000, 0);
        CHECK(a >= 0 && b >= 0 && a != b);
        CHECK(t.acquire(0, 0x1000, 0) == a && t.acquire(0, 0x2000, 0) == b);
        // the default stream (handle 0) is a stream like any other
        const int d = t.acquire(0, 0, 0);
        CHECK(d >= 0 && d != a && d != b);
        // a capture on stream 0x1000 gets its own slot, distinct from the stream's eager one;
        // calls inside one capture share it; another capture of the same stream gets another
        const int c1 = t.acquire(0, 0x1000, 0x8000000000000001ull);
        const int c2 = t.acquire(0, 0x1000, 0x8000000000000002ull);
        CHECK(c1 >= 0 && c2 >= 0 && c1 != c2 && c1 != a && c2 != a && c1 != b && c1 != d);
        CHECK(t.acquire(0, 0x1000, 0x8000000000000001ull) == c1);
        // two streams captured in one sequence get separate slots
        const int c3 = t.acquire(0, 0x3000, 0x8000000000000001ull);
        CHECK(c3 >= 0 && c3 != c1);
        // devices are independent
        CHECK(t.acquire(1, 0x1000, 0) >= 0 && t.bound(1) == 1);
        CHECK(t.acquire(4, 0x1000, 0) == -1 && t.acquire(-1, 0x1000, 0) == -1);
        // exhaustion: no slot is handed out twice; the 17th binding gets -1
        std::set<int> seen = {a, b, d, c1, c2, c3};
        for (uintptr_t s = 0x10000; seen.size() < (size_t)N; s += 0x100) {
            const int x = t.acquire(0, s, 0);
            CHECK(x >= 0 && !seen.count(x));
            seen.insert(x);
        }
        CHECK(t.bound(0) == N);
        CHECK(t.acquire(0, 0xDEAD00, 0) == -1);
        CHECK(t.acquire(0, 0x1000, 0x8000000000000009ull) == -1);
        // existing bindings keep working after exhaustion
        CHECK(t.acquire(0, 0x2000, 0) == b && t.acquire(0, 0x1000, 0x8000000000000002ull) == c2);
    }
    {
        // release: a released slot is handed out again; releasing a capture drops all its streams
        va::SlotTable<N, 2> t;
        const int a = t.acquire(0, 0x1000, 0);
        const int c = t.acquire(0, 0x1000, 0x8000000000000005ull);
        const int c2 = t.acquire(1, 0x2000, 0x8000000000000005ull);
        CHECK(a >= 0 && c >= 0 && c2 >= 0 && t.bound(0) == 2 && t.bound(1) == 1);
        t.release(0, 0x1000, 0);
        CHECK(t.bound(0) == 1 && t.acquire(0, 0x1000, 0x8000000000000005ull) == c);
        t.release_capture(0x8000000000000005ull);
        CHECK(t.bound(0) == 0 && t.bound(1) == 0);
        t.release(0, 0x9999, 0);                          // unknown binding: no effect
        for (uintptr_t s = 1; s <= (uintptr_t)N; ++s) CHECK(t.acquire(0, s, 0) >= 0);
        CHECK(t.acquire(0, 0x777, 0) == -1);
        t.release(0, 5, 0);
        CHECK(t.acquire(0, 0x777, 0) >= 0);               // the freed slot is reused
    }
    {
        // concurrent first calls from many threads: every stream gets a distinct slot
        va::SlotTable<N, 2> t;
        std::vector<int> got(N, -2);
        std::vector<std::thread> th;
        for (int i = 0; i < N; ++i)
            th.emplace_back([&, i] {
                for (int r = 0; r < 1000; ++r) {
                    const int x = t.acquire(0, 0x100 * (uintptr_t)(i + 1), 0);
                    if (got[i] == -2) got[i] = x;
                    CHECK(x == got[i]);
                }
            });
        for (auto& x : th) x.join();
        std::set<int> s(got.begin(), got.end());
        CHECK(s.size() == (size_t)N && !s.count(-1));
    }
    {
        // leases: acquire() marks a binding pending until done(); a take-over needs
        // an eager caller, an eager owner the predicate calls idle, and no pending call
        va::SlotTable<2, 1> t;
        const uintptr_t A = 0x1000, B = 0x2000, C = 0x3000, P = 0x4000;
        const unsigned long long cap = 0x8000000000000007ull;
        auto idle_all = [](uintptr_t) { return true; };
        auto idle_none = [](uintptr_t) { return false; };
        const int a = t.acquire(0, A, 0, idle_all);       // pending
        const int b = t.acquire(0, B, 0, idle_all);       // pending
        CHECK(a >= 0 && b >= 0 && a != b);
        CHECK(t.acquire(0, C, 0, idle_all) == -1);        // both pending: no take-over
        t.done(0, a, A, 0);
        CHECK(t.acquire(0, C, 0, idle_none) == -1);       // A not idle
        const int c = t.acquire(0, C, 0, idle_all);       // A idle, nothing pending: C takes A's slot
        CHECK(c == a && t.find(0, A, 0) == -1 && t.find(0, C, 0) == a);
        CHECK(t.acquire(0, A, 0, idle_all) == -1);        // B and C pending
        t.done(0, b, B, 0);
        t.done(0, c, C, 0);
        // a capturing caller may take over an idle eager binding; a capture's
        // binding is never taken over
        CHECK(t.acquire(0, P, cap, idle_none) == -1);
        const int p = t.acquire(0, P, cap, [&](uintptr_t s) { return s == B; });
        CHECK(p == b && t.find(0, B, 0) == -1 && t.find(0, P, cap) == b);
        t.done(0, p, P, cap);
        int asked = 0;
        CHECK(t.acquire(0, A, 0, [&](uintptr_t s) { ++asked; return s == C; }) == c);   // C idle
        CHECK(asked == 1);                                // the capture binding is not even asked about
        t.done(0, c, A, 0);
        // done() from a call that does not own the binding changes nothing
        const int again = t.acquire(0, A, 0, idle_none);  // pending 1
        t.done(0, again, C, 0);                           // not the owner
        CHECK(t.acquire(0, C, 0, idle_all) == -1);        // A still pending
        t.done(0, again, A, 0);
        // call counters belong to the slot: they survive release and rebinding
        CHECK(t.count(0, p) == 1 && t.count(0, p) == 2);
        int got_d = -1, got_s = -1;
        t.release_capture(cap, [&](int d, int s) { got_d = d; got_s = s; });
        CHECK(got_d == 0 && got_s == p && t.bound(0) == 1);
        const int p2 = t.acquire(0, P, 0, idle_none);
        CHECK(p2 == p && t.count(0, p2) == 3);
        t.reset_count(0, p2);
        CHECK(t.count(0, p2) == 1);
    }
    {
        // concurrent take-overs: 8 threads on 8 streams share 2 slots, each stream
        // is idle whenever it has no call in progress; no two calls ever hold one
        // slot at the same time
        va::SlotTable<2, 1> t;
        std::atomic<int> holder[2];
        holder[0] = holder[1] = -1;
        std::atomic<bool> busy[8];
        for (auto& x : busy) x = false;
        std::atomic<int> granted{0};
        std::vector<std::thread> th;
        for (int i = 0; i < 8; ++i)
            th.emplace_back([&, i] {
                const uintptr_t s = 0x100 * (uintptr_t)(i + 1);
                for (int r = 0; r < 2000; ++r) {
                    busy[i] = true;
                    const int x = t.acquire(0, s, 0, [&](uintptr_t o) { return !busy[o / 0x100 - 1]; });
                    if (x >= 0) {
                        int expect = -1;
                        CHECK(holder[x].compare_exchange_strong(expect, i));
                        holder[x] = -1;
                        ++granted;
                        t.done(0, x, s, 0);
                    }
                    busy[i] = false;
                }
            });
        for (auto& x : th) x.join();
        CHECK(granted > 0);
    }
    std::printf("slots: ok\n");
    return 0;
}
