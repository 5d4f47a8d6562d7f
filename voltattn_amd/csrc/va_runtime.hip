// va_runtime.hip — the C ABI (include/voltattn.h): argument validation,
// format -> kernel dispatch, ticket-slot binding, and the thin HIP runtime
// shims the host harness uses. Apart from the kernel launches and the two
// lost-merge counter reads (va_fused.hpp), this is the only translation unit
// that calls the HIP runtime API.
#include "voltattn.h"
#include "va_kernels.hpp"
#include "va_slots.hpp"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <unordered_map>
#include <vector>

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return code;
}

int hip_fail(hipError_t e, const char* what) {
    return fail(VA_EHIP, "%s: %s (%s)", what, hipGetErrorName(e), hipGetErrorString(e));
}

#define VA_HIP(call, what)                               \
    do {                                                 \
        const hipError_t e_ = (call);                    \
        if (e_ != hipSuccess) return hip_fail(e_, what); \
    } while (0)

hipStream_t as_stream(void* s) { return static_cast<hipStream_t>(s); }

bool valid_fmt(int f) { return f >= VA_F16 && f <= VA_Q3P; }
bool is_f16(va_fmt f) { return f == VA_F16 || f == VA_F16P; }
int  kind_of(va_fmt f) {
    switch (f) {
        case VA_F16: case VA_F16P: return 0;
        case VA_Q8:  case VA_Q8P:  return 1;
        case VA_Q4:  case VA_Q4P:  return 2;
        default:                   return 3;
    }
}
bool tiled_of(va_fmt f) { return f == VA_F16P || f == VA_Q8P || f == VA_Q4P || f == VA_Q3P; }
int  bits_of(va_fmt f) { static const int b[] = {16, 16, 8, 8, 4, 4, 3}; return b[f]; }
size_t row_bytes(va_fmt f, int D) { return (size_t)D * bits_of(f) / 8; }

bool aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

int validate(va_fmt fmt, const va_bufs* b, int H, int L, int D, int G, int S, bool need_out,
             bool need_ws = true) {
    if (!valid_fmt(fmt)) return fail(VA_EINVAL, "invalid format %d", (int)fmt);
    if (!b) return fail(VA_ENULL, "bufs is NULL");
    if (D != 64 && D != 128) return fail(VA_EINVAL, "D must be 64 or 128 (got %d)", D);
    const bool quant = !is_f16(fmt);
    if (quant && !((G == 32 || G == 64) && G <= D))
        return fail(VA_EINVAL, "G must be 32 or 64 and <= D (got G=%d, D=%d)", G, D);
    if (H < 1) return fail(VA_EINVAL, "H must be >= 1 (got %d)", H);
    if (L < 1) return fail(VA_EINVAL, "L must be >= 1 (got %d)", L);
    if (S < 1) return fail(VA_EINVAL, "S must be >= 1 (got %d)", S);
    if ((long long)H * S > 0x7FFFFFFFLL) return fail(VA_ERANGE, "H*S too large");
    if (((size_t)L + 256) * row_bytes(fmt, D) >= 0x7FFFFFFFull)
        return fail(VA_ERANGE, "L*row bytes must stay below 2^31 (L=%d)", L);
    if (!b->k || !b->v || !b->q) return fail(VA_ENULL, "k, v and q must be non-NULL");
    if (need_ws && !b->ws) return fail(VA_ENULL, "ws must be non-NULL");
    if (need_out && !b->out) return fail(VA_ENULL, "out must be non-NULL");
    if (quant && (!b->sk || !b->sv)) return fail(VA_ENULL, "quantized formats need sk and sv");
    const size_t kal = kind_of(fmt) == 3 ? 4 : 16;
    if (!aligned(b->k, kal) || !aligned(b->v, kal))
        return fail(VA_EALIGN, "k and v must be %zu-byte aligned", kal);
    if (!aligned(b->q, 16)) return fail(VA_EALIGN, "q must be 16-byte aligned");
    if (need_ws && !aligned(b->ws, 4)) return fail(VA_EALIGN, "ws must be 4-byte aligned");
    if (need_out && !aligned(b->out, 2)) return fail(VA_EALIGN, "out must be 2-byte aligned");
    if (quant) {
        const size_t sal = (D / G) >= 2 ? 4 : 2;
        if (!aligned(b->sk, sal) || !aligned(b->sv, sal))
            return fail(VA_EALIGN, "sk and sv must be %zu-byte aligned", sal);
    }
    return VA_OK;
}

va::SlotTable<va::TICKET_SLOTS> g_slots;
// Owner of the allocation-free entry point's workspace on each device.
va::SlotTable<1> g_scratch_owner;
// Capture sequence of each graph made by va_graph_end (its slots are released
// by va_graph_destroy).
std::mutex g_graph_mu;
std::unordered_map<void*, unsigned long long> g_graph_capture;

// Owner key of `stream` for the calling thread: the handle, except for the
// per-thread default stream (hipStreamPerThread), one handle that names a
// different stream on each host thread, whose key is an odd address private
// to the thread (never a stream handle, which is aligned).
thread_local char g_thread_tag;
uintptr_t owner_key(void* stream) {
    if (as_stream(stream) == hipStreamPerThread) return reinterpret_cast<uintptr_t>(&g_thread_tag) | 1u;
    return reinterpret_cast<uintptr_t>(stream);
}

// Capture sequence of `stream` (0: not capturing); false if HIP cannot tell.
bool capture_of(void* stream, unsigned long long* capture) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    unsigned long long id = 0;
    if (hipStreamGetCaptureInfo(as_stream(stream), &cs, &id) != hipSuccess) return false;
    *capture = cs == hipStreamCaptureStatusActive ? (id | (1ull << 63)) : 0ull;
    return true;
}

// Whether an eager owner's stream has completed all its work, asked when a
// binding is to be taken over. Per-thread keys are never asked about (another
// thread's per-thread stream cannot be named). The query runs in relaxed
// capture mode, and never on a stream that is capturing, so it cannot
// disturb a capture in progress on this or another thread.
bool owner_idle(uintptr_t key) {
    if (key & 1u) return false;
    const hipStream_t st = reinterpret_cast<hipStream_t>(key);
    hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
    if (hipThreadExchangeStreamCaptureMode(&mode) != hipSuccess) return false;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusActive;
    const bool idle = hipStreamIsCapturing(st, &cs) == hipSuccess && cs == hipStreamCaptureStatusNone &&
                      hipStreamQuery(st) == hipSuccess;
    (void)hipThreadExchangeStreamCaptureMode(&mode);
    return idle;
}

// Zero one ticket slot's tagged partials in both code objects, on `stream`.
hipError_t clear_slot(int slot, hipStream_t stream) {
    hipError_t e = va::clear_tagged_decode(slot, stream);
    if (e == hipSuccess) e = va::clear_tagged_ex(slot, stream);
    return e;
}

// A binding held by one call: the slot (or -1) and its owner; done() once the
// call's work is enqueued (va_slots.hpp).
struct Lease {
    int dev = 0;
    int slot = -1;
    uintptr_t key = 0;
    unsigned long long capture = 0;
};

// Ticket slot of a fused call on `stream` (va_slots.hpp: one per eager stream,
// one per stream and capture sequence while capturing; an idle eager stream's
// slot may be taken over), or slot -1: the call runs the two-pass form. The
// per-thread default stream always runs the two-pass form.
//
// Stale tagged partials (va_kernels.hpp, TAG_EPOCH_BITS): every eager call is
// counted against its slot, and after SLOT_CLEAR_CALLS of them the slot's
// store is cleared on `stream` ahead of the call, so a word left by an eager
// call is gone before any merge group's epoch has advanced 2^TAG_EPOCH_BITS
// past it. Replays of a captured graph are not seen here: a capture's slot is
// cleared when its binding is released (release_capture_all), before any
// other owner can use it.
Lease ticket_slot_for(void* stream) {
    Lease l;
    if (as_stream(stream) == hipStreamPerThread) return l;
    if (hipGetDevice(&l.dev) != hipSuccess || !capture_of(stream, &l.capture)) return l;
    l.key = owner_key(stream);
    l.slot = g_slots.acquire(l.dev, l.key, l.capture, owner_idle);
    if (l.slot >= 0 && l.capture == 0 && g_slots.count(l.dev, l.slot) >= va::SLOT_CLEAR_CALLS) {
        if (clear_slot(l.slot, as_stream(stream)) != hipSuccess) {
            g_slots.done(l.dev, l.slot, l.key, l.capture);
            l.slot = -1;                          // two-pass form instead
            return l;
        }
        g_slots.reset_count(l.dev, l.slot);
    }
    return l;
}
void lease_done(const Lease& l) {
    if (l.slot >= 0) g_slots.done(l.dev, l.slot, l.key, l.capture);
}

// Drop (device, key, capture)'s ticket slot and workspace bindings once its
// work is done, clearing the slot's tagged partials on `stream` (synchronised
// here) so that its next owner starts from a clear store.
hipError_t release_owner(int dev, uintptr_t key, unsigned long long capture, hipStream_t stream) {
    hipError_t e = hipSuccess;
    const int slot = g_slots.find(dev, key, capture);
    if (slot >= 0) {
        e = clear_slot(slot, stream);
        if (e == hipSuccess) e = hipStreamSynchronize(stream);
        g_slots.release(dev, key, capture);
        g_slots.reset_count(dev, slot);
    }
    g_scratch_owner.release(dev, key, capture);
    return e;
}

// Drop every binding of a capture sequence; the device has finished all work
// (the caller synchronised it). The dropped slots are cleared on the null
// stream and waited for.
hipError_t release_capture_all(unsigned long long capture) {
    if (capture == 0) return hipSuccess;
    std::vector<std::pair<int, int>> dropped;
    g_slots.release_capture(capture, [&](int d, int slot) { dropped.emplace_back(d, slot); });
    g_scratch_owner.release_capture(capture);
    int cur = 0;
    hipError_t e = hipGetDevice(&cur);
    for (const auto& x : dropped) {
        if (e != hipSuccess) break;
        e = hipSetDevice(x.first);
        if (e == hipSuccess) e = clear_slot(x.second, nullptr);
        if (e == hipSuccess) e = hipDeviceSynchronize();
        g_slots.reset_count(x.first, x.second);
    }
    if (!dropped.empty()) (void)hipSetDevice(cur);
    return e;
}

// slot >= 0: merge inside the decode kernel on that ticket slot (the caller
// checked H <= TICKET_MAXH, S <= 64 and H*S <= PART_CAP); -1: the partials
// are left in ws for a separate merge pass.
int run_splits(va_fmt fmt, const va_bufs* b, int H, int L, int D, int G, int S, void* stream,
               int slot) {
    va::DecodeArgs a{};
    a.hkv = H;                    // the reference's shape: one query head per K/V head
    a.qgroup = 1;
    a.nsub = 1;
    a.k  = static_cast<const uint8_t*>(b->k);
    a.v  = static_cast<const uint8_t*>(b->v);
    a.sk = b->sk;
    a.sv = b->sv;
    a.q  = b->q;
    a.ws = b->ws;
    a.out = b->out;
    a.ticket_slot = slot;
    a.L = L;
    a.S = S;
    a.chunk  = (L + S - 1) / S;
    a.qscale = (float)(1.4426950408889634074 / std::sqrt((double)D));
    const hipError_t e = va::launch_decode(kind_of(fmt), tiled_of(fmt), H, D, is_f16(fmt) ? 64 : G,
                                           a, as_stream(stream));
    if (e != hipSuccess) return hip_fail(e, "decode launch");
    return VA_OK;
}

std::atomic<int> g_cu_count{0};

// CUs of the first device asked (the split rule assumes identical devices).
int cu_count() {
    const int c = g_cu_count.load(std::memory_order_relaxed);
    if (c > 0) return c;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    g_cu_count.store(n, std::memory_order_relaxed);
    return n;
}

} // namespace

extern "C" {

int va_abi_version(void) { return VA_ABI_VERSION; }

const char* va_last_error(void) { return g_err; }

const char* va_fmt_name(va_fmt fmt) {
    static const char* names[] = {"f16", "f16+", "q8", "q8+", "q4", "q4+", "q3+"};
    return valid_fmt(fmt) ? names[fmt] : "?";
}

size_t va_ws_bytes(int H, int D, int S) {
    if (H < 1 || D < 1 || S < 1) return 0;
    return (size_t)H * S * (D + 2) * sizeof(float);
}

size_t va_payload_bytes(va_fmt fmt, int H, int L, int D) {
    if (!valid_fmt(fmt) || H < 1 || L < 1 || D < 1) return 0;
    return (size_t)H * L * row_bytes(fmt, D);
}

size_t va_scale_bytes(va_fmt fmt, int H, int L, int D, int G) {
    if (!valid_fmt(fmt) || is_f16(fmt) || H < 1 || L < 1 || G < 1 || D % G) return 0;
    return (size_t)H * L * (D / G) * 2;
}

int va_split_chunk(int L, int S) { return (L < 1 || S < 1) ? 0 : (L + S - 1) / S; }

int va_pick_splits(va_fmt fmt, int H, int L, int D, int* S) {
    if (!S) return fail(VA_ENULL, "S is NULL");
    if (!valid_fmt(fmt) || H < 1 || L < 1 || (D != 64 && D != 128))
        return fail(VA_EINVAL, "invalid arguments to va_pick_splits");
    int cus = cu_count();
    if (cus <= 0) cus = 256;
    const int tb    = va::tile_positions(kind_of(fmt), tiled_of(fmt), D);
    const int tiles = (L + tb - 1) / tb;
    // Tiled kernels: the kind's configured groups per CU (one or two groups
    // stream a CU at full rate; more splits only lengthen the merge). Naive
    // kernels keep one position per wave in flight, so they need ~8 per CU.
    int per_cu = va::groups_per_cu(kind_of(fmt), tiled_of(fmt));
    // (q3 once took a second work-group per CU on long contexts, while its
    // kernel fit four waves per SIMD. The kernel now holds ~150 VGPRs, one
    // group per CU, and one split per CU measured faster on MI355X (H=32,
    // D=128): L=65536 46.2 -> 42.4 us, L=262144 157.6 -> 156.2 us.)
    const int target = std::max(1, (per_cu * cus + H - 1) / H);
    const int s0     = std::max(1, std::min(tiles, target));
    const int tps    = (tiles + s0 - 1) / s0;               // tiles per split
    *S = std::max(1, (L + tps * tb - 1) / (tps * tb));
    return VA_OK;
}

int va_decode(va_fmt fmt, const va_bufs* b, int H, int L, int D, int G, int S, void* stream) {
    int rc = validate(fmt, b, H, L, D, G, S, true);
    if (rc) return rc;
    const bool fits = H <= va::TICKET_MAXH && S <= 64 && (long long)H * S <= va::PART_CAP;
    const Lease lease = fits ? ticket_slot_for(stream) : Lease{};
    rc = run_splits(fmt, b, H, L, D, G, S, stream, lease.slot);
    lease_done(lease);
    if (rc || lease.slot >= 0) return rc;
    const hipError_t e = va::launch_merge(b->ws, b->out, H, D, S, as_stream(stream));
    if (e != hipSuccess) return hip_fail(e, "merge launch");
    return VA_OK;
}

} // extern "C"

// ------------------------------------------------ allocation-free decode --
// Workspace of va_decode_noalloc: the two-pass form's partials (H*S*(D+2)
// floats) live in this file-scope device array instead of a caller-provided
// ws. Each device holds its own copy for the life of the process. Host code
// never uses the array's name as an address: the per-device address comes
// from hipGetSymbolAddress on the device's first call.
namespace {

constexpr size_t SCRATCH_FLOATS = VA_NOALLOC_MAX_FLOATS;   // 4 MiB: H*S*(D+2) <= 1,048,576
static __device__ __align__(256) float scratch[SCRATCH_FLOATS];

constexpr int SCRATCH_DEVICES = 64;
float* g_scratch_ptr[SCRATCH_DEVICES];
std::mutex g_scratch_mu;

// This device's address of `scratch` (looked up once per device, with the
// device current), or nullptr with the failure recorded.
float* scratch_ptr(int* rc) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) { *rc = hip_fail(e, "hipGetDevice"); return nullptr; }
    if (dev < 0 || dev >= SCRATCH_DEVICES) { *rc = fail(VA_ENODEV, "device index %d out of range", dev); return nullptr; }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) { *rc = hip_fail(e, "hipGetSymbolAddress(scratch)"); return nullptr; }
        g_scratch_ptr[dev] = static_cast<float*>(p);
    }
    return g_scratch_ptr[dev];
}

} // namespace

extern "C" {

int va_decode_noalloc(va_fmt fmt, const va_bufs* b, int H, int L, int D, int G, int S, void* stream) {
    if (!b) return fail(VA_ENULL, "bufs is NULL");
    if (H >= 1 && S >= 1 && (D == 64 || D == 128) &&
        (unsigned long long)H * S * (D + 2) > SCRATCH_FLOATS)
        return fail(VA_ERANGE, "H*S*(D+2) = %llu floats exceeds the allocation-free workspace (%zu floats)",
                    (unsigned long long)H * S * (D + 2), SCRATCH_FLOATS);
    int rc = validate(fmt, b, H, L, D, G, S, true, false);
    if (rc) return rc;
    va_bufs nb = *b;
    nb.ws = scratch_ptr(&rc);
    if (!nb.ws) return rc;
    const bool fits = H <= va::TICKET_MAXH && S <= 64 && (long long)H * S <= va::PART_CAP;
    const Lease lease = fits ? ticket_slot_for(stream) : Lease{};
    if (lease.slot >= 0) {                       // fused merge: the workspace is not used
        rc = run_splits(fmt, &nb, H, L, D, G, S, stream, lease.slot);
        lease_done(lease);
        return rc;
    }
    // Two-pass form: the device's workspace is bound to one owner (stream, or
    // stream and capture sequence) at a time, taken over only from an idle
    // eager stream with no call in progress; any other owner is refused.
    Lease ws;
    if (hipGetDevice(&ws.dev) != hipSuccess || !capture_of(stream, &ws.capture))
        return fail(VA_EHIP, "cannot identify the calling stream");
    ws.key = owner_key(stream);
    ws.slot = g_scratch_owner.acquire(ws.dev, ws.key, ws.capture, owner_idle);
    if (ws.slot < 0)
        return fail(VA_EBUSY, "the allocation-free workspace of device %d is bound to another stream or graph "
                              "(va_stream_release / va_capture_release free it)", ws.dev);
    rc = run_splits(fmt, &nb, H, L, D, G, S, stream, -1);
    if (rc == VA_OK) {
        const hipError_t e = va::launch_merge(nb.ws, nb.out, H, D, S, as_stream(stream));
        if (e != hipSuccess) rc = hip_fail(e, "merge launch");
    }
    g_scratch_owner.done(ws.dev, ws.slot, ws.key, ws.capture);
    return rc;
}

int va_decode_splits(va_fmt fmt, const va_bufs* b, int H, int L, int D, int G, int S, void* stream) {
    const int rc = validate(fmt, b, H, L, D, G, S, false);
    if (rc) return rc;
    return run_splits(fmt, b, H, L, D, G, S, stream, -1);
}

int va_merge(const float* ws, uint16_t* out, int H, int D, int S, void* stream) {
    if (!ws || !out) return fail(VA_ENULL, "ws and out must be non-NULL");
    if (H < 1 || S < 1 || (D != 64 && D != 128)) return fail(VA_EINVAL, "invalid H/D/S");
    if (!aligned(ws, 4) || !aligned(out, 2)) return fail(VA_EALIGN, "ws/out misaligned");
    const hipError_t e = va::launch_merge(ws, out, H, D, S, as_stream(stream));
    if (e != hipSuccess) return hip_fail(e, "merge launch");
    return VA_OK;
}

// Fused merges that gave up waiting for a partial, per device, as last reported
// (the device counters only grow; the difference is what is new).
unsigned g_lost_seen[64];
std::mutex g_lost_mu;

int va_merge_faults(void* stream, unsigned* count) {
    if (!count) return fail(VA_ENULL, "count is NULL");
    *count = 0;
    int dev = 0;
    VA_HIP(hipGetDevice(&dev), "hipGetDevice");
    if (dev < 0 || dev >= 64) return fail(VA_ENODEV, "device index %d out of range", dev);
    VA_HIP(hipStreamSynchronize(as_stream(stream)), "hipStreamSynchronize");
    unsigned n1 = 0, n2 = 0;
    VA_HIP(va::lost_merges_decode(&n1), "lost-merge counter");
    VA_HIP(va::lost_merges_ex(&n2), "lost-merge counter");
    std::lock_guard<std::mutex> lock(g_lost_mu);
    const unsigned total = n1 + n2;
    *count = total - g_lost_seen[dev];
    g_lost_seen[dev] = total;
    if (*count)
        return fail(VA_ELOST, "%u fused merge(s) gave up waiting for a partial (their outputs are NaN)", *count);
    return VA_OK;
}

} // extern "C"

// ------------------------------------------ grouped-query / paged decode --
namespace {

bool pow2(int x) { return x > 0 && (x & (x - 1)) == 0; }
int  log2i(int x) { int s = 0; while ((1 << s) < x) ++s; return s; }

// Query slots per work-group (QG, a power of two) and sub-groups per KV head:
// as few sub-groups as the kind's slot limit allows (each re-reads the rows),
// then the smallest QG that covers the group.
void pick_qg(int kind, int D, int qgroup, int* qg, int* nsub) {
    const int qmax = va::max_query_slots(kind, D);
    const int ns = (qgroup + qmax - 1) / qmax;
    const int per = (qgroup + ns - 1) / ns;
    int q = 1;
    while (q < per) q <<= 1;
    *qg = q;
    *nsub = ns;
}

// Split count and split length for `groups` merge groups over sequences of up
// to max_len positions: the kernel's work-groups per CU (one or two 4-wave
// groups), splits of whole kernel tiles, at most 64 splits (the fused merge's
// limit). S_req > 0 fixes S.
void splits_ex(int kind, int D, int qg, int groups, int max_len, int S_req, int* S, int* chunk) {
    int cus = cu_count();
    if (cus <= 0) cus = 256;
    cus *= va::ex_groups_per_cu(kind, D, qg);
    const int tb = va::tile_positions_ex(kind, D);
    const int tiles = std::max(1, (max_len + tb - 1) / tb);
    int s0 = S_req;
    if (s0 <= 0) s0 = std::max(1, std::min(std::min(tiles, 64), (cus + groups - 1) / groups));
    const int tps = (tiles + s0 - 1) / s0;
    *chunk = tps * tb;
    *S = S_req > 0 ? S_req : std::max(1, (max_len + *chunk - 1) / *chunk);
}

bool fused_ok(int groups, int qg, int S) {
    return S <= 64 && groups <= va::TICKET_MAXH && (long long)groups * qg * S <= va::PART_CAP;
}

int launch_ex(va_fmt fmt, va::DecodeArgs& a, int D, int G, int qg, bool paged, int groups,
              int heads_total, void* stream) {
    const Lease lease = fused_ok(groups, qg, a.S) ? ticket_slot_for(stream) : Lease{};
    a.ticket_slot = lease.slot;
    const bool fused = a.ticket_slot >= 0;
    a.qscale = (float)(1.4426950408889634074 / std::sqrt((double)D));
    hipError_t e = va::launch_decode_ex(kind_of(fmt), D, is_f16(fmt) ? 64 : G, qg, paged, groups, a,
                                        as_stream(stream));
    lease_done(lease);
    if (e != hipSuccess) return hip_fail(e, "decode launch");
    if (!fused) {
        e = va::launch_merge(a.ws, a.out, heads_total, D, a.S, as_stream(stream));
        if (e != hipSuccess) return hip_fail(e, "merge launch");
    }
    return VA_OK;
}

} // namespace

extern "C" {

int va_pick_splits_gqa(va_fmt fmt, int Hq, int Hkv, int L, int D, int* S) {
    if (!S) return fail(VA_ENULL, "S is NULL");
    if (!valid_fmt(fmt) || Hq < 1 || Hkv < 1 || Hq % Hkv || L < 1 || (D != 64 && D != 128))
        return fail(VA_EINVAL, "invalid arguments to va_pick_splits_gqa");
    if (Hq == Hkv) return va_pick_splits(fmt, Hq, L, D, S);
    if (!tiled_of(fmt)) return fail(VA_EINVAL, "grouped-query decode needs a tiled format (f16+, q8+, q4+, q3+)");
    int qg, nsub, chunk;
    pick_qg(kind_of(fmt), D, Hq / Hkv, &qg, &nsub);
    splits_ex(kind_of(fmt), D, qg, Hkv * nsub, L, 0, S, &chunk);
    return VA_OK;
}

int va_decode_gqa(va_fmt fmt, const va_bufs* b, int Hq, int Hkv, int L, int D, int G, int S,
                  void* stream) {
    if (!valid_fmt(fmt)) return fail(VA_EINVAL, "invalid format %d", (int)fmt);
    if (Hq < 1 || Hkv < 1 || Hq % Hkv)
        return fail(VA_EINVAL, "Hq must be a positive multiple of Hkv (Hq=%d, Hkv=%d)", Hq, Hkv);
    if (S < 0) return fail(VA_EINVAL, "S must be >= 0 (0 picks it)");
    if (Hq == Hkv) {
        int s = S;
        if (s == 0) {
            const int rc = va_pick_splits(fmt, Hq, L, D, &s);
            if (rc) return rc;
        }
        return va_decode(fmt, b, Hq, L, D, G, s, stream);
    }
    if (!tiled_of(fmt)) return fail(VA_EINVAL, "grouped-query decode needs a tiled format (f16+, q8+, q4+, q3+)");
    int rc = validate(fmt, b, Hkv, L, D, G, 1, true);
    if (rc) return rc;
    int qg, nsub, Sx, chunk;
    pick_qg(kind_of(fmt), D, Hq / Hkv, &qg, &nsub);
    const int groups = Hkv * nsub;
    splits_ex(kind_of(fmt), D, qg, groups, L, S, &Sx, &chunk);
    if ((long long)Hq * Sx > 0x7FFFFFFFLL || (long long)groups * Sx > 0x7FFFFFFFLL)
        return fail(VA_ERANGE, "Hq*S too large");
    va::DecodeArgs a{};
    a.k = static_cast<const uint8_t*>(b->k);
    a.v = static_cast<const uint8_t*>(b->v);
    a.sk = b->sk;
    a.sv = b->sv;
    a.q = b->q;
    a.ws = b->ws;
    a.out = b->out;
    a.L = L;
    a.S = Sx;
    a.chunk = chunk;
    a.hkv = Hkv;
    a.qgroup = Hq / Hkv;
    a.nsub = nsub;
    return launch_ex(fmt, a, D, G, qg, false, groups, Hq, stream);
}

size_t va_page_bytes(va_fmt fmt, int Hkv, int page_rows, int D) {
    if (!valid_fmt(fmt) || Hkv < 1 || page_rows < 1 || D < 1) return 0;
    return (size_t)Hkv * page_rows * row_bytes(fmt, D);
}

size_t va_page_scale_bytes(va_fmt fmt, int Hkv, int page_rows, int D, int G) {
    if (!valid_fmt(fmt) || is_f16(fmt) || Hkv < 1 || page_rows < 1 || G < 1 || D % G) return 0;
    return (size_t)Hkv * page_rows * (D / G) * 2;
}

} // extern "C"

namespace {

int validate_shape(va_fmt fmt, const va_paged_shape* sh, bool decode) {
    if (!valid_fmt(fmt)) return fail(VA_EINVAL, "invalid format %d", (int)fmt);
    if (!sh) return fail(VA_ENULL, "shape is NULL");
    if (sh->B < 1 || sh->Hkv < 1) return fail(VA_EINVAL, "B and Hkv must be >= 1");
    if (sh->D != 64 && sh->D != 128) return fail(VA_EINVAL, "D must be 64 or 128 (got %d)", sh->D);
    if (!is_f16(fmt) && !((sh->G == 32 || sh->G == 64) && sh->G <= sh->D))
        return fail(VA_EINVAL, "G must be 32 or 64 and <= D (got G=%d)", sh->G);
    if (sh->max_pages < 1 || sh->num_pages < 1) return fail(VA_EINVAL, "max_pages and num_pages must be >= 1");
    if (sh->page_rows < 1) return fail(VA_EINVAL, "page_rows must be >= 1");
    if ((long long)sh->num_pages * sh->Hkv * sh->page_rows > (1LL << 40))
        return fail(VA_ERANGE, "page pool too large");
    if (!decode) return VA_OK;
    if (!tiled_of(fmt)) return fail(VA_EINVAL, "paged decode needs a tiled format (f16+, q8+, q4+, q3+)");
    if (sh->Hq < 1 || sh->Hq % sh->Hkv)
        return fail(VA_EINVAL, "Hq must be a positive multiple of Hkv (Hq=%d, Hkv=%d)", sh->Hq, sh->Hkv);
    if (!pow2(sh->page_rows) || sh->page_rows < 64 || sh->page_rows > (1 << 24))
        return fail(VA_EINVAL, "page_rows must be a power of two in [64, 2^24] (got %d)", sh->page_rows);
    if (sh->max_seq_len < 0 || (long long)sh->max_seq_len > (long long)sh->max_pages * sh->page_rows)
        return fail(VA_EINVAL, "max_seq_len must be in [0, max_pages*page_rows]");
    if ((long long)sh->max_pages * sh->page_rows > 0x7FFFFFFFLL)
        return fail(VA_ERANGE, "max_pages*page_rows must stay below 2^31");
    return VA_OK;
}

} // namespace

extern "C" {

int va_pick_splits_paged(va_fmt fmt, const va_paged_shape* sh, int* S) {
    if (!S) return fail(VA_ENULL, "S is NULL");
    int rc = validate_shape(fmt, sh, true);
    if (rc) return rc;
    int qg, nsub, chunk;
    pick_qg(kind_of(fmt), sh->D, sh->Hq / sh->Hkv, &qg, &nsub);
    splits_ex(kind_of(fmt), sh->D, qg, sh->B * sh->Hkv * nsub, std::max(1, sh->max_seq_len), 0, S, &chunk);
    // a split may span at most MAX_SPLIT_PAGES pages
    while ((chunk / sh->page_rows) + 2 > va::MAX_SPLIT_PAGES && *S < 0x7FFF) {
        splits_ex(kind_of(fmt), sh->D, qg, sh->B * sh->Hkv * nsub, std::max(1, sh->max_seq_len), *S * 2, S, &chunk);
    }
    return VA_OK;
}

int va_decode_paged(va_fmt fmt, const va_paged_bufs* b, const va_paged_shape* sh, int S,
                    void* stream) {
    int rc = validate_shape(fmt, sh, true);
    if (rc) return rc;
    if (!b) return fail(VA_ENULL, "bufs is NULL");
    if (S < 0) return fail(VA_EINVAL, "S must be >= 0 (0 picks it)");
    const bool quant = !is_f16(fmt);
    if (!b->k || !b->v || !b->q || !b->out || !b->ws || !b->block_table || !b->seq_lens)
        return fail(VA_ENULL, "k, v, q, out, ws, block_table and seq_lens must be non-NULL");
    if (quant && (!b->sk || !b->sv)) return fail(VA_ENULL, "quantized formats need sk and sv");
    const size_t kal = kind_of(fmt) == 3 ? 4 : 16;
    if (!aligned(b->k, kal) || !aligned(b->v, kal))
        return fail(VA_EALIGN, "k and v must be %zu-byte aligned", kal);
    if (!aligned(b->q, 16)) return fail(VA_EALIGN, "q must be 16-byte aligned");
    if (!aligned(b->out, 2) || !aligned(b->ws, 4) || !aligned(b->block_table, 4) || !aligned(b->seq_lens, 4))
        return fail(VA_EALIGN, "out, ws, block_table or seq_lens misaligned");
    if (quant) {
        const size_t sal = (sh->D / sh->G) >= 2 ? 4 : 2;
        if (!aligned(b->sk, sal) || !aligned(b->sv, sal))
            return fail(VA_EALIGN, "sk and sv must be %zu-byte aligned", sal);
    }
    int qg, nsub, Sx, chunk;
    pick_qg(kind_of(fmt), sh->D, sh->Hq / sh->Hkv, &qg, &nsub);
    const long long groups = (long long)sh->B * sh->Hkv * nsub;
    if (S == 0) {
        rc = va_pick_splits_paged(fmt, sh, &Sx);
        if (rc) return rc;
        S = Sx;
    }
    splits_ex(kind_of(fmt), sh->D, qg, (int)std::min<long long>(groups, 1 << 30), std::max(1, sh->max_seq_len), S,
              &Sx, &chunk);
    if (chunk / sh->page_rows + 2 > va::MAX_SPLIT_PAGES)
        return fail(VA_EINVAL, "a split of %d positions spans more than %d pages; raise S", chunk,
                    va::MAX_SPLIT_PAGES);
    if (groups * Sx > 0x7FFFFFFFLL || (long long)sh->B * sh->Hq * Sx > 0x7FFFFFFFLL)
        return fail(VA_ERANGE, "B*Hq*S too large");
    va::DecodeArgs a{};
    a.k = static_cast<const uint8_t*>(b->k);
    a.v = static_cast<const uint8_t*>(b->v);
    a.sk = b->sk;
    a.sv = b->sv;
    a.q = b->q;
    a.ws = b->ws;
    a.out = b->out;
    a.L = sh->max_seq_len;           // the paged kernels' length cap
    a.S = Sx;
    a.chunk = chunk;
    a.hkv = sh->Hkv;
    a.qgroup = sh->Hq / sh->Hkv;
    a.nsub = nsub;
    a.block_table = b->block_table;
    a.seq_lens = b->seq_lens;
    a.max_pages = sh->max_pages;
    a.page_shift = log2i(sh->page_rows);
    a.num_pages = sh->num_pages;
    return launch_ex(fmt, a, sh->D, sh->G, qg, true, (int)groups, sh->B * sh->Hq, stream);
}

int va_append_kv(va_fmt fmt, const uint16_t* x, int n, const int32_t* start,
                 const int32_t* block_table, const va_paged_shape* sh, void* pages,
                 uint16_t* scales, void* stream) {
    int rc = validate_shape(fmt, sh, false);
    if (rc) return rc;
    if (n < 0) return fail(VA_EINVAL, "n must be >= 0");
    if (n == 0) return VA_OK;
    const bool quant = !is_f16(fmt);
    if (!x || !start || !block_table || !pages || (quant && !scales))
        return fail(VA_ENULL, "x, start, block_table, pages (and scales) must be non-NULL");
    if (!aligned(x, 16)) return fail(VA_EALIGN, "x must be 16-byte aligned");
    if (!aligned(pages, quant ? 4 : 16)) return fail(VA_EALIGN, "pages misaligned");
    if (quant && !aligned(scales, 2)) return fail(VA_EALIGN, "scales must be 2-byte aligned");
    if (!aligned(start, 4) || !aligned(block_table, 4)) return fail(VA_EALIGN, "start/block_table misaligned");
    va::AppendArgs a{};
    a.x = x;
    a.start = start;
    a.block_table = block_table;
    a.pages = static_cast<uint8_t*>(pages);
    a.scales = scales;
    a.B = sh->B;
    a.hkv = sh->Hkv;
    a.n = n;
    a.D = sh->D;
    a.page_rows = sh->page_rows;
    a.max_pages = sh->max_pages;
    a.num_pages = sh->num_pages;
    const hipError_t e = va::launch_append(bits_of(fmt), is_f16(fmt) ? 32 : sh->G, a, as_stream(stream));
    if (e != hipSuccess) return hip_fail(e, "append launch");
    return VA_OK;
}

int va_quantize(int bits, int G, const float* x, size_t rows, int D, void* packed,
                uint16_t* scales, void* stream) {
    if (!(bits == 8 || bits == 4 || bits == 3)) return fail(VA_EINVAL, "bits must be 8, 4 or 3");
    if (!((G == 32 || G == 64) && D >= G && D % G == 0 && D % 8 == 0))
        return fail(VA_EINVAL, "G must be 32 or 64 and divide D");
    if (!x || !packed || !scales) return fail(VA_ENULL, "x, packed and scales must be non-NULL");
    if (!aligned(x, 16) || !aligned(packed, 4) || !aligned(scales, 2))
        return fail(VA_EALIGN, "x needs 16-byte, packed 4-byte, scales 2-byte alignment");
    if (rows == 0) return VA_OK;
    const hipError_t e = va::launch_quantize(bits, G, x, rows, D, static_cast<uint8_t*>(packed),
                                             scales, as_stream(stream));
    if (e != hipSuccess) return hip_fail(e, "quantize launch");
    return VA_OK;
}

int va_dequantize(int bits, int G, const void* packed, const uint16_t* scales, size_t rows, int D,
                  float* out, void* stream) {
    if (!(bits == 8 || bits == 4 || bits == 3)) return fail(VA_EINVAL, "bits must be 8, 4 or 3");
    if (!((G == 32 || G == 64) && D >= G && D % G == 0 && D % 8 == 0))
        return fail(VA_EINVAL, "G must be 32 or 64 and divide D");
    if (!packed || !scales || !out) return fail(VA_ENULL, "packed, scales and out must be non-NULL");
    if (!aligned(packed, 4) || !aligned(scales, 2) || !aligned(out, 16))
        return fail(VA_EALIGN, "packed needs 4-byte, scales 2-byte, out 16-byte alignment");
    if (rows == 0) return VA_OK;
    const hipError_t e = va::launch_dequantize(bits, G, static_cast<const uint8_t*>(packed), scales, rows, D,
                                               out, as_stream(stream));
    if (e != hipSuccess) return hip_fail(e, "dequantize launch");
    return VA_OK;
}

int va_f32_to_f16(const float* x, size_t n, uint16_t* out, void* stream) {
    if (!x || !out) return fail(VA_ENULL, "x and out must be non-NULL");
    if (n == 0) return VA_OK;
    const hipError_t e = va::launch_f32_to_f16(x, n, out, as_stream(stream));
    if (e != hipSuccess) return hip_fail(e, "f32_to_f16 launch");
    return VA_OK;
}

int va_fill_normal(float* x, size_t n, uint64_t seed, void* stream) {
    if (!x) return fail(VA_ENULL, "x must be non-NULL");
    if (n == 0) return VA_OK;
    const hipError_t e = va::launch_fill_normal(x, n, seed, as_stream(stream));
    if (e != hipSuccess) return hip_fail(e, "fill_normal launch");
    return VA_OK;
}

int va_probe_launch(int launches, double* us_per_launch) {
    if (!us_per_launch) return fail(VA_ENULL, "us_per_launch is NULL");
    if (launches < 1 || launches > 1000000) return fail(VA_EINVAL, "launches must be in [1, 10^6]");
    *us_per_launch = 0.0;
    float* sink = nullptr;
    VA_HIP(hipMalloc(&sink, 4), "hipMalloc sink");
    hipStream_t st = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    int rc = VA_OK;
    do {
        hipError_t e;
        if ((e = hipStreamCreateWithFlags(&st, hipStreamNonBlocking)) != hipSuccess) { rc = hip_fail(e, "hipStreamCreate"); break; }
        if ((e = hipEventCreate(&e0)) != hipSuccess || (e = hipEventCreate(&e1)) != hipSuccess) {
            rc = hip_fail(e, "hipEventCreate");
            break;
        }
        const int grid = cu_count() > 0 ? cu_count() : 256;
        for (int i = 0; i < 50 && e == hipSuccess; ++i) e = va::launch_empty(grid, sink, st);
        if (e == hipSuccess) e = hipStreamSynchronize(st);
        if (e == hipSuccess) e = hipEventRecord(e0, st);
        for (int i = 0; i < launches && e == hipSuccess; ++i) e = va::launch_empty(grid, sink, st);
        if (e == hipSuccess) e = hipEventRecord(e1, st);
        if (e == hipSuccess) e = hipEventSynchronize(e1);
        float ms = 0.f;
        if (e == hipSuccess) e = hipEventElapsedTime(&ms, e0, e1);
        if (e != hipSuccess) { rc = hip_fail(e, "launch probe"); break; }
        *us_per_launch = (double)ms * 1e3 / launches;
    } while (0);
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    if (st) (void)hipStreamDestroy(st);
    (void)hipFree(sink);
    return rc;
}

int va_probe_read(size_t bytes, int reps, double* best_gbps) {
    if (!best_gbps) return fail(VA_ENULL, "best_gbps is NULL");
    if (bytes < (1u << 20) || reps < 1) return fail(VA_EINVAL, "probe needs >= 1 MiB and reps >= 1");
    bytes &= ~(size_t)15;
    const int cus = cu_count() > 0 ? cu_count() : 256;
    const int grids[]   = {cus * 4, cus * 8, cus * 16, cus * 32};
    const int unrolls[] = {4, 8};
    void* src = nullptr;
    uint32_t* dig = nullptr;
    VA_HIP(hipMalloc(&src, bytes), "hipMalloc probe buffer");
    if (hipMalloc(&dig, (size_t)cus * 32 * va::PROBE_DIGEST_WORDS * 4) != hipSuccess) {
        (void)hipFree(src);
        return fail(VA_EHIP, "hipMalloc digest");
    }
    int rc = VA_OK;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    double best = 0.0;
    do {
        hipError_t e;
        if ((e = hipMemset(src, 1, bytes)) != hipSuccess) { rc = hip_fail(e, "hipMemset"); break; }
        if ((e = hipEventCreate(&e0)) != hipSuccess || (e = hipEventCreate(&e1)) != hipSuccess) {
            rc = hip_fail(e, "hipEventCreate");
            break;
        }
        // Both forms read all `bytes` (va_probe_digest checks each form's coverage).
        for (int form = 0; form < 2 && e == hipSuccess; ++form) {
            for (int gi = 0; gi < (form == 0 ? 4 : 2) && e == hipSuccess; ++gi) {
                const int gsz = form == 0 ? grids[gi] : cus * (gi + 1);   // chunked: 1 or 2 groups per CU
                for (int un : unrolls) {
                    auto launch = [&]() {
                        return form == 0 ? va::launch_probe(src, bytes, dig, gsz, un, nullptr)
                                         : va::launch_probe_chunks(src, bytes, dig, gsz, un, nullptr);
                    };
                    if ((e = launch()) != hipSuccess) break;
                    for (int r = 0; r < reps && e == hipSuccess; ++r) {
                        (void)hipEventRecord(e0, nullptr);
                        e = launch();
                        (void)hipEventRecord(e1, nullptr);
                        if (e == hipSuccess) e = hipEventSynchronize(e1);
                        float ms = 0.f;
                        if (e == hipSuccess) e = hipEventElapsedTime(&ms, e0, e1);
                        if (e == hipSuccess && ms > 0.f) best = std::max(best, (double)bytes / (ms * 1e6));
                    }
                    if (e != hipSuccess) break;
                }
            }
        }
        if (e != hipSuccess) rc = hip_fail(e, "probe");
    } while (0);
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    (void)hipFree(dig);
    (void)hipFree(src);
    if (rc == VA_OK) *best_gbps = best;
    return rc;
}

int va_probe_digest(const void* src, size_t bytes, int form, int grid, int unroll, uint32_t* xor4,
                    uint64_t* loads, size_t* bytes_read) {
    if (!src || !xor4 || !loads || !bytes_read) return fail(VA_ENULL, "src, xor4, loads and bytes_read must be non-NULL");
    if (form != 0 && form != 1) return fail(VA_EINVAL, "form must be 0 (grid-stride) or 1 (chunked)");
    if (grid < 1 || grid > 65536) return fail(VA_EINVAL, "grid must be in [1, 65536] (got %d)", grid);
    if (unroll != 4 && unroll != 8 && !(form == 0 && unroll == 2))
        return fail(VA_EINVAL, "unroll must be 4 or 8 (2 also for the grid-stride form)");
    if (bytes == 0 || bytes % 16) return fail(VA_EINVAL, "bytes must be a positive multiple of 16");
    if (!aligned(src, 16)) return fail(VA_EALIGN, "src must be 16-byte aligned");
    if (form == 1 && va::probe_chunk_bytes(bytes, grid) > 0x7FFFFFFFu)
        return fail(VA_ERANGE, "chunk per work-group must stay below 2^31 bytes");
    uint32_t* dig = nullptr;
    const size_t dwords = (size_t)grid * va::PROBE_DIGEST_WORDS;
    VA_HIP(hipMalloc(&dig, dwords * 4), "hipMalloc digest");
    std::vector<uint32_t> h(dwords);
    hipError_t e = form == 0 ? va::launch_probe(src, bytes, dig, grid, unroll, nullptr)
                             : va::launch_probe_chunks(src, bytes, dig, grid, unroll, nullptr);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e == hipSuccess) e = hipMemcpy(h.data(), dig, dwords * 4, hipMemcpyDeviceToHost);
    (void)hipFree(dig);
    if (e != hipSuccess) return hip_fail(e, "probe digest");
    uint32_t x[4] = {0, 0, 0, 0};
    uint64_t n = 0;
    for (int g = 0; g < grid; ++g) {
        const uint32_t* d = h.data() + (size_t)g * va::PROBE_DIGEST_WORDS;
        for (int i = 0; i < 4; ++i) x[i] ^= d[i];
        n += d[4];
    }
    for (int i = 0; i < 4; ++i) xor4[i] = x[i];
    *loads = n;
    *bytes_read = bytes;
    return VA_OK;
}

int va_probe_read_sized(size_t bytes, size_t min_set, int launches, double* us_per_launch, double* gbps) {
    if (!us_per_launch || !gbps) return fail(VA_ENULL, "us_per_launch and gbps must be non-NULL");
    bytes &= ~(size_t)15;
    if (bytes < 4096 || launches < 1 || launches > 100000)
        return fail(VA_EINVAL, "sized probe needs >= 4096 bytes and launches in [1, 10^5]");
    const int cus = cu_count() > 0 ? cu_count() : 256;
    if (va::probe_chunk_bytes(bytes, cus) > 0x7FFFFFFFu) return fail(VA_ERANGE, "bytes too large for the chunked probe");
    const size_t stride = (bytes + 4095) & ~(size_t)4095;
    const size_t copies = std::max<size_t>(1, std::min<size_t>(4096, (min_set + stride - 1) / stride));
    void* src = nullptr;
    uint32_t* dig = nullptr;
    VA_HIP(hipMalloc(&src, copies * stride), "hipMalloc sized probe buffer");
    if (hipMalloc(&dig, (size_t)cus * 2 * va::PROBE_DIGEST_WORDS * 4) != hipSuccess) {
        (void)hipFree(src);
        return fail(VA_EHIP, "hipMalloc digest");
    }
    hipStream_t st = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    int rc = VA_OK;
    double best_ms = 0.0;
    do {
        hipError_t e;
        if ((e = hipMemset(src, 1, copies * stride)) != hipSuccess) { rc = hip_fail(e, "hipMemset"); break; }
        if ((e = hipStreamCreateWithFlags(&st, hipStreamNonBlocking)) != hipSuccess) { rc = hip_fail(e, "hipStreamCreate"); break; }
        if ((e = hipEventCreate(&e0)) != hipSuccess || (e = hipEventCreate(&e1)) != hipSuccess) {
            rc = hip_fail(e, "hipEventCreate");
            break;
        }
        // The chunked form's four shapes (1 or 2 groups per CU, 4 or 8 loads per
        // lane in flight), each `launches` back to back over rotating copies;
        // the best mean is the ceiling. Each shape first runs untimed for at
        // least 50 ms of wall time: an idle MI355X sits near its lowest clocks,
        // and a cold 142.6 MB read measured ~2 us (9 %) slower per launch.
        for (int gpc = 1; gpc <= 2 && e == hipSuccess; ++gpc) {
            for (int un : {4, 8}) {
                size_t c = 0;
                auto launch = [&]() {
                    const void* p = static_cast<const uint8_t*>(src) + (c++ % copies) * stride;
                    return va::launch_probe_chunks(p, bytes, dig, cus * gpc, un, st);
                };
                const auto warm_end = std::chrono::steady_clock::now() + std::chrono::milliseconds(50);
                for (int batch = 0; batch < 4096 && e == hipSuccess; ++batch) {
                    for (int i = 0; i < 16 && e == hipSuccess; ++i) e = launch();
                    if (e == hipSuccess) e = hipStreamSynchronize(st);
                    if (std::chrono::steady_clock::now() >= warm_end) break;
                }
                for (int i = 0; i < 5 && e == hipSuccess; ++i) e = launch();
                if (e == hipSuccess) e = hipStreamSynchronize(st);
                if (e == hipSuccess) e = hipEventRecord(e0, st);
                for (int i = 0; i < launches && e == hipSuccess; ++i) e = launch();
                if (e == hipSuccess) e = hipEventRecord(e1, st);
                if (e == hipSuccess) e = hipEventSynchronize(e1);
                float ms = 0.f;
                if (e == hipSuccess) e = hipEventElapsedTime(&ms, e0, e1);
                if (e != hipSuccess) break;
                const double per = (double)ms / launches;
                if (per > 0.0 && (best_ms == 0.0 || per < best_ms)) best_ms = per;
            }
        }
        if (e != hipSuccess) rc = hip_fail(e, "sized probe");
    } while (0);
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    if (st) (void)hipStreamDestroy(st);
    (void)hipFree(dig);
    (void)hipFree(src);
    if (rc == VA_OK) {
        *us_per_launch = best_ms * 1e3;
        *gbps = best_ms > 0.0 ? (double)bytes / (best_ms * 1e6) : 0.0;
    }
    return rc;
}

// ---------------------------------------------------------------- shims --
int va_device_count(int* n) {
    if (!n) return fail(VA_ENULL, "n is NULL");
    const hipError_t e = hipGetDeviceCount(n);
    if (e != hipSuccess) { *n = 0; return hip_fail(e, "hipGetDeviceCount"); }
    return VA_OK;
}

int va_set_device(int dev) {
    VA_HIP(hipSetDevice(dev), "hipSetDevice");
    g_cu_count = 0;
    return VA_OK;
}

int va_device_info(va_device_info_t* info) {
    if (!info) return fail(VA_ENULL, "info is NULL");
    int dev = 0;
    VA_HIP(hipGetDevice(&dev), "hipGetDevice");
    hipDeviceProp_t p;
    VA_HIP(hipGetDeviceProperties(&p, dev), "hipGetDeviceProperties");
    std::memset(info, 0, sizeof *info);
    std::snprintf(info->name, sizeof info->name, "%s", p.name);
    std::snprintf(info->arch, sizeof info->arch, "%s", p.gcnArchName);
    info->compute_units = p.multiProcessorCount;
    info->clock_khz     = p.clockRate;
    info->mem_clock_khz = p.memoryClockRate;
    info->mem_bus_bits  = p.memoryBusWidth;
    info->total_mem     = p.totalGlobalMem;
    info->l2_bytes      = (size_t)p.l2CacheSize;
    return VA_OK;
}

int va_malloc(void** p, size_t bytes) {
    if (!p) return fail(VA_ENULL, "p is NULL");
    VA_HIP(hipMalloc(p, bytes ? bytes : 1), "hipMalloc");
    return VA_OK;
}
int va_free(void* p) {
    VA_HIP(hipFree(p), "hipFree");
    return VA_OK;
}
int va_memcpy_h2d(void* dst, const void* src, size_t bytes) {
    VA_HIP(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice), "hipMemcpy H2D");
    return VA_OK;
}
int va_memcpy_d2h(void* dst, const void* src, size_t bytes) {
    VA_HIP(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost), "hipMemcpy D2H");
    return VA_OK;
}
int va_memcpy_d2d(void* dst, const void* src, size_t bytes, void* stream) {
    VA_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, as_stream(stream)), "hipMemcpy D2D");
    return VA_OK;
}
int va_memset(void* p, int value, size_t bytes) {
    VA_HIP(hipMemset(p, value, bytes), "hipMemset");
    return VA_OK;
}
int va_sync(void) {
    VA_HIP(hipDeviceSynchronize(), "hipDeviceSynchronize");
    return VA_OK;
}
int va_stream_create(void** stream) {
    if (!stream) return fail(VA_ENULL, "stream is NULL");
    hipStream_t s = nullptr;
    VA_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreate");
    *stream = s;
    return VA_OK;
}
int va_stream_destroy(void* stream) {
    // The stream's bindings are freed once its last call has finished.
    VA_HIP(hipStreamSynchronize(as_stream(stream)), "hipStreamSynchronize");
    int dev = 0;
    VA_HIP(hipGetDevice(&dev), "hipGetDevice");
    VA_HIP(release_owner(dev, owner_key(stream), 0, as_stream(stream)), "release stream bindings");
    VA_HIP(hipStreamDestroy(as_stream(stream)), "hipStreamDestroy");
    return VA_OK;
}
int va_stream_release(void* stream) {
    VA_HIP(hipStreamSynchronize(as_stream(stream)), "hipStreamSynchronize");
    int dev = 0;
    VA_HIP(hipGetDevice(&dev), "hipGetDevice");
    VA_HIP(release_owner(dev, owner_key(stream), 0, as_stream(stream)), "release stream bindings");
    return VA_OK;
}
int va_capture_release(unsigned long long capture_id) {
    VA_HIP(hipDeviceSynchronize(), "hipDeviceSynchronize");
    VA_HIP(release_capture_all(capture_id | (1ull << 63)), "release capture bindings");
    return VA_OK;
}
int va_stream_sync(void* stream) {
    VA_HIP(hipStreamSynchronize(as_stream(stream)), "hipStreamSynchronize");
    return VA_OK;
}
int va_event_create(void** ev) {
    if (!ev) return fail(VA_ENULL, "ev is NULL");
    hipEvent_t e = nullptr;
    VA_HIP(hipEventCreate(&e), "hipEventCreate");
    *ev = e;
    return VA_OK;
}
int va_event_destroy(void* ev) {
    VA_HIP(hipEventDestroy(static_cast<hipEvent_t>(ev)), "hipEventDestroy");
    return VA_OK;
}
int va_event_record(void* ev, void* stream) {
    VA_HIP(hipEventRecord(static_cast<hipEvent_t>(ev), as_stream(stream)), "hipEventRecord");
    return VA_OK;
}
int va_event_sync(void* ev) {
    VA_HIP(hipEventSynchronize(static_cast<hipEvent_t>(ev)), "hipEventSynchronize");
    return VA_OK;
}
int va_event_elapsed_ms(void* start, void* stop, float* ms) {
    if (!ms) return fail(VA_ENULL, "ms is NULL");
    VA_HIP(hipEventElapsedTime(ms, static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(stop)),
           "hipEventElapsedTime");
    return VA_OK;
}

int va_graph_begin(void* stream) {
    if (!stream) return fail(VA_EINVAL, "graph capture needs a non-default stream");
    VA_HIP(hipStreamBeginCapture(as_stream(stream), hipStreamCaptureModeThreadLocal),
           "hipStreamBeginCapture");
    return VA_OK;
}
int va_graph_end(void* stream, void** graph_exec) {
    if (!stream || !graph_exec) return fail(VA_ENULL, "stream and graph_exec must be non-NULL");
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    unsigned long long id = 0;
    VA_HIP(hipStreamGetCaptureInfo(as_stream(stream), &cs, &id), "hipStreamGetCaptureInfo");
    const unsigned long long capture = cs == hipStreamCaptureStatusActive ? (id | (1ull << 63)) : 0ull;
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamEndCapture(as_stream(stream), &g);
    if (e != hipSuccess) {                       // no graph: nothing can replay the capture's slots
        (void)release_capture_all(capture);
        return hip_fail(e, "hipStreamEndCapture");
    }
    hipGraphExec_t x = nullptr;
    e = hipGraphInstantiate(&x, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) {
        (void)release_capture_all(capture);
        return hip_fail(e, "hipGraphInstantiate");
    }
    if (capture) {
        std::lock_guard<std::mutex> lock(g_graph_mu);
        g_graph_capture[x] = capture;
    }
    *graph_exec = x;
    return VA_OK;
}
int va_graph_launch(void* graph_exec, void* stream) {
    VA_HIP(hipGraphLaunch(static_cast<hipGraphExec_t>(graph_exec), as_stream(stream)), "hipGraphLaunch");
    return VA_OK;
}
int va_graph_destroy(void* graph_exec) {
    // The ticket slots the capture bound are freed once no replay is running.
    unsigned long long capture = 0;
    {
        std::lock_guard<std::mutex> lock(g_graph_mu);
        auto it = g_graph_capture.find(graph_exec);
        if (it != g_graph_capture.end()) {
            capture = it->second;
            g_graph_capture.erase(it);
        }
    }
    if (capture) VA_HIP(hipDeviceSynchronize(), "hipDeviceSynchronize");
    VA_HIP(hipGraphExecDestroy(static_cast<hipGraphExec_t>(graph_exec)), "hipGraphExecDestroy");
    VA_HIP(release_capture_all(capture), "release capture bindings");
    return VA_OK;
}

} // extern "C"
