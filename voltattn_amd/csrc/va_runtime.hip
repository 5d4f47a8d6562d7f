// va_runtime.hip — the C ABI (include/voltattn.h): argument validation,
// format -> kernel dispatch, and the thin HIP runtime shims the host harness
// uses. This is the only translation unit that calls the HIP runtime API.
#include "voltattn.h"
#include "va_kernels.hpp"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>

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

int validate(va_fmt fmt, const va_bufs* b, int H, int L, int D, int G, int S, bool need_out) {
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
    if (!b->k || !b->v || !b->q || !b->ws) return fail(VA_ENULL, "k, v, q and ws must be non-NULL");
    if (need_out && !b->out) return fail(VA_ENULL, "out must be non-NULL");
    if (quant && (!b->sk || !b->sv)) return fail(VA_ENULL, "quantized formats need sk and sv");
    const size_t kal = kind_of(fmt) == 3 ? 4 : 16;
    if (!aligned(b->k, kal) || !aligned(b->v, kal))
        return fail(VA_EALIGN, "k and v must be %zu-byte aligned", kal);
    if (!aligned(b->q, 16)) return fail(VA_EALIGN, "q must be 16-byte aligned");
    if (!aligned(b->ws, 4)) return fail(VA_EALIGN, "ws must be 4-byte aligned");
    if (need_out && !aligned(b->out, 2)) return fail(VA_EALIGN, "out must be 2-byte aligned");
    if (quant) {
        const size_t sal = (D / G) >= 2 ? 4 : 2;
        if (!aligned(b->sk, sal) || !aligned(b->sv, sal))
            return fail(VA_EALIGN, "sk and sv must be %zu-byte aligned", sal);
    }
    return VA_OK;
}

std::atomic<unsigned> g_ticket_seq{0};

// fused: merge inside the decode kernel (needs H <= TICKET_MAXH, S <= 64 and
// H*S <= PART_CAP), else the partials are left in ws for a separate merge pass.
int run_splits(va_fmt fmt, const va_bufs* b, int H, int L, int D, int G, int S, void* stream,
               bool fused) {
    va::DecodeArgs a;
    a.k  = static_cast<const uint8_t*>(b->k);
    a.v  = static_cast<const uint8_t*>(b->v);
    a.sk = b->sk;
    a.sv = b->sv;
    a.q  = b->q;
    a.ws = b->ws;
    a.out = b->out;
    a.ticket_slot = fused ? (int)(g_ticket_seq.fetch_add(1u) % va::TICKET_SLOTS) : -1;
    a.L = L;
    a.S = S;
    a.chunk  = (L + S - 1) / S;
    a.qscale = (float)(1.4426950408889634074 / std::sqrt((double)D));
    const hipError_t e = va::launch_decode(kind_of(fmt), tiled_of(fmt), H, D, is_f16(fmt) ? 64 : G,
                                           a, as_stream(stream));
    if (e != hipSuccess) return hip_fail(e, "decode launch");
    return VA_OK;
}

int g_cu_count = 0;

int cu_count() {
    if (g_cu_count > 0) return g_cu_count;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    g_cu_count = n;
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
    const int per_cu = va::groups_per_cu(kind_of(fmt), tiled_of(fmt));
    const int target = std::max(1, (per_cu * cus + H - 1) / H);
    const int s0     = std::max(1, std::min(tiles, target));
    const int tps    = (tiles + s0 - 1) / s0;               // tiles per split
    *S = std::max(1, (L + tps * tb - 1) / (tps * tb));
    return VA_OK;
}

int va_decode(va_fmt fmt, const va_bufs* b, int H, int L, int D, int G, int S, void* stream) {
    int rc = validate(fmt, b, H, L, D, G, S, true);
    if (rc) return rc;
    const bool fused = H <= va::TICKET_MAXH && S <= 64 && (long long)H * S <= va::PART_CAP;
    rc = run_splits(fmt, b, H, L, D, G, S, stream, fused);
    if (rc || fused) return rc;
    const hipError_t e = va::launch_merge(b->ws, b->out, H, D, S, as_stream(stream));
    if (e != hipSuccess) return hip_fail(e, "merge launch");
    return VA_OK;
}

int va_decode_splits(va_fmt fmt, const va_bufs* b, int H, int L, int D, int G, int S, void* stream) {
    const int rc = validate(fmt, b, H, L, D, G, S, false);
    if (rc) return rc;
    return run_splits(fmt, b, H, L, D, G, S, stream, false);
}

int va_merge(const float* ws, uint16_t* out, int H, int D, int S, void* stream) {
    if (!ws || !out) return fail(VA_ENULL, "ws and out must be non-NULL");
    if (H < 1 || S < 1 || (D != 64 && D != 128)) return fail(VA_EINVAL, "invalid H/D/S");
    if (!aligned(ws, 4) || !aligned(out, 2)) return fail(VA_EALIGN, "ws/out misaligned");
    const hipError_t e = va::launch_merge(ws, out, H, D, S, as_stream(stream));
    if (e != hipSuccess) return hip_fail(e, "merge launch");
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

int va_probe_read(size_t bytes, int reps, double* best_gbps) {
    if (!best_gbps) return fail(VA_ENULL, "best_gbps is NULL");
    if (bytes < (1u << 20) || reps < 1) return fail(VA_EINVAL, "probe needs >= 1 MiB and reps >= 1");
    bytes &= ~(size_t)15;
    void* src = nullptr;
    float* sink = nullptr;
    VA_HIP(hipMalloc(&src, bytes), "hipMalloc probe buffer");
    if (hipMalloc(&sink, 4) != hipSuccess) { (void)hipFree(src); return fail(VA_EHIP, "hipMalloc sink"); }
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
        const int cus = cu_count() > 0 ? cu_count() : 256;
        const int grids[]   = {cus * 4, cus * 8, cus * 16, cus * 32};
        const int unrolls[] = {4, 8};
        for (int gsz : grids) {
            for (int un : unrolls) {
                if ((e = va::launch_probe(src, bytes, sink, gsz, un, nullptr)) != hipSuccess) break;
                for (int r = 0; r < reps && e == hipSuccess; ++r) {
                    (void)hipEventRecord(e0, nullptr);
                    e = va::launch_probe(src, bytes, sink, gsz, un, nullptr);
                    (void)hipEventRecord(e1, nullptr);
                    if (e == hipSuccess) e = hipEventSynchronize(e1);
                    float ms = 0.f;
                    if (e == hipSuccess) e = hipEventElapsedTime(&ms, e0, e1);
                    if (e == hipSuccess && ms > 0.f) best = std::max(best, (double)bytes / (ms * 1e6));
                }
                if (e != hipSuccess) break;
            }
            if (e != hipSuccess) break;
        }
        if (e != hipSuccess) rc = hip_fail(e, "probe");
    } while (0);
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    (void)hipFree(sink);
    (void)hipFree(src);
    if (rc == VA_OK) *best_gbps = best;
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
    VA_HIP(hipStreamDestroy(as_stream(stream)), "hipStreamDestroy");
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
    hipGraph_t g = nullptr;
    VA_HIP(hipStreamEndCapture(as_stream(stream), &g), "hipStreamEndCapture");
    hipGraphExec_t x = nullptr;
    const hipError_t e = hipGraphInstantiate(&x, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) return hip_fail(e, "hipGraphInstantiate");
    *graph_exec = x;
    return VA_OK;
}
int va_graph_launch(void* graph_exec, void* stream) {
    VA_HIP(hipGraphLaunch(static_cast<hipGraphExec_t>(graph_exec), as_stream(stream)), "hipGraphLaunch");
    return VA_OK;
}
int va_graph_destroy(void* graph_exec) {
    VA_HIP(hipGraphExecDestroy(static_cast<hipGraphExec_t>(graph_exec)), "hipGraphExecDestroy");
    return VA_OK;
}

} // extern "C"
