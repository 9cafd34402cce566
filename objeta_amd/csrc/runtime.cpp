// runtime.cpp — device discovery, context, streams, memory, events and graph
// capture behind the C ABI. Mirrors the reference's L1 device runtime
// (crates/objeta-cuda/src/{context,stream,memory,telemetry,lib}.rs).
#include <cstdlib>
#include <cstring>
#include <string>

#include "host_common.hpp"
#include "kernels.hpp"

namespace objeta {

namespace {
struct LastError {
    int32_t status = 0;
    objeta_hip_error rec{};
};
thread_local LastError g_last;

void copy_str(char* dst, size_t cap, const std::string& s) {
    size_t n = s.size() < cap - 1 ? s.size() : cap - 1;
    std::memcpy(dst, s.data(), n);
    dst[n] = 0;
}
}  // namespace

int32_t set_error(Kind kind, const char* file, unsigned line, const char* module,
                  const std::string& action, const std::string& message) {
    g_last.status = static_cast<int32_t>(kind) + 1;
    g_last.rec.kind = static_cast<int32_t>(kind);
    g_last.rec.line = line;
    const char* base = std::strrchr(file, '/');
    copy_str(g_last.rec.file, sizeof(g_last.rec.file), base ? base + 1 : file);
    copy_str(g_last.rec.module, sizeof(g_last.rec.module), module);
    copy_str(g_last.rec.action, sizeof(g_last.rec.action), action);
    copy_str(g_last.rec.source_message, sizeof(g_last.rec.source_message), message);
    return g_last.status;
}

std::string strf(const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    return std::string(buf);
}

int32_t check_ctx(const objeta_hip_context* ctx, const char* action) {
    if (!ctx) OBJ_FAIL(kInvalidInput, action, "context is NULL");
    return 0;
}

hipStream_t resolve_stream(objeta_hip_context* ctx, objeta_hip_stream s) {
    return s ? static_cast<hipStream_t>(s) : ctx->streams[0];
}

static int32_t fail_if_capturing(hipStream_t stream, const char* action, const std::string& what) {
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    OBJ_HIP(hipStreamIsCapturing(stream, &st), "query stream capture status");
    if (st != hipStreamCaptureStatusNone)
        OBJ_FAIL(kUnsupported, action, what + " needed while capturing; run the call once outside capture first");
    return 0;
}

int32_t stream_scratch(objeta_hip_context* ctx, hipStream_t stream, StreamScratch** out) {
    for (StreamScratch* sc : ctx->scratch)
        if (sc->stream == stream) {
            *out = sc;
            return 0;
        }
    OBJ_TRY(fail_if_capturing(stream, "create stream scratch", "scratch for a new stream"));
    auto* sc = new StreamScratch();
    sc->stream = stream;
    const size_t bytes = kEpochWords * sizeof(uint32_t);
    hipError_t e = hipMalloc(&sc->epochs, bytes);
    // cleared on the caller's stream and waited for: a clear on the null stream is
    // not ordered before kernels on the context's non-blocking streams
    if (e == hipSuccess) e = hipMemsetAsync(sc->epochs, 0, bytes, stream);
    if (e == hipSuccess) e = hipStreamSynchronize(stream);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        if (sc->epochs) (void)hipFree(sc->epochs);
        delete sc;
        OBJ_FAIL(kDriver, "allocate router epoch counters", hipGetErrorString(e));
    }
    ctx->scratch.push_back(sc);
    *out = sc;
    return 0;
}

int32_t ensure_workspace(objeta_hip_context* ctx, hipStream_t stream, int slot, size_t bytes, void** out) {
    StreamScratch* sc = nullptr;
    OBJ_TRY(stream_scratch(ctx, stream, &sc));
    Workspace& ws = sc->ws[slot];
    if (ws.bytes >= bytes) {
        *out = ws.ptr;
        return 0;
    }
    OBJ_TRY(fail_if_capturing(stream, "grow workspace",
                              strf("workspace of %zu bytes (have %zu)", bytes, ws.bytes)));
    size_t grow = bytes < (size_t(1) << 20) ? (size_t(1) << 20) : bytes;
    void* p = nullptr;
    OBJ_HIP(hipMalloc(&p, grow), "allocate workspace");
    // epoch-tagged words in a workspace must start at zero
    OBJ_HIP(hipMemsetAsync(p, 0, grow, stream), "clear workspace");
    OBJ_HIP(hipStreamSynchronize(stream), "clear workspace");
    if (ws.ptr) ctx->retired_ws.push_back(ws.ptr);
    ws.ptr = p;
    ws.bytes = grow;
    *out = p;
    return 0;
}

int32_t ensure_host_stage(objeta_hip_context* ctx, size_t bytes, void** out) {
    if (ctx->host_stage_bytes < bytes) {
        OBJ_HIP(hipDeviceSynchronize(), "synchronize before staging growth");
        if (ctx->host_stage) OBJ_HIP(hipHostFree(ctx->host_stage), "free host staging");
        ctx->host_stage = nullptr;
        ctx->host_stage_bytes = 0;
        size_t grow = bytes < (size_t(1) << 16) ? (size_t(1) << 16) : bytes;
        OBJ_HIP(hipHostMalloc(&ctx->host_stage, grow, hipHostMallocDefault), "allocate host staging");
        ctx->host_stage_bytes = grow;
    }
    *out = ctx->host_stage;
    return 0;
}

static int32_t fill_info(int ordinal, objeta_hip_device_info* out) {
    hipDeviceProp_t p{};
    hipError_t e = hipGetDeviceProperties(&p, ordinal);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        OBJ_FAIL(kRuntime, strf("hipGetDeviceProperties(device=%d)", ordinal), hipGetErrorString(e));
    }
    std::memset(out, 0, sizeof(*out));
    out->ordinal = static_cast<uint64_t>(ordinal);
    std::snprintf(out->name, sizeof(out->name), "%s", p.name);
    std::snprintf(out->arch, sizeof(out->arch), "%s", p.gcnArchName);
    out->total_global_mem_bytes = p.totalGlobalMem;
    out->compute_capability_major = p.major;
    out->compute_capability_minor = p.minor;
    int drv = 0, rt = 0;
    (void)hipDriverGetVersion(&drv);
    (void)hipRuntimeGetVersion(&rt);
    out->driver_version = drv;
    out->runtime_version = rt;
    out->compute_units = p.multiProcessorCount;
    out->wavefront_size = p.warpSize;
    out->l2_cache_bytes = p.l2CacheSize;
    out->max_shared_memory_per_block = static_cast<int32_t>(p.sharedMemPerBlock);
    out->clock_khz = p.clockRate;
    out->memory_clock_khz = p.memoryClockRate;
    out->memory_bus_width_bits = p.memoryBusWidth;
    return 0;
}

}  // namespace objeta

using namespace objeta;

extern "C" {

int32_t objeta_hip_last_error(objeta_hip_error* out) {
    if (out) {
        if (g_last.status == 0) {
            std::memset(out, 0, sizeof(*out));
            out->kind = -1;
        } else {
            *out = g_last.rec;
        }
    }
    return g_last.status;
}

void objeta_hip_clear_error(void) { g_last = LastError{}; }

int32_t objeta_hip_abi_version(void) { return OBJETA_HIP_ABI_VERSION; }

int32_t objeta_hip_block_size(int32_t format) {
    return (format >= OBJETA_HIP_Q4_0 && format <= OBJETA_HIP_FP4_E2M1) ? 32 : -1;
}

int32_t objeta_hip_block_bytes(int32_t format) {
    switch (format) {
        case OBJETA_HIP_Q4_0: return 18;
        case OBJETA_HIP_Q5_0: return 22;
        case OBJETA_HIP_IQ3_0: return 14;
        case OBJETA_HIP_FP4_E2M1: return 17;
        default: return -1;
    }
}

int64_t objeta_hip_quantized_matrix_bytes(int32_t format, uint64_t rows, uint64_t cols) {
    int32_t bb = objeta_hip_block_bytes(format);
    if (bb < 0 || cols % 32 != 0) return -1;
    return static_cast<int64_t>(rows * (cols / 32) * static_cast<uint64_t>(bb));
}

int32_t objeta_hip_device_count(int32_t* out) {
    OBJ_GUARD_BEGIN
    if (!out) OBJ_FAIL(kInvalidInput, "hipGetDeviceCount", "out is NULL");
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        *out = 0;
        OBJ_FAIL(kRuntime, "hipGetDeviceCount", hipGetErrorString(e));
    }
    *out = n;
    return 0;
    OBJ_GUARD_END
}

int32_t objeta_hip_discover_device(uint64_t ordinal, objeta_hip_device_info* out) {
    OBJ_GUARD_BEGIN
    if (!out) OBJ_FAIL(kInvalidInput, "discover device", "out is NULL");
    int n = 0;
    OBJ_TRY(objeta_hip_device_count(&n));
    if (ordinal >= static_cast<uint64_t>(n))
        OBJ_FAIL(kInvalidInput, "select device",
                 strf("device ordinal %llu out of range; %d devices", (unsigned long long)ordinal, n));
    return fill_info(static_cast<int>(ordinal), out);
    OBJ_GUARD_END
}

int32_t objeta_hip_init(const objeta_hip_init_options* opts, objeta_hip_context** out) {
    OBJ_GUARD_BEGIN
    if (!out) OBJ_FAIL(kInvalidInput, "init context", "out is NULL");
    *out = nullptr;
    objeta_hip_init_options o{0, 1};
    if (opts) o = *opts;
    if (o.stream_count < 1) o.stream_count = 1;
    objeta_hip_device_info info{};
    OBJ_TRY(objeta_hip_discover_device(o.device_ordinal, &info));
    auto* ctx = new objeta_hip_context();
    ctx->device = static_cast<int>(o.device_ordinal);
    ctx->info = info;
    if (const char* v = std::getenv("OBJETA_HIP_ROUTER_SPIN_LIMIT")) {
        char* end = nullptr;
        const unsigned long n = std::strtoul(v, &end, 10);
        if (end != v && *end == '\0' && n <= 0xFFFFFFFFul) ctx->router_spin_limit = static_cast<uint32_t>(n);
    }
    auto fail_cleanup = [&](int32_t rc) {
        objeta_hip_destroy(ctx);
        return rc;
    };
    hipError_t e = hipSetDevice(ctx->device);
    if (e != hipSuccess) {
        int32_t rc = set_error(kDriver, __FILE__, __LINE__, __func__, "hipSetDevice", hipGetErrorString(e));
        return fail_cleanup(rc);
    }
    for (uint64_t i = 0; i < o.stream_count; ++i) {
        hipStream_t s = nullptr;
        e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
        if (e != hipSuccess) {
            int32_t rc = set_error(kDriver, __FILE__, __LINE__, __func__,
                                   strf("create HIP stream %llu", (unsigned long long)i), hipGetErrorString(e));
            return fail_cleanup(rc);
        }
        ctx->streams.push_back(s);
    }
    e = hipStreamCreateWithFlags(&ctx->copy_stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
        int32_t rc = set_error(kDriver, __FILE__, __LINE__, __func__, "create copy stream", hipGetErrorString(e));
        return fail_cleanup(rc);
    }
    {
        // the device address of the no-allocation entry point's scratch array
        const int32_t rc = bind_static_scratch(ctx);
        if (rc != 0) return fail_cleanup(rc);
    }
    e = hipMalloc(&ctx->err_word, 64 * sizeof(uint32_t));
    if (e == hipSuccess) e = hipMemset(ctx->err_word, 0, 64 * sizeof(uint32_t));
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        int32_t rc = set_error(kDriver, __FILE__, __LINE__, __func__, "allocate device error word", hipGetErrorString(e));
        return fail_cleanup(rc);
    }
    *out = ctx;
    return 0;
    OBJ_GUARD_END
}

int32_t objeta_hip_destroy(objeta_hip_context* ctx) {
    OBJ_GUARD_BEGIN
    if (!ctx) return 0;
    (void)hipSetDevice(ctx->device);
    (void)hipDeviceSynchronize();
    if (ctx->transient_pool) (void)objeta_hip_cache_destroy(static_cast<objeta_hip_expert_cache*>(ctx->transient_pool));
    ctx->transient_pool = nullptr;
    objeta::detach_caches(ctx);
    for (hipStream_t s : ctx->streams) (void)hipStreamDestroy(s);
    if (ctx->copy_stream) (void)hipStreamDestroy(ctx->copy_stream);
    for (StreamScratch* sc : ctx->scratch) {
        for (auto& w : sc->ws)
            if (w.ptr) (void)hipFree(w.ptr);
        if (sc->epochs) (void)hipFree(sc->epochs);
        delete sc;
    }
    ctx->scratch.clear();
    for (void* p : ctx->retired_ws) (void)hipFree(p);
    if (ctx->host_stage) (void)hipHostFree(ctx->host_stage);
    if (ctx->err_word) (void)hipFree(ctx->err_word);
    (void)hipGetLastError();
    delete ctx;
    return 0;
    OBJ_GUARD_END
}

int32_t objeta_hip_device_info_get(const objeta_hip_context* ctx, objeta_hip_device_info* out) {
    OBJ_TRY(check_ctx(ctx, "device info"));
    if (!out) OBJ_FAIL(kInvalidInput, "device info", "out is NULL");
    *out = ctx->info;
    return 0;
}

int32_t objeta_hip_stream_get(objeta_hip_context* ctx, uint64_t index, objeta_hip_stream* out) {
    OBJ_TRY(check_ctx(ctx, "select stream"));
    if (!out) OBJ_FAIL(kInvalidInput, "select stream", "out is NULL");
    if (index >= ctx->streams.size())
        OBJ_FAIL(kInvalidInput, strf("select HIP stream %llu", (unsigned long long)index),
                 strf("stream index out of range; pool len=%zu", ctx->streams.size()));
    *out = ctx->streams[index];
    return 0;
}

int32_t objeta_hip_stream_synchronize(objeta_hip_context* ctx, objeta_hip_stream stream) {
    OBJ_TRY(check_ctx(ctx, "synchronize stream"));
    OBJ_HIP(hipSetDevice(ctx->device), "hipSetDevice");
    OBJ_HIP(hipStreamSynchronize(resolve_stream(ctx, stream)), "synchronize HIP stream");
    return 0;
}

int32_t objeta_hip_malloc(objeta_hip_context* ctx, uint64_t bytes, void** d_out) {
    OBJ_TRY(check_ctx(ctx, "device allocation"));
    if (!d_out) OBJ_FAIL(kInvalidInput, "device allocation", "out is NULL");
    *d_out = nullptr;
    OBJ_HIP(hipSetDevice(ctx->device), "hipSetDevice");
    if (bytes == 0) return 0;
    OBJ_HIP(hipMalloc(d_out, bytes), strf("hipMalloc(%llu)", (unsigned long long)bytes));
    return 0;
}

int32_t objeta_hip_free(objeta_hip_context* ctx, void* d_ptr) {
    OBJ_TRY(check_ctx(ctx, "device free"));
    if (!d_ptr) return 0;
    OBJ_HIP(hipSetDevice(ctx->device), "hipSetDevice");
    OBJ_HIP(hipFree(d_ptr), "hipFree");
    return 0;
}

int32_t objeta_hip_alloc_pinned_host(objeta_hip_context* ctx, uint64_t bytes, void** h_out) {
    OBJ_TRY(check_ctx(ctx, "pinned host allocation"));
    if (!h_out) OBJ_FAIL(kInvalidInput, "pinned host allocation", "out is NULL");
    *h_out = nullptr;
    OBJ_HIP(hipSetDevice(ctx->device), "hipSetDevice");
    if (bytes == 0) return 0;
    OBJ_HIP(hipHostMalloc(h_out, bytes, hipHostMallocDefault),
            strf("hipHostMalloc(%llu)", (unsigned long long)bytes));
    return 0;
}

int32_t objeta_hip_free_pinned_host(objeta_hip_context* ctx, void* h_ptr) {
    OBJ_TRY(check_ctx(ctx, "pinned host free"));
    if (!h_ptr) return 0;
    OBJ_HIP(hipHostFree(h_ptr), "hipHostFree");
    return 0;
}

static int32_t copy_async(objeta_hip_context* ctx, objeta_hip_stream stream, void* dst,
                          const void* src, uint64_t bytes, hipMemcpyKind kind, const char* what) {
    OBJ_TRY(check_ctx(ctx, what));
    if (bytes == 0) return 0;
    if (!dst || !src) OBJ_FAIL(kInvalidInput, what, "NULL pointer");
    OBJ_HIP(hipSetDevice(ctx->device), "hipSetDevice");
    OBJ_HIP(hipMemcpyAsync(dst, src, bytes, kind, resolve_stream(ctx, stream)), what);
    return 0;
}

int32_t objeta_hip_copy_h2d(objeta_hip_context* ctx, objeta_hip_stream stream, void* d_dst,
                            const void* h_src, uint64_t bytes) {
    // pinned, 16-byte aligned sources through a kernel (copy.hip), the rest by HIP's copy
    if (ctx && d_dst && reinterpret_cast<uintptr_t>(d_dst) % 16 == 0) {
        OBJ_TRY(check_ctx(ctx, "copy host to device"));
        if (const void* src = objeta::pinned_device_ptr(h_src, bytes)) {
            OBJ_HIP(hipSetDevice(ctx->device), "hipSetDevice");
            return objeta::launch_h2d_copy(resolve_stream(ctx, stream), d_dst, src, bytes);
        }
    }
    return copy_async(ctx, stream, d_dst, h_src, bytes, hipMemcpyHostToDevice, "copy host to device");
}

int32_t objeta_hip_copy_d2h(objeta_hip_context* ctx, objeta_hip_stream stream, void* h_dst,
                            const void* d_src, uint64_t bytes) {
    return copy_async(ctx, stream, h_dst, d_src, bytes, hipMemcpyDeviceToHost, "copy device to host");
}

int32_t objeta_hip_copy_d2d(objeta_hip_context* ctx, objeta_hip_stream stream, void* d_dst,
                            const void* d_src, uint64_t bytes) {
    return copy_async(ctx, stream, d_dst, d_src, bytes, hipMemcpyDeviceToDevice, "copy device to device");
}

int32_t objeta_hip_event_create(objeta_hip_context* ctx, objeta_hip_event* out) {
    OBJ_TRY(check_ctx(ctx, "create event"));
    if (!out) OBJ_FAIL(kInvalidInput, "create event", "out is NULL");
    OBJ_HIP(hipSetDevice(ctx->device), "hipSetDevice");
    hipEvent_t ev = nullptr;
    OBJ_HIP(hipEventCreate(&ev), "create HIP event");
    *out = ev;
    return 0;
}

int32_t objeta_hip_event_record(objeta_hip_context* ctx, objeta_hip_event ev, objeta_hip_stream stream) {
    OBJ_TRY(check_ctx(ctx, "record event"));
    if (!ev) OBJ_FAIL(kInvalidInput, "record event", "event is NULL");
    OBJ_HIP(hipEventRecord(static_cast<hipEvent_t>(ev), resolve_stream(ctx, stream)), "record HIP event");
    return 0;
}

int32_t objeta_hip_event_elapsed_ms(objeta_hip_context* ctx, objeta_hip_event start,
                                    objeta_hip_event end, float* ms_out) {
    OBJ_TRY(check_ctx(ctx, "event elapsed time"));
    if (!start || !end || !ms_out) OBJ_FAIL(kInvalidInput, "event elapsed time", "NULL argument");
    OBJ_HIP(hipEventSynchronize(static_cast<hipEvent_t>(end)), "synchronize end event");
    OBJ_HIP(hipEventElapsedTime(ms_out, static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(end)),
            "measure HIP event elapsed time");
    return 0;
}

int32_t objeta_hip_event_destroy(objeta_hip_context* ctx, objeta_hip_event ev) {
    OBJ_TRY(check_ctx(ctx, "destroy event"));
    if (!ev) return 0;
    OBJ_HIP(hipEventDestroy(static_cast<hipEvent_t>(ev)), "destroy HIP event");
    return 0;
}

int32_t objeta_hip_graph_begin_capture(objeta_hip_context* ctx, objeta_hip_stream stream) {
    OBJ_TRY(check_ctx(ctx, "begin graph capture"));
    OBJ_HIP(hipSetDevice(ctx->device), "hipSetDevice");
    OBJ_HIP(hipStreamBeginCapture(resolve_stream(ctx, stream), hipStreamCaptureModeThreadLocal),
            "begin stream capture");
    return 0;
}

int32_t objeta_hip_graph_end_capture(objeta_hip_context* ctx, objeta_hip_stream stream,
                                     objeta_hip_graph* out) {
    OBJ_TRY(check_ctx(ctx, "end graph capture"));
    if (!out) OBJ_FAIL(kInvalidInput, "end graph capture", "out is NULL");
    *out = nullptr;
    hipGraph_t g = nullptr;
    OBJ_HIP(hipStreamEndCapture(resolve_stream(ctx, stream), &g), "end stream capture");
    hipGraphExec_t ex = nullptr;
    hipError_t e = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        OBJ_FAIL(kDriver, "instantiate graph", hipGetErrorString(e));
    }
    *out = ex;
    return 0;
}

int32_t objeta_hip_graph_launch(objeta_hip_context* ctx, objeta_hip_graph graph, objeta_hip_stream stream) {
    OBJ_TRY(check_ctx(ctx, "launch graph"));
    if (!graph) OBJ_FAIL(kInvalidInput, "launch graph", "graph is NULL");
    OBJ_HIP(hipGraphLaunch(static_cast<hipGraphExec_t>(graph), resolve_stream(ctx, stream)), "launch graph");
    return 0;
}

int32_t objeta_hip_graph_destroy(objeta_hip_context* ctx, objeta_hip_graph graph) {
    OBJ_TRY(check_ctx(ctx, "destroy graph"));
    if (!graph) return 0;
    OBJ_HIP(hipGraphExecDestroy(static_cast<hipGraphExec_t>(graph)), "destroy graph");
    return 0;
}

}  // extern "C"
