// host_common.hpp — host-side plumbing shared by the C-ABI translation units:
// the per-thread error record, HIP error mapping and the context object.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <mutex>
#include <new>
#include <string>
#include <vector>

#include "../../include/objeta_hip.h"

namespace objeta {

// CudaErrorKind ordinals (crates/objeta-cuda/src/lib.rs:39-48).
enum Kind : int32_t {
    kDriver = 0,
    kRuntime = 1,
    kNvrtc = 2,
    kIo = 3,
    kInvalidInput = 4,
    kUnsupported = 5,
    kInternal = 6
};

// Records the error for this thread and returns its status (kind + 1).
int32_t set_error(Kind kind, const char* file, unsigned line, const char* module,
                  const std::string& action, const std::string& message);
std::string strf(const char* fmt, ...) __attribute__((format(printf, 1, 2)));

#define OBJ_FAIL(kind, action, msg) \
    return ::objeta::set_error((kind), __FILE__, __LINE__, __func__, (action), (msg))

#define OBJ_HIP(call, action)                                                          \
    do {                                                                               \
        hipError_t e_ = (call);                                                        \
        if (e_ != hipSuccess) {                                                        \
            (void)hipGetLastError();                                                   \
            return ::objeta::set_error(::objeta::kDriver, __FILE__, __LINE__, __func__, \
                                       (action), hipGetErrorString(e_));               \
        }                                                                              \
    } while (0)

#define OBJ_TRY(expr)               \
    do {                            \
        int32_t rc_ = (expr);       \
        if (rc_ != 0) return rc_;   \
    } while (0)

// Wraps a C entry point body so that no C++ exception crosses the C boundary.
#define OBJ_GUARD_BEGIN try {
#define OBJ_GUARD_END                                                                  \
    }                                                                                  \
    catch (const std::bad_alloc&) {                                                    \
        return ::objeta::set_error(::objeta::kInternal, __FILE__, __LINE__, __func__,  \
                                   "host allocation", "std::bad_alloc");              \
    }                                                                                  \
    catch (const std::exception& ex) {                                                 \
        return ::objeta::set_error(::objeta::kInternal, __FILE__, __LINE__, __func__,  \
                                   "host exception", ex.what());                      \
    }

// Device scratch owned by the context, one region per purpose. A region grows
// only outside graph capture, and a replaced region stays allocated until the
// context is destroyed, so graphs captured earlier keep valid pointers.
struct Workspace {
    void* ptr = nullptr;
    size_t bytes = 0;
};
enum WsSlot : int {
    kWsRouter = 0,
    kWsMoeAct = 1,
    kWsMoeTable = 2,
    kWsGrouped = 3,
    kWsSelTab = 4,
    kWsOfficial = 5,  // dequantized FP8 activations of the official path
    kWsGemv = 6,      // split activations and partial sums of the batched MFMA GEMV
    kWsStack = 7,     // routing results and expert tables of the cached decode stack
    kWsSlots = 8
};

// The scratch of one stream. Calls on different streams of a context may be in
// flight at the same time, so every stream that a call names gets its own
// workspace regions and its own router epoch counters (created on the first call
// on that stream made outside graph capture).
struct StreamScratch {
    hipStream_t stream = nullptr;
    Workspace ws[kWsSlots];
    uint32_t* epochs = nullptr;  // kEpochWords zero-initialised router counters, one per token
};
constexpr size_t kEpochWords = 4096;

}  // namespace objeta

struct objeta_hip_context {
    int device = 0;
    objeta_hip_device_info info{};
    std::vector<hipStream_t> streams;  // streams[0] is the default compute stream
    hipStream_t copy_stream = nullptr;  // side stream for cache H2D traffic
    std::vector<objeta::StreamScratch*> scratch;  // per-stream scratch, see StreamScratch
    std::vector<void*> retired_ws;                // replaced regions, freed at destroy
    void* host_stage = nullptr;                   // pinned host staging (expert tables)
    void* transient_pool = nullptr;               // objeta_hip_expert_cache for uncached copies
    std::vector<void*> caches;                    // live caches created on this context
    size_t host_stage_bytes = 0;
    uint32_t* err_word = nullptr;  // device error word (bits set by kernels, read by objeta_hip_device_error)
    // polls of the router's selecting workgroup before it computes the missing logits
    // itself (OBJETA_HIP_ROUTER_SPIN_LIMIT at init; default about a second)
    uint32_t router_spin_limit = 1u << 20;
    float* static_act = nullptr;   // device address of this device's static activation scratch
    std::mutex mu;
};

namespace objeta {

int32_t check_ctx(const objeta_hip_context* ctx, const char* action);
hipStream_t resolve_stream(objeta_hip_context* ctx, objeta_hip_stream s);
// The scratch of `stream` (created on first use; Unsupported while `stream` is
// capturing and has none yet).
int32_t stream_scratch(objeta_hip_context* ctx, hipStream_t stream, StreamScratch** out);
// Makes sure workspace region `slot` of `stream` holds at least `bytes` and returns
// it in *out; fails (Unsupported) if it would have to grow while `stream` is capturing.
int32_t ensure_workspace(objeta_hip_context* ctx, hipStream_t stream, int slot, size_t bytes, void** out);
// Releases the device memory of every cache still alive on `ctx` (the caches stay
// valid as accounting-only objects until destroyed).
void detach_caches(objeta_hip_context* ctx);
// Pinned host staging of at least `bytes` (grown outside capture only).
int32_t ensure_host_stage(objeta_hip_context* ctx, size_t bytes, void** out);

}  // namespace objeta
