// copy.hip — host-to-device copies of pinned host memory through a kernel.
//
// The expert cache's misses are host-to-device copies on the copy stream, each
// ordered after other streams' events (the block's last readers, the compute
// stream's position). On MI355X a DMA-engine copy that follows such a wait starts
// about 0.3 ms late, where a kernel that follows one starts within microseconds; a
// kernel reading the pinned source through its device mapping also moves a
// 0.6-1.2 MB tensor at 35-48 GB/s, against 30-39 GB/s for a DMA copy of that size
// with no wait at all (a 256 MiB copy reaches 57 GB/s either way). So pinned,
// 16-byte aligned sources are copied by h2d_copy_kernel; anything else (pageable
// memory) by hipMemcpyAsync.
#include <hip/hip_runtime.h>

#include "host_common.hpp"
#include "kernels.hpp"

namespace objeta {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// dst[i] = src[i] for i < n16 (16-byte units); four units of each thread in flight.
__global__ __launch_bounds__(256) void h2d_copy_kernel(u32x4* __restrict__ dst, const u32x4* __restrict__ src,
                                                       size_t n16) {
    const size_t stride = static_cast<size_t>(gridDim.x) * 256;
    size_t i = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x;
    for (; i + 3 * stride < n16; i += 4 * stride) {
        const u32x4 a = __builtin_nontemporal_load(src + i);
        const u32x4 b = __builtin_nontemporal_load(src + i + stride);
        const u32x4 c = __builtin_nontemporal_load(src + i + 2 * stride);
        const u32x4 d = __builtin_nontemporal_load(src + i + 3 * stride);
        dst[i] = a;
        dst[i + stride] = b;
        dst[i + 2 * stride] = c;
        dst[i + 3 * stride] = d;
    }
    for (; i < n16; i += stride) dst[i] = __builtin_nontemporal_load(src + i);
}

}  // namespace

const void* pinned_device_ptr(const void* h, size_t n) {
    if (!h || n == 0 || reinterpret_cast<uintptr_t>(h) % 16 || n % 16) return nullptr;
    hipPointerAttribute_t a{};
    if (hipPointerGetAttributes(&a, h) != hipSuccess) {
        (void)hipGetLastError();  // pageable memory: not an error of the caller's
        return nullptr;
    }
    if (a.type != hipMemoryTypeHost || !a.devicePointer || reinterpret_cast<uintptr_t>(a.devicePointer) % 16)
        return nullptr;
    return a.devicePointer;
}

int32_t launch_h2d_copy(hipStream_t s, void* dst, const void* src_dev, size_t n) {
    const char* action = "copy pinned host bytes to the device";
    if (n == 0) return 0;
    if (!dst || !src_dev || reinterpret_cast<uintptr_t>(dst) % 16 || reinterpret_cast<uintptr_t>(src_dev) % 16 ||
        n % 16)
        OBJ_FAIL(kInvalidInput, action, "pointers and size must be 16-byte multiples");
    const size_t n16 = n / 16;
    // about 32 KiB per workgroup, at most 64 workgroups (the rate of a 1 MB copy was
    // best at 32-64)
    size_t grid = (n + (32u << 10) - 1) >> 15;
    grid = grid < 1 ? 1 : (grid > 64 ? 64 : grid);
    hipLaunchKernelGGL(h2d_copy_kernel, dim3(static_cast<uint32_t>(grid)), dim3(256), 0, s,
                       static_cast<u32x4*>(dst), static_cast<const u32x4*>(src_dev), n16);
    OBJ_HIP(hipGetLastError(), action);
    return 0;
}

}  // namespace objeta
