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
// memory) by hipMemcpyAsync. The misses of one call go in one launch of
// h2d_copy_batch_kernel, which copies them one after the other: launched one by one,
// consecutive copies were about 6 us apart.
#include <hip/hip_runtime.h>

#include "host_common.hpp"
#include "kernels.hpp"

namespace objeta {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// dst[i] = src[i] for i < n16 (16-byte units) by the gridDim.x workgroups of one
// grid row; four units of each thread in flight.
__device__ __forceinline__ void copy_units(u32x4* __restrict__ dst, const u32x4* __restrict__ src, size_t n16) {
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

__global__ __launch_bounds__(256) void h2d_copy_kernel(u32x4* __restrict__ dst, const u32x4* __restrict__ src,
                                                       size_t n16) {
    copy_units(dst, src, n16);
}

// Up to kH2dBatch copies in one launch, by value in the kernel arguments, one after
// the other: every workgroup copies its share of entry 0, then of entry 1, ... (as
// many reads in flight as one copy's launch, without a launch between copies).
struct H2dBatchArgs {
    u32x4* dst[kH2dBatch];
    const u32x4* src[kH2dBatch];
    uint64_t n16[kH2dBatch];
    uint32_t count;
};

__global__ __launch_bounds__(256) void h2d_copy_batch_kernel(H2dBatchArgs a) {
    for (uint32_t y = 0; y < a.count; ++y) copy_units(a.dst[y], a.src[y], a.n16[y]);
}

// about 32 KiB per workgroup, at most 64 workgroups per copy (the rate of a 1 MB copy
// was best at 32-64)
uint32_t copy_grid(size_t n) {
    size_t grid = (n + (32u << 10) - 1) >> 15;
    return static_cast<uint32_t>(grid < 1 ? 1 : (grid > 64 ? 64 : grid));
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
    hipLaunchKernelGGL(h2d_copy_kernel, dim3(copy_grid(n)), dim3(256), 0, s, static_cast<u32x4*>(dst),
                       static_cast<const u32x4*>(src_dev), n16);
    OBJ_HIP(hipGetLastError(), action);
    return 0;
}

int32_t launch_h2d_copy_batch(hipStream_t s, const H2dCopy* c, size_t n) {
    const char* action = "copy pinned host bytes to the device";
    for (size_t i = 0; i < n; ++i)
        if (!c[i].dst || !c[i].src_dev || reinterpret_cast<uintptr_t>(c[i].dst) % 16 ||
            reinterpret_cast<uintptr_t>(c[i].src_dev) % 16 || c[i].n % 16)
            OBJ_FAIL(kInvalidInput, action, "pointers and sizes must be 16-byte multiples");
    for (size_t i0 = 0; i0 < n; i0 += kH2dBatch) {
        const size_t m = n - i0 < static_cast<size_t>(kH2dBatch) ? n - i0 : static_cast<size_t>(kH2dBatch);
        H2dBatchArgs a{};
        size_t most = 0;
        for (size_t j = 0; j < m; ++j) {
            a.dst[j] = static_cast<u32x4*>(c[i0 + j].dst);
            a.src[j] = static_cast<const u32x4*>(c[i0 + j].src_dev);
            a.n16[j] = c[i0 + j].n / 16;
            most = c[i0 + j].n > most ? c[i0 + j].n : most;
        }
        a.count = static_cast<uint32_t>(m);
        hipLaunchKernelGGL(h2d_copy_batch_kernel, dim3(copy_grid(most)), dim3(256), 0, s, a);
        OBJ_HIP(hipGetLastError(), action);
    }
    return 0;
}

}  // namespace objeta
