// quantize.hip — device weight packing (bit-identical to quantize_matrix_cpu,
// crates/objeta-cuda/src/quant.rs:506-926), synthetic input generators, and a
// graph-safe zero fill.
#include "host_common.hpp"
#include "kernels.hpp"
#include "quant_rules.hpp"

namespace objeta {
namespace {

constexpr int kThreads = 256;

template <int F>
__device__ __forceinline__ void quantize_one(const float* v, uint8_t* dst) {
    if constexpr (F == 0) rules::q4_block(v, dst);
    else if constexpr (F == 1) rules::q5_block(v, dst);
    else if constexpr (F == 2) rules::iq3_block(v, dst);
    else rules::fp4_block(v, dst);
}

constexpr int block_bytes_of(int f) { return f == 0 ? 18 : f == 1 ? 22 : f == 2 ? 14 : 17; }

// One thread per 32-value block.
template <int F>
__global__ __launch_bounds__(kThreads) void quantize_matrix_kernel(const float* __restrict__ m,
                                                                   uint8_t* __restrict__ out,
                                                                   uint64_t n_blocks) {
    const uint64_t b = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (b >= n_blocks) return;
    float v[32];
    const float4* src = reinterpret_cast<const float4*>(m + b * 32);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float4 t = src[i];
        v[4 * i] = t.x; v[4 * i + 1] = t.y; v[4 * i + 2] = t.z; v[4 * i + 3] = t.w;
    }
    uint8_t blk[block_bytes_of(F)];
    quantize_one<F>(v, blk);
    uint8_t* dst = out + b * block_bytes_of(F);
#pragma unroll
    for (int i = 0; i < block_bytes_of(F); ++i) dst[i] = blk[i];
}

// Unaligned input fallback (element loads).
template <int F>
__global__ __launch_bounds__(kThreads) void quantize_matrix_kernel_u(const float* __restrict__ m,
                                                                     uint8_t* __restrict__ out,
                                                                     uint64_t n_blocks) {
    const uint64_t b = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (b >= n_blocks) return;
    float v[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) v[i] = m[b * 32 + i];
    uint8_t blk[block_bytes_of(F)];
    quantize_one<F>(v, blk);
    uint8_t* dst = out + b * block_bytes_of(F);
#pragma unroll
    for (int i = 0; i < block_bytes_of(F); ++i) dst[i] = blk[i];
}

template <int F>
__global__ __launch_bounds__(kThreads) void gauss_quantized_kernel(uint8_t* __restrict__ out,
                                                                   uint64_t n_blocks, uint64_t key,
                                                                   float sigma) {
    const uint64_t b = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (b >= n_blocks) return;
    float v[32];
#pragma unroll 4
    for (int i = 0; i < 32; ++i) v[i] = rules::gauss_from_key(key, b * 32 + i, sigma);
    uint8_t blk[block_bytes_of(F)];
    quantize_one<F>(v, blk);
    uint8_t* dst = out + b * block_bytes_of(F);
#pragma unroll
    for (int i = 0; i < block_bytes_of(F); ++i) dst[i] = blk[i];
}

__global__ __launch_bounds__(kThreads) void gauss_kernel(float* __restrict__ out, uint64_t n,
                                                         uint64_t key, uint64_t first, float sigma) {
    const uint64_t i = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (i >= n) return;
    out[i] = rules::gauss_from_key(key, first + i, sigma);
}

// One split FP4 matrix of synthetic bytes: weight byte i is byte (i mod 8) of
// splitmix64(kw + i / 8) (nibbles uniform over the 16 E2M1 codes), scale byte i is
// 119 + splitmix64(ks + i) mod 9 (E8M0 2^-8 .. 2^0). Thread t writes weight word t
// and scale byte t.
__global__ __launch_bounds__(kThreads) void fp4_split_random_kernel(uint8_t* __restrict__ w, uint8_t* __restrict__ sc,
                                                                    uint64_t n_w, uint64_t n_s, uint64_t kw,
                                                                    uint64_t ks) {
    const uint64_t t = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x;
    const uint64_t i0 = t * 8;
    if (i0 < n_w) {
        const uint64_t v = rules::splitmix64(kw + t);
        for (uint32_t b = 0; b < 8 && i0 + b < n_w; ++b) w[i0 + b] = static_cast<uint8_t>(v >> (8 * b));
    }
    if (t < n_s) sc[t] = static_cast<uint8_t>(119u + static_cast<uint32_t>(rules::splitmix64(ks + t) % 9u));
}

__global__ __launch_bounds__(kThreads) void zero_kernel(uint32_t* __restrict__ d, uint64_t words) {
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x; i < words;
         i += static_cast<uint64_t>(gridDim.x) * kThreads)
        d[i] = 0u;
}

__global__ void zero_bytes_kernel(uint8_t* __restrict__ d, uint64_t n) {
    const uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) d[i] = 0;
}

dim3 grid_for(uint64_t n) { return dim3(static_cast<uint32_t>((n + kThreads - 1) / kThreads)); }

}  // namespace

int32_t launch_zero(hipStream_t s, void* d, uint64_t bytes) {
    if (bytes == 0) return 0;
    if (!d) OBJ_FAIL(kInvalidInput, "zero device memory", "NULL device pointer");
    uint8_t* p = static_cast<uint8_t*>(d);
    const uint64_t head = (4 - (reinterpret_cast<uintptr_t>(p) & 3)) & 3;
    const uint64_t h = head < bytes ? head : bytes;
    if (h) hipLaunchKernelGGL(zero_bytes_kernel, dim3(1), dim3(64), 0, s, p, h);
    const uint64_t words = (bytes - h) / 4;
    if (words) {
        uint64_t blocks = (words + kThreads - 1) / kThreads;
        if (blocks > 65535) blocks = 65535;
        hipLaunchKernelGGL(zero_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(kThreads), 0, s,
                           reinterpret_cast<uint32_t*>(p + h), words);
    }
    const uint64_t tail = bytes - h - words * 4;
    if (tail) hipLaunchKernelGGL(zero_bytes_kernel, dim3(1), dim3(64), 0, s, p + h + words * 4, tail);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) OBJ_FAIL(kDriver, "launch zero fill", hipGetErrorString(e));
    return 0;
}

}  // namespace objeta

using namespace objeta;

extern "C" {

int32_t objeta_hip_zero_device(objeta_hip_context* ctx, objeta_hip_stream stream, void* d_dst, uint64_t bytes) {
    OBJ_GUARD_BEGIN
    OBJ_TRY(check_ctx(ctx, "zero device memory"));
    OBJ_HIP(hipSetDevice(ctx->device), "hipSetDevice");
    return launch_zero(resolve_stream(ctx, stream), d_dst, bytes);
    OBJ_GUARD_END
}

int32_t objeta_hip_quantize_matrix_device(objeta_hip_context* ctx, int32_t format, objeta_hip_stream stream,
                                          const float* d_m, uint64_t rows, uint64_t cols, void* d_out) {
    OBJ_GUARD_BEGIN
    OBJ_TRY(check_ctx(ctx, "quantize_matrix_device"));
    if (objeta_hip_block_bytes(format) < 0)
        OBJ_FAIL(kInvalidInput, "validate format", strf("unknown format %d", format));
    if (cols % 32 != 0)
        OBJ_FAIL(kInvalidInput, "validate column alignment",
                 strf("cols %llu must be a multiple of block_size 32", (unsigned long long)cols));
    const uint64_t nb = rows * (cols / 32);
    if (nb == 0) return 0;
    if (!d_m || !d_out) OBJ_FAIL(kInvalidInput, "quantize_matrix_device", "NULL device pointer");
    OBJ_HIP(hipSetDevice(ctx->device), "hipSetDevice");
    hipStream_t s = resolve_stream(ctx, stream);
    uint8_t* out = static_cast<uint8_t*>(d_out);
    const bool al = reinterpret_cast<uintptr_t>(d_m) % 16 == 0;
    const dim3 g = grid_for(nb);
    switch (format) {
#define OBJ_Q(F)                                                                                  \
    if (al) hipLaunchKernelGGL(quantize_matrix_kernel<F>, g, dim3(kThreads), 0, s, d_m, out, nb); \
    else hipLaunchKernelGGL(quantize_matrix_kernel_u<F>, g, dim3(kThreads), 0, s, d_m, out, nb);   \
    break;
        case 0: OBJ_Q(0)
        case 1: OBJ_Q(1)
        case 2: OBJ_Q(2)
        default: OBJ_Q(3)
#undef OBJ_Q
    }
    OBJ_HIP(hipGetLastError(), "launch quantize_matrix kernel");
    return 0;
    OBJ_GUARD_END
}

int32_t objeta_hip_fill_gauss_device(objeta_hip_context* ctx, objeta_hip_stream stream, float* d_out, uint64_t n,
                                     uint64_t seed, uint64_t first, float sigma) {
    OBJ_GUARD_BEGIN
    OBJ_TRY(check_ctx(ctx, "fill_gauss_device"));
    if (n == 0) return 0;
    if (!d_out) OBJ_FAIL(kInvalidInput, "fill_gauss_device", "NULL device pointer");
    OBJ_HIP(hipSetDevice(ctx->device), "hipSetDevice");
    hipLaunchKernelGGL(gauss_kernel, grid_for(n), dim3(kThreads), 0, resolve_stream(ctx, stream), d_out, n,
                       rules::splitmix64(seed), first, sigma);
    OBJ_HIP(hipGetLastError(), "launch gauss kernel");
    return 0;
    OBJ_GUARD_END
}

int32_t objeta_hip_fill_gauss_quantized_device(objeta_hip_context* ctx, int32_t format, objeta_hip_stream stream,
                                               void* d_out, uint64_t rows, uint64_t cols, uint64_t seed,
                                               float sigma) {
    OBJ_GUARD_BEGIN
    OBJ_TRY(check_ctx(ctx, "fill_gauss_quantized_device"));
    if (objeta_hip_block_bytes(format) < 0)
        OBJ_FAIL(kInvalidInput, "validate format", strf("unknown format %d", format));
    if (cols % 32 != 0)
        OBJ_FAIL(kInvalidInput, "validate column alignment",
                 strf("cols %llu must be a multiple of block_size 32", (unsigned long long)cols));
    const uint64_t nb = rows * (cols / 32);
    if (nb == 0) return 0;
    if (!d_out) OBJ_FAIL(kInvalidInput, "fill_gauss_quantized_device", "NULL device pointer");
    OBJ_HIP(hipSetDevice(ctx->device), "hipSetDevice");
    hipStream_t s = resolve_stream(ctx, stream);
    uint8_t* out = static_cast<uint8_t*>(d_out);
    const uint64_t key = rules::splitmix64(seed);
    const dim3 g = grid_for(nb);
    switch (format) {
        case 0: hipLaunchKernelGGL(gauss_quantized_kernel<0>, g, dim3(kThreads), 0, s, out, nb, key, sigma); break;
        case 1: hipLaunchKernelGGL(gauss_quantized_kernel<1>, g, dim3(kThreads), 0, s, out, nb, key, sigma); break;
        case 2: hipLaunchKernelGGL(gauss_quantized_kernel<2>, g, dim3(kThreads), 0, s, out, nb, key, sigma); break;
        default: hipLaunchKernelGGL(gauss_quantized_kernel<3>, g, dim3(kThreads), 0, s, out, nb, key, sigma); break;
    }
    OBJ_HIP(hipGetLastError(), "launch gauss_quantized kernel");
    return 0;
    OBJ_GUARD_END
}

// Host evaluation of the E8M0 exponent rule used by the device FP4 quantizer, so
// the rule can be checked against the CPU reference over every float.
int32_t objeta_hip_fill_fp4_split_device(objeta_hip_context* ctx, objeta_hip_stream stream, void* d_w, void* d_s,
                                         uint64_t rows, uint64_t cols, uint64_t seed) {
    OBJ_GUARD_BEGIN
    OBJ_TRY(check_ctx(ctx, "fill_fp4_split_device"));
    if (cols % 32 != 0)
        OBJ_FAIL(kInvalidInput, "fill_fp4_split_device",
                 strf("cols %llu must be a multiple of block_size 32", (unsigned long long)cols));
    const uint64_t n_w = rows * cols / 2, n_s = rows * cols / 32;
    if (n_w == 0) return 0;
    if (!d_w || !d_s) OBJ_FAIL(kInvalidInput, "fill_fp4_split_device", "NULL device pointer");
    OBJ_HIP(hipSetDevice(ctx->device), "hipSetDevice");
    const uint64_t threads = (n_w + 7) / 8 > n_s ? (n_w + 7) / 8 : n_s;
    hipLaunchKernelGGL(fp4_split_random_kernel, grid_for(threads), dim3(kThreads), 0, resolve_stream(ctx, stream),
                       static_cast<uint8_t*>(d_w), static_cast<uint8_t*>(d_s), n_w, n_s, rules::splitmix64(seed),
                       rules::splitmix64(seed ^ 0x5CA1E5CA1E5CA1E5ull));
    OBJ_HIP(hipGetLastError(), "launch fp4 split fill");
    return 0;
    OBJ_GUARD_END
}

int32_t objeta_hip_fp4_scale_raw_host(const float* amax, uint8_t* out, uint64_t n) {
    if (n && (!amax || !out)) OBJ_FAIL(kInvalidInput, "fp4_scale_raw_host", "NULL pointer");
    for (uint64_t i = 0; i < n; ++i) out[i] = rules::fp4_scale_raw(amax[i]);
    return 0;
}

}  // extern "C"
