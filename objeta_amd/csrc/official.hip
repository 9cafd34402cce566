// official.hip — the FP8-activation ("official arithmetic") DeepSeek path on gfx950.
//
// Replaces the act_quant, fp8_act_fp4_wt and fp8_act_fp8_wt kernels with their host
// paths cuda_act_quant_device / cuda_fp8_act_fp4_weight_gemv_device /
// cuda_fp8_act_fp8_weight_gemv_device (crates/objeta-cuda/src/quant.rs:1219-1362),
// and the per-expert launch chain of execute_selected_moe_official_routed_fp4_cuda
// (crates/objeta-cuda/src/moe.rs:1393-1663).
//
// Arithmetic follows the reference's CPU restatement (cpu_act_quant and the
// official expert compositions, crates/objeta-parser/src/deepseek.rs:1444-1716):
// act_quant emits the CPU's bytes exactly; the GEMVs multiply each weight by the
// dequantized activation act_v * act_s (an exact product: the scale is a power of
// two), so an FP8-activation GEMV is the float GEMV of the streaming engine over
// the dequantized vector. The official SwiGLU clamps only the up projection.
//
// act_quant layout: one wave per 128-element block, lane l holding elements 2l and
// 2l + 1; the block maximum is a wave max-reduction (exact in any order).
#include "device_common.hpp"
#include "gemv_stream.hpp"
#include "host_common.hpp"
#include "kernels.hpp"
#include "quant_rules.hpp"

namespace objeta {
namespace dev {

// n_blocks 128-element blocks of x; values / scales / deq each nullable. deq may
// alias x: every lane reads its two elements before any lane of the wave writes.
__global__ __launch_bounds__(kThreads) void act_quant_kernel(const float* x, uint64_t n_blocks,
                                                             uint8_t* __restrict__ values,
                                                             uint8_t* __restrict__ scales, float* deq) {
    const uint64_t b = static_cast<uint64_t>(blockIdx.x) * kWaves + (threadIdx.x >> 6);
    if (b >= n_blocks) return;
    const uint32_t lane = threadIdx.x & 63;
    const float2 v = reinterpret_cast<const float2*>(x + b * 128)[lane];
    // max |x| with NaN ignored (`if a > amax { amax = a }`), then the wave maximum
    float m = 0.0f;
    const float a0 = __builtin_fabsf(v.x), a1 = __builtin_fabsf(v.y);
    if (a0 > m) m = a0;
    if (a1 > m) m = a1;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float o = __shfl_xor(m, off, 64);
        m = o > m ? o : m;
    }
    const rules::Fp8ActScale sc = rules::fp8_act_scale(m);
    const uint8_t q0 = rules::fp8_act_code(v.x, sc.inv);
    const uint8_t q1 = rules::fp8_act_code(v.y, sc.inv);
    if (values)
        reinterpret_cast<uint16_t*>(values + b * 128)[lane] =
            static_cast<uint16_t>(q0 | (static_cast<uint32_t>(q1) << 8));
    if (scales && lane == 0) scales[b] = sc.raw;
    if (deq) {
        const float s = e8m0_to_f32(sc.raw);
        reinterpret_cast<float2*>(deq + b * 128)[lane] =
            make_float2(rules::f8e4m3_to_f32(q0) * s, rules::f8e4m3_to_f32(q1) * s);
    }
}

// deq[i] = f8e4m3(values[i]) * e8m0(scales[i / 128]), two elements per thread.
__global__ __launch_bounds__(kThreads) void fp8_dequant_kernel(const uint8_t* __restrict__ values,
                                                               const uint8_t* __restrict__ scales, uint64_t n2,
                                                               float* __restrict__ deq) {
    const uint64_t i = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (i >= n2) return;
    const uint32_t q = reinterpret_cast<const uint16_t*>(values)[i];
    const float s = e8m0_to_f32(scales[(2 * i) >> 7]);
    reinterpret_cast<float2*>(deq)[i] =
        make_float2(rules::f8e4m3_to_f32(q & 0xFFu) * s, rules::f8e4m3_to_f32(q >> 8) * s);
}

}  // namespace dev

using namespace dev;

int32_t launch_act_quant(hipStream_t s, const float* d_x, uint64_t rows, uint64_t cols, uint8_t* d_values,
                         uint8_t* d_scales, float* d_deq) {
    const char* action = "launch act_quant";
    if (cols % 128 != 0)
        OBJ_FAIL(kInvalidInput, action, strf("cols %llu not divisible by 128", (unsigned long long)cols));
    const uint64_t n_blocks = rows * (cols / 128);
    if (n_blocks == 0) return 0;
    if (!d_x) OBJ_FAIL(kInvalidInput, action, "NULL input pointer");
    if (!d_values && !d_scales && !d_deq) OBJ_FAIL(kInvalidInput, action, "no output requested");
    if (reinterpret_cast<uintptr_t>(d_x) % 8 || reinterpret_cast<uintptr_t>(d_deq) % 8 ||
        reinterpret_cast<uintptr_t>(d_values) % 2)
        OBJ_FAIL(kInvalidInput, action, "x and the dequantized output must be 8-byte, values 2-byte aligned");
    const uint64_t grid = (n_blocks + kWaves - 1) / kWaves;
    if (grid > 0xFFFFFFFFull) OBJ_FAIL(kInvalidInput, action, "too many blocks for one launch");
    hipLaunchKernelGGL(act_quant_kernel, dim3(static_cast<uint32_t>(grid)), dim3(kThreads), 0, s, d_x, n_blocks,
                       d_values, d_scales, d_deq);
    OBJ_HIP(hipGetLastError(), action);
    return 0;
}

int32_t launch_fp8_dequant(hipStream_t s, const uint8_t* d_values, const uint8_t* d_scales, uint64_t rows,
                           uint64_t cols, float* d_out) {
    const char* action = "launch FP8 activation dequantize";
    if (cols % 128 != 0)
        OBJ_FAIL(kInvalidInput, action, strf("cols %llu not divisible by 128", (unsigned long long)cols));
    const uint64_t n2 = rows * cols / 2;
    if (n2 == 0) return 0;
    if (!d_values || !d_scales || !d_out) OBJ_FAIL(kInvalidInput, action, "NULL device pointer");
    if (reinterpret_cast<uintptr_t>(d_values) % 2 || reinterpret_cast<uintptr_t>(d_out) % 8)
        OBJ_FAIL(kInvalidInput, action, "values must be 2-byte and the output 8-byte aligned");
    const uint64_t grid = (n2 + kThreads - 1) / kThreads;
    if (grid > 0xFFFFFFFFull) OBJ_FAIL(kInvalidInput, action, "too many elements for one launch");
    hipLaunchKernelGGL(fp8_dequant_kernel, dim3(static_cast<uint32_t>(grid)), dim3(kThreads), 0, s, d_values,
                       d_scales, n2, d_out);
    OBJ_HIP(hipGetLastError(), action);
    return 0;
}

namespace {

// Dequantized activations [batch][cols] in the stream's official-path workspace.
int32_t dequant_to_workspace(objeta_hip_context* ctx, hipStream_t s, const uint8_t* d_values,
                             const uint8_t* d_scales, uint64_t batch, uint64_t cols, float** out) {
    void* p = nullptr;
    OBJ_TRY(ensure_workspace(ctx, s, kWsOfficial, static_cast<size_t>(batch * cols) * sizeof(float) + 64, &p));
    *out = static_cast<float*>(p);
    return launch_fp8_dequant(s, d_values, d_scales, batch, cols, *out);
}

}  // namespace

}  // namespace objeta

using namespace objeta;

extern "C" {

int32_t objeta_hip_act_quant_fp8_device(objeta_hip_context* ctx, objeta_hip_stream stream, const float* d_x,
                                        uint64_t rows, uint64_t cols, uint8_t* d_values, uint8_t* d_scales,
                                        float* d_dequant) {
    OBJ_GUARD_BEGIN
    OBJ_TRY(check_ctx(ctx, "act_quant_fp8_device"));
    OBJ_HIP(hipSetDevice(ctx->device), "hipSetDevice");
    return launch_act_quant(resolve_stream(ctx, stream), d_x, rows, cols, d_values, d_scales, d_dequant);
    OBJ_GUARD_END
}

int32_t objeta_hip_fp8_act_fp4_weight_gemv_device(objeta_hip_context* ctx, objeta_hip_stream stream,
                                                  const uint8_t* d_act_values, const uint8_t* d_act_scales,
                                                  const uint8_t* d_weight, const uint8_t* d_weight_scales,
                                                  float* d_out, uint64_t rows, uint64_t k_logical, uint64_t batch) {
    OBJ_GUARD_BEGIN
    OBJ_TRY(check_ctx(ctx, "fp8_act_fp4_weight_gemv_device"));
    if (k_logical % 128 != 0)
        OBJ_FAIL(kInvalidInput, "fp8_act_fp4_weight_gemv_device",
                 strf("K_logical %llu must be multiple of 128", (unsigned long long)k_logical));
    if (rows == 0 || batch == 0) return 0;
    OBJ_HIP(hipSetDevice(ctx->device), "hipSetDevice");
    const hipStream_t s = resolve_stream(ctx, stream);
    float* xd = nullptr;
    OBJ_TRY(dequant_to_workspace(ctx, s, d_act_values, d_act_scales, batch, k_logical, &xd));
    return launch_fp4_split(ctx, s, d_weight, d_weight_scales, xd, d_out, rows, k_logical, batch);
    OBJ_GUARD_END
}

int32_t objeta_hip_fp8_act_fp8_weight_gemv_device(objeta_hip_context* ctx, objeta_hip_stream stream,
                                                  const uint8_t* d_act_values, const uint8_t* d_act_scales,
                                                  const uint8_t* d_weight, const uint8_t* d_weight_scales,
                                                  float* d_out, uint64_t rows, uint64_t k_logical, uint64_t batch) {
    OBJ_GUARD_BEGIN
    OBJ_TRY(check_ctx(ctx, "fp8_act_fp8_weight_gemv_device"));
    if (k_logical % 128 != 0)
        OBJ_FAIL(kInvalidInput, "fp8_act_fp8_weight_gemv_device",
                 strf("K_logical %llu must be multiple of 128", (unsigned long long)k_logical));
    if (rows == 0 || batch == 0) return 0;
    OBJ_HIP(hipSetDevice(ctx->device), "hipSetDevice");
    const hipStream_t s = resolve_stream(ctx, stream);
    float* xd = nullptr;
    OBJ_TRY(dequant_to_workspace(ctx, s, d_act_values, d_act_scales, batch, k_logical, &xd));
    return launch_fp8_rows(ctx, s, d_weight, d_weight_scales, xd, d_out, rows, k_logical, batch);
    OBJ_GUARD_END
}

}  // extern "C"
