// qgemv.hip — block-dequant GEMV for Q4_0 / Q5_0 / IQ3_0 / FP4-E2M1 on gfx950.
//
// Replaces q4_gemv_f32_accum / q5_gemv_f32_accum / iq3_gemv_f32_accum /
// fp4_e2m1_gemv / fp4_e2m1_gemv_split (crates/objeta-cuda/kernels/*.cu) and the
// host paths QuantBackend::gemv / launch_kernel / launch_kernel_split_fp4
// (crates/objeta-cuda/src/quant.rs:256-408).
//
// Fast path (cols % 64 == 0, 4-byte aligned weights): a wave64 lane owns one
// *pair* of consecutive blocks (36 / 44 / 28 bytes, always 4-byte aligned) and
// streams it with dwordx4 loads; consecutive lanes own consecutive pairs, so a
// wave reads contiguous bytes. A lane keeps U rows of the same pair in flight and
// reuses each activation read from LDS across them. Activations are staged once
// per workgroup in LDS with 4 floats of padding per 64 so that lanes reading
// different pairs hit different banks. Row sums are reduced across the lanes of
// a row with DPP/permute shuffles.
#include "device_common.hpp"
#include "host_common.hpp"
#include "gemv_stream.hpp"
#include "kernels.hpp"

#include <cstdlib>

namespace objeta {
namespace dev {

// Generic path: any cols % 32 == 0 and any alignment, including the interleaved
// 17-byte FP4 layout. One wave per row, lanes stride over blocks, byte loads.
template <int F, int NT>
__global__ __launch_bounds__(kThreads) void qgemv_generic(const uint8_t* __restrict__ q,
                                                          const float* __restrict__ x,
                                                          float* __restrict__ y, uint32_t rows,
                                                          uint32_t cols) {
    constexpr int BB = Fmt<F>::kBlockBytes;
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t row = blockIdx.x * kWaves + (threadIdx.x >> 6);
    if (row >= rows) return;
    const uint32_t nb = cols >> 5;
    const uint8_t* rq = q + static_cast<size_t>(row) * nb * BB;
    float acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = 0.f;
    for (uint32_t b = lane; b < nb; b += 64) {
        const uint8_t* blk = rq + static_cast<size_t>(b) * BB;
        float scale;
        if constexpr (F == kFP4) scale = e8m0_to_f32(blk[0]);
        else scale = f16_to_f32(static_cast<uint32_t>(blk[0]) | (static_cast<uint32_t>(blk[1]) << 8));
        for (int i = 0; i < 32; ++i) {
            float w;
            if constexpr (F == kQ4) {
                const uint32_t pk = blk[2 + i / 2];
                w = static_cast<float>(static_cast<int>((i & 1) ? (pk >> 4) : (pk & 15)) - 8);
            } else if constexpr (F == kQ5) {
                const uint32_t pk = blk[6 + i / 2];
                const uint32_t lo = (i & 1) ? (pk >> 4) : (pk & 15);
                const uint32_t hi = (blk[2 + i / 8] >> (i & 7)) & 1u;
                w = static_cast<float>(static_cast<int>(lo | (hi << 4)) - 16);
            } else if constexpr (F == kIQ3) {
                const uint32_t lo = (blk[2 + i / 4] >> (2 * (i & 3))) & 3u;
                const uint32_t hi = (blk[10 + i / 8] >> (i & 7)) & 1u;
                w = static_cast<float>(static_cast<int>(lo | (hi << 2)) - 4);
            } else {
                const uint32_t pk = blk[1 + i / 2];
                const uint32_t c = (i & 1) ? (pk >> 4) : (pk & 15);
                w = f16_to_f32(((c & 7u) << 9) | ((c & 8u) << 12)) * 16384.0f;
            }
            // the reference's w = value * scale, then sum += w * x (quant.rs:928-1019)
            w *= scale;
#pragma unroll
            for (int t = 0; t < NT; ++t)
                acc[t] = __builtin_fmaf(w, x[static_cast<size_t>(t) * cols + b * 32 + i], acc[t]);
        }
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const float v = wave_reduce(acc[t]);
        if (lane == 0) y[static_cast<size_t>(t) * rows + row] = v;
    }
}

template <int NT>
__global__ __launch_bounds__(kThreads) void fp4_split_generic(const uint8_t* __restrict__ w,
                                                              const uint8_t* __restrict__ sc,
                                                              const float* __restrict__ x,
                                                              float* __restrict__ y, uint32_t rows,
                                                              uint32_t cols) {
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t row = blockIdx.x * kWaves + (threadIdx.x >> 6);
    if (row >= rows) return;
    const uint32_t nb = cols >> 5;
    const uint8_t* rw = w + static_cast<size_t>(row) * (cols >> 1);
    const uint8_t* rs = sc + static_cast<size_t>(row) * nb;
    float acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = 0.f;
    for (uint32_t b = lane; b < nb; b += 64) {
        const float scale = e8m0_to_f32(rs[b]);
        for (int i = 0; i < 32; ++i) {
            const uint32_t pk = rw[b * 16 + i / 2];
            const uint32_t c = (i & 1) ? (pk >> 4) : (pk & 15);
            const float wv = f16_to_f32(((c & 7u) << 9) | ((c & 8u) << 12)) * 16384.0f * scale;
#pragma unroll
            for (int t = 0; t < NT; ++t)
                acc[t] = __builtin_fmaf(wv, x[static_cast<size_t>(t) * cols + b * 32 + i], acc[t]);
        }
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const float v = wave_reduce(acc[t]);
        if (lane == 0) y[static_cast<size_t>(t) * rows + row] = v;
    }
}

}  // namespace dev

// ------------------------------------------------------------------ launchers
namespace {

using namespace dev;

constexpr int kStreamWgsPerCu = 4;  // resident workgroups per CU for the streaming GEMV

// Persistent grid: enough workgroups to cover every group once, capped at
// `per_cu` workgroups per compute unit so that each wave streams several items.
template <typename K>
uint32_t grid_for_stream(const objeta_hip_context* ctx, K kernel, size_t lds, uint32_t n_groups) {
    const uint32_t cus = ctx->info.compute_units > 0 ? static_cast<uint32_t>(ctx->info.compute_units) : 256u;
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, kThreads, lds) != hipSuccess || per_cu < 1)
        per_cu = 1;
    if (per_cu > kStreamWgsPerCu) per_cu = kStreamWgsPerCu;
    const uint32_t need = (n_groups + kWaves - 1) / kWaves;
    const uint32_t cap = cus * static_cast<uint32_t>(per_cu);
    return need < cap ? need : cap;
}

template <class R, int NT, int U>
hipError_t launch_stream_u(const objeta_hip_context* ctx, hipStream_t s, const R& rm, const float* x, float* y,
                           uint32_t rows, uint32_t cols, uint32_t lpr, size_t lds) {
    const uint32_t g = 64 / lpr;
    const uint32_t n_groups = (rows + g * U - 1) / (g * U);
    auto kern = gemv_stream<R, NT, U>;
    const uint32_t grid = grid_for_stream(ctx, kern, lds, n_groups);
    hipLaunchKernelGGL(kern, dim3(grid), dim3(kThreads), lds, s, rm, x, y, rows, cols, lpr, n_groups);
    return hipGetLastError();
}

// One row group per wave item: the streaming grid already keeps every resident
// wave busy at the shapes of the MoE layers (two rows per item measured no faster).
template <class R, int NT>
hipError_t launch_stream(const objeta_hip_context* ctx, hipStream_t s, const R& rm, const float* x, float* y,
                         uint32_t rows, uint32_t cols, uint32_t lpr, size_t lds) {
    return launch_stream_u<R, NT, 1>(ctx, s, rm, x, y, rows, cols, lpr, lds);
}

template <int F>
hipError_t launch_generic(hipStream_t s, const uint8_t* q, const float* x, float* y, uint32_t rows,
                          uint32_t cols, int nt) {
    const dim3 grid((rows + kWaves - 1) / kWaves);
    switch (nt) {
        case 8: hipLaunchKernelGGL((qgemv_generic<F, 8>), grid, dim3(kThreads), 0, s, q, x, y, rows, cols); break;
        case 4: hipLaunchKernelGGL((qgemv_generic<F, 4>), grid, dim3(kThreads), 0, s, q, x, y, rows, cols); break;
        case 2: hipLaunchKernelGGL((qgemv_generic<F, 2>), grid, dim3(kThreads), 0, s, q, x, y, rows, cols); break;
        default: hipLaunchKernelGGL((qgemv_generic<F, 1>), grid, dim3(kThreads), 0, s, q, x, y, rows, cols); break;
    }
    return hipGetLastError();
}

int max_nt_for_lds(size_t per_token, size_t limit, uint64_t remaining) {
    for (int nt : {8, 4, 2, 1})
        if (static_cast<uint64_t>(nt) <= remaining && per_token * nt <= limit) return nt;
    return 0;
}

}  // namespace

int32_t launch_qgemv(objeta_hip_context* ctx, int32_t format, hipStream_t s, const void* d_q,
                     const float* d_x, float* d_y, uint64_t rows, uint64_t cols, uint64_t batch) {
    const char* action = "launch quantized GEMV";
    if (objeta_hip_block_bytes(format) < 0) OBJ_FAIL(kInvalidInput, action, strf("unknown format %d", format));
    if (cols % 32 != 0)
        OBJ_FAIL(kInvalidInput, action, strf("cols %llu must be a multiple of block_size 32", (unsigned long long)cols));
    if (rows == 0 || batch == 0) return 0;
    if (!d_q || !d_x || !d_y) OBJ_FAIL(kInvalidInput, action, "NULL device pointer");
    if (rows > 0x7FFFFFFFull || cols > 0x7FFFFFFFull)
        OBJ_FAIL(kInvalidInput, action, "rows/cols exceed 2^31");
    // several vectors: each weight decoded once for all of them, on the matrix cores
    if (format != OBJETA_HIP_FP4_E2M1 && gemv_mfma_supported(format, rows, cols, batch, d_q, d_x))
        return launch_gemv_mfma(ctx, s, format, d_q, nullptr, d_x, d_y, rows, cols, batch);
    const uint32_t r = static_cast<uint32_t>(rows), c = static_cast<uint32_t>(cols);
    const uint8_t* q = static_cast<const uint8_t*>(d_q);
    const bool aligned = (reinterpret_cast<uintptr_t>(q) % 4 == 0) && (reinterpret_cast<uintptr_t>(d_x) % 16 == 0);
    const bool fast = format != OBJETA_HIP_FP4_E2M1 && cols % 64 == 0 && aligned && pick_lpr(c / 64) != 0;
    const size_t lds_limit = 65536;  // at most 64 KB of staged activations per workgroup
    uint64_t done = 0;
    while (done < batch) {
        const uint64_t rem = batch - done;
        const float* xb = d_x + done * cols;
        float* yb = d_y + done * rows;
        hipError_t e = hipSuccess;
        int nt;
        if (fast) {
            const uint32_t pairs = c / 64;
            const uint32_t lpr = pick_lpr(pairs);
            const size_t per_token = static_cast<size_t>(pairs) * kPad * sizeof(float);
            nt = max_nt_for_lds(per_token, lds_limit, rem);
            if (nt == 0) OBJ_FAIL(kUnsupported, action, strf("cols %u exceed the LDS activation stage", c));
            const size_t lds = per_token * nt + 4 * sizeof(float);
            const size_t row_bytes = static_cast<size_t>(c / 32) * static_cast<size_t>(objeta_hip_block_bytes(format));
#define OBJ_FAST(F)                                                                              \
    {                                                                                            \
        const QRows<F> rm{q, row_bytes};                                                         \
        switch (nt) {                                                                            \
            case 8: e = launch_stream<QRows<F>, 8>(ctx, s, rm, xb, yb, r, c, lpr, lds); break;   \
            case 4: e = launch_stream<QRows<F>, 4>(ctx, s, rm, xb, yb, r, c, lpr, lds); break;   \
            case 2: e = launch_stream<QRows<F>, 2>(ctx, s, rm, xb, yb, r, c, lpr, lds); break;   \
            default: e = launch_stream<QRows<F>, 1>(ctx, s, rm, xb, yb, r, c, lpr, lds); break;  \
        }                                                                                        \
    }
            if (format == OBJETA_HIP_Q4_0) OBJ_FAST(kQ4)
            else if (format == OBJETA_HIP_Q5_0) OBJ_FAST(kQ5)
            else OBJ_FAST(kIQ3)
#undef OBJ_FAST
        } else {
            nt = rem >= 8 ? 8 : rem >= 4 ? 4 : rem >= 2 ? 2 : 1;
            switch (format) {
                case OBJETA_HIP_Q4_0: e = launch_generic<kQ4>(s, q, xb, yb, r, c, nt); break;
                case OBJETA_HIP_Q5_0: e = launch_generic<kQ5>(s, q, xb, yb, r, c, nt); break;
                case OBJETA_HIP_IQ3_0: e = launch_generic<kIQ3>(s, q, xb, yb, r, c, nt); break;
                default: e = launch_generic<kFP4>(s, q, xb, yb, r, c, nt); break;
            }
        }
        if (e != hipSuccess) OBJ_FAIL(kDriver, action, hipGetErrorString(e));
        done += static_cast<uint64_t>(nt);
    }
    return 0;
}

int32_t launch_fp4_split(objeta_hip_context* ctx, hipStream_t s, const void* d_w, const void* d_s,
                         const float* d_x, float* d_y, uint64_t rows, uint64_t cols, uint64_t batch) {
    const char* action = "launch fp4_e2m1_gemv_split";
    if (cols % 32 != 0)
        OBJ_FAIL(kInvalidInput, action, strf("cols %llu must be a multiple of block_size 32", (unsigned long long)cols));
    if (rows == 0 || batch == 0) return 0;
    if (!d_w || !d_s || !d_x || !d_y) OBJ_FAIL(kInvalidInput, action, "NULL device pointer");
    if (rows > 0x7FFFFFFFull || cols > 0x7FFFFFFFull) OBJ_FAIL(kInvalidInput, action, "rows/cols exceed 2^31");
    if (reinterpret_cast<uintptr_t>(d_s) % 4 == 0 &&
        gemv_mfma_supported(OBJETA_HIP_FP4_E2M1, rows, cols, batch, d_w, d_x))
        return launch_gemv_mfma(ctx, s, OBJETA_HIP_FP4_E2M1, d_w, d_s, d_x, d_y, rows, cols, batch);
    const uint32_t r = static_cast<uint32_t>(rows), c = static_cast<uint32_t>(cols);
    const uint8_t* w = static_cast<const uint8_t*>(d_w);
    const uint8_t* sc = static_cast<const uint8_t*>(d_s);
    const bool fast = cols % 64 == 0 && pick_lpr(c / 64) != 0 && reinterpret_cast<uintptr_t>(w) % 16 == 0 &&
                      reinterpret_cast<uintptr_t>(sc) % 2 == 0 && reinterpret_cast<uintptr_t>(d_x) % 16 == 0;
    const size_t lds_limit = 65536;  // at most 64 KB of staged activations per workgroup
    uint64_t done = 0;
    while (done < batch) {
        const uint64_t rem = batch - done;
        const float* xb = d_x + done * cols;
        float* yb = d_y + done * rows;
        hipError_t e = hipSuccess;
        int nt;
        if (fast) {
            const uint32_t pairs = c / 64;
            const uint32_t lpr = pick_lpr(pairs);
            const size_t per_token = static_cast<size_t>(pairs) * kPad * sizeof(float);
            nt = max_nt_for_lds(per_token, lds_limit, rem);
            if (nt == 0) OBJ_FAIL(kUnsupported, action, strf("cols %u exceed the LDS activation stage", c));
            const size_t lds = per_token * nt + 4 * sizeof(float);
            const Fp4Rows rm{w, sc, static_cast<size_t>(c / 2), static_cast<size_t>(c / 32)};
            switch (nt) {
                case 8: e = launch_stream<Fp4Rows, 8>(ctx, s, rm, xb, yb, r, c, lpr, lds); break;
                case 4: e = launch_stream<Fp4Rows, 4>(ctx, s, rm, xb, yb, r, c, lpr, lds); break;
                case 2: e = launch_stream<Fp4Rows, 2>(ctx, s, rm, xb, yb, r, c, lpr, lds); break;
                default: e = launch_stream<Fp4Rows, 1>(ctx, s, rm, xb, yb, r, c, lpr, lds); break;
            }
        } else {
            nt = rem >= 8 ? 8 : rem >= 4 ? 4 : rem >= 2 ? 2 : 1;
            const dim3 grid((r + kWaves - 1) / kWaves);
            switch (nt) {
                case 8: hipLaunchKernelGGL((fp4_split_generic<8>), grid, dim3(kThreads), 0, s, w, sc, xb, yb, r, c); break;
                case 4: hipLaunchKernelGGL((fp4_split_generic<4>), grid, dim3(kThreads), 0, s, w, sc, xb, yb, r, c); break;
                case 2: hipLaunchKernelGGL((fp4_split_generic<2>), grid, dim3(kThreads), 0, s, w, sc, xb, yb, r, c); break;
                default: hipLaunchKernelGGL((fp4_split_generic<1>), grid, dim3(kThreads), 0, s, w, sc, xb, yb, r, c); break;
            }
            e = hipGetLastError();
        }
        if (e != hipSuccess) OBJ_FAIL(kDriver, action, hipGetErrorString(e));
        done += static_cast<uint64_t>(nt);
    }
    return 0;
}

int32_t launch_fp8_rows(objeta_hip_context* ctx, hipStream_t s, const void* d_w, const void* d_s,
                        const float* d_x, float* d_y, uint64_t rows, uint64_t cols, uint64_t batch) {
    const char* action = "launch fp8_act_fp8_weight_gemv";
    if (cols % 128 != 0)
        OBJ_FAIL(kInvalidInput, action, strf("cols %llu must be a multiple of 128", (unsigned long long)cols));
    if (rows == 0 || batch == 0) return 0;
    if (!d_w || !d_s || !d_x || !d_y) OBJ_FAIL(kInvalidInput, action, "NULL device pointer");
    if (rows > 0x7FFFFFFFull || cols > 0x7FFFFFFFull) OBJ_FAIL(kInvalidInput, action, "rows/cols exceed 2^31");
    if (reinterpret_cast<uintptr_t>(d_w) % 16 != 0 || reinterpret_cast<uintptr_t>(d_x) % 16 != 0)
        OBJ_FAIL(kInvalidInput, action, "weights and activations must be 16-byte aligned");
    const uint32_t r = static_cast<uint32_t>(rows), c = static_cast<uint32_t>(cols);
    const uint32_t pairs = c / 64;
    const uint32_t lpr = pick_lpr(pairs);
    if (lpr == 0) OBJ_FAIL(kUnsupported, action, strf("cols %u has no lane split", c));
    const Fp8Rows rm{static_cast<const uint8_t*>(d_w), static_cast<const uint8_t*>(d_s), c, (c + 127) / 128};
    const size_t per_token = static_cast<size_t>(pairs) * kPad * sizeof(float);
    uint64_t done = 0;
    while (done < batch) {
        const int nt = max_nt_for_lds(per_token, 65536, batch - done);
        if (nt == 0) OBJ_FAIL(kUnsupported, action, strf("cols %u exceed the LDS activation stage", c));
        const size_t lds = per_token * nt + 4 * sizeof(float);
        const float* xb = d_x + done * cols;
        float* yb = d_y + done * rows;
        hipError_t e;
        switch (nt) {
            case 8: e = launch_stream<Fp8Rows, 8>(ctx, s, rm, xb, yb, r, c, lpr, lds); break;
            case 4: e = launch_stream<Fp8Rows, 4>(ctx, s, rm, xb, yb, r, c, lpr, lds); break;
            case 2: e = launch_stream<Fp8Rows, 2>(ctx, s, rm, xb, yb, r, c, lpr, lds); break;
            default: e = launch_stream<Fp8Rows, 1>(ctx, s, rm, xb, yb, r, c, lpr, lds); break;
        }
        if (e != hipSuccess) OBJ_FAIL(kDriver, action, hipGetErrorString(e));
        done += static_cast<uint64_t>(nt);
    }
    return 0;
}

}  // namespace objeta

using namespace objeta;

extern "C" {

int32_t objeta_hip_qgemv_device(objeta_hip_context* ctx, int32_t format, objeta_hip_stream stream,
                                const void* d_qweights, const float* d_x, float* d_y, uint64_t rows,
                                uint64_t cols, uint64_t batch) {
    OBJ_GUARD_BEGIN
    OBJ_TRY(check_ctx(ctx, "qgemv_device"));
    OBJ_HIP(hipSetDevice(ctx->device), "hipSetDevice");
    return launch_qgemv(ctx, format, resolve_stream(ctx, stream), d_qweights, d_x, d_y, rows, cols, batch);
    OBJ_GUARD_END
}

int32_t objeta_hip_fp4_gemv_split_device(objeta_hip_context* ctx, objeta_hip_stream stream, const void* d_w,
                                         const void* d_scales, const float* d_x, float* d_y, uint64_t rows,
                                         uint64_t cols, uint64_t batch) {
    OBJ_GUARD_BEGIN
    OBJ_TRY(check_ctx(ctx, "fp4_gemv_split_device"));
    OBJ_HIP(hipSetDevice(ctx->device), "hipSetDevice");
    return launch_fp4_split(ctx, resolve_stream(ctx, stream), d_w, d_scales, d_x, d_y, rows, cols, batch);
    OBJ_GUARD_END
}

// QuantBackend::gemv (quant.rs:256-302) with validate_quant_inputs (quant.rs:751-793).
int32_t objeta_hip_qgemv(objeta_hip_context* ctx, int32_t format, objeta_hip_stream stream,
                         const uint8_t* qweights, uint64_t qweights_len, const float* x, uint64_t x_len,
                         uint64_t rows, uint64_t cols, float* y, objeta_hip_qgemv_telemetry* tel) {
    OBJ_GUARD_BEGIN
    OBJ_TRY(check_ctx(ctx, "qgemv"));
    const int32_t bb = objeta_hip_block_bytes(format);
    if (bb < 0) OBJ_FAIL(kInvalidInput, "validate format", strf("unknown format %d", format));
    static const char* labels[] = {"q4_0", "q5_0", "iq3_0", "deepseek_fp4_e2m1"};
    const char* label = labels[format];
    if (cols % 32 != 0)
        OBJ_FAIL(kInvalidInput, strf("validate %s column alignment", label),
                 strf("cols %llu must be a multiple of block_size 32", (unsigned long long)cols));
    const uint64_t expected = rows * (cols / 32) * static_cast<uint64_t>(bb);
    if (qweights_len != expected)
        OBJ_FAIL(kInvalidInput, strf("validate %s quantized matrix size", label),
                 strf("qweights len %llu != expected %llu", (unsigned long long)qweights_len,
                      (unsigned long long)expected));
    if (x_len != cols)
        OBJ_FAIL(kInvalidInput, strf("validate %s GEMV vector size", label),
                 strf("x len %llu != cols %llu", (unsigned long long)x_len, (unsigned long long)cols));
    if ((rows && !y) || (expected && !qweights) || (cols && !x)) OBJ_FAIL(kInvalidInput, "qgemv", "NULL host pointer");
    OBJ_HIP(hipSetDevice(ctx->device), "hipSetDevice");
    hipStream_t s = resolve_stream(ctx, stream);
    if (rows == 0) {
        if (tel) *tel = objeta_hip_qgemv_telemetry{};
        return 0;
    }
    void *dq = nullptr, *dx = nullptr, *dy = nullptr;
    hipEvent_t ev[6] = {};
    int32_t rc = 0;
    auto cleanup = [&]() {
        (void)hipStreamSynchronize(s);
        if (dq) (void)hipFree(dq);
        if (dx) (void)hipFree(dx);
        if (dy) (void)hipFree(dy);
        for (auto& e : ev) if (e) (void)hipEventDestroy(e);
    };
    do {
        hipError_t e = hipSuccess;
        for (auto& v : ev) if (e == hipSuccess) e = hipEventCreate(&v);
        if (e == hipSuccess) e = hipMalloc(&dq, expected ? expected : 4);
        if (e == hipSuccess) e = hipMalloc(&dx, cols * sizeof(float) + 16);
        if (e == hipSuccess) e = hipMalloc(&dy, rows * sizeof(float));
        if (e != hipSuccess) { rc = set_error(kDriver, __FILE__, __LINE__, __func__, "allocate GEMV buffers", hipGetErrorString(e)); break; }
        e = hipEventRecord(ev[0], s);                                        // total start
        if (e == hipSuccess) e = hipEventRecord(ev[1], s);                   // h2d start
        if (e == hipSuccess) e = hipMemcpyAsync(dq, qweights, expected, hipMemcpyHostToDevice, s);
        if (e == hipSuccess) e = hipMemcpyAsync(dx, x, cols * sizeof(float), hipMemcpyHostToDevice, s);
        if (e == hipSuccess) e = hipEventRecord(ev[2], s);                   // h2d end / kernel start
        if (e != hipSuccess) { rc = set_error(kDriver, __FILE__, __LINE__, __func__, strf("%s_h2d", label), hipGetErrorString(e)); break; }
        rc = launch_qgemv(ctx, format, s, dq, static_cast<const float*>(dx), static_cast<float*>(dy), rows, cols, 1);
        if (rc) break;
        e = hipEventRecord(ev[3], s);                                        // kernel end / d2h start
        if (e == hipSuccess) e = hipMemcpyAsync(y, dy, rows * sizeof(float), hipMemcpyDeviceToHost, s);
        if (e == hipSuccess) e = hipEventRecord(ev[4], s);                   // d2h end
        if (e == hipSuccess) e = hipEventRecord(ev[5], s);                   // total end
        if (e == hipSuccess) e = hipEventSynchronize(ev[5]);
        if (e != hipSuccess) { rc = set_error(kDriver, __FILE__, __LINE__, __func__, strf("%s_d2h", label), hipGetErrorString(e)); break; }
        if (tel) {
            float h2d = 0, ker = 0, d2h = 0, tot = 0;
            (void)hipEventElapsedTime(&h2d, ev[1], ev[2]);
            (void)hipEventElapsedTime(&ker, ev[2], ev[3]);
            (void)hipEventElapsedTime(&d2h, ev[3], ev[4]);
            (void)hipEventElapsedTime(&tot, ev[0], ev[5]);
            tel->h2d_ms = h2d;
            tel->kernel_ms = ker;
            tel->d2h_ms = d2h;
            tel->total_ms = tot;
            const float un = tot - h2d - ker - d2h;
            tel->unaccounted_ms = un > 0.f ? un : 0.f;
            tel->bytes_read = expected + cols * sizeof(float);
            tel->effective_gbps = ker > 0.f ? static_cast<float>(tel->bytes_read) / (ker / 1000.0f) / 1.0e9f : 0.f;
        }
    } while (false);
    cleanup();
    return rc;
    OBJ_GUARD_END
}

}  // extern "C"
