// kernels.hpp — host-side launchers shared between translation units. Each
// launcher validates its shape arguments, enqueues on `s` and allocates nothing.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

struct objeta_hip_context;

namespace objeta {

int32_t launch_qgemv(objeta_hip_context* ctx, int32_t format, hipStream_t s, const void* d_q,
                     const float* d_x, float* d_y, uint64_t rows, uint64_t cols, uint64_t batch);

int32_t launch_fp4_split(objeta_hip_context* ctx, hipStream_t s, const void* d_w, const void* d_s,
                         const float* d_x, float* d_y, uint64_t rows, uint64_t cols, uint64_t batch);

int32_t launch_zero(hipStream_t s, void* d, uint64_t bytes);

}  // namespace objeta
