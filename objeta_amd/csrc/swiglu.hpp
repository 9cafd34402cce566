// swiglu.hpp — the two SwiGLU forms of the expert compositions, shared by the
// per-assignment kernels (moe.hip) and the grouped-token products (grouped.hip).
#pragma once

#include "router_math.hpp"

namespace objeta {
namespace dev {

// silu_mul (kernels/moe.cu:2-22); the CPU reference is moe.rs:1308-1315.
__device__ __forceinline__ float silu_mul(float g, float u, float limit) {
    if (limit > 0.0f) {
        u = fminf(limit, fmaxf(-limit, u));
        g = fminf(limit, g);
    }
    const float silu = g / (1.0f + expf(-g));
    return silu * u;
}

// The SwiGLU of the official compositions (crates/objeta-parser/src/deepseek.rs:
// 1680-1686, 1708-1713): only the up projection is clamped, exp is glibc's expf
// (Rust's f32::exp) and the division is the IEEE float quotient, here the double
// quotient rounded once to float (exact: a double carries more than 2 * 24 + 2
// bits, so the double rounding of a float division is innocuous). __fdiv_rn in this
// spot gave every kernel of the file a private stack.
__device__ __forceinline__ float swiglu_official(float g, float u, float limit) {
    if (u < -limit) u = -limit;
    else if (u > limit) u = limit;
    const float d = 1.0f + rmath::expf_glibc(-g);
    return static_cast<float>(static_cast<double>(g) / static_cast<double>(d)) * u;
}

__device__ __forceinline__ float swiglu(float g, float u, float limit, uint32_t official) {
    return official ? swiglu_official(g, u, limit) : silu_mul(g, u, limit);
}

}  // namespace dev
}  // namespace objeta
