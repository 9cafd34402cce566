// device_common.hpp — gfx950 device helpers shared by the HIP kernels: block
// formats, aligned block-pair loads, in-register dequantisation and wave64
// reductions.
//
// Dequantisation keeps the reference's values exactly: (q - 8), (q - 16), (q - 4)
// and the E2M1 table values are built as fp16 bit patterns (exact), multiplied by
// fp32 activations in v_fma_mix_f32 (exact product, fp32 accumulate), and the f16
// block scale is applied once per block.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace objeta {
namespace dev {

enum : int { kQ4 = 0, kQ5 = 1, kIQ3 = 2, kFP4 = 3 };

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4), aligned(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2), aligned(4)));

template <int F> struct Fmt;
template <> struct Fmt<kQ4> { static constexpr int kBlockBytes = 18; static constexpr int kPairDw = 9; };
template <> struct Fmt<kQ5> { static constexpr int kBlockBytes = 22; static constexpr int kPairDw = 11; };
template <> struct Fmt<kIQ3> { static constexpr int kBlockBytes = 14; static constexpr int kPairDw = 7; };
template <> struct Fmt<kFP4> { static constexpr int kBlockBytes = 17; static constexpr int kPairDw = 0; };

__device__ __forceinline__ float f16_to_f32(uint32_t bits16) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits16)));
}

__device__ __forceinline__ h2 as_h2(uint32_t v) { return __builtin_bit_cast(h2, v); }

__device__ __forceinline__ uint32_t alignb(uint32_t hi, uint32_t lo, uint32_t bytes) {
    return __builtin_amdgcn_alignbyte(hi, lo, bytes);
}

// A pointer to device memory as a global-address-space pointer. Weight pointers
// read from a device table are otherwise generic, and generic (flat) loads are
// also counted by the LDS counter: every LDS wait would then wait for all weight
// loads in flight, which serialises prefetching with LDS work.
template <class T>
using gptr = const __attribute__((address_space(1))) T*;
template <class T>
__device__ __forceinline__ gptr<T> as_global(const T* p) {
    return (gptr<T>)(p);
}

// Loads N dwords starting at a 4-byte aligned address. Lanes of a wave read
// consecutive 36/44/28-byte pairs, so every cache line is touched by each of the
// (up to three) load instructions of a pair: ordinary cached loads let the CU's L1
// serve the second and third touch, where non-temporal loads sent each of them on
// to the L2 (measured on MI355X: the Qwen3-A3B gate/up kernel 7.1 -> 6.3 us).
template <int N>
__device__ __forceinline__ void load_dwords(const uint32_t* __restrict__ p, uint32_t (&d)[N]) {
    const gptr<uint32_t> g = as_global(p);
    int i = 0;
#pragma unroll
    for (; i + 4 <= N; i += 4) {
        const u32x4 v = *(gptr<u32x4>)(g + i);
        d[i] = v.x; d[i + 1] = v.y; d[i + 2] = v.z; d[i + 3] = v.w;
    }
    if constexpr (N % 4 >= 2) {
        const u32x2 v = *(gptr<u32x2>)(g + i);
        d[i] = v.x; d[i + 1] = v.y;
        i += 2;
    }
    if constexpr (N % 2 == 1) d[i] = g[i];
}

// ---------------------------------------------------------------- Q4_0
// 8 weights from one nibble dword n (byte k: weight 2k low nibble, 2k+1 high
// nibble) against x[0..7] = xa (w0..w3), xb (w4..w7). `lo` accumulates
// (q-8)*x for w0,w2,w4,w6; `hi` accumulates 16*(q-8)*x for w1,w3,w5,w7.
// Constants the nibble unpacking combines in one 3-input bit op. gfx9 VOP3
// encodings cannot carry literals, so the constants are pinned in registers
// (the empty asm hides their values from constant folding) and the compiler
// emits v_and_or / v_bitop3 instead of separate v_and + v_or with literals.
struct NibbleConsts {
    uint32_t lo_mask, hi_mask, magic;
    __device__ __forceinline__ NibbleConsts() : lo_mask(0x000F000Fu), hi_mask(0x00F000F0u), magic(0x64006400u) {
        asm volatile("" : "+v"(lo_mask), "+v"(hi_mask), "+v"(magic));
    }
};

template <int NT>
__device__ __forceinline__ void q4_dot8(uint32_t n, const float4 (&xa)[NT], const float4 (&xb)[NT],
                                        float (&lo)[NT], float (&hi)[NT], const NibbleConsts& k) {
    const h2 k_lo = {(_Float16)1032.0f, (_Float16)1032.0f};
    const h2 k_hi = {(_Float16)1152.0f, (_Float16)1152.0f};
    uint32_t n8 = n >> 8;
    h2 a = as_h2((n & k.lo_mask) | k.magic) - k_lo;   // (q0-8, q4-8)
    h2 b = as_h2((n & k.hi_mask) | k.magic) - k_hi;   // 16*(q1-8, q5-8)
    h2 c = as_h2((n8 & k.lo_mask) | k.magic) - k_lo;  // (q2-8, q6-8)
    h2 d = as_h2((n8 & k.hi_mask) | k.magic) - k_hi;  // 16*(q3-8, q7-8)
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        lo[t] = __builtin_fmaf((float)a.x, xa[t].x, lo[t]);
        lo[t] = __builtin_fmaf((float)a.y, xb[t].x, lo[t]);
        lo[t] = __builtin_fmaf((float)c.x, xa[t].z, lo[t]);
        lo[t] = __builtin_fmaf((float)c.y, xb[t].z, lo[t]);
        hi[t] = __builtin_fmaf((float)b.x, xa[t].y, hi[t]);
        hi[t] = __builtin_fmaf((float)b.y, xb[t].y, hi[t]);
        hi[t] = __builtin_fmaf((float)d.x, xa[t].w, hi[t]);
        hi[t] = __builtin_fmaf((float)d.y, xb[t].w, hi[t]);
    }
}

// ---------------------------------------------------------------- Q5_0
// As q4_dot8 with the 5th bit from the high mask byte m (bit j: weight j):
// (q0-16, q4-16), 16*(q1-16, q5-16), ...
template <int NT>
__device__ __forceinline__ void q5_dot8(uint32_t n, uint32_t m, const float4 (&xa)[NT],
                                        const float4 (&xb)[NT], float (&lo)[NT], float (&hi)[NT]) {
    const uint32_t magic = 0x64006400u;
    const h2 k_lo = {(_Float16)1040.0f, (_Float16)1040.0f};  // 1024 + 16
    const h2 k_hi = {(_Float16)1280.0f, (_Float16)1280.0f};  // 1024 + 256
    uint32_t n8 = n >> 8;
    uint32_t sa = ((m & 0x11u) * 0x10010u) & 0x00100010u;   // m0 -> bit 4, m4 -> bit 20
    uint32_t sb = ((m & 0x22u) * 0x80080u) & 0x01000100u;   // m1 -> bit 8, m5 -> bit 24
    uint32_t sc = ((m & 0x44u) * 0x04004u) & 0x00100010u;   // m2 -> bit 4, m6 -> bit 20
    uint32_t sd = ((m & 0x88u) * 0x20020u) & 0x01000100u;   // m3 -> bit 8, m7 -> bit 24
    h2 a = as_h2((n & 0x000F000Fu) | sa | magic) - k_lo;
    h2 b = as_h2((n & 0x00F000F0u) | sb | magic) - k_hi;
    h2 c = as_h2((n8 & 0x000F000Fu) | sc | magic) - k_lo;
    h2 d = as_h2((n8 & 0x00F000F0u) | sd | magic) - k_hi;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        lo[t] = __builtin_fmaf((float)a.x, xa[t].x, lo[t]);
        lo[t] = __builtin_fmaf((float)a.y, xb[t].x, lo[t]);
        lo[t] = __builtin_fmaf((float)c.x, xa[t].z, lo[t]);
        lo[t] = __builtin_fmaf((float)c.y, xb[t].z, lo[t]);
        hi[t] = __builtin_fmaf((float)b.x, xa[t].y, hi[t]);
        hi[t] = __builtin_fmaf((float)b.y, xb[t].y, hi[t]);
        hi[t] = __builtin_fmaf((float)d.x, xa[t].w, hi[t]);
        hi[t] = __builtin_fmaf((float)d.y, xb[t].w, hi[t]);
    }
}

// ---------------------------------------------------------------- IQ3_0
// One IQ3 block: lows l0 (weights 0..15, 2 bits each) and l1 (16..31), highs h
// (bit j: weight j). Pairs weight i with i+16 so that both the low fields (after a
// byte interleave) and the high bits sit 16 bits apart. Accumulates (q-4)*x.
template <int NT>
__device__ __forceinline__ void iq3_block_dot(uint32_t l0, uint32_t l1, uint32_t h,
                                              const float* const (&xs)[NT], float (&acc)[NT]) {
    const uint32_t magic = 0x64006400u;
    const h2 k4 = {(_Float16)1028.0f, (_Float16)1028.0f};  // 1024 + 4
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        // bytes: [l0.byte_k, 0, l1.byte_k, 0] -> lows of weights 4k..4k+3 and 16+4k..
        uint32_t p = __builtin_amdgcn_perm(l1, l0, 0x0C040C00u + (uint32_t)k * 0x00010001u);
        float4 xa[NT], xb[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            xa[t] = *reinterpret_cast<const float4*>(xs[t] + 4 * k);
            xb[t] = *reinterpret_cast<const float4*>(xs[t] + 16 + 4 * k);
        }
#pragma unroll
        for (int f = 0; f < 4; ++f) {
            const int j = 4 * k + f;  // weights j and j + 16
            uint32_t hb = (j >= 2) ? (h >> (j - 2)) : (h << (2 - j));
            uint32_t v = ((p >> (2 * f)) & 0x00030003u) | (hb & 0x00040004u) | magic;
            h2 w = as_h2(v) - k4;
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                float x0 = f == 0 ? xa[t].x : f == 1 ? xa[t].y : f == 2 ? xa[t].z : xa[t].w;
                float x1 = f == 0 ? xb[t].x : f == 1 ? xb[t].y : f == 2 ? xb[t].z : xb[t].w;
                acc[t] = __builtin_fmaf((float)w.x, x0, acc[t]);
                acc[t] = __builtin_fmaf((float)w.y, x1, acc[t]);
            }
        }
    }
}

// ------------------------------------------- reference-form block (specials)
// The reference's per-weight form w = value * scale; sum += w * x
// (quant.rs:928-1019), decoding from the block's dwords already in registers.
// Used only when a block scale is not finite: there the per-weight products
// (e.g. 0 * inf = NaN) decide the result, so the factored form must not be used.
// n[0..3]: the 16 nibble bytes (Q4, Q5) or, for IQ3, n[0..1] the 8 low bytes and
// n[2] the 4 high bytes; m: Q5 high-bit mask.
template <int F>
__device__ __forceinline__ int reg_value(const uint32_t (&n)[4], uint32_t m, int i) {
    if constexpr (F == kQ4) {
        return static_cast<int>((n[i >> 3] >> (4 * (i & 7))) & 15u) - 8;
    } else if constexpr (F == kQ5) {
        const uint32_t lo = (n[i >> 3] >> (4 * (i & 7))) & 15u;
        return static_cast<int>(lo | (((m >> i) & 1u) << 4)) - 16;
    } else {
        const uint32_t lo = (n[i >> 4] >> (2 * (i & 15))) & 3u;
        const uint32_t hi = (n[2] >> i) & 1u;
        return static_cast<int>(lo | (hi << 2)) - 4;
    }
}

// Inlined, with a rolled loop: an out-of-line call (arrays passed by reference, a
// call frame) gave every kernel using it a private stack although this path runs
// only for non-finite block scales; the small arrays indexed in the loop stay in
// registers.
template <int F, int NT>
__device__ __forceinline__ void block_dot_reference_form(const uint32_t (&n)[4], uint32_t m, float scale,
                                                         const float* const (&xs)[NT], int xoff,
                                                         float (&acc)[NT]) {
#pragma unroll 1
    for (int i = 0; i < 32; ++i) {
        const float w = static_cast<float>(reg_value<F>(n, m, i)) * scale;
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[t] = __builtin_fmaf(w, xs[t][xoff + i], acc[t]);
    }
}

// ------------------------------------------------------- block pair dots
// Dot product of a pair of consecutive blocks (64 weights, 4-byte aligned pair
// start `pair`, already loaded into d) with NT activation vectors xs[t][0..63]
// (LDS or global), adding to acc.
// xs_slow: the same activations for the reference-form path (indexed at run time,
// so it must be addressable memory even when xs points at registers).
template <int F, int NT>
__device__ __forceinline__ void pair_dot(const uint32_t (&d)[Fmt<F>::kPairDw],
                                         const float* const (&xs)[NT], float (&acc)[NT],
                                         const float* const (&xs_slow)[NT]) {
    {
        const float s0 = f16_to_f32(d[0] & 0xFFFFu);
        const float s1 = F == kQ4 ? f16_to_f32(d[4] >> 16)
                                  : F == kQ5 ? f16_to_f32(d[5] >> 16) : f16_to_f32(d[3] >> 16);
        if (!__builtin_isfinite(s0) || !__builtin_isfinite(s1)) {
            uint32_t n0[4], n1[4], m0 = 0, m1 = 0;
            if constexpr (F == kQ4) {
                for (int j = 0; j < 4; ++j) { n0[j] = alignb(d[j + 1], d[j], 2); n1[j] = d[5 + j]; }
            } else if constexpr (F == kQ5) {
                m0 = alignb(d[1], d[0], 2);
                m1 = d[6];
                for (int j = 0; j < 4; ++j) { n0[j] = alignb(d[j + 2], d[j + 1], 2); n1[j] = d[7 + j]; }
            } else {
                n0[0] = alignb(d[1], d[0], 2); n0[1] = alignb(d[2], d[1], 2); n0[2] = alignb(d[3], d[2], 2);
                n1[0] = d[4]; n1[1] = d[5]; n1[2] = d[6];
                n0[3] = n1[3] = 0;
            }
            block_dot_reference_form<F, NT>(n0, m0, s0, xs_slow, 0, acc);
            block_dot_reference_form<F, NT>(n1, m1, s1, xs_slow, 32, acc);
            return;
        }
    }
    if constexpr (F == kQ4) {
        // bytes 0-1 scale0, 2-17 nibbles0, 18-19 scale1, 20-35 nibbles1
        const NibbleConsts kc;
        const float s0 = f16_to_f32(d[0] & 0xFFFFu);
        const float s1 = f16_to_f32(d[4] >> 16);
#pragma unroll
        for (int blk = 0; blk < 2; ++blk) {
            float lo[NT], hi[NT];
#pragma unroll
            for (int t = 0; t < NT; ++t) { lo[t] = 0.f; hi[t] = 0.f; }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                uint32_t n = blk == 0 ? alignb(d[j + 1], d[j], 2) : d[5 + j];
                float4 xa[NT], xb[NT];
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    xa[t] = *reinterpret_cast<const float4*>(xs[t] + blk * 32 + 8 * j);
                    xb[t] = *reinterpret_cast<const float4*>(xs[t] + blk * 32 + 8 * j + 4);
                }
                q4_dot8<NT>(n, xa, xb, lo, hi, kc);
            }
            const float s = blk == 0 ? s0 : s1;
#pragma unroll
            for (int t = 0; t < NT; ++t) acc[t] = __builtin_fmaf(s, __builtin_fmaf(hi[t], 0.0625f, lo[t]), acc[t]);
        }
    } else if constexpr (F == kQ5) {
        // bytes 0-1 scale0, 2-5 mask0, 6-21 nibbles0, 22-23 scale1, 24-27 mask1, 28-43 nibbles1
        const float s0 = f16_to_f32(d[0] & 0xFFFFu);
        const float s1 = f16_to_f32(d[5] >> 16);
#pragma unroll
        for (int blk = 0; blk < 2; ++blk) {
            const uint32_t mask = blk == 0 ? alignb(d[1], d[0], 2) : d[6];
            float lo[NT], hi[NT];
#pragma unroll
            for (int t = 0; t < NT; ++t) { lo[t] = 0.f; hi[t] = 0.f; }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                uint32_t n = blk == 0 ? alignb(d[j + 2], d[j + 1], 2) : d[7 + j];
                float4 xa[NT], xb[NT];
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    xa[t] = *reinterpret_cast<const float4*>(xs[t] + blk * 32 + 8 * j);
                    xb[t] = *reinterpret_cast<const float4*>(xs[t] + blk * 32 + 8 * j + 4);
                }
                q5_dot8<NT>(n, (mask >> (8 * j)) & 0xFFu, xa, xb, lo, hi);
            }
            const float s = blk == 0 ? s0 : s1;
#pragma unroll
            for (int t = 0; t < NT; ++t) acc[t] = __builtin_fmaf(s, __builtin_fmaf(hi[t], 0.0625f, lo[t]), acc[t]);
        }
    } else if constexpr (F == kIQ3) {
        // bytes 0-1 scale0, 2-9 lows0, 10-13 highs0, 14-15 scale1, 16-23 lows1, 24-27 highs1
        const float s0 = f16_to_f32(d[0] & 0xFFFFu);
        const float s1 = f16_to_f32(d[3] >> 16);
#pragma unroll
        for (int blk = 0; blk < 2; ++blk) {
            uint32_t l0 = blk == 0 ? alignb(d[1], d[0], 2) : d[4];
            uint32_t l1 = blk == 0 ? alignb(d[2], d[1], 2) : d[5];
            uint32_t hb = blk == 0 ? alignb(d[3], d[2], 2) : d[6];
            float a[NT];
            const float* xb[NT];
#pragma unroll
            for (int t = 0; t < NT; ++t) { a[t] = 0.f; xb[t] = xs[t] + blk * 32; }
            iq3_block_dot<NT>(l0, l1, hb, xb, a);
            const float s = blk == 0 ? s0 : s1;
#pragma unroll
            for (int t = 0; t < NT; ++t) acc[t] = __builtin_fmaf(s, a[t], acc[t]);
        }
    }
}

template <int F, int NT>
__device__ __forceinline__ void pair_dot(const uint32_t (&d)[Fmt<F>::kPairDw],
                                         const float* const (&xs)[NT], float (&acc)[NT]) {
    pair_dot<F, NT>(d, xs, acc, xs);
}

// ------------------------------------------------------------- FP4 E2M1
// fp16 bits (c & 7) << 9 encode E2M1(c) * 2^-14 exactly (the f16 subnormal
// covers E2M1's e=0 codes), and bit 3 of the code is the sign. One nibble dword
// n (byte k: weight 2k low, 2k+1 high) against x[0..7]; accumulates
// The 8 E2M1 codes of a dword (element 2j in the low nibble of byte j, 2j + 1 in
// the high one) as exact fp16 pairs (w_{2j}, w_{2j+1}): gfx950's
// v_cvt_scalef32_pk_f16_fp4 with scale 1, one instruction per byte (checked against
// the E2M1 table on every byte and byte select, -0 for code 8 included).
__device__ __forceinline__ void fp4_to_h2x4(uint32_t n, h2 (&p)[4]) {
    p[0] = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(n, 1.0f, 0);
    p[1] = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(n, 1.0f, 1);
    p[2] = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(n, 1.0f, 2);
    p[3] = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(n, 1.0f, 3);
}

// Four of the reference's E4M3 codes (rules::f8e4m3_to_f32, deepseek.rs:799-829)
// rewritten to the OCP E4M3 codes of the same values, so that gfx950's hardware E4M3
// conversion decodes them: exponent field 0 means m * 2^-5 in the reference (m * 2^-9
// in OCP), so m goes to the code of m / 32 (0, 0x10, 0x18, 0x1C, 0x20, 0x22, 0x24,
// 0x26, picked by v_perm); field 15 means +-448 for every mantissa (OCP: 256 (1 +
// m/8), NaN at m = 7), so it goes to 0x7E. Signs are kept; other codes pass through.
__device__ __forceinline__ uint32_t fp8_ref_to_ocp(uint32_t d) {
    const uint32_t e = d & 0x78787878u;
    const uint32_t z = ~(e + 0x78787878u) & 0x80808080u;  // bit 7 of the bytes whose field is 0
    const uint32_t f = (e + 0x08080808u) & 0x80808080u;   // bit 7 of the bytes whose field is 15
    const uint32_t zb = z >> 7, fb = f >> 7;
    const uint32_t zm = (zb << 8) - zb, fm = (fb << 8) - fb;  // 0xFF in those bytes
    const uint32_t sign = d & 0x80808080u;
    const uint32_t small = __builtin_amdgcn_perm(0x26242220u, 0x1C181000u, d & 0x07070707u) | sign;
    const uint32_t t = (small & zm) | (d & ~zm);
    return ((0x7E7E7E7Eu | sign) & fm) | (t & ~fm);
}

// The reference's decode of the 4 E4M3 codes of a dword (byte i -> w[i]), exact.
__device__ __forceinline__ void fp8x4_to_f32(uint32_t d, float (&w)[4]) {
    typedef float f2 __attribute__((ext_vector_type(2)));
    const uint32_t r = fp8_ref_to_ocp(d);
    const f2 lo = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(r, 1.0f, false);
    const f2 hi = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(r, 1.0f, true);
    w[0] = lo.x;
    w[1] = lo.y;
    w[2] = hi.x;
    w[3] = hi.y;
}

// The same as fp16 pairs (bytes 0, 1 and 2, 3): every value the reference decodes is
// an exact fp16 (|v| in [2^-5, 448], or 0).
__device__ __forceinline__ void fp8x4_to_h2x2(uint32_t d, h2& lo, h2& hi) {
    const uint32_t r = fp8_ref_to_ocp(d);
    lo = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(r, 1.0f, false);
    hi = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(r, 1.0f, true);
}

// sum_i E2M1(q_i) * x_i over 8 weights (xa = x0..x3, xb = x4..x7); the caller
// multiplies by the block scale.
template <int NT>
__device__ __forceinline__ void fp4_dot8(uint32_t n, const float4 (&xa)[NT], const float4 (&xb)[NT],
                                         float (&acc)[NT]) {
    h2 p[4];
    fp4_to_h2x4(n, p);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        acc[t] = __builtin_fmaf((float)p[0].x, xa[t].x, acc[t]);
        acc[t] = __builtin_fmaf((float)p[0].y, xa[t].y, acc[t]);
        acc[t] = __builtin_fmaf((float)p[1].x, xa[t].z, acc[t]);
        acc[t] = __builtin_fmaf((float)p[1].y, xa[t].w, acc[t]);
        acc[t] = __builtin_fmaf((float)p[2].x, xb[t].x, acc[t]);
        acc[t] = __builtin_fmaf((float)p[2].y, xb[t].y, acc[t]);
        acc[t] = __builtin_fmaf((float)p[3].x, xb[t].z, acc[t]);
        acc[t] = __builtin_fmaf((float)p[3].y, xb[t].w, acc[t]);
    }
}

// E8M0 scale byte -> 2^(raw-127) as f32 (raw 0 -> 2^-127, 255 -> inf), the
// decode of quant.rs:886-892 and deepseek.rs:838-856 (identical on all bytes).
__device__ __forceinline__ float e8m0_to_f32(uint32_t raw) {
    return raw == 0 ? __builtin_bit_cast(float, 1u << 22) : __builtin_bit_cast(float, raw << 23);
}

// ------------------------------------------------------------- reductions
// Sum over lanes [seg*L, seg*L + L) of a wave; the total lands in the segment's
// first lane. L need not be a power of two (L <= 64).
template <int L>
__device__ __forceinline__ float seg_reduce(float v, int lane_in_seg) {
    if constexpr ((L & (L - 1)) == 0) {
#pragma unroll
        for (int off = L / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
        return v;
    } else {
#pragma unroll
        for (int off = 1; off < L; off <<= 1) {
            float o = __shfl_down(v, off, 64);
            v += (lane_in_seg + off < L) ? o : 0.0f;
        }
        return v;
    }
}

__device__ __forceinline__ float wave_reduce(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

}  // namespace dev
}  // namespace objeta
