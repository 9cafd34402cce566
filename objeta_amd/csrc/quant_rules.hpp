// quant_rules.hpp — bit-level rules of the reference's CPU quantizers, written
// once for host and device so the device quantizer emits the same bytes as
// quantize_matrix_cpu (crates/objeta-cuda/src/quant.rs:506-926).
#pragma once

#include <stdint.h>

// Under hipcc the rules are host and device functions; a plain C++ compiler sees
// ordinary inline functions (the host checks of the scale rules build that way).
#if defined(__HIPCC__)
#include <hip/hip_runtime.h>
#define OBJ_HD __host__ __device__ __forceinline__
#else
#define OBJ_HD inline
#endif

namespace objeta {
namespace rules {

OBJ_HD uint32_t f2u(float f) { return __builtin_bit_cast(uint32_t, f); }
OBJ_HD float u2f(uint32_t u) { return __builtin_bit_cast(float, u); }

// f32_to_f16_bits (quant.rs:1046-1079): round-half-up on mantissa bit 12 without a
// sticky bit; subnormals round half-up on the shifted-out bit; NaN -> 0x7E00|sign.
OBJ_HD uint16_t f32_to_f16_bits(float value) {
    const uint32_t bits = f2u(value);
    const uint16_t sign = static_cast<uint16_t>((bits >> 16) & 0x8000u);
    const int32_t exp = static_cast<int32_t>((bits >> 23) & 0xFFu);
    const uint32_t mant = bits & 0x7FFFFFu;
    if (exp == 255) return static_cast<uint16_t>(sign | 0x7C00u | (mant ? 0x0200u : 0u));
    const int32_t half_exp = exp - 127 + 15;
    if (half_exp >= 0x1F) return static_cast<uint16_t>(sign | 0x7C00u);
    if (half_exp <= 0) {
        if (half_exp < -10) return sign;
        const uint32_t m = mant | 0x800000u;
        const int32_t shift = 14 - half_exp;
        uint16_t half = static_cast<uint16_t>(m >> shift);
        if ((m >> (shift - 1)) & 1u) half = static_cast<uint16_t>(half + 1);
        return static_cast<uint16_t>(sign | half);
    }
    uint16_t half = static_cast<uint16_t>(sign | (static_cast<uint32_t>(half_exp) << 10) | (mant >> 13));
    if (mant & 0x1000u) half = static_cast<uint16_t>(half + 1);
    return half;
}

// `(v).round().clamp(0.0, hi) as u8` in Rust: round half away from zero, NaN
// survives clamp, the saturating cast maps NaN to 0.
OBJ_HD uint8_t round_clamp_u8(float v, float hi) {
    float r = __builtin_roundf(v);
    if (r != r) return 0;
    if (r < 0.0f) r = 0.0f;
    if (r > hi) r = hi;
    return static_cast<uint8_t>(r);
}

// IEEE division, correctly rounded on host and device alike.
OBJ_HD float div_rn(float a, float b) {
#if defined(__HIP_DEVICE_COMPILE__)
    return __fdiv_rn(a, b);
#else
    return a / b;
#endif
}

// ceil(log2f(y)) as the reference evaluates it (glibc log2f, which is correctly
// rounded on these inputs), for finite y > 0, in integers: the exact ceiling,
// except that y = 2^k * (1 + m*2^-23) with 1 <= m <= T rounds log2 down to k,
// where T is the largest m with log2(1 + m*2^-23) under half an ulp of k. T
// depends only on the binade of the float nearest k (the binade below for
// k = -2^j). Subnormal y behave the same way relative to their leading bit.
OBJ_HD int32_t ceil_log2_cr(float y) {
    const uint32_t b = f2u(y);
    const uint32_t e = (b >> 23) & 0xFFu;
    const uint32_t m = b & 0x7FFFFFu;
    if (e == 0) {
        // y = m * 2^-149, m > 0; p = floor(log2 m)
        const int32_t p = 31 - __builtin_clz(m);
        const uint32_t rest = m - (1u << p);
        if (rest == 0) return -149 + p;
        // log2 rounds to -149+p when rest <= T(p); p <= 22 here.
        uint32_t t = 0;
        if (p == 22) t = 11;
        else if (p == 20 || p == 21) t = 5;
        else if (p == 19) t = 2;
        else if (p == 18) t = 1;
        return (rest <= t) ? (-149 + p) : (-149 + p + 1);
    }
    const int32_t k = static_cast<int32_t>(e) - 127;
    if (m == 0) return k;
    // binade index j of |k| as represented: floor(log2|k|), one lower for k = -2^j.
    int32_t ak = k < 0 ? -k : k;
    uint32_t t = 0;
    if (ak >= 2) {
        int32_t j = 31 - __builtin_clz(static_cast<uint32_t>(ak));
        if (k < 0 && (ak & (ak - 1)) == 0) j -= 1;
        // T = floor(2^(j-1) / ln 2 ... ) evaluated: j=1 -> 0, 2 -> 1, 3 -> 2, 4 -> 5, 5 -> 11, 6 -> 22
        switch (j) {
            case 2: t = 1; break;
            case 3: t = 2; break;
            case 4: t = 5; break;
            case 5: t = 11; break;
            case 6: t = 22; break;
            default: t = j >= 7 ? 44u : 0u; break;
        }
    }
    return (m <= t) ? k : k + 1;
}

// E8M0 exponent choice of fp4_quantize_block (quant.rs:913-918).
OBJ_HD uint8_t fp4_scale_raw(float amax) {
    if (amax > 0.0f && amax < __builtin_inff()) {
        const float y = div_rn(amax, 6.0f);
        if (y == 0.0f) return 0;  // log2(0) = -inf -> saturating cast -> clamp to 0
        int32_t v = ceil_log2_cr(y) + 127;
        if (v < 0) v = 0;
        if (v > 255) v = 255;
        return static_cast<uint8_t>(v);
    }
    return 0;
}

// decode_f8_e8m0 (quant.rs:886-892)
OBJ_HD float decode_e8m0(uint32_t raw) { return raw == 0 ? u2f(1u << 22) : u2f(raw << 23); }

// quantize_val (quant.rs:894-906): first minimum over the 16-entry table.
OBJ_HD uint8_t fp4_quantize_val(float val, float scale) {
    const float table[16] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f,
                             -0.0f, -0.5f, -1.0f, -1.5f, -2.0f, -3.0f, -4.0f, -6.0f};
    const float scaled = div_rn(val, scale);
    int best = 0;
    float min_diff = __builtin_inff();
    for (int q = 0; q < 16; ++q) {
        const float diff = __builtin_fabsf(scaled - table[q]);
        if (diff < min_diff) { min_diff = diff; best = q; }
    }
    return static_cast<uint8_t>(best);
}

// Block quantizers (quant.rs:814-926). src: 32 floats.
OBJ_HD float block_amax(const float* src) {
    float amax = 0.0f;
    for (int i = 0; i < 32; ++i) amax = __builtin_fmaxf(amax, __builtin_fabsf(src[i]));
    return amax;
}

OBJ_HD void q4_block(const float* src, uint8_t* dst) {
    const float amax = block_amax(src);
    const float scale = amax > 0.0f ? div_rn(amax, 7.0f) : 1.0e-10f;
    const uint16_t h = f32_to_f16_bits(scale);
    dst[0] = static_cast<uint8_t>(h & 0xFF);
    dst[1] = static_cast<uint8_t>(h >> 8);
    for (int i = 0; i < 16; ++i) {
        const uint8_t q0 = round_clamp_u8(div_rn(src[2 * i], scale) + 8.0f, 15.0f);
        const uint8_t q1 = round_clamp_u8(div_rn(src[2 * i + 1], scale) + 8.0f, 15.0f);
        dst[2 + i] = static_cast<uint8_t>(q0 | (q1 << 4));
    }
}

OBJ_HD void q5_block(const float* src, uint8_t* dst) {
    const float amax = block_amax(src);
    const float scale = amax > 0.0f ? div_rn(amax, 15.0f) : 1.0e-10f;
    const uint16_t h = f32_to_f16_bits(scale);
    uint8_t out[22] = {};
    out[0] = static_cast<uint8_t>(h & 0xFF);
    out[1] = static_cast<uint8_t>(h >> 8);
    for (int i = 0; i < 32; ++i) {
        const uint8_t q = round_clamp_u8(div_rn(src[i], scale) + 16.0f, 31.0f);
        const uint8_t low = q & 0x0F, high = (q >> 4) & 1;
        out[6 + i / 2] |= static_cast<uint8_t>((i & 1) ? (low << 4) : low);
        if (high) out[2 + i / 8] |= static_cast<uint8_t>(1u << (i % 8));
    }
    for (int i = 0; i < 22; ++i) dst[i] = out[i];
}

OBJ_HD void iq3_block(const float* src, uint8_t* dst) {
    const float amax = block_amax(src);
    const float scale = amax > 0.0f ? div_rn(amax, 4.0f) : 1.0e-10f;
    const uint16_t h = f32_to_f16_bits(scale);
    uint8_t out[14] = {};
    out[0] = static_cast<uint8_t>(h & 0xFF);
    out[1] = static_cast<uint8_t>(h >> 8);
    for (int i = 0; i < 32; ++i) {
        const uint8_t q = round_clamp_u8(div_rn(src[i], scale) + 4.0f, 7.0f);
        out[2 + i / 4] |= static_cast<uint8_t>((q & 3) << (2 * (i % 4)));
        out[10 + i / 8] |= static_cast<uint8_t>(((q >> 2) & 1) << (i % 8));
    }
    for (int i = 0; i < 14; ++i) dst[i] = out[i];
}

OBJ_HD void fp4_block(const float* src, uint8_t* dst) {
    const uint8_t raw = fp4_scale_raw(block_amax(src));
    dst[0] = raw;
    const float s = decode_e8m0(raw);
    for (int i = 0; i < 16; ++i) {
        const uint8_t q0 = fp4_quantize_val(src[2 * i], s);
        const uint8_t q1 = fp4_quantize_val(src[2 * i + 1], s);
        dst[1 + i] = static_cast<uint8_t>(q0 | (q1 << 4));
    }
}

// ------------------------------------------- FP8 official arithmetic (DeepSeek)
// f8e4m3_to_f32 (crates/objeta-parser/src/deepseek.rs:799-829): exponent field 0
// decodes as mant * 2^-5 (the reference's subnormal rule), 15 as +-448, the rest as
// normals (sign, exponent + 120, mantissa << 20).
OBJ_HD float f8e4m3_to_f32(uint32_t raw) {
    const uint32_t sign = (raw & 0x80u) << 24;
    const uint32_t exp = (raw >> 3) & 0x0Fu, mant = raw & 0x07u;
    if (exp == 0) return u2f(f2u(static_cast<float>(mant) * 0.03125f) | sign);
    if (exp == 15) return u2f(f2u(448.0f) | sign);
    return u2f(sign | ((exp + 120u) << 23) | (mant << 20));
}

// f32_to_f8e4m3_exact (deepseek.rs:1444-1473). Below 1/128 the reference rounds
// |v| * 16 (always < 0.125, so the code is a signed zero); at or above 448 it
// saturates to 0x7E / 0xFE; otherwise the exponent is biased by 7 (clamped at 0),
// the mantissa rounded half-up to 3 bits, and exponents above 14 saturate to 0x77.
OBJ_HD uint8_t f32_to_f8e4m3_exact(float v) {
    const uint32_t bits = f2u(v);
    const uint32_t abits = bits & 0x7FFFFFFFu;
    const float a = u2f(abits);
    const bool neg = v < 0.0f;  // false for NaN, as in the reference
    if (a < 1.0f / 128.0f) {
        const float q = __builtin_roundf(a * 16.0f);
        const uint32_t quant = q >= 7.0f ? 7u : static_cast<uint32_t>(q);
        return static_cast<uint8_t>((neg ? 0x80u : 0u) | quant);
    }
    if (a >= 448.0f) return neg ? 0xFEu : 0x7Eu;
    int32_t exp_f8 = static_cast<int32_t>((abits >> 23) & 0xFFu) - 127 + 7;
    if (exp_f8 < 0) exp_f8 = 0;
    uint32_t mant3 = ((abits & 0x7FFFFFu) + (1u << 19)) >> 20;
    uint32_t exp_final = static_cast<uint32_t>(exp_f8) & 0xFFu;
    if (mant3 >= 8) {
        mant3 = 0;
        exp_final = exp_final == 255 ? 255 : exp_final + 1;
    }
    if (exp_final > 14) {
        exp_final = 14;
        mant3 = 7;
    }
    return static_cast<uint8_t>((neg ? 0x80u : 0u) | (exp_final << 3) | (mant3 & 7u));
}

// The block exponent of cpu_act_quant (deepseek.rs:1494-1513) for a block maximum
// amax (NaN already ignored): ceil(log2(max(amax, 1e-4) * (1 / 448))) with glibc's
// log2f (ceil_log2_cr); the scale is 2^result and its E8M0 byte result + 127.
OBJ_HD int32_t fp8_act_log2_scale(float amax) {
    const float m = amax > 1e-4f ? amax : 1e-4f;
    return ceil_log2_cr(m * (1.0f / 448.0f));
}
OBJ_HD uint8_t fp8_act_scale_raw(int32_t log2_scale) {
    const int32_t e = log2_scale + 127;
    return static_cast<uint8_t>(e < 0 ? 0 : (e > 255 ? 255 : e));
}

// The whole block scale of cpu_act_quant: its E8M0 byte and the factor that turns
// x / scale into one exact multiplication. For finite amax the exponent lies in
// [-22, 120], so 2^-exponent is a normal float and x * 2^-exponent rounds exactly
// as x / 2^exponent does. For amax = +inf the reference's `log2().ceil() as i32`
// saturates to i32::MAX: the byte `e = log2 + 127` wraps negative and clamps to 0,
// 2^i32::MAX is +inf and x / inf is x * 0 (+-0 for finite x, NaN for +-inf).
struct Fp8ActScale {
    uint8_t raw;
    float inv;
};
OBJ_HD Fp8ActScale fp8_act_scale(float amax) {
    if (amax == __builtin_inff()) return Fp8ActScale{0, 0.0f};
    const int32_t l = fp8_act_log2_scale(amax);
    return Fp8ActScale{fp8_act_scale_raw(l), u2f(static_cast<uint32_t>(127 - l) << 23)};
}

// One element of cpu_act_quant: clamp(x / scale, -448, 448) encoded (NaN stays NaN
// through the clamp, as f32::clamp keeps it).
OBJ_HD uint8_t fp8_act_code(float x, float inv) {
    float v = x * inv;
    if (v < -448.0f) v = -448.0f;
    else if (v > 448.0f) v = 448.0f;
    return f32_to_f8e4m3_exact(v);
}

// Counter-based synthetic generator: element i of stream `seed` is
// sigma * z with z an Irwin-Hall(12) draw from four splitmix64 words (3 x 21-bit
// fields each). The integer sum is exact and its centred value stays below 2^24,
// so the float conversion and the 2^-21 scaling are exact; only `* sigma` rounds.
OBJ_HD uint64_t splitmix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

OBJ_HD float gauss_from_key(uint64_t key, uint64_t i, float sigma) {
    const uint64_t base = key + 4ull * i;
    int32_t s = 0;
    for (uint64_t t = 0; t < 4; ++t) {
        const uint64_t w = splitmix64(base + t);
        s += static_cast<int32_t>(w & 0x1FFFFFu);
        s += static_cast<int32_t>((w >> 21) & 0x1FFFFFu);
        s += static_cast<int32_t>((w >> 42) & 0x1FFFFFu);
    }
    const float z = static_cast<float>(s - 12582906) * (1.0f / 2097152.0f);
    return z * sigma;
}

#undef OBJ_HD

}  // namespace rules
}  // namespace objeta
