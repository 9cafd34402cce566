/*
 * oracle.c — CPU restatement of the reference's selected-expert MoE decode path.
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.h). Compile with -O2 -ffp-contract=off and
 * without -ffast-math: every `a * b + c` below must round twice, as in Rust.
 */
#include "oracle.h"

#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* CudaErrorKind ordinals (crates/objeta-cuda/src/lib.rs:39-48); functions return kind+1. */
enum { K_DRIVER = 0, K_RUNTIME, K_NVRTC, K_IO, K_INVALID_INPUT, K_UNSUPPORTED, K_INTERNAL };

static int fail(int kind, char* err, size_t err_len, const char* fmt, ...)
    __attribute__((format(printf, 4, 5)));
static int fail(int kind, char* err, size_t err_len, const char* fmt, ...) {
    if (err && err_len) {
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(err, err_len, fmt, ap);
        va_end(ap);
    }
    return kind + 1;
}

static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

int orc_block_bytes(int fmt) {
    /* quant.rs:44-51 */
    switch (fmt) {
    case ORC_Q4_0: return 18;
    case ORC_Q5_0: return 22;
    case ORC_IQ3_0: return 14;
    case ORC_FP4: return 17;
    default: return -1;
    }
}

/* f16_to_f32_bits, quant.rs:1021-1044 */
float orc_f16_to_f32_bits(uint16_t bits) {
    uint32_t sign = ((uint32_t)(bits >> 15)) << 31;
    int32_t exp = (bits >> 10) & 0x1F;
    uint32_t mant = bits & 0x03FF;
    uint32_t f;
    if (exp == 0) {
        if (mant == 0) {
            f = sign;
        } else {
            uint32_t m = mant;
            int32_t e = -14;
            while ((m & 0x0400) == 0) { m <<= 1; e -= 1; }
            m &= 0x03FF;
            f = sign | ((uint32_t)(e + 127) << 23) | (m << 13);
        }
    } else if (exp == 0x1F) {
        f = sign | 0x7F800000u | (mant << 13);
    } else {
        f = sign | ((uint32_t)(exp - 15 + 127) << 23) | (mant << 13);
    }
    return u2f(f);
}

/* f32_to_f16_bits, quant.rs:1046-1079: round-half-up on bit 12, no sticky bit. */
uint16_t orc_f32_to_f16_bits(float value) {
    uint32_t bits = f2u(value);
    uint16_t sign = (uint16_t)((bits >> 16) & 0x8000);
    int32_t exp = (int32_t)((bits >> 23) & 0xFF);
    uint32_t mant = bits & 0x7FFFFF;
    if (exp == 255) {
        uint16_t nan_bits = mant == 0 ? 0 : 0x0200;
        return (uint16_t)(sign | 0x7C00 | nan_bits);
    }
    int32_t half_exp = exp - 127 + 15;
    if (half_exp >= 0x1F) return (uint16_t)(sign | 0x7C00);
    if (half_exp <= 0) {
        if (half_exp < -10) return sign;
        uint32_t mantissa = mant | 0x800000u;
        int32_t shift = 14 - half_exp;
        uint16_t half = (uint16_t)(mantissa >> shift);
        if ((mantissa >> (shift - 1)) & 1u) half = (uint16_t)(half + 1);
        return (uint16_t)(sign | half);
    }
    uint16_t half = (uint16_t)(sign | ((uint16_t)half_exp << 10) | (uint16_t)(mant >> 13));
    if (mant & 0x00001000u) half = (uint16_t)(half + 1);
    return half;
}

void orc_f32_to_f16_bits_n(const float* v, uint16_t* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = orc_f32_to_f16_bits(v[i]);
}
void orc_f16_to_f32_bits_n(const uint16_t* h, float* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = orc_f16_to_f32_bits(h[i]);
}

/* decode_f8_e8m0, quant.rs:886-892 */
float orc_decode_f8_e8m0(uint8_t raw) {
    if (raw == 0) return u2f(1u << 22);
    return u2f((uint32_t)raw << 23);
}

/* f8e8m0_to_f32, crates/objeta-parser/src/deepseek.rs:838-856 */
float orc_f8e8m0_to_f32(uint8_t raw) {
    int32_t exponent = (int32_t)raw - 127;
    if (exponent < -126) {
        if (exponent < -149) return 0.0f;
        return u2f(1u << (23 + (exponent + 126)));
    } else if (exponent > 127) {
        return INFINITY;
    }
    return u2f((uint32_t)(exponent + 127) << 23);
}

/* Rust `x.round().clamp(0.0, hi) as u8`: round half away from zero, clamp leaves
 * NaN alone, and the saturating `as u8` cast maps NaN to 0. */
static uint8_t round_clamp_u8(float v, float hi) {
    float r = roundf(v);
    if (r != r) return 0;
    if (r < 0.0f) r = 0.0f;
    if (r > hi) r = hi;
    return (uint8_t)r;
}

/* Rust `f as i32` (saturating, NaN -> 0). */
static int32_t sat_f32_to_i32(float f) {
    if (f != f) return 0;
    if (f >= 2147483648.0f) return INT32_MAX;
    if (f <= -2147483648.0f) return INT32_MIN;
    return (int32_t)f;
}

static float block_amax(const float* src) {
    /* amax = amax.max(v.abs()); f32::max ignores NaN like fmaxf. */
    float amax = 0.0f;
    for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(src[i]));
    return amax;
}

/* q4_quantize_block, quant.rs:814-829 */
void orc_q4_quantize_block(const float* src, uint8_t* dst) {
    float amax = block_amax(src);
    float scale = amax > 0.0f ? amax / 7.0f : 1.0e-10f;
    uint16_t h = orc_f32_to_f16_bits(scale);
    dst[0] = (uint8_t)(h & 0xFF);
    dst[1] = (uint8_t)(h >> 8);
    for (int i = 0; i < 16; ++i) {
        uint8_t q0 = round_clamp_u8((src[2 * i] / scale) + 8.0f, 15.0f);
        uint8_t q1 = round_clamp_u8((src[2 * i + 1] / scale) + 8.0f, 15.0f);
        dst[2 + i] = (uint8_t)(q0 | (q1 << 4));
    }
}

/* q5_quantize_block, quant.rs:831-858 */
void orc_q5_quantize_block(const float* src, uint8_t* dst) {
    float amax = block_amax(src);
    float scale = amax > 0.0f ? amax / 15.0f : 1.0e-10f;
    uint16_t h = orc_f32_to_f16_bits(scale);
    memset(dst, 0, 22);
    dst[0] = (uint8_t)(h & 0xFF);
    dst[1] = (uint8_t)(h >> 8);
    for (int i = 0; i < 32; ++i) {
        uint8_t q = round_clamp_u8((src[i] / scale) + 16.0f, 31.0f);
        uint8_t low = q & 0x0F;
        uint8_t high = (q >> 4) & 0x01;
        int nib = i / 2;
        if (i % 2 == 0) dst[6 + nib] = low;
        else dst[6 + nib] |= (uint8_t)(low << 4);
        if (high) dst[2 + i / 8] |= (uint8_t)(1u << (i % 8));
    }
}

/* iq3_quantize_block, quant.rs:860-879 */
void orc_iq3_quantize_block(const float* src, uint8_t* dst) {
    float amax = block_amax(src);
    float scale = amax > 0.0f ? amax / 4.0f : 1.0e-10f;
    uint16_t h = orc_f32_to_f16_bits(scale);
    memset(dst, 0, 14);
    dst[0] = (uint8_t)(h & 0xFF);
    dst[1] = (uint8_t)(h >> 8);
    for (int i = 0; i < 32; ++i) {
        uint8_t q = round_clamp_u8((src[i] / scale) + 4.0f, 7.0f);
        uint8_t low = q & 0x03;
        uint8_t high = (q >> 2) & 0x01;
        dst[2 + i / 4] |= (uint8_t)(low << (2 * (i % 4)));
        dst[10 + i / 8] |= (uint8_t)(high << (i % 8));
    }
}

/* FP4_TABLE, quant.rs:881-884 (entry 8 is -0.0 here). */
static const float FP4_TABLE[16] = {
    0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f,
    -0.0f, -0.5f, -1.0f, -1.5f, -2.0f, -3.0f, -4.0f, -6.0f,
};
/* FP4_E2M1FN_TABLE, crates/objeta-parser/src/deepseek.rs:791-794 (entry 8 is +0.0). */
static const float FP4_E2M1FN_TABLE[16] = {
    0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f,
    0.0f, -0.5f, -1.0f, -1.5f, -2.0f, -3.0f, -4.0f, -6.0f,
};

/* quantize_val, quant.rs:894-906: first minimum of |v/scale - table[q]|. */
static uint8_t fp4_quantize_val(float val, float scale) {
    float scaled = val / scale;
    int best = 0;
    float min_diff = INFINITY;
    for (int q = 0; q < 16; ++q) {
        float diff = fabsf(scaled - FP4_TABLE[q]);
        if (diff < min_diff) { min_diff = diff; best = q; }
    }
    return (uint8_t)best;
}

/* The E8M0 exponent choice of fp4_quantize_block, quant.rs:913-918. */
uint8_t orc_fp4_scale_raw(float amax) {
    if (amax > 0.0f && isfinite(amax)) {
        int32_t k = sat_f32_to_i32(ceilf(log2f(amax / 6.0f)));
        int64_t v = (int64_t)k + 127;
        if (v < 0) v = 0;
        if (v > 255) v = 255;
        return (uint8_t)v;
    }
    return 0;
}

void orc_fp4_scale_raw_n(const float* amax, uint8_t* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = orc_fp4_scale_raw(amax[i]);
}

/* fp4_quantize_block, quant.rs:908-926 */
void orc_fp4_quantize_block(const float* src, uint8_t* dst) {
    float amax = block_amax(src);
    uint8_t raw = orc_fp4_scale_raw(amax);
    dst[0] = raw;
    float s = orc_decode_f8_e8m0(raw);
    for (int i = 0; i < 16; ++i) {
        uint8_t q0 = fp4_quantize_val(src[2 * i], s);
        uint8_t q1 = fp4_quantize_val(src[2 * i + 1], s);
        dst[1 + i] = (uint8_t)(q0 | (q1 << 4));
    }
}

static const char* fmt_label(int fmt) {
    switch (fmt) {
    case ORC_Q4_0: return "q4_0";
    case ORC_Q5_0: return "q5_0";
    case ORC_IQ3_0: return "iq3_0";
    case ORC_FP4: return "deepseek_fp4_e2m1";
    default: return "?";
    }
}

/* quantize_matrix_cpu, quant.rs:506-581; validate_dense_matrix, quant.rs:725-749 */
int orc_quantize_matrix(int fmt, const float* m, size_t m_len, size_t rows, size_t cols,
                        uint8_t* out, size_t out_len, char* err, size_t err_len) {
    int bb = orc_block_bytes(fmt);
    if (bb < 0) return fail(K_INVALID_INPUT, err, err_len, "unknown format %d", fmt);
    if (m_len != rows * cols)
        return fail(K_INVALID_INPUT, err, err_len, "matrix len %zu != rows*cols %zu", m_len,
                    rows * cols);
    if (cols % 32 != 0)
        return fail(K_INVALID_INPUT, err, err_len,
                    "cols %zu must be a multiple of block_size %d", cols, 32);
    size_t nb = cols / 32, row_bytes = nb * (size_t)bb;
    if (out_len != rows * row_bytes)
        return fail(K_INVALID_INPUT, err, err_len, "output len %zu != expected %zu", out_len,
                    rows * row_bytes);
    (void)fmt_label;
    for (size_t r = 0; r < rows; ++r) {
        for (size_t b = 0; b < nb; ++b) {
            const float* src = m + r * cols + b * 32;
            uint8_t* dst = out + r * row_bytes + b * (size_t)bb;
            switch (fmt) {
            case ORC_Q4_0: orc_q4_quantize_block(src, dst); break;
            case ORC_Q5_0: orc_q5_quantize_block(src, dst); break;
            case ORC_IQ3_0: orc_iq3_quantize_block(src, dst); break;
            default: orc_fp4_quantize_block(src, dst); break;
            }
        }
    }
    return 0;
}

static float rd_f16(const uint8_t* p) { return orc_f16_to_f32_bits((uint16_t)(p[0] | (p[1] << 8))); }

/* q4/q5/iq3/fp4_dot_row, quant.rs:928-1019: sequential sum, product rounded
 * before the add. */
float orc_dot_row(int fmt, const uint8_t* row_q, const float* x, size_t cols) {
    size_t nb = cols / 32;
    float sum = 0.0f;
    for (size_t b = 0; b < nb; ++b) {
        if (fmt == ORC_Q4_0) {
            const uint8_t* blk = row_q + b * 18;
            float scale = rd_f16(blk);
            for (int lane = 0; lane < 32; ++lane) {
                size_t col = b * 32 + (size_t)lane;
                uint8_t packed = blk[2 + lane / 2];
                uint8_t q = (lane % 2 == 0) ? (packed & 0x0F) : (packed >> 4);
                float w = (float)((int)q - 8) * scale;
                if (col < cols) sum = sum + w * x[col];
            }
        } else if (fmt == ORC_Q5_0) {
            const uint8_t* blk = row_q + b * 22;
            float scale = rd_f16(blk);
            for (int lane = 0; lane < 32; ++lane) {
                size_t col = b * 32 + (size_t)lane;
                uint8_t lb = blk[6 + lane / 2];
                uint8_t low = (lane % 2 == 0) ? (lb & 0x0F) : (lb >> 4);
                uint8_t high = (blk[2 + lane / 8] >> (lane % 8)) & 0x01;
                uint8_t q = (uint8_t)(low | (high << 4));
                float w = (float)((int)q - 16) * scale;
                if (col < cols) sum = sum + w * x[col];
            }
        } else if (fmt == ORC_IQ3_0) {
            const uint8_t* blk = row_q + b * 14;
            float scale = rd_f16(blk);
            for (int lane = 0; lane < 32; ++lane) {
                size_t col = b * 32 + (size_t)lane;
                uint8_t low = (blk[2 + lane / 4] >> (2 * (lane % 4))) & 0x03;
                uint8_t high = (blk[10 + lane / 8] >> (lane % 8)) & 0x01;
                uint8_t q = (uint8_t)(low | (high << 2));
                float w = (float)((int)q - 4) * scale;
                if (col < cols) sum = sum + w * x[col];
            }
        } else {
            const uint8_t* blk = row_q + b * 17;
            float scale = orc_decode_f8_e8m0(blk[0]);
            for (int lane = 0; lane < 32; ++lane) {
                size_t col = b * 32 + (size_t)lane;
                if (col < cols) {
                    uint8_t packed = blk[1 + lane / 2];
                    uint8_t q = (lane % 2 == 0) ? (packed & 0x0F) : (packed >> 4);
                    float w = FP4_TABLE[q] * scale;
                    sum = sum + w * x[col];
                }
            }
        }
    }
    return sum;
}

/* Threads of the row loops (GEMV rows, router logits, FP4 decode rows). Each row's
 * sum stays one sequential loop, so the results do not depend on the count; the
 * reference's CPU path is single-threaded (1, the default), more threads give the
 * row-parallel CPU baseline. */
static int g_threads = 1;
void orc_set_threads(int n) { g_threads = n < 1 ? 1 : n; }
int orc_get_threads(void) { return g_threads; }

/* gemv_cpu, quant.rs:627-646; validate_quant_inputs, quant.rs:751-793 */
int orc_gemv(int fmt, const uint8_t* q, size_t q_len, const float* x, size_t x_len,
             size_t rows, size_t cols, float* y, char* err, size_t err_len) {
    int bb = orc_block_bytes(fmt);
    if (bb < 0) return fail(K_INVALID_INPUT, err, err_len, "unknown format %d", fmt);
    if (cols % 32 != 0)
        return fail(K_INVALID_INPUT, err, err_len,
                    "cols %zu must be a multiple of block_size %d", cols, 32);
    size_t row_bytes = (cols / 32) * (size_t)bb;
    if (q_len != rows * row_bytes)
        return fail(K_INVALID_INPUT, err, err_len, "qweights len %zu != expected %zu", q_len,
                    rows * row_bytes);
    if (x_len != cols)
        return fail(K_INVALID_INPUT, err, err_len, "x len %zu != cols %zu", x_len, cols);
#pragma omp parallel for num_threads(g_threads) if (g_threads > 1) schedule(static)
    for (size_t r = 0; r < rows; ++r) y[r] = orc_dot_row(fmt, q + r * row_bytes, x, cols);
    return 0;
}

/* dense_gemv_cpu, quant.rs:599-625. Rust's f32 `Sum` folds from -0.0 (current
 * std); the start value only shows in the sign of an all-(-0.0) row. */
static float dense_row(const float* row, const float* x, size_t cols) {
    float s = -0.0f;
    for (size_t c = 0; c < cols; ++c) s = s + row[c] * x[c];
    return s;
}

int orc_dense_gemv(const float* m, size_t m_len, const float* x, size_t x_len, size_t rows,
                   size_t cols, float* y, char* err, size_t err_len) {
    if (m_len != rows * cols)
        return fail(K_INVALID_INPUT, err, err_len, "matrix len %zu != rows * cols %zu", m_len,
                    rows * cols);
    if (x_len != cols)
        return fail(K_INVALID_INPUT, err, err_len, "vector len %zu != cols %zu", x_len, cols);
#pragma omp parallel for num_threads(g_threads) if (g_threads > 1) schedule(static)
    for (size_t r = 0; r < rows; ++r) y[r] = dense_row(m + r * cols, x, cols);
    return 0;
}

/* decode_deepseek_fp4_to_f32, crates/objeta-parser/src/deepseek.rs:866-918 */
void orc_decode_fp4_split(const uint8_t* w, const uint8_t* s, size_t rows, size_t cols,
                          float* out) {
    size_t phys = cols / 2, scols = cols / 32;
#pragma omp parallel for num_threads(g_threads) if (g_threads > 1) schedule(static)
    for (size_t r = 0; r < rows; ++r) {
        for (size_t g = 0; g < phys; ++g) {
            uint8_t b = w[r * phys + g];
            size_t lo = g * 2, hi = lo + 1;
            float s_lo = orc_f8e8m0_to_f32(s[r * scols + lo / 32]);
            float s_hi = orc_f8e8m0_to_f32(s[r * scols + hi / 32]);
            out[r * cols + lo] = FP4_E2M1FN_TABLE[b & 0x0F] * s_lo;
            out[r * cols + hi] = FP4_E2M1FN_TABLE[(b >> 4) & 0x0F] * s_hi;
        }
    }
}

void orc_fp4_split_gemv(const uint8_t* w, const uint8_t* s, const float* x, size_t rows,
                        size_t cols, float* y) {
    float* row = (float*)malloc(cols * sizeof(float));
    size_t phys = cols / 2, scols = cols / 32;
    for (size_t r = 0; r < rows; ++r) {
        orc_decode_fp4_split(w + r * phys, s + r * scols, 1, cols, row);
        y[r] = dense_row(row, x, cols);
    }
    free(row);
}

/* silu·mul of selected_moe_cpu, moe.rs:1308-1315 */
static void silu_mul(const float* gate, const float* up, float* act, size_t n) {
    for (size_t i = 0; i < n; ++i) {
        float g = gate[i];
        float silu = g / (1.0f + expf(-g));
        act[i] = silu * up[i];
    }
}

int orc_selected_moe(int fmt, size_t n_experts, const void* const* gate,
                     const void* const* up, const void* const* down,
                     const uint8_t* const* gate_s, const uint8_t* const* up_s,
                     const uint8_t* const* down_s, const uint32_t* sel_ids,
                     const float* sel_w, size_t k, const float* x, size_t hidden,
                     size_t inter, size_t out_dim, float* out, char* err, size_t err_len) {
    int rc = 0;
    for (size_t i = 0; i < out_dim; ++i) out[i] = 0.0f;
    float* g = (float*)malloc(inter * sizeof(float));
    float* u = (float*)malloc(inter * sizeof(float));
    float* a = (float*)malloc(inter * sizeof(float));
    float* d = (float*)malloc(out_dim * sizeof(float));
    float* deq = NULL;
    if (fmt == ORC_FP4) {
        size_t big = inter * hidden > out_dim * inter ? inter * hidden : out_dim * inter;
        deq = (float*)malloc(big * sizeof(float));
    }
    for (size_t j = 0; j < k && rc == 0; ++j) {
        size_t e = sel_ids[j];
        float wt = sel_w[j];
        if (e >= n_experts) {
            rc = fail(K_INVALID_INPUT, err, err_len, "expert index %zu out of bounds (len=%zu)",
                      e, n_experts);
            break;
        }
        if (fmt == -1) {
            /* selected_moe_cpu_fp32, moe.rs:1326-1367 */
            orc_dense_gemv((const float*)gate[e], inter * hidden, x, hidden, inter, hidden, g, 0, 0);
            orc_dense_gemv((const float*)up[e], inter * hidden, x, hidden, inter, hidden, u, 0, 0);
            silu_mul(g, u, a, inter);
            orc_dense_gemv((const float*)down[e], out_dim * inter, a, inter, out_dim, inter, d, 0, 0);
        } else if (fmt == ORC_FP4) {
            /* selected_moe_cpu_native_fp4, moe.rs:1665-1735 */
            orc_decode_fp4_split((const uint8_t*)gate[e], gate_s[e], inter, hidden, deq);
            orc_dense_gemv(deq, inter * hidden, x, hidden, inter, hidden, g, 0, 0);
            orc_decode_fp4_split((const uint8_t*)up[e], up_s[e], inter, hidden, deq);
            orc_dense_gemv(deq, inter * hidden, x, hidden, inter, hidden, u, 0, 0);
            silu_mul(g, u, a, inter);
            orc_decode_fp4_split((const uint8_t*)down[e], down_s[e], out_dim, inter, deq);
            orc_dense_gemv(deq, out_dim * inter, a, inter, out_dim, inter, d, 0, 0);
        } else {
            /* selected_moe_cpu, moe.rs:1283-1324 (Q4_0 there; the block formats share
             * the loop through gemv_cpu). */
            int bb = orc_block_bytes(fmt);
            if (bb < 0 || fmt == ORC_FP4) {
                rc = fail(K_UNSUPPORTED, err, err_len, "unsupported MoE format %d", fmt);
                break;
            }
            size_t gu_bytes = inter * (hidden / 32) * (size_t)bb;
            size_t dn_bytes = out_dim * (inter / 32) * (size_t)bb;
            rc = orc_gemv(fmt, (const uint8_t*)gate[e], gu_bytes, x, hidden, inter, hidden, g, err, err_len);
            if (!rc) rc = orc_gemv(fmt, (const uint8_t*)up[e], gu_bytes, x, hidden, inter, hidden, u, err, err_len);
            if (rc) break;
            silu_mul(g, u, a, inter);
            rc = orc_gemv(fmt, (const uint8_t*)down[e], dn_bytes, a, inter, out_dim, inter, d, err, err_len);
            if (rc) break;
        }
        for (size_t i = 0; i < out_dim; ++i) out[i] = out[i] + wt * d[i];
    }
    free(g); free(u); free(a); free(d); free(deq);
    return rc;
}

/* cpu_router, crates/objeta-cuda/src/bin/deepseek_single_layer_moe.rs:687-743, plus the
 * optional bias add and renormalisation described in oracle.h. */
int orc_router(const float* w_r, const float* bias, const float* x, size_t n_experts,
               size_t hidden, size_t k, int renormalize, uint32_t* ids, float* weights,
               float* logits_out, float* probs_out, char* err, size_t err_len) {
    if (k == 0 || k > n_experts)
        return fail(K_INVALID_INPUT, err, err_len, "top_k %zu must be in 1..=num_experts %zu", k,
                    n_experts);
    float* logits = (float*)malloc(n_experts * sizeof(float));
    float* probs = (float*)malloc(n_experts * sizeof(float));
    uint32_t* order = (uint32_t*)malloc(n_experts * sizeof(uint32_t));
#pragma omp parallel for num_threads(g_threads) if (g_threads > 1) schedule(static)
    for (size_t e = 0; e < n_experts; ++e) {
        float sum = 0.0f;
        const float* row = w_r + e * hidden;
        for (size_t h = 0; h < hidden; ++h) sum = sum + row[h] * x[h];
        if (bias) sum = sum + bias[e];
        logits[e] = sum;
    }
    float mx = -INFINITY;
    for (size_t e = 0; e < n_experts; ++e) mx = fmaxf(mx, logits[e]);
    float sum_exp = 0.0f;
    for (size_t e = 0; e < n_experts; ++e) {
        float v = expf(logits[e] - mx);
        probs[e] = v;
        sum_exp = sum_exp + v;
    }
    for (size_t e = 0; e < n_experts; ++e) probs[e] = probs[e] / sum_exp;
    /* Stable sort, descending probability (Rust sort_by is stable; ties keep the
     * lower index first). Insertion sort is stable. */
    for (size_t e = 0; e < n_experts; ++e) order[e] = (uint32_t)e;
    for (size_t i = 1; i < n_experts; ++i) {
        size_t j = i;
        while (j > 0 && probs[order[j - 1]] < probs[order[j]]) {
            uint32_t t = order[j - 1]; order[j - 1] = order[j]; order[j] = t;
            --j;
        }
    }
    float sel_sum = 0.0f;
    for (size_t j = 0; j < k; ++j) sel_sum = sel_sum + probs[order[j]];
    for (size_t j = 0; j < k; ++j) {
        ids[j] = order[j];
        weights[j] = renormalize ? probs[order[j]] / sel_sum : probs[order[j]];
    }
    if (logits_out) memcpy(logits_out, logits, n_experts * sizeof(float));
    if (probs_out) memcpy(probs_out, probs, n_experts * sizeof(float));
    free(logits); free(probs); free(order);
    return 0;
}

/* compare_outputs, quant.rs:676-723 */
int orc_compare(const float* ref, const float* act, size_t n, float* out3) {
    double dot = 0.0, rn = 0.0, an = 0.0, sq = 0.0;
    float max_abs = 0.0f;
    for (size_t i = 0; i < n; ++i) {
        double r = ref[i], a = act[i];
        dot += r * a;
        rn += r * r;
        an += a * a;
        float diff = act[i] - ref[i];
        sq += (double)diff * (double)diff;
        max_abs = fmaxf(max_abs, fabsf(diff));
    }
    out3[0] = (rn > 0.0 && an > 0.0) ? (float)(dot / (sqrt(rn) * sqrt(an))) : 1.0f;
    out3[1] = rn > 0.0 ? (float)(sqrt(sq) / sqrt(rn)) : 0.0f;
    out3[2] = max_abs;
    return 0;
}

/* seeded_f32s, crates/objeta-cuda/src/bin/bench_qgemv.rs:39-49 */
void orc_seeded_f32s(uint64_t seed, float* out, size_t n) {
    uint64_t state = seed;
    for (size_t i = 0; i < n; ++i) {
        state = state * 6364136223846793005ULL + 1ULL;
        uint32_t bits = ((uint32_t)(state >> 32)) | 1u;
        float unit = (float)bits / (float)UINT32_MAX;
        out[i] = (unit * 2.0f) - 1.0f;
    }
}

uint64_t orc_splitmix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ULL;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

/* Irwin-Hall(12) from four splitmix64 words, 3 x 21-bit fields each. The integer
 * sum is exact; its centred value is < 2^24 in magnitude, so the float conversion
 * and the 2^-21 scaling are exact and only the final `* sigma` rounds. */
float orc_gauss(uint64_t seed, uint64_t i, float sigma) {
    uint64_t key = orc_splitmix64(seed) + 4ULL * i;
    int32_t s = 0;
    for (uint64_t t = 0; t < 4; ++t) {
        uint64_t w = orc_splitmix64(key + t);
        s += (int32_t)(w & 0x1FFFFF);
        s += (int32_t)((w >> 21) & 0x1FFFFF);
        s += (int32_t)((w >> 42) & 0x1FFFFF);
    }
    float z = (float)(s - 12582906) * (1.0f / 2097152.0f);
    return z * sigma;
}

void orc_gauss_fill(uint64_t seed, uint64_t first, float sigma, float* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = orc_gauss(seed, first + i, sigma);
}

/* ------------------------------------------------------------- expf restated
 * glibc (2.28 and later) computes expf with the method of Arm's optimized-routines
 * (Szabolcs Nagy, 2017): in double, x * 32/ln2 = k + r with k the nearest integer
 * (through the 1.5 * 2^52 shift), 2^(k/32) from a 32-entry table of 2^(i/32),
 * 2^(r/32) from a degree-3 polynomial, one final rounding to float. On x86-64 with
 * FMA (the GPU hosts' CPUs) glibc selects the build of it with the products fused
 * into the adds that consume them, which is the form below: it agrees with glibc's
 * expf on every argument (tests/test_oracle_crosscheck.py checks all of
 * [-110, 0] and samples of the rest). Table entry i is the correctly rounded double
 * 2^(i/32) with i << 47 subtracted, so that adding k << 47 yields 2^(k/32). */
static const uint64_t kExp2Tab[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull};

static uint32_t f32_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, sizeof u);
    return u;
}
static float bits_f32(uint32_t u) {
    float f;
    memcpy(&f, &u, sizeof f);
    return f;
}
static double bits_f64(uint64_t u) {
    double d;
    memcpy(&d, &u, sizeof d);
    return d;
}
static uint64_t f64_bits(double d) {
    uint64_t u;
    memcpy(&u, &d, sizeof u);
    return u;
}

float orc_expf_restated(float x) {
    const uint32_t ux = f32_bits(x);
    const uint32_t abstop = (ux >> 20) & 0x7ff;
    if (abstop >= 0x42b) { /* |x| >= 88, inf or nan */
        if (ux == 0xff800000u) return 0.0f;
        if (abstop >= 0x7f8) return x + x;
        if (x > 0x1.62e42ep6f) return INFINITY;
        if (x < -0x1.9fe368p6f) return 0.0f;
    }
    const double inv_ln2_n = 0x1.71547652b82fep+0 * 32, shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32, c1 = 0x1.ebfce50fac4f3p-3 / 32 / 32,
                 c2 = 0x1.62e42ff0c52d6p-1 / 32;
    const double xd = (double)x;
    double kd = fma(inv_ln2_n, xd, shift);
    const uint64_t ki = f64_bits(kd);
    kd -= shift;
    const double r = fma(inv_ln2_n, xd, -kd);
    const double s = bits_f64(kExp2Tab[ki % 32] + (ki << 47));
    const double z = fma(c0, r, c1);
    const double r2 = r * r;
    double y = fma(c2, r, 1.0);
    y = fma(z, r2, y);
    return (float)(y * s);
}

void orc_expf_glibc(const float* in, float* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = expf(in[i]);
}

void orc_expf_range_check(uint32_t lo_bits, uint32_t hi_bits, uint64_t* restated_mismatch,
                          uint64_t* double_mismatch) {
    uint64_t a = 0, b = 0;
#pragma omp parallel for reduction(+ : a, b) schedule(static)
    for (int64_t u = (int64_t)lo_bits; u <= (int64_t)hi_bits; ++u) {
        const float x = bits_f32((uint32_t)u);
        const uint32_t g = f32_bits(expf(x));
        if (f32_bits(orc_expf_restated(x)) != g) ++a;
        if (f32_bits((float)exp((double)x)) != g) ++b;
    }
    *restated_mismatch = a;
    *double_mismatch = b;
}

size_t orc_expf_double_disagreements(uint32_t lo_bits, uint32_t hi_bits, float* out, size_t cap) {
    size_t n = 0;
#pragma omp parallel for schedule(static)
    for (int64_t u = (int64_t)lo_bits; u <= (int64_t)hi_bits; ++u) {
        const float x = bits_f32((uint32_t)u);
        if (f32_bits((float)exp((double)x)) != f32_bits(expf(x))) {
            size_t slot;
#pragma omp atomic capture
            slot = n++;
            if (slot < cap) out[slot] = x;
        }
    }
    return n;
}

/* ------------------------------------------------------ FP8 official arithmetic
 * The DeepSeek "official arithmetic" CPU path of crates/objeta-parser/src/deepseek.rs:
 * activations quantized to F8_E4M3 bytes with one F8_E8M0 scale per 128 elements,
 * FP8 x FP4 and FP8 x FP8 GEMVs, and the routed / shared expert compositions. */

/* f8e4m3_to_f32, deepseek.rs:799-829: exponent field 0 decodes as mant * 2^-5 (the
 * reference's subnormal rule), 15 as +-448, the rest as IEEE-style normals. */
float orc_f8e4m3_to_f32(uint8_t raw) {
    const uint32_t sign = raw >> 7, exp = (raw >> 3) & 0x0Fu, mant = raw & 0x07u;
    if (exp == 0) {
        if (mant == 0) return u2f(sign << 31);
        return (float)mant * 0.03125f * (sign == 0 ? 1.0f : -1.0f); /* 2f32.powi(1 - 6) = 2^-5 */
    }
    if (exp == 15) return sign == 0 ? 448.0f : -448.0f;
    return u2f((sign << 31) | ((exp + 120u) << 23) | (mant << 20));
}

/* f32_to_f8e4m3_exact, deepseek.rs:1444-1473. */
uint8_t orc_f32_to_f8e4m3_exact(float v) {
    if (fabsf(v) < 1.0f / 128.0f) { /* below min normal */
        const uint8_t sign = v < 0.0f ? 0x80u : 0u;
        const float scaled = fabsf(v) * 16.0f;
        float q = roundf(scaled); /* f32::round, half away from zero; `as u8` saturates */
        uint8_t quant = q >= 255.0f ? 255u : (uint8_t)q;
        return (uint8_t)(sign | (quant < 7 ? quant : 7));
    }
    if (fabsf(v) >= 448.0f) return v < 0.0f ? 0xFEu : 0x7Eu;
    const uint8_t sign = v < 0.0f ? 0x80u : 0u;
    const uint32_t bits = f2u(fabsf(v));
    const int32_t exp32 = (int32_t)((bits >> 23) & 0xFFu) - 127;
    int32_t exp_f8 = exp32 + 7;
    if (exp_f8 < 0) exp_f8 = 0;
    const uint32_t mant_bits = bits & 0x7FFFFFu;
    uint8_t mant3 = (uint8_t)((mant_bits + (1u << 19)) >> 20);
    uint8_t exp_final = (uint8_t)exp_f8;
    if (mant3 >= 8) {
        mant3 = 0;
        exp_final = exp_final == 255 ? 255 : (uint8_t)(exp_final + 1);
    }
    if (exp_final > 14) {
        exp_final = 14;
        mant3 = 7;
    }
    return (uint8_t)(sign | (exp_final << 3) | (mant3 & 7));
}

/* cpu_act_quant, deepseek.rs:1484-1525: per block, amax = max |x| (NaN ignored) and at
 * least 1e-4; scale = 2^ceil(log2(amax * (1/448))); y = f32_to_f8e4m3_exact(clamp(x /
 * scale, -448, 448)); s = clamp(log2 scale + 127, 0, 255). n % block == 0. */
void orc_act_quant(const float* x, size_t n, size_t block, uint8_t* y, uint8_t* s) {
    const float fp8_max = 448.0f, fp8_max_inv = 1.0f / 448.0f;
    for (size_t b = 0; b < n / block; ++b) {
        const size_t start = b * block, end = start + block;
        float amax = 0.0f;
        for (size_t i = start; i < end; ++i) {
            const float a = fabsf(x[i]);
            if (a > amax) amax = a;
        }
        amax = fmaxf(amax, 1e-4f);
        const float raw = amax * fp8_max_inv;
        float scale;
        if (isinf(raw)) {
            /* `inf.log2().ceil() as i32` saturates to i32::MAX; e = MAX + 127 wraps
             * negative in a release build (byte 0) and 2f32.powi(MAX) is +inf */
            scale = INFINITY;
            s[b] = 0;
        } else {
            const int32_t log2_ceil = raw > 0.0f ? (int32_t)ceilf(log2f(raw)) : -127;
            /* 2.0f32.powi(log2_ceil): an exact power of two over the range raw can take */
            scale = ldexpf(1.0f, log2_ceil);
            const int32_t e = log2_ceil + 127;
            s[b] = (uint8_t)(e < 0 ? 0 : (e > 255 ? 255 : e));
        }
        for (size_t i = start; i < end; ++i) {
            float v = x[i] / scale;
            if (v < -fp8_max) v = -fp8_max;
            else if (v > fp8_max) v = fp8_max;
            y[i] = orc_f32_to_f8e4m3_exact(v);
        }
    }
}

/* cpu_fp8_act_fp4_weight_gemv_f32, deepseek.rs:1528-1566: per row, over byte
 * col_group, the low then the high nibble, sum += act_v * act_s * fp4 * ws in f32. */
void orc_fp8_act_fp4_weight_gemv_f32(const uint8_t* act_v, const uint8_t* act_s, const uint8_t* w,
                                     const uint8_t* ws, size_t rows, size_t cols, float* out) {
    const size_t phys = cols / 2, scols = cols / 32;
#pragma omp parallel for num_threads(g_threads) if (g_threads > 1) schedule(static)
    for (size_t r = 0; r < rows; ++r) {
        float sum = 0.0f;
        for (size_t g = 0; g < phys; ++g) {
            const uint8_t bv = w[r * phys + g];
            const size_t lo = g * 2, hi = lo + 1;
            const float fp4_lo = FP4_E2M1FN_TABLE[bv & 0x0F], fp4_hi = FP4_E2M1FN_TABLE[(bv >> 4) & 0x0F];
            const float ws_lo = orc_f8e8m0_to_f32(ws[r * scols + lo / 32]);
            const float ws_hi = orc_f8e8m0_to_f32(ws[r * scols + hi / 32]);
            const float av_lo = orc_f8e4m3_to_f32(act_v[lo]), av_hi = orc_f8e4m3_to_f32(act_v[hi]);
            const float as_lo = orc_f8e8m0_to_f32(act_s[lo / 128]), as_hi = orc_f8e8m0_to_f32(act_s[hi / 128]);
            sum = sum + av_lo * as_lo * fp4_lo * ws_lo;
            sum = sum + av_hi * as_hi * fp4_hi * ws_hi;
        }
        out[r] = sum;
    }
}

/* cpu_fp8_act_fp8_weight_gemv, deepseek.rs:1630-1661: weight scales on a 128 x 128
 * tile grid [ceil(rows/128)][ceil(cols/128)], products and sum in f64, result
 * rounded to f32. */
void orc_fp8_act_fp8_weight_gemv(const uint8_t* act_v, const uint8_t* act_s, const uint8_t* w,
                                 const uint8_t* ws, size_t rows, size_t cols, float* out) {
    const size_t wt_scale_cols = (cols + 127) / 128;
#pragma omp parallel for num_threads(g_threads) if (g_threads > 1) schedule(static)
    for (size_t r = 0; r < rows; ++r) {
        const size_t srow = r / 128;
        double sum = 0.0;
        for (size_t c = 0; c < cols; ++c) {
            const float av = orc_f8e4m3_to_f32(act_v[c]);
            const float as = orc_f8e8m0_to_f32(act_s[c / 128]);
            const float wv = orc_f8e4m3_to_f32(w[r * cols + c]);
            const float wsv = orc_f8e8m0_to_f32(ws[srow * wt_scale_cols + c / 128]);
            sum += (double)av * (double)as * (double)wv * (double)wsv;
        }
        out[r] = (float)sum;
    }
}

/* The SwiGLU of the official compositions (deepseek.rs:1680-1686, 1708-1713): only the
 * up projection is clamped; act = g / (1 + exp(-g)) * clamp(u). */
static void official_swiglu(const float* g, const float* u, float* act, size_t n, float limit) {
    for (size_t i = 0; i < n; ++i) {
        float uc = u[i];
        if (uc < -limit) uc = -limit;
        else if (uc > limit) uc = limit;
        act[i] = g[i] / (1.0f + expf(-g[i])) * uc;
    }
}

/* cpu_routed_expert_fp4_official_f32 (deepseek.rs:1694-1716) with FP4 split weights,
 * and cpu_shared_expert_fp8_official (deepseek.rs:1664-1692) with FP8 weights on a
 * 128 x 128 scale tile grid. act_pre (nullable, [inter]) receives the activation
 * before its act_quant, act_q / act_qs (nullable) its FP8 bytes and scales. */
int orc_expert_official(int fp8_weights, const uint8_t* gw, const uint8_t* gs, const uint8_t* uw,
                        const uint8_t* us, const uint8_t* dw, const uint8_t* ds, const float* x,
                        size_t dim, size_t inter, float swiglu_limit, float* out, float* act_pre,
                        uint8_t* act_q, uint8_t* act_qs, char* err, size_t err_len) {
    if (dim % 128 != 0 || inter % 128 != 0)
        return fail(K_INVALID_INPUT, err, err_len, "dim %zu and inter %zu must be multiples of 128", dim, inter);
    uint8_t* xq = (uint8_t*)malloc(dim);
    uint8_t* xs = (uint8_t*)malloc(dim / 128);
    float* g = (float*)malloc(inter * sizeof(float));
    float* u = (float*)malloc(inter * sizeof(float));
    float* a = (float*)malloc(inter * sizeof(float));
    uint8_t* aq = (uint8_t*)malloc(inter);
    uint8_t* as = (uint8_t*)malloc(inter / 128);
    orc_act_quant(x, dim, 128, xq, xs);
    if (fp8_weights) {
        orc_fp8_act_fp8_weight_gemv(xq, xs, gw, gs, inter, dim, g);
        orc_fp8_act_fp8_weight_gemv(xq, xs, uw, us, inter, dim, u);
    } else {
        orc_fp8_act_fp4_weight_gemv_f32(xq, xs, gw, gs, inter, dim, g);
        orc_fp8_act_fp4_weight_gemv_f32(xq, xs, uw, us, inter, dim, u);
    }
    official_swiglu(g, u, a, inter, swiglu_limit);
    orc_act_quant(a, inter, 128, aq, as);
    if (fp8_weights) orc_fp8_act_fp8_weight_gemv(aq, as, dw, ds, dim, inter, out);
    else orc_fp8_act_fp4_weight_gemv_f32(aq, as, dw, ds, dim, inter, out);
    if (act_pre) memcpy(act_pre, a, inter * sizeof(float));
    if (act_q) memcpy(act_q, aq, inter);
    if (act_qs) memcpy(act_qs, as, inter / 128);
    free(xq); free(xs); free(g); free(u); free(a); free(aq); free(as);
    return 0;
}

void orc_f8e4m3_to_f32_n(const uint8_t* raw, float* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = orc_f8e4m3_to_f32(raw[i]);
}
void orc_f32_to_f8e4m3_exact_n(const float* v, uint8_t* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = orc_f32_to_f8e4m3_exact(v[i]);
}
