/*
 * oracle.h — CPU restatement of the reference's selected-expert MoE decode path.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product library links, loads or
 * calls this code. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may use it, and there only as the checker (or as the timed
 * CPU baseline), never as the thing measured or shipped.
 *
 * Built with `gcc -O2 -ffp-contract=off` (no -ffast-math) so that every f32
 * multiply and add rounds separately, exactly as the reference's Rust code does
 * (Rust never contracts a*b+c into an FMA). Each function cites the reference
 * file:line it restates; paths are relative to the reference repository root.
 *
 * Parity pinning (what checks each function against something other than a
 * retyping of this file) is listed in the tests: tests/test_oracle_*.py.
 */
#ifndef OBJETA_ORACLE_H
#define OBJETA_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* QuantFormat ordinals (crates/objeta-cuda/src/quant.rs:25-31). */
enum { ORC_Q4_0 = 0, ORC_Q5_0 = 1, ORC_IQ3_0 = 2, ORC_FP4 = 3 };

/* block_bytes (quant.rs:44-51); block_size is 32 for all formats. */
int orc_block_bytes(int fmt);

/* Bit-level f16 conversions (quant.rs:1021-1079). */
uint16_t orc_f32_to_f16_bits(float v);
float orc_f16_to_f32_bits(uint16_t h);
void orc_f32_to_f16_bits_n(const float* v, uint16_t* out, size_t n);
void orc_f16_to_f32_bits_n(const uint16_t* h, float* out, size_t n);

/* E8M0 decodes: quant.rs:886-892 (raw 0 -> 2^-127) and
 * crates/objeta-parser/src/deepseek.rs:838-856 (2^(raw-127), subnormals kept). */
float orc_decode_f8_e8m0(uint8_t raw);
float orc_f8e8m0_to_f32(uint8_t raw);

/* Block quantizers (quant.rs:814-926). src: 32 floats. */
void orc_q4_quantize_block(const float* src, uint8_t* dst18);
void orc_q5_quantize_block(const float* src, uint8_t* dst22);
void orc_iq3_quantize_block(const float* src, uint8_t* dst14);
void orc_fp4_quantize_block(const float* src, uint8_t* dst17);
uint8_t orc_fp4_scale_raw(float amax);
void orc_fp4_scale_raw_n(const float* amax, uint8_t* out, size_t n);

/* quantize_matrix_cpu (quant.rs:506-581) with validation (quant.rs:725-749).
 * Returns 0 on success, else a CudaErrorKind ordinal + 1 with a message in err. */
int orc_quantize_matrix(int fmt, const float* m, size_t m_len, size_t rows, size_t cols,
                        uint8_t* out, size_t out_len, char* err, size_t err_len);

/* Per-row dot products (quant.rs:928-1019). */
float orc_dot_row(int fmt, const uint8_t* row_q, const float* x, size_t cols);

/* gemv_cpu (quant.rs:627-646) with validate_quant_inputs (quant.rs:751-793). */
int orc_gemv(int fmt, const uint8_t* q, size_t q_len, const float* x, size_t x_len,
             size_t rows, size_t cols, float* y, char* err, size_t err_len);

/* dense_gemv_cpu (quant.rs:599-625). */
int orc_dense_gemv(const float* m, size_t m_len, const float* x, size_t x_len,
                   size_t rows, size_t cols, float* y, char* err, size_t err_len);

/* decode_deepseek_fp4_to_f32 (crates/objeta-parser/src/deepseek.rs:866-918) for the
 * split layout: w [rows][cols/2], s [rows][cols/32]. */
void orc_decode_fp4_split(const uint8_t* w, const uint8_t* s, size_t rows, size_t cols, float* out);

/* fp4_e2m1_gemv_split CPU counterpart: decode then dense_gemv_cpu, as
 * selected_moe_cpu_native_fp4 does per matrix (moe.rs:1665-1735). */
void orc_fp4_split_gemv(const uint8_t* w, const uint8_t* s, const float* x,
                        size_t rows, size_t cols, float* y);

/* One selected-expert MoE pass.
 *   fmt ORC_Q4_0  : selected_moe_cpu          (moe.rs:1283-1324); gate/up/down are Q4_0 bytes.
 *   fmt ORC_FP4   : selected_moe_cpu_native_fp4 (moe.rs:1665-1735); split layout,
 *                   gate_s/up_s/down_s are the E8M0 scale arrays.
 *   fmt -1        : selected_moe_cpu_fp32     (moe.rs:1326-1367); gate/up/down are f32.
 * Experts are passed as arrays of pointers indexed by expert id. `out` is
 * zero-initialised by the function (the reference's vec![0.0; out_dim]). */
int orc_selected_moe(int fmt, size_t n_experts,
                     const void* const* gate, const void* const* up, const void* const* down,
                     const uint8_t* const* gate_s, const uint8_t* const* up_s,
                     const uint8_t* const* down_s,
                     const uint32_t* sel_ids, const float* sel_w, size_t k,
                     const float* x, size_t hidden, size_t inter, size_t out_dim,
                     float* out, char* err, size_t err_len);

/* Router: logits -> softmax -> stable top-k (cpu_router,
 * crates/objeta-cuda/src/bin/deepseek_single_layer_moe.rs:687-743), then an optional
 * renormalisation of the k selected probabilities (the softmax -> top-k ->
 * renormalize routing of crates/objeta-qwen36-executor/src/moe_dispatch.rs:403-435).
 * bias may be NULL (then logits are exactly cpu_router's). logits_out/probs_out may
 * be NULL. */
int orc_router(const float* w_r, const float* bias, const float* x, size_t n_experts,
               size_t hidden, size_t k, int renormalize, uint32_t* ids, float* weights,
               float* logits_out, float* probs_out, char* err, size_t err_len);

/* compare_outputs (quant.rs:676-723): out[0]=cosine, out[1]=rel_l2, out[2]=max_abs. */
int orc_compare(const float* ref, const float* act, size_t n, float* out3);

/* FP8 official arithmetic (crates/objeta-parser/src/deepseek.rs): F8_E4M3 decode and
 * encode, act_quant (128-element E8M0 blocks), the FP8 x FP4 (f32 sums) and FP8 x FP8
 * (f64 sums) GEMVs, and one expert of the official routed (fp8_weights = 0, FP4 split
 * weights) or shared (fp8_weights = 1) composition. */
float orc_f8e4m3_to_f32(uint8_t raw);
uint8_t orc_f32_to_f8e4m3_exact(float v);
void orc_act_quant(const float* x, size_t n, size_t block, uint8_t* y, uint8_t* s);
void orc_f8e4m3_to_f32_n(const uint8_t* raw, float* out, size_t n);
void orc_f32_to_f8e4m3_exact_n(const float* v, uint8_t* out, size_t n);
void orc_fp8_act_fp4_weight_gemv_f32(const uint8_t* act_v, const uint8_t* act_s, const uint8_t* w,
                                     const uint8_t* ws, size_t rows, size_t cols, float* out);
void orc_fp8_act_fp8_weight_gemv(const uint8_t* act_v, const uint8_t* act_s, const uint8_t* w,
                                 const uint8_t* ws, size_t rows, size_t cols, float* out);
int orc_expert_official(int fp8_weights, const uint8_t* gw, const uint8_t* gs, const uint8_t* uw,
                        const uint8_t* us, const uint8_t* dw, const uint8_t* ds, const float* x,
                        size_t dim, size_t inter, float swiglu_limit, float* out, float* act_pre,
                        uint8_t* act_q, uint8_t* act_qs, char* err, size_t err_len);

/* Threads of the row loops (default 1, the reference's single thread); results are
 * identical for every count because each row's sum stays sequential. */
void orc_set_threads(int n);
int orc_get_threads(void);

/* glibc's expf (Rust's f32::exp on Linux), element-wise: the value the reference's
 * softmax uses (deepseek_single_layer_moe.rs:687-743). */
void orc_expf_glibc(const float* in, float* out, size_t n);
/* The restatement of glibc's expf method that the device router evaluates (see
 * oracle.c). */
float orc_expf_restated(float x);
/* Over every float whose bits lie in [lo_bits, hi_bits]: the number of arguments
 * where the restatement, and where exp in double rounded once to float, differ
 * from glibc's expf. */
void orc_expf_range_check(uint32_t lo_bits, uint32_t hi_bits, uint64_t* restated_mismatch,
                          uint64_t* double_mismatch);
/* The arguments (up to cap, in no particular order) where exp in double rounded once
 * to float differs from glibc's expf; returns how many there are. */
size_t orc_expf_double_disagreements(uint32_t lo_bits, uint32_t hi_bits, float* out, size_t cap);

/* seeded_f32s LCG (crates/objeta-cuda/src/bin/bench_qgemv.rs:39-49, quant.rs:1610-1620). */
void orc_seeded_f32s(uint64_t seed, float* out, size_t n);

/* Counter-based generator shared with the device generator kernels:
 * value(i) = sigma * z(seed, i), z an Irwin-Hall(12) approximation of N(0,1) built
 * from splitmix64 words with integer-exact arithmetic, so CPU and GPU produce the
 * same bits. Not a reference function: it is the synthetic-input recipe. */
float orc_gauss(uint64_t seed, uint64_t i, float sigma);
void orc_gauss_fill(uint64_t seed, uint64_t first, float sigma, float* out, size_t n);
uint64_t orc_splitmix64(uint64_t z);

#ifdef __cplusplus
}
#endif
#endif
