// kernels.hpp — host-side launchers shared between translation units. Each
// launcher validates its shape arguments, enqueues on `s` and allocates nothing.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/objeta_hip.h"

struct objeta_hip_context;

namespace objeta {

int32_t launch_qgemv(objeta_hip_context* ctx, int32_t format, hipStream_t s, const void* d_q,
                     const float* d_x, float* d_y, uint64_t rows, uint64_t cols, uint64_t batch);

int32_t launch_fp4_split(objeta_hip_context* ctx, hipStream_t s, const void* d_w, const void* d_s,
                         const float* d_x, float* d_y, uint64_t rows, uint64_t cols, uint64_t batch);

int32_t launch_zero(hipStream_t s, void* d, uint64_t bytes);

// The device address of pinned host bytes [h, h + n) when a kernel can copy them
// (host memory from hipHostMalloc, h and n 16-byte multiples), else nullptr.
const void* pinned_device_ptr(const void* h, size_t n);
// dst[0, n) = the pinned host bytes at device address src_dev, by a kernel on `s`
// (n, dst and src_dev 16-byte multiples).
int32_t launch_h2d_copy(hipStream_t s, void* dst, const void* src_dev, size_t n);
// One copy of a batch: n bytes from a pinned source's device address to dst.
struct H2dCopy {
    void* dst;
    const void* src_dev;
    size_t n;
};
constexpr int kH2dBatch = 32;  // copies per launch (kernel arguments of 768 bytes)
// The n copies of c[] in ceil(n / kH2dBatch) launches on s (pointers and sizes 16-byte
// multiples, as for launch_h2d_copy).
int32_t launch_h2d_copy_batch(hipStream_t s, const H2dCopy* c, size_t n);

// GEMV over an FP8 E4M3 matrix with 128 x 128 E8M0 scale tiles (cols % 128 == 0).
int32_t launch_fp8_rows(objeta_hip_context* ctx, hipStream_t s, const void* d_w, const void* d_s,
                        const float* d_x, float* d_y, uint64_t rows, uint64_t cols, uint64_t batch);

// act_quant (deepseek.rs:1484-1525) of `rows` vectors of `cols` floats (cols % 128
// == 0): F8_E4M3 bytes to d_values, one E8M0 scale per 128 to d_scales, and when
// d_deq is set the dequantized values act_v * act_s (the factors of the reference's
// FP8 GEMVs) as floats. d_deq may alias d_x.
int32_t launch_act_quant(hipStream_t s, const float* d_x, uint64_t rows, uint64_t cols, uint8_t* d_values,
                         uint8_t* d_scales, float* d_deq);
// act_v * act_s as floats for FP8 activations and their 128-element scales.
int32_t launch_fp8_dequant(hipStream_t s, const uint8_t* d_values, const uint8_t* d_scales, uint64_t rows,
                           uint64_t cols, float* d_out);

// The router launch behind objeta_hip_router_topk_device (its epoch words and
// counters are the scratch of stream `s`). With table and sel_tab given and *sel_tab non-null, the router also
// writes the selected experts' table entries to (*sel_tab)[t * k + r] when it can
// (up to kSelTabMaxExperts experts, hidden a multiple of 1024); *sel_tab is set to
// nullptr when it does not.
constexpr uint64_t kSelTabMaxExperts = 256;
constexpr uint64_t kMaxRouterExperts = 1024;  // router workspace: 2 words per expert and token
int32_t launch_router(objeta_hip_context* ctx, hipStream_t s, const float* w_r, const float* bias,
                      const float* x, uint64_t n_tokens, uint64_t n_experts, uint64_t hidden, uint64_t k,
                      int32_t renormalize, uint32_t* ids, float* weights,
                      const objeta_hip_expert_ptrs* table, objeta_hip_expert_ptrs** sel_tab);

int32_t launch_moe_gate_up(objeta_hip_context* ctx, int32_t format, hipStream_t s, const objeta_hip_expert_ptrs* table,
                           uint64_t n_table, const uint32_t* ids, uint64_t n_tokens, uint64_t k, const float* x,
                           float* act, uint64_t hidden, uint64_t inter, float limit,
                           const objeta_hip_expert_ptrs* sel = nullptr, const objeta_hip_expert_ptrs* shared = nullptr,
                           bool official = false);

// sel (optional): the assignments' table entries as the router resolved them; the
// kernels then skip the id and table lookups. shared (optional, a device pointer to
// one table entry): the shared expert, an extra slot per token with weight 1 added
// after the routed sum; act then holds k + 1 slots per token.
// Events recorded after the phases of launch_moe_official_fp4 (each nullable).
struct OfficialMarks {
    hipEvent_t gate_up_end, shared_gate_up_end, act_quant_end, down_end;
};
// The official-arithmetic FP4 MoE layer (FP8 activations, FP4 split routed experts,
// optional FP8 shared expert with 128 x 128 scale tiles).
int32_t launch_moe_official_fp4(objeta_hip_context* ctx, hipStream_t s, const objeta_hip_expert_ptrs* table,
                                uint64_t n_table, const objeta_hip_expert_ptrs* shared, const uint32_t* ids,
                                const float* wts, uint64_t n_tokens, uint64_t k, const float* x, float* out,
                                uint64_t hidden, uint64_t inter, uint64_t out_dim, float limit,
                                uint8_t* inter_values, uint8_t* inter_scales, const OfficialMarks* marks);

// The same layer on the grouped-token products (grouped.hip), for batches of at
// least kOfficialGroupedMinTokens tokens in the grouped path's limits (at the
// DeepSeek shape the per-token kernels are faster up to 4 tokens, the grouped ones
// from 6: the per-token path reads the FP8 shared expert once per token).
constexpr uint64_t kOfficialGroupedMinTokens = 6;
bool official_grouped_supported(uint64_t n_table, uint64_t n_tokens, uint64_t k, uint64_t hidden, uint64_t inter,
                                uint64_t out_dim);
int32_t launch_moe_official_grouped(objeta_hip_context* ctx, hipStream_t s, const objeta_hip_expert_ptrs* table,
                                    uint64_t n_table, const objeta_hip_expert_ptrs* shared, const uint32_t* ids,
                                    const float* wts, uint64_t n_tokens, uint64_t k, const float* x, float* out,
                                    uint64_t hidden, uint64_t inter, uint64_t out_dim, float limit,
                                    uint8_t* inter_values, uint8_t* inter_scales, const OfficialMarks* marks);

int32_t launch_moe_down(objeta_hip_context* ctx, int32_t format, hipStream_t s, const objeta_hip_expert_ptrs* table,
                        uint64_t n_table, const uint32_t* ids, const float* wts, uint64_t n_tokens, uint64_t k,
                        const float* act, const float* resid, float* out, uint64_t inter, uint64_t out_dim,
                        const objeta_hip_expert_ptrs* sel = nullptr, const objeta_hip_expert_ptrs* shared = nullptr);

// Looks up (once per device, with the context's device current) the device address
// of the static activation scratch of objeta_hip_moe_selected_device_noalloc and
// keeps it in ctx->static_act.
constexpr uint64_t kStaticActFloats = uint64_t(1) << 20;
int32_t bind_static_scratch(objeta_hip_context* ctx);

int32_t moe_act_scratch(objeta_hip_context* ctx, hipStream_t s, uint64_t n_tokens, uint64_t k, uint64_t inter,
                        float** out);

// Batched GEMV on the matrix cores (every weight decoded once for up to 8 vectors):
// Q4_0 / Q5_0 / IQ3_0 (cols % 64 == 0) or the split FP4 layout (cols % 128 == 0),
// weights 4-byte and x 16-byte aligned, from kGemvMfmaMinBatch vectors. Results
// within the fp32 tolerance of the per-vector kernels (activations split into two
// fp16 parts, 22 significant bits).
constexpr uint64_t kGemvMfmaMinBatch = 5;
bool gemv_mfma_supported(int32_t format, uint64_t rows, uint64_t cols, uint64_t batch, const void* w,
                         const float* x);
int32_t launch_gemv_mfma(objeta_hip_context* ctx, hipStream_t s, int32_t format, const void* w, const void* ws,
                         const float* x, float* y, uint64_t rows, uint64_t cols, uint64_t batch);
// Batches from this many tokens run the grouped-token products in the layer entry
// points (measured on MI355X over 48 Qwen3-A3B-shaped layers, hidden 2048, 128
// experts, top-8, us per layer per-assignment / grouped: 10 tokens 63.7 / 66.7, 12
// tokens 73.3 / 72.0, 16 tokens 85.1 / 76.4, 32 tokens 146.8 / 104.4).
constexpr uint64_t kGroupedMinTokens = 12;
// From 2 tokens when one expert's three matrices take at least this many bytes: at
// hidden 7168 / intermediate 2048 (23 MB FP4 experts, a shared expert) the grouped
// path takes 160 / 258 / 314 us at 2 / 3 / 4 tokens against 218 / 360 / 459 on the
// per-assignment kernels; the Qwen3-A3B shape's 2.6 MB experts keep the 12-token
// switch.
constexpr uint64_t kGroupedLargeExpertBytes = uint64_t(8) << 20;
// Whether the layer entry points run a batch of n_tokens on the grouped path.
bool grouped_preferred(int32_t format, uint64_t n_tokens, uint64_t hidden, uint64_t inter, uint64_t out_dim);
// Whether launch_moe_grouped takes this shape.
bool grouped_supported(int32_t format, uint64_t n_table, uint64_t n_tokens, uint64_t k, uint64_t hidden,
                       uint64_t inter, uint64_t out_dim);
int32_t launch_moe_grouped(objeta_hip_context* ctx, int32_t format, hipStream_t s, const objeta_hip_expert_ptrs* table,
                           uint64_t n_table, const objeta_hip_expert_ptrs* shared, const uint32_t* ids, const float* wts, uint64_t n_tokens, uint64_t k,
                           const float* x, const float* resid, float* out, uint64_t hidden, uint64_t inter,
                           uint64_t out_dim, float limit);

}  // namespace objeta
