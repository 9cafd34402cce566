/*
 * objeta_hip.h — C ABI of the MI355X (gfx950) selected-expert MoE decode path.
 *
 * This is the drop-in boundary for the reference's objeta-cuda crate
 * (crates/objeta-cuda/src). Every entry point takes plain pointers and sizes and
 * returns an int32 status: 0 on success, otherwise the reference's CudaErrorKind
 * ordinal + 1 (crates/objeta-cuda/src/lib.rs:39-48). The failing call's details
 * (the fields of the reference's CudaError, lib.rs:50-79) are kept per thread and
 * read back with objeta_hip_last_error().
 *
 * Ownership: the caller owns every host buffer and output array; the library
 * owns device memory it allocates (cache residents, workspaces). Device pointers
 * passed in ("d_" arguments) stay owned by the caller.
 *
 * Threading: a context may be used from one thread at a time (the reference's
 * QuantBackend / MoeExecutor are &self but serialise on their stream). A cache
 * handle is not internally locked, matching the reference's `&mut CudaExpertCache`.
 *
 * Streams: `objeta_hip_stream` is a hipStream_t. NULL means the context's stream 0.
 * All *_device entry points are asynchronous on the given stream, allocate
 * nothing on the hot path and may be captured into a hipGraph.
 */
#ifndef OBJETA_HIP_H
#define OBJETA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define OBJETA_HIP_ABI_VERSION 1

/* ------------------------------------------------------------------ errors */
/* CudaErrorKind + 1 (lib.rs:39-48). */
enum {
    OBJETA_HIP_OK = 0,
    OBJETA_HIP_ERR_DRIVER = 1,
    OBJETA_HIP_ERR_RUNTIME = 2,
    OBJETA_HIP_ERR_NVRTC = 3, /* kept for ordinal parity; this library compiles ahead of time */
    OBJETA_HIP_ERR_IO = 4,
    OBJETA_HIP_ERR_INVALID_INPUT = 5,
    OBJETA_HIP_ERR_UNSUPPORTED = 6,
    OBJETA_HIP_ERR_INTERNAL = 7
};

/* CudaError{kind, action, file, line, module, source_message} (lib.rs:50-79). */
typedef struct {
    int32_t kind; /* CudaErrorKind ordinal (status - 1); -1 when no error recorded */
    uint32_t line;
    char action[160];
    char file[96];
    char module[64];
    char source_message[320];
} objeta_hip_error;

/* Copies this thread's last error; returns its status (0 if none). */
int32_t objeta_hip_last_error(objeta_hip_error* out);
void objeta_hip_clear_error(void);
int32_t objeta_hip_abi_version(void);

/* ----------------------------------------------------------------- formats */
/* QuantFormat (crates/objeta-cuda/src/quant.rs:25-31). */
enum {
    OBJETA_HIP_Q4_0 = 0,     /* 18-byte blocks: f16 scale + 16 nibble bytes */
    OBJETA_HIP_Q5_0 = 1,     /* 22-byte blocks: f16 scale + 4-byte high mask + 16 nibble bytes */
    OBJETA_HIP_IQ3_0 = 2,    /* 14-byte blocks: f16 scale + 8 bytes 2-bit lows + 4 bytes highs */
    OBJETA_HIP_FP4_E2M1 = 3  /* 17-byte interleaved blocks: E8M0 scale + 16 nibble bytes */
};

/* QuantFormat::block_size / block_bytes (quant.rs:34-51); -1 for an unknown format. */
int32_t objeta_hip_block_size(int32_t format);
int32_t objeta_hip_block_bytes(int32_t format);
/* QGemvShape::quantized_matrix_bytes (quant.rs:140-142); -1 if cols % 32 != 0. */
int64_t objeta_hip_quantized_matrix_bytes(int32_t format, uint64_t rows, uint64_t cols);

/* ----------------------------------------------------------------- devices */
typedef struct objeta_hip_context objeta_hip_context;
typedef void* objeta_hip_stream; /* hipStream_t */
typedef void* objeta_hip_event;  /* hipEvent_t */
typedef void* objeta_hip_graph;  /* hipGraphExec_t */

/* BackendInitOptions (crates/objeta-cuda/src/ffi.rs:1-7) / CudaBackendBuilder
 * (context.rs:37-70). stream_count is clamped to >= 1. */
typedef struct {
    uint64_t device_ordinal;
    uint64_t stream_count;
} objeta_hip_init_options;

/* CudaDeviceInfo (context.rs:16-24) plus the CDNA facts the kernels size for.
 * compute_capability_major/minor carry the gfx major/minor (9, 5 for gfx950). */
typedef struct {
    uint64_t ordinal;
    char name[256];
    char arch[64];
    uint64_t total_global_mem_bytes;
    int32_t compute_capability_major;
    int32_t compute_capability_minor;
    int32_t driver_version;
    int32_t runtime_version;
    int32_t compute_units;
    int32_t wavefront_size;
    int32_t l2_cache_bytes;
    int32_t max_shared_memory_per_block;
    int32_t clock_khz;
    int32_t memory_clock_khz;
    int32_t memory_bus_width_bits;
    int32_t reserved;
} objeta_hip_device_info;

/* CudaBackend::discover_devices (context.rs:73-104). */
int32_t objeta_hip_device_count(int32_t* out);
int32_t objeta_hip_discover_device(uint64_t ordinal, objeta_hip_device_info* out);
/* CudaBackend::new (context.rs:106-141). */
int32_t objeta_hip_init(const objeta_hip_init_options* opts, objeta_hip_context** out);
int32_t objeta_hip_destroy(objeta_hip_context* ctx);
int32_t objeta_hip_device_info_get(const objeta_hip_context* ctx, objeta_hip_device_info* out);
/* CudaStreamPool::stream (stream.rs:38-51). */
int32_t objeta_hip_stream_get(objeta_hip_context* ctx, uint64_t index, objeta_hip_stream* out);
/* CudaStreamHandle::synchronize (stream.rs:67-74). */
int32_t objeta_hip_stream_synchronize(objeta_hip_context* ctx, objeta_hip_stream stream);

/* ------------------------------------------------------------------ memory */
/* DeviceBuffer / alloc_zeros / alloc_uninit (memory.rs:8-28, stream.rs:76-102). */
int32_t objeta_hip_malloc(objeta_hip_context* ctx, uint64_t bytes, void** d_out);
int32_t objeta_hip_free(objeta_hip_context* ctx, void* d_ptr);
/* PinnedHostBuffer (memory.rs:31-80, context.rs:143-165). */
int32_t objeta_hip_alloc_pinned_host(objeta_hip_context* ctx, uint64_t bytes, void** h_out);
int32_t objeta_hip_free_pinned_host(objeta_hip_context* ctx, void* h_ptr);
/* copy_from_slice / copy_to_vec / copy_dtod (stream.rs:104-201), asynchronous on
 * `stream` (pageable host memory makes the HIP runtime stage the copy). A host to
 * device copy from pinned memory (objeta_hip_alloc_pinned_host) whose source,
 * destination and size are 16-byte multiples runs as a kernel reading the host
 * memory through its device mapping, which on MI355X outruns the DMA engine. */
int32_t objeta_hip_copy_h2d(objeta_hip_context* ctx, objeta_hip_stream stream, void* d_dst,
                            const void* h_src, uint64_t bytes);
int32_t objeta_hip_copy_d2h(objeta_hip_context* ctx, objeta_hip_stream stream, void* h_dst,
                            const void* d_src, uint64_t bytes);
int32_t objeta_hip_copy_d2d(objeta_hip_context* ctx, objeta_hip_stream stream, void* d_dst,
                            const void* d_src, uint64_t bytes);
/* Zero-fill with a kernel (safe to capture into a graph). */
int32_t objeta_hip_zero_device(objeta_hip_context* ctx, objeta_hip_stream stream, void* d_dst,
                               uint64_t bytes);

/* ------------------------------------------------------- events and graphs */
/* CudaEventTimer (telemetry.rs:14-44) split into its parts. */
int32_t objeta_hip_event_create(objeta_hip_context* ctx, objeta_hip_event* out);
int32_t objeta_hip_event_record(objeta_hip_context* ctx, objeta_hip_event ev, objeta_hip_stream stream);
/* Waits for `end` and returns the elapsed milliseconds between the two events. */
int32_t objeta_hip_event_elapsed_ms(objeta_hip_context* ctx, objeta_hip_event start,
                                    objeta_hip_event end, float* ms_out);
int32_t objeta_hip_event_destroy(objeta_hip_context* ctx, objeta_hip_event ev);
/* hipGraph capture of everything enqueued on `stream` between begin and end. No
 * reference counterpart: the reference syncs after every launch. */
int32_t objeta_hip_graph_begin_capture(objeta_hip_context* ctx, objeta_hip_stream stream);
int32_t objeta_hip_graph_end_capture(objeta_hip_context* ctx, objeta_hip_stream stream,
                                     objeta_hip_graph* out);
int32_t objeta_hip_graph_launch(objeta_hip_context* ctx, objeta_hip_graph graph,
                                objeta_hip_stream stream);
int32_t objeta_hip_graph_destroy(objeta_hip_context* ctx, objeta_hip_graph graph);

/* -------------------------------------------------------------------- GEMV */
/* QGemvTelemetry (quant.rs:145-154). bytes_read = W + 4*cols, as quant.rs:282. */
typedef struct {
    float h2d_ms;
    float kernel_ms;
    float d2h_ms;
    float unaccounted_ms;
    float total_ms;
    float effective_gbps;
    uint64_t bytes_read;
} objeta_hip_qgemv_telemetry;

/* QuantBackend::gemv (quant.rs:256-302): host qweights and x in, host y out.
 * Validation and messages follow validate_quant_inputs (quant.rs:751-793).
 * format: any block format (Q4_0, Q5_0, IQ3_0, FP4_E2M1 interleaved). tel may be NULL. */
int32_t objeta_hip_qgemv(objeta_hip_context* ctx, int32_t format, objeta_hip_stream stream,
                         const uint8_t* qweights, uint64_t qweights_len, const float* x,
                         uint64_t x_len, uint64_t rows, uint64_t cols, float* y,
                         objeta_hip_qgemv_telemetry* tel);

/* QuantBackend::launch_kernel (quant.rs:324-366) generalised to `batch` activation
 * vectors: d_x is [batch][cols] f32, d_y is [batch][rows] f32 (overwritten). */
int32_t objeta_hip_qgemv_device(objeta_hip_context* ctx, int32_t format, objeta_hip_stream stream,
                                const void* d_qweights, const float* d_x, float* d_y,
                                uint64_t rows, uint64_t cols, uint64_t batch);

/* QuantBackend::launch_kernel_split_fp4 (quant.rs:368-408): DeepSeek split FP4
 * layout, d_w [rows][cols/2] nibbles, d_scales [rows][cols/32] E8M0 bytes. */
int32_t objeta_hip_fp4_gemv_split_device(objeta_hip_context* ctx, objeta_hip_stream stream,
                                         const void* d_w, const void* d_scales, const float* d_x,
                                         float* d_y, uint64_t rows, uint64_t cols, uint64_t batch);

/* --------------------------------------------------- quantizer / generators */
/* quantize_matrix_cpu (quant.rs:506-581) on the device; bytes identical to the
 * CPU quantizer. d_m: [rows][cols] f32; d_out: quantized_matrix_bytes. */
int32_t objeta_hip_quantize_matrix_device(objeta_hip_context* ctx, int32_t format,
                                          objeta_hip_stream stream, const float* d_m,
                                          uint64_t rows, uint64_t cols, void* d_out);
/* Synthetic inputs (no reference counterpart; the reference generates on the CPU
 * with seeded_f32s, bench_qgemv.rs:39-49). Element i is sigma * z(seed, first + i)
 * with z a counter-based Irwin-Hall(12) draw; the CPU recipe gives the same bits. */
int32_t objeta_hip_fill_gauss_device(objeta_hip_context* ctx, objeta_hip_stream stream,
                                     float* d_out, uint64_t n, uint64_t seed, uint64_t first,
                                     float sigma);
/* Generate a [rows][cols] matrix as above (element r*cols+c) and quantize it in
 * one pass; bytes equal quantize_matrix_cpu of the generated matrix. */
int32_t objeta_hip_fill_gauss_quantized_device(objeta_hip_context* ctx, int32_t format,
                                               objeta_hip_stream stream, void* d_out,
                                               uint64_t rows, uint64_t cols, uint64_t seed,
                                               float sigma);
/* One split FP4 matrix of synthetic bytes (no reference counterpart; the reference's
 * FP4 inputs come from checkpoints): d_w [rows][cols/2] nibbles uniform over the 16
 * E2M1 codes, d_s [rows][cols/32] E8M0 scales uniform over raw 119..127 (2^-8 ..
 * 2^0), from a counter-based splitmix64 recipe that the host reproduces. */
int32_t objeta_hip_fill_fp4_split_device(objeta_hip_context* ctx, objeta_hip_stream stream, void* d_w, void* d_s,
                                         uint64_t rows, uint64_t cols, uint64_t seed);
/* The E8M0 exponent rule of the device FP4 quantizer (fp4_quantize_block,
 * quant.rs:913-918) evaluated on the host, element-wise over n block maxima. */
int32_t objeta_hip_fp4_scale_raw_host(const float* amax, uint8_t* out, uint64_t n);

/* ------------------------------------------------------------------ router */
/* Router for n_tokens activation rows: logits = W_r x (+ bias), softmax over all
 * experts, stable top-k by probability (ties keep the lower expert id), then the
 * k probabilities renormalised to sum 1 when `renormalize` != 0. Follows cpu_router
 * (crates/objeta-cuda/src/bin/deepseek_single_layer_moe.rs:687-743) and the
 * renormalised top-k of router_topk_cpu
 * (crates/objeta-qwen36-executor/src/moe_dispatch.rs:403-435).
 * d_w_r [n_experts][hidden] f32; d_bias [n_experts] or NULL; d_x [n_tokens][hidden];
 * d_ids [n_tokens][k] u32; d_weights [n_tokens][k] f32. n_experts <= 1024, k <= 32. */
int32_t objeta_hip_router_topk_device(objeta_hip_context* ctx, objeta_hip_stream stream,
                                      const float* d_w_r, const float* d_bias, const float* d_x,
                                      uint64_t n_tokens, uint64_t n_experts, uint64_t hidden,
                                      uint64_t k, int32_t renormalize, uint32_t* d_ids,
                                      float* d_weights);

/* y[i] = exp(x[i]) as the router's softmax evaluates it on the device: glibc's
 * expf (the f32::exp of the reference's cpu_router, deepseek_single_layer_moe.rs:
 * 687-743), bit for bit. Exposed so that tests can compare it with the host's
 * expf; no reference counterpart. n <= 2^32. */
int32_t objeta_hip_router_softmax_exp_device(objeta_hip_context* ctx, objeta_hip_stream stream,
                                             const float* d_x, float* d_y, uint64_t n);

/* --------------------------------------------------------------- MoE path */
/* Device addresses of one expert's projections: ExpertWeights (moe.rs:13-18) for
 * the block formats, DeepSeekFp4ExpertWeights (moe.rs:27-35) for FP4. gate and up
 * are [intermediate][hidden] matrices, down is [out_dim][intermediate]. With
 * format OBJETA_HIP_FP4_E2M1 the MoE entry points read the split FP4 layout of
 * execute_selected_moe_native_fp4_cuda (moe.rs:816-1280): gate/up/down hold the
 * nibbles [rows][cols/2] and *_scale the E8M0 bytes [rows][cols/32]. For block
 * formats the *_scale fields are ignored. */
typedef struct {
    const void* gate;
    const void* up;
    const void* down;
    const void* gate_scale;
    const void* up_scale;
    const void* down_scale;
} objeta_hip_expert_ptrs;

/* The per-expert kernels of execute_selected_moe_cuda (moe.rs:587-652) fused and
 * batched over tokens, all on the device. For token t and selection slot j the
 * expert is e = d_ids[t*k + j], an index into d_table (n_table entries; NULL
 * d_ids means e = t*k + j), and
 *   act_j  = silu(gate_e x_t) * (up_e x_t)          silu_mul (moe.cu:2-22)
 *   out_t  = residual_t + sum_j d_weights[t*k + j] * (down_e act_j)
 * with the sum taken in slot order (weighted_accum, moe.cu:24-34). swiglu_limit
 * > 0 applies the reference's clamp (up to [-L, L], gate to <= L). d_residual NULL
 * means zero (the reference's zero-initialised out); d_out may alias d_residual
 * and d_x. An expert id >= n_table makes that slot contribute NaN and sets the
 * context's device error word (objeta_hip_device_error). Allocates nothing after
 * the first call with a given size; graph-capturable. d_x [n_tokens][hidden],
 * d_out/d_residual [n_tokens][out_dim] f32. */
int32_t objeta_hip_moe_selected_device(objeta_hip_context* ctx, int32_t format, objeta_hip_stream stream,
                                       const objeta_hip_expert_ptrs* d_table, uint64_t n_table,
                                       const uint32_t* d_ids, const float* d_weights, uint64_t n_tokens,
                                       uint64_t k, const float* d_x, const float* d_residual, float* d_out,
                                       uint64_t hidden, uint64_t intermediate, uint64_t out_dim,
                                       float swiglu_limit);

/* objeta_hip_moe_selected_device plus a shared expert: d_shared (a device pointer to
 * one objeta_hip_expert_ptrs, or NULL for none) is applied to every token with
 * weight 1.0 after the routed sum,
 *   out_t = residual_t + sum_j d_weights[t*k + j] * down_j(act_j) + down_s(act_s),
 * as execute_selected_moe_official_routed_fp4_cuda adds its shared expert
 * (moe.rs:1552-1600: weighted_accum with weight 1.0 after the routed experts). Same
 * format, shapes and limits as the routed experts. */
int32_t objeta_hip_moe_selected_shared_device(objeta_hip_context* ctx, int32_t format, objeta_hip_stream stream,
                                              const objeta_hip_expert_ptrs* d_table, uint64_t n_table,
                                              const objeta_hip_expert_ptrs* d_shared, const uint32_t* d_ids,
                                              const float* d_weights, uint64_t n_tokens, uint64_t k, const float* d_x,
                                              const float* d_residual, float* d_out, uint64_t hidden,
                                              uint64_t intermediate, uint64_t out_dim, float swiglu_limit);

/* objeta_hip_moe_selected_device without any allocation, for callers that cannot
 * allocate device memory (code under graph capture before a first eager call,
 * tight serving loops, harnesses that forbid hipMalloc). No counterpart in the
 * reference. Same arguments and results as objeta_hip_moe_selected_device (the
 * same kernels); the activations [n_tokens * k][intermediate] live in a static
 * device array of 2^20 floats (4 MiB) per device, held until the process ends.
 * n_tokens * k * intermediate > 2^20 fails with InvalidInput. Every call on a
 * device shares that array: calls that overlap on one device race. */
int32_t objeta_hip_moe_selected_device_noalloc(objeta_hip_context* ctx, int32_t format, objeta_hip_stream stream,
                                               const objeta_hip_expert_ptrs* d_table, uint64_t n_table,
                                               const uint32_t* d_ids, const float* d_weights, uint64_t n_tokens,
                                               uint64_t k, const float* d_x, const float* d_residual, float* d_out,
                                               uint64_t hidden, uint64_t intermediate, uint64_t out_dim,
                                               float swiglu_limit);

/* objeta_hip_moe_selected_device for a batch whose tokens share experts: the
 * (token, slot) assignments are grouped by expert on the device and every selected
 * expert's gate, up and down matrices are read once for all of its tokens, with
 * the products on the matrix cores (fp16 weights, exact for every format, times
 * activations split into two fp16 parts; fp32 accumulation). Same arguments and
 * result (within the fp32 tolerance) as objeta_hip_moe_selected_device; no
 * reference counterpart as one call (execute_selected_moe_cuda, moe.rs:352-751,
 * runs each selected expert per token). Limits: n_experts <= 1024, n_tokens * k
 * <= 1024, hidden and intermediate multiples of 64; Unsupported outside them.
 * d_ids is required. An out-of-table id sets bit 1 of the device error word and
 * makes that token's output NaN. Non-finite block scales give a non-finite output
 * element, but not necessarily the same special value as the reference's
 * per-weight products. */
int32_t objeta_hip_moe_grouped_device(objeta_hip_context* ctx, int32_t format, objeta_hip_stream stream,
                                      const objeta_hip_expert_ptrs* d_table, uint64_t n_table,
                                      const uint32_t* d_ids, const float* d_weights, uint64_t n_tokens,
                                      uint64_t k, const float* d_x, const float* d_residual, float* d_out,
                                      uint64_t hidden, uint64_t intermediate, uint64_t out_dim,
                                      float swiglu_limit);

/* The two launches of objeta_hip_moe_selected_device, for callers that keep the
 * activations: d_act [n_tokens*k][intermediate] f32 (16-byte aligned) receives
 * silu(gate x) * (up x) per (token, slot); the down phase combines them. */
int32_t objeta_hip_moe_gate_up_device(objeta_hip_context* ctx, int32_t format, objeta_hip_stream stream,
                                      const objeta_hip_expert_ptrs* d_table, uint64_t n_table,
                                      const uint32_t* d_ids, uint64_t n_tokens, uint64_t k, const float* d_x,
                                      float* d_act, uint64_t hidden, uint64_t intermediate, float swiglu_limit);
int32_t objeta_hip_moe_down_device(objeta_hip_context* ctx, int32_t format, objeta_hip_stream stream,
                                   const objeta_hip_expert_ptrs* d_table, uint64_t n_table, const uint32_t* d_ids,
                                   const float* d_weights, uint64_t n_tokens, uint64_t k, const float* d_act,
                                   const float* d_residual, float* d_out, uint64_t intermediate, uint64_t out_dim);

/* One MoE layer on the device: the router of objeta_hip_router_topk_device over
 * d_router_w [n_experts][hidden] (+ d_router_bias) writes d_ids_out/d_weights_out
 * [n_tokens][k], then the selected experts of d_table (n_experts entries) run:
 * below 12 tokens on the per-assignment kernels of objeta_hip_moe_selected_device,
 * from 12 tokens on the grouped-token products of objeta_hip_moe_grouped_device
 * whenever that path takes the shape (on MI355X at hidden 2048, 128 experts,
 * top-8 the per-assignment kernels are faster up to 10 tokens, the two are even at
 * 12 and the grouped ones faster from 14 on). When one expert's three matrices
 * take 8 MiB or more (hidden 7168, intermediate 2048) the grouped products run
 * from 2 tokens. The two agree within the fp32
 * tolerance, not bit for bit. No host
 * synchronisation; graph-capturable. No reference counterpart as one call: the
 * reference routes on the host (deepseek_single_layer_moe.rs:687-743) and then
 * calls execute_selected_moe_cuda. */
int32_t objeta_hip_moe_layer_device(objeta_hip_context* ctx, int32_t format, objeta_hip_stream stream,
                                    const objeta_hip_expert_ptrs* d_table, uint64_t n_experts,
                                    const float* d_router_w, const float* d_router_bias, uint64_t k,
                                    int32_t renormalize, uint64_t n_tokens, const float* d_x,
                                    const float* d_residual, float* d_out, uint32_t* d_ids_out,
                                    float* d_weights_out, uint64_t hidden, uint64_t intermediate,
                                    uint64_t out_dim, float swiglu_limit);

/* objeta_hip_moe_layer_device with the shared expert of
 * objeta_hip_moe_selected_shared_device (d_shared NULL: none); on the grouped
 * path the shared expert is one more group holding every token. */
int32_t objeta_hip_moe_layer_shared_device(objeta_hip_context* ctx, int32_t format, objeta_hip_stream stream,
                                           const objeta_hip_expert_ptrs* d_table, uint64_t n_experts,
                                           const objeta_hip_expert_ptrs* d_shared, const float* d_router_w,
                                           const float* d_router_bias, uint64_t k, int32_t renormalize,
                                           uint64_t n_tokens, const float* d_x, const float* d_residual, float* d_out,
                                           uint32_t* d_ids_out, float* d_weights_out, uint64_t hidden,
                                           uint64_t intermediate, uint64_t out_dim, float swiglu_limit);

/* Reads and clears the context's device error word. Bit 0: a kernel met an expert
 * id outside its table. Bit 1 (a report, not a failure): a router call's selecting
 * workgroup found other workgroups' logits still missing after its spin limit (the
 * device kept them from running, about a second by default) and computed every
 * logit itself in the reference's order, so its result is exact. The spin limit is
 * read at objeta_hip_init from the environment variable OBJETA_HIP_ROUTER_SPIN_LIMIT
 * (polls; 0 = never wait). Synchronises the context's streams. */
int32_t objeta_hip_device_error(objeta_hip_context* ctx, uint32_t* out);

/* ------------------------------------------------------------ expert cache */
/* ExpertTensorKind (moe.rs:37-54). */
enum {
    OBJETA_HIP_TENSOR_GATE = 0,
    OBJETA_HIP_TENSOR_UP = 1,
    OBJETA_HIP_TENSOR_DOWN = 2,
    OBJETA_HIP_TENSOR_GATE_WEIGHT = 3,
    OBJETA_HIP_TENSOR_GATE_SCALE = 4,
    OBJETA_HIP_TENSOR_UP_WEIGHT = 5,
    OBJETA_HIP_TENSOR_UP_SCALE = 6,
    OBJETA_HIP_TENSOR_DOWN_WEIGHT = 7,
    OBJETA_HIP_TENSOR_DOWN_SCALE = 8,
    OBJETA_HIP_TENSOR_SHARED_GATE_WEIGHT = 9,
    OBJETA_HIP_TENSOR_SHARED_GATE_SCALE = 10,
    OBJETA_HIP_TENSOR_SHARED_UP_WEIGHT = 11,
    OBJETA_HIP_TENSOR_SHARED_UP_SCALE = 12,
    OBJETA_HIP_TENSOR_SHARED_DOWN_WEIGHT = 13,
    OBJETA_HIP_TENSOR_SHARED_DOWN_SCALE = 14
};

/* ExpertCacheKey (moe.rs:56-62). */
typedef struct {
    uint64_t layer_id;
    uint64_t expert_id;
    int32_t tensor_kind;  /* OBJETA_HIP_TENSOR_* */
    int32_t quant_format; /* OBJETA_HIP_Q4_0 .. OBJETA_HIP_FP4_E2M1 */
} objeta_hip_cache_key;

/* The public fields of CudaExpertCache (moe.rs:70-90). */
typedef struct {
    uint64_t capacity_bytes;
    uint64_t resident_bytes;
    uint64_t pinned_bytes;
    uint64_t hit_count;
    uint64_t miss_count;
    uint64_t eviction_count;
    uint64_t cache_insert_attempt_count;
    uint64_t cache_insert_accept_count;
    uint64_t cache_insert_bypass_count;
    uint64_t oversized_tensor_bypass_count;
    uint64_t oversized_expert_bypass_count;
    uint64_t self_eviction_risk_count;
    uint64_t entry_count;           /* tensors resident */
    uint64_t device_bytes_reserved; /* resident + recycled blocks held for reuse */
    int32_t bypass_oversized_experts;
    int32_t reserved;
} objeta_hip_cache_stats;

/* One expert's host tensors: gate/up/down bytes (and, for FP4, the E8M0 scale
 * arrays) with their lengths. Mirrors ExpertWeights (moe.rs:13-18) and
 * DeepSeekFp4ExpertWeights (moe.rs:27-35). Pinned host memory
 * (objeta_hip_alloc_pinned_host) lets cache misses overlap compute. */
typedef struct {
    const void* gate;
    uint64_t gate_len;
    const void* up;
    uint64_t up_len;
    const void* down;
    uint64_t down_len;
    const void* gate_scale;
    uint64_t gate_scale_len;
    const void* up_scale;
    uint64_t up_scale_len;
    const void* down_scale;
    uint64_t down_scale_len;
} objeta_hip_host_expert;

/* A single-GPU VRAM expert cache: LRU over tensors, pinned (never evicted) entries,
 * admission by size. Device memory comes from blocks that are recycled after an
 * eviction only once the work that may read them has passed (event fences, no host
 * waits): every stream of the context for a block whose pointer this API returned,
 * the streams of the library calls that read it otherwise (a call whose end has
 * already passed needs no fence). Not internally locked (the reference's
 * &mut CudaExpertCache). With ctx == NULL the cache keeps the accounting only and
 * owns no device memory (device pointers are NULL): the counters and LRU order
 * behave identically. */
typedef struct objeta_hip_expert_cache objeta_hip_expert_cache;

/* CudaExpertCache::new (moe.rs:92-111). */
int32_t objeta_hip_cache_create(objeta_hip_context* ctx, uint64_t capacity_bytes, objeta_hip_expert_cache** out);
int32_t objeta_hip_cache_destroy(objeta_hip_expert_cache* cache);
int32_t objeta_hip_cache_stats_get(const objeta_hip_expert_cache* cache, objeta_hip_cache_stats* out);
/* The bypass_oversized_experts field (moe.rs:77). */
int32_t objeta_hip_cache_set_bypass_oversized_experts(objeta_hip_expert_cache* cache, int32_t enable);
/* get (moe.rs:113-122): on a hit *hit = 1, the entry becomes most recent and its
 * device address/size are returned; on a miss *hit = 0. d_ptr/nbytes may be NULL. */
int32_t objeta_hip_cache_get(objeta_hip_expert_cache* cache, const objeta_hip_cache_key* key, int32_t* hit,
                             const void** d_ptr, uint64_t* nbytes);
/* insert (moe.rs:124-158) of the host bytes `h_src` (nbytes): the bytes are copied
 * into cache-owned device memory on the context's copy stream (ordered after
 * `stream` and before the next use on `stream`). *cached = 0 when the tensor is
 * larger than the capacity: it is then not kept and *d_ptr is a transient copy
 * that the caller releases with objeta_hip_cache_release_transient. */
int32_t objeta_hip_cache_insert(objeta_hip_expert_cache* cache, const objeta_hip_cache_key* key, const void* h_src,
                                uint64_t nbytes, objeta_hip_stream stream, const void** d_ptr, int32_t* cached);
/* get, then insert on a miss: the get_or_insert of the reference's README
 * (README.md:123), which its executor inlines (moe.rs:498-583). */
int32_t objeta_hip_cache_get_or_insert(objeta_hip_expert_cache* cache, const objeta_hip_cache_key* key,
                                       const void* h_src, uint64_t nbytes, objeta_hip_stream stream,
                                       const void** d_ptr, int32_t* hit, int32_t* cached);
/* insert_pinned (moe.rs:192-210): resident and never evicted. */
int32_t objeta_hip_cache_insert_pinned(objeta_hip_expert_cache* cache, const objeta_hip_cache_key* key,
                                       const void* h_src, uint64_t nbytes, objeta_hip_stream stream,
                                       const void** d_ptr);
/* pin (moe.rs:182-190), touch (moe.rs:160-165). */
int32_t objeta_hip_cache_pin(objeta_hip_expert_cache* cache, const objeta_hip_cache_key* key);
int32_t objeta_hip_cache_touch(objeta_hip_expert_cache* cache, const objeta_hip_cache_key* key);
/* evict_lru (moe.rs:167-180): *evicted = 1 and the key when an entry left. */
int32_t objeta_hip_cache_evict_lru(objeta_hip_expert_cache* cache, int32_t* evicted, objeta_hip_cache_key* key_out);
/* clear (moe.rs:212-218), reset_counters (moe.rs:221-226). */
int32_t objeta_hip_cache_clear(objeta_hip_expert_cache* cache);
int32_t objeta_hip_cache_reset_counters(objeta_hip_expert_cache* cache);
/* Returns a transient copy made by insert/get_or_insert with *cached == 0. */
int32_t objeta_hip_cache_release_transient(objeta_hip_expert_cache* cache, const void* d_ptr);
/* Cross-layer prefetch: starts the copies of host tensors into the cache on the
 * context's copy stream and returns without waiting, so that a later call finds
 * them resident (executor calls order their kernels after the copy; cache_get waits
 * for it on the host). Keys already resident, and tensors larger than the capacity,
 * are skipped; the others are admitted as insert admits them (counted as inserts,
 * evicting least recent entries). Not a get: hit and miss counters are unchanged.
 * No counterpart in the reference, whose executor copies misses synchronously.
 * *issued (nullable) = copies started. h_srcs must stay valid until the copies end
 * (pinned host memory lets them run asynchronously). */
int32_t objeta_hip_cache_prefetch(objeta_hip_expert_cache* cache, const objeta_hip_cache_key* keys,
                                  const void* const* h_srcs, const uint64_t* nbytes, uint64_t n, uint64_t* issued);
/* The shared-expert preload of deepseek_single_layer_moe.rs:1698-1730: for each of
 * n_layers layers, insert_pinned of the six FP8 shared tensors (gate weight/scale,
 * up weight/scale, down weight/scale of shared[l]) under the keys (first_layer + l,
 * 0, OBJETA_HIP_TENSOR_SHARED_*, OBJETA_HIP_FP4_E2M1). *bytes / *ms (nullable): the
 * bytes preloaded and the host time including the copies. */
int32_t objeta_hip_cache_preload_shared(objeta_hip_expert_cache* cache, const objeta_hip_host_expert* shared,
                                        uint64_t n_layers, uint64_t first_layer, objeta_hip_stream stream,
                                        uint64_t* bytes, float* ms);
/* The keys in LRU order (least recent first), up to cap of them; *n = count. */
int32_t objeta_hip_cache_order(const objeta_hip_expert_cache* cache, objeta_hip_cache_key* keys, uint64_t cap,
                               uint64_t* n);

/* ---------------------------------------- FP8-activation ("official") path */
/* The DeepSeek official arithmetic: activations quantized to F8_E4M3 bytes with
 * one F8_E8M0 scale per 128 elements, FP8 x FP4 and FP8 x FP8 GEMVs, and the
 * routed / shared expert compositions. Results follow the reference's CPU
 * definitions (crates/objeta-parser/src/deepseek.rs:1444-1716): act_quant bytes
 * exactly; GEMV sums in another order (within 1e-4 relative). */

/* cuda_act_quant_device (quant.rs:1229-1281) with cpu_act_quant's bytes
 * (deepseek.rs:1484-1525), over rows x cols floats (cols % 128 == 0): d_values
 * [rows][cols] F8_E4M3, d_scales [rows][cols/128] F8_E8M0, and, when d_dequant is
 * set, the dequantized values act_v * act_s as floats (d_dequant may alias d_x).
 * Each output is nullable; at least one is required. d_x and d_dequant 8-byte,
 * d_values 2-byte aligned. */
int32_t objeta_hip_act_quant_fp8_device(objeta_hip_context* ctx, objeta_hip_stream stream, const float* d_x,
                                        uint64_t rows, uint64_t cols, uint8_t* d_values, uint8_t* d_scales,
                                        float* d_dequant);

/* cuda_fp8_act_fp4_weight_gemv_device (quant.rs:1284-1325), arithmetic of
 * cpu_fp8_act_fp4_weight_gemv_f32 (deepseek.rs:1528-1566), for `batch`
 * activation vectors: d_out[b][r] = sum_c act(b, c) * fp4(r, c) * ws(r, c / 32)
 * with act = f8e4m3(d_act_values[b][c]) * e8m0(d_act_scales[b][c / 128]); weights
 * in the split layout (nibbles [rows][k/2], E8M0 [rows][k/32]). k_logical % 128 == 0. */
int32_t objeta_hip_fp8_act_fp4_weight_gemv_device(objeta_hip_context* ctx, objeta_hip_stream stream,
                                                  const uint8_t* d_act_values, const uint8_t* d_act_scales,
                                                  const uint8_t* d_weight, const uint8_t* d_weight_scales,
                                                  float* d_out, uint64_t rows, uint64_t k_logical, uint64_t batch);

/* cuda_fp8_act_fp8_weight_gemv_device (quant.rs:1328-1362), arithmetic of
 * cpu_fp8_act_fp8_weight_gemv (deepseek.rs:1630-1661): FP8 E4M3 weights
 * [rows][k] with E8M0 scales on a 128 x 128 tile grid [ceil(rows/128)][k/128];
 * products summed in f32 (the reference sums in f64). k_logical % 128 == 0;
 * d_weight 16-byte aligned. */
int32_t objeta_hip_fp8_act_fp8_weight_gemv_device(objeta_hip_context* ctx, objeta_hip_stream stream,
                                                  const uint8_t* d_act_values, const uint8_t* d_act_scales,
                                                  const uint8_t* d_weight, const uint8_t* d_weight_scales,
                                                  float* d_out, uint64_t rows, uint64_t k_logical, uint64_t batch);

/* The device part of execute_selected_moe_official_routed_fp4_cuda
 * (moe.rs:1393-1663) batched over tokens. For token t:
 *   xq     = act_quant(x_t)                               (dequantized)
 *   act_j  = swiglu(gate_e xq, up_e xq), e = d_table[d_ids[t*k + j]] (FP4 split)
 *   act_s  = swiglu(gate_s xq, up_s xq)                   (d_shared_fp8, FP8 tiles)
 *   out_t  = sum_j d_weights[t*k + j] * down_e(act_quant(act_j)) + down_s(act_quant(act_s))
 * swiglu(g, u) = g / (1 + exp(-g)) * clamp(u, -L, L) (the CPU compositions,
 * deepseek.rs:1680-1686, 1708-1713; the reference's CUDA silu_mul also clamps g
 * to <= L). L = swiglu_limit >= 0. d_shared_fp8: a device pointer to one
 * objeta_hip_expert_ptrs whose tensors are FP8 E4M3 with 128 x 128 E8M0 scale
 * tiles, or NULL. k = 0 leaves the shared expert alone. hidden and intermediate
 * are multiples of 128. d_inter_values [n_tokens*kk][intermediate] and
 * d_inter_scales [n_tokens*kk][intermediate/128] (nullable; kk = k + 1 with a
 * shared expert, else k) receive the intermediates' FP8 codes: rows t*k + j for
 * the routed slots, then n_tokens*k + t for the shared expert. From 6 tokens
 * (and up to 1024 (token, slot) assignments over at most 1024 experts) the layer
 * runs on the grouped-token products of objeta_hip_moe_grouped_device: each selected
 * expert, and the shared expert, read once per set of up to 8 of its tokens. The
 * results agree with the per-token kernels within the fp32 tolerance (the sums run
 * in another order), so an intermediate code near a rounding boundary can differ. */
int32_t objeta_hip_moe_official_fp4_device(objeta_hip_context* ctx, objeta_hip_stream stream,
                                           const objeta_hip_expert_ptrs* d_table, uint64_t n_table,
                                           const objeta_hip_expert_ptrs* d_shared_fp8, const uint32_t* d_ids,
                                           const float* d_weights, uint64_t n_tokens, uint64_t k, const float* d_x,
                                           float* d_out, uint64_t hidden, uint64_t intermediate, uint64_t out_dim,
                                           float swiglu_limit, uint8_t* d_inter_values, uint8_t* d_inter_scales);

/* ------------------------------------------------ host-in/host-out executor */

/* MoeTelemetry (moe.rs:236-276); bytes_by_tensor_kind flattened. The fused
 * kernels report their time under gate_up_qgemv_ms (gate + up + SiLU) and
 * down_qgemv_ms (down + weighted combine); activation_ms and accum_ms are 0. */
typedef struct {
    uint64_t selected_expert_count;
    uint64_t logical_expert_bytes_requested;
    uint64_t actual_expert_bytes_loaded;
    uint64_t resident_cache_bytes_reused;
    uint64_t weight_bytes_loaded;
    uint64_t weight_bytes_reused;
    uint64_t scale_bytes_loaded;
    uint64_t scale_bytes_reused;
    uint64_t resident_cache_resident_bytes;
    uint64_t resident_cache_capacity_bytes;
    uint64_t resident_cache_hit_count;
    uint64_t resident_cache_miss_count;
    uint64_t resident_cache_eviction_count;
    uint64_t resident_cache_insert_attempt_count;
    uint64_t resident_cache_insert_accept_count;
    uint64_t resident_cache_insert_bypass_count;
    uint64_t resident_cache_oversized_tensor_bypass_count;
    uint64_t resident_cache_oversized_expert_bypass_count;
    uint64_t resident_cache_self_eviction_risk_count;
    uint64_t dequantized_scratch_bytes;
    float h2d_ms;
    float gate_up_qgemv_ms;
    float activation_ms;
    float down_qgemv_ms;
    float accum_ms;
    float unaccounted_ms;
    float total_ms;
    float shared_expert_ms;
    uint64_t bytes_by_tensor_kind_gate;
    uint64_t bytes_by_tensor_kind_up;
    uint64_t bytes_by_tensor_kind_down;
    uint64_t bytes_per_expert;
    uint64_t selected_working_set_bytes;
    uint64_t routed_fp4_bytes_loaded;
    uint64_t routed_fp4_bytes_reused;
    uint64_t shared_fp8_bytes_loaded;
    uint64_t shared_fp8_bytes_reused;
    uint64_t total_logical_bytes;
    uint64_t total_loaded_bytes;
    uint64_t total_reused_bytes;
} objeta_hip_moe_telemetry;

/* MoeExecutor::execute_selected_moe_cuda (moe.rs:352-751) for the block formats
 * (the reference hard-codes Q4_0; Q5_0 and IQ3_0 are accepted too) and
 * execute_selected_moe_native_fp4_cuda (moe.rs:816-1280) for
 * OBJETA_HIP_FP4_E2M1 (split layout). Host x in, host out[out_dim] out (zero
 * based, as the reference). Selection (sel_ids[i], sel_weights[i]) in order;
 * experts[n_experts]. cache may be NULL. Validation messages, cache keys,
 * admission and the telemetry byte invariant
 * logical == loaded + reused (moe.rs:743-748) follow the reference. The weights
 * of cache misses are copied on the context's copy stream; each expert's kernels
 * wait only for its own copies. tel may be NULL. */
int32_t objeta_hip_moe_execute_selected(objeta_hip_context* ctx, int32_t format, objeta_hip_stream stream,
                                        const objeta_hip_host_expert* experts, uint64_t n_experts,
                                        const uint64_t* sel_ids, const float* sel_weights, uint64_t n_selected,
                                        const float* x, uint64_t x_len, uint64_t hidden, uint64_t intermediate,
                                        uint64_t out_dim, uint64_t layer_id, objeta_hip_expert_cache* cache,
                                        float* out, objeta_hip_moe_telemetry* tel);

/* execute_selected_moe_official_routed_fp4_cuda (moe.rs:1393-1663): host x in,
 * host out[out_dim] out, for one token; experts are FP4 split host tensors
 * (gate/up/down weight and scale, cached under the reference's keys), shared_fp8
 * (nullable) a host struct of device addresses of the FP8 shared expert (device
 * resident, as DeepSeekFp8SharedExpertWeightsDevice). The reference passes 10.0
 * as swiglu_limit. Telemetry follows the reference's official accounting:
 * logical bytes = the unique selected experts' working set; routed_fp4_* and
 * shared_fp8_* / total_* fields filled; resident-cache counters other than
 * hit/miss/eviction 0; activation_ms = the intermediate act_quant; shared_expert_ms =
 * the shared expert's launches. shared_from_cache != 0 (with a cache) first resolves
 * the shared expert from the cache's entries (layer_id, 0, OBJETA_HIP_TENSOR_SHARED_*,
 * OBJETA_HIP_FP4_E2M1), as objeta_hip_cache_preload_shared leaves them, by get in
 * key order stopping at the first miss (the sketch in
 * crates/objeta-cuda/src/moe_tmp.txt:1-35); shared_fp8 is the fallback. A shared
 * expert from the cache counts its resident bytes under shared_fp8_bytes_reused. */
int32_t objeta_hip_moe_execute_official_fp4(objeta_hip_context* ctx, objeta_hip_stream stream,
                                            const objeta_hip_host_expert* experts, uint64_t n_experts,
                                            const uint64_t* sel_ids, const float* sel_weights, uint64_t n_selected,
                                            const float* x, uint64_t x_len, uint64_t hidden, uint64_t intermediate,
                                            uint64_t out_dim, uint64_t layer_id, objeta_hip_expert_cache* cache,
                                            const objeta_hip_expert_ptrs* shared_fp8, int32_t shared_from_cache,
                                            float swiglu_limit, float* out, objeta_hip_moe_telemetry* tel);

/* One layer of a cached decode stack: its routed experts in host memory (pinned,
 * so that cache misses copy asynchronously) and its router on the device. */
typedef struct {
    const objeta_hip_host_expert* experts; /* [n_experts] */
    uint64_t n_experts;
    const float* d_router_w;    /* [n_experts][hidden] device */
    const float* d_router_bias; /* [n_experts] device, or NULL */
    uint64_t layer_id;          /* the layer of the cache keys */
} objeta_hip_cached_layer;

/* Accounting of one objeta_hip_moe_stack_cached call, summed over its layers.
 * logical = loaded + reused (the byte invariant of moe.rs:743-748, per layer over
 * the union of the batch's selected experts). */
typedef struct {
    uint64_t layers;
    uint64_t tokens;
    uint64_t logical_expert_bytes_requested;
    uint64_t actual_expert_bytes_loaded;  /* copied on the copy stream for the layers' own selections */
    uint64_t resident_cache_bytes_reused; /* cache hits, prefetched tensors included */
    uint64_t distinct_experts;            /* sum over layers of the union's size */
    uint64_t prefetch_experts_predicted;  /* (token, slot) predictions made for the next layer */
    uint64_t prefetch_experts_correct;    /* of those, selected by the next layer's router */
    uint64_t prefetch_tensors_issued;     /* tensors copied ahead by the predictions */
    uint64_t prefetch_bytes_issued;
    float total_ms;     /* the call's work on its stream, first router to last layer */
    float copy_ms;      /* copy-stream time of the layers' own misses */
    float host_wait_ms; /* host time blocked on the routers' results */
    float reserved;
} objeta_hip_stack_telemetry;

/* A decode stack with the experts behind the expert cache: n_tokens tokens through
 * n_layers layers, the hidden state d_h [n_tokens][hidden] updated in place (h +=
 * MoE(h) per layer, the residual stream). No counterpart in the reference as one
 * call: it is the loop its drivers run over execute_selected_moe_cuda
 * (moe.rs:352-751; bench_selected_moe.rs:292-299, deepseek_single_layer_moe.rs
 * 2160-2207) with the hidden state kept on the device. Per layer: the router on
 * the device (softmax -> top-k, renormalised when renormalize != 0), its ids to the
 * host, the cache resolving the union of the batch's selected experts (get, then
 * insert with a copy on the copy stream for misses: the reference's admission and
 * counters), and the expert kernels waiting for that layer's copies only; batches
 * of 12 tokens and more run the grouped-token products. prefetch_next != 0 also
 * evaluates layer l+1's router on layer l's input and starts copying its predicted
 * experts' absent tensors behind layer l's own (objeta_hip_cache_prefetch).
 * ids_out / weights_out (host, [n_layers][n_tokens][k], nullable) receive the
 * selections; d_trace (device, [n_layers][n_tokens][hidden], nullable) the hidden
 * state after each layer. Returns after the last layer completed. Experts of every
 * layer are validated against (hidden, intermediate) before any launch. */
int32_t objeta_hip_moe_stack_cached(objeta_hip_context* ctx, int32_t format, objeta_hip_stream stream,
                                    const objeta_hip_cached_layer* layers, uint64_t n_layers, uint64_t k,
                                    int32_t renormalize, uint64_t n_tokens, float* d_h, uint64_t hidden,
                                    uint64_t intermediate, objeta_hip_expert_cache* cache, int32_t prefetch_next,
                                    uint32_t* ids_out, float* weights_out, float* d_trace,
                                    objeta_hip_stack_telemetry* tel);

/* ------------------------------------------------------ checkpoint ingest */
/* Memory-mapped safetensors files: ModelWeights (crates/objeta-parser/src/lib.rs:
 * 88-293). A path names one file or a directory whose *.safetensors shards are
 * read in file-name order (a later shard's tensor replaces an earlier one of the
 * same name). Tensor data stays in the mapping until objeta_hip_st_close; raw
 * pointers are zero-copy views of it. Errors of files and headers are
 * OBJETA_HIP_ERR_IO, as the reference's driver wraps ModelWeights errors. */
typedef struct objeta_hip_st_model objeta_hip_st_model;

/* Dtype (lib.rs:30-41). */
enum {
    OBJETA_HIP_DT_F32 = 0,
    OBJETA_HIP_DT_F16 = 1,
    OBJETA_HIP_DT_BF16 = 2,
    OBJETA_HIP_DT_I64 = 3,
    OBJETA_HIP_DT_I32 = 4,
    OBJETA_HIP_DT_I8 = 5,
    OBJETA_HIP_DT_U8 = 6,
    OBJETA_HIP_DT_F8_E8M0 = 7,
    OBJETA_HIP_DT_F8_E4M3 = 8,
    OBJETA_HIP_DT_BOOL = 9
};

/* TensorInfo (lib.rs:20-28); shape holds the first 8 dimensions, file the index of
 * the shard the tensor came from. */
typedef struct {
    int32_t dtype;
    uint32_t ndim;
    uint64_t shape[8];
    uint64_t nbytes;
    uint64_t nelem;
    uint32_t file;
    uint32_t reserved;
} objeta_hip_st_info;

/* ModelWeights::open (lib.rs:104-178) with parse_header (lib.rs:180-213). */
int32_t objeta_hip_st_open(const char* path, objeta_hip_st_model** out);
int32_t objeta_hip_st_close(objeta_hip_st_model* model);
/* len (lib.rs:279-281); keys (lib.rs:221-224) by index, in sorted name order:
 * *len = the name's length, buf (nullable) receives it NUL-terminated. */
int32_t objeta_hip_st_len(const objeta_hip_st_model* model, uint64_t* n);
int32_t objeta_hip_st_key(const objeta_hip_st_model* model, uint64_t i, char* buf, uint64_t cap, uint64_t* len);
/* info / contains (lib.rs:216-230): *found = 0 when the name is absent. */
int32_t objeta_hip_st_info_get(const objeta_hip_st_model* model, const char* name, int32_t* found,
                               objeta_hip_st_info* out);
/* get_raw (lib.rs:232-241): the tensor's bytes in the mapping. */
int32_t objeta_hip_st_get_raw(const objeta_hip_st_model* model, const char* name, const void** ptr,
                              uint64_t* nbytes);
/* get_f32 (lib.rs:243-276): F32 copied, F16 and BF16 converted (half_to_f32 and
 * bf16_to_f32, lib.rs:297-330); other dtypes fail. out NULL: only *nelem. */
int32_t objeta_hip_st_get_f32(const objeta_hip_st_model* model, const char* name, float* out, uint64_t cap,
                              uint64_t* nelem);
/* A routed DeepSeek expert of layer `layer` (mtp != 0: the "mtp.<layer>" block
 * family) found by classify_tensor's rules (crates/objeta-parser/src/deepseek.rs:
 * 178-262; w1 = gate, w3 = up, w2 = down, ".scale" = E8M0 scales), as
 * find_fp4_expert_tensors does (deepseek_single_layer_moe.rs:410-520): the split
 * FP4 tensors (I8/U8 [rows][cols/2] + F8_E8M0 [rows][cols/32]) as zero-copy host
 * tensors for the executors, with the expert's dimensions. */
int32_t objeta_hip_st_deepseek_expert(const objeta_hip_st_model* model, uint64_t layer, uint64_t expert,
                                      int32_t mtp, objeta_hip_host_expert* out, uint64_t* hidden,
                                      uint64_t* intermediate, uint64_t* out_dim);
/* load_shared_expert_fp8 (deepseek_single_layer_moe.rs:1034-1080): the FP8 shared
 * expert "<prefix>.ffn.shared_experts.w{1,3,2}.{weight,scale}" (F8_E4M3 [rows][cols]
 * with E8M0 scales on the 128 x 128 tile grid). */
int32_t objeta_hip_st_deepseek_shared_expert(const objeta_hip_st_model* model, uint64_t layer, int32_t mtp,
                                             objeta_hip_host_expert* out, uint64_t* hidden,
                                             uint64_t* intermediate, uint64_t* out_dim);
/* find_router_tensor (deepseek_single_layer_moe.rs:226-330): the single router
 * "...gate.weight" tensor [num_experts][hidden] of the layer and block family
 * (Hyper-Connection hc_ffn_* tensors excluded). name_buf (nullable) receives its
 * name; read it with objeta_hip_st_get_f32. */
int32_t objeta_hip_st_deepseek_router(const objeta_hip_st_model* model, uint64_t layer, int32_t mtp,
                                      char* name_buf, uint64_t cap, objeta_hip_st_info* info);

#ifdef __cplusplus
}
#endif
#endif /* OBJETA_HIP_H */
