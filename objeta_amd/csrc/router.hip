// router.hip — router logits, softmax and top-k on gfx950.
//
// Reference semantics: cpu_router (crates/objeta-cuda/src/bin/
// deepseek_single_layer_moe.rs:687-743) computes each logit as a *sequential*
// fp32 sum of rounded products, takes a softmax over all experts and a stable
// descending sort (ties keep the lower expert id); the k selected probabilities
// are then renormalised (crates/objeta-qwen36-executor/src/moe_dispatch.rs:403-435).
//
// A sequential 2048-term sum per expert is a ~2048-deep dependency chain, far
// too slow for the decode critical path. Instead each wave computes one expert's
// exact sum S of the rounded products in double precision together with a
// rigorous bound B on |S - sequential fp32 sum| (Higham's recursive-summation
// bound u * sum_k |S_k| / (1 - n u), with the prefix sums S_k from a wave scan).
// Workgroup 0 of a token gathers the epoch-tagged words and ranks the experts; if
// every decision the top-k depends on is separated by more than the bounds, the
// ids are provably those of the sequential sums. Otherwise it recomputes every
// logit in the reference's sequential order (one lane per expert) and ranks those
// exact values.
#include "device_common.hpp"
#include "router_math.hpp"
#include "host_common.hpp"
#include "kernels.hpp"

namespace objeta {
namespace {

using namespace rmath;
using dev::gptr;
using dev::as_global;

// Workgroup 0 of token t: gathers the words of this epoch, selects, writes the
// ids and weights and advances counters[t]. If some words have not arrived after
// spin_limit polls (the other workgroups not yet scheduled: the device busy with
// other work), it computes every logit itself in the reference's order, so the
// result never depends on which workgroups are resident together, and sets bit 1
// of the error word. spin_limit 0: it never waits.
template <class XAt>
__device__ void router_select(const float* __restrict__ w_r, const float* __restrict__ bias,
                              const float* __restrict__ xt, XAt xat, uint32_t n_experts, uint32_t hidden, uint32_t k,
                              int renormalize, uint32_t* __restrict__ ids, float* __restrict__ weights,
                              const uint64_t* ws_logit, const uint64_t* ws_bound, uint32_t epoch,
                              uint32_t* __restrict__ counter, uint32_t* __restrict__ err, float* scratch,
                              uint32_t scratch_floats, uint32_t spin_limit,
                              const objeta_hip_expert_ptrs* tab_lds = nullptr,
                              objeta_hip_expert_ptrs* sel_tab = nullptr) {
    __shared__ SelectLds<kMaxExperts> s;
    __shared__ int s_pending;
    stage_exptab(s);  // the softmax exps' table, in LDS before the ranking needs it
    bool starved = spin_limit == 0;  // 0: never wait
    for (uint32_t spin = 0; !starved; ++spin) {
        if (threadIdx.x == 0) s_pending = 0;
        __syncthreads();
        int pending = 0;
        for (uint32_t j = threadIdx.x; j < n_experts; j += kRThreads) {
            const uint64_t a = __hip_atomic_load(&ws_logit[j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const uint64_t b = __hip_atomic_load(&ws_bound[j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (static_cast<uint32_t>(a >> 32) != epoch || static_cast<uint32_t>(b >> 32) != epoch) pending = 1;
            s.val[j] = __builtin_bit_cast(float, static_cast<uint32_t>(a));
            s.bnd[j] = __builtin_bit_cast(float, static_cast<uint32_t>(b));
        }
        if (pending) s_pending = 1;
        __syncthreads();
        if (!s_pending) break;
        if (spin >= spin_limit) {  // uniform: every thread read the same s_pending
            starved = true;
            break;
        }
        __builtin_amdgcn_s_sleep(1);
    }
    if (starved && threadIdx.x == 0) atomicOr(err, 2u);  // reported; the result stays exact
    if (starved || (!select_certain(s, n_experts, k, renormalize) &&
                    !select_refine(s, w_r, bias, xat, n_experts, hidden, k, renormalize, scratch, scratch_floats) &&
                    !select_underflow(s, w_r, bias, xat, n_experts, hidden, k, scratch, scratch_floats)))
        select_sequential(s, w_r, bias, xat, n_experts, hidden, k);
    write_selection(s, k, renormalize, ids, weights);
    // the selected experts' table entries (the table was staged in LDS while the
    // logits were awaited), so that the expert kernels need not look up id, then table
    if (sel_tab && threadIdx.x < k) sel_tab[threadIdx.x] = tab_lds[s.sel[threadIdx.x]];
    if (threadIdx.x == 0) __hip_atomic_store(counter, epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// General form: each wave reads its expert's row and x from global memory.
template <bool VEC>
__global__ __launch_bounds__(kRThreads) void router_kernel(
    const float* __restrict__ w_r, const float* __restrict__ bias, const float* __restrict__ x,
    uint32_t n_experts, uint32_t hidden, uint32_t k, int renormalize, uint32_t* __restrict__ ids,
    float* __restrict__ weights, uint64_t* __restrict__ ws, uint32_t* __restrict__ counters,
    uint32_t* __restrict__ err, uint32_t spin_limit) {
    const uint32_t t = blockIdx.y;
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t e = blockIdx.x * kRWaves + (threadIdx.x >> 6);
    const float* xt = x + static_cast<size_t>(t) * hidden;
    // fixed stride per token: a word's address always belongs to the same token's
    // epoch sequence, so words left by earlier calls carry older epochs
    uint64_t* ws_logit = ws + static_cast<size_t>(t) * 2 * kMaxExperts;
    uint64_t* ws_bound = ws_logit + kMaxExperts;
    const uint32_t epoch = __hip_atomic_load(&counters[t], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;

    if (e < n_experts) {
        // the bias requested without a branch (a load under `if (bias)` is waited for at
        // the branch's end, before the row loads), its value selected where it is used
        const float bias_raw = *(bias ? bias + e : w_r);
        const float* row = w_r + static_cast<size_t>(e) * hidden;
        double total, abs_prefix;
        if constexpr (VEC) exact_logit_vec(row, xt, hidden, lane, total, abs_prefix);
        else exact_logit_scalar(row, xt, hidden, lane, total, abs_prefix);
        if (lane == 0) {
            float lhat, bnd;
            finish_logit(total, abs_prefix, bias ? bias_raw : 0.0f, hidden, lhat, bnd);
            __hip_atomic_store(&ws_logit[e], tag(lhat, epoch), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(&ws_bound[e], tag(bnd, epoch), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    if (blockIdx.x != 0) return;
    __shared__ float scratch[kRWaves * 256];
    router_select(w_r, bias, xt, [xt](uint32_t h) { return xt[h]; }, n_experts, hidden, k, renormalize,
                  ids + static_cast<size_t>(t) * k, weights + static_cast<size_t>(t) * k, ws_logit, ws_bound, epoch,
                  &counters[t], err, scratch, kRWaves * 256, spin_limit);
}

// hidden % 256 == 0, hidden <= 256 * NB: the row sits lane-contiguously in
// registers (lane l: elements [l*hidden/64, (l+1)*hidden/64)) and x is staged in
// LDS, so a logit is one pass of lane-local prefix sums (exact_logit_lanes)
// instead of a wave scan per 256 elements.
constexpr uint32_t kRefineScratch = kRWaves * 4096;  // floats of row chunks for select_refine

template <int NB>
__global__ __launch_bounds__(kRThreads) void router_lanes_kernel(
    const float* __restrict__ w_r, const float* __restrict__ bias, const float* __restrict__ x,
    uint32_t n_experts, uint32_t hidden, uint32_t k, int renormalize, uint32_t* __restrict__ ids,
    float* __restrict__ weights, uint64_t* __restrict__ ws, uint32_t* __restrict__ counters,
    uint32_t* __restrict__ err, uint32_t spin_limit) {
    extern __shared__ float xs[];  // x in the padded pair layout: (hidden / 64) * kPadX floats
    const uint32_t t = blockIdx.y;
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t e = blockIdx.x * kRWaves + (threadIdx.x >> 6);
    const float* xt = x + static_cast<size_t>(t) * hidden;
    uint64_t* ws_logit = ws + static_cast<size_t>(t) * 2 * kMaxExperts;
    uint64_t* ws_bound = ws_logit + kMaxExperts;
    const uint32_t epoch = __hip_atomic_load(&counters[t], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;
    const uint32_t n4 = hidden >> 8;  // float4 per lane
    const uint32_t ec = e < n_experts ? e : n_experts - 1;
    // the bias requested without a branch (a load under `if (bias)` is waited for at the
    // branch's end, before the row loads), its value selected where it is used
    const float bias_raw = *(bias ? bias + ec : w_r);
    float4 wr[NB];
    {
        typedef float f32x4 __attribute__((ext_vector_type(4)));
        const gptr<f32x4> r4 = as_global(reinterpret_cast<const f32x4*>(w_r + static_cast<size_t>(ec) * hidden));
#pragma unroll
        for (int g = 0; g < NB; ++g) {
            const f32x4 v = r4[lane * n4 + (static_cast<uint32_t>(g) < n4 ? static_cast<uint32_t>(g) : n4 - 1)];
            wr[g] = make_float4(v.x, v.y, v.z, v.w);
        }
    }
    for (uint32_t i = threadIdx.x; i < (hidden >> 2); i += kRThreads) {
        const uint32_t c = i << 2;
        *reinterpret_cast<float4*>(xs + (c >> 6) * kPadX + (c & 63)) = reinterpret_cast<const float4*>(xt)[i];
    }
    __syncthreads();
    if (e < n_experts) {
        double total, abs_bound;
        exact_logit_lanes<NB>(wr, xs, n4, lane, total, abs_bound);
        if (lane == 0) {
            float lhat, bnd;
            finish_logit(total, abs_bound, bias ? bias_raw : 0.0f, hidden, lhat, bnd);
            __hip_atomic_store(&ws_logit[e], tag(lhat, epoch), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(&ws_bound[e], tag(bnd, epoch), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    if (blockIdx.x != 0) return;
    // x stays in LDS for the refinement; the row chunks go behind it
    const uint32_t x_floats = (hidden / 64) * kPadX;
    const float* xl = xs;
    router_select(w_r, bias, xt, [xl](uint32_t h) { return xl[(h >> 6) * kPadX + (h & 63)]; }, n_experts, hidden, k,
                  renormalize, ids + static_cast<size_t>(t) * k, weights + static_cast<size_t>(t) * k, ws_logit,
                  ws_bound, epoch, &counters[t], err, xs + x_floats, kRefineScratch, spin_limit);
}

// hidden % 1024 == 0, hidden <= 1024 * NB: one workgroup per expert, the row split
// over its four waves (exact_logit_split), so each lane holds 4*hidden/1024
// elements and the exact sum is a short chain per lane; four times as many
// workgroups as router_lanes_kernel share the row loads.
template <int NB>
__global__ __launch_bounds__(kRThreads) void router_split_kernel(
    const float* __restrict__ w_r, const float* __restrict__ bias, const float* __restrict__ x,
    uint32_t n_experts, uint32_t hidden, uint32_t k, int renormalize, uint32_t* __restrict__ ids,
    float* __restrict__ weights, uint64_t* __restrict__ ws, uint32_t* __restrict__ counters,
    uint32_t* __restrict__ err, uint32_t spin_limit, const objeta_hip_expert_ptrs* __restrict__ table,
    objeta_hip_expert_ptrs* __restrict__ sel_tab) {
    extern __shared__ float xs[];  // x in the padded pair layout: (hidden / 64) * kPadX floats
    __shared__ double red[8];
    const uint32_t t = blockIdx.y;
    const uint32_t e = blockIdx.x;
    // workgroup 0 resolving the selection to table entries: the table's words are
    // requested first (they wait in registers until the selection needs them)
    constexpr uint32_t kTabWords = static_cast<uint32_t>(kSelTabMaxExperts) * 6 / kRThreads;
    uint64_t tw[kTabWords];
    const uint32_t n_tab = n_experts * 6;
    if (sel_tab && blockIdx.x == 0) {
        const uint64_t* tsrc = reinterpret_cast<const uint64_t*>(table);
#pragma unroll
        for (uint32_t q = 0; q < kTabWords; ++q) {
            const uint32_t i = threadIdx.x + q * kRThreads;
            tw[q] = tsrc[i < n_tab ? i : n_tab - 1];
        }
    }
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const float* xt = x + static_cast<size_t>(t) * hidden;
    uint64_t* ws_logit = ws + static_cast<size_t>(t) * 2 * kMaxExperts;
    uint64_t* ws_bound = ws_logit + kMaxExperts;
    const uint32_t epoch = __hip_atomic_load(&counters[t], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;
    const uint32_t n4 = hidden >> 10;  // float4 per lane
    // the bias requested without a branch (a load under `if (bias)` is waited for at the
    // branch's end, before the row loads), its value selected where it is used
    const float bias_raw = *(bias ? bias + e : w_r);
    // the lane's row elements and the matching activations, straight into registers
    float4 wr[NB], xv[NB];
    {
        typedef float f32x4 __attribute__((ext_vector_type(4)));
        const gptr<f32x4> r4 = as_global(reinterpret_cast<const f32x4*>(w_r + static_cast<size_t>(e) * hidden));
        const gptr<f32x4> x4 = as_global(reinterpret_cast<const f32x4*>(xt));
        const uint32_t q0 = wave * n4 * 64u + lane * n4;
#pragma unroll
        for (int g = 0; g < NB; ++g) {
            const uint32_t q = q0 + (static_cast<uint32_t>(g) < n4 ? static_cast<uint32_t>(g) : n4 - 1);
            const f32x4 v = r4[q];
            wr[g] = make_float4(v.x, v.y, v.z, v.w);
            const f32x4 u = x4[q];
            xv[g] = make_float4(u.x, u.y, u.z, u.w);
        }
    }
    double total, abs_bound;
    exact_logit_split<NB>(wr, xv, n4, lane, wave, red, total, abs_bound);
    if (threadIdx.x == 0) {
        float lhat, bnd;
        finish_logit(total, abs_bound, bias ? bias_raw : 0.0f, hidden, lhat, bnd);
        __hip_atomic_store(&ws_logit[e], tag(lhat, epoch), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(&ws_bound[e], tag(bnd, epoch), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (blockIdx.x != 0) return;
    // workgroup 0 selects; x in LDS serves the recomputation of close calls (written
    // from the registers that hold it for the logit: the lanes' float4s cover all of
    // x), the table its resolution
    {
        const uint32_t q0 = wave * n4 * 64u + lane * n4;
#pragma unroll
        for (int g = 0; g < NB; ++g) {
            if (static_cast<uint32_t>(g) < n4) {
                const uint32_t c = (q0 + static_cast<uint32_t>(g)) << 2;
                *reinterpret_cast<float4*>(xs + (c >> 6) * kPadX + (c & 63)) = xv[g];
            }
        }
    }
    const uint32_t x_floats = (hidden / 64) * kPadX;
    auto* tab_lds = reinterpret_cast<objeta_hip_expert_ptrs*>(xs + x_floats + kRefineScratch);
    if (sel_tab) {
        uint64_t* tl = reinterpret_cast<uint64_t*>(tab_lds);
#pragma unroll
        for (uint32_t q = 0; q < kTabWords; ++q) {
            const uint32_t i = threadIdx.x + q * kRThreads;
            if (i < n_tab) tl[i] = tw[q];
        }
    }
    __syncthreads();
    const float* xl = xs;
    router_select(w_r, bias, xt, [xl](uint32_t h) { return xl[(h >> 6) * kPadX + (h & 63)]; }, n_experts, hidden, k,
                  renormalize, ids + static_cast<size_t>(t) * k, weights + static_cast<size_t>(t) * k, ws_logit,
                  ws_bound, epoch, &counters[t], err, xs + x_floats, kRefineScratch, spin_limit, tab_lds,
                  sel_tab ? sel_tab + static_cast<size_t>(t) * k : nullptr);
}

// Batches (n_tokens >= 2) of router_split_kernel's shapes in two launches. First the
// logits: the same arithmetic per (expert, token) as router_split_kernel, so a token
// gets the same words as in a call of its own, but each row is read once for a group
// of tb tokens (one workgroup per row and token holds a full-size LDS allocation for
// the selection, which capped a batch at two workgroups per CU). grid = (E,
// ceil(T / tb)); workgroup (e, g) keeps row e in registers and publishes its logit
// and bound for tokens g*tb .. g*tb + tb - 1, the next token's activations in flight
// during each sum.
template <int NB>
__global__ __launch_bounds__(kRThreads) void router_logits_batch_kernel(
    const float* __restrict__ w_r, const float* __restrict__ bias, const float* __restrict__ x, uint32_t n_tokens,
    uint32_t hidden, uint32_t tb, uint64_t* __restrict__ ws, const uint32_t* __restrict__ counters) {
    __shared__ double red[8];
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    const uint32_t e = blockIdx.x;
    const uint32_t t0 = blockIdx.y * tb;
    const uint32_t t1 = t0 + tb < n_tokens ? t0 + tb : n_tokens;
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t n4 = hidden >> 10;  // float4 per lane
    const uint32_t q0 = wave * n4 * 64u + lane * n4;
    // the bias requested without a branch (a load under `if (bias)` is waited for at the
    // branch's end, before the row loads), its value selected where it is used
    const float bias_raw = *(bias ? bias + e : w_r);
    float4 wr[NB], xv[NB], xn[NB];
    auto load_x = [&](uint32_t t, float4 (&dst)[NB]) {
        const gptr<f32x4> x4 = as_global(reinterpret_cast<const f32x4*>(x + static_cast<size_t>(t) * hidden));
#pragma unroll
        for (int g = 0; g < NB; ++g) {
            const f32x4 u = x4[q0 + (static_cast<uint32_t>(g) < n4 ? static_cast<uint32_t>(g) : n4 - 1)];
            dst[g] = make_float4(u.x, u.y, u.z, u.w);
        }
    };
    {
        const gptr<f32x4> r4 = as_global(reinterpret_cast<const f32x4*>(w_r + static_cast<size_t>(e) * hidden));
#pragma unroll
        for (int g = 0; g < NB; ++g) {
            const f32x4 v = r4[q0 + (static_cast<uint32_t>(g) < n4 ? static_cast<uint32_t>(g) : n4 - 1)];
            wr[g] = make_float4(v.x, v.y, v.z, v.w);
        }
    }
    load_x(t0, xv);
    for (uint32_t t = t0; t < t1; ++t) {
        if (t + 1 < t1) load_x(t + 1, xn);
        // red: every wave has passed both barriers of the previous sum before this
        // one writes it again
        double total, abs_bound;
        exact_logit_split<NB>(wr, xv, n4, lane, wave, red, total, abs_bound);
        if (threadIdx.x == 0) {
            const uint32_t epoch = __hip_atomic_load(&counters[t], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;
            uint64_t* ws_logit = ws + static_cast<size_t>(t) * 2 * kMaxExperts;
            float lhat, bnd;
            finish_logit(total, abs_bound, bias ? bias_raw : 0.0f, hidden, lhat, bnd);
            __hip_atomic_store(&ws_logit[e], tag(lhat, epoch), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(&ws_logit[kMaxExperts + e], tag(bnd, epoch), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        }
#pragma unroll
        for (int g = 0; g < NB; ++g) xv[g] = xn[g];
    }
}

// Then one workgroup per token selects from the published words (all of this
// epoch: the logits launch has finished), as workgroup 0 of router_split_kernel
// does, and advances counters[t]; table / sel_tab as there (the table read from
// global memory).
__global__ __launch_bounds__(kRThreads) void router_select_batch_kernel(
    const float* __restrict__ w_r, const float* __restrict__ bias, const float* __restrict__ x,
    uint32_t n_experts, uint32_t hidden, uint32_t k, int renormalize, uint32_t* __restrict__ ids,
    float* __restrict__ weights, uint64_t* __restrict__ ws, uint32_t* __restrict__ counters,
    uint32_t* __restrict__ err, uint32_t spin_limit, const objeta_hip_expert_ptrs* __restrict__ table,
    objeta_hip_expert_ptrs* __restrict__ sel_tab) {
    extern __shared__ float xs[];  // x in the padded pair layout, then the refinement scratch
    const uint32_t t = blockIdx.x;
    const float* xt = x + static_cast<size_t>(t) * hidden;
    uint64_t* ws_logit = ws + static_cast<size_t>(t) * 2 * kMaxExperts;
    uint64_t* ws_bound = ws_logit + kMaxExperts;
    const uint32_t epoch = __hip_atomic_load(&counters[t], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;
    for (uint32_t i = threadIdx.x; i < (hidden >> 2); i += kRThreads) {
        const uint32_t c = i << 2;
        *reinterpret_cast<float4*>(xs + (c >> 6) * kPadX + (c & 63)) = reinterpret_cast<const float4*>(xt)[i];
    }
    __syncthreads();
    const uint32_t x_floats = (hidden / 64) * kPadX;
    const float* xl = xs;
    router_select(w_r, bias, xt, [xl](uint32_t h) { return xl[(h >> 6) * kPadX + (h & 63)]; }, n_experts, hidden, k,
                  renormalize, ids + static_cast<size_t>(t) * k, weights + static_cast<size_t>(t) * k, ws_logit,
                  ws_bound, epoch, &counters[t], err, xs + x_floats, kRefineScratch, spin_limit, table,
                  sel_tab ? sel_tab + static_cast<size_t>(t) * k : nullptr);
}

__global__ __launch_bounds__(256) void softmax_exp_kernel(const float* __restrict__ x, float* __restrict__ y,
                                                          uint64_t n) {
    const uint64_t i = static_cast<uint64_t>(blockIdx.x) * 256u + threadIdx.x;
    if (i < n) y[i] = expf_glibc(x[i]);
}

}  // namespace

static_assert(kMaxRouterExperts == static_cast<uint64_t>(kMaxExperts), "router workspace layout");

int32_t launch_router(objeta_hip_context* ctx, hipStream_t s, const float* w_r, const float* bias,
                      const float* x, uint64_t n_tokens, uint64_t n_experts, uint64_t hidden, uint64_t k,
                      int32_t renormalize, uint32_t* ids, float* weights,
                      const objeta_hip_expert_ptrs* table, objeta_hip_expert_ptrs** sel_tab) {
    const char* action = "launch router_topk";
    if (n_experts == 0 || n_experts > kMaxExperts)
        OBJ_FAIL(kInvalidInput, action, strf("num_experts %llu must be in 1..=%d", (unsigned long long)n_experts, kMaxExperts));
    if (k == 0 || k > n_experts || k > kMaxTopK)
        OBJ_FAIL(kInvalidInput, action,
                 strf("top_k %llu must be in 1..=min(num_experts, %d)", (unsigned long long)k, kMaxTopK));
    if (hidden == 0 || hidden > (1u << 24)) OBJ_FAIL(kInvalidInput, action, "hidden must be in 1..=2^24");
    if (n_tokens == 0) return 0;
    if (n_tokens > kEpochWords) OBJ_FAIL(kInvalidInput, action, strf("n_tokens > %zu", kEpochWords));
    if (!w_r || !x || !ids || !weights) OBJ_FAIL(kInvalidInput, action, "NULL device pointer");
    // the epoch words and counters of this stream's router scratch
    StreamScratch* sc = nullptr;
    OBJ_TRY(stream_scratch(ctx, s, &sc));
    void* wsv = nullptr;
    OBJ_TRY(ensure_workspace(ctx, s, kWsRouter, static_cast<size_t>(n_tokens) * kMaxRouterExperts * 2 * sizeof(uint64_t),
                             &wsv));
    uint64_t* ws = static_cast<uint64_t*>(wsv);
    uint32_t* counters = sc->epochs;
    const dim3 grid(static_cast<uint32_t>((n_experts + kRWaves - 1) / kRWaves), static_cast<uint32_t>(n_tokens));
    const bool vec = hidden % 4 == 0 && reinterpret_cast<uintptr_t>(w_r) % 16 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0;
    uint32_t* err = ctx->err_word;
    const uint32_t spin = ctx->router_spin_limit;
    const bool lanes = vec && hidden % 256 == 0 && hidden <= 256u * 32u;
    const bool split = vec && hidden % 1024 == 0 && hidden <= 1024u * 8u;
    // a batch of the split kernel's shapes: logits for groups of tokens, then one
    // selection workgroup per token
    const bool batched = split && n_tokens >= 2;
    // table resolution (split kernel, up to kSelTabMaxExperts experts) or none
    objeta_hip_expert_ptrs* st = (sel_tab && table && split && n_experts <= kSelTabMaxExperts) ? *sel_tab : nullptr;
    if (sel_tab) *sel_tab = st;
    if (batched) {
        // enough (row, token group) workgroups for about four per CU, up to 8 tokens each
        const uint32_t cus = ctx->info.compute_units > 0 ? static_cast<uint32_t>(ctx->info.compute_units) : 256u;
        uint64_t tb = (n_experts * n_tokens + 4ull * cus - 1) / (4ull * cus);
        tb = tb < 1 ? 1 : (tb > 8 ? 8 : tb);
        const dim3 lgrid(static_cast<uint32_t>(n_experts), static_cast<uint32_t>((n_tokens + tb - 1) / tb));
        if (hidden <= 1024u * 2u)
            hipLaunchKernelGGL(router_logits_batch_kernel<2>, lgrid, dim3(kRThreads), 0, s, w_r, bias, x,
                               static_cast<uint32_t>(n_tokens), static_cast<uint32_t>(hidden),
                               static_cast<uint32_t>(tb), ws, counters);
        else
            hipLaunchKernelGGL(router_logits_batch_kernel<8>, lgrid, dim3(kRThreads), 0, s, w_r, bias, x,
                               static_cast<uint32_t>(n_tokens), static_cast<uint32_t>(hidden),
                               static_cast<uint32_t>(tb), ws, counters);
        const size_t lds = (static_cast<size_t>(hidden / 64) * kPadX + kRefineScratch) * sizeof(float);
        hipLaunchKernelGGL(router_select_batch_kernel, dim3(static_cast<uint32_t>(n_tokens)), dim3(kRThreads), lds, s,
                           w_r, bias, x, static_cast<uint32_t>(n_experts), static_cast<uint32_t>(hidden),
                           static_cast<uint32_t>(k), renormalize, ids, weights, ws, counters, err, spin,
                           st ? table : nullptr, st);
    } else if (split) {
        const size_t lds = (static_cast<size_t>(hidden / 64) * kPadX + kRefineScratch) * sizeof(float) +
                           (st ? static_cast<size_t>(n_experts) * sizeof(objeta_hip_expert_ptrs) : 0);
        const dim3 sgrid(static_cast<uint32_t>(n_experts), static_cast<uint32_t>(n_tokens));
        if (hidden <= 1024u * 2u)
            hipLaunchKernelGGL(router_split_kernel<2>, sgrid, dim3(kRThreads), lds, s, w_r, bias, x,
                               static_cast<uint32_t>(n_experts), static_cast<uint32_t>(hidden),
                               static_cast<uint32_t>(k), renormalize, ids, weights, ws, counters, err, spin,
                               st ? table : nullptr, st);
        else
            hipLaunchKernelGGL(router_split_kernel<8>, sgrid, dim3(kRThreads), lds, s, w_r, bias, x,
                               static_cast<uint32_t>(n_experts), static_cast<uint32_t>(hidden),
                               static_cast<uint32_t>(k), renormalize, ids, weights, ws, counters, err, spin,
                               st ? table : nullptr, st);
    } else if (lanes) {
        const size_t lds = (static_cast<size_t>(hidden / 64) * kPadX + kRefineScratch) * sizeof(float);
        if (hidden <= 256u * 8u)
            hipLaunchKernelGGL(router_lanes_kernel<8>, grid, dim3(kRThreads), lds, s, w_r, bias, x,
                               static_cast<uint32_t>(n_experts), static_cast<uint32_t>(hidden),
                               static_cast<uint32_t>(k), renormalize, ids, weights, ws, counters, err, spin);
        else
            hipLaunchKernelGGL(router_lanes_kernel<32>, grid, dim3(kRThreads), lds, s, w_r, bias, x,
                               static_cast<uint32_t>(n_experts), static_cast<uint32_t>(hidden),
                               static_cast<uint32_t>(k), renormalize, ids, weights, ws, counters, err, spin);
    } else if (vec)
        hipLaunchKernelGGL(router_kernel<true>, grid, dim3(kRThreads), 0, s, w_r, bias, x,
                           static_cast<uint32_t>(n_experts), static_cast<uint32_t>(hidden), static_cast<uint32_t>(k),
                           renormalize, ids, weights, ws, counters, err, spin);
    else
        hipLaunchKernelGGL(router_kernel<false>, grid, dim3(kRThreads), 0, s, w_r, bias, x,
                           static_cast<uint32_t>(n_experts), static_cast<uint32_t>(hidden), static_cast<uint32_t>(k),
                           renormalize, ids, weights, ws, counters, err, spin);
    OBJ_HIP(hipGetLastError(), action);
    return 0;
}

}  // namespace objeta

using namespace objeta;

extern "C" int32_t objeta_hip_router_topk_device(objeta_hip_context* ctx, objeta_hip_stream stream,
                                                 const float* d_w_r, const float* d_bias, const float* d_x,
                                                 uint64_t n_tokens, uint64_t n_experts, uint64_t hidden,
                                                 uint64_t k, int32_t renormalize, uint32_t* d_ids,
                                                 float* d_weights) {
    OBJ_GUARD_BEGIN
    OBJ_TRY(check_ctx(ctx, "router_topk_device"));
    OBJ_HIP(hipSetDevice(ctx->device), "hipSetDevice");
    hipStream_t s = resolve_stream(ctx, stream);
    return launch_router(ctx, s, d_w_r, d_bias, d_x, n_tokens, n_experts, hidden, k, renormalize, d_ids,
                         d_weights, nullptr, nullptr);
    OBJ_GUARD_END
}

extern "C" int32_t objeta_hip_router_softmax_exp_device(objeta_hip_context* ctx, objeta_hip_stream stream,
                                                        const float* d_x, float* d_y, uint64_t n) {
    OBJ_GUARD_BEGIN
    OBJ_TRY(check_ctx(ctx, "router_softmax_exp_device"));
    if (n == 0) return 0;
    if (!d_x || !d_y) OBJ_FAIL(kInvalidInput, "router_softmax_exp_device", "NULL device pointer");
    if (n > (uint64_t(1) << 32)) OBJ_FAIL(kInvalidInput, "router_softmax_exp_device", "n exceeds 2^32");
    OBJ_HIP(hipSetDevice(ctx->device), "hipSetDevice");
    hipStream_t s = resolve_stream(ctx, stream);
    hipLaunchKernelGGL(softmax_exp_kernel, dim3(static_cast<uint32_t>((n + 255) / 256)), dim3(256), 0, s, d_x, d_y, n);
    OBJ_HIP(hipGetLastError(), "launch softmax exp");
    return 0;
    OBJ_GUARD_END
}
