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
// The last workgroup of a token ranks the experts; if every decision the top-k
// depends on is separated by more than the bounds, the ids are provably those of
// the sequential sums. Otherwise it recomputes every logit in the reference's
// sequential order (one lane per expert) and ranks those exact values.
#include "device_common.hpp"
#include "host_common.hpp"
#include "kernels.hpp"

namespace objeta {
namespace {

constexpr int kRThreads = 256;
constexpr int kRWaves = kRThreads / 64;
constexpr int kMaxExperts = 1024;
constexpr int kMaxTopK = 32;
constexpr int kChunkBatch = 8;  // 256-element chunks loaded per batch (8 float4 per lane)

__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// Inclusive scan over the wave (Hillis-Steele, in double).
__device__ __forceinline__ double wave_scan_d(double v, int lane) {
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const double o = __shfl_up(v, off, 64);
        if (lane >= off) v += o;
    }
    return v;
}

// The exact sum S of the rounded products fl(row[h] * x[h]) (accumulated in
// double) and sum_h |S_h| over the sequential prefix sums S_h = sum_{h' <= h},
// the quantity that bounds the reference's sequential fp32 rounding error.
// Vector form: the row is read as 256-element chunks, lane l holding elements
// 4l..4l+3 of each chunk (coalesced float4 loads, 8 chunks in flight); the prefix
// of an element is (chunks before) + (lanes before, a wave scan) + (its lane's own).
__device__ __forceinline__ void exact_logit_vec(const float* __restrict__ row, const float* __restrict__ xt,
                                                uint32_t hidden, uint32_t lane, double& total, double& abs_prefix) {
    const uint32_t n4 = hidden >> 2;
    const uint32_t nchunks = (hidden + 255) >> 8;
    const float4* r4 = reinterpret_cast<const float4*>(row);
    const float4* x4 = reinterpret_cast<const float4*>(xt);
    double base = 0.0, absacc = 0.0;
    for (uint32_t c0 = 0; c0 < nchunks; c0 += kChunkBatch) {
        float4 w[kChunkBatch], v[kChunkBatch];
#pragma unroll
        for (int g = 0; g < kChunkBatch; ++g) {
            const uint32_t i = (c0 + g) * 64 + lane;
            const uint32_t ic = i < n4 ? i : n4 - 1;
            w[g] = r4[ic];
            v[g] = x4[ic];
        }
        // the batch's scans are independent: run them side by side
        double p[kChunkBatch][4], local[kChunkBatch], incl[kChunkBatch];
#pragma unroll
        for (int g = 0; g < kChunkBatch; ++g) {
            const bool ok = (c0 + g) * 64 + lane < n4;
            p[g][0] = ok ? static_cast<double>(__fmul_rn(w[g].x, v[g].x)) : 0.0;
            p[g][1] = ok ? static_cast<double>(__fmul_rn(w[g].y, v[g].y)) : 0.0;
            p[g][2] = ok ? static_cast<double>(__fmul_rn(w[g].z, v[g].z)) : 0.0;
            p[g][3] = ok ? static_cast<double>(__fmul_rn(w[g].w, v[g].w)) : 0.0;
            local[g] = ((p[g][0] + p[g][1]) + p[g][2]) + p[g][3];
            incl[g] = local[g];
        }
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
#pragma unroll
            for (int g = 0; g < kChunkBatch; ++g) {
                const double o = __shfl_up(incl[g], off, 64);
                if (static_cast<int>(lane) >= off) incl[g] += o;
            }
        }
#pragma unroll
        for (int g = 0; g < kChunkBatch; ++g) {
            const bool ok = (c0 + g) * 64 + lane < n4;
            const double s0 = base + (incl[g] - local[g]) + p[g][0];
            const double s1 = s0 + p[g][1], s2 = s1 + p[g][2], s3 = s2 + p[g][3];
            if (ok) absacc += fabs(s0) + fabs(s1) + fabs(s2) + fabs(s3);
            base += __shfl(incl[g], 63, 64);
        }
    }
    total = base;
    abs_prefix = wave_sum_d(absacc);
}

// Scalar form for any hidden and alignment: lane l owns the contiguous range
// [l*chunk, (l+1)*chunk) of the sequential order.
__device__ __forceinline__ void exact_logit_scalar(const float* __restrict__ row, const float* __restrict__ xt,
                                                   uint32_t hidden, uint32_t lane, double& total,
                                                   double& abs_prefix) {
    const uint32_t chunk = (hidden + 63) / 64;
    const uint32_t c0 = lane * chunk < hidden ? lane * chunk : hidden;
    const uint32_t c1 = c0 + chunk < hidden ? c0 + chunk : hidden;
    double local = 0.0;
    for (uint32_t h = c0; h < c1; ++h) local += static_cast<double>(__fmul_rn(row[h], xt[h]));
    const double incl = wave_scan_d(local, static_cast<int>(lane));
    double run = incl - local, absacc = 0.0;
    for (uint32_t h = c0; h < c1; ++h) {
        run += static_cast<double>(__fmul_rn(row[h], xt[h]));
        absacc += fabs(run);
    }
    total = __shfl(incl, 63, 64);
    abs_prefix = wave_sum_d(absacc);
}

__device__ float block_max(float v, float* red) {
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float m = red[0];
    for (int w = 1; w < kRWaves; ++w) m = fmaxf(m, red[w]);
    __syncthreads();
    return m;
}

__device__ float block_sum(float v, float* red) {
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float s = red[0];
    for (int w = 1; w < kRWaves; ++w) s += red[w];
    __syncthreads();
    return s;
}

// Order key of (value, index): a larger key means a larger value, or an equal
// value at a lower index, which is the order of the reference's stable descending
// sort. -0.0 is folded into +0.0 (they compare equal as floats).
__device__ __forceinline__ uint64_t order_key(float v, uint32_t index) {
    uint32_t u = __builtin_bit_cast(uint32_t, v + 0.0f);
    u ^= (u >> 31) ? 0xFFFFFFFFu : 0x80000000u;
    return (static_cast<uint64_t>(u) << 32) | (0xFFFFFFFFu - index);
}

// Rank of every value among n by key (keys padded with 0 to a multiple of 8). The
// ids of ranks < want go to sel[]. Each value's comparisons are split over up to 8
// threads (as many as 256 threads allow) whose partial counts meet in part[].
__device__ void rank_select(const uint64_t* keys, int n, int want, int* rank, int* sel, int* part) {
    const int n8 = (n + 7) >> 3;
    int parts = 1;
    while (parts < 8 && parts * 2 * n <= kRThreads) parts *= 2;
    const int per = (n8 + parts - 1) / parts;  // 8-key groups per part
    for (int w = threadIdx.x; w < n * parts; w += kRThreads) {
        const int e = w % n, p = w / n;
        const uint64_t me = keys[e];
        int r = 0;
        const int g1 = (p + 1) * per < n8 ? (p + 1) * per : n8;
        for (int g = p * per; g < g1; ++g) {
#pragma unroll
            for (int i = 0; i < 8; ++i) r += keys[8 * g + i] > me;
        }
        if (parts == 1) {
            rank[e] = r;
            if (r < want) sel[r] = e;
        } else {
            part[p * n + e] = r;
        }
    }
    if (parts > 1) {
        __syncthreads();
        for (int e = threadIdx.x; e < n; e += kRThreads) {
            int r = 0;
            for (int p = 0; p < parts; ++p) r += part[p * n + e];
            rank[e] = r;
            if (r < want) sel[r] = e;
        }
    }
}

// A 64-bit word {value bits, epoch}: one atomic store publishes both, so a reader
// that sees the current epoch also sees the value written with it.
__device__ __forceinline__ uint64_t tag(float v, uint32_t epoch) {
    return (static_cast<uint64_t>(epoch) << 32) | __builtin_bit_cast(uint32_t, v);
}

constexpr uint32_t kSpinLimit = 1u << 20;  // bounded waits (about a second), then the error word

// grid = (ceil(E / 4), T). Wave w of block b handles expert b*4 + w of token y and
// publishes {logit, epoch} and {bound, epoch}. Workgroup 0 of each token then
// waits for all experts' words of the current epoch (counters[t] + 1), selects, and
// advances counters[t]. No fences: the words are read and written with agent-scope
// atomics, and the epoch in each word makes stale words detectable.
template <bool VEC>
__global__ __launch_bounds__(kRThreads) void router_kernel(
    const float* __restrict__ w_r, const float* __restrict__ bias, const float* __restrict__ x,
    uint32_t n_experts, uint32_t hidden, uint32_t k, int renormalize, uint32_t* __restrict__ ids,
    float* __restrict__ weights, uint64_t* __restrict__ ws, uint32_t* __restrict__ counters,
    uint32_t* __restrict__ err) {
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
        const float* row = w_r + static_cast<size_t>(e) * hidden;
        double total, abs_prefix;
        if constexpr (VEC) exact_logit_vec(row, xt, hidden, lane, total, abs_prefix);
        else exact_logit_scalar(row, xt, hidden, lane, total, abs_prefix);
        if (lane == 0) {
            const double b = bias ? static_cast<double>(bias[e]) : 0.0;
            const float lhat = static_cast<float>(total + b);
            const double u = 5.9604644775390625e-08;  // 2^-24
            const double n = static_cast<double>(hidden);
            double bound = u * abs_prefix / (1.0 - n * u);
            bound += u * (fabs(total + b) + fabs(static_cast<double>(lhat))) * 1.0001;
            bound += 1e-12 * abs_prefix + 1e-30;
            __hip_atomic_store(&ws_logit[e], tag(lhat, epoch), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(&ws_bound[e], tag(static_cast<float>(bound * 1.0001), epoch), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    if (blockIdx.x != 0) return;

    // ---- workgroup 0 of token t: gather, select
    __shared__ float s_val[kMaxExperts];
    __shared__ float s_bnd[kMaxExperts];
    __shared__ int s_rank[kMaxExperts];
    __shared__ int s_part[kRThreads];
    __shared__ __align__(16) uint64_t s_key[kMaxExperts + 8];
    __shared__ int s_sel[kMaxTopK + 1];
    __shared__ float s_red[kRWaves];
    __shared__ float s_e[kMaxTopK];
    __shared__ int s_pending, s_uncertain;
    if (threadIdx.x == 0) s_uncertain = 0;
    for (uint32_t spin = 0;; ++spin) {
        if (threadIdx.x == 0) s_pending = 0;
        __syncthreads();
        int pending = 0;
        for (uint32_t j = threadIdx.x; j < n_experts; j += kRThreads) {
            const uint64_t a = __hip_atomic_load(&ws_logit[j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const uint64_t b = __hip_atomic_load(&ws_bound[j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (static_cast<uint32_t>(a >> 32) != epoch || static_cast<uint32_t>(b >> 32) != epoch) pending = 1;
            s_val[j] = __builtin_bit_cast(float, static_cast<uint32_t>(a));
            s_bnd[j] = __builtin_bit_cast(float, static_cast<uint32_t>(b));
        }
        if (pending) s_pending = 1;
        __syncthreads();
        if (!s_pending) break;
        if (spin >= kSpinLimit) {  // a producer never published: flag it and stop waiting
            if (threadIdx.x == 0) atomicOr(err, 2u);
            break;
        }
        __builtin_amdgcn_s_sleep(2);
    }
    for (uint32_t j = threadIdx.x; j < ((n_experts + 7) & ~7u); j += kRThreads)
        s_key[j] = j < n_experts ? order_key(s_val[j], j) : 0ull;
    __syncthreads();
    const uint32_t want = k + 1 <= n_experts ? k + 1 : n_experts;
    rank_select(s_key, static_cast<int>(n_experts), static_cast<int>(want), s_rank, s_sel, s_part);
    __syncthreads();

    // Certainty: consecutive selected logits must be separated beyond their bounds
    // plus a margin that keeps their softmax probabilities distinct after rounding,
    // and the k-th selected must beat every unselected expert likewise.
    float mx = s_val[s_sel[0]];
    {
        const float lk = s_val[s_sel[k - 1]];
        const float kmin_lo = lk - s_bnd[s_sel[k - 1]];
        int unsure = 0;
        for (uint32_t j = threadIdx.x; j < n_experts; j += kRThreads) {
            if (s_rank[j] >= static_cast<int>(k)) {
                const float margin = 9.5367431640625e-07f * (1.0f + fabsf(s_val[j] - mx) + fabsf(lk - mx));
                if (!(s_val[j] + s_bnd[j] + margin < kmin_lo)) unsure = 1;
            }
        }
        if (threadIdx.x + 1 < k) {
            const int a = s_sel[threadIdx.x], b = s_sel[threadIdx.x + 1];
            const float margin = 9.5367431640625e-07f * (1.0f + fabsf(s_val[a] - mx) + fabsf(s_val[b] - mx));
            if (!(s_val[a] - s_bnd[a] > s_val[b] + s_bnd[b] + margin)) unsure = 1;
        }
        if (unsure) s_uncertain = 1;
    }
    __syncthreads();

    __shared__ float s_sum_exp;
    const bool uncertain = s_uncertain != 0;
    if (uncertain) {
        // Reference order throughout (cpu_router): logits[e] = sum_h fl(W[e,h] * x[h])
        // accumulated left to right in fp32 (+ bias); probs = exp(l - max) / sum with
        // the sum taken in expert order; stable descending sort of the probs. exp is
        // evaluated in double and rounded once, which agrees with glibc's expf on all
        // but ~0.03% of arguments (only a probability tie could expose that).
        for (uint32_t j = threadIdx.x; j < n_experts; j += kRThreads) {
            // every product and every add rounds on its own, as in the reference
#pragma clang fp contract(off)
            const float* row = w_r + static_cast<size_t>(j) * hidden;
            float sacc = 0.0f;
            for (uint32_t h = 0; h < hidden; ++h) {
                const float p = row[h] * xt[h];
                sacc = sacc + p;
            }
            if (bias) sacc = sacc + bias[j];
            s_val[j] = sacc;
        }
        __syncthreads();
        mx = -INFINITY;
        for (uint32_t j = threadIdx.x; j < n_experts; j += kRThreads) mx = fmaxf(mx, s_val[j]);
        mx = block_max(mx, s_red);
        for (uint32_t j = threadIdx.x; j < n_experts; j += kRThreads)
            s_bnd[j] = static_cast<float>(exp(static_cast<double>(__fsub_rn(s_val[j], mx))));
        __syncthreads();
        if (threadIdx.x == 0) {
            float sum = 0.0f;
            for (uint32_t j = 0; j < n_experts; ++j) sum = __fadd_rn(sum, s_bnd[j]);
            s_sum_exp = sum;
        }
        __syncthreads();
        for (uint32_t j = threadIdx.x; j < n_experts; j += kRThreads) s_bnd[j] = __fdiv_rn(s_bnd[j], s_sum_exp);
        for (uint32_t j = threadIdx.x; j < ((n_experts + 7) & ~7u); j += kRThreads)
            s_key[j] = j < n_experts ? order_key(s_bnd[j], j) : 0ull;
        __syncthreads();
        rank_select(s_key, static_cast<int>(n_experts), static_cast<int>(want), s_rank, s_sel, s_part);
        __syncthreads();
        if (threadIdx.x < k) s_e[threadIdx.x] = s_bnd[s_sel[threadIdx.x]];
    } else {
        float z = 1.0f;
        if (!renormalize) {
            float part = 0.0f;
            for (uint32_t j = threadIdx.x; j < n_experts; j += kRThreads) part += expf(s_val[j] - mx);
            z = block_sum(part, s_red);
        }
        if (threadIdx.x < k) {
            const float ev = expf(__fsub_rn(s_val[s_sel[threadIdx.x]], mx));
            s_e[threadIdx.x] = renormalize ? ev : __fdiv_rn(ev, z);
        }
    }
    __syncthreads();

    // the k selected probabilities, renormalised in selection order
    if (threadIdx.x < 64) {
        float sel_sum = 0.0f;
        for (uint32_t r = 0; r < k; ++r) sel_sum = __fadd_rn(sel_sum, s_e[r]);
        for (uint32_t r = threadIdx.x; r < k; r += 64) {
            ids[static_cast<size_t>(t) * k + r] = static_cast<uint32_t>(s_sel[r]);
            weights[static_cast<size_t>(t) * k + r] = renormalize ? __fdiv_rn(s_e[r], sel_sum) : s_e[r];
        }
        if (threadIdx.x == 0) __hip_atomic_store(&counters[t], epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

}  // namespace

int32_t launch_router(objeta_hip_context* ctx, hipStream_t s, const float* w_r, const float* bias,
                      const float* x, uint64_t n_tokens, uint64_t n_experts, uint64_t hidden, uint64_t k,
                      int32_t renormalize, uint32_t* ids, float* weights, uint64_t* ws) {
    const char* action = "launch router_topk";
    if (n_experts == 0 || n_experts > kMaxExperts)
        OBJ_FAIL(kInvalidInput, action, strf("num_experts %llu must be in 1..=%d", (unsigned long long)n_experts, kMaxExperts));
    if (k == 0 || k > n_experts || k > kMaxTopK)
        OBJ_FAIL(kInvalidInput, action,
                 strf("top_k %llu must be in 1..=min(num_experts, %d)", (unsigned long long)k, kMaxTopK));
    if (hidden == 0 || hidden > (1u << 24)) OBJ_FAIL(kInvalidInput, action, "hidden must be in 1..=2^24");
    if (n_tokens == 0) return 0;
    if (n_tokens > ctx->counter_words) OBJ_FAIL(kInvalidInput, action, strf("n_tokens > %zu", ctx->counter_words));
    if (!w_r || !x || !ids || !weights) OBJ_FAIL(kInvalidInput, action, "NULL device pointer");
    const dim3 grid(static_cast<uint32_t>((n_experts + kRWaves - 1) / kRWaves), static_cast<uint32_t>(n_tokens));
    const bool vec = hidden % 4 == 0 && reinterpret_cast<uintptr_t>(w_r) % 16 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0;
    uint32_t* err = ctx->counters + ctx->counter_words;
    if (vec)
        hipLaunchKernelGGL(router_kernel<true>, grid, dim3(kRThreads), 0, s, w_r, bias, x,
                           static_cast<uint32_t>(n_experts), static_cast<uint32_t>(hidden), static_cast<uint32_t>(k),
                           renormalize, ids, weights, ws, ctx->counters, err);
    else
        hipLaunchKernelGGL(router_kernel<false>, grid, dim3(kRThreads), 0, s, w_r, bias, x,
                           static_cast<uint32_t>(n_experts), static_cast<uint32_t>(hidden), static_cast<uint32_t>(k),
                           renormalize, ids, weights, ws, ctx->counters, err);
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
    const size_t need = static_cast<size_t>(n_tokens) * kMaxExperts * 2 * sizeof(uint64_t);
    void* ws = nullptr;
    OBJ_TRY(ensure_workspace(ctx, s, kWsRouter, need, &ws));
    return launch_router(ctx, s, d_w_r, d_bias, d_x, n_tokens, n_experts, hidden, k, renormalize, d_ids,
                         d_weights, static_cast<uint64_t*>(ws));
    OBJ_GUARD_END
}
