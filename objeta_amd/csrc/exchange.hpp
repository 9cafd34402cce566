// exchange.hpp — hand-offs between the workgroups of one launch.
//
// Small intermediate vectors (logits, activations, hidden states) pass between
// workgroups as 64-bit words {value bits, epoch}: the producer publishes each word
// with one agent-scope atomic store, a consumer polls with agent-scope atomic loads
// until every word it needs carries the current epoch. Value and epoch travel
// together, so no fences are needed, and words left by earlier launches are
// recognised by their older epoch. Every wait is bounded: a timeout sets bit 2 of
// the device error word and returns, so a grid always drains.
#pragma once

#include "device_common.hpp"
#include "gemv_stream.hpp"
#include "router_math.hpp"

namespace objeta {
namespace xchg {

using namespace dev;
using rmath::tag;

constexpr uint32_t kWaitLimit = 1u << 18;  // polls per gather (a fraction of a second)

__device__ __forceinline__ uint64_t load_word(const uint64_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_word(uint64_t* p, float v, uint32_t epoch) {
    __hip_atomic_store(p, tag(v, epoch), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float word_value(uint64_t w) { return __builtin_bit_cast(float, static_cast<uint32_t>(w)); }

// Waits cheaply until a sample of the words is current: wave 0 polls 64 words
// spread evenly over [p, p+n) (one per lane, so one per producer region) with
// back-off, while the other waves wait at the barrier. The full gather that
// follows verifies every word; the sample only keeps hundreds of workgroups from
// re-reading whole buffers while the producers are still working.
__device__ void wait_sample(const uint64_t* __restrict__ p, uint32_t n, uint32_t epoch, uint32_t* err) {
    if (threadIdx.x < 64) {
        const uint32_t i = static_cast<uint32_t>((static_cast<uint64_t>(threadIdx.x) * n) / 64u + (n / 64u) - (n >= 64u ? 1u : 0u));
        const uint32_t ic = i < n ? i : n - 1;
        bool done = false;
        for (uint32_t spin = 0; spin < kWaitLimit; ++spin) {
            if (!done) done = static_cast<uint32_t>(load_word(p + ic) >> 32) == epoch;
            if (__all(done)) break;
            if (spin == 1 && (__hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) & 4u)) break;
            if (spin < 16) __builtin_amdgcn_s_sleep(1);
            else __builtin_amdgcn_s_sleep(4);
        }
    }
    __syncthreads();
}

// Block-wide gather of n words that must carry `epoch`; sink(i, value) is called
// once per word when it is seen current. Each thread issues its loads in batches of
// kGatherBatch before it waits for any of them (one memory latency per batch, not
// per word), and remembers which of its words are still pending so that later
// rounds re-check only those. Segments of 32 words per thread keep the pending set
// in one 32-bit mask.
//
// SHARED: the first round uses ordinary (L2-cached) loads. Hundreds of workgroups
// gather the same vector, and the 32 CUs of an XCD then share one L2 copy instead
// of each fetching every word across the fabric. A line cached before its
// producer wrote it shows an older epoch; those words are re-read with agent-scope
// loads, which bypass the caches.
constexpr int kGatherBatch = 16;
template <bool SHARED, class Sink>
__device__ void gather(const uint64_t* __restrict__ p, uint32_t n, uint32_t epoch, uint32_t* err, int* s_flag,
                       Sink sink) {
    wait_sample(p, n, epoch, err);
    constexpr uint32_t kSeg = 32u * kThreads;
    for (uint32_t s0 = 0; s0 < n; s0 += kSeg) {
        const uint32_t ns = n - s0 < kSeg ? n - s0 : kSeg;
        const uint32_t per = (ns + kThreads - 1) / kThreads;  // <= 32
        uint32_t mask = 0;
        for (uint32_t q = 0; q < per; ++q)
            if (threadIdx.x + q * kThreads < ns) mask |= 1u << q;
        for (uint32_t spin = 0;; ++spin) {
            // after one timed-out wait every later wait gives up at once, so the grid drains
            if (spin == 1 && (__hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) & 4u)) return;
            for (uint32_t q0 = 0; q0 < per; q0 += kGatherBatch) {
                if (((mask >> q0) & ((1u << kGatherBatch) - 1u)) == 0) continue;
                uint64_t w[kGatherBatch];
#pragma unroll
                for (int j = 0; j < kGatherBatch; ++j) {
                    const uint32_t i = threadIdx.x + (q0 + static_cast<uint32_t>(j)) * kThreads;
                    const uint64_t* wp = p + s0 + (i < ns ? i : ns - 1);
                    w[j] = (SHARED && spin == 0) ? *as_global(wp) : load_word(wp);
                }
#pragma unroll
                for (int j = 0; j < kGatherBatch; ++j) {
                    const uint32_t q = q0 + static_cast<uint32_t>(j);
                    if (q < 32 && ((mask >> q) & 1u) && static_cast<uint32_t>(w[j] >> 32) == epoch) {
                        sink(s0 + threadIdx.x + q * kThreads, word_value(w[j]));
                        mask &= ~(1u << q);
                    }
                }
            }
            if (threadIdx.x == 0) *s_flag = 0;
            __syncthreads();
            if (mask) *s_flag = 1;
            __syncthreads();
            const int pending = *s_flag;
            __syncthreads();
            if (!pending) break;
            if (spin >= kWaitLimit) {
                if (threadIdx.x == 0) atomicOr(err, 4u);
                return;
            }
            __builtin_amdgcn_s_sleep(8);
        }
    }
}

__device__ __forceinline__ float silu_mul_s(float g, float u, float limit) {
    if (limit > 0.0f) {
        u = fminf(limit, fmaxf(-limit, u));
        g = fminf(limit, g);
    }
    return (g / (1.0f + expf(-g))) * u;
}

// Sums of N values over aligned groups of lpr lanes (a power of two): an xor
// butterfly, the N values interleaved step by step so that their shuffles overlap.
// Every lane of a group ends with the group's sums.
template <int N>
__device__ __forceinline__ void reduce_groups(float (&v)[N], uint32_t lpr) {
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        if (static_cast<uint32_t>(off) < lpr) {
#pragma unroll
            for (int i = 0; i < N; ++i) v[i] += __shfl_xor(v[i], off, 64);
        }
    }
}

// ------------------------------------------------- hand-offs inside one XCD
// Words exchanged among the workgroups of one XCD (the producers and consumers of
// a word share an XCD, so its pollers come from 32 CUs, not from the whole
// device). Both sides use relaxed agent-scope atomics, like the cross-XCD words:
// a workgroup-scope load may be served by the CU's L1 and never see the update.
// Atomics (not volatile accesses, which the compiler serialises, waiting for each
// to complete) let a thread keep a batch of loads in flight.
__device__ __forceinline__ void l1_invalidate() { asm volatile("buffer_inv sc0" ::: "memory"); }
__device__ __forceinline__ uint64_t load_l2(const uint64_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_l2(uint64_t* p, float v, uint32_t epoch) {
    __hip_atomic_store(p, tag(v, epoch), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Block-wide gather of n words written on this XCD that must carry `epoch`;
// sink(i, value) once per word. Thread 0 first polls the last word, then every
// thread loads its words (up to 32 per thread) each round, re-reading only the
// ones still stale. Bounded like gather().
template <class Sink>
__device__ void gather_l2(const uint64_t* __restrict__ p, uint32_t n, uint32_t epoch, uint32_t* err, int* s_flag,
                          Sink sink) {
    if (threadIdx.x == 0) {
        for (uint32_t spin = 0; spin < kWaitLimit; ++spin) {
            l1_invalidate();
            if (static_cast<uint32_t>(load_l2(p + n - 1) >> 32) == epoch) break;
            if (spin == 1 && (__hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) & 4u)) break;
            __builtin_amdgcn_s_sleep(1);
        }
    }
    __syncthreads();
    const uint32_t per = (n + kThreads - 1) / kThreads;  // <= 32
    uint32_t mask = 0;
    for (uint32_t q = 0; q < per; ++q)
        if (threadIdx.x + q * kThreads < n) mask |= 1u << q;
    for (uint32_t spin = 0;; ++spin) {
        if (spin == 1 && (__hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) & 4u)) return;
        l1_invalidate();
        for (uint32_t q0 = 0; q0 < per; q0 += kGatherBatch) {
            if (((mask >> q0) & ((1u << kGatherBatch) - 1u)) == 0) continue;
            uint64_t w[kGatherBatch];
#pragma unroll
            for (int j = 0; j < kGatherBatch; ++j) {
                const uint32_t i = threadIdx.x + (q0 + static_cast<uint32_t>(j)) * kThreads;
                w[j] = load_l2(p + (i < n ? i : n - 1));
            }
#pragma unroll
            for (int j = 0; j < kGatherBatch; ++j) {
                const uint32_t q = q0 + static_cast<uint32_t>(j);
                if (q < 32 && ((mask >> q) & 1u) && static_cast<uint32_t>(w[j] >> 32) == epoch) {
                    sink(threadIdx.x + q * kThreads, word_value(w[j]));
                    mask &= ~(1u << q);
                }
            }
        }
        if (threadIdx.x == 0) *s_flag = 0;
        __syncthreads();
        if (mask) *s_flag = 1;
        __syncthreads();
        const int pending = *s_flag;
        __syncthreads();
        if (!pending) break;
        if (spin >= kWaitLimit) {
            if (threadIdx.x == 0) atomicOr(err, 4u);
            return;
        }
        __builtin_amdgcn_s_sleep(1);
    }
}

}  // namespace xchg
}  // namespace objeta
