// router_math.hpp — the router's arithmetic (exact logit sums with error bounds,
// the reference's softmax and stable top-k).
//
// Reference semantics: cpu_router (crates/objeta-cuda/src/bin/
// deepseek_single_layer_moe.rs:687-743) takes each logit as a sequential fp32 sum
// of rounded products, a softmax over all experts, and a stable descending sort
// (ties keep the lower expert id); the k selected probabilities are renormalised
// (crates/objeta-qwen36-executor/src/moe_dispatch.rs:403-435). The device takes the
// exact sum S of the same rounded products (in double) with a rigorous bound on
// |S - sequential fp32 sum| (Higham: u * sum_k |S_k| / (1 - n u) over the
// sequential prefix sums S_k); decisions closer than the bounds are recomputed in
// the reference's order by the caller.
#pragma once

#include "device_common.hpp"

namespace objeta {
namespace rmath {

constexpr int kPadX = 68;  // floats per 64-activation slot of the padded LDS layout

constexpr int kRThreads = 256;
constexpr int kRWaves = kRThreads / 64;
constexpr int kMaxExperts = 1024;
constexpr int kMaxTopK = 32;
constexpr int kChunkBatch = 8;  // 256-element chunks loaded per batch (8 float4 per lane)

// The reference's softmax calls Rust's f32::exp, which is glibc's expf on Linux.
// glibc (2.28 and later) evaluates it with the method of Arm's optimized-routines
// (Szabolcs Nagy, 2017): in double, x * 32/ln2 = k + r with k the nearest integer
// (through the 1.5 * 2^52 shift), 2^(k/32) from a table of 2^(i/32), 2^(r/32)
// from a degree-3 polynomial, one final rounding to float; on x86-64 with FMA it
// runs the build with every product fused into the add that consumes it. This is
// that form, operation for operation (fused where glibc fuses, separate products
// elsewhere), so the device gets glibc's float on every argument; the same
// restatement in the oracle agrees with glibc on all of [-110, 0] (exhaustively)
// and double exp rounded once to float differs from it on 97,052 of those
// arguments. Table entry i: the correctly rounded double 2^(i/32) minus i << 47.
// (a file-scope table: a function-local one indexed per lane is placed in private
// scratch memory in some kernels)
static __device__ const uint64_t kExpTab[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull};

// The table is read per lane at an index that depends on x; a caller on a latency
// path passes a copy staged in LDS (tab), others read the file-scope table.
template <class Tab>
__device__ __forceinline__ float expf_glibc_tab(float x, Tab tab) {
    const uint32_t ux = __builtin_bit_cast(uint32_t, x);
    const uint32_t abstop = (ux >> 20) & 0x7ffu;
    if (abstop >= 0x42bu) {  // |x| >= 88, inf or nan
        if (ux == 0xff800000u) return 0.0f;
        if (abstop >= 0x7f8u) return x + x;
        if (x > 0x1.62e42ep6f) return __builtin_inff();
        if (x < -0x1.9fe368p6f) return 0.0f;
    }
    constexpr double kInvLn2N = 0x1.71547652b82fep+0 * 32, kShift = 0x1.8p+52;
    constexpr double kC0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32, kC1 = 0x1.ebfce50fac4f3p-3 / 32 / 32,
                     kC2 = 0x1.62e42ff0c52d6p-1 / 32;
    const double xd = static_cast<double>(x);
    double kd = __builtin_fma(kInvLn2N, xd, kShift);
    const uint64_t ki = __builtin_bit_cast(uint64_t, kd);
    kd = __dsub_rn(kd, kShift);
    const double r = __builtin_fma(kInvLn2N, xd, -kd);
    const double sc = __builtin_bit_cast(double, tab[ki % 32] + (ki << 47));
    const double z = __builtin_fma(kC0, r, kC1);
    const double r2 = __dmul_rn(r, r);
    double y = __builtin_fma(kC2, r, 1.0);
    y = __builtin_fma(z, r2, y);
    return static_cast<float>(__dmul_rn(y, sc));
}

__device__ __forceinline__ float expf_glibc(float x) { return expf_glibc_tab(x, kExpTab); }

typedef const __attribute__((address_space(3))) uint64_t* LdsTab;

// Wave-wide double scans through DPP row shifts and lane reads, not shuffles: a
// shuffle goes through the LDS crossbar (over 100 cycles a step, 12 dependent
// steps per scan), a DPP move is an ordinary VALU operation.
template <int CTRL>
__device__ __forceinline__ double dpp_d(double v) {  // lanes without a source read 0
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = static_cast<uint32_t>(
        __builtin_amdgcn_update_dpp(0, static_cast<int>(static_cast<uint32_t>(u)), CTRL, 0xF, 0xF, true));
    const uint32_t hi = static_cast<uint32_t>(
        __builtin_amdgcn_update_dpp(0, static_cast<int>(static_cast<uint32_t>(u >> 32)), CTRL, 0xF, 0xF, true));
    return __builtin_bit_cast(double, (static_cast<uint64_t>(hi) << 32) | lo);
}
__device__ __forceinline__ double readlane_d(double v, int l) {
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(u)), l));
    const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(u >> 32)), l));
    return __builtin_bit_cast(double, (static_cast<uint64_t>(hi) << 32) | lo);
}
// Inclusive scan within each row of 16 lanes (row_shr 1, 2, 4, 8).
__device__ __forceinline__ double row_scan_d(double v) {
    v += dpp_d<0x111>(v);
    v += dpp_d<0x112>(v);
    v += dpp_d<0x114>(v);
    v += dpp_d<0x118>(v);
    return v;
}

// Sum over the wave, in every lane.
__device__ __forceinline__ double wave_sum_d(double v) {
    v = row_scan_d(v);
    return ((readlane_d(v, 15) + readlane_d(v, 31)) + readlane_d(v, 47)) + readlane_d(v, 63);
}

// Inclusive scan over the wave (in double): rows of 16 lanes, then the totals of
// the rows before.
__device__ __forceinline__ double wave_scan_d(double v, int lane) {
    v = row_scan_d(v);
    const double r0 = readlane_d(v, 15);
    const double r01 = r0 + readlane_d(v, 31);
    const double r012 = r01 + readlane_d(v, 47);
    const int row = lane >> 4;
    return row == 0 ? v : v + (row == 1 ? r0 : (row == 2 ? r01 : r012));
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
    total = readlane_d(incl, 63);
    abs_prefix = wave_sum_d(absacc);
}

__device__ __forceinline__ float block_max(float v, float* red) {
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float m = red[0];
    for (int w = 1; w < kRWaves; ++w) m = fmaxf(m, red[w]);
    __syncthreads();
    return m;
}

__device__ __forceinline__ float block_sum(float v, float* red) {
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
__device__ __forceinline__ void rank_select(const uint64_t* keys, int n, int want, int* rank, int* sel, int* part) {
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


// grid = (ceil(E / 4), T). Wave w of block b handles expert b*4 + w of token y and
// publishes {logit, epoch} and {bound, epoch}. Workgroup 0 of each token then
// waits for all experts' words of the current epoch (counters[t] + 1), selects, and
// advances counters[t]. No fences: the words are read and written with agent-scope
// atomics, and the epoch in each word makes stale words detectable.

// ------------------------------------------------------------ logits and bounds
// Rounds the exact sum to the logit the device reports and bounds its distance to
// the reference's sequential fp32 logit (+ bias), for one expert.
__device__ __forceinline__ void finish_logit(double total, double abs_prefix, float bias_e, uint32_t hidden,
                                             float& lhat, float& bnd) {
    const double b = static_cast<double>(bias_e);
    lhat = static_cast<float>(total + b);
    const double u = 5.9604644775390625e-08;  // 2^-24
    const double n = static_cast<double>(hidden);
    double bound = u * abs_prefix / (1.0 - n * u);
    bound += u * (fabs(total + b) + fabs(static_cast<double>(lhat))) * 1.0001;
    bound += 1e-12 * abs_prefix + 1e-30;
    bnd = static_cast<float>(bound * 1.0001);
}

// exact_logit_vec for a row whose 256-element chunks are already in registers
// (w[c] = elements 256c + 4 lane .. +3) and an activation vector staged in LDS in
// the padded pair layout (68 floats per 64). nchunks <= NB.
template <int NB>
__device__ __forceinline__ void exact_logit_regs(const float4 (&w)[NB], const float* __restrict__ x_lds,
                                                 uint32_t hidden, uint32_t lane, double& total, double& abs_prefix) {
    const uint32_t n4 = hidden >> 2;
    const uint32_t nchunks = (hidden + 255) >> 8;
    double p[NB][4], local[NB], incl[NB];
#pragma unroll
    for (int g = 0; g < NB; ++g) {
        const bool ok = static_cast<uint32_t>(g) < nchunks && g * 64 + lane < n4;
        const uint32_t idx = static_cast<uint32_t>(g) * 256 + 4 * lane;
        const float4 v = ok ? *reinterpret_cast<const float4*>(x_lds + (idx >> 6) * kPadX + (idx & 63))
                            : make_float4(0.f, 0.f, 0.f, 0.f);
        p[g][0] = ok ? static_cast<double>(__fmul_rn(w[g].x, v.x)) : 0.0;
        p[g][1] = ok ? static_cast<double>(__fmul_rn(w[g].y, v.y)) : 0.0;
        p[g][2] = ok ? static_cast<double>(__fmul_rn(w[g].z, v.z)) : 0.0;
        p[g][3] = ok ? static_cast<double>(__fmul_rn(w[g].w, v.w)) : 0.0;
        local[g] = ((p[g][0] + p[g][1]) + p[g][2]) + p[g][3];
        incl[g] = local[g];
    }
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
#pragma unroll
        for (int g = 0; g < NB; ++g) {
            const double o = __shfl_up(incl[g], off, 64);
            if (static_cast<int>(lane) >= off) incl[g] += o;
        }
    }
    double base = 0.0, absacc = 0.0;
#pragma unroll
    for (int g = 0; g < NB; ++g) {
        const bool ok = static_cast<uint32_t>(g) < nchunks && g * 64 + lane < n4;
        const double s0 = base + (incl[g] - local[g]) + p[g][0];
        const double s1 = s0 + p[g][1], s2 = s1 + p[g][2], s3 = s2 + p[g][3];
        if (ok) absacc += fabs(s0) + fabs(s1) + fabs(s2) + fabs(s3);
        base += __shfl(incl[g], 63, 64);
    }
    total = base;
    abs_prefix = wave_sum_d(absacc);
}


// exact_logit_regs with the products recomputed in the second pass instead of
// kept: two arrays of NB doubles live instead of six, for kernels that hold other
// state in registers.
template <int NB>
__device__ __forceinline__ void exact_logit_regs_lean(const float4 (&w)[NB], const float* __restrict__ x_lds,
                                                      uint32_t hidden, uint32_t lane, double& total,
                                                      double& abs_prefix) {
    const uint32_t n4 = hidden >> 2;
    const uint32_t nchunks = (hidden + 255) >> 8;
    double local[NB], incl[NB];
    auto xat = [&](int g) {
        const uint32_t idx = static_cast<uint32_t>(g) * 256 + 4 * lane;
        return *reinterpret_cast<const float4*>(x_lds + (idx >> 6) * kPadX + (idx & 63));
    };
#pragma unroll
    for (int g = 0; g < NB; ++g) {
        const bool ok = static_cast<uint32_t>(g) < nchunks && g * 64 + lane < n4;
        double l = 0.0;
        if (ok) {
            const float4 v = xat(g);
            l = ((static_cast<double>(__fmul_rn(w[g].x, v.x)) + static_cast<double>(__fmul_rn(w[g].y, v.y))) +
                 static_cast<double>(__fmul_rn(w[g].z, v.z))) +
                static_cast<double>(__fmul_rn(w[g].w, v.w));
        }
        local[g] = l;
        incl[g] = l;
    }
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
#pragma unroll
        for (int g = 0; g < NB; ++g) {
            const double o = __shfl_up(incl[g], off, 64);
            if (static_cast<int>(lane) >= off) incl[g] += o;
        }
    }
    double base = 0.0, absacc = 0.0;
#pragma unroll
    for (int g = 0; g < NB; ++g) {
        const bool ok = static_cast<uint32_t>(g) < nchunks && g * 64 + lane < n4;
        if (ok) {
            const float4 v = xat(g);
            const double s0 = base + (incl[g] - local[g]) + static_cast<double>(__fmul_rn(w[g].x, v.x));
            const double s1 = s0 + static_cast<double>(__fmul_rn(w[g].y, v.y));
            const double s2 = s1 + static_cast<double>(__fmul_rn(w[g].z, v.z));
            const double s3 = s2 + static_cast<double>(__fmul_rn(w[g].w, v.w));
            absacc += fabs(s0) + fabs(s1) + fabs(s2) + fabs(s3);
        }
        base += __shfl(incl[g], 63, 64);
    }
    total = base;
    abs_prefix = wave_sum_d(absacc);
}

// The exact sum and a bound on sum_h |S_h| for a row held lane-contiguously: lane
// l owns elements [l*4*n4, (l+1)*4*n4) as w[0..n4) (float4s) against x staged in
// LDS in the padded pair layout (4*n4 divides 64). The lane's range is cut into 4
// sub-blocks of NB/4 float4s, each running its own prefix sums s_i and sum |s_i|
// (four independent dependency chains); one wave scan gives every sub-block's
// offset T, and sum_i |T + s_i| <= n_b |T| + sum_i |s_i| bounds its share of
// sum_h |S_h|. The bound is at most twice the exact one and needs no scans per
// element.
template <int NB>
__device__ __forceinline__ void exact_logit_lanes(const float4 (&w)[NB], const float* __restrict__ x_lds,
                                                  uint32_t n4, uint32_t lane, double& total, double& abs_bound) {
    static_assert(NB % 4 == 0, "four sub-blocks per lane");
    constexpr int kSub = NB / 4;  // float4 per sub-block
    double s[4] = {0.0, 0.0, 0.0, 0.0}, a[4] = {0.0, 0.0, 0.0, 0.0};
    const uint32_t base = lane * n4 * 4;
#pragma unroll
    for (int g = 0; g < NB; ++g) {
        const int sb = g / kSub;
        if (static_cast<uint32_t>(g) < n4) {
            const uint32_t h = base + 4u * static_cast<uint32_t>(g);
            const float4 v = *reinterpret_cast<const float4*>(x_lds + (h >> 6) * kPadX + (h & 63));
            s[sb] += static_cast<double>(__fmul_rn(w[g].x, v.x));
            a[sb] += fabs(s[sb]);
            s[sb] += static_cast<double>(__fmul_rn(w[g].y, v.y));
            a[sb] += fabs(s[sb]);
            s[sb] += static_cast<double>(__fmul_rn(w[g].z, v.z));
            a[sb] += fabs(s[sb]);
            s[sb] += static_cast<double>(__fmul_rn(w[g].w, v.w));
            a[sb] += fabs(s[sb]);
        }
    }
    const double lane_sum = ((s[0] + s[1]) + s[2]) + s[3];
    const double incl = wave_scan_d(lane_sum, static_cast<int>(lane));
    // the lanes before (within a double rounding, which the bound's margin covers)
    double t = lane == 0 ? 0.0 : incl - lane_sum;
    double b = 0.0;
#pragma unroll
    for (int sb = 0; sb < 4; ++sb) {
        const int lo = sb * kSub;
        const int cnt = static_cast<int>(n4) - lo < 0 ? 0 : (static_cast<int>(n4) - lo > kSub ? kSub : static_cast<int>(n4) - lo);
        b += static_cast<double>(4 * cnt) * fabs(t) + a[sb];
        t += s[sb];
    }
    total = readlane_d(incl, 63);
    abs_bound = wave_sum_d(b);
}

// exact_logit_lanes for a row split over the four waves of a workgroup: wave w owns
// elements [w*H/4, (w+1)*H/4) and its lane l the 4*n4 elements from
// w*H/4 + 4*n4*l, held as w[0..n4) with the matching activations in xv[0..n4)
// (H = 1024*n4, n4 <= NB). Each lane runs one
// chain of prefix sums s_i and sum |s_i|; a wave scan gives the lane's offset
// inside its wave, the four wave totals meet in LDS (added in wave order), and a
// lane at global offset T adds 4*n4*|T| + sum |s_i| to the bound. Block-wide: every
// thread reaches both barriers. red: 8 doubles of LDS. total and abs_bound are
// returned in every thread.
template <int NB>
__device__ __forceinline__ void exact_logit_split(const float4 (&w)[NB], const float4 (&xv)[NB],
                                                  uint32_t n4, uint32_t lane, uint32_t wave, double* red,
                                                  double& total, double& abs_bound) {
    double s = 0.0, a = 0.0;
#pragma unroll
    for (int g = 0; g < NB; ++g) {
        if (static_cast<uint32_t>(g) < n4) {
            const float4 v = xv[g];
            s += static_cast<double>(__fmul_rn(w[g].x, v.x));
            a += fabs(s);
            s += static_cast<double>(__fmul_rn(w[g].y, v.y));
            a += fabs(s);
            s += static_cast<double>(__fmul_rn(w[g].z, v.z));
            a += fabs(s);
            s += static_cast<double>(__fmul_rn(w[g].w, v.w));
            a += fabs(s);
        }
    }
    const double incl = wave_scan_d(s, static_cast<int>(lane));
    // the lanes before (within a double rounding, which the bound's margin covers)
    const double t = lane == 0 ? 0.0 : incl - s;
    if (lane == 63) red[wave] = incl;
    __syncthreads();
    double tw = 0.0;
    for (uint32_t q = 0; q < wave; ++q) tw += red[q];
    total = ((red[0] + red[1]) + red[2]) + red[3];
    const double bw = wave_sum_d(static_cast<double>(4u * n4) * fabs(tw + t) + a);
    if (lane == 0) red[4 + wave] = bw;
    __syncthreads();
    abs_bound = ((red[4] + red[5]) + red[6]) + red[7];
}

// -------------------------------------------------------------------- selection
template <int MAXE>
struct SelectLds {
    float val[MAXE];
    float bnd[MAXE];
    int rank[MAXE];
    int part[kRThreads];
    __align__(16) uint64_t key[MAXE + 16];
    int sel[kMaxTopK + 1];
    float sv[kMaxTopK + 1];  // val and bnd of the ranked experts, in rank order
    float sb[kMaxTopK + 1];
    float red[kRWaves];
    float e[kMaxTopK];
    int flag;
    int need[MAXE];
    int nlist[64];
    int ncount;
    uint64_t exptab[32];  // kExpTab staged by the selecting workgroup (stage_exptab)
};

// Copies kExpTab into s.exptab; visible after the caller's next barrier.
template <int MAXE>
__device__ __forceinline__ void stage_exptab(SelectLds<MAXE>& s) {
    if (threadIdx.x < 32) s.exptab[threadIdx.x] = kExpTab[threadIdx.x];
}

template <int MAXE>
__device__ __forceinline__ LdsTab exptab_of(const SelectLds<MAXE>& s) {
    return (LdsTab)(s.exptab);
}

// With s.val / s.bnd holding all n logits and bounds (visible to the block):
// ranks the experts and checks that every decision the top-k depends on is
// separated beyond the bounds plus a margin that keeps the softmax probabilities
// distinct after rounding. When certain (returns true), s.sel[0..k) holds the ids
// and s.e[0..k) exp(l - max) (renormalize) or the probabilities. Block-wide; 256
// threads.
template <int MAXE>
__device__ bool select_certain(SelectLds<MAXE>& s, uint32_t n, uint32_t k, int renormalize) {
    const uint32_t tid = threadIdx.x;
    const uint32_t n16 = (n + 15) & ~15u;
    for (uint32_t j = tid; j < n16; j += kRThreads) s.key[j] = j < n ? order_key(s.val[j], j) : 0ull;
    if (tid == 0) s.flag = 0;
    __syncthreads();
    // rank of every key: P adjacent lanes share a key's comparisons and add their
    // counts with xor shuffles (no barrier); each lane reads its keys 16 at a time
    // with all reads in flight together. The ranked experts' values and bounds are
    // recorded in rank order for the checks below.
    const uint32_t want = k + 1 <= n ? k + 1 : n;
    uint32_t P = 1;
    while (P < 8 && P * 2 * n <= kRThreads) P *= 2;
    const uint32_t groups = n16 >> 4;
    const uint32_t per = (groups + P - 1) / P;
    for (uint32_t w = tid; w < n * P; w += kRThreads) {
        const uint32_t e = w / P, part = w % P;
        const uint64_t me = s.key[e];
        int r = 0;
        const uint32_t g0 = part * per, g1 = g0 + per < groups ? g0 + per : groups;
        for (uint32_t g = g0; g < g1; ++g) {
            ulonglong2 kv[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) kv[i] = *reinterpret_cast<const ulonglong2*>(&s.key[16 * g + 2 * i]);
#pragma unroll
            for (int i = 0; i < 8; ++i) r += (kv[i].x > me) + (kv[i].y > me);
        }
        for (uint32_t off = 1; off < P; off <<= 1) r += __shfl_xor(r, static_cast<int>(off), 64);
        if (part == 0) {
            s.rank[e] = r;
            if (r < static_cast<int>(want)) {
                s.sel[r] = static_cast<int>(e);
                s.sv[r] = s.val[e];
                s.sb[r] = s.bnd[e];
            }
        }
    }
    __syncthreads();
    const float mx = s.sv[0];
    const float lk = s.sv[k - 1];
    const float kmin_lo = lk - s.sb[k - 1];
    int unsure = 0;
    for (uint32_t j = tid; j < n; j += kRThreads) {
        if (s.rank[j] >= static_cast<int>(k)) {
            const float margin = 9.5367431640625e-07f * (1.0f + fabsf(s.val[j] - mx) + fabsf(lk - mx));
            if (!(s.val[j] + s.bnd[j] + margin < kmin_lo)) unsure = 1;
        }
    }
    if (tid + 1 < k) {
        const float va = s.sv[tid], vb = s.sv[tid + 1];
        const float margin = 9.5367431640625e-07f * (1.0f + fabsf(va - mx) + fabsf(vb - mx));
        if (!(va - s.sb[tid] > vb + s.sb[tid + 1] + margin)) unsure = 1;
    }
    // The margins assume normal probabilities: once exp(l_k - max) / sum can be
    // subnormal or zero, distinct logits can give equal probabilities, which the
    // reference's stable sort orders by index.
    if (tid == 0 && !(kmin_lo - mx > -80.0f)) unsure = 1;
    if (unsure) s.flag = 1;
    __syncthreads();
    if (s.flag) return false;
    float z = 1.0f;
    if (!renormalize) {
        float part = 0.0f;
        for (uint32_t j = tid; j < n; j += kRThreads) part += expf_glibc_tab(__fsub_rn(s.val[j], mx), exptab_of(s));
        z = block_sum(part, s.red);
    }
    if (tid < k) {
        const float ev = expf_glibc_tab(__fsub_rn(s.sv[tid], mx), exptab_of(s));
        s.e[tid] = renormalize ? ev : __fdiv_rn(ev, z);
    }
    __syncthreads();
    return true;
}

// Recomputes the logits of experts s.nlist[0..cnt) in the reference's order (each
// product rounded, then added in sequence, then the bias) into s.val, with bound 0.
// A sequential sum is one long dependency chain, so the candidates' chains run side
// by side: lane j of wave 0 adds candidate j's products while waves 1..3 stream the
// rows in chunks of C elements (coalesced loads), round the products and store them
// in LDS, one chunk ahead (double buffer; a candidate's chunk is C floats at stride
// C + 4, so the wave's 16-byte reads of 16 consecutive lanes hit distinct banks).
// Up to 64 candidates per pass, fewer when the scratch (>= 40 floats) is small.
// Block-wide; 256 threads.
template <int MAXE, class XAt>
__device__ void refine_rows(SelectLds<MAXE>& s, const float* __restrict__ w_r, const float* __restrict__ bias,
                            XAt xat, uint32_t hidden, int cnt, float* scratch, uint32_t scratch_floats) {
    // every product and every add rounds on its own, as in the reference, also in
    // translation units built with contraction on: the operators are written in this
    // scope (a multiply and an add inlined from __fmul_rn / __fadd_rn could fuse)
#pragma clang fp contract(off)
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    uint32_t G = cnt < 64 ? static_cast<uint32_t>(cnt) : 64u;  // candidates per pass
    if (G > scratch_floats / 40u) G = scratch_floats / 40u;
    const uint32_t h16 = (hidden + 15u) & ~15u;
    for (uint32_t g0 = 0; g0 < static_cast<uint32_t>(cnt); g0 += G) {
        const uint32_t ng = static_cast<uint32_t>(cnt) - g0 < G ? static_cast<uint32_t>(cnt) - g0 : G;
        uint32_t C = (scratch_floats / (2u * ng) - 4u) & ~15u;
        if (C > h16) C = h16;
        const uint32_t S = C + 4u;
        const uint32_t nchunks = (hidden + C - 1u) / C;
        // waves 1..3: rounded products of chunk c into buffer c & 1 (16-byte row reads
        // where the rows are 16-byte aligned; C is a multiple of 16)
        const bool v4 = (hidden & 3u) == 0 && (reinterpret_cast<uintptr_t>(w_r) & 15u) == 0;
        typedef __attribute__((address_space(3))) float lds_float;
        auto fill = [&](uint32_t c) {
            lds_float* buf = (lds_float*)(scratch + (c & 1u) * ng * S);
            const uint32_t c0 = c * C;
            const uint32_t m = hidden - c0 < C ? hidden - c0 : C;
            if (v4) {
                const uint32_t C4 = C >> 2, m4 = m >> 2;
#pragma unroll 2
                for (uint32_t item = threadIdx.x - 64u; item < ng * C4; item += kRThreads - 64u) {
                    const uint32_t r = item / C4, i4 = item - r * C4;
                    if (i4 < m4) {
                        const uint32_t e = static_cast<uint32_t>(s.nlist[g0 + r]);
                        const uint32_t h = c0 + 4u * i4;
                        typedef float f32x4 __attribute__((ext_vector_type(4)));
                        const f32x4 w = *dev::as_global(reinterpret_cast<const f32x4*>(w_r + static_cast<size_t>(e) * hidden + h));
                        f32x4 p;
                        p[0] = w[0] * xat(h);
                        p[1] = w[1] * xat(h + 1u);
                        p[2] = w[2] * xat(h + 2u);
                        p[3] = w[3] * xat(h + 3u);
                        *(__attribute__((address_space(3))) f32x4*)(buf + r * S + 4u * i4) = p;
                    }
                }
            } else {
#pragma unroll 4
                for (uint32_t item = threadIdx.x - 64u; item < ng * C; item += kRThreads - 64u) {
                    const uint32_t r = item / C, i = item - r * C;
                    if (i < m) {
                        const uint32_t e = static_cast<uint32_t>(s.nlist[g0 + r]);
                        const float w = w_r[static_cast<size_t>(e) * hidden + c0 + i];
                        const float p = w * xat(c0 + i);
                        buf[r * S + i] = p;
                    }
                }
            }
        };
        if (wave != 0) fill(0);
        __syncthreads();
        float acc = 0.0f;
        for (uint32_t c = 0; c < nchunks; ++c) {
            if (wave != 0) {
                if (c + 1u < nchunks) fill(c + 1u);
            } else if (lane < ng) {
                // the scratch is LDS in every caller: reading it as such gives LDS loads
                // (a generic pointer would give flat loads, counted with the memory loads)
                typedef float f32x4 __attribute__((ext_vector_type(4)));
                typedef __attribute__((address_space(3))) const f32x4 lds_f4;
                const float* row = scratch + (c & 1u) * ng * S + lane * S;
                lds_f4* row4 = (lds_f4*)(row);
                const uint32_t m = hidden - c * C < C ? hidden - c * C : C;
                const uint32_t nb = m >> 4;  // blocks of 16 products
                // two register buffers: block j + 1 is read while block j is added (an
                // LDS read takes far longer than the four adds it feeds)
                f32x4 va[4], vb[4];
                auto add4 = [&](const f32x4 (&v)[4]) {
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        acc = acc + v[q][0];
                        acc = acc + v[q][1];
                        acc = acc + v[q][2];
                        acc = acc + v[q][3];
                    }
                };
                auto load4 = [&](f32x4 (&v)[4], uint32_t j) {
#pragma unroll
                    for (int q = 0; q < 4; ++q) v[q] = row4[4 * j + q];
                };
                // straight-line pairs (the last read of a pair re-reads a block in
                // range), so the wait before each add covers that block's reads only
                if (nb) load4(va, 0);
                uint32_t j = 0;
                for (; j + 2 <= nb; j += 2) {
                    load4(vb, j + 1);
                    add4(va);
                    load4(va, j + 2 < nb ? j + 2 : j + 1);
                    add4(vb);
                }
                if (j < nb) add4(va);
                const uint32_t m32 = nb << 4;
                for (uint32_t i = m32; i < m; ++i) acc = acc + row[i];
            }
            __syncthreads();
        }
        if (wave == 0 && lane < ng) {
            const uint32_t e = static_cast<uint32_t>(s.nlist[g0 + lane]);
            if (bias) acc = acc + bias[e];
            s.val[e] = acc;
            s.bnd[e] = 0.0f;
        }
    }
    __syncthreads();
}

// After select_certain failed: recomputes, in the reference's sequential order,
// only the logits of experts involved in an undecided comparison (a selected
// expert whose interval val +- (bnd + margin) overlaps another expert's), sets
// their bounds to zero and decides again. Usually a handful of experts instead of
// all n, recomputed side by side by refine_rows through `scratch` (LDS). Returns
// false when the selection is still not certain (or too many experts are
// involved); the caller then runs select_underflow or select_sequential. xat(h)
// returns x[h] (best from LDS). Block-wide; 256 threads.
constexpr int kMaxRefine = 64;
template <int MAXE, class XAt>
__device__ __noinline__ bool select_refine(SelectLds<MAXE>& s, const float* __restrict__ w_r, const float* __restrict__ bias,
                              XAt xat, uint32_t n, uint32_t hidden, uint32_t k, int renormalize, float* scratch,
                              uint32_t scratch_floats) {
    for (uint32_t j = threadIdx.x; j < n; j += kRThreads) s.need[j] = 0;
    if (threadIdx.x == 0) s.ncount = 0;
    __syncthreads();
    const float mx = s.val[s.sel[0]];
    for (uint32_t w = threadIdx.x; w < k * n; w += kRThreads) {
        const uint32_t b = w % n;
        const int a = s.sel[w / n];
        if (static_cast<int>(b) == a) continue;
        const float m = 9.5367431640625e-07f * (1.0f + fabsf(s.val[a] - mx) + fabsf(s.val[b] - mx));
        const bool apart = (s.val[a] - s.bnd[a] > s.val[b] + s.bnd[b] + m) || (s.val[b] - s.bnd[b] > s.val[a] + s.bnd[a] + m);
        if (!apart) {
            s.need[a] = 1;
            s.need[b] = 1;
        }
    }
    __syncthreads();
    for (uint32_t j = threadIdx.x; j < n; j += kRThreads) {
        if (s.need[j]) {
            const int slot = atomicAdd(&s.ncount, 1);
            if (slot < kMaxRefine) s.nlist[slot] = static_cast<int>(j);
        }
    }
    __syncthreads();
    const int cnt = s.ncount;
    if (cnt == 0 || cnt > kMaxRefine || scratch_floats < 40u) return false;
    refine_rows(s, w_r, bias, xat, hidden, cnt, scratch, scratch_floats);
    return select_certain(s, n, k, renormalize);
}

// The reference's order throughout (cpu_router): logits[e] = sum_h fl(W[e,h] * x[h])
// accumulated left to right in fp32 (+ bias); probs = exp(l - max) / sum with the
// sum taken in expert order; stable descending sort of the probs, with exp as
// glibc's expf (expf_glibc, bit-identical), so equal probabilities tie exactly where
// the reference's tie. Fills s.sel and s.e (the probabilities). xat(h) returns x[h].
// Block-wide; 256 threads.
// With s.val holding the logits the reference computes (or -inf where its exp
// is exactly 0): the reference's softmax in fp32 (glibc's expf, the sum in
// expert order, one division each) and its stable descending sort of the
// probabilities; the top k ids go to s.sel, their probabilities to s.e. Block-wide.
template <int MAXE>
__device__ void softmax_rank(SelectLds<MAXE>& s, uint32_t n, uint32_t k) {
    __shared__ float s_sum_exp;
    float mx = -INFINITY;
    for (uint32_t j = threadIdx.x; j < n; j += kRThreads) mx = fmaxf(mx, s.val[j]);
    mx = block_max(mx, s.red);
    for (uint32_t j = threadIdx.x; j < n; j += kRThreads)
        s.bnd[j] = expf_glibc_tab(__fsub_rn(s.val[j], mx), exptab_of(s));
    __syncthreads();
    if (threadIdx.x == 0) {
        float sum = 0.0f;
        for (uint32_t j = 0; j < n; ++j) sum = __fadd_rn(sum, s.bnd[j]);
        s_sum_exp = sum;
    }
    __syncthreads();
    for (uint32_t j = threadIdx.x; j < n; j += kRThreads) s.bnd[j] = __fdiv_rn(s.bnd[j], s_sum_exp);
    __syncthreads();
    for (uint32_t j = threadIdx.x; j < ((n + 7) & ~7u); j += kRThreads) s.key[j] = j < n ? order_key(s.bnd[j], j) : 0ull;
    __syncthreads();
    const uint32_t want = k + 1 <= n ? k + 1 : n;
    rank_select(s.key, static_cast<int>(n), static_cast<int>(want), s.rank, s.sel, s.part);
    __syncthreads();
    if (threadIdx.x < k) s.e[threadIdx.x] = s.bnd[s.sel[threadIdx.x]];
    __syncthreads();
}

template <int MAXE, class XAt>
__device__ __noinline__ void select_sequential(SelectLds<MAXE>& s, const float* __restrict__ w_r, const float* __restrict__ bias,
                                  XAt xat, uint32_t n, uint32_t hidden, uint32_t k) {
    for (uint32_t j = threadIdx.x; j < n; j += kRThreads) {
        // every product and every add rounds on its own, as in the reference
#pragma clang fp contract(off)
        const float* row = w_r + static_cast<size_t>(j) * hidden;
        float sacc = 0.0f;
        for (uint32_t h = 0; h < hidden; ++h) {
            const float p = row[h] * xat(h);
            sacc = sacc + p;
        }
        if (bias) sacc = sacc + bias[j];
        s.val[j] = sacc;
    }
    __syncthreads();
    softmax_rank(s, n, k);
}

// When the softmax cannot be ranked on logits alone (some selected probability may
// be subnormal or zero, where the reference's stable sort breaks equal
// probabilities by index): an expert whose logit upper bound lies more than 110
// below the lower bound of the largest logit has exp(l - max) < 2^-158 in double,
// which is 0 in fp32 in the reference too. Only the others need their logits in the
// reference's order; the rest enter the softmax as -inf (exactly 0). Returns false
// (nothing changed) when more than kMaxRefine experts remain.
template <int MAXE, class XAt>
__device__ __noinline__ bool select_underflow(SelectLds<MAXE>& s, const float* __restrict__ w_r,
                                              const float* __restrict__ bias, XAt xat, uint32_t n, uint32_t hidden,
                                              uint32_t k, float* scratch, uint32_t scratch_floats) {
    float lo = -INFINITY;
    for (uint32_t j = threadIdx.x; j < n; j += kRThreads) lo = fmaxf(lo, s.val[j] - s.bnd[j]);
    lo = block_max(lo, s.red);
    if (threadIdx.x == 0) s.ncount = 0;
    __syncthreads();
    const float cut = lo - 110.0f;
    for (uint32_t j = threadIdx.x; j < n; j += kRThreads) {
        if (s.val[j] + s.bnd[j] >= cut || !(s.val[j] == s.val[j])) {
            const int slot = atomicAdd(&s.ncount, 1);
            if (slot < kMaxRefine) s.nlist[slot] = static_cast<int>(j);
        }
    }
    __syncthreads();
    const int cnt = s.ncount;
    if (cnt == 0 || cnt > kMaxRefine || scratch_floats < 40u || !(cut > -INFINITY)) return false;
    for (uint32_t j = threadIdx.x; j < n; j += kRThreads) s.need[j] = 0;
    __syncthreads();
    for (int q = static_cast<int>(threadIdx.x); q < cnt; q += kRThreads) s.need[s.nlist[q]] = 1;
    __syncthreads();
    for (uint32_t j = threadIdx.x; j < n; j += kRThreads)
        if (!s.need[j]) s.val[j] = -INFINITY;
    __syncthreads();
    refine_rows(s, w_r, bias, xat, hidden, cnt, scratch, scratch_floats);
    softmax_rank(s, n, k);
    return true;
}

// The k selected weights in selection order: renormalised (p / sum of the selected
// p, summed in selection order) or as they are. Threads 0..63 write.
template <int MAXE>
__device__ __forceinline__ void write_selection(const SelectLds<MAXE>& s, uint32_t k, int renormalize,
                                                uint32_t* __restrict__ ids, float* __restrict__ weights) {
    if (threadIdx.x < 64) {
        float sel_sum = 0.0f;
        for (uint32_t r = 0; r < k; ++r) sel_sum = __fadd_rn(sel_sum, s.e[r]);
        // global (not generic) stores: a generic store could alias LDS, and every
        // later LDS read would then wait for it to complete
        auto* gi = (__attribute__((address_space(1))) uint32_t*)(ids);
        auto* gw = (__attribute__((address_space(1))) float*)(weights);
        for (uint32_t r = threadIdx.x; r < k; r += 64) {
            gi[r] = static_cast<uint32_t>(s.sel[r]);
            gw[r] = renormalize ? __fdiv_rn(s.e[r], sel_sum) : s.e[r];
        }
    }
}

}  // namespace rmath
}  // namespace objeta
