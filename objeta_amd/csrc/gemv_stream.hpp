// gemv_stream.hpp — the streaming row-dot engine shared by the GEMV entry points
// and the MoE kernels.
//
// Work layout: a row is split into 64-weight "pairs" (two 32-weight blocks); a
// wave64 covers g = 64 / lpr rows with lpr lanes per row, lane lp owning pairs
// lp, lp + lpr, ... ("chunks"). A wave item is (row group, chunk): U row slots of
// g rows each at one chunk. Waves are persistent and walk their items in a
// grid-stride loop. The first item is requested before the workgroup stages its
// activations into LDS, so the two memory latencies overlap.
#pragma once

#include "device_common.hpp"
#include "quant_rules.hpp"

namespace objeta {
namespace dev {

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
constexpr int kPad = 68;       // floats per 64-activation pair slot in LDS (bank spread)
constexpr int kMaxStage = 16;  // float4 per thread staged at once (64 KB per workgroup)

// Rows of a block-quantized matrix (Q4_0 / Q5_0 / IQ3_0), row-major blocks.
template <int F>
struct QRows {
    static constexpr int kDw = Fmt<F>::kPairDw;
    static constexpr int kPairBytes = 2 * Fmt<F>::kBlockBytes;
    const uint8_t* __restrict__ q;
    size_t row_bytes;

    __device__ __forceinline__ const uint8_t* pair_ptr(uint32_t r, uint32_t p) const {
        return q + static_cast<size_t>(r) * row_bytes + static_cast<size_t>(p) * kPairBytes;
    }
    __device__ __forceinline__ void load(uint32_t r, uint32_t p, uint32_t (&d)[kDw]) const {
        load_dwords<kDw>(reinterpret_cast<const uint32_t*>(pair_ptr(r, p)), d);
    }
    template <int NT>
    __device__ __forceinline__ void dot(const uint32_t (&d)[kDw], const float* const (&xs)[NT],
                                        float (&acc)[NT]) const {
        pair_dot<F, NT>(d, xs, acc);
    }
    template <int NT>
    __device__ __forceinline__ void dot(const uint32_t (&d)[kDw], const float* const (&xs)[NT],
                                        float (&acc)[NT], const float* const (&xs_slow)[NT]) const {
        pair_dot<F, NT>(d, xs, acc, xs_slow);
    }
};

// Rows of a DeepSeek split FP4 matrix: nibbles [rows][cols/2], E8M0 [rows][cols/32].
struct Fp4Rows {
    static constexpr int kDw = 9;  // 8 nibble dwords + the pair's two scale bytes
    const uint8_t* __restrict__ w;
    const uint8_t* __restrict__ s;
    size_t wrow, srow;

    __device__ __forceinline__ void load(uint32_t r, uint32_t p, uint32_t (&d)[kDw]) const {
        uint32_t n[8];
        load_dwords<8>(reinterpret_cast<const uint32_t*>(w + static_cast<size_t>(r) * wrow + p * 32u), n);
#pragma unroll
        for (int i = 0; i < 8; ++i) d[i] = n[i];
        d[8] = *as_global(reinterpret_cast<const uint16_t*>(s + static_cast<size_t>(r) * srow + p * 2u));
    }
    template <int NT>
    __device__ __forceinline__ void dot(const uint32_t (&d)[kDw], const float* const (&xs)[NT],
                                        float (&acc)[NT]) const {
        dot<NT>(d, xs, acc, xs);
    }
    template <int NT>
    __device__ __forceinline__ void dot(const uint32_t (&d)[kDw], const float* const (&xs)[NT],
                                        float (&acc)[NT], const float* const (&xs_slow)[NT]) const {
#pragma unroll
        for (int blk = 0; blk < 2; ++blk) {
            const float scale = e8m0_to_f32((d[8] >> (8 * blk)) & 0xFFu);
            if (__builtin_isfinite(scale)) {
                float a[NT];
#pragma unroll
                for (int t = 0; t < NT; ++t) a[t] = 0.f;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    float4 xa[NT], xb[NT];
#pragma unroll
                    for (int t = 0; t < NT; ++t) {
                        xa[t] = *reinterpret_cast<const float4*>(xs[t] + blk * 32 + 8 * j);
                        xb[t] = *reinterpret_cast<const float4*>(xs[t] + blk * 32 + 8 * j + 4);
                    }
                    fp4_dot8<NT>(d[blk * 4 + j], xa, xb, a);
                }
#pragma unroll
                for (int t = 0; t < NT; ++t) acc[t] = __builtin_fmaf(scale, a[t], acc[t]);
            } else {
                // the reference's w = table[q] * scale per weight (deepseek.rs:866-918)
                for (int i = 0; i < 32; ++i) {
                    const uint32_t c = (d[blk * 4 + i / 8] >> (4 * (i & 7))) & 15u;
                    const float wv = f16_to_f32(((c & 7u) << 9) | ((c & 8u) << 12)) * 16384.0f * scale;
#pragma unroll
                    for (int t = 0; t < NT; ++t) acc[t] = __builtin_fmaf(wv, xs_slow[t][blk * 32 + i], acc[t]);
                }
            }
        }
    }
};

// Rows of an FP8 E4M3 matrix (the DeepSeek shared expert): bytes [rows][cols] and
// E8M0 scales on a 128 x 128 tile grid [ceil(rows/128)][ceil(cols/128)]
// (deepseek.rs:1630-1661); a 64-weight pair lies inside one tile. Bytes decode with
// the reference's f8e4m3_to_f32 (deepseek.rs:799-829). cols % 128 == 0.
struct Fp8Rows {
    static constexpr int kDw = 17;  // 16 weight dwords + the tile's scale byte
    const uint8_t* __restrict__ w;
    const uint8_t* __restrict__ s;
    size_t wrow;     // bytes per row (cols)
    uint32_t scols;  // scale tiles per row of tiles

    __device__ __forceinline__ void load(uint32_t r, uint32_t p, uint32_t (&d)[kDw]) const {
        uint32_t n[16];
        load_dwords<16>(reinterpret_cast<const uint32_t*>(w + static_cast<size_t>(r) * wrow + p * 64u), n);
#pragma unroll
        for (int i = 0; i < 16; ++i) d[i] = n[i];
        d[16] = *as_global(s + static_cast<size_t>(r >> 7) * scols + (p >> 1));
    }
    template <int NT>
    __device__ __forceinline__ void dot(const uint32_t (&d)[kDw], const float* const (&xs)[NT],
                                        float (&acc)[NT]) const {
        dot<NT>(d, xs, acc, xs);
    }
    template <int NT>
    __device__ __forceinline__ void dot(const uint32_t (&d)[kDw], const float* const (&xs)[NT],
                                        float (&acc)[NT], const float* const (&xs_slow)[NT]) const {
        const float scale = e8m0_to_f32(d[16] & 0xFFu);
        const bool finite = __builtin_isfinite(scale);
        float a[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) a[t] = 0.f;
#pragma unroll
        for (int q = 0; q < 16; ++q) {
            float wv[4];
            fp8x4_to_f32(d[q], wv);
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const float4 xv = *reinterpret_cast<const float4*>(xs[t] + 4 * q);
                if (finite) {
                    a[t] = __builtin_fmaf(wv[0], xv.x, a[t]);
                    a[t] = __builtin_fmaf(wv[1], xv.y, a[t]);
                    a[t] = __builtin_fmaf(wv[2], xv.z, a[t]);
                    a[t] = __builtin_fmaf(wv[3], xv.w, a[t]);
                } else {  // the reference's per-weight w * s (NaN / inf propagate as there)
                    acc[t] = __builtin_fmaf(wv[0] * scale, xs_slow[t][4 * q], acc[t]);
                    acc[t] = __builtin_fmaf(wv[1] * scale, xs_slow[t][4 * q + 1], acc[t]);
                    acc[t] = __builtin_fmaf(wv[2] * scale, xs_slow[t][4 * q + 2], acc[t]);
                    acc[t] = __builtin_fmaf(wv[3] * scale, xs_slow[t][4 * q + 3], acc[t]);
                }
            }
        }
        if (finite) {
#pragma unroll
            for (int t = 0; t < NT; ++t) acc[t] = __builtin_fmaf(scale, a[t], acc[t]);
        }
    }
};

// A row accessor over one expert tensor: pointer(s) from an expert table entry and
// the tensor's column count.
template <class R>
struct RowsOf;
template <int F>
struct RowsOf<QRows<F>> {
    static __device__ __forceinline__ QRows<F> make(const void* w, const void*, uint32_t cols) {
        return QRows<F>{static_cast<const uint8_t*>(w), static_cast<size_t>(cols >> 5) * Fmt<F>::kBlockBytes};
    }
};
template <>
struct RowsOf<Fp8Rows> {
    static __device__ __forceinline__ Fp8Rows make(const void* w, const void* s, uint32_t cols) {
        return Fp8Rows{static_cast<const uint8_t*>(w), static_cast<const uint8_t*>(s), cols, (cols + 127) >> 7};
    }
};
template <>
struct RowsOf<Fp4Rows> {
    static __device__ __forceinline__ Fp4Rows make(const void* w, const void* s, uint32_t cols) {
        return Fp4Rows{static_cast<const uint8_t*>(w), static_cast<const uint8_t*>(s), cols >> 1, cols >> 5};
    }
};

// Stages NT activation vectors of `cols` floats (cols % 64 == 0) into LDS, padded
// per 64, with every global load issued before the first LDS write. The LDS
// allocation must hold NT * pairs * kPad + 4 floats (a spare slot at the end).
template <int NT>
__device__ __forceinline__ void stage_x(float* __restrict__ lds, const float* __restrict__ x,
                                        uint32_t cols, uint32_t pairs) {
    const uint32_t n4 = NT * cols / 4;
    const uint32_t per_tok4 = cols / 4;
    constexpr int kBatch = 4;
    const float4* src = reinterpret_cast<const float4*>(x);
    for (uint32_t base = 0; base < n4; base += kBatch * kThreads) {
        // Branch-free loads (indices clamped in range) keep the memory counter exact,
        // so the weight bytes requested before the stage stay in flight.
        uint32_t ii[kBatch];
        float4 v[kBatch];
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
            ii[j] = base + threadIdx.x + j * kThreads;
            v[j] = src[ii[j] < n4 ? ii[j] : n4 - 1];
        }
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
            // out-of-range lanes write the spare slot just past the stage
            const uint32_t t = ii[j] / per_tok4;
            const uint32_t c = (ii[j] - t * per_tok4) * 4;
            const uint32_t off = ii[j] < n4 ? (t * pairs + (c >> 6)) * kPad + (c & 63) : NT * pairs * kPad;
            *reinterpret_cast<float4*>(lds + off) = v[j];
        }
    }
}

// Staging in two steps around the weight loads. Vector-memory loads complete in
// issue order, so a wait for activations requested after the weights also waits
// for the weights; requesting the activations first (stage_x_issue), then the
// weights, then writing the activations to LDS (stage_x_commit) waits for the
// activations only. Thread t holds float4s t, t + 256, ... of the NT vectors
// (NV per thread: NT * cols <= 1024 * NV).
template <int NV>
struct XRegs {
    float4 v[NV];
};

template <int NT, int NV>
__device__ __forceinline__ void stage_x_issue(const float* __restrict__ x, uint32_t cols, XRegs<NV>& r) {
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    const uint32_t n4 = NT * cols / 4;
    const gptr<f32x4> src = as_global(reinterpret_cast<const f32x4*>(x));
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const uint32_t i = threadIdx.x + static_cast<uint32_t>(j) * kThreads;
        if (i < n4) {
            const f32x4 v = src[i];
            r.v[j] = make_float4(v.x, v.y, v.z, v.w);
        }
    }
}

template <int NT, int NV>
__device__ __forceinline__ void stage_x_commit(float* __restrict__ lds, uint32_t cols, uint32_t pairs,
                                               const XRegs<NV>& r) {
    const uint32_t n4 = NT * cols / 4;
    const uint32_t per_tok4 = cols / 4;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const uint32_t i = threadIdx.x + static_cast<uint32_t>(j) * kThreads;
        if (i < n4) {
            const uint32_t t = i / per_tok4;
            const uint32_t c = (i - t * per_tok4) * 4;
            *reinterpret_cast<float4*>(lds + (t * pairs + (c >> 6)) * kPad + (c & 63)) = r.v[j];
        }
    }
}

// Segmented sum over the lpr lanes of a row; the total lands in the row's first lane.
__device__ __forceinline__ float row_reduce(float v, uint32_t lp, uint32_t lpr) {
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const float o = __shfl_down(v, off, 64);
        v += (lp + off < lpr) ? o : 0.0f;
    }
    return v;
}

// Per-lane coordinates of the streaming layout.
struct StreamLane {
    uint32_t lane, g, slot, lp, chunks;
    bool active;
    __device__ __forceinline__ StreamLane(uint32_t lpr, uint32_t pairs) {
        lane = threadIdx.x & 63;
        g = 64 / lpr;
        slot = lane / lpr;
        lp = lane - slot * lpr;
        active = slot < g;
        chunks = pairs / lpr;
    }
    // row of slot u in group grp
    __device__ __forceinline__ uint32_t row(uint32_t grp, int u, int U) const {
        return (grp * static_cast<uint32_t>(U) + static_cast<uint32_t>(u)) * g + slot;
    }
};

// Requests the weight bytes of item (grp, c). Branch-free: rows past the end (and
// lanes outside any row) read a clamped, valid row; their sums are never stored.
template <class R, int U>
__device__ __forceinline__ void load_item(const R& rm, const StreamLane& sl, uint32_t grp, uint32_t c,
                                          uint32_t rows, uint32_t lpr, uint32_t (&d)[U][R::kDw]) {
    const uint32_t p = sl.lp + c * lpr;
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const uint32_t r = sl.row(grp, u, U);
        rm.load(r < rows ? r : rows - 1, p, d[u]);
    }
}

// Advances (grp, c) to the wave's next item.
__device__ __forceinline__ void next_item(uint32_t& grp, uint32_t& c, uint32_t chunks, uint32_t nw) {
    if (++c == chunks) { c = 0; grp += nw; }
}

// y[t][r] = sum_c W[r][c] * x[t][c] for all rows, NT tokens. Waves are
// persistent and walk their items in a grid-stride loop; latency is hidden by
// the many waves resident per SIMD (each item's loads are issued as one batch),
// and the first item's loads overlap the activation stage.
template <class R, int NT, int U>
__global__ __launch_bounds__(kThreads) void gemv_stream(R rm, const float* __restrict__ x,
                                                        float* __restrict__ y, uint32_t rows,
                                                        uint32_t cols, uint32_t lpr, uint32_t n_groups) {
    extern __shared__ float lds[];
    const uint32_t pairs = cols >> 6;
    const StreamLane sl(lpr, pairs);
    const uint32_t nw = gridDim.x * kWaves;
    uint32_t grp = blockIdx.x * kWaves + (threadIdx.x >> 6);
    uint32_t c = 0;

    uint32_t cur[U][R::kDw];
    load_item<R, U>(rm, sl, grp, c, rows, lpr, cur);
    stage_x<NT>(lds, x, cols, pairs);
    __syncthreads();

    float acc[U][NT];
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[u][t] = 0.f;

    while (grp < n_groups) {
        const uint32_t p = sl.lp + c * lpr;
        const float* xs[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) xs[t] = lds + (t * pairs + p) * kPad;
#pragma unroll
        for (int u = 0; u < U; ++u) rm.template dot<NT>(cur[u], xs, acc[u]);
        const uint32_t g0 = grp;
        next_item(grp, c, sl.chunks, nw);
        if (c == 0) {  // that item closed its row group
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const uint32_t r = sl.row(g0, u, U);
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    const float v = row_reduce(acc[u][t], sl.lp, lpr);
                    if (sl.active && sl.lp == 0 && r < rows) y[static_cast<size_t>(t) * rows + r] = v;
                    acc[u][t] = 0.f;
                }
            }
        }
        if (grp < n_groups) load_item<R, U>(rm, sl, grp, c, rows, lpr, cur);
    }
}

// Lanes per row: the largest divisor of `pairs` in [16, 64] (pairs itself when
// pairs <= 64); 0 when none exists (then the generic kernel runs).
inline uint32_t pick_lpr(uint32_t pairs) {
    if (pairs <= 64) return pairs;
    for (uint32_t l = 64; l >= 16; --l)
        if (pairs % l == 0) return l;
    return 0;
}

}  // namespace dev
}  // namespace objeta
