// moe.hip — selected-expert MoE kernels for gfx950.
//
// Replaces the per-expert launch chain of execute_selected_moe_cuda
// (crates/objeta-cuda/src/moe.rs:587-652): gate GEMV, up GEMV, silu_mul, down
// GEMV and weighted_accum (kernels/moe.cu:2-34) become two launches for all
// tokens and all selected experts:
//
//   moe_gate_up   one workgroup per (token, slot) assignment and row block; every
//                 lane streams the same weight pair of the gate row and the up row,
//                 so after the row reduction one lane holds both dot products and
//                 writes silu(gate) * up. The token's activation vector is staged
//                 once per workgroup in LDS while the weight loads are in flight.
//   moe_down      one workgroup per (token, row block); wave w streams the down
//                 rows of slots [w*JW, w*JW + JW) against their activations
//                 (staged in LDS), the per-slot row sums meet in LDS and one lane
//                 per row adds them into the residual in slot order. There is one
//                 writer per output element, so no atomics and a fixed order.
//
// Both kernels are one-shot (every lane issues all of its weight loads before it
// touches LDS) rather than persistent: an MoE layer at batch 1 is a few MB per
// phase, so the whole phase is in flight at once.
#include "device_common.hpp"
#include "gemv_stream.hpp"
#include "host_common.hpp"
#include "kernels.hpp"
#include "quant_rules.hpp"
#include "router_math.hpp"
#include "swiglu.hpp"

namespace objeta {
namespace dev {


// Expert id of assignment a; ids == nullptr means the identity. Returns false
// (and raises the device error word) when the id is outside the table.
__device__ __forceinline__ bool expert_of(const uint32_t* __restrict__ ids, uint32_t a, uint32_t n_table,
                                          uint32_t* __restrict__ err, uint32_t& e) {
    e = ids ? ids[a] : a;
    if (e < n_table) return true;
    if ((threadIdx.x & 63) == 0) atomicOr(err, 1u);
    e = 0;
    return false;
}

// Wave-cooperative copy of `cols` floats (cols % 64 == 0) from global memory into
// an LDS slot padded to kPad floats per 64 (the layout pair_dot reads).
__device__ __forceinline__ void stage_vec_wave(float* __restrict__ dst, const float* __restrict__ src,
                                               uint32_t cols, uint32_t lane) {
    const float4* s4 = reinterpret_cast<const float4*>(src);
    const uint32_t n4 = cols >> 2;
    for (uint32_t i = lane; i < n4; i += 64) {
        const uint32_t c = i << 2;
        *reinterpret_cast<float4*>(dst + (c >> 6) * kPad + (c & 63)) = s4[i];
    }
}

// ------------------------------------------------------------------ gate/up
// grid.x = n_assign * blocks_per_assign, block = 256 (4 waves). A wave owns
// g = 64 / lpr row slots (lpr lanes each) times U rows; lane lp of a slot owns
// pairs lp + c * lpr, c < CH (pairs == CH * lpr). A token has kk slots: k routed
// ones (ids, sel and wts have stride k) and, when kk > k, the shared expert in
// slot k; assignment a = t * kk + j indexes the activations.
// The rows of block `bid` of that grid (the body of moe_gate_up_kernel).
template <class R, int U, int CH>
__device__ __forceinline__ void gate_up_block(
    uint32_t bid, const objeta_hip_expert_ptrs* __restrict__ table, uint32_t n_table, const uint32_t* __restrict__ ids,
    const float* __restrict__ x, float* __restrict__ act, uint32_t hidden, uint32_t inter, uint32_t k,
    uint32_t lpr, uint32_t blocks_per_assign, float limit, uint32_t* __restrict__ err,
    const objeta_hip_expert_ptrs* __restrict__ sel, uint32_t kk, const objeta_hip_expert_ptrs* __restrict__ shared,
    uint32_t official) {
    extern __shared__ float lds[];
    const uint32_t a = bid / blocks_per_assign;
    const uint32_t rb = bid - a * blocks_per_assign;
    const uint32_t t = a / kk;
    const uint32_t j = a - t * kk;
    const bool is_shared = j >= k;
    const uint32_t ar = t * k + (is_shared ? 0u : j);  // routed index into ids / sel
    // The expert id and table entry come through scalar loads, issued first; the
    // activations are requested while they are in flight and before the weights,
    // so that writing them to LDS waits for them alone.
    // sel: the router resolved the assignments to table entries (valid ids)
    uint32_t e = 0;
    const bool ok = (is_shared || sel) ? true : expert_of(ids, ar, n_table, err, e);
    constexpr int kXV = 8;
    const bool x_regs = hidden <= 4u * kXV * kThreads;
    XRegs<kXV> xr;
    if (x_regs) stage_x_issue<1, kXV>(x + static_cast<size_t>(t) * hidden, hidden, xr);
    const objeta_hip_expert_ptrs P = is_shared ? *shared : (sel ? sel[ar] : table[e]);
    const R gm = RowsOf<R>::make(P.gate, P.gate_scale, hidden);
    const R um = RowsOf<R>::make(P.up, P.up_scale, hidden);

    const uint32_t pairs = hidden >> 6;
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t gs = 64 / lpr, slot = lane / lpr, lp = lane - slot * lpr;
    const uint32_t row0 = (rb * kWaves + wave) * gs * U;

    uint32_t dg[U][CH][R::kDw], du[U][CH][R::kDw];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const uint32_t r = row0 + static_cast<uint32_t>(u) * gs + slot;
        const uint32_t rc = r < inter ? r : inter - 1;
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            const uint32_t p = lp + static_cast<uint32_t>(c) * lpr;
            gm.load(rc, p, dg[u][c]);
            um.load(rc, p, du[u][c]);
        }
    }
    if (x_regs) stage_x_commit<1, kXV>(lds, hidden, pairs, xr);
    else stage_x<1>(lds, x + static_cast<size_t>(t) * hidden, hidden, pairs);
    __syncthreads();

    // with one pair per lane, the lane's 64 activations are read from LDS once and
    // serve the gate and up rows of every row slot from registers
    float4 xr4[CH == 1 ? 16 : 1];
    if constexpr (CH == 1) {
        const float* xl = lds + lp * kPad;
#pragma unroll
        for (int q = 0; q < 16; ++q) xr4[q] = *reinterpret_cast<const float4*>(xl + 4 * q);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
        float ag[1] = {0.f}, au[1] = {0.f};
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            const float* xl[1] = {lds + (lp + static_cast<uint32_t>(c) * lpr) * kPad};
            if constexpr (CH == 1) {
                const float* xr[1] = {reinterpret_cast<const float*>(xr4)};
                gm.template dot<1>(dg[u][c], xr, ag, xl);
                um.template dot<1>(du[u][c], xr, au, xl);
            } else {
                gm.template dot<1>(dg[u][c], xl, ag);
                um.template dot<1>(du[u][c], xl, au);
            }
        }
        const float g = row_reduce(ag[0], lp, lpr);
        const float v = row_reduce(au[0], lp, lpr);
        const uint32_t r = row0 + static_cast<uint32_t>(u) * gs + slot;
        if (slot < gs && lp == 0 && r < inter)
            act[static_cast<size_t>(a) * inter + r] = ok ? swiglu(g, v, limit, official) : __builtin_nanf("");
    }
}

template <class R, int U, int CH>
__global__ __launch_bounds__(kThreads) void moe_gate_up_kernel(
    const objeta_hip_expert_ptrs* __restrict__ table, uint32_t n_table, const uint32_t* __restrict__ ids,
    const float* __restrict__ x, float* __restrict__ act, uint32_t hidden, uint32_t inter, uint32_t k,
    uint32_t lpr, uint32_t blocks_per_assign, float limit, uint32_t* __restrict__ err,
    const objeta_hip_expert_ptrs* __restrict__ sel, uint32_t kk, const objeta_hip_expert_ptrs* __restrict__ shared,
    uint32_t official) {
    gate_up_block<R, U, CH>(blockIdx.x, table, n_table, ids, x, act, hidden, inter, k, lpr, blocks_per_assign, limit, err,
                            sel, kk, shared, official);
}

// The official layer's routed gate/up (format R, kk = k) and its shared expert's
// (format RS, one slot per token, act rows act_sh) in one launch: blocks
// [0, nb_shared) are the shared expert's (dispatched first: its FP8 rows take the
// longest per block), the rest the routed assignments', so both stream together (in
// two launches the second waits for the first).
template <class R, int U, int CH, class RS, int US, int CHS>
__global__ __launch_bounds__(kThreads) void moe_gate_up_pair_kernel(
    const objeta_hip_expert_ptrs* __restrict__ table, uint32_t n_table, const uint32_t* __restrict__ ids,
    const float* __restrict__ x, float* __restrict__ act, float* __restrict__ act_sh, uint32_t hidden, uint32_t inter,
    uint32_t k, uint32_t lpr, uint32_t bpa_routed, uint32_t bpa_shared, uint32_t nb_shared, float limit,
    uint32_t* __restrict__ err, const objeta_hip_expert_ptrs* __restrict__ shared, uint32_t official) {
    if (blockIdx.x < nb_shared)
        gate_up_block<RS, US, CHS>(blockIdx.x, shared, 1, nullptr, x, act_sh, hidden, inter, 0, lpr, bpa_shared, limit,
                                   err, nullptr, 1, shared, official);
    else
        gate_up_block<R, U, CH>(blockIdx.x - nb_shared, table, n_table, ids, x, act, hidden, inter, k, lpr, bpa_routed,
                                limit, err, nullptr, k, nullptr, official);
}

// -------------------------------------------------------------------- down
// grid.x = n_tokens * blocks_per_token, block = ceil(kk / JW) waves. All waves of
// a block cover the same g * U output rows; wave w takes slots [w*JW, w*JW+JW).
// Slots j < k are routed (ids, sel, wts with stride k); slot k, when kk > k, is the
// shared expert with weight 1, combined last as the reference adds it after the
// routed sum. LDS: red [kk][g*U] row sums, then one padded activation slot per
// (wave, jj).
template <class R, int U, int CH, int JW>
__global__ __launch_bounds__(1024) void moe_down_kernel(
    const objeta_hip_expert_ptrs* __restrict__ table, uint32_t n_table, const uint32_t* __restrict__ ids,
    const float* __restrict__ wts, const float* __restrict__ act, const float* resid, float* out,
    uint32_t inter, uint32_t out_dim, uint32_t k, uint32_t lpr, uint32_t blocks_per_token,
    uint32_t* __restrict__ err, const objeta_hip_expert_ptrs* __restrict__ sel, uint32_t kk,
    const objeta_hip_expert_ptrs* __restrict__ shared) {
    extern __shared__ float lds[];
    // The dispatcher hands consecutive workgroups to the eight XCDs in turn, so the
    // workgroups b with one b % 8 share an XCD (and its L2). They take contiguous
    // (token, row block) ranges: a 128-byte line shared by neighbouring row blocks
    // (rows of inter/32 blocks need not end on a line) is then fetched once, not
    // once per XCD.
    const uint32_t nb = gridDim.x, xq = nb >> 3, xr = nb & 7, xc = blockIdx.x & 7;
    const uint32_t g = xc * xq + (xc < xr ? xc : xr) + (blockIdx.x >> 3);
    const uint32_t t = g / blocks_per_token;
    const uint32_t rb = g - t * blocks_per_token;
    const uint32_t pairs = inter >> 6;
    // wave-uniform, so the expert id and table entry come through scalar loads,
    // which do not wait behind the vector loads of the activations
    const uint32_t lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t gs = 64 / lpr, slot = lane / lpr, lp = lane - slot * lpr;
    const uint32_t rows_blk = gs * U;
    const uint32_t row0 = rb * rows_blk;
    float* red = lds;
    float* xst = lds + ((kk * rows_blk + 3u) & ~3u) + wave * JW * pairs * kPad;

    // the wave's activation slots are requested before the weights (loads complete
    // in order, so the LDS writes below then wait for the activations alone): lane l
    // holds float4s l, l + 64, ... of each of its JW slots
    constexpr int kAV = 8 / JW;
    const uint32_t n4a = inter >> 2;
    const bool a_regs = n4a <= 64u * kAV;
    float4 av[JW][kAV];
    if (a_regs) {
        typedef float f32x4 __attribute__((ext_vector_type(4)));
#pragma unroll
        for (int jj = 0; jj < JW; ++jj) {
            const uint32_t j = wave * JW + jj;
            const uint32_t jc = j < kk ? j : kk - 1;
            const gptr<f32x4> src = as_global(reinterpret_cast<const f32x4*>(act + (static_cast<size_t>(t) * kk + jc) * inter));
#pragma unroll
            for (int q = 0; q < kAV; ++q) {
                const uint32_t i = lane + static_cast<uint32_t>(q) * 64;
                if (i < n4a) {
                    const f32x4 v = src[i];
                    av[jj][q] = make_float4(v.x, v.y, v.z, v.w);
                }
            }
        }
    }
    R m[JW];
    bool ok[JW];
    uint32_t d[JW][U][CH][R::kDw];
    // every slot's id, then every slot's table entry, then the weights: one scalar
    // round trip per step rather than per slot
    uint32_t es[JW];
#pragma unroll
    for (int jj = 0; jj < JW; ++jj) es[jj] = 0;
    if (sel) {  // the router resolved the assignments to table entries (valid ids)
#pragma unroll
        for (int jj = 0; jj < JW; ++jj) {
            const uint32_t j = wave * JW + jj;
            const objeta_hip_expert_ptrs* f = (j >= k && j < kk) ? shared : sel + (t * k + (j < k ? j : k - 1));
            ok[jj] = true;
            m[jj] = RowsOf<R>::make(f->down, f->down_scale, inter);
        }
    } else {
#pragma unroll
        for (int jj = 0; jj < JW; ++jj) {
            const uint32_t j = wave * JW + jj;
            const uint32_t jc = j < k ? j : k - 1;
            ok[jj] = (j >= k && j < kk) ? true : expert_of(ids, t * k + jc, n_table, err, es[jj]);
            es[jj] = __builtin_amdgcn_readfirstlane(es[jj]);
        }
#pragma unroll
        for (int jj = 0; jj < JW; ++jj) {
            const uint32_t j = wave * JW + jj;
            const objeta_hip_expert_ptrs* f = (j >= k && j < kk) ? shared : table + es[jj];
            m[jj] = RowsOf<R>::make(f->down, f->down_scale, inter);
        }
    }
#pragma unroll
    for (int jj = 0; jj < JW; ++jj) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint32_t r = row0 + static_cast<uint32_t>(u) * gs + slot;
            const uint32_t rc = r < out_dim ? r : out_dim - 1;
#pragma unroll
            for (int c = 0; c < CH; ++c) m[jj].load(rc, lp + static_cast<uint32_t>(c) * lpr, d[jj][u][c]);
        }
    }
#pragma unroll
    for (int jj = 0; jj < JW; ++jj) {
        if (a_regs) {
#pragma unroll
            for (int q = 0; q < kAV; ++q) {
                const uint32_t i = lane + static_cast<uint32_t>(q) * 64;
                if (i < n4a) {
                    const uint32_t c = i << 2;
                    *reinterpret_cast<float4*>(xst + jj * pairs * kPad + (c >> 6) * kPad + (c & 63)) = av[jj][q];
                }
            }
        } else {
            const uint32_t j = wave * JW + jj;
            const uint32_t jc = j < kk ? j : kk - 1;
            stage_vec_wave(xst + jj * pairs * kPad, act + (static_cast<size_t>(t) * kk + jc) * inter, inter, lane);
        }
    }
    __syncthreads();

#pragma unroll
    for (int jj = 0; jj < JW; ++jj) {
        const uint32_t j = wave * JW + jj;
        float acc[U][1];
#pragma unroll
        for (int u = 0; u < U; ++u) acc[u][0] = 0.f;
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            const float* xl[1] = {xst + (jj * pairs + lp + static_cast<uint32_t>(c) * lpr) * kPad};
            if constexpr (U > 1) {
                // the chunk's 64 activations, read from LDS once for all U rows
                float4 xr4[16];
#pragma unroll
                for (int q = 0; q < 16; ++q) xr4[q] = *reinterpret_cast<const float4*>(xl[0] + 4 * q);
                const float* xr[1] = {reinterpret_cast<const float*>(xr4)};
#pragma unroll
                for (int u = 0; u < U; ++u) m[jj].template dot<1>(d[jj][u][c], xr, acc[u], xl);
            } else {
                m[jj].template dot<1>(d[jj][0][c], xl, acc[0]);
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const float v = row_reduce(acc[u][0], lp, lpr);
            if (slot < gs && lp == 0 && j < kk)
                red[j * rows_blk + static_cast<uint32_t>(u) * gs + slot] = ok[jj] ? v : __builtin_nanf("");
        }
    }
    __syncthreads();

    if (threadIdx.x < rows_blk) {
        const uint32_t r = row0 + threadIdx.x;
        if (r < out_dim) {
            const size_t o = static_cast<size_t>(t) * out_dim + r;
            float acc = resid ? resid[o] : 0.0f;
            for (uint32_t j = 0; j < k; ++j) acc = __builtin_fmaf(wts[t * k + j], red[j * rows_blk + threadIdx.x], acc);
            if (kk > k) acc += red[k * rows_blk + threadIdx.x];  // the shared expert, weight 1
            out[o] = acc;
        }
    }
}

// ------------------------------------------- general shapes (cols % 32 == 0)
// Used when hidden or intermediate is not a multiple of 64 or the activation
// stage would not fit in LDS: one wave per row, lanes stride over blocks.
template <int F>
__device__ __forceinline__ float block_weight(const uint8_t* __restrict__ blk, const uint8_t* __restrict__ sb,
                                              uint32_t i) {
    if constexpr (F == kQ4) {
        const uint32_t pk = blk[2 + i / 2];
        return static_cast<float>(static_cast<int>((i & 1) ? (pk >> 4) : (pk & 15)) - 8);
    } else if constexpr (F == kQ5) {
        const uint32_t pk = blk[6 + i / 2];
        const uint32_t lo = (i & 1) ? (pk >> 4) : (pk & 15);
        const uint32_t hi = (blk[2 + i / 8] >> (i & 7)) & 1u;
        return static_cast<float>(static_cast<int>(lo | (hi << 4)) - 16);
    } else if constexpr (F == kIQ3) {
        const uint32_t lo = (blk[2 + i / 4] >> (2 * (i & 3))) & 3u;
        const uint32_t hi = (blk[10 + i / 8] >> (i & 7)) & 1u;
        return static_cast<float>(static_cast<int>(lo | (hi << 2)) - 4);
    } else {
        (void)sb;
        const uint32_t pk = blk[i / 2];
        const uint32_t c = (i & 1) ? (pk >> 4) : (pk & 15);
        return f16_to_f32(((c & 7u) << 9) | ((c & 8u) << 12)) * 16384.0f;
    }
}

// Row r of an expert matrix against v[cols]; result in every lane of the wave.
template <int F>
__device__ __forceinline__ float row_dot_general(const uint8_t* __restrict__ w, const uint8_t* __restrict__ s,
                                                 uint32_t r, uint32_t cols, const float* __restrict__ v,
                                                 uint32_t lane) {
    const uint32_t nb = cols >> 5;
    float acc = 0.f;
    for (uint32_t b = lane; b < nb; b += 64) {
        const uint8_t* blk;
        float scale;
        if constexpr (F == kFP4) {
            blk = w + static_cast<size_t>(r) * (cols >> 1) + b * 16;
            scale = e8m0_to_f32(s[static_cast<size_t>(r) * nb + b]);
        } else {
            blk = w + (static_cast<size_t>(r) * nb + b) * Fmt<F>::kBlockBytes;
            scale = f16_to_f32(static_cast<uint32_t>(blk[0]) | (static_cast<uint32_t>(blk[1]) << 8));
        }
        for (uint32_t i = 0; i < 32; ++i)
            acc = __builtin_fmaf(block_weight<F>(blk, nullptr, i) * scale, v[b * 32 + i], acc);
    }
    return wave_reduce(acc);
}

// grid.x = ceil(n_assign * inter / 4); one wave per (assignment, row). Slots as
// in moe_gate_up_kernel (kk per token, the shared expert in slot k when kk > k).
template <int F>
__global__ __launch_bounds__(kThreads) void moe_gate_up_general(
    const objeta_hip_expert_ptrs* __restrict__ table, uint32_t n_table, const uint32_t* __restrict__ ids,
    const float* __restrict__ x, float* __restrict__ act, uint32_t hidden, uint32_t inter, uint32_t k,
    uint32_t n_assign, float limit, uint32_t* __restrict__ err, uint32_t kk,
    const objeta_hip_expert_ptrs* __restrict__ shared, uint32_t official) {
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t item = blockIdx.x * kWaves + (threadIdx.x >> 6);
    if (item >= n_assign * inter) return;
    const uint32_t a = item / inter, r = item - a * inter;
    const uint32_t t = a / kk, j = a - t * kk;
    uint32_t e = 0;
    const bool ok = j >= k ? true : expert_of(ids, t * k + j, n_table, err, e);
    const objeta_hip_expert_ptrs P = j >= k ? *shared : table[e];
    const float* xt = x + static_cast<size_t>(t) * hidden;
    const float g = row_dot_general<F>(static_cast<const uint8_t*>(P.gate), static_cast<const uint8_t*>(P.gate_scale),
                                       r, hidden, xt, lane);
    const float u = row_dot_general<F>(static_cast<const uint8_t*>(P.up), static_cast<const uint8_t*>(P.up_scale), r,
                                       hidden, xt, lane);
    if (lane == 0) act[static_cast<size_t>(a) * inter + r] = ok ? swiglu(g, u, limit, official) : __builtin_nanf("");
}

// grid.x = ceil(n_tokens * out_dim / 4); one wave per (token, row), slots in order.
template <int F>
__global__ __launch_bounds__(kThreads) void moe_down_general(
    const objeta_hip_expert_ptrs* __restrict__ table, uint32_t n_table, const uint32_t* __restrict__ ids,
    const float* __restrict__ wts, const float* __restrict__ act, const float* resid, float* out, uint32_t inter,
    uint32_t out_dim, uint32_t k, uint32_t n_tokens, uint32_t* __restrict__ err, uint32_t kk,
    const objeta_hip_expert_ptrs* __restrict__ shared) {
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t item = blockIdx.x * kWaves + (threadIdx.x >> 6);
    if (item >= n_tokens * out_dim) return;
    const uint32_t t = item / out_dim, r = item - t * out_dim;
    const size_t o = static_cast<size_t>(t) * out_dim + r;
    float acc = resid ? resid[o] : 0.0f;
    for (uint32_t j = 0; j < kk; ++j) {
        uint32_t e = 0;
        const bool ok = j >= k ? true : expert_of(ids, t * k + j, n_table, err, e);
        const objeta_hip_expert_ptrs P = j >= k ? *shared : table[e];
        const float v = row_dot_general<F>(static_cast<const uint8_t*>(P.down),
                                           static_cast<const uint8_t*>(P.down_scale), r, inter,
                                           act + (static_cast<size_t>(t) * kk + j) * inter, lane);
        const float w = j >= k ? 1.0f : wts[t * k + j];
        acc = __builtin_fmaf(w, ok ? v : __builtin_nanf(""), acc);
    }
    if (lane == 0) out[o] = acc;
}

}  // namespace dev

// ------------------------------------------------------------------ launchers
namespace {

using namespace dev;

constexpr uint32_t kMaxK = 32;  // selection slots per token (router's top-k bound)

// k routed slots per token plus, when `shared` is set, the shared expert in slot k:
// kk = k + (shared != nullptr) slots in all.
struct MoeShape {
    uint32_t n_table, n_tokens, k, hidden, inter, out_dim;
    const objeta_hip_expert_ptrs* shared = nullptr;
    bool official = false;  // gate/up applies the official SwiGLU
    uint32_t kk() const { return k + (shared ? 1u : 0u); }
};

size_t max_lds(const objeta_hip_context* ctx) {
    return ctx->info.max_shared_memory_per_block > 0 ? static_cast<size_t>(ctx->info.max_shared_memory_per_block)
                                                     : 65536u;
}

template <class R, int U, int CH>
hipError_t gate_up_fast(hipStream_t s, const objeta_hip_expert_ptrs* table, const uint32_t* ids, const float* x,
                        float* act, const MoeShape& sh, uint32_t lpr, float limit, uint32_t* err,
                        const objeta_hip_expert_ptrs* sel) {
    const uint32_t gs = 64 / lpr;
    const uint32_t rows_blk = kWaves * gs * U;
    const uint32_t bpa = (sh.inter + rows_blk - 1) / rows_blk;
    const uint32_t n_assign = sh.n_tokens * sh.kk();
    const size_t lds = static_cast<size_t>(sh.hidden >> 6) * kPad * sizeof(float) + 4 * sizeof(float);
    hipLaunchKernelGGL((moe_gate_up_kernel<R, U, CH>), dim3(n_assign * bpa), dim3(kThreads), lds, s, table,
                       sh.n_table, ids, x, act, sh.hidden, sh.inter, sh.k, lpr, bpa, limit, err, sel, sh.kk(),
                       sh.shared, sh.official ? 1u : 0u);
    return hipGetLastError();
}

template <class R, int U, int CH, int JW>
hipError_t down_fast(hipStream_t s, const objeta_hip_expert_ptrs* table, const uint32_t* ids, const float* wts,
                     const float* act, const float* resid, float* out, const MoeShape& sh, uint32_t lpr,
                     uint32_t* err, const objeta_hip_expert_ptrs* sel) {
    const uint32_t gs = 64 / lpr;
    const uint32_t rows_blk = gs * U;
    const uint32_t bpt = (sh.out_dim + rows_blk - 1) / rows_blk;
    const uint32_t waves = (sh.kk() + JW - 1) / JW;
    const size_t lds = (((sh.kk() * rows_blk + 3u) & ~3u) + static_cast<size_t>(waves) * JW * (sh.inter >> 6) * kPad) *
                       sizeof(float);
    hipLaunchKernelGGL((moe_down_kernel<R, U, CH, JW>), dim3(sh.n_tokens * bpt), dim3(waves * 64), lds, s, table,
                       sh.n_table, ids, wts, act, resid, out, sh.inter, sh.out_dim, sh.k, lpr, bpt, err, sel, sh.kk(),
                       sh.shared);
    return hipGetLastError();
}

size_t down_lds_bytes(const MoeShape& sh, uint32_t jw, uint32_t u) {
    const uint32_t lpr = pick_lpr(sh.inter >> 6);
    const uint32_t rows_blk = (64 / lpr) * u;
    const uint32_t waves = (sh.kk() + jw - 1) / jw;
    return (((sh.kk() * rows_blk + 3u) & ~3u) + static_cast<size_t>(waves) * jw * (sh.inter >> 6) * kPad) * sizeof(float);
}

// Dispatch on chunks per lane (pairs / lpr).
template <class R>
hipError_t launch_gate_up_rows(hipStream_t s, const objeta_hip_expert_ptrs* table, const uint32_t* ids,
                               const float* x, float* act, const MoeShape& sh, float limit, uint32_t* err,
                               uint32_t cus, const objeta_hip_expert_ptrs* sel) {
    const uint32_t pairs = sh.hidden >> 6;
    const uint32_t lpr = pick_lpr(pairs);
    const uint32_t ch = pairs / lpr;
    // two rows per slot when that still leaves a few workgroups per CU
    const uint32_t gs = 64 / lpr;
    const uint64_t blocks_u2 = static_cast<uint64_t>(sh.n_tokens) * sh.kk() * ((sh.inter + kWaves * gs * 2 - 1) / (kWaves * gs * 2));
    // FP8 rows carry 17 dwords each: two row slots, or more than two chunks per
    // lane, would spill (the official layer rejects shapes with more)
    if constexpr (R::kDw > 9) {
        if (ch == 1) return gate_up_fast<R, 1, 1>(s, table, ids, x, act, sh, lpr, limit, err, sel);
        return gate_up_fast<R, 1, 2>(s, table, ids, x, act, sh, lpr, limit, err, sel);
    } else {
        // (not with two chunks per lane: at hidden 7168 one row per slot is faster, DeepSeek
        // layer at one token 79.9 -> 76.7 us)
        const bool u2 = blocks_u2 >= 2ull * cus && ch == 1;
        switch (ch) {
            case 1: return u2 ? gate_up_fast<R, 2, 1>(s, table, ids, x, act, sh, lpr, limit, err, sel)
                              : gate_up_fast<R, 1, 1>(s, table, ids, x, act, sh, lpr, limit, err, sel);
            case 2: return gate_up_fast<R, 1, 2>(s, table, ids, x, act, sh, lpr, limit, err, sel);
            case 3: return gate_up_fast<R, 1, 3>(s, table, ids, x, act, sh, lpr, limit, err, sel);
            default: return gate_up_fast<R, 1, 4>(s, table, ids, x, act, sh, lpr, limit, err, sel);
        }
    }
}

template <class R>
hipError_t launch_down_rows(hipStream_t s, const objeta_hip_expert_ptrs* table, const uint32_t* ids,
                            const float* wts, const float* act, const float* resid, float* out, const MoeShape& sh,
                            uint32_t jw, uint32_t* err, const objeta_hip_expert_ptrs* sel) {
    const uint32_t pairs = sh.inter >> 6;
    const uint32_t lpr = pick_lpr(pairs);
    const uint32_t ch = pairs / lpr;
    if constexpr (R::kDw > 9) {  // FP8 rows: one or two chunks per lane (see launch_gate_up_rows)
        if (jw == 2) return ch == 1 ? down_fast<R, 1, 1, 2>(s, table, ids, wts, act, resid, out, sh, lpr, err, sel)
                                    : down_fast<R, 1, 2, 2>(s, table, ids, wts, act, resid, out, sh, lpr, err, sel);
        return ch == 1 ? down_fast<R, 1, 1, 1>(s, table, ids, wts, act, resid, out, sh, lpr, err, sel)
                       : down_fast<R, 1, 2, 1>(s, table, ids, wts, act, resid, out, sh, lpr, err, sel);
    } else {
        if (jw == 2) {
            switch (ch) {
                case 1: return down_fast<R, 1, 1, 2>(s, table, ids, wts, act, resid, out, sh, lpr, err, sel);
                case 2: return down_fast<R, 1, 2, 2>(s, table, ids, wts, act, resid, out, sh, lpr, err, sel);
                case 3: return down_fast<R, 1, 3, 2>(s, table, ids, wts, act, resid, out, sh, lpr, err, sel);
                default: return down_fast<R, 1, 4, 2>(s, table, ids, wts, act, resid, out, sh, lpr, err, sel);
            }
        }
        // long rows (32 lanes per row, two rows per wave): four rows per lane group, so
        // each wave's staged activations (inter floats) serve 8 rows instead of 2
        // (DeepSeek down at one token: 29 -> 21 us); only with the slots spread evenly
        // over the four SIMDs (with 9 waves the WG waits for the SIMD holding three)
        if (ch == 1 && lpr >= 32 && sh.kk() % 4 == 0)
            return down_fast<R, 4, 1, 1>(s, table, ids, wts, act, resid, out, sh, lpr, err, sel);
        switch (ch) {
            case 1: return down_fast<R, 1, 1, 1>(s, table, ids, wts, act, resid, out, sh, lpr, err, sel);
            case 2: return down_fast<R, 1, 2, 1>(s, table, ids, wts, act, resid, out, sh, lpr, err, sel);
            case 3: return down_fast<R, 1, 3, 1>(s, table, ids, wts, act, resid, out, sh, lpr, err, sel);
            default: return down_fast<R, 1, 4, 1>(s, table, ids, wts, act, resid, out, sh, lpr, err, sel);
        }
    }
}

template <int F>
hipError_t launch_general(hipStream_t s, const objeta_hip_expert_ptrs* table, const uint32_t* ids, const float* wts,
                          const float* x, float* act, const float* resid, float* out, const MoeShape& sh,
                          float limit, uint32_t* err, int phase) {
    if (phase == 0) {
        const uint64_t items = static_cast<uint64_t>(sh.n_tokens) * sh.kk() * sh.inter;
        hipLaunchKernelGGL((moe_gate_up_general<F>), dim3(static_cast<uint32_t>((items + kWaves - 1) / kWaves)),
                           dim3(kThreads), 0, s, table, sh.n_table, ids, x, act, sh.hidden, sh.inter, sh.k,
                           sh.n_tokens * sh.kk(), limit, err, sh.kk(), sh.shared, sh.official ? 1u : 0u);
    } else {
        const uint64_t items = static_cast<uint64_t>(sh.n_tokens) * sh.out_dim;
        hipLaunchKernelGGL((moe_down_general<F>), dim3(static_cast<uint32_t>((items + kWaves - 1) / kWaves)),
                           dim3(kThreads), 0, s, table, sh.n_table, ids, wts, act, resid, out, sh.inter, sh.out_dim,
                           sh.k, sh.n_tokens, err, sh.kk(), sh.shared);
    }
    return hipGetLastError();
}

bool fast_shape(uint32_t cols) {
    if (cols % 64 != 0) return false;
    const uint32_t pairs = cols >> 6;
    const uint32_t lpr = pick_lpr(pairs);
    return lpr != 0 && pairs / lpr <= 4;
}

}  // namespace

namespace {

int32_t validate_moe(const char* action, int32_t format, uint64_t n_table, uint64_t n_tokens, uint64_t k,
                     uint64_t hidden, uint64_t inter, uint64_t out_dim) {
    if (format < OBJETA_HIP_Q4_0 || format > OBJETA_HIP_FP4_E2M1)
        OBJ_FAIL(kInvalidInput, action, strf("unknown format %d", format));
    if (hidden % 32 != 0 || inter % 32 != 0)
        OBJ_FAIL(kInvalidInput, action,
                 strf("hidden %llu and intermediate %llu must be multiples of block_size 32",
                      (unsigned long long)hidden, (unsigned long long)inter));
    if (k == 0 || k > kMaxK) OBJ_FAIL(kInvalidInput, action, strf("k %llu must be in 1..=%u", (unsigned long long)k, kMaxK));
    if (hidden == 0 || inter == 0) OBJ_FAIL(kInvalidInput, action, "hidden and intermediate must be non-zero");
    if (n_table == 0) OBJ_FAIL(kInvalidInput, action, "expert table is empty");
    if (hidden > (1u << 24) || inter > (1u << 24) || out_dim > (1u << 26) || n_table > 0xFFFFFFFFull ||
        n_tokens * k * inter > 0x7FFFFFFFull || n_tokens * out_dim > 0x7FFFFFFFull || n_tokens * k > 0x7FFFFFFFull)
        OBJ_FAIL(kInvalidInput, action, "shape exceeds the 32-bit index range of the kernels");
    return 0;
}

MoeShape shape_of(uint64_t n_table, uint64_t n_tokens, uint64_t k, uint64_t hidden, uint64_t inter, uint64_t out_dim) {
    return MoeShape{static_cast<uint32_t>(n_table), static_cast<uint32_t>(n_tokens), static_cast<uint32_t>(k),
                    static_cast<uint32_t>(hidden), static_cast<uint32_t>(inter), static_cast<uint32_t>(out_dim)};
}

}  // namespace

// The official layer's routed FP4 gate/up and its FP8 shared expert's in one launch
// (moe_gate_up_pair_kernel): the routed rows as launch_gate_up_rows<Fp4Rows> blocks
// them, the shared expert's one row per slot. Returns false (nothing launched) when a
// lane would take more than two 64-column chunks of a row (FP8 rows spill there).
bool launch_gate_up_pair(objeta_hip_context* ctx, hipStream_t s, const objeta_hip_expert_ptrs* table,
                         const uint32_t* ids, const float* x, float* act, float* act_sh, const MoeShape& sh,
                         const objeta_hip_expert_ptrs* shared, float limit, hipError_t& e) {
    const uint32_t pairs = sh.hidden >> 6;
    const uint32_t lpr = pick_lpr(pairs);
    if (!fast_shape(sh.hidden) || lpr == 0 || pairs / lpr > 2 ||
        static_cast<size_t>(sh.hidden >> 6) * kPad * sizeof(float) + 16 > max_lds(ctx))
        return false;
    const uint32_t ch = pairs / lpr, gs = 64 / lpr;
    const uint32_t cus = ctx->info.compute_units > 0 ? static_cast<uint32_t>(ctx->info.compute_units) : 256u;
    const uint64_t routed = static_cast<uint64_t>(sh.n_tokens) * sh.k;
    // two rows per slot only with one chunk per lane, as in launch_gate_up_rows
    const bool u2 = routed * ((sh.inter + kWaves * gs * 2 - 1) / (kWaves * gs * 2)) >= 2ull * cus && ch == 1;
    const uint32_t bpa_r = (sh.inter + kWaves * gs * (u2 ? 2 : 1) - 1) / (kWaves * gs * (u2 ? 2 : 1));
    const uint32_t bpa_s = (sh.inter + kWaves * gs - 1) / (kWaves * gs);
    const uint32_t nb_s = sh.n_tokens * bpa_s;
    const dim3 grid(static_cast<uint32_t>(routed) * bpa_r + nb_s);
    const size_t lds = static_cast<size_t>(sh.hidden >> 6) * kPad * sizeof(float) + 4 * sizeof(float);
#define OBJ_PAIR(U, CH)                                                                                             \
    hipLaunchKernelGGL((moe_gate_up_pair_kernel<Fp4Rows, U, CH, Fp8Rows, 1, CH>), grid, dim3(kThreads), lds, s, table, \
                       sh.n_table, ids, x, act, act_sh, sh.hidden, sh.inter, sh.k, lpr, bpa_r, bpa_s, nb_s, limit,     \
                       ctx->err_word, shared, 1u)
    if (u2) OBJ_PAIR(2, 1);
    else if (ch == 1) OBJ_PAIR(1, 1);
    else OBJ_PAIR(1, 2);
#undef OBJ_PAIR
    e = hipGetLastError();
    return true;
}

int32_t launch_moe_gate_up(objeta_hip_context* ctx, int32_t format, hipStream_t s, const objeta_hip_expert_ptrs* table,
                           uint64_t n_table, const uint32_t* ids, uint64_t n_tokens, uint64_t k, const float* x,
                           float* act, uint64_t hidden, uint64_t inter, float limit,
                           const objeta_hip_expert_ptrs* sel, const objeta_hip_expert_ptrs* shared, bool official) {
    const char* action = "launch MoE gate/up";
    OBJ_TRY(validate_moe(action, format, n_table, n_tokens, k, hidden, inter, 1));
    if (n_tokens == 0) return 0;
    if (!table || !x || !act) OBJ_FAIL(kInvalidInput, action, "NULL device pointer");
    if (reinterpret_cast<uintptr_t>(x) % 16) OBJ_FAIL(kInvalidInput, action, "x must be 16-byte aligned");
    MoeShape sh = shape_of(n_table, n_tokens, k, hidden, inter, 1);
    sh.shared = shared;
    sh.official = official;
    uint32_t* err = ctx->err_word;
    const uint32_t cus = ctx->info.compute_units > 0 ? static_cast<uint32_t>(ctx->info.compute_units) : 256u;
    const bool fast = fast_shape(sh.hidden) && static_cast<size_t>(sh.hidden >> 6) * kPad * sizeof(float) + 16 <= max_lds(ctx);
    hipError_t e;
    if (fast) {
        switch (format) {
            case OBJETA_HIP_Q4_0: e = launch_gate_up_rows<QRows<kQ4>>(s, table, ids, x, act, sh, limit, err, cus, sel); break;
            case OBJETA_HIP_Q5_0: e = launch_gate_up_rows<QRows<kQ5>>(s, table, ids, x, act, sh, limit, err, cus, sel); break;
            case OBJETA_HIP_IQ3_0: e = launch_gate_up_rows<QRows<kIQ3>>(s, table, ids, x, act, sh, limit, err, cus, sel); break;
            default: e = launch_gate_up_rows<Fp4Rows>(s, table, ids, x, act, sh, limit, err, cus, sel); break;
        }
    } else {
        switch (format) {
            case OBJETA_HIP_Q4_0: e = launch_general<kQ4>(s, table, ids, nullptr, x, act, nullptr, nullptr, sh, limit, err, 0); break;
            case OBJETA_HIP_Q5_0: e = launch_general<kQ5>(s, table, ids, nullptr, x, act, nullptr, nullptr, sh, limit, err, 0); break;
            case OBJETA_HIP_IQ3_0: e = launch_general<kIQ3>(s, table, ids, nullptr, x, act, nullptr, nullptr, sh, limit, err, 0); break;
            default: e = launch_general<kFP4>(s, table, ids, nullptr, x, act, nullptr, nullptr, sh, limit, err, 0); break;
        }
    }
    if (e != hipSuccess) OBJ_FAIL(kDriver, action, hipGetErrorString(e));
    return 0;
}

int32_t launch_moe_down(objeta_hip_context* ctx, int32_t format, hipStream_t s, const objeta_hip_expert_ptrs* table,
                        uint64_t n_table, const uint32_t* ids, const float* wts, uint64_t n_tokens, uint64_t k,
                        const float* act, const float* resid, float* out, uint64_t inter, uint64_t out_dim,
                        const objeta_hip_expert_ptrs* sel, const objeta_hip_expert_ptrs* shared) {
    const char* action = "launch MoE down + combine";
    OBJ_TRY(validate_moe(action, format, n_table, n_tokens, k, 32, inter, out_dim));
    if (n_tokens == 0 || out_dim == 0) return 0;
    if (!table || !wts || !act || !out) OBJ_FAIL(kInvalidInput, action, "NULL device pointer");
    if (reinterpret_cast<uintptr_t>(act) % 16) OBJ_FAIL(kInvalidInput, action, "act must be 16-byte aligned");
    MoeShape sh = shape_of(n_table, n_tokens, k, 32, inter, out_dim);
    sh.shared = shared;
    uint32_t* err = ctx->err_word;
    uint32_t jw = 0;
    if (fast_shape(sh.inter)) {
        // one token: one selection slot per wave (k waves per workgroup), measured
        // 0.2 us faster per Qwen3-A3B layer; batches: two slots per wave (16 tokens:
        // 4.3 against 4.7 ms per 48-layer step)
        const bool jw1 = down_lds_bytes(sh, 1, 1) <= max_lds(ctx) && sh.kk() <= 16;
        const bool jw2 = down_lds_bytes(sh, 2, 1) <= max_lds(ctx) && (sh.kk() + 1) / 2 <= 16;
        if (sh.n_tokens == 1 && jw1) jw = 1;
        else if (jw2) jw = 2;
        else if (jw1) jw = 1;
    }
    hipError_t e;
    // one token with a shared expert as slot k: when the k routed slots spread evenly
    // over the four SIMDs with four rows per lane group, they run in one launch and the
    // shared expert is added by a second (out = (resid + routed sum) + shared, the
    // order of the one-launch form), instead of nine waves of one row each (DeepSeek
    // shape: 31.9 us in one launch)
    if (jw == 1 && shared && sh.n_tokens == 1 && sh.k % 4 == 0) {
        const uint32_t pairs = sh.inter >> 6, lpr = pick_lpr(pairs);
        if (lpr >= 32 && pairs / lpr == 1) {
            MoeShape rsh = sh;
            rsh.shared = nullptr;
            MoeShape ssh = shape_of(1, 1, 0, 32, inter, out_dim);
            ssh.shared = shared;
            const float* act_sh = act + static_cast<size_t>(sh.k) * sh.inter;
            switch (format) {
                case OBJETA_HIP_Q4_0:
                    e = launch_down_rows<QRows<kQ4>>(s, table, ids, wts, act, resid, out, rsh, 1, err, sel);
                    if (e == hipSuccess) e = launch_down_rows<QRows<kQ4>>(s, shared, nullptr, nullptr, act_sh, out, out, ssh, 1, err, nullptr);
                    break;
                case OBJETA_HIP_Q5_0:
                    e = launch_down_rows<QRows<kQ5>>(s, table, ids, wts, act, resid, out, rsh, 1, err, sel);
                    if (e == hipSuccess) e = launch_down_rows<QRows<kQ5>>(s, shared, nullptr, nullptr, act_sh, out, out, ssh, 1, err, nullptr);
                    break;
                case OBJETA_HIP_IQ3_0:
                    e = launch_down_rows<QRows<kIQ3>>(s, table, ids, wts, act, resid, out, rsh, 1, err, sel);
                    if (e == hipSuccess) e = launch_down_rows<QRows<kIQ3>>(s, shared, nullptr, nullptr, act_sh, out, out, ssh, 1, err, nullptr);
                    break;
                default:
                    e = launch_down_rows<Fp4Rows>(s, table, ids, wts, act, resid, out, rsh, 1, err, sel);
                    if (e == hipSuccess) e = launch_down_rows<Fp4Rows>(s, shared, nullptr, nullptr, act_sh, out, out, ssh, 1, err, nullptr);
                    break;
            }
            if (e != hipSuccess) OBJ_FAIL(kDriver, action, hipGetErrorString(e));
            return 0;
        }
    }
    if (jw) {
        switch (format) {
            case OBJETA_HIP_Q4_0: e = launch_down_rows<QRows<kQ4>>(s, table, ids, wts, act, resid, out, sh, jw, err, sel); break;
            case OBJETA_HIP_Q5_0: e = launch_down_rows<QRows<kQ5>>(s, table, ids, wts, act, resid, out, sh, jw, err, sel); break;
            case OBJETA_HIP_IQ3_0: e = launch_down_rows<QRows<kIQ3>>(s, table, ids, wts, act, resid, out, sh, jw, err, sel); break;
            default: e = launch_down_rows<Fp4Rows>(s, table, ids, wts, act, resid, out, sh, jw, err, sel); break;
        }
    } else {
        switch (format) {
            case OBJETA_HIP_Q4_0: e = launch_general<kQ4>(s, table, ids, wts, nullptr, const_cast<float*>(act), resid, out, sh, 0.f, err, 1); break;
            case OBJETA_HIP_Q5_0: e = launch_general<kQ5>(s, table, ids, wts, nullptr, const_cast<float*>(act), resid, out, sh, 0.f, err, 1); break;
            case OBJETA_HIP_IQ3_0: e = launch_general<kIQ3>(s, table, ids, wts, nullptr, const_cast<float*>(act), resid, out, sh, 0.f, err, 1); break;
            default: e = launch_general<kFP4>(s, table, ids, wts, nullptr, const_cast<float*>(act), resid, out, sh, 0.f, err, 1); break;
        }
    }
    if (e != hipSuccess) OBJ_FAIL(kDriver, action, hipGetErrorString(e));
    return 0;
}

int32_t launch_moe_selected(objeta_hip_context* ctx, int32_t format, hipStream_t s,
                            const objeta_hip_expert_ptrs* table, uint64_t n_table, const uint32_t* ids,
                            const float* wts, uint64_t n_tokens, uint64_t k, const float* x, const float* resid,
                            float* out, uint64_t hidden, uint64_t inter, uint64_t out_dim, float limit, float* act,
                            const objeta_hip_expert_ptrs* sel, const objeta_hip_expert_ptrs* shared) {
    OBJ_TRY(validate_moe("launch selected-expert MoE", format, n_table, n_tokens, k, hidden, inter, out_dim));
    if (n_tokens == 0 || out_dim == 0) return 0;
    OBJ_TRY(launch_moe_gate_up(ctx, format, s, table, n_table, ids, n_tokens, k, x, act, hidden, inter, limit, sel,
                               shared));
    return launch_moe_down(ctx, format, s, table, n_table, ids, wts, n_tokens, k, act, resid, out, inter, out_dim,
                           sel, shared);
}

// ------------------------------------------------------- official FP4 layer
// execute_selected_moe_official_routed_fp4_cuda (moe.rs:1393-1663) for a batch of
// tokens (from kOfficialGroupedMinTokens tokens on, launch_moe_official_grouped), in
// six launches: act_quant(x) dequantized; the routed gate/up (FP4 split
// weights, official SwiGLU) of every (token, slot); the shared expert's gate/up
// (FP8 weights) into the rows after them; act_quant of all intermediates,
// dequantized in place; the routed down with the weighted combine from zero
// (d_out += w * down in selection order); the shared down added with weight 1.
// Workspace: x dequantized [n_tokens][hidden], then the intermediates
// [n_tokens * k routed rows | n_tokens shared rows][inter]. inter_values /
// inter_scales (nullable) receive the intermediates' FP8 bytes and scales in that
// row order.
int32_t launch_moe_official_fp4(objeta_hip_context* ctx, hipStream_t s, const objeta_hip_expert_ptrs* table,
                                uint64_t n_table, const objeta_hip_expert_ptrs* shared, const uint32_t* ids,
                                const float* wts, uint64_t n_tokens, uint64_t k, const float* x, float* out,
                                uint64_t hidden, uint64_t inter, uint64_t out_dim, float limit,
                                uint8_t* inter_values, uint8_t* inter_scales, const OfficialMarks* marks) {
    const char* action = "launch official FP4 MoE";
    // k = 0 (an empty selection) leaves the shared expert alone, over zeros
    OBJ_TRY(validate_moe(action, OBJETA_HIP_FP4_E2M1, n_table, n_tokens, k ? k : 1, hidden, inter, out_dim));
    if (hidden % 128 != 0 || inter % 128 != 0)
        OBJ_FAIL(kInvalidInput, action,
                 strf("hidden %llu and intermediate %llu must be multiples of the act_quant block 128",
                      (unsigned long long)hidden, (unsigned long long)inter));
    if (!(limit >= 0.0f)) OBJ_FAIL(kInvalidInput, action, "swiglu_limit must be a number >= 0 (clamp(-l, l))");
    if (n_tokens == 0 || out_dim == 0) return 0;
    if ((k && (!table || !ids || !wts)) || !x || !out) OBJ_FAIL(kInvalidInput, action, "NULL device pointer");
    const uint64_t kk = k + (shared ? 1 : 0);
    MoeShape ssh = shape_of(1, n_tokens, 0, hidden, inter, out_dim);
    ssh.shared = shared;
    ssh.official = true;
    if (shared) {
        auto chunks = [](uint32_t cols) { return (cols >> 6) / pick_lpr(cols >> 6); };
        const bool fits = fast_shape(ssh.hidden) && fast_shape(ssh.inter) && chunks(ssh.hidden) <= 2 &&
                          chunks(ssh.inter) <= 2 &&
                          static_cast<size_t>(ssh.hidden >> 6) * kPad * sizeof(float) + 16 <= max_lds(ctx) &&
                          down_lds_bytes(ssh, 1, 1) <= max_lds(ctx);
        if (!fits)
            OBJ_FAIL(kUnsupported, action,
                     strf("FP8 shared expert needs hidden %llu and intermediate %llu with a streaming lane split",
                          (unsigned long long)hidden, (unsigned long long)inter));
    }
    // a batch: every routed expert's matrices (and the shared expert's) read once per
    // member set instead of once per (token, slot)
    if (official_grouped_supported(n_table, n_tokens, k, hidden, inter, out_dim))
        return launch_moe_official_grouped(ctx, s, table, n_table, shared, ids, wts, n_tokens, k, x, out, hidden,
                                           inter, out_dim, limit, inter_values, inter_scales, marks);
    const size_t xb = (static_cast<size_t>(n_tokens * hidden) * sizeof(float) + 255) & ~size_t(255);
    const size_t ab = static_cast<size_t>(n_tokens * kk * inter) * sizeof(float);
    void* ws = nullptr;
    OBJ_TRY(ensure_workspace(ctx, s, kWsOfficial, xb + ab + 64, &ws));
    float* xd = static_cast<float*>(ws);
    float* act = reinterpret_cast<float*>(static_cast<char*>(ws) + xb);
    float* act_sh = act + n_tokens * k * inter;
    uint32_t* err = ctx->err_word;
    const uint32_t cus = ctx->info.compute_units > 0 ? static_cast<uint32_t>(ctx->info.compute_units) : 256u;
    auto mark = [&](hipEvent_t e) -> int32_t {
        if (e) OBJ_HIP(hipEventRecord(e, s), "record event");
        return 0;
    };
    OBJ_TRY(launch_act_quant(s, x, n_tokens, hidden, nullptr, nullptr, xd));
    // routed and shared gate/up in one launch, unless the executor times them apart
    bool paired = false;
    if (k && shared && !marks) {
        MoeShape rsh = shape_of(n_table, n_tokens, k, hidden, inter, out_dim);
        rsh.official = true;
        hipError_t e = hipSuccess;
        paired = launch_gate_up_pair(ctx, s, table, ids, xd, act, act_sh, rsh, shared, limit, e);
        if (paired && e != hipSuccess) OBJ_FAIL(kDriver, action, hipGetErrorString(e));
    }
    if (!paired) {
        if (k)
            OBJ_TRY(launch_moe_gate_up(ctx, OBJETA_HIP_FP4_E2M1, s, table, n_table, ids, n_tokens, k, xd, act, hidden,
                                       inter, limit, nullptr, nullptr, true));
        OBJ_TRY(mark(marks ? marks->gate_up_end : nullptr));
        if (shared) {
            const hipError_t e = launch_gate_up_rows<Fp8Rows>(s, shared, nullptr, xd, act_sh, ssh, limit, err, cus, nullptr);
            if (e != hipSuccess) OBJ_FAIL(kDriver, action, hipGetErrorString(e));
        }
        OBJ_TRY(mark(marks ? marks->shared_gate_up_end : nullptr));
    }
    if (kk) OBJ_TRY(launch_act_quant(s, act, n_tokens * kk, inter, inter_values, inter_scales, act));
    OBJ_TRY(mark(marks ? marks->act_quant_end : nullptr));
    if (k)
        OBJ_TRY(launch_moe_down(ctx, OBJETA_HIP_FP4_E2M1, s, table, n_table, ids, wts, n_tokens, k, act, nullptr, out,
                                inter, out_dim));
    else
        OBJ_TRY(launch_zero(s, out, n_tokens * out_dim * sizeof(float)));
    OBJ_TRY(mark(marks ? marks->down_end : nullptr));
    if (shared) {
        const hipError_t e = launch_down_rows<Fp8Rows>(s, shared, nullptr, nullptr, act_sh, out, out, ssh, 1, err, nullptr);
        if (e != hipSuccess) OBJ_FAIL(kDriver, action, hipGetErrorString(e));
    }
    return 0;
}

// ------------------------------------------------ static activation scratch
// The activations [n_tokens * k][intermediate] of objeta_hip_moe_selected_device_noalloc
// live in this file-scope array (4 MiB on every device the library runs on, held
// until the process ends) instead of a context workspace. In host code `scratch`
// names a host-side stand-in, not the device array: only the address that
// hipGetSymbolAddress returns (per device, with that device current) is passed to
// kernels. Every call on a device shares the array; calls that overlap on one
// device race. Nothing in it needs clearing: gate/up writes every activation that
// down reads.
static __device__ __align__(256) float scratch[kStaticActFloats];

namespace {
std::mutex g_scratch_mu;
constexpr int kMaxDevices = 64;
void* g_scratch_ptr[kMaxDevices] = {};
}  // namespace

int32_t bind_static_scratch(objeta_hip_context* ctx) {
    if (ctx->device < 0 || ctx->device >= kMaxDevices)
        OBJ_FAIL(kUnsupported, "bind static scratch", strf("device ordinal %d >= %d", ctx->device, kMaxDevices));
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[ctx->device]) {
        void* p = nullptr;
        OBJ_HIP(hipSetDevice(ctx->device), "hipSetDevice");
        OBJ_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(static activation scratch)");
        if (!p) OBJ_FAIL(kDriver, "bind static scratch", "hipGetSymbolAddress returned NULL");
        g_scratch_ptr[ctx->device] = p;
    }
    ctx->static_act = static_cast<float*>(g_scratch_ptr[ctx->device]);
    return 0;
}

int32_t moe_act_scratch(objeta_hip_context* ctx, hipStream_t s, uint64_t n_tokens, uint64_t k, uint64_t inter,
                        float** out) {
    void* p = nullptr;
    OBJ_TRY(ensure_workspace(ctx, s, kWsMoeAct, static_cast<size_t>(n_tokens * k * inter) * sizeof(float) + 64, &p));
    *out = static_cast<float*>(p);
    return 0;
}

}  // namespace objeta

using namespace objeta;

extern "C" {

int32_t objeta_hip_moe_selected_shared_device(objeta_hip_context* ctx, int32_t format, objeta_hip_stream stream,
                                              const objeta_hip_expert_ptrs* d_table, uint64_t n_table,
                                              const objeta_hip_expert_ptrs* d_shared, const uint32_t* d_ids,
                                              const float* d_weights, uint64_t n_tokens, uint64_t k, const float* d_x,
                                              const float* d_residual, float* d_out, uint64_t hidden,
                                              uint64_t intermediate, uint64_t out_dim, float swiglu_limit) {
    OBJ_GUARD_BEGIN
    OBJ_TRY(check_ctx(ctx, "moe_selected_device"));
    OBJ_HIP(hipSetDevice(ctx->device), "hipSetDevice");
    hipStream_t s = resolve_stream(ctx, stream);
    if (n_tokens == 0 || out_dim == 0) return 0;
    float* act = nullptr;
    const uint64_t kk = (k ? k : 1) + (d_shared ? 1 : 0);
    OBJ_TRY(moe_act_scratch(ctx, s, n_tokens, kk, intermediate ? intermediate : 1, &act));
    return launch_moe_selected(ctx, format, s, d_table, n_table, d_ids, d_weights, n_tokens, k, d_x, d_residual,
                               d_out, hidden, intermediate, out_dim, swiglu_limit, act, nullptr, d_shared);
    OBJ_GUARD_END
}

int32_t objeta_hip_moe_selected_device(objeta_hip_context* ctx, int32_t format, objeta_hip_stream stream,
                                       const objeta_hip_expert_ptrs* d_table, uint64_t n_table,
                                       const uint32_t* d_ids, const float* d_weights, uint64_t n_tokens,
                                       uint64_t k, const float* d_x, const float* d_residual, float* d_out,
                                       uint64_t hidden, uint64_t intermediate, uint64_t out_dim,
                                       float swiglu_limit) {
    return objeta_hip_moe_selected_shared_device(ctx, format, stream, d_table, n_table, nullptr, d_ids, d_weights,
                                                 n_tokens, k, d_x, d_residual, d_out, hidden, intermediate, out_dim,
                                                 swiglu_limit);
}

int32_t objeta_hip_moe_selected_device_noalloc(objeta_hip_context* ctx, int32_t format, objeta_hip_stream stream,
                                               const objeta_hip_expert_ptrs* d_table, uint64_t n_table,
                                               const uint32_t* d_ids, const float* d_weights, uint64_t n_tokens,
                                               uint64_t k, const float* d_x, const float* d_residual, float* d_out,
                                               uint64_t hidden, uint64_t intermediate, uint64_t out_dim,
                                               float swiglu_limit) {
    OBJ_GUARD_BEGIN
    const char* action = "moe_selected_device_noalloc";
    OBJ_TRY(check_ctx(ctx, action));
    OBJ_HIP(hipSetDevice(ctx->device), "hipSetDevice");
    hipStream_t s = resolve_stream(ctx, stream);
    OBJ_TRY(validate_moe(action, format, n_table, n_tokens, k, hidden, intermediate, out_dim));
    if (n_tokens == 0 || out_dim == 0) return 0;
    if (n_tokens * k * intermediate > kStaticActFloats)
        OBJ_FAIL(kInvalidInput, action,
                 strf("n_tokens * k * intermediate = %llu exceeds the static scratch of %llu floats",
                      (unsigned long long)(n_tokens * k * intermediate), (unsigned long long)kStaticActFloats));
    if (!ctx->static_act) OBJ_FAIL(kInternal, action, "static scratch not bound");
    return launch_moe_selected(ctx, format, s, d_table, n_table, d_ids, d_weights, n_tokens, k, d_x, d_residual,
                               d_out, hidden, intermediate, out_dim, swiglu_limit, ctx->static_act, nullptr, nullptr);
    OBJ_GUARD_END
}

int32_t objeta_hip_moe_gate_up_device(objeta_hip_context* ctx, int32_t format, objeta_hip_stream stream,
                                      const objeta_hip_expert_ptrs* d_table, uint64_t n_table,
                                      const uint32_t* d_ids, uint64_t n_tokens, uint64_t k, const float* d_x,
                                      float* d_act, uint64_t hidden, uint64_t intermediate, float swiglu_limit) {
    OBJ_GUARD_BEGIN
    OBJ_TRY(check_ctx(ctx, "moe_gate_up_device"));
    OBJ_HIP(hipSetDevice(ctx->device), "hipSetDevice");
    return launch_moe_gate_up(ctx, format, resolve_stream(ctx, stream), d_table, n_table, d_ids, n_tokens, k, d_x,
                              d_act, hidden, intermediate, swiglu_limit, nullptr, nullptr);
    OBJ_GUARD_END
}

int32_t objeta_hip_moe_down_device(objeta_hip_context* ctx, int32_t format, objeta_hip_stream stream,
                                   const objeta_hip_expert_ptrs* d_table, uint64_t n_table, const uint32_t* d_ids,
                                   const float* d_weights, uint64_t n_tokens, uint64_t k, const float* d_act,
                                   const float* d_residual, float* d_out, uint64_t intermediate, uint64_t out_dim) {
    OBJ_GUARD_BEGIN
    OBJ_TRY(check_ctx(ctx, "moe_down_device"));
    OBJ_HIP(hipSetDevice(ctx->device), "hipSetDevice");
    return launch_moe_down(ctx, format, resolve_stream(ctx, stream), d_table, n_table, d_ids, d_weights, n_tokens, k,
                           d_act, d_residual, d_out, intermediate, out_dim, nullptr, nullptr);
    OBJ_GUARD_END
}

int32_t objeta_hip_moe_layer_shared_device(objeta_hip_context* ctx, int32_t format, objeta_hip_stream stream,
                                           const objeta_hip_expert_ptrs* d_table, uint64_t n_experts,
                                           const objeta_hip_expert_ptrs* d_shared, const float* d_router_w,
                                           const float* d_router_bias, uint64_t k, int32_t renormalize,
                                           uint64_t n_tokens, const float* d_x, const float* d_residual, float* d_out,
                                           uint32_t* d_ids_out, float* d_weights_out, uint64_t hidden,
                                           uint64_t intermediate, uint64_t out_dim, float swiglu_limit) {
    OBJ_GUARD_BEGIN
    OBJ_TRY(check_ctx(ctx, "moe_layer_device"));
    OBJ_HIP(hipSetDevice(ctx->device), "hipSetDevice");
    hipStream_t s = resolve_stream(ctx, stream);
    if (n_tokens == 0) return 0;
    if (!d_ids_out || !d_weights_out) OBJ_FAIL(kInvalidInput, "moe_layer_device", "NULL routing output");
    // a batch whose tokens share experts: each selected expert's matrices once for
    // all of its tokens
    if (out_dim > 0 && d_table && grouped_preferred(format, n_tokens, hidden, intermediate, out_dim) &&
        grouped_supported(format, n_experts, n_tokens, k, hidden, intermediate, out_dim)) {
        OBJ_TRY(launch_router(ctx, s, d_router_w, d_router_bias, d_x, n_tokens, n_experts, hidden, k, renormalize,
                              d_ids_out, d_weights_out, nullptr, nullptr));
        return launch_moe_grouped(ctx, format, s, d_table, n_experts, d_shared, d_ids_out, d_weights_out, n_tokens, k,
                                  d_x, d_residual, d_out, hidden, intermediate, out_dim, swiglu_limit);
    }
    // the router also resolves the selection to table entries for the expert kernels
    void* sws = nullptr;
    OBJ_TRY(ensure_workspace(ctx, s, kWsSelTab, static_cast<size_t>(n_tokens * (k ? k : 1)) * sizeof(objeta_hip_expert_ptrs),
                             &sws));
    objeta_hip_expert_ptrs* sel = d_table ? static_cast<objeta_hip_expert_ptrs*>(sws) : nullptr;
    OBJ_TRY(launch_router(ctx, s, d_router_w, d_router_bias, d_x, n_tokens, n_experts, hidden, k, renormalize,
                          d_ids_out, d_weights_out, d_table, &sel));
    if (out_dim == 0) return 0;
    float* act = nullptr;
    OBJ_TRY(moe_act_scratch(ctx, s, n_tokens, k + (d_shared ? 1 : 0), intermediate ? intermediate : 1, &act));
    return launch_moe_selected(ctx, format, s, d_table, n_experts, d_ids_out, d_weights_out, n_tokens, k, d_x,
                               d_residual, d_out, hidden, intermediate, out_dim, swiglu_limit, act, sel, d_shared);
    OBJ_GUARD_END
}

int32_t objeta_hip_moe_layer_device(objeta_hip_context* ctx, int32_t format, objeta_hip_stream stream,
                                    const objeta_hip_expert_ptrs* d_table, uint64_t n_experts,
                                    const float* d_router_w, const float* d_router_bias, uint64_t k,
                                    int32_t renormalize, uint64_t n_tokens, const float* d_x,
                                    const float* d_residual, float* d_out, uint32_t* d_ids_out,
                                    float* d_weights_out, uint64_t hidden, uint64_t intermediate,
                                    uint64_t out_dim, float swiglu_limit) {
    return objeta_hip_moe_layer_shared_device(ctx, format, stream, d_table, n_experts, nullptr, d_router_w,
                                              d_router_bias, k, renormalize, n_tokens, d_x, d_residual, d_out,
                                              d_ids_out, d_weights_out, hidden, intermediate, out_dim, swiglu_limit);
}

int32_t objeta_hip_moe_official_fp4_device(objeta_hip_context* ctx, objeta_hip_stream stream,
                                           const objeta_hip_expert_ptrs* d_table, uint64_t n_table,
                                           const objeta_hip_expert_ptrs* d_shared_fp8, const uint32_t* d_ids,
                                           const float* d_weights, uint64_t n_tokens, uint64_t k, const float* d_x,
                                           float* d_out, uint64_t hidden, uint64_t intermediate, uint64_t out_dim,
                                           float swiglu_limit, uint8_t* d_inter_values, uint8_t* d_inter_scales) {
    OBJ_GUARD_BEGIN
    OBJ_TRY(check_ctx(ctx, "moe_official_fp4_device"));
    OBJ_HIP(hipSetDevice(ctx->device), "hipSetDevice");
    return launch_moe_official_fp4(ctx, resolve_stream(ctx, stream), d_table, n_table, d_shared_fp8, d_ids, d_weights,
                                   n_tokens, k, d_x, d_out, hidden, intermediate, out_dim, swiglu_limit,
                                   d_inter_values, d_inter_scales, nullptr);
    OBJ_GUARD_END
}

int32_t objeta_hip_device_error(objeta_hip_context* ctx, uint32_t* out) {
    OBJ_GUARD_BEGIN
    OBJ_TRY(check_ctx(ctx, "device error word"));
    if (!out) OBJ_FAIL(kInvalidInput, "device error word", "out is NULL");
    OBJ_HIP(hipSetDevice(ctx->device), "hipSetDevice");
    for (hipStream_t st : ctx->streams) OBJ_HIP(hipStreamSynchronize(st), "synchronize stream");
    uint32_t* err = ctx->err_word;
    OBJ_HIP(hipMemcpy(out, err, sizeof(uint32_t), hipMemcpyDeviceToHost), "read device error word");
    const uint32_t zero = 0;
    OBJ_HIP(hipMemcpy(err, &zero, sizeof(uint32_t), hipMemcpyHostToDevice), "clear device error word");
    return 0;
    OBJ_GUARD_END
}

}  // extern "C"
