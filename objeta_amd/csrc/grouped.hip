// grouped.hip — the grouped-token expert product on gfx950 matrix cores.
//
// With a batch of tokens, the per-(token, slot) kernels of moe.hip stream an
// expert's matrices once per assignment that selected it. Here the assignments
// are grouped by expert on the device and each selected expert's gate, up and
// down matrices are read once for all of its tokens, the products running on
// MFMA (v_mfma_f32_16x16x32_f16). Per layer:
//
//   moe_group_kernel     assignments (token, slot) sorted by expert, stable; one
//                        group per distinct selected expert
//   moe_split_kernel     activation rows -> two fp16 parts (see below), per token
//   moe_grouped_kernel   per (group, 16 rows): silu(gate x) * (up x) for the group
//   moe_split_kernel     the activations of every assignment
//   moe_grouped_kernel   per (group, 16 rows): down act for every assignment
//   moe_combine_kernel   out = residual + sum_j w_j down_j in slot order
//
// Exactness. Weights enter the MFMA as fp16 values that are exact for every
// format: q-8 (Q4_0), q-16 (Q5_0), q-4 (IQ3_0), the E2M1 value * 2^-14 (FP4). The
// block scale multiplies the fp32 block sum. An activation row x is scaled by a
// power of two 2^s (|x 2^s| < 2^14, exact) and split x 2^s = hi + lo with hi, lo
// fp16: hi + lo carries 22 significant bits of x, every weight * part product is
// exact in fp32 and the MFMA accumulates in fp32. The result is within the fp32
// tolerance of the reference's sequential sums (not bit-identical: the order of
// the additions differs, as in every parallel kernel here).
//
// Layout trick: within each 8-element k group the weights come out of the nibble
// unpacking as (w0,w4),(w1,w5),(w2,w6),(w3,w7); the split activations are stored
// in that same order, so no unpacking shuffle is needed (a k permutation applied
// to both operands leaves the products unchanged).
//
// MFMA roles (D = A B, 16x16x32): A = activation parts, row m = 2 * token + part
// (8 tokens per instruction); B = weights, column n = output row. Lane l holds
// B[k = 8(l/16) .. +7][n = l%16] and D[m = 4(l/16) + i][n = l%16]: every lane
// owns one output row, so the block scale it applies is its own row's and the hi
// and lo parts of a token land in the same lane (i = 2q, 2q+1).
//
// Reference: execute_selected_moe_cuda (crates/objeta-cuda/src/moe.rs:352-751)
// runs each selected expert per token; its combine adds w * down in selection
// order (moe.rs:1319-1321), which moe_combine_kernel keeps.
#include "device_common.hpp"
#include "gemv_stream.hpp"
#include "host_common.hpp"
#include "kernels.hpp"

namespace objeta {
namespace {

using namespace dev;

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr uint32_t kGMaxTable = 1024;   // experts per table
constexpr uint32_t kGMaxAssign = 1024;  // tokens * k per call
constexpr uint32_t kPerm[8] = {0, 4, 1, 5, 2, 6, 3, 7};

struct GroupWs {
    uint32_t* hdr;         // [0] number of groups
    uint32_t* grp_expert;  // [A]
    uint32_t* grp_start;   // [A + 1]
    uint32_t* alist;       // [A] assignment t*k + j, grouped by expert
};

// ------------------------------------------------------------------ grouping
__global__ __launch_bounds__(256) void moe_group_kernel(const uint32_t* __restrict__ ids, uint32_t n_assign,
                                                        uint32_t n_table, GroupWs w, uint32_t* __restrict__ err) {
    __shared__ uint32_t cnt[kGMaxTable];
    __shared__ uint32_t pos[kGMaxTable];
    __shared__ uint32_t sid[kGMaxAssign];
    __shared__ uint32_t wtot[2][4];
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    for (uint32_t e = tid; e < n_table; e += 256) cnt[e] = 0;
    for (uint32_t a = tid; a < n_assign; a += 256) sid[a] = ids[a];
    __syncthreads();
    bool bad = false;
    for (uint32_t a = tid; a < n_assign; a += 256) {
        if (sid[a] < n_table) atomicAdd(&cnt[sid[a]], 1u);
        else bad = true;
    }
    if (bad) atomicOr(err, 1u);
    __syncthreads();
    // exclusive prefix over experts of the counts (positions) and of the non-empty
    // flags (group numbers); thread t owns experts [t*per, (t+1)*per)
    const uint32_t per = (n_table + 255) / 256;
    const uint32_t e0 = tid * per < n_table ? tid * per : n_table;
    const uint32_t e1 = e0 + per < n_table ? e0 + per : n_table;
    uint32_t sc = 0, sg = 0;
    for (uint32_t e = e0; e < e1; ++e) {
        sc += cnt[e];
        sg += cnt[e] ? 1u : 0u;
    }
    uint32_t ic = sc, ig = sg;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const uint32_t oc = __shfl_up(ic, off, 64), og = __shfl_up(ig, off, 64);
        if (static_cast<int>(lane) >= off) {
            ic += oc;
            ig += og;
        }
    }
    if (lane == 63) {
        wtot[0][wave] = ic;
        wtot[1][wave] = ig;
    }
    __syncthreads();
    uint32_t bc = 0, bg = 0, tc = 0, tg = 0;
    for (uint32_t v = 0; v < 4; ++v) {
        if (v < wave) {
            bc += wtot[0][v];
            bg += wtot[1][v];
        }
        tc += wtot[0][v];
        tg += wtot[1][v];
    }
    uint32_t pc = bc + ic - sc, pg = bg + ig - sg;
    for (uint32_t e = e0; e < e1; ++e) {
        if (cnt[e]) {
            w.grp_expert[pg] = e;
            w.grp_start[pg] = pc;
            pos[e] = pc;
            pc += cnt[e];
            ++pg;
        }
    }
    if (tid == 0) {
        w.hdr[0] = tg;
        w.grp_start[tg] = tc;
    }
    __syncthreads();
    // stable order inside a group: rank among the earlier assignments of the expert
    for (uint32_t a = tid; a < n_assign; a += 256) {
        const uint32_t e = sid[a];
        if (e >= n_table) continue;
        uint32_t r = 0;
        for (uint32_t b = 0; b < a; ++b) r += sid[b] == e ? 1u : 0u;
        w.alist[pos[e] + r] = a;
    }
}

// ------------------------------------------------------------- split rows
// One workgroup per row: scale = 2^s with |x 2^s| < 2^14, then hi = fp16(x 2^s),
// lo = fp16(x 2^s - hi), stored in the (w0,w4),(w1,w5),.. order of each group of
// 8; mult[row] = 2^-s restores the products. A non-finite row keeps s = 0 (its
// infinities and NaNs propagate).
__global__ __launch_bounds__(256) void moe_split_kernel(const float* __restrict__ src, uint32_t cols,
                                                        _Float16* __restrict__ hi, _Float16* __restrict__ lo,
                                                        float* __restrict__ mult) {
    __shared__ float red[4];
    const uint32_t row = blockIdx.x;
    const float* x = src + static_cast<size_t>(row) * cols;
    float m = 0.0f;
    bool finite = true;
    for (uint32_t c = threadIdx.x; c < cols; c += 256) {
        const float v = x[c];
        finite = finite && __builtin_isfinite(v);
        m = fmaxf(m, fabsf(v));
    }
    if (!finite) m = __builtin_inff();
    for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    int s = 0;
    if (m > 0.0f && __builtin_isfinite(m)) {
        int ex;
        (void)frexpf(m, &ex);  // m < 2^ex
        s = 14 - ex;
        s = s > 100 ? 100 : (s < -100 ? -100 : s);
    }
    if (threadIdx.x == 0) mult[row] = ldexpf(1.0f, -s);
    _Float16* h = hi + static_cast<size_t>(row) * cols;
    _Float16* l = lo + static_cast<size_t>(row) * cols;
    for (uint32_t g = threadIdx.x; g < cols / 8; g += 256) {
        const float4 a = *reinterpret_cast<const float4*>(x + 8 * g);
        const float4 b = *reinterpret_cast<const float4*>(x + 8 * g + 4);
        const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
        half8 vh, vl;
#pragma unroll
        for (int d = 0; d < 8; ++d) {
            const float xs = ldexpf(v[kPerm[d]], s);
            const _Float16 th = static_cast<_Float16>(xs);
            vh[d] = th;
            vl[d] = static_cast<_Float16>(xs - static_cast<float>(th));
        }
        *reinterpret_cast<half8*>(h + 8 * g) = vh;
        *reinterpret_cast<half8*>(l + 8 * g) = vl;
    }
}

// ------------------------------------------------------ weights -> B operand
// The lane's 8 weights (k group kg of block blk of its pair d) as fp16 exact
// values in the (w0,w4),(w1,w5),(w2,w6),(w3,w7) order, and the block's scale
// (times the format's constant). kg is lane-dependent: registers are picked with
// selects, never indexed.
__device__ __forceinline__ uint32_t pick4(uint32_t kg, uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    const uint32_t lo = (kg & 1) ? b : a, hi = (kg & 1) ? d : c;
    return (kg & 2) ? hi : lo;
}

__device__ __forceinline__ half8 pack8(h2 a, h2 b, h2 c, h2 d) {
    half8 r;
    r[0] = a.x; r[1] = a.y; r[2] = b.x; r[3] = b.y;
    r[4] = c.x; r[5] = c.y; r[6] = d.x; r[7] = d.y;
    return r;
}

// nibble dword n (weights 2m, 2m+1 in byte m), optional 5th bits m8 (bit i: weight i)
template <bool Q5>
__device__ __forceinline__ half8 nibbles_to_b(uint32_t n, uint32_t m8) {
    const uint32_t magic = 0x64006400u;
    const uint32_t n8 = n >> 8;
    const _Float16 blo = Q5 ? (_Float16)1040.0f : (_Float16)1032.0f;  // 1024 + zero point
    const _Float16 bhi = Q5 ? (_Float16)-80.0f : (_Float16)-72.0f;    // 64 + zero point
    const h2 klo = {blo, blo}, khi = {bhi, bhi}, k16 = {(_Float16)0.0625f, (_Float16)0.0625f};
    uint32_t sa = 0, sb = 0, sc = 0, sd = 0;
    if constexpr (Q5) {
        sa = ((m8 & 0x11u) * 0x10010u) & 0x00100010u;
        sb = ((m8 & 0x22u) * 0x80080u) & 0x01000100u;
        sc = ((m8 & 0x44u) * 0x04004u) & 0x00100010u;
        sd = ((m8 & 0x88u) * 0x20020u) & 0x01000100u;
    }
    const h2 a = as_h2((n & 0x000F000Fu) | sa | magic) - klo;
    const h2 b = as_h2((n & 0x00F000F0u) | sb | magic) * k16 + khi;
    const h2 c = as_h2((n8 & 0x000F000Fu) | sc | magic) - klo;
    const h2 d = as_h2((n8 & 0x00F000F0u) | sd | magic) * k16 + khi;
    return pack8(a, b, c, d);
}

template <class R>
struct LaneBlock;

template <int F>
struct LaneBlock<QRows<F>> {
    static __device__ __forceinline__ half8 get(const uint32_t (&d)[Fmt<F>::kPairDw], int blk, uint32_t kg,
                                                float& scale) {
        if constexpr (F == kQ4) {
            // bytes 0-1 scale0, 2-17 nibbles0, 18-19 scale1, 20-35 nibbles1
            if (blk == 0) {
                scale = f16_to_f32(d[0] & 0xFFFFu);
                const uint32_t n = pick4(kg, alignb(d[1], d[0], 2), alignb(d[2], d[1], 2), alignb(d[3], d[2], 2),
                                         alignb(d[4], d[3], 2));
                return nibbles_to_b<false>(n, 0);
            }
            scale = f16_to_f32(d[4] >> 16);
            return nibbles_to_b<false>(pick4(kg, d[5], d[6], d[7], d[8]), 0);
        } else if constexpr (F == kQ5) {
            // bytes 0-1 scale0, 2-5 mask0, 6-21 nibbles0, 22-23 scale1, 24-27 mask1, 28-43 nibbles1
            if (blk == 0) {
                scale = f16_to_f32(d[0] & 0xFFFFu);
                const uint32_t m = (alignb(d[1], d[0], 2) >> (8 * kg)) & 0xFFu;
                const uint32_t n = pick4(kg, alignb(d[2], d[1], 2), alignb(d[3], d[2], 2), alignb(d[4], d[3], 2),
                                         alignb(d[5], d[4], 2));
                return nibbles_to_b<true>(n, m);
            }
            scale = f16_to_f32(d[5] >> 16);
            return nibbles_to_b<true>(pick4(kg, d[7], d[8], d[9], d[10]), (d[6] >> (8 * kg)) & 0xFFu);
        } else {
            // bytes 0-1 scale0, 2-9 lows0, 10-13 highs0, 14-15 scale1, 16-23 lows1, 24-27 highs1
            uint32_t l0, l1, hb;
            if (blk == 0) {
                scale = f16_to_f32(d[0] & 0xFFFFu);
                l0 = alignb(d[1], d[0], 2);
                l1 = alignb(d[2], d[1], 2);
                hb = alignb(d[3], d[2], 2);
            } else {
                scale = f16_to_f32(d[3] >> 16);
                l0 = d[4];
                l1 = d[5];
                hb = d[6];
            }
            const uint32_t lo16 = ((kg & 2) ? l1 : l0) >> (16 * (kg & 1)) & 0xFFFFu;  // 2 bits per weight
            const uint32_t h8 = (hb >> (8 * kg)) & 0xFFu;                             // 1 bit per weight
            const h2 k4 = {(_Float16)1028.0f, (_Float16)1028.0f};
            h2 p[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {  // weights i and i + 4
                const uint32_t t = (lo16 >> (2 * i)) & 0x303u;
                const uint32_t hh = (h8 >> i) & 0x11u;
                const uint32_t v = (t & 3u) | ((t & 0x300u) << 8) | ((hh & 1u) << 2) | ((hh & 0x10u) << 14);
                p[i] = as_h2(v | 0x64006400u) - k4;
            }
            return pack8(p[0], p[1], p[2], p[3]);
        }
    }
};

template <>
struct LaneBlock<Fp4Rows> {
    static __device__ __forceinline__ half8 get(const uint32_t (&d)[9], int blk, uint32_t kg, float& scale) {
        scale = e8m0_to_f32((d[8] >> (8 * blk)) & 0xFFu) * 16384.0f;
        const uint32_t n = blk == 0 ? pick4(kg, d[0], d[1], d[2], d[3]) : pick4(kg, d[4], d[5], d[6], d[7]);
        // E2M1 code c -> fp16 bits ((c & 7) << 9) | ((c & 8) << 12) = value * 2^-14
        h2 p[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t t = (n >> (4 * i)) & 0x000F000Fu;
            p[i] = as_h2(((t & 0x00070007u) << 9) | ((t & 0x00080008u) << 12));
        }
        return pack8(p[0], p[1], p[2], p[3]);
    }
};

// ----------------------------------------------------------- grouped GEMMs
// Cached (not non-temporal) pair loads: the four lanes of a row read the same
// bytes and consecutive pairs share cache lines, so the lines must stay in L1/L2
// until the wave has used them.
template <class R>
struct PairLoad;
template <int F>
struct PairLoad<QRows<F>> {
    static __device__ __forceinline__ void load(const QRows<F>& m, uint32_t r, uint32_t p, uint32_t (&d)[Fmt<F>::kPairDw]) {
        const gptr<uint32_t> q = as_global(reinterpret_cast<const uint32_t*>(m.pair_ptr(r, p)));
#pragma unroll
        for (int i = 0; i < Fmt<F>::kPairDw; ++i) d[i] = q[i];
    }
};
template <>
struct PairLoad<Fp4Rows> {
    static __device__ __forceinline__ void load(const Fp4Rows& m, uint32_t r, uint32_t p, uint32_t (&d)[9]) {
        const gptr<uint32_t> q = as_global(reinterpret_cast<const uint32_t*>(m.w + static_cast<size_t>(r) * m.wrow + p * 32u));
#pragma unroll
        for (int i = 0; i < 8; ++i) d[i] = q[i];
        d[8] = *as_global(reinterpret_cast<const uint16_t*>(m.s + static_cast<size_t>(r) * m.srow + p * 2u));
    }
};

constexpr int kGPairs = 1;  // pairs per wave per step (more in flight measured slower: registers)

// grid = (ceil(rows / 16), max groups), 4 waves: the workgroup owns output rows
// [16 blockIdx.x, +16) of the group's expert and wave w the w-th quarter of the
// pairs (k split); the four partial sums meet in LDS. 8 group members per MFMA
// column set. GATEUP: rows = inter over x (cols = hidden), writes act; else
// rows = out_dim over act (cols = inter), writes part.
template <class R, bool GATEUP>
__global__ __launch_bounds__(256) void moe_grouped_kernel(
    const objeta_hip_expert_ptrs* __restrict__ table, GroupWs gw, const _Float16* __restrict__ vh,
    const _Float16* __restrict__ vl, const float* __restrict__ vmult, float* __restrict__ out, uint32_t cols,
    uint32_t rows, uint32_t k, float limit) {
    __shared__ f32x4 red[GATEUP ? 2 : 1][3][64];
    const uint32_t g = blockIdx.y;
    if (g >= gw.hdr[0]) return;
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t row = blockIdx.x * 16 + (lane & 15), kg = lane >> 4;
    const uint32_t rc = row < rows ? row : rows - 1;
    const uint32_t e = gw.grp_expert[g];
    const uint32_t s0 = gw.grp_start[g], m = gw.grp_start[g + 1] - s0;
    const objeta_hip_expert_ptrs P = table[e];
    const R w0 = GATEUP ? RowsOf<R>::make(P.gate, P.gate_scale, cols) : RowsOf<R>::make(P.down, P.down_scale, cols);
    const R w1 = RowsOf<R>::make(P.up, P.up_scale, cols);
    const uint32_t pairs = cols >> 6;
    const uint32_t ppw = (pairs + 3) / 4;
    const uint32_t p0 = wave * ppw < pairs ? wave * ppw : pairs;
    const uint32_t p1 = p0 + ppw < pairs ? p0 + ppw : pairs;
    for (uint32_t c0 = 0; c0 < m; c0 += 8) {
        // A operand: member c0 + (lane&15)/2 of the group, part (lane&1)
        const uint32_t jm = c0 + ((lane & 15) >> 1);
        const uint32_t am = gw.alist[s0 + (jm < m ? jm : m - 1)];
        const uint32_t vrow = GATEUP ? am / k : am;  // token row of x, or the assignment's act row
        const gptr<half8> src = as_global(reinterpret_cast<const half8*>(
            ((lane & 1) ? vl : vh) + static_cast<size_t>(vrow) * cols + 8 * kg));
        f32x4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
        for (uint32_t pb = p0; pb < p1; pb += kGPairs) {
            uint32_t d0[kGPairs][R::kDw], d1[kGPairs][R::kDw];
            half8 xa[kGPairs][2];
#pragma unroll
            for (int i = 0; i < kGPairs; ++i) {
                const uint32_t p = pb + i < p1 ? pb + i : p1 - 1;
                PairLoad<R>::load(w0, rc, p, d0[i]);
                if constexpr (GATEUP) PairLoad<R>::load(w1, rc, p, d1[i]);
                xa[i][0] = src[8 * p];  // half8 units: 64 halves per pair
                xa[i][1] = src[8 * p + 4];
            }
            // every load of the batch is in flight before the first product; pairs
            // past p1 (clamped copies) are computed and dropped, so the batch has no
            // branch for the scheduler to sink loads into
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < kGPairs; ++i) {
                const bool use = pb + i < p1;
#pragma unroll
                for (int blk = 0; blk < 2; ++blk) {
                    const f32x4 z = {0.f, 0.f, 0.f, 0.f};
                    float sc0;
                    const half8 b0 = LaneBlock<R>::get(d0[i], blk, kg, sc0);
                    const f32x4 r0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[i][blk], b0, z, 0, 0, 0);
#pragma unroll
                    for (int q = 0; q < 4; ++q) acc0[q] = use ? __builtin_fmaf(sc0, r0[q], acc0[q]) : acc0[q];
                    if constexpr (GATEUP) {
                        float sc1;
                        const half8 b1 = LaneBlock<R>::get(d1[i], blk, kg, sc1);
                        const f32x4 r1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[i][blk], b1, z, 0, 0, 0);
#pragma unroll
                        for (int q = 0; q < 4; ++q) acc1[q] = use ? __builtin_fmaf(sc1, r1[q], acc1[q]) : acc1[q];
                    }
                }
            }
        }
        // the four waves' partial sums (same lane layout) meet in LDS; wave 0 adds
        if (wave > 0) {
            red[0][wave - 1][lane] = acc0;
            if constexpr (GATEUP) red[GATEUP ? 1 : 0][wave - 1][lane] = acc1;
        }
        __syncthreads();
        if (wave == 0) {
#pragma unroll
            for (int v = 0; v < 3; ++v) {
                acc0 += red[0][v][lane];
                if constexpr (GATEUP) acc1 += red[GATEUP ? 1 : 0][v][lane];
            }
            // lane: output row `row`, members c0 + 2kg + q (q = 0, 1) as (hi, lo) in 2q, 2q+1
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                const uint32_t j = c0 + 2 * kg + static_cast<uint32_t>(q);
                if (j < m && row < rows) {
                    const uint32_t a = gw.alist[s0 + j];
                    const float mul = vmult[GATEUP ? a / k : a];
                    const float v0 = (acc0[2 * q] + acc0[2 * q + 1]) * mul;
                    if constexpr (GATEUP) {
                        const float v1 = (acc1[2 * q] + acc1[2 * q + 1]) * mul;
                        float gv = v0, uv = v1;
                        if (limit > 0.0f) {
                            uv = fminf(limit, fmaxf(-limit, uv));
                            gv = fminf(limit, gv);
                        }
                        out[static_cast<size_t>(a) * rows + row] = (gv / (1.0f + expf(-gv))) * uv;
                    } else {
                        out[static_cast<size_t>(a) * rows + row] = v0;
                    }
                }
            }
        }
        __syncthreads();  // red is reused by the next member set
    }
}

// out[t][r] = residual[t][r] + sum_j w[t][j] * part[t*k + j][r], slots in order; an
// out-of-table id makes the element NaN (the id was reported by the grouping).
__global__ __launch_bounds__(256) void moe_combine_kernel(const uint32_t* __restrict__ ids, const float* __restrict__ wts,
                                                          const float* __restrict__ part, const float* resid, float* out,
                                                          uint32_t k, uint32_t out_dim, uint32_t n_table) {
    const uint32_t t = blockIdx.y;
    const uint32_t r = blockIdx.x * 256 + threadIdx.x;
    if (r >= out_dim) return;
    float acc = resid ? resid[static_cast<size_t>(t) * out_dim + r] : 0.0f;
    for (uint32_t j = 0; j < k; ++j) {
        const uint32_t a = t * k + j;
        const float v = ids[a] < n_table ? part[static_cast<size_t>(a) * out_dim + r] : __builtin_nanf("");
        acc = __builtin_fmaf(wts[a], v, acc);
    }
    out[static_cast<size_t>(t) * out_dim + r] = acc;
}

size_t align256(size_t v) { return (v + 255) & ~size_t(255); }

template <class R>
hipError_t launch_grouped(hipStream_t s, const objeta_hip_expert_ptrs* table, GroupWs gw, const _Float16* xh,
                          const _Float16* xl, const float* xmult, float* act, _Float16* ah, _Float16* al,
                          float* amult, float* part, uint32_t n_assign, uint32_t max_groups, uint32_t k,
                          uint32_t hidden, uint32_t inter, uint32_t out_dim, float limit) {
    hipLaunchKernelGGL((moe_grouped_kernel<R, true>), dim3((inter + 15) / 16, max_groups), dim3(256), 0, s, table, gw,
                       xh, xl, xmult, act, hidden, inter, k, limit);
    hipLaunchKernelGGL(moe_split_kernel, dim3(n_assign), dim3(256), 0, s, act, inter, ah, al, amult);
    hipLaunchKernelGGL((moe_grouped_kernel<R, false>), dim3((out_dim + 15) / 16, max_groups), dim3(256), 0, s, table,
                       gw, ah, al, amult, part, inter, out_dim, k, 0.0f);
    return hipGetLastError();
}

}  // namespace

int32_t launch_moe_grouped(objeta_hip_context* ctx, int32_t format, hipStream_t s, const objeta_hip_expert_ptrs* table,
                           uint64_t n_table, const uint32_t* ids, const float* wts, uint64_t n_tokens, uint64_t k,
                           const float* x, const float* resid, float* out, uint64_t hidden, uint64_t inter,
                           uint64_t out_dim, float limit) {
    const char* action = "launch grouped-token MoE";
    if (format < OBJETA_HIP_Q4_0 || format > OBJETA_HIP_FP4_E2M1)
        OBJ_FAIL(kInvalidInput, action, strf("unknown format %d", format));
    if (n_tokens == 0 || out_dim == 0) return 0;
    if (k == 0 || k > 32) OBJ_FAIL(kInvalidInput, action, "k must be in 1..=32");
    if (n_table == 0 || n_table > kGMaxTable)
        OBJ_FAIL(kUnsupported, action, strf("the grouped path takes up to %u experts", kGMaxTable));
    if (n_tokens * k > kGMaxAssign)
        OBJ_FAIL(kUnsupported, action, strf("the grouped path takes up to %u (token, slot) assignments", kGMaxAssign));
    if (hidden == 0 || inter == 0 || hidden % 64 || inter % 64 || hidden > (1u << 20) || inter > (1u << 20) ||
        out_dim > (1u << 20))
        OBJ_FAIL(kUnsupported, action, "hidden and intermediate must be non-zero multiples of 64 (<= 2^20)");
    if (!table || !ids || !wts || !x || !out) OBJ_FAIL(kInvalidInput, action, "NULL device pointer");
    if (reinterpret_cast<uintptr_t>(x) % 16) OBJ_FAIL(kInvalidInput, action, "x must be 16-byte aligned");
    const uint32_t A = static_cast<uint32_t>(n_tokens * k), T = static_cast<uint32_t>(n_tokens);
    const uint32_t H = static_cast<uint32_t>(hidden), I = static_cast<uint32_t>(inter), O = static_cast<uint32_t>(out_dim);
    // workspace: group lists, split x, act, split act, per-assignment down rows
    size_t off = 0;
    const size_t o_hdr = off; off += align256(16);
    const size_t o_ge = off; off += align256(4ull * A);
    const size_t o_gs = off; off += align256(4ull * (A + 1));
    const size_t o_al = off; off += align256(4ull * A);
    const size_t o_xm = off; off += align256(4ull * T);
    const size_t o_am = off; off += align256(4ull * A);
    const size_t o_xh = off; off += align256(2ull * T * H);
    const size_t o_xl = off; off += align256(2ull * T * H);
    const size_t o_act = off; off += align256(4ull * A * I);
    const size_t o_ah = off; off += align256(2ull * A * I);
    const size_t o_all = off; off += align256(2ull * A * I);
    const size_t o_part = off; off += align256(4ull * A * O);
    void* wsp = nullptr;
    OBJ_TRY(ensure_workspace(ctx, s, kWsGrouped, off, &wsp));
    char* b = static_cast<char*>(wsp);
    GroupWs gw{reinterpret_cast<uint32_t*>(b + o_hdr), reinterpret_cast<uint32_t*>(b + o_ge),
               reinterpret_cast<uint32_t*>(b + o_gs), reinterpret_cast<uint32_t*>(b + o_al)};
    float* xmult = reinterpret_cast<float*>(b + o_xm);
    float* amult = reinterpret_cast<float*>(b + o_am);
    auto* xh = reinterpret_cast<_Float16*>(b + o_xh);
    auto* xl = reinterpret_cast<_Float16*>(b + o_xl);
    float* act = reinterpret_cast<float*>(b + o_act);
    auto* ah = reinterpret_cast<_Float16*>(b + o_ah);
    auto* al = reinterpret_cast<_Float16*>(b + o_all);
    float* part = reinterpret_cast<float*>(b + o_part);
    uint32_t* err = ctx->err_word;
    const uint32_t max_groups = A < n_table ? A : static_cast<uint32_t>(n_table);
    hipLaunchKernelGGL(moe_group_kernel, dim3(1), dim3(256), 0, s, ids, A, static_cast<uint32_t>(n_table), gw, err);
    hipLaunchKernelGGL(moe_split_kernel, dim3(T), dim3(256), 0, s, x, H, xh, xl, xmult);
    hipError_t e;
    const uint32_t kk = static_cast<uint32_t>(k);
    switch (format) {
        case OBJETA_HIP_Q4_0:
            e = launch_grouped<QRows<kQ4>>(s, table, gw, xh, xl, xmult, act, ah, al, amult, part, A, max_groups, kk, H,
                                           I, O, limit);
            break;
        case OBJETA_HIP_Q5_0:
            e = launch_grouped<QRows<kQ5>>(s, table, gw, xh, xl, xmult, act, ah, al, amult, part, A, max_groups, kk, H,
                                           I, O, limit);
            break;
        case OBJETA_HIP_IQ3_0:
            e = launch_grouped<QRows<kIQ3>>(s, table, gw, xh, xl, xmult, act, ah, al, amult, part, A, max_groups, kk,
                                            H, I, O, limit);
            break;
        default:
            e = launch_grouped<Fp4Rows>(s, table, gw, xh, xl, xmult, act, ah, al, amult, part, A, max_groups, kk, H, I,
                                        O, limit);
            break;
    }
    if (e == hipSuccess) {
        hipLaunchKernelGGL(moe_combine_kernel, dim3((O + 255) / 256, T), dim3(256), 0, s, ids, wts, part, resid, out, kk,
                           O, static_cast<uint32_t>(n_table));
        e = hipGetLastError();
    }
    if (e != hipSuccess) OBJ_FAIL(kDriver, action, hipGetErrorString(e));
    return 0;
}

}  // namespace objeta

using namespace objeta;

extern "C" int32_t objeta_hip_moe_grouped_device(objeta_hip_context* ctx, int32_t format, objeta_hip_stream stream,
                                                 const objeta_hip_expert_ptrs* d_table, uint64_t n_table,
                                                 const uint32_t* d_ids, const float* d_weights, uint64_t n_tokens,
                                                 uint64_t k, const float* d_x, const float* d_residual, float* d_out,
                                                 uint64_t hidden, uint64_t intermediate, uint64_t out_dim,
                                                 float swiglu_limit) {
    OBJ_GUARD_BEGIN
    OBJ_TRY(check_ctx(ctx, "moe_grouped_device"));
    OBJ_HIP(hipSetDevice(ctx->device), "hipSetDevice");
    return launch_moe_grouped(ctx, format, resolve_stream(ctx, stream), d_table, n_table, d_ids, d_weights, n_tokens,
                              k, d_x, d_residual, d_out, hidden, intermediate, out_dim, swiglu_limit);
    OBJ_GUARD_END
}
