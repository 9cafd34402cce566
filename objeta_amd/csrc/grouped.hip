// grouped.hip — the grouped-token expert product on gfx950 matrix cores.
//
// With a batch of tokens, the per-(token, slot) kernels of moe.hip stream an
// expert's matrices once per assignment that selected it. Here the assignments
// are grouped by expert on the device and each selected expert's gate, up and
// down matrices are read once for all of its tokens, the products running on
// MFMA (v_mfma_f32_16x16x32_f16). Per layer:
//
//   moe_prepare_kernel   assignments (token, slot) sorted by expert, stable, cut
//                        into sets of up to 8 per expert; and each token's
//                        activation row -> two fp16 parts (see below)
//   moe_grouped_kernel   per (set, 16 rows): silu(gate x) * (up x) for the set
//   moe_split_kernel     the activations of every assignment
//   moe_grouped_kernel   per (set, 16 rows): down act for every assignment
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
// Layout trick: within each 8-element k group the weights of the block formats come
// out of the nibble unpacking as (w0,w4),(w1,w5),(w2,w6),(w3,w7); for them the split
// activations are stored in that same order, so no unpacking shuffle is needed (a k
// permutation applied to both operands leaves the products unchanged). FP4 (the
// hardware conversion's pairs) and FP8 weights come in element order, and so do
// their split activations.
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
#include "quant_rules.hpp"
#include "swiglu.hpp"

namespace objeta {
namespace {

using namespace dev;

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr uint32_t kGMaxTable = 1024;   // experts per table
constexpr uint32_t kGMaxAssign = 1024;  // tokens * k per call
constexpr uint32_t kPerm[8] = {0, 4, 1, 5, 2, 6, 3, 7};

// One work item of the grouped products: up to 8 assignments (token, slot) that
// selected the same expert, with that expert's table entry copied in, so a
// workgroup reaches its weights and activations through one load.
struct SetRec {
    objeta_hip_expert_ptrs p;
    uint16_t mem[8];  // act rows: assignments t*k + j (in order), or n_assign + t for the
                      // shared expert; unused slots repeat the last; mem[0] bits
                      // 12..15 hold the member count - 1
};
static_assert(sizeof(SetRec) == 64, "one 64-byte record per set");

struct GroupWs {
    uint32_t* hdr;  // [0] number of groups, [1] number of member sets
    SetRec* sets;   // [A] (a set holds at least one assignment)
};

// The power of two 2^s that brings a row of maximum magnitude m below 2^14 (s = 0
// for a zero or non-finite row).
__device__ __forceinline__ int split_shift(float m) {
    int s = 0;
    if (m > 0.0f && __builtin_isfinite(m)) {
        int ex;
        (void)frexpf(m, &ex);  // m < 2^ex
        s = 14 - ex;
        s = s > 100 ? 100 : (s < -100 ? -100 : s);
    }
    return s;
}

// ------------------------------------------------------------------ grouping
// The shared expert (when given) follows as one more group: member t is token t,
// its act row n_assign + t. Its member sets go after the routed ones in w, or, when
// wsh.hdr is set (a shared expert of another format, multiplied by a launch of its
// own), into wsh.
__device__ void group_assignments(const uint32_t* __restrict__ ids, uint32_t n_assign, uint32_t n_table,
                                  const objeta_hip_expert_ptrs* __restrict__ table,
                                  const objeta_hip_expert_ptrs* __restrict__ shared, uint32_t n_tokens, GroupWs w,
                                  GroupWs wsh, uint32_t* __restrict__ err) {
    __shared__ uint32_t cnt[kGMaxTable];
    __shared__ uint32_t pos[kGMaxTable];
    __shared__ uint32_t sid[kGMaxAssign];
    __shared__ uint32_t sal[kGMaxAssign];   // assignments grouped by expert
    __shared__ uint32_t sinfo[kGMaxAssign];  // set: expert | first member << 11 | (count - 1) << 22
    __shared__ uint32_t wtot[3][4];
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
    // exclusive prefix over experts of the counts (positions), of the non-empty
    // flags (group numbers) and of the member sets; thread t owns experts
    // [t*per, (t+1)*per)
    const uint32_t per = (n_table + 255) / 256;
    const uint32_t e0 = tid * per < n_table ? tid * per : n_table;
    const uint32_t e1 = e0 + per < n_table ? e0 + per : n_table;
    uint32_t sc = 0, sg = 0, ss = 0;
    for (uint32_t e = e0; e < e1; ++e) {
        sc += cnt[e];
        sg += cnt[e] ? 1u : 0u;
        ss += (cnt[e] + 7) / 8;
    }
    uint32_t ic = sc, ig = sg, is = ss;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const uint32_t oc = __shfl_up(ic, off, 64), og = __shfl_up(ig, off, 64), os = __shfl_up(is, off, 64);
        if (static_cast<int>(lane) >= off) {
            ic += oc;
            ig += og;
            is += os;
        }
    }
    if (lane == 63) {
        wtot[0][wave] = ic;
        wtot[1][wave] = ig;
        wtot[2][wave] = is;
    }
    __syncthreads();
    uint32_t bc = 0, bs = 0, tg = 0, ts = 0;
    for (uint32_t v = 0; v < 4; ++v) {
        if (v < wave) {
            bc += wtot[0][v];
            bs += wtot[2][v];
        }
        tg += wtot[1][v];
        ts += wtot[2][v];
    }
    uint32_t pc = bc + ic - sc, ps = bs + is - ss;
    for (uint32_t e = e0; e < e1; ++e) {
        if (cnt[e]) {
            pos[e] = pc;
            for (uint32_t j = 0; j < cnt[e]; j += 8) {
                const uint32_t m = cnt[e] - j < 8 ? cnt[e] - j : 8;
                sinfo[ps++] = e | ((pc + j) << 11) | ((m - 1) << 22);
            }
            pc += cnt[e];
        }
    }
    const uint32_t n_sh = shared ? (n_tokens + 7) / 8 : 0;
    const bool apart = wsh.hdr != nullptr;
    if (tid == 0) {
        w.hdr[0] = tg + (shared && !apart ? 1 : 0);
        w.hdr[1] = ts + (apart ? 0 : n_sh);
        if (apart) {
            wsh.hdr[0] = shared ? 1 : 0;
            wsh.hdr[1] = n_sh;
        }
    }
    __syncthreads();
    // stable order inside a group: rank among the earlier assignments of the expert
    for (uint32_t a = tid; a < n_assign; a += 256) {
        const uint32_t e = sid[a];
        if (e >= n_table) continue;
        uint32_t r = 0;
        for (uint32_t b = 0; b < a; ++b) r += sid[b] == e ? 1u : 0u;
        sal[pos[e] + r] = a;
    }
    __syncthreads();
    for (uint32_t si = tid; si < ts + n_sh; si += 256) {
        // the record: the expert's table entry, then 8 uint16 act rows (4 dwords),
        // written field by field (a record assembled in a local lands in scratch)
        const objeta_hip_expert_ptrs* src;
        uint32_t first, m1;
        if (si < ts) {
            const uint32_t info = sinfo[si];
            src = table + (info & 0x7FFu);
            first = (info >> 11) & 0x7FFu;
            m1 = info >> 22;
        } else {
            const uint32_t t0 = 8 * (si - ts);
            src = shared;
            first = t0;
            m1 = (n_tokens - t0 < 8 ? n_tokens - t0 : 8) - 1;
        }
        auto row = [&](uint32_t j) {
            const uint32_t jj = j < m1 ? j : m1;
            return si < ts ? sal[first + jj] : n_assign + first + jj;
        };
        uint4 mem;
        mem.x = (row(0) | (m1 << 12)) | (row(1) << 16);
        mem.y = row(2) | (row(3) << 16);
        mem.z = row(4) | (row(5) << 16);
        mem.w = row(6) | (row(7) << 16);
        SetRec* dst = si >= ts && apart ? &wsh.sets[si - ts] : &w.sets[si];
        dst->p = *src;
        *reinterpret_cast<uint4*>(dst->mem) = mem;
    }
}

// ------------------------------------------------------------- split rows
// One workgroup per row: scale = 2^s with |x 2^s| < 2^14, then hi = fp16(x 2^s),
// lo = fp16(x 2^s - hi), stored in the (w0,w4),(w1,w5),.. order of each group of
// 8 when perm is set, else in element order; mult[row] = 2^-s restores the
// products. A non-finite row keeps s = 0 (its infinities and NaNs propagate).
__device__ void split_row(const float* __restrict__ src, uint32_t cols, _Float16* __restrict__ hi,
                          _Float16* __restrict__ lo, float* __restrict__ mult, uint32_t row, uint32_t perm) {
    __shared__ float red[4];
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
    const int s = split_shift(m);
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
            const float xs = ldexpf(v[perm ? kPerm[d] : d], s);
            const _Float16 th = static_cast<_Float16>(xs);
            vh[d] = th;
            vl[d] = static_cast<_Float16>(xs - static_cast<float>(th));
        }
        *reinterpret_cast<half8*>(h + 8 * g) = vh;
        *reinterpret_cast<half8*>(l + 8 * g) = vl;
    }
}

// Block 0 groups the assignments; block 1 + t splits row t of x.
__global__ __launch_bounds__(256) void moe_prepare_kernel(const uint32_t* __restrict__ ids, uint32_t n_assign,
                                                          uint32_t n_table,
                                                          const objeta_hip_expert_ptrs* __restrict__ table,
                                                          const objeta_hip_expert_ptrs* __restrict__ shared,
                                                          uint32_t n_tokens, GroupWs w, GroupWs wsh,
                                                          uint32_t* __restrict__ err, const float* __restrict__ x,
                                                          uint32_t cols, _Float16* __restrict__ xh,
                                                          _Float16* __restrict__ xl, float* __restrict__ xmult,
                                                          uint32_t perm) {
    if (blockIdx.x == 0) group_assignments(ids, n_assign, n_table, table, shared, n_tokens, w, wsh, err);
    else split_row(x, cols, xh, xl, xmult, blockIdx.x - 1, perm);
}

// One workgroup per row.
__global__ __launch_bounds__(256) void moe_split_kernel(const float* __restrict__ src, uint32_t cols,
                                                        _Float16* __restrict__ hi, _Float16* __restrict__ lo,
                                                        float* __restrict__ mult, uint32_t perm) {
    split_row(src, cols, hi, lo, mult, blockIdx.x, perm);
}


// ------------------------------------------------------ weights -> B operand
// A lane's 8 weights of one block as exact fp16 values in the (w0,w4),(w1,w5),
// (w2,w6),(w3,w7) order of the split activations.
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

// IQ3_0: 2-bit lows lo16 (weights 8kg .. 8kg+7) and 1-bit highs h8 -> the 8 weights
// q - 4 as exact fp16 in the (w0,w4),(w1,w5),.. order.
__device__ __forceinline__ half8 iq3_to_b(uint32_t lo16, uint32_t h8) {
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

// ----------------------------------------------------------- grouped GEMMs
// A workgroup streams a 16-row slab of one group's expert (gate and up together,
// or down) through LDS in chunks of Tile<R>::kChunkGU / kChunkDn columns, double-buffered: while its
// four waves multiply chunk c (wave w: the w-th quarter of the chunk's blocks), the
// loads of chunk c+1 (every thread's share, 64-byte runs within rows) and the next
// activation operands are already in flight. Each lane takes its MFMA operand (8
// weights of one output row) and the block scale from LDS; the four waves' partial
// sums meet in LDS at the end. 8 group members per MFMA column set; the member
// sets of all groups are separate work items (a larger group's sets stream the slab
// in parallel workgroups).
constexpr uint32_t kSlab = 16;      // rows per workgroup (one MFMA tile)

// Staged row segments of a 16-row slab: weights (and, for the split FP4 layout,
// the E8M0 scales) of columns [c0, c0 + kc), row stride padded by one dword so the
// lanes of different rows read different banks. kChunkGU / kChunkDn: columns per
// staged chunk for gate and up together / for down (16 and 8 blocks of 32 for the
// block formats, 16 and 16 for split FP4: the widths that measured fastest, as
// narrower chunks keep more workgroups resident; 8 blocks of FP8 bytes fill the
// same LDS). kTileScale: one
// E8M0 byte per 128 x 128 tile (FP8), taken per chunk into a register by
// tile_scales instead of being staged per row.
template <class R>
struct Tile;

template <int F>
struct Tile<QRows<F>> {
    static constexpr int kBB = Fmt<F>::kBlockBytes;
    static constexpr bool kPermuted = true;  // weights in the (w0,w4),(w1,w5),.. order
    static constexpr bool kScales = false;
    static constexpr bool kTileScale = false;
    static constexpr uint32_t kChunkGU = 512, kChunkDn = 256;
    static constexpr __host__ __device__ uint32_t wdw(uint32_t kc) { return kc / 32 * kBB / 4; }  // dwords per row segment
    static constexpr __host__ __device__ uint32_t sdw(uint32_t) { return 0; }
    static constexpr __host__ __device__ uint32_t lds_dw(uint32_t kc) { return kSlab * (wdw(kc) + 4); }
    static __device__ __forceinline__ size_t wpitch(const QRows<F>& m) { return m.row_bytes; }
    static __device__ __forceinline__ size_t spitch(const QRows<F>&) { return 0; }
    static __device__ __forceinline__ const uint8_t* wrow(const QRows<F>& m, uint32_t c0) {
        return m.q + static_cast<size_t>(c0 / 32) * kBB;
    }
    static __device__ __forceinline__ const uint8_t* srow(const QRows<F>&, uint32_t) { return nullptr; }
    static __device__ __forceinline__ uint32_t tile_scales(const QRows<F>&, uint32_t, uint32_t, uint32_t) { return 0; }
    // block b of a row (LDS row base `w`), k group kg: 8 weights and the scale
    static __device__ __forceinline__ half8 get(const uint8_t* w, const uint8_t*, uint32_t, uint32_t b, uint32_t kg,
                                                float& scale) {
        const uint8_t* blk = w + b * kBB;
        auto u16 = [&](uint32_t o) { return static_cast<uint32_t>(*reinterpret_cast<const uint16_t*>(blk + o)); };
        scale = f16_to_f32(u16(0));
        if constexpr (F == kQ4) {
            return nibbles_to_b<false>(u16(2 + 4 * kg) | (u16(4 + 4 * kg) << 16), 0);
        } else if constexpr (F == kQ5) {
            return nibbles_to_b<true>(u16(6 + 4 * kg) | (u16(8 + 4 * kg) << 16), blk[2 + kg]);
        } else {
            return iq3_to_b(u16(2 + 2 * kg), blk[10 + kg]);
        }
    }
};

template <>
struct Tile<Fp4Rows> {
    static constexpr bool kPermuted = false;
    static constexpr bool kScales = true;
    static constexpr bool kTileScale = false;
    static constexpr uint32_t kChunkGU = 512, kChunkDn = 512;
    static constexpr __host__ __device__ uint32_t wdw(uint32_t kc) { return kc / 8; }   // kc / 2 bytes
    static constexpr __host__ __device__ uint32_t sdw(uint32_t kc) { return kc / 128; }  // kc / 32 bytes (kc % 128 == 0)
    static constexpr __host__ __device__ uint32_t lds_dw(uint32_t kc) {
        return kSlab * (wdw(kc) + 4) + kSlab * (sdw(kc) + 1);
    }
    static __device__ __forceinline__ size_t wpitch(const Fp4Rows& m) { return m.wrow; }
    static __device__ __forceinline__ size_t spitch(const Fp4Rows& m) { return m.srow; }
    static __device__ __forceinline__ const uint8_t* wrow(const Fp4Rows& m, uint32_t c0) { return m.w + c0 / 2; }
    static __device__ __forceinline__ const uint8_t* srow(const Fp4Rows& m, uint32_t c0) { return m.s + c0 / 32; }
    static __device__ __forceinline__ uint32_t tile_scales(const Fp4Rows&, uint32_t, uint32_t, uint32_t) { return 0; }
    // the 8 weights in element order (the hardware conversion's pairs)
    static __device__ __forceinline__ half8 get(const uint8_t* w, const uint8_t* sc, uint32_t, uint32_t b, uint32_t kg,
                                                float& scale) {
        scale = e8m0_to_f32(sc[b]);
        const uint32_t n = *reinterpret_cast<const uint32_t*>(w + 16 * b + 4 * kg);
        h2 p[4];
        fp4_to_h2x4(n, p);
        return pack8(p[0], p[1], p[2], p[3]);
    }
};

// FP8 E4M3 rows ([rows][cols] bytes) with an E8M0 byte per 128 x 128 tile. A code
// decodes by the reference's rule (rules::f8e4m3_to_f32: exponent field 0 as
// mant * 2^-5, 15 as +-448), and every such value (|v| in [2^-5, 448] or 0) is an
// exact fp16. A 16-row slab lies inside one 128-row tile, so the chunk's scales are
// one byte per 128 columns for all of its rows.
template <>
struct Tile<Fp8Rows> {
    static constexpr bool kPermuted = false;
    static constexpr bool kScales = false;
    static constexpr bool kTileScale = true;
    static constexpr uint32_t kChunkGU = 256, kChunkDn = 256;
    static constexpr __host__ __device__ uint32_t wdw(uint32_t kc) { return kc / 4; }  // kc bytes
    static constexpr __host__ __device__ uint32_t sdw(uint32_t) { return 0; }
    static constexpr __host__ __device__ uint32_t lds_dw(uint32_t kc) { return kSlab * (wdw(kc) + 4); }
    static __device__ __forceinline__ size_t wpitch(const Fp8Rows& m) { return m.wrow; }
    static __device__ __forceinline__ size_t spitch(const Fp8Rows&) { return 0; }
    static __device__ __forceinline__ const uint8_t* wrow(const Fp8Rows& m, uint32_t c0) { return m.w + c0; }
    static __device__ __forceinline__ const uint8_t* srow(const Fp8Rows&, uint32_t) { return nullptr; }
    // the scale bytes of the tiles under columns [c0, c0 + kc) (kc <= 512) of row r0's
    // tile row, byte i for columns [c0 + 128 i, c0 + 128 i + 128); c0 % 128 == 0
    static __device__ __forceinline__ uint32_t tile_scales(const Fp8Rows& m, uint32_t r0, uint32_t c0, uint32_t kc) {
        const gptr<uint8_t> s = as_global(m.s + static_cast<size_t>(r0 >> 7) * m.scols + (c0 >> 7));
        const uint32_t n = (kc + 127) >> 7;
        uint32_t v = 0;
#pragma unroll
        for (uint32_t i = 0; i < 4; ++i)
            if (i < n) v |= static_cast<uint32_t>(s[i]) << (8 * i);
        return v;
    }
    static __device__ __forceinline__ half8 get(const uint8_t* w, const uint8_t*, uint32_t ts, uint32_t b, uint32_t kg,
                                                float& scale) {
        scale = e8m0_to_f32((ts >> (8 * (b >> 2))) & 0xFFu);
        const uint32_t d0 = *reinterpret_cast<const uint32_t*>(w + 32 * b + 8 * kg);
        const uint32_t d1 = *reinterpret_cast<const uint32_t*>(w + 32 * b + 8 * kg + 4);
        h2 p[4];  // element order
        fp8x4_to_h2x2(d0, p[0], p[1]);
        fp8x4_to_h2x2(d1, p[2], p[3]);
        return pack8(p[0], p[1], p[2], p[3]);
    }
};

// A slab's row segments of a chunk (seg dwords per row, at most kSeg) move in 16-byte
// units: unit c of a row covers dwords [min(4c, seg - 4), +4) (seg >= 4 for every
// chunk width and format), so a short last chunk reads inside its rows; thread t takes
// units t, t + 256, ... of the 16 rows in row order. Rows past `rows` read the last
// row. In LDS a row takes kSeg + 4 dwords (16-byte rows; a stride of 12 mod 64 dwords
// spreads the 16 rows x 4 k groups of an MFMA operand read over distinct banks).
template <uint32_t kSeg>
struct SlabUnits {
    static constexpr uint32_t kUpr = (kSeg + 3) / 4;                 // units per row of a full chunk
    static constexpr uint32_t kN = (kSlab * kUpr + 255) / 256;        // units per thread
    static constexpr uint32_t kStride = kSeg + 4;                      // LDS dwords per row
};
// Buffer loads over one matrix: the per-lane offsets stay in registers of their own
// from chunk to chunk (the chunk's offset is a scalar), so issuing the next chunk's
// loads never waits on registers that earlier loads still write.
// `base` is the same in every lane (a member set's matrix).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t matrix_rsrc(const void* base) {
    const uint64_t a = reinterpret_cast<uint64_t>(base);
    const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(a));
    const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(a >> 32));
    void* p = reinterpret_cast<void*>((static_cast<uint64_t>(hi) << 32) | lo);
    return __builtin_amdgcn_make_buffer_rsrc(p, 0, 0x7FFFFFFF, 0x00020000);
}
// This thread's units of a slab: row byte offsets (rows past `rows` read the last row)
// and unit indices, fixed for a member set.
template <uint32_t kSeg>
struct SlabLanes {
    uint32_t off[SlabUnits<kSeg>::kN];  // byte offset of the unit in a full chunk
    uint32_t c[SlabUnits<kSeg>::kN];    // unit index in its row (0xFFFF: none)
    __device__ __forceinline__ void init(uint32_t r0, uint32_t rows, size_t pitch) {
        using SU = SlabUnits<kSeg>;
#pragma unroll
        for (uint32_t i = 0; i < SU::kN; ++i) {
            const uint32_t u = threadIdx.x + 256u * i;
            const uint32_t rr = u / SU::kUpr;
            c[i] = rr < kSlab ? u - rr * SU::kUpr : 0xFFFFu;
            const uint32_t r = r0 + rr < rows ? r0 + rr : rows - 1;
            off[i] = static_cast<uint32_t>(static_cast<size_t>(r) * pitch) + 16u * (c[i] & 0xFFFu);
        }
    }
};
template <uint32_t kSeg, bool FULL>
__device__ __forceinline__ void slab_load4(__amdgpu_buffer_rsrc_t rs, uint32_t chunk_off, const SlabLanes<kSeg>& ln,
                                           uint32_t seg, u32x4 (&v)[SlabUnits<kSeg>::kN]) {
    using SU = SlabUnits<kSeg>;
    if (FULL || seg == kSeg) {  // a full chunk: the precomputed offsets as they are
#pragma unroll
        for (uint32_t i = 0; i < SU::kN; ++i) {
            if (SU::kN * 256u == kSlab * SU::kUpr || ln.c[i] < SU::kUpr) {
                const auto q = __builtin_amdgcn_raw_buffer_load_b128(rs, static_cast<int>(ln.off[i]),
                                                                     static_cast<int>(chunk_off), 0);
                v[i] = u32x4{q[0], q[1], q[2], q[3]};
            }
        }
        return;
    }
    const uint32_t upr = (seg + 3) / 4;
#pragma unroll
    for (uint32_t i = 0; i < SU::kN; ++i) {
        if (ln.c[i] < upr) {
            const uint32_t d = 4 * ln.c[i] < seg - 4 ? 4 * ln.c[i] : seg - 4;
            const auto q = __builtin_amdgcn_raw_buffer_load_b128(rs, static_cast<int>(ln.off[i] - 16u * ln.c[i] + 4u * d),
                                                                 static_cast<int>(chunk_off), 0);
            v[i] = u32x4{q[0], q[1], q[2], q[3]};
        }
    }
}
template <uint32_t kSeg, bool FULL>
__device__ __forceinline__ void slab_store4(uint32_t* lds, uint32_t seg, const u32x4 (&v)[SlabUnits<kSeg>::kN]) {
    using SU = SlabUnits<kSeg>;
    const uint32_t upr = (seg + 3) / 4;
#pragma unroll
    for (uint32_t i = 0; i < SU::kN; ++i) {
        const uint32_t u = threadIdx.x + 256u * i;
        const uint32_t rr = u / SU::kUpr, c = u - rr * SU::kUpr;
        if (rr < kSlab && c < upr) {
            uint32_t* dst = lds + rr * SU::kStride;
            if (FULL || seg == kSeg) {  // a full chunk: aligned 16-byte stores
                typedef uint32_t u32x4s __attribute__((ext_vector_type(4), aligned(16)));
                *reinterpret_cast<u32x4s*>(dst + 4 * c) = u32x4s{v[i].x, v[i].y, v[i].z, v[i].w};
            } else {
                const uint32_t d = 4 * c < seg - 4 ? 4 * c : seg - 4;
                dst[d] = v[i].x; dst[d + 1] = v[i].y; dst[d + 2] = v[i].z; dst[d + 3] = v[i].w;
            }
        }
    }
}
// FP4 scale rows (seg <= 16 dwords): one dword per thread, thread t row t / 16.
__device__ __forceinline__ void scale_load(const uint8_t* base, size_t pitch, uint32_t r0, uint32_t rows, uint32_t seg,
                                           uint32_t& v) {
    const uint32_t rr = threadIdx.x >> 4, c = threadIdx.x & 15;
    const uint32_t r = r0 + rr < rows ? r0 + rr : rows - 1;
    if (c < seg) v = as_global(reinterpret_cast<const uint32_t*>(base + static_cast<size_t>(r) * pitch))[c];
}
__device__ __forceinline__ void scale_store(uint32_t* lds, uint32_t stride, uint32_t seg, uint32_t v) {
    const uint32_t rr = threadIdx.x >> 4, c = threadIdx.x & 15;
    if (c < seg) lds[rr * stride + c] = v;
}

// One chunk's staged bytes of every matrix of the workgroup, in registers.
template <class R, int M, uint32_t CH>
struct Staged {
    static constexpr uint32_t kSeg = Tile<R>::wdw(CH);
    u32x4 w[M][SlabUnits<kSeg>::kN];
    uint32_t s[M];   // FP4 scales: CH / 128 <= 16 dwords per row
    uint32_t ts[M];  // FP8 tile scales of the chunk
};

// grid = (ceil(rows / 16), gy), 256 threads; workgroup (x, y) takes member sets y,
// y + gy, ... (the number of sets is known only on the device). GATEUP: rows = inter
// over the split x rows (cols = hidden), writes act (the official SwiGLU when
// `official` is set); else rows = out_dim over the split act rows (cols = inter),
// writes part. Dynamic LDS: two chunk buffers of every matrix.
template <class R, bool GATEUP, bool FULL>
__global__ __launch_bounds__(256) void moe_grouped_kernel(GroupWs gw, const _Float16* __restrict__ vh,
                                                          const _Float16* __restrict__ vl,
                                                          const float* __restrict__ vmult, float* __restrict__ out,
                                                          uint32_t cols, uint32_t rows, uint32_t k, uint32_t n_assign,
                                                          float limit, uint32_t official) {
    extern __shared__ uint32_t tl[];
    // the cross-wave partial sums reuse the chunk buffers once a set's products are done
    auto red = reinterpret_cast<f32x4 (*)[3][64]>(tl);
    constexpr int kMats = GATEUP ? 2 : 1;
    constexpr uint32_t kChunk = GATEUP ? Tile<R>::kChunkGU : Tile<R>::kChunkDn;
    constexpr int kB = kChunk / 32 / 4;  // blocks per wave and chunk
    constexpr uint32_t kSeg = Tile<R>::wdw(kChunk);           // weight dwords per row of a full chunk
    constexpr uint32_t kWStride = SlabUnits<kSeg>::kStride;    // LDS dwords per staged weight row
    constexpr uint32_t kSStride = Tile<R>::sdw(kChunk) + 1;    // LDS dwords per staged scale row (FP4)
    static_assert(Tile<R>::lds_dw(kChunk) == kSlab * kWStride + (Tile<R>::kScales ? kSlab * kSStride : 0u),
                  "LDS chunk layout");
    const uint32_t n_sets = gw.hdr[1];
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t r0 = blockIdx.x * kSlab;
    const uint32_t row = r0 + (lane & 15), kg = lane >> 4;
    const uint32_t nchunks = (cols + kChunk - 1) / kChunk;
    const uint32_t buf_dw = kMats * Tile<R>::lds_dw(kChunk);
    for (uint32_t si = blockIdx.y; si < n_sets; si += gridDim.y) {
        const SetRec sr = gw.sets[si];
        const objeta_hip_expert_ptrs& P = sr.p;
        const uint32_t m = (sr.mem[0] >> 12) + 1u;
        auto member = [&](uint32_t j) {  // assignment of member j (< 8)
            uint32_t a = sr.mem[0] & 0xFFFu;
#pragma unroll
            for (uint32_t q = 1; q < 8; ++q) a = j == q ? sr.mem[q] : a;
            return a;
        };
        R mt[kMats];
        mt[0] = GATEUP ? RowsOf<R>::make(P.gate, P.gate_scale, cols) : RowsOf<R>::make(P.down, P.down_scale, cols);
        if constexpr (GATEUP) mt[kMats - 1] = RowsOf<R>::make(P.up, P.up_scale, cols);
        const size_t wpitch = Tile<R>::wpitch(mt[0]), spitch = Tile<R>::spitch(mt[0]);
        SlabLanes<kSeg> lanes;
        lanes.init(r0, rows, wpitch);
        __amdgpu_buffer_rsrc_t rs[kMats];
#pragma unroll
        for (int t = 0; t < kMats; ++t) rs[t] = matrix_rsrc(Tile<R>::wrow(mt[t], 0));
        // A operand rows: member (lane&15)/2 of the set, part (lane&1)
        const uint32_t am = member((lane & 15) >> 1);
        // token row of x (routed or shared act row), or the act row itself
        auto xrow = [&](uint32_t a) { return a < n_assign ? a / k : a - n_assign; };
        const uint32_t vrow = GATEUP ? xrow(am) : am;
        auto stage = [&](uint32_t kc0, Staged<R, kMats, kChunk>& st) {
            const uint32_t kc = FULL ? kChunk : (cols - kc0 < kChunk ? cols - kc0 : kChunk);
#pragma unroll
            for (int t = 0; t < kMats; ++t) {
                slab_load4<kSeg, FULL>(rs[t], static_cast<uint32_t>(Tile<R>::wrow(mt[t], kc0) - Tile<R>::wrow(mt[t], 0)), lanes,
                                 Tile<R>::wdw(kc), st.w[t]);
                if constexpr (Tile<R>::kScales)
                    scale_load(Tile<R>::srow(mt[t], kc0), spitch, r0, rows, Tile<R>::sdw(kc), st.s[t]);
                if constexpr (Tile<R>::kTileScale) st.ts[t] = Tile<R>::tile_scales(mt[t], r0, kc0, kc);
            }
        };
        uint32_t ts_cur[kMats];  // the tile scales of the chunk being multiplied
        auto operands = [&](uint32_t kc0, half8 (&xr)[kB]) {
            const uint32_t kc = FULL ? kChunk : (cols - kc0 < kChunk ? cols - kc0 : kChunk);
            const uint32_t nb = kc / 32, per = (nb + 3) / 4;
            const uint32_t b0 = wave * per < nb ? wave * per : nb, b1 = b0 + per < nb ? b0 + per : nb;
#pragma unroll
            for (int i = 0; i < kB; ++i) {
                const uint32_t b = b0 + static_cast<uint32_t>(i) < b1 ? b0 + static_cast<uint32_t>(i) : (b1 ? b1 - 1 : 0);
                const size_t at = static_cast<size_t>(vrow) * cols + kc0 + 32 * b + 8 * kg;
                xr[i] = *as_global(reinterpret_cast<const half8*>(((lane & 1) ? vl : vh) + at));
            }
        };
        auto commit = [&](uint32_t kc0, uint32_t buf, const Staged<R, kMats, kChunk>& st) {
            const uint32_t kc = FULL ? kChunk : (cols - kc0 < kChunk ? cols - kc0 : kChunk);
#pragma unroll
            for (int t = 0; t < kMats; ++t) {
                uint32_t* base = tl + buf * buf_dw + t * Tile<R>::lds_dw(kChunk);
                slab_store4<kSeg, FULL>(base, Tile<R>::wdw(kc), st.w[t]);
                if constexpr (Tile<R>::kScales)
                    scale_store(base + kSlab * kWStride, kSStride, Tile<R>::sdw(kc), st.s[t]);
                ts_cur[t] = st.ts[t];  // read only after the products of the previous chunk
            }
        };
        f32x4 acc[kMats];
#pragma unroll
        for (int t = 0; t < kMats; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
        Staged<R, kMats, kChunk> st;
        half8 xa[kB];
        stage(0, st);
        operands(0, xa);
        commit(0, 0, st);
        __syncthreads();
        for (uint32_t c = 0; c < nchunks; ++c) {
            const uint32_t kc0 = c * kChunk;
            const uint32_t kc = FULL ? kChunk : (cols - kc0 < kChunk ? cols - kc0 : kChunk);
            if (c + 1 < nchunks) stage(kc0 + kChunk, st);  // in flight during the products below
            asm volatile("" ::: "memory");  // the loads stay ahead of the products
            __builtin_amdgcn_sched_barrier(0);
            const uint32_t nb = kc / 32, per = (nb + 3) / 4;
            const uint32_t b0 = wave * per < nb ? wave * per : nb, b1 = b0 + per < nb ? b0 + per : nb;
#pragma unroll
            for (int t = 0; t < kMats; ++t) {
                const uint32_t* base = tl + (c & 1) * buf_dw + t * Tile<R>::lds_dw(kChunk);
                const uint8_t* wl = reinterpret_cast<const uint8_t*>(base + (lane & 15) * kWStride);
                const uint8_t* sl = reinterpret_cast<const uint8_t*>(base + kSlab * kWStride + (lane & 15) * kSStride);
#pragma unroll
                for (int i = 0; i < kB; ++i) {
                    if (b0 + static_cast<uint32_t>(i) >= b1) break;
                    float sc;
                    const half8 bw = Tile<R>::get(wl, sl, ts_cur[t], b0 + static_cast<uint32_t>(i), kg, sc);
                    const f32x4 z = {0.f, 0.f, 0.f, 0.f};
                    const f32x4 r = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[i], bw, z, 0, 0, 0);
#pragma unroll
                    for (int q = 0; q < 4; ++q) acc[t][q] = __builtin_fmaf(sc, r[q], acc[t][q]);
                }
            }
            if (c + 1 < nchunks) {
                // the next activation operands (into the registers just used) travel
                // while the staged weights are stored; buffer (c+1)&1 was last read in
                // iteration c-1, which every wave has finished (the barrier below)
                operands(kc0 + kChunk, xa);
                commit(kc0 + kChunk, (c + 1) & 1, st);
            }
            __syncthreads();
        }
        // the four waves' partial sums (same lane layout) meet in LDS; wave 0 adds
        if (wave > 0) {
#pragma unroll
            for (int t = 0; t < kMats; ++t) red[t][wave - 1][lane] = acc[t];
        }
        __syncthreads();
        if (wave == 0) {
#pragma unroll
            for (int v = 0; v < 3; ++v)
#pragma unroll
                for (int t = 0; t < kMats; ++t) acc[t] += red[t][v][lane];
            // lane: output row `row`, members 2kg + q (q = 0, 1) as (hi, lo) in 2q, 2q+1
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                const uint32_t j = 2 * kg + static_cast<uint32_t>(q);  // uniform over 16 lanes
                const bool live = j < m && row < rows;
                const uint32_t a = member(j);  // unused slots repeat the last member
                const float mul = vmult[GATEUP ? xrow(a) : a];
                const float v0 = (acc[0][2 * q] + acc[0][2 * q + 1]) * mul;
                if constexpr (GATEUP) {
                    const float v1 = (acc[kMats - 1][2 * q] + acc[kMats - 1][2 * q + 1]) * mul;
                    if (live) out[static_cast<size_t>(a) * rows + row] = swiglu(v0, v1, limit, official);
                } else {
                    if (live) out[static_cast<size_t>(a) * rows + row] = v0;
                }
            }
        }
        __syncthreads();  // red is reused by the next member set
    }
}

// ------------------------------------------------------ batched GEMV on MFMA
// y[b][r] = sum_c W[r][c] x[b][c] for up to 8 vectors at once: the grouped
// products' down form with the matrix as the one expert and the vectors as the
// members, so every weight is decoded once for all of them. A workgroup covers
// S slabs of 16 rows over the column range [y * kGemvRange, (y + 1) * kGemvRange):
//   1. every thread issues its share of the tile's weight loads (the whole tile is
//      in flight at once: an 8-vector GEMV is a few MB to a few tens of MB, and the
//      loads in flight, not the arithmetic, set its time at these sizes);
//   2. meanwhile it splits that slice of every vector into two fp16 parts in LDS
//      (with the slice's own power of two, which the partial sums take back): the
//      split is shared by the 16 S rows of the workgroup;
//   3. the weights go to LDS, one row per padded LDS row;
//   4. wave w multiplies slabs w, w + 4, ... over every block of the range (no
//      barrier inside the loop, no cross-wave sum) and writes the partial sums of
//      its rows to part[range][b][r]; gemv_reduce_kernel adds the ranges in order.
constexpr uint32_t kGemvRange = 512;               // columns per workgroup
constexpr uint32_t kGemvXStride = kGemvRange + 8;  // halves per staged vector part (padded)

typedef uint32_t u32x4a __attribute__((ext_vector_type(4), aligned(16)));

// LDS layout of a tile: 16 S rows of kWStride dwords (a full range's row segment,
// padded to keep 16-byte rows), then, for the split FP4 layout, 16 S rows of
// kSStride dwords of E8M0 scales.
template <class R, int S>
struct GemvTile {
    static constexpr uint32_t kRows = 16u * S;
    static constexpr uint32_t kWdw = Tile<R>::wdw(kGemvRange);
    static constexpr uint32_t kWStride = kWdw + 4;
    static constexpr uint32_t kSdw = Tile<R>::kScales ? Tile<R>::sdw(kGemvRange) : 0u;
    static constexpr uint32_t kSStride = Tile<R>::kScales ? kSdw + 1 : 0u;
    static constexpr size_t lds_bytes() { return 4ull * kRows * (kWStride + kSStride); }
};

// Weight units of V dwords (V = 4: 16-byte rows and range starts, every range full;
// V = 1: any 4-byte aligned layout, the last range possibly short).
template <int V>
struct WUnit;
template <>
struct WUnit<4> {
    typedef u32x4a T;
    static __device__ __forceinline__ T load(gptr<uint32_t> p) { return *(gptr<u32x4a>)(p); }
};
template <>
struct WUnit<1> {
    typedef uint32_t T;
    static __device__ __forceinline__ T load(gptr<uint32_t> p) { return *p; }
};

template <class R, int S, int V>
__global__ __launch_bounds__(256) void gemv_mfma_kernel(const void* __restrict__ w, const void* __restrict__ ws,
                                                        const float* __restrict__ x, float* __restrict__ part,
                                                        uint32_t rows, uint32_t cols, uint32_t n_vec) {
    using TL = GemvTile<R, S>;
    using U = typename WUnit<V>::T;
    extern __shared__ __align__(16) uint32_t tl[];
    __shared__ __align__(16) _Float16 xs[2][8][kGemvXStride];  // [hi / lo][vector][column of the range]
    __shared__ float xmul[8];
    constexpr uint32_t kUpr = TL::kWdw / V;                  // units per row of a full range
    constexpr uint32_t kNU = (TL::kRows * kUpr + 255) / 256;  // units per thread
    constexpr uint32_t kSUpr = TL::kSdw;                      // scale dwords per row (FP4)
    constexpr uint32_t kNS = (TL::kRows * kSUpr + 255) / 256;
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t r0 = blockIdx.x * TL::kRows;
    const uint32_t k0 = blockIdx.y * kGemvRange, k1 = k0 + kGemvRange < cols ? k0 + kGemvRange : cols;
    const uint32_t kc = k1 - k0;
    const uint32_t wdw = Tile<R>::wdw(kc);  // dwords of this range's row segments
    const R mt = RowsOf<R>::make(w, ws, cols);
    // 1. the vectors' slices (32 threads per vector, 16 consecutive columns each), then
    // the tile's weight (and scale) loads, all in flight together (the split below
    // waits for the slices alone)
    const uint32_t xb = threadIdx.x >> 5, xc = (threadIdx.x & 31) * 16;
    const bool xlive = xb < n_vec && k0 + xc < k1;
    float v[16];
    if (xlive) {
        const gptr<f32x4> src = as_global(reinterpret_cast<const f32x4*>(x + static_cast<size_t>(xb) * cols + k0 + xc));
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const f32x4 f = src[q];
            v[4 * q] = f[0]; v[4 * q + 1] = f[1]; v[4 * q + 2] = f[2]; v[4 * q + 3] = f[3];
        }
    }
    // rows past `rows` read the last row, units past the range's end are not read
    U wv[kNU];
    {
        const uint8_t* wb = Tile<R>::wrow(mt, k0);
        const size_t pitch = Tile<R>::wpitch(mt);
#pragma unroll
        for (uint32_t i = 0; i < kNU; ++i) {
            const uint32_t u = threadIdx.x + 256u * i;
            const uint32_t rr = u / kUpr, c = u - rr * kUpr;
            if (rr < TL::kRows && c * V < wdw) {
                const uint32_t r = r0 + rr < rows ? r0 + rr : rows - 1;
                wv[i] = WUnit<V>::load(as_global(reinterpret_cast<const uint32_t*>(wb + static_cast<size_t>(r) * pitch)) + c * V);
            }
        }
    }
    uint32_t sv[kNS > 0 ? kNS : 1];
    if constexpr (kNS > 0) {
        const uint8_t* sb = Tile<R>::srow(mt, k0);
        const size_t spitch = Tile<R>::spitch(mt);
        const uint32_t sdw = Tile<R>::sdw(kc);
#pragma unroll
        for (uint32_t i = 0; i < kNS; ++i) {
            const uint32_t u = threadIdx.x + 256u * i;
            const uint32_t rr = u / kSUpr, c = u - rr * kSUpr;
            if (rr < TL::kRows && c < sdw) {
                const uint32_t r = r0 + rr < rows ? r0 + rr : rows - 1;
                sv[i] = as_global(reinterpret_cast<const uint32_t*>(sb + static_cast<size_t>(r) * spitch))[c];
            }
        }
    }
    // 2. the slices split into two fp16 parts (the slice's power of two in xmul)
    {
        const uint32_t b = xb, c = xc;
        const bool live = xlive;
        float m = 0.0f;
        bool finite = true;
        if (live) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                finite = finite && __builtin_isfinite(v[i]);
                m = fmaxf(m, fabsf(v[i]));
            }
        }
        if (!finite) m = __builtin_inff();
#pragma unroll
        for (int off = 1; off < 32; off <<= 1) m = fmaxf(m, __shfl_xor(m, off, 64));  // the vector's 32 threads
        const int sh = split_shift(m);
        if (live) {
#pragma unroll
            for (int g = 0; g < 2; ++g) {
                half8 vh, vl;
#pragma unroll
                for (int d = 0; d < 8; ++d) {
                    const float xv = ldexpf(v[8 * g + (Tile<R>::kPermuted ? kPerm[d] : d)], sh);
                    const _Float16 th = static_cast<_Float16>(xv);
                    vh[d] = th;
                    vl[d] = static_cast<_Float16>(xv - static_cast<float>(th));
                }
                *reinterpret_cast<half8*>(&xs[0][b][c + 8 * g]) = vh;
                *reinterpret_cast<half8*>(&xs[1][b][c + 8 * g]) = vl;
            }
        }
        if (b < 8 && (threadIdx.x & 31) == 0) xmul[b] = ldexpf(1.0f, -sh);
    }
    // 3. the weights (and scales) into LDS
#pragma unroll
    for (uint32_t i = 0; i < kNU; ++i) {
        const uint32_t u = threadIdx.x + 256u * i;
        const uint32_t rr = u / kUpr, c = u - rr * kUpr;
        if (rr < TL::kRows && c * V < wdw) {
            if constexpr (V == 4) *reinterpret_cast<u32x4a*>(tl + rr * TL::kWStride + 4 * c) = wv[i];
            else tl[rr * TL::kWStride + c] = wv[i];
        }
    }
    if constexpr (kNS > 0) {
        const uint32_t sdw = Tile<R>::sdw(kc);
#pragma unroll
        for (uint32_t i = 0; i < kNS; ++i) {
            const uint32_t u = threadIdx.x + 256u * i;
            const uint32_t rr = u / kSUpr, c = u - rr * kSUpr;
            if (rr < TL::kRows && c < sdw) tl[TL::kRows * TL::kWStride + rr * TL::kSStride + c] = sv[i];
        }
    }
    __syncthreads();
    // 4. A operand rows: vector lr / 2 (the last one repeated past n_vec), part lr & 1
    const uint32_t lr = lane & 15, kg = lane >> 4;
    const _Float16* xa_row = &xs[lane & 1][(lr >> 1) < n_vec ? (lr >> 1) : n_vec - 1][0];
    constexpr int kSW = S / 4;  // slabs per wave
    f32x4 acc[kSW];
#pragma unroll
    for (int j = 0; j < kSW; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
    auto step = [&](uint32_t bb) {
        const half8 xa = *reinterpret_cast<const half8*>(xa_row + 32 * bb + 8 * kg);
#pragma unroll
        for (int j = 0; j < kSW; ++j) {
            const uint32_t row_l = (wave + 4u * static_cast<uint32_t>(j)) * 16u + lr;
            const uint8_t* wl = reinterpret_cast<const uint8_t*>(tl + row_l * TL::kWStride);
            const uint8_t* sl = reinterpret_cast<const uint8_t*>(tl + TL::kRows * TL::kWStride + row_l * TL::kSStride);
            float sc;
            const half8 bw = Tile<R>::get(wl, sl, 0u, bb, kg, sc);
            const f32x4 z = {0.f, 0.f, 0.f, 0.f};
            const f32x4 r = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa, bw, z, 0, 0, 0);
#pragma unroll
            for (int q = 0; q < 4; ++q) acc[j][q] = __builtin_fmaf(sc, r[q], acc[j][q]);
        }
    };
    if (kc == kGemvRange) {  // a full range: four blocks' loads and products interleave
#pragma unroll 1
        for (uint32_t b0 = 0; b0 < kGemvRange / 32; b0 += 4) {
#pragma unroll
            for (uint32_t i = 0; i < 4; ++i) step(b0 + i);
        }
    } else {
        for (uint32_t bb = 0; bb < kc / 32; ++bb) step(bb);
    }
    // lane: row r0 + (wave + 4j) * 16 + lr, vectors 2kg + q (q = 0, 1) as (hi, lo) in 2q, 2q+1
#pragma unroll
    for (int j = 0; j < kSW; ++j) {
        const uint32_t row = r0 + (wave + 4u * static_cast<uint32_t>(j)) * 16u + lr;
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const uint32_t jv = 2 * kg + static_cast<uint32_t>(q);
            if (jv < n_vec && row < rows)
                part[(static_cast<size_t>(blockIdx.y) * n_vec + jv) * rows + row] =
                    (acc[j][2 * q] + acc[j][2 * q + 1]) * xmul[jv];
        }
    }
}

// y[b][r] = sum over ranges s (in order) of part[s][b][r]; the loads of 8 ranges are
// in flight together, the additions keep the range order.
__global__ __launch_bounds__(256) void gemv_reduce_kernel(const float* __restrict__ part, float* __restrict__ y,
                                                          uint32_t rows, uint32_t n_vec, uint32_t n_ranges) {
    const size_t i = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x;
    const size_t n = static_cast<size_t>(n_vec) * rows;
    if (i >= n) return;
    float s = part[i];
    for (uint32_t r0 = 1; r0 < n_ranges; r0 += 8) {
        float v[8];
#pragma unroll
        for (uint32_t j = 0; j < 8; ++j)
            if (r0 + j < n_ranges) v[j] = part[static_cast<size_t>(r0 + j) * n + i];
#pragma unroll
        for (uint32_t j = 0; j < 8; ++j)
            if (r0 + j < n_ranges) s += v[j];
    }
    y[i] = s;
}

// out[t][r] = residual[t][r] + sum_j w[t][j] * part[t*k + j][r], slots in order, then
// + shared_part[t][r] (the shared expert, weight 1, last); an out-of-table id makes
// the element NaN (the id was reported by the grouping).
__global__ __launch_bounds__(256) void moe_combine_kernel(const uint32_t* __restrict__ ids, const float* __restrict__ wts,
                                                          const float* __restrict__ part,
                                                          const float* __restrict__ shared_part, const float* resid,
                                                          float* out, uint32_t k, uint32_t out_dim, uint32_t n_table) {
    const uint32_t t = blockIdx.y;
    const uint32_t r = blockIdx.x * 256 + threadIdx.x;
    if (r >= out_dim) return;
    float acc = resid ? resid[static_cast<size_t>(t) * out_dim + r] : 0.0f;
    for (uint32_t j = 0; j < k; ++j) {
        const uint32_t a = t * k + j;
        const float v = ids[a] < n_table ? part[static_cast<size_t>(a) * out_dim + r] : __builtin_nanf("");
        acc = __builtin_fmaf(wts[a], v, acc);
    }
    if (shared_part) acc += shared_part[static_cast<size_t>(t) * out_dim + r];
    out[static_cast<size_t>(t) * out_dim + r] = acc;
}

size_t align256(size_t v) { return (v + 255) & ~size_t(255); }

// about sixteen workgroups per CU over all slabs, at most one per member set
uint32_t grouped_gy(uint32_t rows, uint32_t max_sets, uint32_t cus) {
    const uint32_t slabs = (rows + kSlab - 1) / kSlab;
    const uint32_t want = (16 * cus + slabs - 1) / slabs;
    return want < 1 ? 1u : (want > max_sets ? max_sets : want);
}

// One grouped product launch: GATEUP over the split x rows (hidden columns) into
// act, else over the split act rows (inter columns) into part.
template <class R, bool GATEUP>
void launch_grouped_products(hipStream_t s, GroupWs gw, const _Float16* vh, const _Float16* vl, const float* vmult,
                             float* dst, uint32_t cols, uint32_t rows, uint32_t k, uint32_t n_assign, float limit,
                             bool official, uint32_t max_sets, uint32_t cus) {
    const size_t lds = (GATEUP ? 2 : 1) * 2 * 4 *
                       static_cast<size_t>(Tile<R>::lds_dw(GATEUP ? Tile<R>::kChunkGU : Tile<R>::kChunkDn));
    const dim3 grid((rows + kSlab - 1) / kSlab, grouped_gy(rows, max_sets, cus));
    if (cols % (GATEUP ? Tile<R>::kChunkGU : Tile<R>::kChunkDn) == 0)
        hipLaunchKernelGGL((moe_grouped_kernel<R, GATEUP, true>), grid, dim3(256), lds, s, gw, vh, vl, vmult, dst, cols,
                           rows, k, n_assign, limit, official ? 1u : 0u);
    else
        hipLaunchKernelGGL((moe_grouped_kernel<R, GATEUP, false>), grid, dim3(256), lds, s, gw, vh, vl, vmult, dst, cols,
                           rows, k, n_assign, limit, official ? 1u : 0u);
}

template <class R>
hipError_t launch_grouped(hipStream_t s, GroupWs gw, const _Float16* xh, const _Float16* xl, const float* xmult,
                          float* act, _Float16* ah, _Float16* al, float* amult, float* part, uint32_t n_assign,
                          uint32_t n_rows, uint32_t max_sets, uint32_t k,
                          uint32_t hidden, uint32_t inter, uint32_t out_dim, float limit, uint32_t cus) {
    launch_grouped_products<R, true>(s, gw, xh, xl, xmult, act, hidden, inter, k, n_assign, limit, false, max_sets,
                                     cus);
    hipLaunchKernelGGL(moe_split_kernel, dim3(n_rows), dim3(256), 0, s, act, inter, ah, al, amult,
                       Tile<R>::kPermuted ? 1u : 0u);
    launch_grouped_products<R, false>(s, gw, ah, al, amult, part, inter, out_dim, k, n_assign, 0.0f, false, max_sets,
                                      cus);
    return hipGetLastError();
}

}  // namespace

bool gemv_mfma_supported(int32_t format, uint64_t rows, uint64_t cols, uint64_t batch, const void* w,
                         const float* x) {
    if (batch < kGemvMfmaMinBatch || rows == 0 || rows > (1u << 24) || cols == 0 || cols > (1u << 20)) return false;
    if (reinterpret_cast<uintptr_t>(w) % 4 || reinterpret_cast<uintptr_t>(x) % 16) return false;
    if (format == OBJETA_HIP_FP4_E2M1) return cols % 128 == 0;  // the split layout
    return format >= OBJETA_HIP_Q4_0 && format <= OBJETA_HIP_IQ3_0 && cols % 64 == 0;
}

namespace {
template <class R, int S, int V>
hipError_t launch_gemv_mfma_sv(hipStream_t s, const void* w, const void* ws, const float* x, float* y, float* part,
                               uint32_t rows, uint32_t cols, uint32_t nv, uint32_t ks) {
    const uint32_t groups = (rows + 16 * S - 1) / (16 * S);
    const size_t lds = GemvTile<R, S>::lds_bytes();
    // one range: the partial sums are the result
    hipLaunchKernelGGL((gemv_mfma_kernel<R, S, V>), dim3(groups, ks), dim3(256), lds, s, w, ws, x,
                       ks > 1 ? part : y, rows, cols, nv);
    if (ks > 1) {
        const size_t n = static_cast<size_t>(nv) * rows;
        hipLaunchKernelGGL(gemv_reduce_kernel, dim3(static_cast<uint32_t>((n + 255) / 256)), dim3(256), 0, s, part, y,
                           rows, nv, ks);
    }
    return hipGetLastError();
}

// 8 slabs (128 rows) per workgroup for Q4_0 / Q5_0 when that still gives two
// workgroups per CU, else 4; 16-byte weight units when every range is full and its
// rows 16-byte aligned. IQ3_0 and split FP4 keep 4 slabs: their 8-slab forms need
// 212 and 256 VGPRs (one or two waves per SIMD), and measured slower at 14336 x 4096
// and 8 vectors (IQ3_0 29.3 against 22.9 us, FP4 38.8 against 18.5 us), where Q4_0
// and Q5_0 gain from 8 (19.0 against 23.9, 23.0 against 33.4 us).
template <class R>
constexpr bool kGemvWideTiles = false;
template <>
constexpr bool kGemvWideTiles<QRows<kQ4>> = true;
template <>
constexpr bool kGemvWideTiles<QRows<kQ5>> = true;

template <class R>
hipError_t launch_gemv_mfma_t(hipStream_t s, const void* w, const void* ws, const float* x, float* y, float* part,
                              uint32_t rows, uint32_t cols, uint32_t nv, uint32_t ks, uint32_t cus) {
    const bool v4 = cols % kGemvRange == 0 && reinterpret_cast<uintptr_t>(w) % 16 == 0;
    if constexpr (kGemvWideTiles<R>) {
        if (static_cast<uint64_t>((rows + 127) / 128) * ks >= 2ull * cus)
            return v4 ? launch_gemv_mfma_sv<R, 8, 4>(s, w, ws, x, y, part, rows, cols, nv, ks)
                      : launch_gemv_mfma_sv<R, 8, 1>(s, w, ws, x, y, part, rows, cols, nv, ks);
    }
    return v4 ? launch_gemv_mfma_sv<R, 4, 4>(s, w, ws, x, y, part, rows, cols, nv, ks)
              : launch_gemv_mfma_sv<R, 4, 1>(s, w, ws, x, y, part, rows, cols, nv, ks);
}
}  // namespace

int32_t launch_gemv_mfma(objeta_hip_context* ctx, hipStream_t s, int32_t format, const void* w, const void* ws,
                         const float* x, float* y, uint64_t rows, uint64_t cols, uint64_t batch) {
    const char* action = "launch batched GEMV (MFMA)";
    if (!gemv_mfma_supported(format, rows, cols, batch, w, x))
        OBJ_FAIL(kUnsupported, action, "shape, batch or alignment outside the MFMA GEMV");
    const uint32_t R = static_cast<uint32_t>(rows), K = static_cast<uint32_t>(cols);
    const uint32_t ks = (K + kGemvRange - 1) / kGemvRange;  // column ranges
    const uint32_t nvmax = static_cast<uint32_t>(batch < 8 ? batch : 8);
    const uint32_t cus = ctx->info.compute_units > 0 ? static_cast<uint32_t>(ctx->info.compute_units) : 256u;
    float* part = nullptr;
    if (ks > 1) {
        void* wsp = nullptr;
        OBJ_TRY(ensure_workspace(ctx, s, kWsGemv, 4ull * ks * nvmax * R, &wsp));
        part = static_cast<float*>(wsp);
    }
    for (uint64_t done = 0; done < batch; done += 8) {
        const uint32_t nv = static_cast<uint32_t>(batch - done < 8 ? batch - done : 8);
        const float* xb = x + done * cols;
        float* yb = y + done * rows;
        hipError_t e;
        switch (format) {
            case OBJETA_HIP_Q4_0: e = launch_gemv_mfma_t<QRows<kQ4>>(s, w, nullptr, xb, yb, part, R, K, nv, ks, cus); break;
            case OBJETA_HIP_Q5_0: e = launch_gemv_mfma_t<QRows<kQ5>>(s, w, nullptr, xb, yb, part, R, K, nv, ks, cus); break;
            case OBJETA_HIP_IQ3_0: e = launch_gemv_mfma_t<QRows<kIQ3>>(s, w, nullptr, xb, yb, part, R, K, nv, ks, cus); break;
            default: e = launch_gemv_mfma_t<Fp4Rows>(s, w, ws, xb, yb, part, R, K, nv, ks, cus); break;
        }
        if (e != hipSuccess) OBJ_FAIL(kDriver, action, hipGetErrorString(e));
    }
    return 0;
}

bool grouped_supported(int32_t format, uint64_t n_table, uint64_t n_tokens, uint64_t k, uint64_t hidden,
                       uint64_t inter, uint64_t out_dim) {
    if (format < OBJETA_HIP_Q4_0 || format > OBJETA_HIP_FP4_E2M1) return false;
    if (k == 0 || k > 32 || n_table == 0 || n_table > kGMaxTable || n_tokens * k > kGMaxAssign) return false;
    if (hidden == 0 || inter == 0 || hidden % 64 || inter % 64 || hidden > (1u << 20) || inter > (1u << 20) ||
        out_dim > (1u << 20))
        return false;
    return format != OBJETA_HIP_FP4_E2M1 || (hidden % 128 == 0 && inter % 128 == 0);
}

bool grouped_preferred(int32_t format, uint64_t n_tokens, uint64_t hidden, uint64_t inter, uint64_t out_dim) {
    if (n_tokens >= kGroupedMinTokens) return true;
    if (n_tokens < 2) return false;
    // bytes per 32 weights of each format
    const uint64_t per32 = format == OBJETA_HIP_Q4_0 ? 18 : format == OBJETA_HIP_Q5_0 ? 22
                         : format == OBJETA_HIP_IQ3_0 ? 14 : 17;
    const uint64_t bytes = (2 * inter * hidden + out_dim * inter) / 32 * per32;
    return bytes >= kGroupedLargeExpertBytes;
}

int32_t launch_moe_grouped(objeta_hip_context* ctx, int32_t format, hipStream_t s, const objeta_hip_expert_ptrs* table,
                           uint64_t n_table, const objeta_hip_expert_ptrs* shared, const uint32_t* ids, const float* wts, uint64_t n_tokens, uint64_t k,
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
    if (format == OBJETA_HIP_FP4_E2M1 && (hidden % 128 || inter % 128))
        OBJ_FAIL(kUnsupported, action, "the grouped path takes split-FP4 experts with hidden and intermediate % 128 == 0");
    if (!table || !ids || !wts || !x || !out) OBJ_FAIL(kInvalidInput, action, "NULL device pointer");
    if (reinterpret_cast<uintptr_t>(x) % 16) OBJ_FAIL(kInvalidInput, action, "x must be 16-byte aligned");
    const uint32_t A = static_cast<uint32_t>(n_tokens * k), T = static_cast<uint32_t>(n_tokens);
    const uint32_t NR = A + (shared ? T : 0);                  // act rows: routed, then shared
    const uint32_t NS = A + (shared ? (T + 7) / 8 : 0);        // member sets at most
    const uint32_t H = static_cast<uint32_t>(hidden), I = static_cast<uint32_t>(inter), O = static_cast<uint32_t>(out_dim);
    // workspace: set records, split x, act, split act, per-assignment down rows
    size_t off = 0;
    const size_t o_hdr = off; off += align256(16);
    const size_t o_set = off; off += align256(sizeof(SetRec) * NS);
    const size_t o_xm = off; off += align256(4ull * T);
    const size_t o_am = off; off += align256(4ull * NR);
    const size_t o_xh = off; off += align256(2ull * T * H);
    const size_t o_xl = off; off += align256(2ull * T * H);
    const size_t o_act = off; off += align256(4ull * NR * I);
    const size_t o_ah = off; off += align256(2ull * NR * I);
    const size_t o_all = off; off += align256(2ull * NR * I);
    const size_t o_part = off; off += align256(4ull * NR * O);
    void* wsp = nullptr;
    OBJ_TRY(ensure_workspace(ctx, s, kWsGrouped, off, &wsp));
    char* b = static_cast<char*>(wsp);
    GroupWs gw{reinterpret_cast<uint32_t*>(b + o_hdr), reinterpret_cast<SetRec*>(b + o_set)};
    float* amult = reinterpret_cast<float*>(b + o_am);
    float* xmult = reinterpret_cast<float*>(b + o_xm);
    auto* xh = reinterpret_cast<_Float16*>(b + o_xh);
    auto* xl = reinterpret_cast<_Float16*>(b + o_xl);
    float* act = reinterpret_cast<float*>(b + o_act);
    auto* ah = reinterpret_cast<_Float16*>(b + o_ah);
    auto* al = reinterpret_cast<_Float16*>(b + o_all);
    float* part = reinterpret_cast<float*>(b + o_part);
    uint32_t* err = ctx->err_word;
    const uint32_t cus = ctx->info.compute_units > 0 ? static_cast<uint32_t>(ctx->info.compute_units) : 256u;
    // the split order follows the weights' order (element order for FP4)
    const bool perm = format == OBJETA_HIP_FP4_E2M1 ? Tile<Fp4Rows>::kPermuted : Tile<QRows<kQ4>>::kPermuted;
    hipLaunchKernelGGL(moe_prepare_kernel, dim3(1 + T), dim3(256), 0, s, ids, A, static_cast<uint32_t>(n_table), table,
                       shared, T, gw, GroupWs{nullptr, nullptr}, err, x, H, xh, xl, xmult, perm ? 1u : 0u);
    hipError_t e;
    const uint32_t kk = static_cast<uint32_t>(k);
    switch (format) {
        case OBJETA_HIP_Q4_0:
            e = launch_grouped<QRows<kQ4>>(s, gw, xh, xl, xmult, act, ah, al, amult, part, A, NR, NS, kk, H,
                                           I, O, limit, cus);
            break;
        case OBJETA_HIP_Q5_0:
            e = launch_grouped<QRows<kQ5>>(s, gw, xh, xl, xmult, act, ah, al, amult, part, A, NR, NS, kk, H,
                                           I, O, limit, cus);
            break;
        case OBJETA_HIP_IQ3_0:
            e = launch_grouped<QRows<kIQ3>>(s, gw, xh, xl, xmult, act, ah, al, amult, part, A, NR, NS, kk,
                                            H, I, O, limit, cus);
            break;
        default:
            e = launch_grouped<Fp4Rows>(s, gw, xh, xl, xmult, act, ah, al, amult, part, A, NR, NS, kk, H, I,
                                        O, limit, cus);
            break;
    }
    if (e == hipSuccess) {
        hipLaunchKernelGGL(moe_combine_kernel, dim3((O + 255) / 256, T), dim3(256), 0, s, ids, wts, part,
                           shared ? part + static_cast<size_t>(A) * O : nullptr, resid, out, kk, O,
                           static_cast<uint32_t>(n_table));
        e = hipGetLastError();
    }
    if (e != hipSuccess) OBJ_FAIL(kDriver, action, hipGetErrorString(e));
    return 0;
}

bool official_grouped_supported(uint64_t n_table, uint64_t n_tokens, uint64_t k, uint64_t hidden, uint64_t inter,
                                uint64_t out_dim) {
    return n_tokens >= kOfficialGroupedMinTokens &&
           grouped_supported(OBJETA_HIP_FP4_E2M1, n_table, n_tokens, k, hidden, inter, out_dim);
}

// The official layer of launch_moe_official_fp4 on the grouped-token products: x is
// quantized and dequantized as there (its values, a 4-bit significand times a power
// of two, split into fp16 parts exactly), the routed FP4 experts and the FP8 shared
// expert (a launch of its own per phase, its member sets apart) read each matrix
// once per member set, the intermediates are quantized in place, and the combine
// adds w * down in slot order from zero, then the shared expert's down.
int32_t launch_moe_official_grouped(objeta_hip_context* ctx, hipStream_t s, const objeta_hip_expert_ptrs* table,
                                    uint64_t n_table, const objeta_hip_expert_ptrs* shared, const uint32_t* ids,
                                    const float* wts, uint64_t n_tokens, uint64_t k, const float* x, float* out,
                                    uint64_t hidden, uint64_t inter, uint64_t out_dim, float limit,
                                    uint8_t* inter_values, uint8_t* inter_scales, const OfficialMarks* marks) {
    const char* action = "launch official FP4 MoE (grouped)";
    // the routed FP4 and the shared FP8 sets multiply the same split activations
    static_assert(Tile<Fp4Rows>::kPermuted == Tile<Fp8Rows>::kPermuted, "one activation order for both tiles");
    if (!official_grouped_supported(n_table, n_tokens, k, hidden, inter, out_dim))
        OBJ_FAIL(kUnsupported, action, "shape outside the grouped official path");
    const uint32_t T = static_cast<uint32_t>(n_tokens), A = static_cast<uint32_t>(n_tokens * k);
    const uint32_t NR = A + (shared ? T : 0);       // act rows: routed, then shared
    const uint32_t NSS = shared ? (T + 7) / 8 : 0;  // shared member sets
    const uint32_t H = static_cast<uint32_t>(hidden), I = static_cast<uint32_t>(inter), O = static_cast<uint32_t>(out_dim);
    size_t off = 0;
    const size_t o_hdr = off; off += align256(16);
    const size_t o_set = off; off += align256(sizeof(SetRec) * A);
    const size_t o_hdr2 = off; off += align256(16);
    const size_t o_set2 = off; off += align256(sizeof(SetRec) * (NSS ? NSS : 1));
    const size_t o_xd = off; off += align256(4ull * T * H);
    const size_t o_xm = off; off += align256(4ull * T);
    const size_t o_am = off; off += align256(4ull * NR);
    const size_t o_xh = off; off += align256(2ull * T * H);
    const size_t o_xl = off; off += align256(2ull * T * H);
    const size_t o_act = off; off += align256(4ull * NR * I);
    const size_t o_ah = off; off += align256(2ull * NR * I);
    const size_t o_al = off; off += align256(2ull * NR * I);
    const size_t o_part = off; off += align256(4ull * NR * O);
    void* wsp = nullptr;
    OBJ_TRY(ensure_workspace(ctx, s, kWsGrouped, off, &wsp));
    char* b = static_cast<char*>(wsp);
    const GroupWs gw{reinterpret_cast<uint32_t*>(b + o_hdr), reinterpret_cast<SetRec*>(b + o_set)};
    const GroupWs gws{reinterpret_cast<uint32_t*>(b + o_hdr2), reinterpret_cast<SetRec*>(b + o_set2)};
    float* xd = reinterpret_cast<float*>(b + o_xd);
    float* xmult = reinterpret_cast<float*>(b + o_xm);
    float* amult = reinterpret_cast<float*>(b + o_am);
    auto* xh = reinterpret_cast<_Float16*>(b + o_xh);
    auto* xl = reinterpret_cast<_Float16*>(b + o_xl);
    float* act = reinterpret_cast<float*>(b + o_act);
    auto* ah = reinterpret_cast<_Float16*>(b + o_ah);
    auto* al = reinterpret_cast<_Float16*>(b + o_al);
    float* part = reinterpret_cast<float*>(b + o_part);
    uint32_t* err = ctx->err_word;
    const uint32_t cus = ctx->info.compute_units > 0 ? static_cast<uint32_t>(ctx->info.compute_units) : 256u;
    const uint32_t kk = static_cast<uint32_t>(k);
    auto mark = [&](hipEvent_t e) -> int32_t {
        if (e) OBJ_HIP(hipEventRecord(e, s), "record event");
        return 0;
    };
    OBJ_TRY(launch_act_quant(s, x, T, H, nullptr, nullptr, xd));
    hipLaunchKernelGGL(moe_prepare_kernel, dim3(1 + T), dim3(256), 0, s, ids, A, static_cast<uint32_t>(n_table), table,
                       shared, T, gw, shared ? gws : GroupWs{nullptr, nullptr}, err, xd, H, xh, xl, xmult,
                       Tile<Fp4Rows>::kPermuted ? 1u : 0u);
    launch_grouped_products<Fp4Rows, true>(s, gw, xh, xl, xmult, act, H, I, kk, A, limit, true, A, cus);
    OBJ_HIP(hipGetLastError(), action);
    OBJ_TRY(mark(marks ? marks->gate_up_end : nullptr));
    if (shared) {
        launch_grouped_products<Fp8Rows, true>(s, gws, xh, xl, xmult, act, H, I, kk, A, limit, true, NSS, cus);
        OBJ_HIP(hipGetLastError(), action);
    }
    OBJ_TRY(mark(marks ? marks->shared_gate_up_end : nullptr));
    OBJ_TRY(launch_act_quant(s, act, NR, I, inter_values, inter_scales, act));
    OBJ_TRY(mark(marks ? marks->act_quant_end : nullptr));
    hipLaunchKernelGGL(moe_split_kernel, dim3(NR), dim3(256), 0, s, act, I, ah, al, amult,
                       Tile<Fp4Rows>::kPermuted ? 1u : 0u);
    launch_grouped_products<Fp4Rows, false>(s, gw, ah, al, amult, part, I, O, kk, A, 0.0f, false, A, cus);
    OBJ_HIP(hipGetLastError(), action);
    OBJ_TRY(mark(marks ? marks->down_end : nullptr));
    if (shared) launch_grouped_products<Fp8Rows, false>(s, gws, ah, al, amult, part, I, O, kk, A, 0.0f, false, NSS, cus);
    hipLaunchKernelGGL(moe_combine_kernel, dim3((O + 255) / 256, T), dim3(256), 0, s, ids, wts, part,
                       shared ? part + static_cast<size_t>(A) * O : nullptr, nullptr, out, kk, O,
                       static_cast<uint32_t>(n_table));
    OBJ_HIP(hipGetLastError(), action);
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
    return launch_moe_grouped(ctx, format, resolve_stream(ctx, stream), d_table, n_table, nullptr, d_ids, d_weights,
                              n_tokens, k, d_x, d_residual, d_out, hidden, intermediate, out_dim, swiglu_limit);
    OBJ_GUARD_END
}
