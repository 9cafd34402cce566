// layer.hip — one MoE layer of one token, top-8 routing, in a single launch:
// router logits and top-k, fused gate/up + SiLU, down + weighted combine into the
// residual.
//
// The three-kernel form of the layer (router, moe_gate_up, moe_down) pays a kernel
// boundary between dependent steps (about 1.4 us inside a graph on MI355X). One
// launch instead needs the intermediate vectors handed between workgroups, and on
// MI355X the cost of a hand-off depends on where it goes: between CUs of one XCD it
// is an L2 round trip (~0.5 us: plain store, L1 invalidate, load), between XCDs it
// goes through memory (~1 us, and slower still when hundreds of workgroups poll
// the same lines). The layout therefore follows the XCDs. The dispatcher hands
// consecutive workgroups to consecutive XCDs, starting wherever the previous launch
// stopped: workgroup b runs on XCD x = (b + o) % 8 for a launch-wide offset o. A
// workgroup reads x from the hardware (HW_REG_XCC_ID) and takes li = b / 8 as its
// index inside the XCD (the grid is a multiple of 8, so every XCD holds li = 0, 1,
// ...); the round-robin is probed once per context. XCD x owns selection slot x:
//
//   li < NR          (router) wave w computes expert 4*li + w's exact logit and
//                    bound and stores them in XCD x's logit buffer. Every XCD
//                    computes all logits itself, so they never leave the XCD.
//   li < NG          (gate/up) gathers the XCD's logits, runs the deterministic
//                    top-k, streams its rows of slot x's gate and up matrices and
//                    stores silu(gate) * up in XCD x's activation buffer.
//   NF <= li < NF+ND (down, NF = max(NR, NG)) selects likewise, requests its rows of slot x's down
//                    matrix at once (they stream with the gate/up rows), gathers
//                    slot x's activations from the L2, and publishes its row
//                    sums to the other XCDs (agent scope). It then combines one
//                    eighth of its rows over the 8 slots, in slot order, into
//                    out = resid + sum_j w_j d_j.
//
// Every wait is bounded (a timeout sets the device error word and the grid
// drains), and the host launches the kernel only when the whole grid fits on the
// device at once. Words are {value, epoch}; the epoch of a launch comes from a
// counter the down workgroups advance by exactly kDoneShare per launch, so no
// host-side state is needed and the launch can be captured in a graph.
//
// Close calls in the selection: gate/up workgroups settle them with select_refine
// (x is in their LDS); what that cannot settle, workgroup li == 0 of the XCD settles
// with select_underflow or select_sequential. Whenever the fast check fails that workgroup stores the
// selection it arrived at for its XCD, and the down workgroups wait for it rather
// than read x, which other down workgroups may already be overwriting when out
// aliases x.
#include "device_common.hpp"
#include "gemv_stream.hpp"
#include "host_common.hpp"
#include "kernels.hpp"
#include "router_math.hpp"
#include "exchange.hpp"

#include <algorithm>
#include <vector>

namespace objeta {
namespace {

using namespace dev;
using namespace rmath;
using namespace xchg;

constexpr uint32_t kXcds = 8;          // XCDs of an MI355X; one selection slot each
constexpr int kLK = 8;                 // top-k of the layer (one slot per XCD)
constexpr int kLMaxE = 256;            // experts
constexpr int kLRouterNB = 8;          // float4 per lane of a router row: hidden <= 2048
constexpr uint64_t kDoneShare = 1024;  // what the down workgroups of one launch add to `done`
constexpr int kLTabWords = 6;          // expert-table words per thread (kLMaxE * 6 / 256)
constexpr uint32_t kRefineFloats = 4 * 512;  // LDS row chunks for select_refine

struct LayerParams {
    const objeta_hip_expert_ptrs* table;
    const float* w_r;
    const float* bias;
    const float* x;
    const float* resid;
    float* out;
    uint32_t* ids_out;
    float* weights_out;
    const uint32_t* ids_in;  // routed kernel: the router's k ids and weights of the token
    const float* wts_in;
    uint32_t E, H, I;
    int renormalize;
    float limit;
    uint64_t* done;   // sum of the down workgroups' shares over all launches
    uint64_t* lbuf;   // [8][l_stride]  per XCD: 2E logit and bound words
    uint64_t* sbuf;   // [8][s_stride]  per XCD: 2K words, the selection settled by li == 0
    uint64_t* abuf;   // [8][a_stride]  per XCD: the I activations of its slot
    uint64_t* pbuf;   // [K][H]         row sums of slot j (agent scope, read by every XCD)
    uint32_t l_stride, s_stride, a_stride;
    uint32_t* err;
    uint32_t n_rt, n_gu, n_dn;  // workgroups per XCD in each role
    uint32_t lpr_h, rw;         // gate/up: wave w owns rows [w*rw, (w+1)*rw) of its slot
    uint32_t lpr_i, rd;         // down: workgroup d owns rows [d*rd, (d+1)*rd) of its slot
};

struct LayerLds {
    SelectLds<kLMaxE> sel;
    float wsel[kLK];
    int flag;
};

__device__ __forceinline__ uint32_t launch_epoch(const LayerParams& a) {
    const uint64_t d = __hip_atomic_load(a.done, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return static_cast<uint32_t>(d / kDoneShare) + 1u;
}

__device__ __forceinline__ uint32_t hw_xcc_id() {
    // HW_REG_XCC_ID (hwreg 20), bits [3:0]
    return __builtin_amdgcn_s_getreg((20 << 0) | (0 << 6) | ((4 - 1) << 11)) & 15u;
}

// x into LDS in the padded pair layout (kPad floats per 64).
__device__ __forceinline__ void stage_x_padded(const float* __restrict__ x, uint32_t H, float* xs) {
    for (uint32_t i = threadIdx.x; i < (H >> 2); i += kThreads) {
        const uint32_t c = i << 2;
        *reinterpret_cast<float4*>(xs + (c >> 6) * kPad + (c & 63)) = reinterpret_cast<const float4*>(x)[i];
    }
}

__device__ __forceinline__ void table_fetch(const LayerParams& a, uint64_t (&tw)[kLTabWords]) {
    const uint32_t n_tab = a.E * (sizeof(objeta_hip_expert_ptrs) / 8);
    const gptr<uint64_t> src = as_global(reinterpret_cast<const uint64_t*>(a.table));
#pragma unroll
    for (int q = 0; q < kLTabWords; ++q) {
        const uint32_t i = threadIdx.x + static_cast<uint32_t>(q) * kThreads;
        tw[q] = src[i < n_tab ? i : n_tab - 1];
    }
}
__device__ __forceinline__ void table_commit(const LayerParams& a, const uint64_t (&tw)[kLTabWords],
                                             objeta_hip_expert_ptrs* tab) {
    const uint32_t n_tab = a.E * (sizeof(objeta_hip_expert_ptrs) / 8);
    uint64_t* tab_w = reinterpret_cast<uint64_t*>(tab);
#pragma unroll
    for (int q = 0; q < kLTabWords; ++q) {
        const uint32_t i = threadIdx.x + static_cast<uint32_t>(q) * kThreads;
        if (i < n_tab) tab_w[i] = tw[q];
    }
}

// Router work of workgroup li of XCD x: wave w computes expert 4*li + w from a row
// held lane-contiguously in registers against x in LDS (xs staged and visible).
__device__ void router_part(const LayerParams& a, const float4 (&wr)[kLRouterNB], const float* xs, uint64_t* lb,
                            uint32_t li, uint32_t epoch) {
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t e = li * kWaves + (threadIdx.x >> 6);
    if (e >= a.E) return;
    double total, abs_bound;
    exact_logit_lanes<kLRouterNB>(wr, xs, a.H >> 8, lane, total, abs_bound);
    if (lane == 0) {
        float lhat, bnd;
        finish_logit(total, abs_bound, a.bias, e, a.H, lhat, bnd);
        store_l2(lb + e, lhat, epoch);
        store_l2(lb + a.E + e, bnd, epoch);
    }
}

// The top-k of XCD x's logits in S.sel.sel / S.sel.e (block-wide). can_refine: x is
// staged in xs and scratch holds kRefineFloats of LDS.
__device__ void select_xcd(const LayerParams& a, LayerLds& S, const float* xs, float* scratch, const uint64_t* lb,
                           uint64_t* sb, uint32_t epoch, bool can_refine, bool settler) {
    const uint32_t E = a.E;
    gather_l2(lb, 2 * E, epoch, a.err, &S.flag, [&](uint32_t i, float v) {
        if (i < E) S.sel.val[i] = v;
        else S.sel.bnd[i - E] = v;
    });
    if (select_certain(S.sel, E, kLK, a.renormalize)) return;
    if (can_refine) {
        auto xat = [xs](uint32_t h) { return xs[(h >> 6) * kPad + (h & 63)]; };
        const bool settled = select_refine(S.sel, a.w_r, a.bias, xat, E, a.H, kLK, a.renormalize, scratch, kRefineFloats);
        if (settler) {
            if (!settled && !select_underflow(S.sel, a.w_r, a.bias, xat, E, a.H, kLK, scratch, kRefineFloats))
                select_sequential(S.sel, a.w_r, a.bias, xat, E, a.H, kLK);
            __syncthreads();
            if (threadIdx.x < static_cast<uint32_t>(kLK)) {
                store_l2(sb + threadIdx.x, __builtin_bit_cast(float, static_cast<uint32_t>(S.sel.sel[threadIdx.x])),
                         epoch);
                store_l2(sb + kLK + threadIdx.x, S.sel.e[threadIdx.x], epoch);
            }
            return;
        }
        if (settled) return;
    }
    gather_l2(sb, 2 * kLK, epoch, a.err, &S.flag, [&](uint32_t i, float v) {
        if (i < static_cast<uint32_t>(kLK)) {
            const uint32_t id = __builtin_bit_cast(uint32_t, v);
            S.sel.sel[i] = static_cast<int>(id < E ? id : 0u);
        } else {
            S.sel.e[i - kLK] = v;
        }
    });
}

// Rows [gi0, gi0 + rw) of slot x's gate and up matrices for wave `wave` of
// gate/up workgroup li: lpr_h lanes per row, one pair per lane, UG row groups.
template <class R, int UG>
struct GateUpRows {
    uint32_t lp_h, slot_h, gs_h, gi0;
    bool has_gu;
    uint32_t dg[UG][R::kDw], du[UG][R::kDw];
    __device__ GateUpRows(const LayerParams& a, uint32_t li) {
        const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
        gs_h = 64 / a.lpr_h;
        slot_h = lane / a.lpr_h;
        lp_h = lane - slot_h * a.lpr_h;
        const uint32_t gwv = li * kWaves + wave;
        const uint32_t n_waves = a.I / a.rw;
        has_gu = gwv < n_waves;
        gi0 = (has_gu ? gwv : n_waves - 1) * a.rw;
    }
    __device__ __forceinline__ void load(const R& gm, const R& um) {
#pragma unroll
        for (int u = 0; u < UG; ++u) {
            const uint32_t r = gi0 + static_cast<uint32_t>(u) * gs_h + slot_h;
            gm.load(r, lp_h, dg[u]);
            um.load(r, lp_h, du[u]);
        }
    }
    // x staged in xs (visible): silu(gate) * up of the rows into XCD x's activation
    // buffer (NaN when the expert id was outside the table)
    __device__ __forceinline__ void finish(const LayerParams& a, const R& gm, const R& um, const float* xs,
                                           uint32_t x, uint32_t epoch, bool ok) {
        // the lane's 64 activations come from LDS once and serve every row of the wave
        const float* xl = xs + lp_h * kPad;
        float4 xr4[16];
#pragma unroll
        for (int q = 0; q < 16; ++q) xr4[q] = *reinterpret_cast<const float4*>(xl + 4 * q);
        const float* xsp[1] = {reinterpret_cast<const float*>(xr4)};
        const float* xsl[1] = {xl};
        float gv[2 * UG];
#pragma unroll
        for (int u = 0; u < UG; ++u) {
            float ag[1] = {0.f}, au[1] = {0.f};
            gm.template dot<1>(dg[u], xsp, ag, xsl);
            um.template dot<1>(du[u], xsp, au, xsl);
            gv[2 * u] = ag[0];
            gv[2 * u + 1] = au[0];
        }
        reduce_groups<2 * UG>(gv, a.lpr_h);
        if (has_gu && lp_h == 0) {
            uint64_t* ab = a.abuf + static_cast<size_t>(x) * a.a_stride;
#pragma unroll
            for (int u = 0; u < UG; ++u) {
                const uint32_t r = gi0 + static_cast<uint32_t>(u) * gs_h + slot_h;
                store_l2(ab + r, ok ? silu_mul_s(gv[2 * u], gv[2 * u + 1], a.limit) : __builtin_nanf(""), epoch);
            }
        }
    }
};

// ----------------------------------------------------- router + gate/up roles
template <class R, int UG>
__device__ void gate_up_role(const LayerParams& a, LayerLds& S, float* xs, float* scratch,
                             objeta_hip_expert_ptrs* tab, uint32_t x, uint32_t li, uint32_t epoch) {
    const uint32_t H = a.H, E = a.E;
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    uint64_t* lb = a.lbuf + static_cast<size_t>(x) * a.l_stride;
    uint64_t* sb = a.sbuf + static_cast<size_t>(x) * a.s_stride;
    // router row first: its latency overlaps the table and x loads
    float4 wr[kLRouterNB];
    const bool router = li < a.n_rt;
    if (router) {
        typedef float f32x4 __attribute__((ext_vector_type(4)));
        const uint32_t e = li * kWaves + wave;
        const uint32_t ec = e < E ? e : E - 1;
        const uint32_t n4 = H >> 8;
        const gptr<f32x4> r4 = as_global(reinterpret_cast<const f32x4*>(a.w_r + static_cast<size_t>(ec) * H));
#pragma unroll
        for (int g = 0; g < kLRouterNB; ++g) {
            const f32x4 v = r4[lane * n4 + (static_cast<uint32_t>(g) < n4 ? static_cast<uint32_t>(g) : n4 - 1)];
            wr[g] = make_float4(v.x, v.y, v.z, v.w);
        }
    }
    uint64_t tw[kLTabWords];
    table_fetch(a, tw);
    stage_x_padded(a.x, H, xs);
    table_commit(a, tw, tab);
    __syncthreads();
    if (router) router_part(a, wr, xs, lb, li, epoch);
    if (li >= a.n_gu) return;  // a router-only workgroup
    select_xcd(a, S, xs, scratch, lb, sb, epoch, true, li == 0);
    __syncthreads();
    if (x == 0 && li == 0 && a.ids_out) write_selection(S.sel, kLK, a.renormalize, a.ids_out, a.weights_out);

    uint32_t eg = static_cast<uint32_t>(S.sel.sel[x]);
    eg = eg < E ? eg : E - 1;
    const R gm = RowsOf<R>::make(tab[eg].gate, tab[eg].gate_scale, H);
    const R um = RowsOf<R>::make(tab[eg].up, tab[eg].up_scale, H);
    GateUpRows<R, UG> g(a, li);
    g.load(gm, um);
    __builtin_amdgcn_sched_barrier(0);
    g.finish(a, gm, um, xs, x, epoch, true);
}

// -------------------------------------------------------------------- down role
// Rows [db*rd, (db+1)*rd) of slot x's down matrix for down workgroup db: lpr_i
// lanes per row, CHI pairs per lane.
template <class R, int CHI>
struct DownRows {
    uint32_t lp_i, r_dn;
    uint32_t dd[CHI][R::kDw];
    __device__ DownRows(const LayerParams& a, uint32_t db) {
        const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
        const uint32_t gs_i = 64 / a.lpr_i, slot_i = lane / a.lpr_i;
        lp_i = lane - slot_i * a.lpr_i;
        r_dn = db * a.rd + wave * gs_i + slot_i;
    }
    __device__ __forceinline__ void load(const LayerParams& a, const R& dm) {
#pragma unroll
        for (int c = 0; c < CHI; ++c) dm.load(r_dn, lp_i + static_cast<uint32_t>(c) * a.lpr_i, dd[c]);
    }
    // Gathers slot x's activations from the XCD's L2, publishes the rows' sums to
    // every XCD, then combines rows [db*rd + x*rd/8, +rd/8) over the 8 slots in slot
    // order into out = resid + sum_j wsel[j] d_j. wsel (LDS) must be written before
    // the call; the gather's barriers make it visible.
    __device__ void finish(const LayerParams& a, const R& dm, int* s_flag, const float* wsel, float* as, float* red,
                           uint32_t x, uint32_t db, uint32_t epoch, bool ok) {
        const uint32_t H = a.H;
        gather_l2(a.abuf + static_cast<size_t>(x) * a.a_stride, a.I, epoch, a.err, s_flag, [&](uint32_t c, float v) {
            as[(c >> 6) * kPad + (c & 63)] = v;
        });
        {
            float acc[1] = {0.f};
#pragma unroll
            for (int c = 0; c < CHI; ++c) {
                const float* al = as + (lp_i + static_cast<uint32_t>(c) * a.lpr_i) * kPad;
                float4 ar4[16];
#pragma unroll
                for (int q = 0; q < 16; ++q) ar4[q] = *reinterpret_cast<const float4*>(al + 4 * q);
                const float* xsp[1] = {reinterpret_cast<const float*>(ar4)};
                const float* xsl[1] = {al};
                dm.template dot<1>(dd[c], xsp, acc, xsl);
            }
            reduce_groups<1>(acc, a.lpr_i);
            if (lp_i == 0) store_word(a.pbuf + static_cast<size_t>(x) * H + r_dn, ok ? acc[0] : __builtin_nanf(""), epoch);
        }
        const uint32_t rc = a.rd / kXcds;
        const uint32_t r0 = db * a.rd + x * rc;
        if (threadIdx.x < static_cast<uint32_t>(kLK) * rc) {
            const uint32_t j = threadIdx.x / rc, t = threadIdx.x - j * rc;
            const uint64_t* pw = a.pbuf + static_cast<size_t>(j) * H + r0 + t;
            uint64_t w = load_word(pw);
            for (uint32_t spin = 0; static_cast<uint32_t>(w >> 32) != epoch; ++spin) {
                if (spin >= kWaitLimit || (spin == 1 && (__hip_atomic_load(a.err, __ATOMIC_RELAXED,
                                                                            __HIP_MEMORY_SCOPE_AGENT) & 4u))) {
                    if (spin >= kWaitLimit) atomicOr(a.err, 4u);
                    w = 0;
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
                w = load_word(pw);
            }
            red[j * rc + t] = word_value(w);
        }
        __syncthreads();
        if (threadIdx.x < rc) {
            const uint32_t r = r0 + threadIdx.x;
            float acc = a.resid ? a.resid[r] : 0.0f;
            for (int j = 0; j < kLK; ++j) acc = __builtin_fmaf(wsel[j], red[j * rc + threadIdx.x], acc);
            a.out[r] = acc;
        }
        // The launch's share of `done`, from XCD 0's down workgroups only (one
        // atomic per workgroup of one XCD, not of all eight). When all of them have
        // combined, every workgroup of the launch has read the epoch: each combine
        // waited for the row sums of all XCDs, and those for all activations of
        // their XCD, which its gate/up (and router) workgroups produced.
        if (a.done && x == 0 && threadIdx.x == 0) {
            const uint64_t share = kDoneShare / a.n_dn + (db == 0 ? kDoneShare % a.n_dn : 0u);
            __hip_atomic_fetch_add(a.done, share, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
};

template <class R, int CHI>
__device__ void down_role(const LayerParams& a, LayerLds& S, float* as, float* red, objeta_hip_expert_ptrs* tab,
                          uint32_t x, uint32_t db, uint32_t epoch) {
    const uint32_t E = a.E;
    uint64_t tw[kLTabWords];
    table_fetch(a, tw);
    table_commit(a, tw, tab);
    __syncthreads();
    select_xcd(a, S, nullptr, nullptr, a.lbuf + static_cast<size_t>(x) * a.l_stride,
               a.sbuf + static_cast<size_t>(x) * a.s_stride, epoch, false, false);
    __syncthreads();
    if (threadIdx.x == 0) {
        float sel_sum = 0.0f;
        for (int r = 0; r < kLK; ++r) sel_sum = __fadd_rn(sel_sum, S.sel.e[r]);
        for (int r = 0; r < kLK; ++r) S.wsel[r] = a.renormalize ? __fdiv_rn(S.sel.e[r], sel_sum) : S.sel.e[r];
    }
    uint32_t ed = static_cast<uint32_t>(S.sel.sel[x]);
    ed = ed < E ? ed : E - 1;
    const R dm = RowsOf<R>::make(tab[ed].down, tab[ed].down_scale, a.I);
    DownRows<R, CHI> d(a, db);
    d.load(a, dm);
    __builtin_amdgcn_sched_barrier(0);
    d.finish(a, dm, &S.flag, S.wsel, as, red, x, db, epoch, true);
}

template <class R, int UG, int CHI>
__global__ __launch_bounds__(kThreads, 3) void moe_layer_kernel(LayerParams a) {
    extern __shared__ float dyn[];
    __shared__ LayerLds S;
    const uint32_t pairs_h = a.H >> 6, pairs_i = a.I >> 6;
    float* xs = dyn;                                  // x, padded: pairs_h * kPad
    float* as = xs + pairs_h * kPad;                  // activations (padded) / refinement rows
    const uint32_t as_n = pairs_i * kPad > kRefineFloats ? pairs_i * kPad : kRefineFloats;
    float* red = as + as_n;                           // slot-by-row sums of the combine: K * rd / 8
    auto* tab = reinterpret_cast<objeta_hip_expert_ptrs*>(red + ((a.rd + 3u) & ~3u));  // E entries
    const uint32_t x = hw_xcc_id() & (kXcds - 1), li = blockIdx.x / kXcds;
    const uint32_t epoch = launch_epoch(a);
    const uint32_t n_front = a.n_rt > a.n_gu ? a.n_rt : a.n_gu;
    if (li < n_front) gate_up_role<R, UG>(a, S, xs, as, tab, x, li, epoch);
    else down_role<R, CHI>(a, S, as, red, tab, x, li - n_front, epoch);
}

// --------------------------------------------------------- routed expert kernel
// The experts of one token once the router kernel has written the ids and weights:
// gate/up + SiLU and down + combine in one launch, laid out like moe_layer_kernel
// (XCD x serves selection slot x, its activations stay in the XCD's L2, the row
// sums cross XCDs once). The selection is already in memory, so every workgroup
// requests its weights as soon as it has its slot's id and table entry (scalar
// loads), and the down rows stream together with the gate/up rows instead of
// after a kernel boundary. The results equal those of moe_gate_up_kernel +
// moe_down_kernel up to the order of the fp32 sums inside a row.
constexpr int kXRegs = 2;  // float4 of x per thread: hidden <= 2048
//
// Epoch: the router launch before it advanced the router's token-0 counter, which
// stays put during this launch; every launch of this kernel follows its own router
// launch, so the value is new for every launch and no counter of its own (whose
// atomic updates from hundreds of workgroups would serialise) is needed.
__device__ __forceinline__ uint32_t routed_epoch(const uint32_t* counter) {
    return __hip_atomic_load(counter, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <class R, int UG, int CHI>
__global__ __launch_bounds__(kThreads, 3) void moe_experts_kernel(LayerParams a, const uint32_t* __restrict__ ids,
                                                                  const float* __restrict__ wts,
                                                                  const objeta_hip_expert_ptrs* __restrict__ table,
                                                                  const uint32_t* counter) {
    extern __shared__ float dyn[];
    __shared__ float wsel[kLK];
    __shared__ int flag;
    const uint32_t x = hw_xcc_id() & (kXcds - 1), li = blockIdx.x / kXcds;
    uint32_t e = ids[x];
    const bool ok = e < a.E;
    if (!ok) {
        if (threadIdx.x == 0) atomicOr(a.err, 1u);
        e = 0;
    }
    if (li < a.n_gu) {
        // x is requested before the weights: writing it to LDS then waits for it alone
        XRegs<kXRegs> xr;
        stage_x_issue<1, kXRegs>(a.x, a.H, xr);
        const R gm = RowsOf<R>::make(table[e].gate, table[e].gate_scale, a.H);
        const R um = RowsOf<R>::make(table[e].up, table[e].up_scale, a.H);
        GateUpRows<R, UG> g(a, li);
        g.load(gm, um);
        // the epoch is first needed with the results: read after the weights are
        // requested, so waiting for it does not hold them back
        const uint32_t epoch = routed_epoch(counter);
        stage_x_commit<1, kXRegs>(dyn, a.H, a.H >> 6, xr);
        __syncthreads();
        g.finish(a, gm, um, dyn, x, epoch, ok);
    } else {
        float wv[kLK];
#pragma unroll
        for (int j = 0; j < kLK; ++j) wv[j] = wts[j];
        const uint32_t db = li - a.n_gu;
        const R dm = RowsOf<R>::make(table[e].down, table[e].down_scale, a.I);
        DownRows<R, CHI> d(a, db);
        d.load(a, dm);
        const uint32_t epoch = routed_epoch(counter);
        if (threadIdx.x < static_cast<uint32_t>(kLK)) wsel[threadIdx.x] = wv[threadIdx.x];
        float* as = dyn;
        float* red = as + (a.I >> 6) * kPad;
        d.finish(a, dm, &flag, wsel, as, red, x, db, epoch, ok);
    }
}

constexpr int kLUG = 2;  // gate/up row groups per wave

template <class R>
void* layer_kernel_for(int chi) {
    switch (chi) {
        case 1: return reinterpret_cast<void*>(&moe_layer_kernel<R, kLUG, 1>);
        case 2: return reinterpret_cast<void*>(&moe_layer_kernel<R, kLUG, 2>);
        case 3: return reinterpret_cast<void*>(&moe_layer_kernel<R, kLUG, 3>);
        default: return reinterpret_cast<void*>(&moe_layer_kernel<R, kLUG, 4>);
    }
}

template <class R>
void* experts_kernel_for(int chi) {
    switch (chi) {
        case 1: return reinterpret_cast<void*>(&moe_experts_kernel<R, kLUG, 1>);
        case 2: return reinterpret_cast<void*>(&moe_experts_kernel<R, kLUG, 2>);
        case 3: return reinterpret_cast<void*>(&moe_experts_kernel<R, kLUG, 3>);
        default: return reinterpret_cast<void*>(&moe_experts_kernel<R, kLUG, 4>);
    }
}

struct FusedPlan {
    void* kern = nullptr;
    uint32_t n_rt = 0, n_gu = 0, n_dn = 0;
    uint32_t lpr_h = 0, rw = 0, lpr_i = 0, rd = 0;
    size_t lds = 0;
};

// Records which XCD every workgroup of a grid runs on.
__global__ void xcd_probe_kernel(uint32_t* out) {
    if (threadIdx.x == 0) out[blockIdx.x] = hw_xcc_id();
}

// Whether workgroup b of a launch runs on XCD (b + o) % 8 of an 8-XCD device for a
// launch-wide offset o (once per context; false when it cannot be checked, e.g.
// when first asked during capture).
bool xcd_round_robin(objeta_hip_context* ctx, hipStream_t s, uint32_t grid) {
    if (ctx->xcd_round_robin >= 0) return ctx->xcd_round_robin == 1;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) {
        (void)hipGetLastError();
        return false;
    }
    uint32_t* d = nullptr;
    std::vector<uint32_t> h(grid);
    bool ok = hipMalloc(&d, grid * sizeof(uint32_t)) == hipSuccess;
    if (ok) {
        hipLaunchKernelGGL(xcd_probe_kernel, dim3(grid), dim3(64), 0, s, d);
        ok = hipGetLastError() == hipSuccess && hipStreamSynchronize(s) == hipSuccess &&
             hipMemcpy(h.data(), d, grid * sizeof(uint32_t), hipMemcpyDeviceToHost) == hipSuccess;
    }
    if (d) (void)hipFree(d);
    (void)hipGetLastError();
    for (uint32_t b = 0; ok && b < grid; ++b) ok = h[b] < kXcds && h[b] == (h[0] + b) % kXcds;
    ctx->xcd_round_robin = ok ? 1 : 0;
    return ok;
}

// Lane layout and grid of the fused layer for this shape; false when the shape is
// outside what the kernel handles or the grid would not fit on the device at once.
// routed: the expert kernel after the router kernel (no router or selection roles).
bool plan_fused(objeta_hip_context* ctx, int32_t format, uint32_t E, uint32_t K, uint32_t H, uint32_t I,
                FusedPlan& p, bool routed = false) {
    if (K != static_cast<uint32_t>(kLK) || E < K || E > static_cast<uint32_t>(kLMaxE)) return false;
    if (H % 256 != 0 || H == 0 || H > 256u * kLRouterNB) return false;
    if (I % 64 != 0 || I == 0 || I > 8192) return false;
    const uint32_t pairs_h = H >> 6, pairs_i = I >> 6;
    if (pairs_h & (pairs_h - 1)) return false;
    const uint32_t lpr_h = pairs_h, gs_h = 64 / lpr_h;
    const uint32_t rw = gs_h * kLUG;
    if (I % rw) return false;
    // down: CHI pairs per lane, lpr_i = I/(64*CHI) lanes (a power of two) per row;
    // a workgroup's four waves cover rd = 4*gs_i rows, combined in eighths
    int chi = 0;
    uint32_t lpr_i = 0, rd = 0;
    for (int c = 1; c <= 4; ++c) {
        if (pairs_i % c) continue;
        const uint32_t l = pairs_i / c;
        if (l == 0 || l > 32 || (l & (l - 1))) continue;
        const uint32_t r = 4 * (64 / l);
        if (H % r) continue;
        chi = c;
        lpr_i = l;
        rd = r;
        break;
    }
    if (!chi) return false;
    p.n_rt = routed ? 0u : (E + kWaves - 1) / kWaves;
    p.n_gu = (I / rw + kWaves - 1) / kWaves;
    p.n_dn = H / rd;
    if (kXcds * p.n_dn > kDoneShare) return false;
    p.lpr_h = lpr_h;
    p.rw = rw;
    p.lpr_i = lpr_i;
    p.rd = rd;
    switch (format) {
        case OBJETA_HIP_Q4_0: p.kern = routed ? experts_kernel_for<QRows<kQ4>>(chi) : layer_kernel_for<QRows<kQ4>>(chi); break;
        case OBJETA_HIP_Q5_0: p.kern = routed ? experts_kernel_for<QRows<kQ5>>(chi) : layer_kernel_for<QRows<kQ5>>(chi); break;
        case OBJETA_HIP_IQ3_0: p.kern = routed ? experts_kernel_for<QRows<kIQ3>>(chi) : layer_kernel_for<QRows<kIQ3>>(chi); break;
        default: p.kern = routed ? experts_kernel_for<Fp4Rows>(chi) : layer_kernel_for<Fp4Rows>(chi); break;
    }
    if (routed) {
        // gate/up: x (padded); down: activations (padded) + the combine's K * rd / 8 sums
        const size_t gu = static_cast<size_t>(pairs_h) * kPad, dn = static_cast<size_t>(pairs_i) * kPad + K * (rd / kXcds);
        p.lds = (gu > dn ? gu : dn) * sizeof(float);
        if (H > 4u * kXRegs * kThreads) return false;
    } else {
        const uint32_t as_n = pairs_i * kPad > kRefineFloats ? pairs_i * kPad : kRefineFloats;
        p.lds = (static_cast<size_t>(pairs_h) * kPad + as_n + ((rd + 3u) & ~3u)) * sizeof(float) +
                static_cast<size_t>(E) * sizeof(objeta_hip_expert_ptrs);
    }
    if (p.lds > 65536) return false;
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, p.kern, kThreads, p.lds) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    const uint32_t cus = ctx->info.compute_units > 0 ? static_cast<uint32_t>(ctx->info.compute_units) : 256u;
    return per_cu >= 1 && kXcds * (std::max(p.n_rt, p.n_gu) + p.n_dn) <= static_cast<uint32_t>(per_cu) * cus;
}

}  // namespace

bool fused_layer_supported(objeta_hip_context* ctx, hipStream_t s, int32_t format, uint64_t n_experts, uint64_t k,
                           uint64_t hidden, uint64_t inter, uint64_t out_dim) {
    if (format < OBJETA_HIP_Q4_0 || format > OBJETA_HIP_FP4_E2M1 || out_dim != hidden) return false;
    if (n_experts > 0xFFFFu || k > 0xFFFFu || hidden > 0xFFFFu || inter > 0xFFFFu) return false;
    FusedPlan p;
    if (!plan_fused(ctx, format, static_cast<uint32_t>(n_experts), static_cast<uint32_t>(k),
                    static_cast<uint32_t>(hidden), static_cast<uint32_t>(inter), p))
        return false;
    return xcd_round_robin(ctx, s, kXcds * (std::max(p.n_rt, p.n_gu) + p.n_dn));
}

namespace {

// Workspace (slot kWsFused for the fused layer, kWsExperts for the expert kernel:
// the `done` counter, then the per-XCD logit, selection and activation words and
// the K x H row sums) and the parameters of either kernel.
int32_t layer_params(objeta_hip_context* ctx, hipStream_t s, int slot, const FusedPlan& p, uint32_t E, uint32_t K,
                     uint32_t H, uint32_t I, LayerParams& a) {
    // per-XCD regions start on separate 256-byte boundaries
    auto round_words = [](size_t w) { return (w + 31) & ~size_t(31); };
    const size_t l_w = round_words(2 * static_cast<size_t>(E)), s_w = round_words(2 * kLK), a_w = round_words(I);
    const size_t words = kXcds * (l_w + s_w + a_w) + static_cast<size_t>(K) * H;
    void* ws = nullptr;
    OBJ_TRY(ensure_workspace(ctx, s, slot, 256 + words * sizeof(uint64_t), &ws));
    a.E = E;
    a.H = H;
    a.I = I;
    char* base = static_cast<char*>(ws);
    a.done = reinterpret_cast<uint64_t*>(base);
    uint64_t* w0 = reinterpret_cast<uint64_t*>(base + 256);
    a.lbuf = w0;
    a.sbuf = a.lbuf + kXcds * l_w;
    a.abuf = a.sbuf + kXcds * s_w;
    a.pbuf = a.abuf + kXcds * a_w;
    a.l_stride = static_cast<uint32_t>(l_w);
    a.s_stride = static_cast<uint32_t>(s_w);
    a.a_stride = static_cast<uint32_t>(a_w);
    a.err = ctx->counters + ctx->counter_words;
    a.n_rt = p.n_rt;
    a.n_gu = p.n_gu;
    a.n_dn = p.n_dn;
    a.lpr_h = p.lpr_h;
    a.rw = p.rw;
    a.lpr_i = p.lpr_i;
    a.rd = p.rd;
    return 0;
}

}  // namespace

int32_t launch_moe_layer_fused(objeta_hip_context* ctx, int32_t format, hipStream_t s,
                               const objeta_hip_expert_ptrs* table, uint64_t n_experts, const float* w_r,
                               const float* bias, uint64_t k, int32_t renormalize, const float* x, const float* resid,
                               float* out, uint32_t* ids_out, float* weights_out, uint64_t hidden, uint64_t inter,
                               float limit) {
    const char* action = "launch fused MoE layer";
    FusedPlan p;
    const uint32_t E = static_cast<uint32_t>(n_experts), K = static_cast<uint32_t>(k);
    const uint32_t H = static_cast<uint32_t>(hidden), I = static_cast<uint32_t>(inter);
    if (!plan_fused(ctx, format, E, K, H, I, p)) OBJ_FAIL(kUnsupported, action, "shape outside the fused layer");
    if (!table || !w_r || !x || !out) OBJ_FAIL(kInvalidInput, action, "NULL device pointer");
    if (reinterpret_cast<uintptr_t>(x) % 16 || reinterpret_cast<uintptr_t>(w_r) % 16)
        OBJ_FAIL(kInvalidInput, action, "x and the router weights must be 16-byte aligned");
    LayerParams a{};
    OBJ_TRY(layer_params(ctx, s, kWsFused, p, E, K, H, I, a));
    a.table = table;
    a.w_r = w_r;
    a.bias = bias;
    a.x = x;
    a.resid = resid;
    a.out = out;
    a.ids_out = ids_out;
    a.weights_out = weights_out;
    a.renormalize = renormalize ? 1 : 0;
    a.limit = limit;
    const uint32_t grid = kXcds * (std::max(p.n_rt, p.n_gu) + p.n_dn);
    void* args[] = {&a};
    OBJ_HIP(hipLaunchKernel(p.kern, dim3(grid), dim3(kThreads), args, p.lds, s), action);
    return 0;
}

bool experts_xcd_supported(objeta_hip_context* ctx, hipStream_t s, int32_t format, uint64_t n_experts, uint64_t k,
                           uint64_t hidden, uint64_t inter, uint64_t out_dim) {
    if (format < OBJETA_HIP_Q4_0 || format > OBJETA_HIP_FP4_E2M1 || out_dim != hidden) return false;
    if (n_experts > 0xFFFFu || k > 0xFFFFu || hidden > 0xFFFFu || inter > 0xFFFFu) return false;
    FusedPlan p;
    if (!plan_fused(ctx, format, static_cast<uint32_t>(n_experts), static_cast<uint32_t>(k),
                    static_cast<uint32_t>(hidden), static_cast<uint32_t>(inter), p, true))
        return false;
    return xcd_round_robin(ctx, s, kXcds * (p.n_gu + p.n_dn));
}

int32_t launch_moe_experts_xcd(objeta_hip_context* ctx, int32_t format, hipStream_t s,
                               const objeta_hip_expert_ptrs* table, uint64_t n_experts, const uint32_t* ids,
                               const float* wts, const float* x, const float* resid, float* out, uint64_t hidden,
                               uint64_t inter, float limit) {
    const char* action = "launch XCD-aligned MoE experts";
    FusedPlan p;
    const uint32_t E = static_cast<uint32_t>(n_experts), K = static_cast<uint32_t>(kLK);
    const uint32_t H = static_cast<uint32_t>(hidden), I = static_cast<uint32_t>(inter);
    if (!plan_fused(ctx, format, E, K, H, I, p, true)) OBJ_FAIL(kUnsupported, action, "shape outside the kernel");
    if (!table || !ids || !wts || !x || !out) OBJ_FAIL(kInvalidInput, action, "NULL device pointer");
    if (reinterpret_cast<uintptr_t>(x) % 16) OBJ_FAIL(kInvalidInput, action, "x must be 16-byte aligned");
    LayerParams a{};
    OBJ_TRY(layer_params(ctx, s, kWsExperts, p, E, K, H, I, a));
    a.done = nullptr;  // the epoch comes from the router's counter
    a.table = table;
    a.x = x;
    a.resid = resid;
    a.out = out;
    a.limit = limit;
    const uint32_t grid = kXcds * (p.n_gu + p.n_dn);
    const uint32_t* counter = ctx->counters;  // token 0's router counter
    void* args[] = {&a, &ids, &wts, &table, &counter};
    OBJ_HIP(hipLaunchKernel(p.kern, dim3(grid), dim3(kThreads), args, p.lds, s), action);
    return 0;
}

}  // namespace objeta
