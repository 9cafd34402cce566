// stack.hip — persistent decode-stack kernel: every MoE layer of one token in one
// cooperative launch.
//
// At batch 1 a layer is a chain of dependent steps: router logits (needs h) ->
// top-k -> gate/up (needs the ids) -> down + combine (needs every activation) ->
// h of the next layer. As separate launches each step pays a kernel boundary
// (about 1.6 us inside a graph on MI355X) plus a full memory latency, while the
// weights themselves take ~3 us per layer at 8 TB/s. Here all workgroups stay
// resident (cooperative launch) and hand the small intermediate vectors to each
// other through per-layer buffers of 64-bit words {value, epoch}: a reader polls
// with agent-scope atomic loads until every word it needs carries the current
// epoch. An atomic 64-bit store publishes value and epoch together, so no fences
// or barriers are needed, and words from earlier runs or layers are recognised by
// their older epoch.
//
// Per layer and workgroup:
//   1. h_l into LDS (layer 0 reads the caller's x; later layers gather h words).
//   2. Router waves (one per expert) compute the exact logit and its bound from a
//      router row already in registers (prefetched during the previous layer) and
//      publish {logit}, {bound}.
//   3. Every workgroup gathers the logit words and runs the same deterministic
//      top-k (router_math.hpp). If a decision is too close to call, workgroup 0
//      recomputes in the reference's sequential order and publishes the selection;
//      the others wait for it.
//   4. Each wave issues the loads of its gate/up rows, of its workgroup's down rows
//      and (router waves) of the next layer's router row, then computes
//      silu(gate) * up and publishes activation words.
//   5. Workgroups owning a down block gather the activations, finish the down
//      products from registers, add sum_j w_j d_j to h_l in selection order and
//      publish the h words of the next layer (the last layer writes the output).
// Every wait is bounded; a timeout sets the device error word and moves on, so the
// grid always drains.
#include "device_common.hpp"
#include "gemv_stream.hpp"
#include "host_common.hpp"
#include "kernels.hpp"
#include "router_math.hpp"
#include "exchange.hpp"

namespace objeta {
namespace {

using namespace dev;
using namespace rmath;
using namespace xchg;

constexpr int kSMaxE = 256;      // experts per layer
constexpr int kSMaxK = 8;        // selection slots
constexpr uint32_t kSMaxH = 2048;  // router rows held in registers: H/64 floats per lane
constexpr int kRouterNB = 8;     // float4 per lane of a router row
constexpr int kTabWords = 6;     // expert-table words per thread (kSMaxE * 6 / 256)

struct StackLayerDev {
    const objeta_hip_expert_ptrs* table;
    const float* w_r;
    const float* bias;
    uint32_t* ids_out;
    float* weights_out;
};

// Work split of the GEMV workgroups (all of them run the same code):
//   gate/up  wave w owns rw = gs_h * UG consecutive rows of the flattened
//            (slot, row) space, lpr_h = H/64 lanes per row (one pair per lane);
//   down     workgroup b owns output rows [b*rd, (b+1)*rd) for every slot; its
//            4 * gs_i (row, slot) combinations take lpr_i = I/(64*CHI) lanes each.
struct StackParams {
    const StackLayerDev* layers;
    uint32_t L, E, K, H, I;
    int renormalize;
    float limit;
    const float* x_in;
    float* h_out;
    uint64_t* hbuf;  // [L][H]   output h of layer l (input of l+1)
    uint64_t* lbuf;  // [L][2][E] logit and bound words
    uint64_t* abuf;  // [L][K][I] activation words
    uint64_t* sbuf;  // [L][2K]  selection of the sequential path
    uint32_t epoch0;
    uint32_t* err;
    uint32_t n_router;    // router workgroups (first in the grid)
    uint32_t lpr_h, rw, n_gu_waves;
    uint32_t lpr_i, rd;
};

struct StackLds {
    SelectLds<kSMaxE> sel;
    float wsel[kSMaxK];
    int flag;
    int uncertain;
};

// h_l into LDS: layer 0 copies the caller's x, later layers gather the h words
// the previous layer published.
__device__ __forceinline__ void load_h(const StackParams& a, StackLds& S, float* xs, uint32_t l, uint32_t epoch) {
    const uint32_t H = a.H;
    if (l == 0) {
        for (uint32_t i = threadIdx.x; i < (H >> 2); i += kThreads) {
            const uint32_t c = i << 2;
            *reinterpret_cast<float4*>(xs + (c >> 6) * kPad + (c & 63)) = reinterpret_cast<const float4*>(a.x_in)[i];
        }
        __syncthreads();
    } else {
        gather<true>(a.hbuf + static_cast<size_t>(l - 1) * H, H, epoch - 1, a.err, &S.flag,
               [&](uint32_t i, float v) { xs[(i >> 6) * kPad + (i & 63)] = v; });
    }
}

// Router workgroups (the first n_router): wave gw owns expert gw. Its router row
// sits in registers lane-contiguously (lane l: elements [l*H/64, (l+1)*H/64)),
// loaded one layer ahead; per layer it waits for h_l and publishes {logit},
// {bound}.
__device__ void router_role(const StackParams& a, StackLds& S, float* xs) {
    const uint32_t H = a.H, E = a.E;
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t gw = blockIdx.x * kWaves + (threadIdx.x >> 6);
    const bool active = gw < E;
    const uint32_t n4 = H >> 8;  // float4 per lane
    float4 wr[kRouterNB];
    auto load_router = [&](uint32_t l) {
        typedef float f32x4 __attribute__((ext_vector_type(4)));
        const gptr<f32x4> r4 = as_global(reinterpret_cast<const f32x4*>(a.layers[l].w_r + static_cast<size_t>(gw) * H));
#pragma unroll
        for (int g = 0; g < kRouterNB; ++g) {
            const f32x4 v = r4[lane * n4 + (static_cast<uint32_t>(g) < n4 ? static_cast<uint32_t>(g) : n4 - 1)];
            wr[g] = make_float4(v.x, v.y, v.z, v.w);
        }
    };
    if (active) load_router(0);
    for (uint32_t l = 0; l < a.L; ++l) {
        const uint32_t epoch = a.epoch0 + l;
        load_h(a, S, xs, l, epoch);
        if (active) {
            double total, abs_bound;
            exact_logit_lanes<kRouterNB>(wr, xs, n4, lane, total, abs_bound);
            if (lane == 0) {
                float lhat, bnd;
                finish_logit(total, abs_bound, a.layers[l].bias, gw, H, lhat, bnd);
                uint64_t* lw = a.lbuf + static_cast<size_t>(l) * 2 * E;
                store_word(lw + gw, lhat, epoch);
                store_word(lw + E + gw, bnd, epoch);
            }
            if (l + 1 < a.L) load_router(l + 1);
        }
        __syncthreads();  // xs is rewritten by the next layer's gather
    }
}

// GEMV workgroups. R: row accessor; UG: gate/up row groups per wave; CHI: pairs
// per lane of a down row.
template <class R, int UG, int CHI>
__device__ void gemv_role(const StackParams& a, StackLds& S, float* xs, float* as, float* red,
                          objeta_hip_expert_ptrs* tab, uint32_t gb) {
    const uint32_t H = a.H, I = a.I, K = a.K, E = a.E;
    const uint32_t pairs_i = I >> 6;
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t gwv = gb * kWaves + wave;  // GEMV wave index
    const uint32_t lpr_h = a.lpr_h, gs_h = 64 / lpr_h, slot_h = lane / lpr_h, lp_h = lane - slot_h * lpr_h;
    const uint32_t lpr_i = a.lpr_i, gs_i = 64 / lpr_i, slot_i = lane / lpr_i, lp_i = lane - slot_i * lpr_i;
    const uint32_t rd = a.rd;
    const bool has_gu = gwv < a.n_gu_waves;
    // waves past the last gate/up chunk re-load the last one and publish nothing
    const uint32_t f0 = (has_gu ? gwv : a.n_gu_waves - 1) * a.rw;  // chunks never straddle slots
    const uint32_t gj = f0 / I, gi0 = f0 - gj * I;
    // this lane group's down (row, slot) combination; spare combinations repeat the last
    const uint32_t combo = wave * gs_i + slot_i;
    const bool has_dn = combo < rd * K;
    const uint32_t cc = has_dn ? combo : rd * K - 1;
    const uint32_t dj = cc % K, drr = cc / K;
    const uint32_t r_dn = gb * rd + drr;
    const uint32_t r_dn_c = r_dn < H ? r_dn : H - 1;
    const bool publisher = gb == 0;  // publishes the sequential-path selection and the ids
    const uint32_t n_tab = E * (sizeof(objeta_hip_expert_ptrs) / 8);
    uint64_t* tab_w = reinterpret_cast<uint64_t*>(tab);

    for (uint32_t l = 0; l < a.L; ++l) {
        const uint32_t epoch = a.epoch0 + l;
        const StackLayerDev& ly = a.layers[l];
        // ---- this layer's expert table: loads issued now, landed by the h wait
        uint64_t tw[kTabWords];
        {
            const gptr<uint64_t> src = as_global(reinterpret_cast<const uint64_t*>(ly.table));
#pragma unroll
            for (int q = 0; q < kTabWords; ++q) {
                const uint32_t i = threadIdx.x + static_cast<uint32_t>(q) * kThreads;
                tw[q] = src[i < n_tab ? i : n_tab - 1];
            }
        }
        load_h(a, S, xs, l, epoch);
#pragma unroll
        for (int q = 0; q < kTabWords; ++q) {
            const uint32_t i = threadIdx.x + static_cast<uint32_t>(q) * kThreads;
            if (i < n_tab) tab_w[i] = tw[q];
        }
        // ---- selection (every GEMV workgroup, same result)
        const uint64_t* lw = a.lbuf + static_cast<size_t>(l) * 2 * E;
        gather<false>(lw, 2 * E, epoch, a.err, &S.flag, [&](uint32_t i, float v) {
            if (i < E) S.sel.val[i] = v;
            else S.sel.bnd[i - E] = v;
        });
        auto xat = [xs](uint32_t h) { return xs[(h >> 6) * kPad + (h & 63)]; };
        // a close call is first settled by recomputing the few logits involved, which
        // every workgroup does for itself (same inputs, same result; the activation
        // area of LDS is free until the gather and holds the row chunks); only what
        // that cannot settle goes to the publisher's full sequential path
        const bool certain = select_certain(S.sel, E, K, a.renormalize) ||
                             select_refine(S.sel, ly.w_r, ly.bias, xat, E, H, K, a.renormalize, as,
                                           K * pairs_i * kPad);
        uint64_t* sw = a.sbuf + static_cast<size_t>(l) * 2 * K;
        if (!certain) {
            if (publisher) {
                if (!select_underflow(S.sel, ly.w_r, ly.bias, xat, E, H, K, as, K * pairs_i * kPad))
                    select_sequential(S.sel, ly.w_r, ly.bias, xat, E, H, K);
                if (threadIdx.x < K) {
                    store_word(sw + threadIdx.x, __builtin_bit_cast(float, static_cast<uint32_t>(S.sel.sel[threadIdx.x])),
                               epoch);
                    store_word(sw + K + threadIdx.x, S.sel.e[threadIdx.x], epoch);
                }
            } else {
                gather<false>(sw, 2 * K, epoch, a.err, &S.flag, [&](uint32_t i, float v) {
                    if (i < K) {
                        const uint32_t id = __builtin_bit_cast(uint32_t, v);
                        S.sel.sel[i] = static_cast<int>(id < E ? id : 0u);
                    } else {
                        S.sel.e[i - K] = v;
                    }
                });
            }
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            float sel_sum = 0.0f;
            for (uint32_t r = 0; r < K; ++r) sel_sum = __fadd_rn(sel_sum, S.sel.e[r]);
            for (uint32_t r = 0; r < K; ++r) S.wsel[r] = a.renormalize ? __fdiv_rn(S.sel.e[r], sel_sum) : S.sel.e[r];
        }

        // ---- every gate/up weight load of the wave, issued back to back
        uint32_t eg = static_cast<uint32_t>(S.sel.sel[gj]);
        eg = eg < E ? eg : E - 1;
        uint32_t ed = static_cast<uint32_t>(S.sel.sel[dj]);
        ed = ed < E ? ed : E - 1;
        const R gm = RowsOf<R>::make(tab[eg].gate, tab[eg].gate_scale, H);
        const R um = RowsOf<R>::make(tab[eg].up, tab[eg].up_scale, H);
        const R dm = RowsOf<R>::make(tab[ed].down, tab[ed].down_scale, I);
        uint32_t dg[UG][R::kDw], du[UG][R::kDw], dd[CHI][R::kDw];
#pragma unroll
        for (int u = 0; u < UG; ++u) {
            const uint32_t r = gi0 + static_cast<uint32_t>(u) * gs_h + slot_h;
            gm.load(r, lp_h, dg[u]);
            um.load(r, lp_h, du[u]);
        }
        // No barrier until the activation gather: a workgroup barrier also waits for
        // every load in flight. (wsel, written by thread 0 above, is read after the
        // gather's barriers.)
        __builtin_amdgcn_sched_barrier(0);

        // ---- gate/up: silu(gate) * up, published as activation words. The lane's
        // 64 activations are read from LDS once (16 reads in flight) and serve every
        // gate and up row of the wave from registers.
        uint64_t* aw = a.abuf + static_cast<size_t>(l) * K * I;
        {
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
            reduce_groups<2 * UG>(gv, lpr_h);
            if (has_gu && lp_h == 0) {
#pragma unroll
                for (int u = 0; u < UG; ++u) {
                    const uint32_t r = gi0 + static_cast<uint32_t>(u) * gs_h + slot_h;
                    store_word(aw + static_cast<size_t>(gj) * I + r, silu_mul_s(gv[2 * u], gv[2 * u + 1], a.limit), epoch);
                }
            }
        }
        // The down rows are requested only now: they land while the workgroup waits
        // for the other workgroups' activations, and the gate/up stream before them
        // has the memory system (and the registers) to itself.
#pragma unroll
        for (int c = 0; c < CHI; ++c) dm.load(r_dn_c, lp_i + static_cast<uint32_t>(c) * lpr_i, dd[c]);
        __builtin_amdgcn_sched_barrier(0);
        if (publisher && ly.ids_out) write_selection(S.sel, K, a.renormalize, ly.ids_out, ly.weights_out);

        // ---- down: gather every activation, finish the row sums from registers
        gather<true>(aw, K * I, epoch, a.err, &S.flag, [&](uint32_t i, float v) {
            const uint32_t j = i / I, c = i - j * I;
            as[(j * pairs_i + (c >> 6)) * kPad + (c & 63)] = v;
        });
        {
            float acc[1] = {0.f};
#pragma unroll
            for (int c = 0; c < CHI; ++c) {
                const float* al = as + (dj * pairs_i + lp_i + static_cast<uint32_t>(c) * lpr_i) * kPad;
                float4 ar4[16];
#pragma unroll
                for (int q = 0; q < 16; ++q) ar4[q] = *reinterpret_cast<const float4*>(al + 4 * q);
                const float* xsp[1] = {reinterpret_cast<const float*>(ar4)};
                const float* xsl[1] = {al};
                dm.template dot<1>(dd[c], xsp, acc, xsl);
            }
            reduce_groups<1>(acc, lpr_i);
            if (has_dn && lp_i == 0) red[dj * rd + drr] = acc[0];
        }
        __syncthreads();
        // ---- combine into the residual in slot order; publish h_{l+1}
        if (threadIdx.x < rd) {
            const uint32_t r = gb * rd + threadIdx.x;
            if (r < H) {
                float acc = xs[(r >> 6) * kPad + (r & 63)];
                for (uint32_t j = 0; j < K; ++j) acc = __builtin_fmaf(S.wsel[j], red[j * rd + threadIdx.x], acc);
                if (l + 1 < a.L) store_word(a.hbuf + static_cast<size_t>(l) * H + r, acc, epoch);
                else a.h_out[r] = acc;
            }
        }
        __syncthreads();
    }
}

template <class R, int UG, int CHI>
__global__ __launch_bounds__(kThreads, 2) void moe_stack_kernel(StackParams a) {
    extern __shared__ float dyn[];
    __shared__ StackLds S;
    const uint32_t pairs_h = a.H >> 6, pairs_i = a.I >> 6;
    float* xs = dyn;                                      // h_l, padded: pairs_h * kPad
    float* as = dyn + pairs_h * kPad;                     // activations, padded: K * pairs_i * kPad
    float* red = as + a.K * pairs_i * kPad;               // down row sums: K * rd
    const uint32_t red_n = (a.K * a.rd + 3u) & ~3u;
    auto* tab = reinterpret_cast<objeta_hip_expert_ptrs*>(red + red_n);  // E entries (16-byte aligned)
    if (blockIdx.x < a.n_router) router_role(a, S, xs);
    else gemv_role<R, UG, CHI>(a, S, xs, as, red, tab, blockIdx.x - a.n_router);
}

template <class R, int UG>
void* stack_kernel_ug(int chi) {
    switch (chi) {
        case 1: return reinterpret_cast<void*>(&moe_stack_kernel<R, UG, 1>);
        case 2: return reinterpret_cast<void*>(&moe_stack_kernel<R, UG, 2>);
        case 3: return reinterpret_cast<void*>(&moe_stack_kernel<R, UG, 3>);
        default: return reinterpret_cast<void*>(&moe_stack_kernel<R, UG, 4>);
    }
}

template <class R>
void* stack_kernel_for(int ug, int chi) {
    switch (ug) {
        case 1: return stack_kernel_ug<R, 1>(chi);
        case 2: return stack_kernel_ug<R, 2>(chi);
        case 3: return stack_kernel_ug<R, 3>(chi);
        default: return stack_kernel_ug<R, 4>(chi);
    }
}

}  // namespace
}  // namespace objeta

using namespace objeta;

struct objeta_hip_moe_stack {
    objeta_hip_context* ctx = nullptr;
    StackParams p{};
    void* kernel = nullptr;
    uint32_t grid = 0;
    size_t lds = 0;
    void* dev = nullptr;  // descriptors + word buffers
    size_t dev_bytes = 0;
    uint64_t next_epoch = 1;
};

extern "C" {

int32_t objeta_hip_moe_stack_create(objeta_hip_context* ctx, int32_t format, const objeta_hip_moe_stack_layer* layers,
                                    uint64_t n_layers, uint64_t n_experts, uint64_t k, int32_t renormalize,
                                    uint64_t hidden, uint64_t intermediate, float swiglu_limit,
                                    objeta_hip_moe_stack** out) {
    OBJ_GUARD_BEGIN
    const char* action = "create MoE decode stack";
    OBJ_TRY(check_ctx(ctx, action));
    if (!out || !layers) OBJ_FAIL(kInvalidInput, action, "NULL argument");
    *out = nullptr;
    if (format < OBJETA_HIP_Q4_0 || format > OBJETA_HIP_FP4_E2M1)
        OBJ_FAIL(kInvalidInput, action, strf("unknown format %d", format));
    if (n_layers == 0 || n_layers > 4096) OBJ_FAIL(kInvalidInput, action, "n_layers must be in 1..=4096");
    if (n_experts == 0 || n_experts > static_cast<uint64_t>(kSMaxE))
        OBJ_FAIL(kUnsupported, action, strf("n_experts must be in 1..=%d", kSMaxE));
    if (k == 0 || k > n_experts || k > static_cast<uint64_t>(kSMaxK))
        OBJ_FAIL(kUnsupported, action, strf("k must be in 1..=min(n_experts, %d)", kSMaxK));
    if (hidden % 256 != 0 || hidden == 0 || hidden > kSMaxH)
        OBJ_FAIL(kUnsupported, action, strf("hidden must be a multiple of 256 and <= %u", kSMaxH));
    if (intermediate % 64 != 0 || intermediate == 0 || intermediate > 16384)
        OBJ_FAIL(kUnsupported, action, "intermediate must be a non-zero multiple of 64, <= 16384");
    for (uint64_t l = 0; l < n_layers; ++l) {
        const auto& ly = layers[l];
        if (!ly.d_table || !ly.d_router_w) OBJ_FAIL(kInvalidInput, action, strf("layer %llu: NULL table or router", (unsigned long long)l));
        if (reinterpret_cast<uintptr_t>(ly.d_router_w) % 16) OBJ_FAIL(kInvalidInput, action, "router weights must be 16-byte aligned");
        if (ly.d_ids_out && !ly.d_weights_out) OBJ_FAIL(kInvalidInput, action, "ids_out without weights_out");
    }
    const uint32_t H = static_cast<uint32_t>(hidden), I = static_cast<uint32_t>(intermediate);
    const uint32_t K = static_cast<uint32_t>(k), E = static_cast<uint32_t>(n_experts), L = static_cast<uint32_t>(n_layers);
    // gate/up: one pair per lane, H/64 lanes per row (a power of two)
    const uint32_t pairs_h = H >> 6, pairs_i = I >> 6;
    if (pairs_h & (pairs_h - 1)) OBJ_FAIL(kUnsupported, action, "hidden/64 must be a power of two");
    const uint32_t lpr_h = pairs_h, gs_h = 64 / lpr_h;
    const uint32_t cus = ctx->info.compute_units > 0 ? static_cast<uint32_t>(ctx->info.compute_units) : 256u;
    // down: CHI pairs per lane, lpr_i = I/(64*CHI) lanes per (row, slot) (a power of
    // two); 4*gs_i combinations per workgroup give rd = 4*gs_i/K rows. Among the
    // layouts whose gate/up rows also fit the same workgroups (UG <= 4, chunks that
    // do not straddle slots), take the one with the most workgroups up to one per CU.
    int best_chi = 0, best_ug = 0;
    uint32_t best_g = 0, best_rd = 0, best_lpr_i = 0, best_rw = 0;
    for (int chi = 1; chi <= 4; ++chi) {
        if (pairs_i % chi) continue;
        const uint32_t lpr_i = pairs_i / chi;
        if (lpr_i == 0 || lpr_i > 64 || (lpr_i & (lpr_i - 1))) continue;
        const uint32_t gs_i = 64 / lpr_i;
        const uint32_t rd = (4 * gs_i / K) > 0 ? 4 * gs_i / K : 1;
        if (rd * K > 4 * gs_i) continue;
        const uint32_t g = (H + rd - 1) / rd;
        for (int ug = 1; ug <= 4; ++ug) {
            const uint32_t rw = gs_h * ug;
            if (I % rw) continue;
            if (K * I / rw > 4 * g) continue;
            const bool better = best_g == 0 || (g <= cus && (best_g > cus || g > best_g));
            if (better) {
                best_chi = chi;
                best_ug = ug;
                best_g = g;
                best_rd = rd;
                best_lpr_i = lpr_i;
                best_rw = rw;
            }
            break;
        }
    }
    if (!best_g) OBJ_FAIL(kUnsupported, action, "no lane layout for these widths");
    void* kern = nullptr;
    switch (format) {
        case OBJETA_HIP_Q4_0: kern = stack_kernel_for<QRows<kQ4>>(best_ug, best_chi); break;
        case OBJETA_HIP_Q5_0: kern = stack_kernel_for<QRows<kQ5>>(best_ug, best_chi); break;
        case OBJETA_HIP_IQ3_0: kern = stack_kernel_for<QRows<kIQ3>>(best_ug, best_chi); break;
        default: kern = stack_kernel_for<Fp4Rows>(best_ug, best_chi); break;
    }
    const uint32_t red_n = (K * best_rd + 3u) & ~3u;
    const size_t lds = (static_cast<size_t>(pairs_h) * kPad + static_cast<size_t>(K) * pairs_i * kPad + red_n) *
                           sizeof(float) +
                       static_cast<size_t>(E) * sizeof(objeta_hip_expert_ptrs);
    OBJ_HIP(hipSetDevice(ctx->device), "hipSetDevice");
    int per_cu = 0;
    OBJ_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void*>(kern), kThreads, lds),
            "query stack kernel occupancy");
    const uint32_t capacity = static_cast<uint32_t>(per_cu) * cus;
    const uint32_t n_router = (E + kWaves - 1) / kWaves;
    const uint32_t need = best_g + n_router;
    if (per_cu < 1 || need > capacity)
        OBJ_FAIL(kUnsupported, action,
                 strf("needs %u co-resident workgroups, the device holds %u (LDS %zu B)", need, capacity, lds));
    auto* st = new objeta_hip_moe_stack();
    st->ctx = ctx;
    st->kernel = kern;
    st->grid = need;
    st->lds = lds;
    // device memory: descriptors, then the word buffers
    const size_t desc_b = (static_cast<size_t>(L) * sizeof(StackLayerDev) + 255) & ~size_t(255);
    const size_t h_b = static_cast<size_t>(L) * H * 8, l_b = static_cast<size_t>(L) * 2 * E * 8;
    const size_t a_b = static_cast<size_t>(L) * K * I * 8, s_b = static_cast<size_t>(L) * 2 * K * 8;
    st->dev_bytes = desc_b + h_b + l_b + a_b + s_b;
    hipError_t e = hipMalloc(&st->dev, st->dev_bytes);
    if (e == hipSuccess) e = hipMemset(st->dev, 0, st->dev_bytes);
    std::vector<StackLayerDev> desc(L);
    for (uint32_t l = 0; l < L; ++l)
        desc[l] = StackLayerDev{layers[l].d_table, layers[l].d_router_w, layers[l].d_router_bias, layers[l].d_ids_out,
                                layers[l].d_weights_out};
    if (e == hipSuccess) e = hipMemcpy(st->dev, desc.data(), L * sizeof(StackLayerDev), hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        if (st->dev) (void)hipFree(st->dev);
        delete st;
        OBJ_FAIL(kDriver, "allocate decode-stack buffers", hipGetErrorString(e));
    }
    char* base = static_cast<char*>(st->dev);
    StackParams& p = st->p;
    p.layers = reinterpret_cast<const StackLayerDev*>(base);
    p.L = L;
    p.E = E;
    p.K = K;
    p.H = H;
    p.I = I;
    p.renormalize = renormalize ? 1 : 0;
    p.limit = swiglu_limit;
    p.hbuf = reinterpret_cast<uint64_t*>(base + desc_b);
    p.lbuf = reinterpret_cast<uint64_t*>(base + desc_b + h_b);
    p.abuf = reinterpret_cast<uint64_t*>(base + desc_b + h_b + l_b);
    p.sbuf = reinterpret_cast<uint64_t*>(base + desc_b + h_b + l_b + a_b);
    p.err = ctx->counters + ctx->counter_words;
    p.n_router = n_router;
    p.lpr_h = lpr_h;
    p.rw = best_rw;
    p.n_gu_waves = K * I / best_rw;
    p.lpr_i = best_lpr_i;
    p.rd = best_rd;
    *out = st;
    return 0;
    OBJ_GUARD_END
}

int32_t objeta_hip_moe_stack_run(objeta_hip_moe_stack* st, objeta_hip_stream stream, const float* d_x, float* d_h_out) {
    OBJ_GUARD_BEGIN
    const char* action = "run MoE decode stack";
    if (!st) OBJ_FAIL(kInvalidInput, action, "stack is NULL");
    if (!d_x || !d_h_out) OBJ_FAIL(kInvalidInput, action, "NULL device pointer");
    if (reinterpret_cast<uintptr_t>(d_x) % 16) OBJ_FAIL(kInvalidInput, action, "x must be 16-byte aligned");
    objeta_hip_context* ctx = st->ctx;
    OBJ_HIP(hipSetDevice(ctx->device), "hipSetDevice");
    hipStream_t s = resolve_stream(ctx, stream);
    if (st->next_epoch + st->p.L >= 0xFFFFFFF0ull) {  // epochs would wrap: forget every word
        OBJ_HIP(hipStreamSynchronize(s), "synchronize before epoch reset");
        char* base = static_cast<char*>(st->dev);
        const size_t desc_b = (static_cast<size_t>(st->p.L) * sizeof(StackLayerDev) + 255) & ~size_t(255);
        // on the run's stream, so the clear is ordered before the launch below
        OBJ_HIP(hipMemsetAsync(base + desc_b, 0, st->dev_bytes - desc_b, s), "clear decode-stack words");
        st->next_epoch = 1;
    }
    StackParams p = st->p;
    p.epoch0 = static_cast<uint32_t>(st->next_epoch);
    p.x_in = d_x;
    p.h_out = d_h_out;
    st->next_epoch += p.L;
    void* args[] = {&p};
    OBJ_HIP(hipLaunchCooperativeKernel(st->kernel, dim3(st->grid), dim3(kThreads), args, st->lds, s),
            "launch decode-stack kernel");
    return 0;
    OBJ_GUARD_END
}

int32_t objeta_hip_moe_stack_info(const objeta_hip_moe_stack* st, uint32_t* grid, uint32_t* lds_bytes) {
    if (!st) OBJ_FAIL(kInvalidInput, "decode stack info", "stack is NULL");
    if (grid) *grid = st->grid;
    if (lds_bytes) *lds_bytes = static_cast<uint32_t>(st->lds);
    return 0;
}

int32_t objeta_hip_moe_stack_destroy(objeta_hip_moe_stack* st) {
    OBJ_GUARD_BEGIN
    if (!st) return 0;
    (void)hipSetDevice(st->ctx->device);
    (void)hipDeviceSynchronize();
    if (st->dev) (void)hipFree(st->dev);
    delete st;
    return 0;
    OBJ_GUARD_END
}

}  // extern "C"
