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

namespace objeta {
namespace {

using namespace dev;
using namespace rmath;

constexpr int kSMaxE = 256;      // experts per layer
constexpr int kSMaxK = 8;        // selection slots (two per wave in the down phase)
constexpr uint32_t kSMaxH = 2048;  // router rows held in registers: 8 chunks of 256
constexpr int kRouterNB = 8;
constexpr int kJW = 2;           // down: selection slots per wave
constexpr uint32_t kWaitLimit = 1u << 18;  // polls per gather (a fraction of a second)

struct StackLayerDev {
    const objeta_hip_expert_ptrs* table;
    const float* w_r;
    const float* bias;
    uint32_t* ids_out;
    float* weights_out;
};

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
    uint32_t lpr_h, lpr_i;  // lanes per row of H-wide and I-wide rows
    uint32_t n_gu_chunks;   // (K*I) / (gs_h * UG)
    uint32_t n_dn_blocks;   // ceil(H / (gs_i * UD))
};

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
            if (spin < 8) __builtin_amdgcn_s_sleep(2);
            else __builtin_amdgcn_s_sleep(8);
        }
    }
    __syncthreads();
}

// Block-wide gather of n words that must carry `epoch`; sink(i, value) is called
// once per word when it is seen current. Threads remember which of their (at most
// 32) positions are still pending, so later rounds re-read only those.
template <class Sink>
__device__ void gather(const uint64_t* __restrict__ p, uint32_t n, uint32_t epoch, uint32_t* err, int* s_flag,
                       Sink sink) {
    wait_sample(p, n, epoch, err);
    const uint32_t per = (n + kThreads - 1) / kThreads;
    uint32_t mask = per >= 32 ? 0xFFFFFFFFu : ((1u << per) - 1u);
    for (uint32_t spin = 0;; ++spin) {
        // after one timed-out wait every later wait gives up at once, so the grid drains
        if (spin == 1 && (__hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) & 4u)) return;
        uint32_t m = mask;
        while (m) {
            const uint32_t q = __builtin_ctz(m);
            m &= m - 1;
            const uint32_t i = threadIdx.x + q * kThreads;
            if (i >= n) {
                mask &= ~(1u << q);
                continue;
            }
            const uint64_t w = load_word(p + i);
            if (static_cast<uint32_t>(w >> 32) == epoch) {
                sink(i, word_value(w));
                mask &= ~(1u << q);
            }
        }
        if (threadIdx.x == 0) *s_flag = 0;
        __syncthreads();
        if (mask) *s_flag = 1;
        __syncthreads();
        const int pending = *s_flag;
        __syncthreads();
        if (!pending) return;
        if (spin >= kWaitLimit) {
            if (threadIdx.x == 0) atomicOr(err, 4u);
            return;
        }
        __builtin_amdgcn_s_sleep(8);
    }
}

template <class R>
struct RowsFor;
template <int F>
struct RowsFor<QRows<F>> {
    static __device__ __forceinline__ QRows<F> make(const void* w, const void*, uint32_t cols) {
        return QRows<F>{static_cast<const uint8_t*>(w), static_cast<size_t>(cols >> 5) * Fmt<F>::kBlockBytes};
    }
};
template <>
struct RowsFor<Fp4Rows> {
    static __device__ __forceinline__ Fp4Rows make(const void* w, const void* s, uint32_t cols) {
        return Fp4Rows{static_cast<const uint8_t*>(w), static_cast<const uint8_t*>(s), cols >> 1, cols >> 5};
    }
};

__device__ __forceinline__ float silu_mul_s(float g, float u, float limit) {
    if (limit > 0.0f) {
        u = fminf(limit, fmaxf(-limit, u));
        g = fminf(limit, g);
    }
    return (g / (1.0f + expf(-g))) * u;
}

struct StackLds {
    SelectLds<kSMaxE> sel;
    float wsel[kSMaxK];
    int flag;
    int uncertain;
};

// Router workgroups (the first ceil(E/4)): wave gw owns expert gw. It keeps its
// router row in registers, loaded one layer ahead, and per layer waits for h_l,
// publishes {logit}, {bound} and loads the next layer's row.
__device__ void router_role(const StackParams& a, StackLds& S, float* xs) {
    const uint32_t H = a.H, E = a.E;
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t gw = blockIdx.x * kWaves + (threadIdx.x >> 6);
    const bool active = gw < E;
    float4 wr[kRouterNB];
    auto load_router = [&](uint32_t l) {
        const float4* r4 = reinterpret_cast<const float4*>(a.layers[l].w_r + static_cast<size_t>(gw) * H);
        const uint32_t n4 = H >> 2;
#pragma unroll
        for (int g = 0; g < kRouterNB; ++g) {
            const uint32_t i = g * 64 + lane;
            wr[g] = r4[i < n4 ? i : n4 - 1];
        }
    };
    if (active) load_router(0);
    for (uint32_t l = 0; l < a.L; ++l) {
        const uint32_t epoch = a.epoch0 + l;
        if (l == 0) {
            for (uint32_t i = threadIdx.x; i < (H >> 2); i += kThreads) {
                const uint32_t c = i << 2;
                *reinterpret_cast<float4*>(xs + (c >> 6) * kPad + (c & 63)) = reinterpret_cast<const float4*>(a.x_in)[i];
            }
            __syncthreads();
        } else {
            gather(a.hbuf + static_cast<size_t>(l - 1) * H, H, epoch - 1, a.err, &S.flag,
                   [&](uint32_t i, float v) { xs[(i >> 6) * kPad + (i & 63)] = v; });
        }
        if (active) {
            double total, abs_prefix;
            exact_logit_regs_lean<kRouterNB>(wr, xs, H, lane, total, abs_prefix);
            if (lane == 0) {
                float lhat, bnd;
                finish_logit(total, abs_prefix, a.layers[l].bias, gw, H, lhat, bnd);
                uint64_t* lw = a.lbuf + static_cast<size_t>(l) * 2 * E;
                store_word(lw + gw, lhat, epoch);
                store_word(lw + E + gw, bnd, epoch);
            }
            if (l + 1 < a.L) load_router(l + 1);
        }
        __syncthreads();  // xs is rewritten by the next layer's gather
    }
}

// GEMV workgroups. R: row accessor; CHH / CHI: pair chunks per lane for H-wide /
// I-wide rows; UG: rows per gate/up slot; UD: rows per down slot.
template <class R, int CHH, int CHI, int UG, int UD>
__device__ void gemv_role(const StackParams& a, StackLds& S, float* xs, float* as, float* red, uint32_t gb) {
    const uint32_t H = a.H, I = a.I, K = a.K, E = a.E;
    const uint32_t pairs_i = I >> 6;
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t gwv = gb * kWaves + wave;  // GEMV wave index
    const uint32_t gs_h = 64 / a.lpr_h, slot_h = lane / a.lpr_h, lp_h = lane - slot_h * a.lpr_h;
    const uint32_t gs_i = 64 / a.lpr_i, slot_i = lane / a.lpr_i, lp_i = lane - slot_i * a.lpr_i;
    const uint32_t rows_dn = gs_i * UD;
    const uint32_t rows_gu = gs_h * UG;
    const bool has_gu = gwv < a.n_gu_chunks;
    const bool has_dn = gb < a.n_dn_blocks;
    const bool publisher = gb == 0;  // publishes the sequential-path selection and the ids

    for (uint32_t l = 0; l < a.L; ++l) {
        const uint32_t epoch = a.epoch0 + l;
        const StackLayerDev& ly = a.layers[l];
        // ---- h_l into LDS
        if (l == 0) {
            for (uint32_t i = threadIdx.x; i < (H >> 2); i += kThreads) {
                const uint32_t c = i << 2;
                *reinterpret_cast<float4*>(xs + (c >> 6) * kPad + (c & 63)) = reinterpret_cast<const float4*>(a.x_in)[i];
            }
            __syncthreads();
        } else {
            gather(a.hbuf + static_cast<size_t>(l - 1) * H, H, epoch - 1, a.err, &S.flag,
                   [&](uint32_t i, float v) { xs[(i >> 6) * kPad + (i & 63)] = v; });
        }
        // ---- selection (every GEMV workgroup, same result)
        const uint64_t* lw = a.lbuf + static_cast<size_t>(l) * 2 * E;
        gather(lw, 2 * E, epoch, a.err, &S.flag, [&](uint32_t i, float v) {
            if (i < E) S.sel.val[i] = v;
            else S.sel.bnd[i - E] = v;
        });
        const bool certain = select_certain(S.sel, E, K, a.renormalize);
        uint64_t* sw = a.sbuf + static_cast<size_t>(l) * 2 * K;
        if (!certain) {
            if (publisher) {
                select_sequential(S.sel, ly.w_r, ly.bias, [xs](uint32_t h) { return xs[(h >> 6) * kPad + (h & 63)]; },
                                  E, H, K);
                if (threadIdx.x < K) {
                    store_word(sw + threadIdx.x, __builtin_bit_cast(float, static_cast<uint32_t>(S.sel.sel[threadIdx.x])),
                               epoch);
                    store_word(sw + K + threadIdx.x, S.sel.e[threadIdx.x], epoch);
                }
            } else {
                gather(sw, 2 * K, epoch, a.err, &S.flag, [&](uint32_t i, float v) {
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
        if (publisher && ly.ids_out) write_selection(S.sel, K, a.renormalize, ly.ids_out, ly.weights_out);
        __syncthreads();

        // ---- issue this wave's loads: its gate/up rows, its workgroup's down rows
        uint32_t dg[UG][CHH][R::kDw], du[UG][CHH][R::kDw];
        uint32_t gj = 0, gi0 = 0;
        R gm{}, um{};
        if (has_gu) {
            const uint32_t f0 = gwv * rows_gu;  // flattened (slot, row); chunks never straddle slots
            gj = f0 / I;
            gi0 = f0 - gj * I;
            const uint32_t e = static_cast<uint32_t>(S.sel.sel[gj]);
            const objeta_hip_expert_ptrs P = ly.table[e < E ? e : E - 1];
            gm = RowsFor<R>::make(P.gate, P.gate_scale, H);
            um = RowsFor<R>::make(P.up, P.up_scale, H);
#pragma unroll
            for (int u = 0; u < UG; ++u) {
                const uint32_t r = gi0 + static_cast<uint32_t>(u) * gs_h + (slot_h < gs_h ? slot_h : 0);
#pragma unroll
                for (int c = 0; c < CHH; ++c) {
                    const uint32_t p = lp_h + static_cast<uint32_t>(c) * a.lpr_h;
                    gm.load(r, p, dg[u][c]);
                    um.load(r, p, du[u][c]);
                }
            }
        }
        uint32_t dd[kJW][UD][CHI][R::kDw];
        R dm[kJW];
        const uint32_t row0_dn = gb * rows_dn;
        if (has_dn) {
#pragma unroll
            for (int jj = 0; jj < kJW; ++jj) {
                const uint32_t j = wave * kJW + jj;
                const uint32_t jc = j < K ? j : K - 1;
                const uint32_t e = static_cast<uint32_t>(S.sel.sel[jc]);
                const objeta_hip_expert_ptrs P = ly.table[e < E ? e : E - 1];
                dm[jj] = RowsFor<R>::make(P.down, P.down_scale, I);
#pragma unroll
                for (int u = 0; u < UD; ++u) {
                    const uint32_t r = row0_dn + static_cast<uint32_t>(u) * gs_i + slot_i;
                    const uint32_t rc = r < H ? r : H - 1;
#pragma unroll
                    for (int c = 0; c < CHI; ++c) dm[jj].load(rc, lp_i + static_cast<uint32_t>(c) * a.lpr_i, dd[jj][u][c]);
                }
            }
        }

        // ---- gate/up compute, activation words
        uint64_t* aw = a.abuf + static_cast<size_t>(l) * K * I;
        if (has_gu) {
#pragma unroll
            for (int u = 0; u < UG; ++u) {
                float ag[1] = {0.f}, au[1] = {0.f};
#pragma unroll
                for (int c = 0; c < CHH; ++c) {
                    const float* xsp[1] = {xs + (lp_h + static_cast<uint32_t>(c) * a.lpr_h) * kPad};
                    gm.template dot<1>(dg[u][c], xsp, ag);
                    um.template dot<1>(du[u][c], xsp, au);
                }
                const float g = row_reduce(ag[0], lp_h, a.lpr_h);
                const float v = row_reduce(au[0], lp_h, a.lpr_h);
                if (slot_h < gs_h && lp_h == 0) {
                    const uint32_t r = gi0 + static_cast<uint32_t>(u) * gs_h + slot_h;
                    store_word(aw + static_cast<size_t>(gj) * I + r, silu_mul_s(g, v, a.limit), epoch);
                }
            }
        }

        // ---- down + combine
        if (has_dn) {
            gather(aw, K * I, epoch, a.err, &S.flag, [&](uint32_t i, float v) {
                const uint32_t j = i / I, c = i - j * I;
                as[(j * pairs_i + (c >> 6)) * kPad + (c & 63)] = v;
            });
#pragma unroll
            for (int jj = 0; jj < kJW; ++jj) {
                const uint32_t j = wave * kJW + jj;
                const uint32_t jc = j < K ? j : K - 1;
#pragma unroll
                for (int u = 0; u < UD; ++u) {
                    float acc[1] = {0.f};
#pragma unroll
                    for (int c = 0; c < CHI; ++c) {
                        const float* xsp[1] = {as + (jc * pairs_i + lp_i + static_cast<uint32_t>(c) * a.lpr_i) * kPad};
                        dm[jj].template dot<1>(dd[jj][u][c], xsp, acc);
                    }
                    const float v = row_reduce(acc[0], lp_i, a.lpr_i);
                    if (slot_i < gs_i && lp_i == 0 && j < K) red[j * rows_dn + static_cast<uint32_t>(u) * gs_i + slot_i] = v;
                }
            }
            __syncthreads();
            if (threadIdx.x < rows_dn) {
                const uint32_t r = row0_dn + threadIdx.x;
                if (r < H) {
                    float acc = xs[(r >> 6) * kPad + (r & 63)];
                    for (uint32_t j = 0; j < K; ++j) acc = __builtin_fmaf(S.wsel[j], red[j * rows_dn + threadIdx.x], acc);
                    if (l + 1 < a.L) store_word(a.hbuf + static_cast<size_t>(l) * H + r, acc, epoch);
                    else a.h_out[r] = acc;
                }
            }
        }
        __syncthreads();
    }
}

template <class R, int CHH, int CHI, int UG, int UD>
__global__ __launch_bounds__(kThreads) void moe_stack_kernel(StackParams a) {
    extern __shared__ float dyn[];
    __shared__ StackLds S;
    const uint32_t pairs_h = a.H >> 6, pairs_i = a.I >> 6;
    float* xs = dyn;                       // h_l, padded: pairs_h * kPad
    float* as = dyn + pairs_h * kPad + 4;  // activations, padded: K * pairs_i * kPad
    float* red = as + a.K * pairs_i * kPad;  // down row sums: K * gs_i * UD
    const uint32_t n_router = (a.E + kWaves - 1) / kWaves;
    if (blockIdx.x < n_router) router_role(a, S, xs);
    else gemv_role<R, CHH, CHI, UG, UD>(a, S, xs, as, red, blockIdx.x - n_router);
}

template <class R, int CHH, int CHI>
void* stack_kernel_ptr(int ug, int ud) {
    if (ug == 2 && ud == 2) return reinterpret_cast<void*>(&moe_stack_kernel<R, CHH, CHI, 2, 2>);
    if (ug == 2) return reinterpret_cast<void*>(&moe_stack_kernel<R, CHH, CHI, 2, 1>);
    if (ud == 2) return reinterpret_cast<void*>(&moe_stack_kernel<R, CHH, CHI, 1, 2>);
    return reinterpret_cast<void*>(&moe_stack_kernel<R, CHH, CHI, 1, 1>);
}

template <class R>
void* stack_kernel_for(uint32_t chh, uint32_t chi, int ug, int ud) {
    if (chh == 1 && chi == 1) return stack_kernel_ptr<R, 1, 1>(ug, ud);
    if (chh == 1) return stack_kernel_ptr<R, 1, 2>(ug, ud);
    if (chi == 1) return stack_kernel_ptr<R, 2, 1>(ug, ud);
    return stack_kernel_ptr<R, 2, 2>(ug, ud);
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
    const uint32_t lpr_h = pick_lpr(H >> 6), lpr_i = pick_lpr(I >> 6);
    if (!lpr_h || !lpr_i || (H >> 6) / lpr_h > 2 || (I >> 6) / lpr_i > 2)
        OBJ_FAIL(kUnsupported, action, "no lane layout for these widths");
    const uint32_t chh = (H >> 6) / lpr_h, chi = (I >> 6) / lpr_i;
    const uint32_t gs_h = 64 / lpr_h, gs_i = 64 / lpr_i;
    int ug = (I % (2 * gs_h) == 0) ? 2 : 1;
    if (I % (gs_h * ug) != 0) OBJ_FAIL(kUnsupported, action, "intermediate not a multiple of the gate/up rows per wave");
    const int ud = 2;
    void* kern = nullptr;
    switch (format) {
        case OBJETA_HIP_Q4_0: kern = stack_kernel_for<QRows<kQ4>>(chh, chi, ug, ud); break;
        case OBJETA_HIP_Q5_0: kern = stack_kernel_for<QRows<kQ5>>(chh, chi, ug, ud); break;
        case OBJETA_HIP_IQ3_0: kern = stack_kernel_for<QRows<kIQ3>>(chh, chi, ug, ud); break;
        default: kern = stack_kernel_for<Fp4Rows>(chh, chi, ug, ud); break;
    }
    const uint32_t n_gu_chunks = K * I / (gs_h * ug);
    const uint32_t rows_dn = gs_i * ud;
    const uint32_t n_dn_blocks = (H + rows_dn - 1) / rows_dn;
    const size_t lds = (static_cast<size_t>(H >> 6) * kPad + 4 + static_cast<size_t>(K) * (I >> 6) * kPad +
                        static_cast<size_t>(K) * rows_dn) * sizeof(float);
    OBJ_HIP(hipSetDevice(ctx->device), "hipSetDevice");
    int per_cu = 0;
    OBJ_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void*>(kern), kThreads, lds),
            "query stack kernel occupancy");
    const uint32_t cus = ctx->info.compute_units > 0 ? static_cast<uint32_t>(ctx->info.compute_units) : 256u;
    const uint32_t capacity = static_cast<uint32_t>(per_cu) * cus;
    uint32_t need = (n_gu_chunks + kWaves - 1) / kWaves;  // GEMV workgroups
    need = need > n_dn_blocks ? need : n_dn_blocks;
    need += (E + kWaves - 1) / kWaves;  // router workgroups
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
    p.lpr_h = lpr_h;
    p.lpr_i = lpr_i;
    p.n_gu_chunks = n_gu_chunks;
    p.n_dn_blocks = n_dn_blocks;
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
        OBJ_HIP(hipMemset(base + desc_b, 0, st->dev_bytes - desc_b), "clear decode-stack words");
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
