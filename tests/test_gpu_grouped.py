"""Grouped-token expert product (objeta_hip_moe_grouped_device) on the GPU.

A batch of tokens whose selections overlap: every token's output must equal the
CPU oracle's selected_moe_cpu (moe.rs:1283-1324) / selected_moe_cpu_native_fp4
(moe.rs:1665-1735) for that token plus its residual, within the fp32 bars used by
the other MoE tests, and agree with the per-assignment path
(objeta_hip_moe_selected_device) on the same inputs. Groups of more than 8 tokens
cover several MFMA column sets."""
import numpy as np
import pytest

from objeta_amd import HipError, MoeExecutor
from oracle import oracle as orc
from test_gpu_moe import FP4, IQ3, Q4, Q5, assert_moe_close, device_table, make_experts, oracle_experts

pytestmark = pytest.mark.gpu


def skewed_selection(T, K, E, seed):
    """Per token K distinct experts, drawn from a Zipf-like popularity so that a few
    experts are shared by many tokens; weights softmax-like and positive."""
    rng = np.random.default_rng(seed)
    p = 1.0 / np.arange(1, E + 1) ** 1.2
    p /= p.sum()
    sel = []
    for _ in range(T):
        ids = rng.choice(E, size=K, replace=False, p=p)
        w = rng.random(K).astype(np.float32) + np.float32(0.1)
        w /= w.sum()
        sel.append([(int(i), float(v)) for i, v in zip(ids, w)])
    return sel


def run_grouped(backend, fmt, experts, sel, xs, hidden, inter, out_dim, residual):
    moe = MoeExecutor(backend)
    table, keep = device_table(backend, fmt, experts)
    T, K = len(sel), len(sel[0])
    ids = np.array([[s[0] for s in row] for row in sel], np.uint32).ravel()
    ws = np.array([[s[1] for s in row] for row in sel], np.float32).ravel()
    d_ids, d_w = backend.to_device(ids), backend.to_device(ws)
    d_x = backend.to_device(np.asarray(xs, np.float32).ravel())
    d_r = backend.to_device(np.asarray(residual, np.float32).ravel())
    out_g = backend.alloc(4 * T * out_dim)
    out_s = backend.alloc(4 * T * out_dim)
    moe.grouped_device(fmt, table, d_ids, d_w, T, K, d_x, d_r, out_g, hidden, inter, out_dim)
    moe.selected_device(fmt, table, d_ids, d_w, T, K, d_x, d_r, out_s, hidden, inter, out_dim)
    backend.synchronize()
    err = moe.device_error()
    g = out_g.download(np.float32, T * out_dim).reshape(T, out_dim)
    s = out_s.download(np.float32, T * out_dim).reshape(T, out_dim)
    del keep
    return g, s, err


@pytest.mark.parametrize("fmt,E,K,T,H,I,O", [
    (Q4, 16, 4, 16, 512, 256, 512),
    (Q4, 128, 8, 16, 2048, 768, 2048),   # Qwen3-A3B layer shape, batch 16
    (Q5, 12, 3, 20, 256, 128, 192),
    (IQ3, 10, 4, 12, 512, 192, 320),
    (FP4, 12, 4, 24, 1024, 512, 1024),
])
def test_grouped_matches_oracle_and_per_assignment(backend, fmt, E, K, T, H, I, O):
    experts = make_experts(fmt, E, H, I, O, seed=E * 7 + K, gen="gauss")
    sel = skewed_selection(T, K, E, seed=T + fmt)
    counts = np.bincount([e for row in sel for e, _ in row], minlength=E)
    xs = orc.gauss(T * H, 11 + fmt, 1.0).reshape(T, H)
    res = orc.gauss(T * O, 12 + fmt, 1.0).reshape(T, O)
    g, s, err = run_grouped(backend, fmt, experts, sel, xs, H, I, O, res)
    assert err == 0
    oe = oracle_experts(fmt, experts)
    for t in range(T):
        ref = orc.selected_moe(fmt, oe, sel[t], xs[t], H, I, O) + res[t]
        assert_moe_close(g[t], ref)
    scale = float(np.max(np.abs(s)))
    assert float(np.max(np.abs(g - s))) <= 1e-4 * scale
    if T >= 16:
        assert counts.max() > 8  # some group spans two MFMA column sets


def test_grouped_lcg_experts_and_no_residual(backend):
    """The reference tests' LCG weights (uniform(-1,1), moe.rs:1770-1790), out = 0 + sum."""
    fmt, E, K, T, H, I, O = Q4, 6, 2, 9, 256, 128, 256
    experts = make_experts(fmt, E, H, I, O, seed=0xC0FFEE)
    sel = skewed_selection(T, K, E, seed=3)
    xs = orc.seeded_f32s(T * H, 0xDEADBEEF).reshape(T, H)
    moe = MoeExecutor(backend)
    table, keep = device_table(backend, fmt, experts)
    ids = np.array([[s[0] for s in row] for row in sel], np.uint32).ravel()
    ws = np.array([[s[1] for s in row] for row in sel], np.float32).ravel()
    out = backend.alloc(4 * T * O)
    moe.grouped_device(fmt, table, backend.to_device(ids), backend.to_device(ws), T, K, backend.to_device(xs.ravel()),
                       None, out, H, I, O)
    backend.synchronize()
    assert moe.device_error() == 0
    got = out.download(np.float32, T * O).reshape(T, O)
    oe = oracle_experts(fmt, experts)
    for t in range(T):
        assert_moe_close(got[t], orc.selected_moe(fmt, oe, sel[t], xs[t], H, I, O))
    del keep


def test_grouped_out_of_table_id_is_reported(backend):
    fmt, E, K, T, H, I, O = Q4, 4, 2, 3, 256, 128, 256
    experts = make_experts(fmt, E, H, I, O, seed=5, gen="gauss")
    sel = [[(0, 0.5), (1, 0.5)], [(2, 0.5), (E + 3, 0.5)], [(3, 0.7), (0, 0.3)]]
    xs = orc.gauss(T * H, 1, 1.0).reshape(T, H)
    res = np.zeros((T, O), np.float32)
    g, _, err = run_grouped(backend, fmt, experts, sel, xs, H, I, O, res)
    assert err & 1
    assert np.all(np.isnan(g[1]))
    oe = oracle_experts(fmt, experts)
    for t in (0, 2):
        assert_moe_close(g[t], orc.selected_moe(fmt, oe, sel[t], xs[t], H, I, O))


def test_grouped_all_ids_out_of_table_and_repeated_expert(backend):
    """The combine runs in the down launch: a token none of whose assignments reaches
    a set (every id out of the table) still gets its NaN row, and a token that selects
    one expert twice is counted once per slot."""
    fmt, E, K, T, H, I, O = Q4, 4, 2, 3, 256, 128, 264  # 264: a last slab of 8 rows
    experts = make_experts(fmt, E, H, I, O, seed=9, gen="gauss")
    sel = [[(E + 1, 0.5), (E + 2, 0.5)], [(1, 0.6), (1, 0.4)], [(0, 0.5), (2, 0.5)]]
    xs = orc.gauss(T * H, 2, 1.0).reshape(T, H)
    res = np.zeros((T, O), np.float32)
    g, s, err = run_grouped(backend, fmt, experts, sel, xs, H, I, O, res)
    assert err & 1
    assert np.all(np.isnan(g[0]))
    oe = oracle_experts(fmt, experts)
    for t in (1, 2):
        assert_moe_close(g[t], orc.selected_moe(fmt, oe, sel[t], xs[t], H, I, O))
        assert_moe_close(g[t], s[t])


def test_grouped_rejects_unsupported_shapes(backend):
    moe = MoeExecutor(backend)
    experts = make_experts(Q4, 2, 96, 64, 64, seed=1, gen="gauss")
    table, keep = device_table(backend, Q4, experts)
    d = backend.alloc(4096)
    with pytest.raises(HipError) as e:
        moe.grouped_device(Q4, table, d, d, 1, 1, d, None, d, 96, 64, 64)  # hidden 96 is not a multiple of 64
    assert e.value.kind == "Unsupported"
    del keep


@pytest.mark.parametrize("fmt,E,K,T,H,I,limit", [
    (Q4, 32, 4, 12, 512, 256, 0.0),     # the smallest batch the layer entry point groups
    (FP4, 16, 4, 20, 1024, 512, 0.0),
    (Q5, 24, 3, 40, 256, 128, 0.0),     # five shared-expert sets
    (Q4, 16, 2, 18, 256, 128, 0.05),    # SwiGLU clamp (against the per-assignment path)
])
def test_layer_batch_runs_grouped_with_shared_expert(backend, fmt, E, K, T, H, I, limit):
    """objeta_hip_moe_layer_shared_device at a batch: router, then the grouped
    products with the shared expert as one more group (every token, weight 1, added
    after the routed sum as moe.rs:1552-1600 does). Each token matches the oracle's
    routing and selected_moe with the shared expert, and the per-assignment path on
    the same selection."""
    experts = make_experts(fmt, E + 1, H, I, H, seed=40 + fmt, gen="gauss")
    table, keep = device_table(backend, fmt, experts[:E])
    shared, keep_s = device_table(backend, fmt, experts[E:])
    w_r = orc.gauss(E * H, 50 + fmt, 0.02)
    xs = orc.gauss(T * H, 60 + fmt, 1.0).reshape(T, H)
    d_x = backend.to_device(xs.ravel())
    d_out, d_ref = backend.alloc(4 * T * H), backend.alloc(4 * T * H)
    d_ids, d_w = backend.alloc(4 * T * K), backend.alloc(4 * T * K)
    moe = MoeExecutor(backend)
    moe.layer_device(fmt, table, backend.to_device(w_r), None, K, T, d_x, d_x, d_out, d_ids, d_w, H, I, H,
                     swiglu_limit=limit, shared=shared)
    moe.selected_device(fmt, table, d_ids, d_w, T, K, d_x, d_x, d_ref, H, I, H, swiglu_limit=limit, shared=shared)
    backend.synchronize()
    assert moe.device_error() == 0
    ids = d_ids.download(np.uint32, T * K).reshape(T, K)
    out = d_out.download(np.float32, T * H).reshape(T, H)
    per = d_ref.download(np.float32, T * H).reshape(T, H)
    oe = oracle_experts(fmt, experts)
    for t in range(T):
        rid, rw, _, _ = orc.router(w_r, xs[t], E, H, K, renormalize=True)
        assert np.array_equal(ids[t], rid), t
        if limit == 0.0:  # the clamp's own oracle check is test_gpu_moe.test_moe_swiglu_limit
            sel = [(int(i), float(v)) for i, v in zip(rid, rw)]
            ref = orc.selected_moe(fmt, oe[:E], sel, xs[t], H, I, H, shared=oe[E])
            assert_moe_close(out[t] - xs[t], ref)
    scale = float(np.max(np.abs(per)))
    assert float(np.max(np.abs(out - per))) <= 1e-4 * scale
    del keep, keep_s


def test_layer_batch_calls_and_graph_replays(backend):
    """The layer entry point at hidden 2048 (the router's two-launch batch form, then
    the grouped products, whose workspace every call on the stream shares): layer
    calls of different batch sizes in a row, a direct grouped call in between, and a
    captured layer replayed with eager layer calls of other sizes between the
    replays must each give the per-assignment path's result on the same selection
    and the oracle router's ids; every replay must equal the eager call bit for
    bit."""
    import ctypes as C
    from objeta_amd.api import check
    E, K, H, I, TM = 32, 4, 2048, 256, 32
    experts = make_experts(Q4, E, H, I, H, seed=71, gen="gauss")
    table, keep = device_table(backend, Q4, experts)
    w_r = orc.gauss(E * H, 72, 0.02)
    d_wr = backend.to_device(w_r)
    xs = orc.gauss(TM * H, 73, 1.0).reshape(TM, H)
    d_x = backend.to_device(xs.ravel())
    d_out, d_ref, d_out2 = backend.alloc(4 * TM * H), backend.alloc(4 * TM * H), backend.alloc(4 * TM * H)
    d_ids, d_w = backend.alloc(4 * TM * K), backend.alloc(4 * TM * K)
    d_ids2, d_w2 = backend.alloc(4 * TM * K), backend.alloc(4 * TM * K)
    moe = MoeExecutor(backend)
    st = backend.stream(0)

    def layer(T, out=d_out, ids=d_ids, w=d_w):
        moe.layer_device(Q4, table, d_wr, None, K, T, d_x, d_x, out, ids, w, H, I, H, stream=st)

    def agrees(T, what):
        moe.selected_device(Q4, table, d_ids, d_w, T, K, d_x, d_x, d_ref, H, I, H, stream=st)
        backend.synchronize(st)
        assert moe.device_error() == 0, what
        ids = d_ids.download(np.uint32, T * K).reshape(T, K)
        for t in (0, T // 2, T - 1):
            rid, _, _, _ = orc.router(w_r, xs[t], E, H, K, renormalize=True)
            assert np.array_equal(ids[t], rid), (what, t)
        out = d_out.download(np.float32, T * H)
        per = d_ref.download(np.float32, T * H)
        assert float(np.max(np.abs(out - per))) <= 1e-4 * float(np.max(np.abs(per))), what

    for T in (16, 12, 32, 13):
        layer(T)
        agrees(T, f"layer {T}")
    # a grouped call on the ids of the last layer call, grouped by a launch of its own
    moe.grouped_device(Q4, table, d_ids, d_w, 13, K, d_x, d_x, d_out, H, I, H, stream=st)
    agrees(13, "grouped 13")
    layer(16)
    agrees(16, "layer 16 after grouped")
    ref = d_out.download(np.float32, 16 * H)
    check(backend.L.objeta_hip_graph_begin_capture(backend.ctx, st))
    layer(16)
    g = C.c_void_p()
    check(backend.L.objeta_hip_graph_end_capture(backend.ctx, st, C.byref(g)))
    try:
        for rep in range(3):
            d_out.upload(np.zeros(16 * H, np.float32), st)
            check(backend.L.objeta_hip_graph_launch(backend.ctx, g, st))
            backend.synchronize(st)
            assert moe.device_error() == 0, rep
            assert np.array_equal(d_out.download(np.float32, 16 * H), ref), rep
            layer(12 + rep, out=d_out2, ids=d_ids2, w=d_w2)
            backend.synchronize(st)
    finally:
        check(backend.L.objeta_hip_graph_destroy(backend.ctx, g))
    agrees(16, "after the replays")
    del keep


@pytest.mark.parametrize("fmt,K", [(Q4, 4), (Q5, 8), (IQ3, 4), (FP4, 8)])
def test_layer_one_token_shared_expert_second_down_launch(backend, fmt, K):
    """One token, intermediate 2048 (32 lanes per row), k % 4 == 0 and a shared
    expert: the routed down runs four rows per lane group and the shared expert is
    added by a second launch; the token matches the oracle's routing and selected_moe
    with the shared expert."""
    test_layer_batch_runs_grouped_with_shared_expert(backend, fmt, 12, K, 1, 256, 2048, 0.0)
