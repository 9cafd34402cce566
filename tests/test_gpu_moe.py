"""Selected-expert MoE on the GPU (fused gate/up + SiLU, down + weighted combine)
through the C ABI, against the CPU oracle's selected_moe_cpu /
selected_moe_cpu_native_fp4 restatements (moe.rs:1283-1324, 1665-1735).

Bars: the reference's own GPU-vs-CPU thresholds (moe.rs:1755-1889: cosine >= 0.9999,
relative L2 <= 1e-4, max-abs <= 1e-2) and the tighter per-element bound
|y - ref| <= 1e-4 * max|ref| in fp32."""
import numpy as np
import pytest

from objeta_amd import ExpertTable, MoeExecutor, QuantFormat
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

Q4, Q5, IQ3, FP4 = int(QuantFormat.Q4_0), int(QuantFormat.Q5_0), int(QuantFormat.IQ3_0), 3


def _quantize(fmt, m, rows, cols):
    if fmt == FP4:
        return orc.split_interleaved_fp4(orc.quantize_matrix(FP4, m, rows, cols), rows, cols)
    return (orc.quantize_matrix(fmt, m, rows, cols),)


def make_experts(fmt, n, hidden, inter, out_dim, seed, gen="lcg"):
    """Host experts as the reference's tests build them (moe.rs:1770-1790)."""
    experts = []
    for e in range(n):
        if gen == "lcg":
            g = orc.seeded_f32s(inter * hidden, seed ^ e ^ 0x1111)
            u = orc.seeded_f32s(inter * hidden, seed ^ e ^ 0x2222)
            d = orc.seeded_f32s(out_dim * inter, seed ^ e ^ 0x3333)
        else:
            g = orc.gauss(inter * hidden, seed * 1000 + 3 * e, 0.02)
            u = orc.gauss(inter * hidden, seed * 1000 + 3 * e + 1, 0.02)
            d = orc.gauss(out_dim * inter, seed * 1000 + 3 * e + 2, 0.02)
        experts.append((_quantize(fmt, g, inter, hidden), _quantize(fmt, u, inter, hidden),
                        _quantize(fmt, d, out_dim, inter)))
    return experts


def oracle_experts(fmt, experts):
    if fmt == FP4:
        return [(g[0], g[1], u[0], u[1], d[0], d[1]) for g, u, d in experts]
    return [(g[0], u[0], d[0]) for g, u, d in experts]


def device_table(backend, fmt, experts):
    keep, entries = [], []
    for g, u, d in experts:
        bufs = [backend.to_device(a) for a in (g[0], u[0], d[0])]
        if fmt == FP4:
            bufs += [backend.to_device(a) for a in (g[1], u[1], d[1])]
        keep += bufs
        entries.append(tuple(bufs))
    return ExpertTable(backend, entries), keep


def assert_moe_close(out, ref, abs_bar=1e-2):
    """abs_bar: the reference's absolute max-abs threshold, meant for outputs of order
    one; None skips it where outputs are orders of magnitude larger (the relative
    per-element bound below still applies)."""
    out = np.asarray(out, np.float32)
    ref = np.asarray(ref, np.float32)
    c = orc.compare(ref, out)
    assert c["cosine_similarity"] >= 0.9999, c
    assert c["relative_l2_error"] <= 1e-4, c
    if abs_bar is not None:
        assert c["max_abs_error"] <= abs_bar, c
    scale = max(float(np.max(np.abs(ref))), 1e-30)
    err = float(np.max(np.abs(out.astype(np.float64) - ref.astype(np.float64))))
    assert err <= 1e-4 * scale, f"max rel err {err / scale:.3e}"


def run_device(backend, fmt, experts, selected_per_token, xs, hidden, inter, out_dim, residual=None,
               in_place=False, limit=0.0):
    moe = MoeExecutor(backend)
    table, keep = device_table(backend, fmt, experts)
    T = len(selected_per_token)
    k = len(selected_per_token[0])
    ids = np.array([[s[0] for s in sel] for sel in selected_per_token], np.uint32).ravel()
    ws = np.array([[s[1] for s in sel] for sel in selected_per_token], np.float32).ravel()
    d_ids, d_w = backend.to_device(ids), backend.to_device(ws)
    d_x = backend.to_device(np.asarray(xs, np.float32).ravel())
    if in_place:
        assert hidden == out_dim
        d_out = d_x
        d_res = d_x
    else:
        d_out = backend.alloc(4 * T * out_dim)
        d_res = None if residual is None else backend.to_device(np.asarray(residual, np.float32).ravel())
    moe.selected_device(fmt, table, d_ids, d_w, T, k, d_x, d_res, d_out, hidden, inter, out_dim,
                        swiglu_limit=limit)
    backend.synchronize()
    out = d_out.download(np.float32, T * out_dim).reshape(T, out_dim)
    assert moe.device_error() == 0
    del keep
    return out


def reference_selection(seed, k, n_experts=8):
    weights = [0.4, 0.3, 0.2, 0.1]
    return [((seed + i) % n_experts, weights[i % 4]) for i in range(k)]


# run_moe_test_case shapes and seeds (moe.rs:1755-1889)
@pytest.mark.parametrize("hidden,inter,out_dim,k", [(256, 512, 256, 1), (256, 512, 256, 2),
                                                    (1024, 2048, 1024, 4)])
@pytest.mark.parametrize("seed", [0, 1, 2, 3, 4, 123])
def test_moe_reference_cases_q4(backend, hidden, inter, out_dim, k, seed):
    experts = make_experts(Q4, 8, hidden, inter, out_dim, seed)
    x = orc.seeded_f32s(hidden, seed ^ 0xDEADBEEF)
    sel = reference_selection(seed, k)
    ref = orc.selected_moe(Q4, oracle_experts(Q4, experts), sel, x, hidden, inter, out_dim)
    out = run_device(backend, Q4, experts, [sel], [x], hidden, inter, out_dim)
    assert_moe_close(out[0], ref)


@pytest.mark.parametrize("fmt", [Q5, IQ3, FP4])
@pytest.mark.parametrize("hidden,inter,out_dim,k", [(256, 512, 256, 2), (1024, 2048, 1024, 4)])
def test_moe_other_formats(backend, fmt, hidden, inter, out_dim, k):
    seed = 7
    experts = make_experts(fmt, 8, hidden, inter, out_dim, seed)
    x = orc.seeded_f32s(hidden, seed ^ 0xDEADBEEF)
    sel = reference_selection(seed, k)
    ref = orc.selected_moe(fmt, oracle_experts(fmt, experts), sel, x, hidden, inter, out_dim)
    out = run_device(backend, fmt, experts, [sel], [x], hidden, inter, out_dim)
    assert_moe_close(out[0], ref)


# Production-like shapes: Qwen3-A3B slice (H 2048, I 768, top-8), the 8-expert stack
# layer (H 2048, I 1024, top-2), the DeepSeek-V3-class FP4 width (H 7168, I 2048),
# and general shapes (multiples of 32 but not 64) that take the one-wave-per-row path.
@pytest.mark.parametrize("fmt,hidden,inter,out_dim,k,n", [
    (Q4, 2048, 768, 2048, 8, 16), (Q4, 2048, 1024, 2048, 2, 8), (FP4, 7168, 2048, 7168, 8, 3),
    (Q4, 96, 160, 96, 3, 5), (Q5, 2048, 96, 224, 2, 4), (IQ3, 4096, 256, 4096, 6, 7),
    (FP4, 128, 96, 64, 2, 3)])
def test_moe_production_shapes(backend, fmt, hidden, inter, out_dim, k, n):
    experts = make_experts(fmt, n, hidden, inter, out_dim, 11, gen="gauss")
    x = orc.gauss(hidden, 99, 1.0)
    rng = np.random.default_rng(5)
    ids = rng.choice(n, size=k, replace=k > n)
    w = rng.random(k).astype(np.float32)
    w /= w.sum()
    sel = [(int(i), float(v)) for i, v in zip(ids, w)]
    ref = orc.selected_moe(fmt, oracle_experts(fmt, experts), sel, x, hidden, inter, out_dim)
    out = run_device(backend, fmt, experts, [sel], [x], hidden, inter, out_dim)
    assert_moe_close(out[0], ref)


def test_moe_tokens_residual_and_repeated_experts(backend):
    """Several tokens with their own selections (repeats allowed), residual add."""
    fmt, hidden, inter, out_dim, n, k, T = Q4, 512, 384, 512, 6, 3, 5
    experts = make_experts(fmt, n, hidden, inter, out_dim, 3, gen="gauss")
    xs = [orc.gauss(hidden, 500 + t, 1.0) for t in range(T)]
    res = [orc.gauss(out_dim, 600 + t, 1.0) for t in range(T)]
    rng = np.random.default_rng(9)
    sels = [[(int(rng.integers(n)), float(rng.random())) for _ in range(k)] for _ in range(T)]
    out = run_device(backend, fmt, experts, sels, xs, hidden, inter, out_dim, residual=res)
    for t in range(T):
        ref = orc.selected_moe(fmt, oracle_experts(fmt, experts), sels[t], xs[t], hidden, inter, out_dim)
        assert_moe_close(out[t] - res[t], ref)


def test_moe_in_place_residual(backend):
    """h <- h + MoE(h) with output, residual and input the same buffer."""
    fmt, hidden, inter, n, k = Q4, 1024, 512, 4, 2
    experts = make_experts(fmt, n, hidden, inter, hidden, 4, gen="gauss")
    x = orc.gauss(hidden, 77, 1.0)
    sel = [(2, 0.7), (0, 0.3)]
    out = run_device(backend, fmt, experts, [sel], [x], hidden, inter, hidden, in_place=True)
    ref = orc.selected_moe(fmt, oracle_experts(fmt, experts), sel, x, hidden, inter, hidden)
    assert_moe_close(out[0] - x, ref)


def test_moe_swiglu_limit(backend):
    """silu_mul with swiglu_limit > 0 clamps up to [-L, L] and gate to <= L (moe.cu:2-22)."""
    fmt, hidden, inter, out_dim = Q4, 256, 128, 64
    experts = make_experts(fmt, 1, hidden, inter, out_dim, 8)
    x = orc.seeded_f32s(hidden, 8) * 40.0
    L = 10.0
    out = run_device(backend, fmt, experts, [[(0, 1.0)]], [x], hidden, inter, out_dim, limit=L)
    g = orc.gemv(fmt, experts[0][0][0], x, inter, hidden)
    u = orc.gemv(fmt, experts[0][1][0], x, inter, hidden)
    assert np.max(np.abs(g)) > L and np.max(np.abs(u)) > L  # the clamp is exercised
    u = np.clip(u, -L, L)
    g = np.minimum(g, L)
    act = (g / (1.0 + np.exp(-g.astype(np.float64)))).astype(np.float32) * u
    ref = orc.gemv(fmt, experts[0][2][0], act, out_dim, inter)
    assert_moe_close(out[0], ref)


def test_moe_bad_expert_id_sets_device_error(backend):
    fmt, hidden, inter, out_dim = Q4, 128, 64, 64
    experts = make_experts(fmt, 2, hidden, inter, out_dim, 1)
    moe = MoeExecutor(backend)
    table, keep = device_table(backend, fmt, experts)
    d_ids = backend.to_device(np.array([1, 5], np.uint32))
    d_w = backend.to_device(np.array([0.5, 0.5], np.float32))
    d_x = backend.to_device(orc.seeded_f32s(hidden, 3))
    d_out = backend.alloc(4 * out_dim)
    moe.selected_device(fmt, table, d_ids, d_w, 1, 2, d_x, None, d_out, hidden, inter, out_dim)
    backend.synchronize()
    out = d_out.download(np.float32, out_dim)
    assert np.all(np.isnan(out))
    assert moe.device_error() == 1
    assert moe.device_error() == 0  # reading clears it
    del keep


@pytest.mark.parametrize("fmt,hidden,inter,n,k,T,bias", [
    (Q4, 2048, 768, 128, 8, 1, True), (Q4, 2048, 1024, 8, 2, 1, False),
    (Q4, 1024, 256, 32, 4, 3, True), (FP4, 1024, 512, 16, 4, 2, False),
    (Q4, 2048, 768, 128, 8, 16, True), (FP4, 1024, 512, 16, 4, 6, False), (Q5, 512, 256, 24, 3, 8, True)])
def test_moe_layer_router_then_experts(backend, fmt, hidden, inter, n, k, T, bias):
    """Router (softmax -> top-k -> renormalise) feeding the experts, one call. The
    table's n entries cycle over a pool of at most 12 distinct experts."""
    pool = make_experts(fmt, min(n, 12), hidden, inter, hidden, 21, gen="gauss")
    experts = [pool[i % len(pool)] for i in range(n)]
    table, keep = device_table(backend, fmt, experts)
    w_r = orc.gauss(n * hidden, 31, 0.02)
    b = orc.gauss(n, 32, 1.0) if bias else None
    xs = np.stack([orc.gauss(hidden, 40 + t, 1.0) for t in range(T)])
    d_x = backend.to_device(xs.ravel())
    d_out = backend.alloc(4 * T * hidden)
    d_ids = backend.alloc(4 * T * k)
    d_w = backend.alloc(4 * T * k)
    moe = MoeExecutor(backend)
    moe.layer_device(fmt, table, backend.to_device(w_r), None if b is None else backend.to_device(b), k, T,
                     d_x, d_x, d_out, d_ids, d_w, hidden, inter, hidden)
    backend.synchronize()
    ids = d_ids.download(np.uint32, T * k).reshape(T, k)
    ws = d_w.download(np.float32, T * k).reshape(T, k)
    out = d_out.download(np.float32, T * hidden).reshape(T, hidden)
    for t in range(T):
        rid, rw, _, _ = orc.router(w_r, xs[t], n, hidden, k, bias=b, renormalize=True)
        assert np.array_equal(ids[t], rid)
        np.testing.assert_allclose(ws[t], rw, rtol=1e-5, atol=1e-7)
        sel = [(int(i), float(v)) for i, v in zip(rid, rw)]
        ref = orc.selected_moe(fmt, oracle_experts(fmt, experts), sel, xs[t], hidden, inter, hidden)
        assert_moe_close(out[t] - xs[t], ref)
    del keep


def test_moe_layer_two_streams_in_flight(backend):
    """Two layer calls on two streams of one context, both enqueued before one
    synchronize: each stream has its own router epochs and workspaces, so each
    result equals the oracle's for its own input."""
    fmt, hidden, inter, n, k, T = Q4, 2048, 768, 64, 8, 2
    pool = make_experts(fmt, 12, hidden, inter, hidden, 23, gen="gauss")
    experts = [pool[i % len(pool)] for i in range(n)]
    table, keep = device_table(backend, fmt, experts)
    w_r = orc.gauss(n * hidden, 41, 0.02)
    d_wr = backend.to_device(w_r)
    moe = MoeExecutor(backend)
    runs = []
    for si in range(2):
        xs = np.stack([orc.gauss(hidden, 300 + 10 * si + t, 1.0) for t in range(T)])
        bufs = dict(x=backend.to_device(xs.ravel()), out=backend.alloc(4 * T * hidden), ids=backend.alloc(4 * T * k),
                    w=backend.alloc(4 * T * k))
        runs.append((xs, bufs))
    backend.synchronize()
    for rep in range(3):
        for si, (xs, b) in enumerate(runs):
            moe.layer_device(fmt, table, d_wr, None, k, T, b["x"], b["x"], b["out"], b["ids"], b["w"], hidden, inter,
                             hidden, stream=backend.stream(si))
        for si in range(2):
            backend.synchronize(backend.stream(si))
        for si, (xs, b) in enumerate(runs):
            ids = b["ids"].download(np.uint32, T * k).reshape(T, k)
            out = b["out"].download(np.float32, T * hidden).reshape(T, hidden)
            for t in range(T):
                rid, rw, _, _ = orc.router(w_r, xs[t], n, hidden, k, renormalize=True)
                assert np.array_equal(ids[t], rid), (rep, si, t)
                sel = [(int(i), float(v)) for i, v in zip(rid, rw)]
                ref = orc.selected_moe(fmt, oracle_experts(fmt, experts), sel, xs[t], hidden, inter, hidden)
                assert_moe_close(out[t] - xs[t], ref)
    assert moe.device_error() == 0
    del keep
