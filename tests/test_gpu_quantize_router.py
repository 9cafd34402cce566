"""Device quantizer, generators and router against the CPU oracle (bit-exact bytes,
bit-exact expert ids).

Router weights: the device takes each logit from the exact sum of the rounded
products, the reference from a sequential fp32 sum whose own rounding error is
~sqrt(hidden) ulps (~3e-6 at hidden 2048); through the softmax that moves a
weight by up to ~1e-5 relative, hence rtol=2e-5 on the weights (ids are exact)."""
import ctypes as C

import numpy as np
import pytest

from objeta_amd import QGemvShape, QuantFormat, check
from oracle import oracle as orc

pytestmark = pytest.mark.gpu


def _special_matrix(rows, cols, seed):
    m = orc.gauss(rows * cols, seed, 0.02).copy()
    blocks = m.reshape(-1, 32)
    blocks[1] = 0.0                                   # zero block
    blocks[2, 5] = np.nan                             # NaN ignored by amax, q = 0
    blocks[3, 7] = np.inf                             # inf scale
    blocks[4] = np.float32(1e-41)                     # subnormals
    blocks[5] = np.linspace(-7, 7, 32).astype(np.float32)       # scale exactly 1 -> ties
    blocks[6] = (np.arange(32) - 15.5).astype(np.float32) / 2   # .25 steps
    blocks[7, 0] = 6.0 * np.float32(2.0 ** -20) * np.float32(1 + 2 ** -23)  # FP4 exponent edge
    return m


@pytest.mark.parametrize("fmt", [0, 1, 2, 3])
@pytest.mark.parametrize("rows,cols,seed", [(16, 32, 1), (64, 256, 2), (768, 2048, 3)])
def test_device_quantizer_bytes_equal_cpu(quant, fmt, rows, cols, seed):
    m = _special_matrix(rows, cols, seed)
    got = quant.quantize_matrix(QuantFormat(fmt), m, QGemvShape.new(QuantFormat(fmt), rows, cols))
    assert np.array_equal(got, orc.quantize_matrix(fmt, m, rows, cols))


@pytest.mark.parametrize("seed", [0, 42])
def test_device_quantizer_reference_lcg_data(quant, seed):
    # the reference's own test data recipe (seeded_f32s, quant.rs:1610-1662)
    rows, cols = 128, 256
    m = orc.seeded_f32s(rows * cols, seed ^ 0xA5A5_5A5A_1234_5678)
    for fmt in range(4):
        got = quant.quantize_matrix(QuantFormat(fmt), m, QGemvShape.new(QuantFormat(fmt), rows, cols))
        assert np.array_equal(got, orc.quantize_matrix(fmt, m, rows, cols))


def test_gauss_generators_bit_exact(backend):
    L = backend.L
    n = 1 << 16
    d = backend.alloc(n * 4)
    check(L.objeta_hip_fill_gauss_device(backend.ctx, None, d.addr(), n, 1234, 77, C.c_float(0.02)))
    assert np.array_equal(d.download(np.float32, n), orc.gauss(n, 1234, 0.02, first=77))
    rows, cols = 96, 512
    for fmt in range(4):
        nb = rows * cols // 32 * orc.BLOCK_BYTES[fmt]
        dq = backend.alloc(nb)
        check(L.objeta_hip_fill_gauss_quantized_device(backend.ctx, fmt, None, dq.addr(), rows, cols, 99,
                                                       C.c_float(0.02)))
        ref = orc.quantize_matrix(fmt, orc.gauss(rows * cols, 99, 0.02), rows, cols)
        assert np.array_equal(dq.download(np.uint8, nb), ref)


def _router(backend, w, x, bias, ne, hidden, k, tokens, renorm=True):
    L = backend.L
    dw = backend.to_device(w)
    dx = backend.to_device(x)
    db = backend.to_device(bias) if bias is not None else None
    ids = backend.alloc(tokens * k * 4)
    ws = backend.alloc(tokens * k * 4)
    check(L.objeta_hip_router_topk_device(backend.ctx, None, dw.addr(), db.addr() if db else None, dx.addr(),
                                          tokens, ne, hidden, k, 1 if renorm else 0, ids.addr(), ws.addr()))
    return (ids.download(np.uint32, tokens * k).reshape(tokens, k),
            ws.download(np.float32, tokens * k).reshape(tokens, k))


@pytest.mark.parametrize("ne,k,hidden,tokens", [(8, 2, 2048, 16), (128, 8, 2048, 64), (256, 8, 7168, 8),
                                                 (60, 4, 96, 32), (4, 4, 64, 4), (1000, 32, 128, 3)])
@pytest.mark.parametrize("use_bias", [False, True])
def test_router_ids_bit_exact(backend, ne, k, hidden, tokens, use_bias):
    w = orc.gauss(ne * hidden, ne * 31 + hidden, 0.02)
    x = orc.gauss(tokens * hidden, 5, 1.0)
    bias = orc.gauss(ne, 6, 1.0) if use_bias else None
    ids, ws = _router(backend, w, x, bias, ne, hidden, k, tokens)
    for t in range(tokens):
        rid, rw, _, _ = orc.router(w, x[t * hidden:(t + 1) * hidden], ne, hidden, k, bias=bias)
        assert list(ids[t]) == list(rid), f"token {t}"
        assert np.allclose(ws[t], rw, rtol=2e-5, atol=1e-6)


def test_router_exact_ties_keep_lower_index(backend):
    ne, hidden, k = 16, 256, 4
    w = orc.gauss(ne * hidden, 3, 0.02).reshape(ne, hidden).copy()
    for e in (3, 9, 12):
        w[e] = 0.5  # identical rows -> exactly tied logits
    x = np.abs(orc.gauss(hidden, 4, 1.0))
    ids, _ = _router(backend, w.ravel(), x, None, ne, hidden, k, 1)
    rid, _, _, _ = orc.router(w.ravel(), x, ne, hidden, k)
    assert list(ids[0]) == list(rid)
    assert list(ids[0][:3]) == [3, 9, 12]


def test_router_near_ties_take_the_sequential_path(backend):
    """Rows that differ by one ulp in one weight: the parallel bound cannot separate
    them, so the kernel must recompute in the reference's sequential order."""
    ne, hidden, k = 32, 2048, 8
    base = orc.gauss(hidden, 8, 0.02)
    w = np.tile(base, (ne, 1)).astype(np.float32)
    rng = np.random.default_rng(1)
    for e in range(ne):
        j = rng.integers(0, hidden)
        w[e, j] = np.nextafter(w[e, j], np.float32(np.inf) if e % 2 else np.float32(-np.inf))
    tokens = 8
    x = orc.gauss(tokens * hidden, 9, 1.0)
    ids, ws = _router(backend, w.ravel(), x, None, ne, hidden, k, tokens)
    for t in range(tokens):
        rid, rw, _, _ = orc.router(w.ravel(), x[t * hidden:(t + 1) * hidden], ne, hidden, k)
        assert list(ids[t]) == list(rid), f"token {t}"
        assert np.allclose(ws[t], rw, rtol=2e-5, atol=1e-6)


def test_router_selects_exactly_without_the_other_workgroups(monkeypatch):
    """The router's selecting workgroup waits for the other workgroups' logits only up
    to its spin limit; then (a device kept busy by other work) it computes every logit
    itself in the reference's order. With the limit at 0 it never waits, on a context
    of its own: the ids and weights still equal the oracle's for the one-launch shapes
    (hidden 2048 and 7168, one workgroup per expert; hidden 512, one wave per expert)
    and for a two-launch batch, and bit 1 of the device error word reports the path
    (bit 0, a bad id, stays clear)."""
    from objeta_amd import HipBackend, MoeExecutor
    monkeypatch.setenv("OBJETA_HIP_ROUTER_SPIN_LIMIT", "0")
    be = HipBackend(0, 1)
    try:
        for ne, k, hidden, tokens in [(128, 8, 2048, 1), (256, 8, 7168, 1), (64, 4, 512, 1), (128, 8, 2048, 4)]:
            w = orc.gauss(ne * hidden, ne + hidden, 0.02)
            x = orc.gauss(tokens * hidden, hidden + 7, 1.0)
            bias = orc.gauss(ne, 11, 0.5)
            ids, ws = _router(be, w, x, bias, ne, hidden, k, tokens)
            for t in range(tokens):
                rid, rw, _, _ = orc.router(w, x[t * hidden:(t + 1) * hidden], ne, hidden, k, bias=bias)
                assert list(ids[t]) == list(rid), (ne, hidden, t)
                assert np.allclose(ws[t], rw, rtol=2e-5, atol=1e-6), (ne, hidden, t)
            assert MoeExecutor(be).device_error() == 2, (ne, hidden)
    finally:
        be.close()


def test_router_validation(backend):
    from objeta_amd import HipError
    with pytest.raises(HipError) as e:
        _router(backend, np.zeros(8 * 64, np.float32), np.zeros(64, np.float32), None, 8, 64, 9, 1)
    assert e.value.kind == "InvalidInput" and "top_k" in e.value.source_message


@pytest.mark.parametrize("ne,hidden,scale,use_bias", [(64, 256, 150.0, False), (128, 2048, 60.0, True),
                                                      (256, 1024, 80.0, False), (200, 512, 40.0, True)])
def test_router_underflowing_probabilities_order_by_index(backend, ne, hidden, scale, use_bias):
    """Logits spread by hundreds: most softmax probabilities are exactly zero (or
    subnormal) and the reference's stable sort orders equal ones by index, not by
    logit. Only the experts within 110 of the top logit are recomputed in the
    reference's order; the rest have probability exactly 0 there too. Where the
    selection is certain without recomputation, a weight comes from the device's
    logits, which at this magnitude (|l| ~ 400) differ from the sequential sums by a
    few ulps (~1e-4 absolute), and a weight moves by that relative amount: the
    tolerance scales with the ulp of the largest selected logit."""
    k = 8
    w = orc.gauss(ne * hidden, 21 + ne, 0.02).reshape(ne, hidden).copy()
    w *= np.float32(scale)
    tokens = 6
    x = orc.gauss(tokens * hidden, 22 + hidden, 3.0)
    bias = orc.gauss(ne, 23, 1.0) if use_bias else None
    ids, ws = _router(backend, w.ravel(), x, bias, ne, hidden, k, tokens)
    zero_tail = 0
    for t in range(tokens):
        rid, rw, logits, probs = orc.router(w.ravel(), x[t * hidden:(t + 1) * hidden], ne, hidden, k, bias=bias)
        zero_tail += int(np.sum(probs[rid] == 0.0))
        assert list(ids[t]) == list(rid), f"token {t}"
        rtol = 2e-5 + 8 * float(np.spacing(np.float32(np.max(np.abs(logits[rid])))))
        assert np.allclose(ws[t], rw, rtol=rtol, atol=1e-6), f"token {t}"
    assert zero_tail > 0  # the index-ordered zero-probability case is exercised


def _close_calls(ne, hidden, seed, gaps, sd=0.02):
    """W_r whose logits for one token have adjacent top-ranked pairs `gaps` apart
    (closer than the parallel error bound, farther than the probability margin)."""
    w = orc.gauss(ne * hidden, seed, sd).reshape(ne, hidden).copy()
    x = orc.gauss(hidden, seed + 1, 1.0)
    j = int(np.argmax(np.abs(x)))
    for r, gap in gaps:
        logits = orc.router(w.ravel(), x, ne, hidden, 1)[2]
        order = np.argsort(-logits.astype(np.float64), kind="stable")
        a, b = order[r], order[r + 1]
        w[b, j] += np.float32((float(logits[a]) - gap - float(logits[b])) / float(x[j]))
    return w, x


@pytest.mark.parametrize("ne,hidden,seed", [(128, 2048, 31), (128, 2048, 32), (128, 2048, 33), (128, 2048, 34),
                                            (256, 7168, 35), (64, 512, 36), (96, 1000, 37), (96, 999, 38)])
def test_router_close_calls_are_settled_exactly(backend, ne, hidden, seed):
    """Selected experts 3e-5 apart (and one pair at the top-8 boundary): the kernel
    recomputes just those logits in the reference's order and must still agree. The
    shapes take each kernel (one workgroup per expert at hidden 2048 and 7168, one
    wave per expert at 512, the generic kernel at 1000 and 999), rows recomputed in
    one chunk or in several, through 16-byte or (999) 4-byte reads."""
    k = 8
    # shorter rows have smaller bounds: larger weights keep the pairs inside them
    w, x = _close_calls(ne, hidden, seed, [(1, 3e-5), (4, 2e-5), (7, 3e-5)], sd=0.08 if hidden < 2048 else 0.02)
    ids, ws = _router(backend, w.ravel(), x, None, ne, hidden, k, 1)
    rid, rw, logits, _ = orc.router(w.ravel(), x, ne, hidden, k)
    order = np.argsort(-logits.astype(np.float64), kind="stable")
    # each constructed pair lies within the sum of its two logits' error bounds
    # (Higham's recursive-summation bound u * sum_k |S_k| / (1 - n u) over the exact
    # prefix sums S_k of the rounded products), so no bound alone can order it
    u = 2.0 ** -24
    prods = (w * x[None, :]).astype(np.float32).astype(np.float64)
    bound = u * np.abs(np.cumsum(prods, axis=1)).sum(axis=1) / (1 - hidden * u)
    for r in (1, 4, 7):
        a, b = order[r], order[r + 1]
        assert float(logits[a]) - float(logits[b]) < bound[a] + bound[b], (r, hidden)
    assert list(ids[0]) == list(rid)
    assert np.allclose(ws[0], rw, rtol=2e-5, atol=1e-6)


def test_router_softmax_exp_is_glibc_expf(backend):
    """The device softmax's exp equals glibc's expf bit for bit: on every argument of
    [-110, 0] where exp in double rounded once to float does not (97,052 of them), on
    a random sample of the softmax domain, and on the special values."""
    import ctypes as C
    from objeta_amd import check
    hard = orc.expf_double_disagreements(0x80000000, 0xC2DC0000)
    assert hard.size > 90000
    rng = np.random.default_rng(17)
    x = np.concatenate([hard, -rng.exponential(8.0, 1 << 20).astype(np.float32),
                        np.array([0.0, -0.0, -np.inf, -103.97, -103.98, -87.9, -88.1, 1.0, 88.7, np.inf],
                                 np.float32)]).astype(np.float32)
    dx, dy = backend.to_device(x), backend.alloc(4 * x.size)
    check(backend.L.objeta_hip_router_softmax_exp_device(backend.ctx, None, dx.addr(), dy.addr(), x.size))
    y = dy.download(np.float32, x.size)
    want = orc.expf_glibc(x)
    bad = np.nonzero(y.view(np.uint32) != want.view(np.uint32))[0]
    assert bad.size == 0, f"{bad.size} mismatches, first at x={x[bad[0]]!r}: {y[bad[0]]!r} != {want[bad[0]]!r}"


def test_fill_fp4_split_device_matches_host_recipe(backend):
    """The device FP4 generator writes the bytes of the host recipe (workloads.fp4_random_split)."""
    import ctypes as C
    from objeta_amd import check
    from objeta_amd.workloads import fp4_random_split
    for rows, cols, seed in ((7, 96, 3), (2048, 7168, 8001)):
        w, s = fp4_random_split(rows, cols, seed)
        dw, ds = backend.alloc(w.size), backend.alloc(s.size)
        check(backend.L.objeta_hip_fill_fp4_split_device(backend.ctx, None, dw.addr(), ds.addr(), rows, cols, seed))
        assert np.array_equal(dw.download(np.uint8, w.size), w)
        assert np.array_equal(ds.download(np.uint8, s.size), s)
        assert s.min() >= 119 and s.max() <= 127
