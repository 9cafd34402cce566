"""The FP8-activation ("official arithmetic") DeepSeek path on the GPU through the C
ABI, against the oracle's restatement of the reference's CPU definitions
(crates/objeta-parser/src/deepseek.rs:1444-1716).

Bars:
  * act_quant: bit-exact bytes and scales (the reference's own CUDA tests accept up to
    1/8 of the codes differing, crates/objeta-cuda/src/quant.rs:1450-1540);
  * GEMVs: NaN / inf positions identical, finite outputs within 1e-4 * max|ref|;
  * the layer: the intermediate act_quant codes equal the oracle's except where the
    oracle's pre-quantization value lies within 2e-4 (relative) of a code or scale
    boundary (a GEMV summed in another order moves it across), and the output equals
    the oracle's down projections of the device's own intermediate codes within
    1e-4 * max|ref|."""
import ctypes as C

import numpy as np
import pytest

from objeta_amd import ExpertCache, ExpertTable, HipError, MoeExecutor
from objeta_amd.workloads import fp4_random_expert, fp8_random_expert, fp8_random_tiles, fp4_random_split
from oracle import oracle as orc
from tests.ref_fixtures import lcg_draws, reference_fp4_fixture  # noqa: F401

pytestmark = pytest.mark.gpu

F32 = np.float32


@pytest.fixture(scope="module", autouse=True)
def _oracle_threads():
    orc.set_threads(8)
    yield
    orc.set_threads(1)


# ------------------------------------------------------------------ helpers
def assert_gemv_close(out, ref):
    out, ref = np.asarray(out, F32), np.asarray(ref, F32)
    assert np.array_equal(np.isnan(out), np.isnan(ref))
    inf = np.isinf(ref)
    assert np.array_equal(np.isinf(out), inf) and np.array_equal(out[inf], ref[inf])
    fin = np.isfinite(ref)
    if fin.any():
        scale = max(float(np.max(np.abs(ref[fin]))), 1e-30)
        err = float(np.max(np.abs(out[fin].astype(np.float64) - ref[fin].astype(np.float64))))
        assert err <= 1e-4 * scale, f"max rel err {err / scale:.3e}"


def ptr_order(t):
    """(gate_w, gate_s, up_w, up_s, down_w, down_s) -> objeta_hip_expert_ptrs order
    (gate, up, down, gate_scale, up_scale, down_scale)."""
    return (t[0], t[2], t[4], t[1], t[3], t[5])


def e8m0(raw) -> np.ndarray:
    r = np.asarray(raw, np.uint32)
    return np.where(r == 0, np.uint32(1 << 22), r << np.uint32(23)).view(F32)


def dequant(q, s) -> np.ndarray:
    return (orc.f8e4m3_to_f32(q) * np.repeat(e8m0(s), 128)).astype(F32)


def device_act_quant(backend, quant, x, rows, cols, in_place=False):
    dx = backend.to_device(np.ascontiguousarray(x, F32).ravel())
    dv, ds = backend.alloc(rows * cols), backend.alloc(max(1, rows * cols // 128))
    dd = dx if in_place else backend.alloc(4 * rows * cols)
    quant.act_quant_device(None, dx, rows, cols, dv, ds, dd)
    return (dv.download(np.uint8, rows * cols), ds.download(np.uint8, rows * cols // 128),
            dd.download(F32, rows * cols))


# ------------------------------------------------------------------ act_quant
def _assert_act_quant_exact(backend, quant, x, rows, cols, in_place=False):
    q, s, d = device_act_quant(backend, quant, x, rows, cols, in_place)
    rq, rs = orc.act_quant(np.asarray(x, F32).ravel())
    bad = np.nonzero(q != rq)[0]
    assert bad.size == 0, f"{bad.size} code mismatches, first at {bad[0]}: x={x.ravel()[bad[0]]!r}"
    assert np.array_equal(s, rs)
    assert np.array_equal(d.view(np.uint32), dequant(rq, rs).view(np.uint32))


def test_act_quant_reference_cases_bit_exact(backend, quant):
    # test_cuda_act_quant_tiny / _multiblock / _multirow (quant.rs:1450-1515)
    _assert_act_quant_exact(backend, quant, np.arange(1, 129, dtype=F32), 1, 128)
    _assert_act_quant_exact(backend, quant, (np.arange(256, dtype=F32) - F32(128)) * F32(0.5), 1, 256)
    _assert_act_quant_exact(backend, quant, (np.sin(np.arange(4 * 256, dtype=F32)) * F32(100)).astype(F32), 4, 256)


def test_act_quant_edge_blocks_bit_exact(backend, quant):
    rng = np.random.default_rng(11)
    blocks = [np.zeros(128, F32), np.full(128, 1e-5, F32)]
    for sigma in (1e-6, 1e-3, 1.0, 37.0, 3e4, 1e30):
        blocks.append((rng.standard_normal(128) * sigma).astype(F32))
    # the block maximum at and around every power-of-two boundary of amax / 448
    for j in range(-20, 40, 3):
        for amax in (F32(448.0 * 2.0 ** j), np.nextafter(F32(448.0 * 2.0 ** j), F32(0)),
                     np.nextafter(F32(448.0 * 2.0 ** j), F32(np.inf))):
            b = (rng.uniform(-1, 1, 128) * amax).astype(F32)
            b[rng.integers(128)] = amax
            blocks.append(b)
    # code midpoints after scaling, and the floats beside them
    codes = np.array([c for c in range(0x08, 0x77)], np.uint8)
    vals = orc.f8e4m3_to_f32(codes)
    mids = ((vals[:-1].astype(np.float64) + vals[1:]) / 2).astype(F32)
    for k in (-7, 0, 5):
        b = np.concatenate([mids, np.nextafter(mids, F32(0))])[:127] * F32(2.0 ** k)
        blocks.append(np.concatenate([b, [F32(448 * 2.0 ** k)]]).astype(F32))
    # NaN, infinities, subnormals, the largest floats, negative values that underflow
    nan_b = rng.standard_normal(128).astype(F32)
    nan_b[::5] = np.nan
    inf_b = rng.standard_normal(128).astype(F32)
    inf_b[3], inf_b[100] = np.inf, -np.inf
    sub_b = (rng.standard_normal(128) * 1e-40).astype(F32)
    big_b = np.full(128, 3.4e38, F32) * np.sign(rng.standard_normal(128)).astype(F32)
    under_b = np.full(128, -1.4e-45, F32)
    under_b[0] = 900.0  # scale 2^2: -2^-149 / 4 rounds to -0 (code 0x00, not 0x80)
    blocks += [nan_b, inf_b, sub_b, big_b, under_b]
    x = np.concatenate(blocks).astype(F32)
    _assert_act_quant_exact(backend, quant, x, len(blocks), 128)
    _assert_act_quant_exact(backend, quant, x, len(blocks), 128, in_place=True)
    _assert_act_quant_exact(backend, quant, x, 1, x.size)


def test_act_quant_random_rows_bit_exact(backend, quant):
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((33, 7168)) * np.exp(rng.uniform(-8, 8, (33, 1)))).astype(F32)
    _assert_act_quant_exact(backend, quant, x, 33, 7168)


def test_act_quant_rejects_non_multiple_cols(backend, quant):
    # test_cuda_act_quant_rejects_non_multiple_cols (quant.rs:1601-1609)
    with pytest.raises((HipError, ValueError)):
        quant.act_quant(None, np.ones(100, F32), 1, 100)
    dx, dv = backend.alloc(400), backend.alloc(100)
    with pytest.raises(HipError):
        quant.act_quant_device(None, dx, 1, 100, dv, None, None)


def test_act_quant_host_entry_matches_device(backend, quant):
    x = np.arange(1, 257, dtype=F32) * F32(0.37)
    v, s = quant.act_quant(None, x, 2, 128)
    rv, rs = orc.act_quant(x)
    assert np.array_equal(v, rv) and np.array_equal(s, rs)


# ------------------------------------------------------------------ GEMVs
@pytest.mark.parametrize("rows,cols,seed", [(1, 128, 42), (2, 256, 123), (2048, 4096, 7), (4096, 2048, 99)])
def test_fp8_act_fp4_gemv_reference_fixtures(backend, quant, rows, cols, seed):
    """test_fp8_act_fp4_wt_gemv_small / _multiblock / _realistic_gate / _realistic_down
    (quant.rs:1543-1598) on their own fixture. Its scale draws saturate most scale
    bytes to 255 (infinite scales), so most outputs are NaN or infinite: the classes
    must agree and finite outputs meet the relative bar."""
    av, asc, w, ws, _ = reference_fp4_fixture(rows, cols, seed)
    ref = orc.fp8_act_fp4_gemv(av, asc, w, ws, rows, cols)
    d = [backend.to_device(a) for a in (av, asc, w, ws)]
    dy = backend.alloc(4 * rows)
    quant.fp8_act_fp4_weight_gemv_device(None, *d, dy, rows, cols)
    assert_gemv_close(dy.download(F32, rows), ref)


@pytest.mark.parametrize("rows,cols,batch", [(2048, 7168, 1), (7168, 2048, 3), (384, 1024, 2)])
def test_fp8_act_fp4_gemv_random(backend, quant, rows, cols, batch):
    w, ws = fp4_random_split(rows, cols, rows + cols)
    x = orc.gauss(batch * cols, 71 + batch, 1.0)
    av, asc = orc.act_quant(x)
    dy = backend.alloc(4 * rows * batch)
    quant.fp8_act_fp4_weight_gemv_device(None, backend.to_device(av), backend.to_device(asc),
                                         backend.to_device(w), backend.to_device(ws), dy, rows, cols, batch)
    y = dy.download(F32, rows * batch).reshape(batch, rows)
    for b in range(batch):
        ref = orc.fp8_act_fp4_gemv(av[b * cols:(b + 1) * cols], asc[b * cols // 128:(b + 1) * cols // 128],
                                   w, ws, rows, cols)
        assert_gemv_close(y[b], ref)


def test_fp8_weight_codes_exhaustive(backend, quant):
    """Every E4M3 weight code through the device decode: row r holds code r in column
    r mod 16 (so each code sits at several byte positions of a dword across rows) and
    zeros elsewhere, against x = 1.0 (code 0x38, scale 2^0) and weight scale 2^0, so
    y[r] is the decoded value of code r. Expected values from the format's closed form
    (deepseek.rs:799-829): field 0 -> m / 32, field 15 -> 448, else 2^(e-7) (1 + m/8)."""
    rows, cols = 256, 128
    w = np.zeros((rows, cols), np.uint8)
    w[np.arange(rows), np.arange(rows) % 16] = np.arange(rows)
    ws = np.array([0x7F, 0x7F], np.uint8)
    av = np.full(cols, 0x38, np.uint8)
    asc = np.array([127], np.uint8)
    want = []
    for c in range(rows):
        e, m = (c >> 3) & 15, c & 7
        v = m / 32 if e == 0 else (448.0 if e == 15 else 2.0 ** (e - 7) * (1 + m / 8))
        want.append(-v if c & 0x80 else v)
    assert orc.f8e4m3_to_f32(np.arange(rows, dtype=np.uint8)).tolist() == want
    dy = backend.alloc(4 * rows)
    quant.fp8_act_fp8_weight_gemv_device(None, backend.to_device(av), backend.to_device(asc),
                                         backend.to_device(w.ravel()), backend.to_device(ws), dy, rows, cols)
    assert dy.download(F32, rows).tolist() == want


def test_fp8_act_fp8_gemv_tile_scaled_kat(backend, quant):
    """test_fp8_gemv_tile_scaled (deepseek.rs:1359-1380) padded to one 128-column tile:
    rows (1, 2) and (3, 4) at scale 1 against x = (1, 1) quantized. act_quant(1.0) at
    block maximum 1 has scale 2^-8 and code 0x77 (240): x' = 0.9375."""
    w = np.zeros((2, 128), np.uint8)
    w[0, :2] = [0x38, 0x40]
    w[1, :2] = [0x44, 0x48]
    ws = np.array([0x7F], np.uint8)
    x = np.zeros(128, F32)
    x[:2] = 1.0
    av, asc = orc.act_quant(x)
    assert av[0] == 0x77 and asc[0] == 127 - 8
    ref = orc.fp8_act_fp8_gemv(av, asc, w.ravel(), ws, 2, 128)
    assert ref.tolist() == [3 * 0.9375, 7 * 0.9375]
    dy = backend.alloc(8)
    quant.fp8_act_fp8_weight_gemv_device(None, backend.to_device(av), backend.to_device(asc),
                                         backend.to_device(w.ravel()), backend.to_device(ws), dy, 2, 128)
    assert dy.download(F32, 2).tolist() == ref.tolist()


@pytest.mark.parametrize("rows,cols,batch", [(2048, 7168, 1), (7168, 2048, 2), (300, 1024, 3)])
def test_fp8_act_fp8_gemv_random(backend, quant, rows, cols, batch):
    w, ws = fp8_random_tiles(rows, cols, rows * 3 + cols)
    x = orc.gauss(batch * cols, 5 + batch, 1.0)
    av, asc = orc.act_quant(x)
    dy = backend.alloc(4 * rows * batch)
    quant.fp8_act_fp8_weight_gemv_device(None, backend.to_device(av), backend.to_device(asc),
                                         backend.to_device(w), backend.to_device(ws), dy, rows, cols, batch)
    y = dy.download(F32, rows * batch).reshape(batch, rows)
    for b in range(batch):
        ref = orc.fp8_act_fp8_gemv(av[b * cols:(b + 1) * cols], asc[b * cols // 128:(b + 1) * cols // 128],
                                   w, ws, rows, cols)
        assert_gemv_close(y[b], ref)


# ------------------------------------------------------------------ the layer
def justify_intermediate(dev_q, dev_s, pre, delta=2e-4):
    """Checks one intermediate vector's device codes against the oracle's
    pre-quantization values: a scale byte may differ only where the block maximum is
    within delta of a scale boundary, a code only where the value scaled by the
    device's own block scale is within delta of a code boundary. Returns the number
    of codes that differ from the oracle's."""
    ref_q, ref_s = orc.act_quant(pre)
    flips = 0
    for b in range(pre.size // 128):
        blk = pre[128 * b:128 * (b + 1)].astype(np.float64)
        q = dev_q[128 * b:128 * (b + 1)]
        if dev_s[b] != ref_s[b]:
            amax = max(float(np.max(np.abs(blk))), 1e-4)
            around = [orc.act_quant(np.full(128, amax * f, F32))[1][0] for f in (1 - delta, 1 + delta)]
            assert dev_s[b] in around, (b, dev_s[b], ref_s[b], amax)
        v = blk / 2.0 ** (int(dev_s[b]) - 127)
        cands = [orc.f32_to_f8e4m3(np.clip(v * f, -448, 448).astype(F32)) for f in (1 - delta, 1.0, 1 + delta)]
        ok = (q == cands[0]) | (q == cands[1]) | (q == cands[2])
        zero = (q & 0x7F) == 0
        ok |= zero & ((cands[1] & 0x7F) == 0)  # +0 and -0 codes of values that vanish
        assert ok.all(), (b, np.nonzero(~ok)[0][:5], q[~ok][:5], cands[1][~ok][:5])
        flips += int(np.sum(q != ref_q[128 * b:128 * (b + 1)]))
    return flips


def run_official(backend, experts, shared, selections, xs, hidden, inter, out_dim, limit=10.0):
    moe = MoeExecutor(backend)
    keep = [[backend.to_device(a) for a in ex] for ex in experts]
    table = ExpertTable(backend, [ptr_order(k) for k in keep])
    sh_table, sh_keep = None, None
    if shared is not None:
        sh_keep = [backend.to_device(a) for a in shared]
        sh_table = ExpertTable(backend, [ptr_order(sh_keep)])
    T, k = len(selections), len(selections[0])
    ids = np.array([[s[0] for s in sel] for sel in selections], np.uint32).ravel()
    ws = np.array([[s[1] for s in sel] for sel in selections], F32).ravel()
    kk = k + (shared is not None)
    d_ids, d_w = backend.to_device(ids if ids.size else np.zeros(1, np.uint32)), backend.to_device(
        ws if ws.size else np.zeros(1, F32))
    d_x = backend.to_device(np.asarray(xs, F32).ravel())
    d_out = backend.alloc(4 * T * out_dim)
    d_q, d_s = backend.alloc(max(1, T * kk * inter)), backend.alloc(max(1, T * kk * inter // 128))
    moe.official_fp4_device(table, d_ids, d_w, T, k, d_x, d_out, hidden, inter, out_dim, limit, None, sh_table,
                            d_q, d_s)
    backend.synchronize()
    assert moe.device_error() == 0
    return (d_out.download(F32, T * out_dim).reshape(T, out_dim),
            d_q.download(np.uint8, T * kk * inter).reshape(T * kk, inter),
            d_s.download(np.uint8, T * kk * inter // 128).reshape(T * kk, inter // 128))


def check_official(out, q, s, experts, shared, selections, xs, hidden, inter, out_dim, limit=10.0):
    # The oracle's expert composition has one `dim` for input and output (the
    # reference's); only its pre-quantization activation is used here, so it runs at
    # dim = hidden, reading hidden of the down matrix's out_dim rows.
    assert out_dim >= hidden
    T, k = len(selections), len(selections[0])
    flips, total = 0, 0
    for t in range(T):
        x = np.asarray(xs[t], F32)
        ref = np.zeros(out_dim, F32)
        for j, (e, w) in enumerate(selections[t]):
            _, pre, _, _ = orc.expert_official(False, experts[e], x, hidden, inter, limit)
            row = t * k + j
            flips += justify_intermediate(q[row], s[row], pre)
            total += inter
            down = orc.fp8_act_fp4_gemv(q[row], s[row], experts[e][4], experts[e][5], out_dim, inter)
            ref = (ref + F32(w) * down).astype(F32)  # d_out += weight * d_down (moe.rs:1530-1545)
        if shared is not None:
            _, pre, _, _ = orc.expert_official(True, shared, x, hidden, inter, limit)
            row = T * k + t
            flips += justify_intermediate(q[row], s[row], pre)
            total += inter
            down = orc.fp8_act_fp8_gemv(q[row], s[row], shared[4], shared[5], out_dim, inter)
            ref = (ref + down).astype(F32)  # weight 1.0 after the routed sum (moe.rs:1590-1600)
        assert_gemv_close(out[t], ref)
    assert flips <= max(2, total // 1000), f"{flips} of {total} intermediate codes moved"
    return flips


@pytest.mark.parametrize("T,k,with_shared", [(1, 8, True), (2, 6, True), (1, 4, False), (12, 8, True)])
def test_official_layer_deepseek_shape(backend, T, k, with_shared):
    hidden, inter, out_dim, n = 7168, 2048, 7168, 10
    experts = [fp4_random_expert(hidden, inter, out_dim, 900 + 7 * e) for e in range(n)]
    shared = fp8_random_expert(hidden, inter, out_dim, 4242) if with_shared else None
    rng = np.random.default_rng(T * 10 + k)
    selections = [[(int(e), float(w)) for e, w in zip(rng.choice(n, k, replace=False),
                                                      rng.dirichlet(np.ones(k)).astype(F32))] for _ in range(T)]
    xs = orc.gauss(T * hidden, 77 + T, 1.0).reshape(T, hidden)
    out, q, s = run_official(backend, experts, shared, selections, xs, hidden, inter, out_dim)
    check_official(out, q, s, experts, shared, selections, xs, hidden, inter, out_dim)


@pytest.mark.parametrize("T,k,with_shared", [(6, 4, True), (12, 4, True), (33, 3, True), (16, 4, False)])
def test_official_layer_batch_grouped(backend, T, k, with_shared):
    """From 6 tokens on, the layer runs on the grouped-token products: the routed FP4
    experts grouped by expert (about 20 assignments per expert at T=33, so groups span
    several member sets of 8), the FP8 shared expert as one group of all tokens with
    launches of its own. Same bar as the per-token path."""
    hidden, inter, out_dim, n = 512, 384, 640, 5
    experts = [fp4_random_expert(hidden, inter, out_dim, 300 + 3 * e) for e in range(n)]
    shared = fp8_random_expert(hidden, inter, out_dim, 77) if with_shared else None
    rng = np.random.default_rng(T * 7 + k)
    selections = [[(int(e), float(w)) for e, w in zip(rng.choice(n, k, replace=False),
                                                      rng.dirichlet(np.ones(k)).astype(F32))] for _ in range(T)]
    xs = orc.gauss(T * hidden, 91 + T, 2.0).reshape(T, hidden)
    out, q, s = run_official(backend, experts, shared, selections, xs, hidden, inter, out_dim)
    check_official(out, q, s, experts, shared, selections, xs, hidden, inter, out_dim)


def test_official_layer_batch_repeats_limits_and_bad_id(backend):
    """The grouped official path with a token that selects one expert twice, the
    clamp at 0.5 and at 0, and an out-of-table id (error bit 1, that token's output
    NaN, the other tokens unaffected)."""
    hidden, inter, out_dim, n = 256, 256, 384, 4
    experts = [fp4_random_expert(hidden, inter, out_dim, 40 + e) for e in range(n)]
    shared = fp8_random_expert(hidden, inter, out_dim, 41)
    T = 14
    rng = np.random.default_rng(5)
    selections = [[(int(rng.integers(n)), float(rng.uniform(-1, 1))) for _ in range(3)] for _ in range(T)]
    selections[3] = [(2, 0.5), (2, 0.25), (1, 0.25)]
    xs = orc.gauss(T * hidden, 12, 3.0).reshape(T, hidden)
    for limit in (0.5, 0.0):
        out, q, s = run_official(backend, experts, shared, selections, xs, hidden, inter, out_dim, limit)
        check_official(out, q, s, experts, shared, selections, xs, hidden, inter, out_dim, limit)
    moe = MoeExecutor(backend)
    keep = [[backend.to_device(a) for a in ex] for ex in experts]
    table = ExpertTable(backend, [ptr_order(kp) for kp in keep])
    sh_keep = [backend.to_device(a) for a in shared]
    sh_table = ExpertTable(backend, [ptr_order(sh_keep)])
    ids = np.array([[e for e, _ in sel] for sel in selections], np.uint32)
    ids[6, 1] = n + 3
    ws = np.array([[w for _, w in sel] for sel in selections], F32)
    d_out = backend.alloc(4 * T * out_dim)
    moe.official_fp4_device(table, backend.to_device(ids.ravel()), backend.to_device(ws.ravel()), T, 3,
                            backend.to_device(xs.ravel()), d_out, hidden, inter, out_dim, 10.0, None, sh_table)
    backend.synchronize()
    assert moe.device_error() & 1
    out = d_out.download(F32, T * out_dim).reshape(T, out_dim)
    assert np.all(np.isnan(out[6]))
    assert np.all(np.isfinite(np.delete(out, 6, axis=0)))


def test_official_layer_small_shapes_and_limits(backend):
    hidden, inter, out_dim, n = 256, 384, 640, 5
    experts = [fp4_random_expert(hidden, inter, out_dim, 31 + e) for e in range(n)]
    shared = fp8_random_expert(hidden, inter, out_dim, 13)
    selections = [[(4, 0.5), (1, 0.25), (4, 0.25)], [(0, 1.0), (2, -0.5), (3, 0.125)]]  # a repeated expert
    xs = orc.gauss(2 * hidden, 5, 3.0).reshape(2, hidden)
    for limit in (10.0, 0.5, 0.0):
        out, q, s = run_official(backend, experts, shared, selections, xs, hidden, inter, out_dim, limit)
        check_official(out, q, s, experts, shared, selections, xs, hidden, inter, out_dim, limit)


def test_official_layer_shared_only(backend):
    hidden, inter, out_dim = 512, 256, 512
    shared = fp8_random_expert(hidden, inter, out_dim, 99)
    experts = [fp4_random_expert(hidden, inter, out_dim, 1)]
    xs = orc.gauss(3 * hidden, 8, 1.0).reshape(3, hidden)
    moe = MoeExecutor(backend)
    keep = [backend.to_device(a) for a in experts[0]]
    table = ExpertTable(backend, [ptr_order(keep)])
    sh_keep = [backend.to_device(a) for a in shared]
    sh_table = ExpertTable(backend, [ptr_order(sh_keep)])
    d_x, d_out = backend.to_device(xs.ravel()), backend.alloc(4 * 3 * out_dim)
    dummy = backend.to_device(np.zeros(1, np.uint32))
    moe.official_fp4_device(table, dummy, dummy, 3, 0, d_x, d_out, hidden, inter, out_dim, 10.0, None, sh_table)
    out = d_out.download(F32, 3 * out_dim).reshape(3, out_dim)
    for t in range(3):
        ref, _, _, _ = orc.expert_official(True, shared, xs[t], out_dim, inter, 10.0)
        # one expert: the oracle composition differs only through intermediate code flips
        c = orc.compare(ref, out[t])
        assert c["cosine_similarity"] >= 0.999, c


def test_official_layer_rejects_bad_inputs(backend):
    moe = MoeExecutor(backend)
    ex = fp4_random_expert(256, 256, 256, 3)
    keep = [backend.to_device(a) for a in ex]
    table = ExpertTable(backend, [ptr_order(keep)])
    ids, ws = backend.to_device(np.zeros(1, np.uint32)), backend.to_device(np.ones(1, F32))
    dx, do = backend.to_device(np.ones(256, F32)), backend.alloc(4 * 256)
    with pytest.raises(HipError):  # hidden not a multiple of 128
        moe.official_fp4_device(table, ids, ws, 1, 1, dx, do, 224, 256, 256)
    with pytest.raises(HipError):  # negative limit: the reference's clamp(-l, l) panics
        moe.official_fp4_device(table, ids, ws, 1, 1, dx, do, 256, 256, 256, -1.0)


# ------------------------------------------------------------------ executor
def test_official_executor_matches_layer_and_reference_telemetry(backend):
    """execute_selected_moe_official_routed_fp4_cuda (moe.rs:1393-1663): output equal to
    the device layer for the same selection, telemetry by the reference's formulas."""
    hidden, inter, out_dim, n = 512, 256, 384, 6
    experts = [fp4_random_expert(hidden, inter, out_dim, 500 + e) for e in range(n)]
    shared = fp8_random_expert(hidden, inter, out_dim, 600)
    sh_dev = [backend.to_device(a) for a in shared]
    sel = [(3, 0.4), (1, 0.3), (3, 0.2), (5, 0.1)]
    x = orc.gauss(hidden, 41, 1.0)
    moe = MoeExecutor(backend)
    one = sum(a.nbytes for a in experts[0])
    cache = ExpertCache(10 * one, backend)
    out1, t1 = moe.execute_selected_moe_official_routed_fp4(None, None, experts, sel, x, hidden, inter, out_dim, 3,
                                                            cache, ptr_order(sh_dev), 10.0)
    out2, t2 = moe.execute_selected_moe_official_routed_fp4(None, None, experts, sel, x, hidden, inter, out_dim, 3,
                                                            cache, ptr_order(sh_dev), 10.0)
    dev, _, _ = run_official(backend, experts, shared, [sel], x[None, :], hidden, inter, out_dim)
    assert np.array_equal(out1.view(np.uint32), dev[0].view(np.uint32))
    assert np.array_equal(out2.view(np.uint32), dev[0].view(np.uint32))

    single = (inter * hidden // 2) * 2 + (inter * hidden // 32) * 2 + out_dim * inter // 2 + out_dim * inter // 32
    assert single == one
    working = 3 * single  # experts 1, 3, 5
    sh_total = 2 * inter * hidden + out_dim * inter + 2 * (inter * hidden // 128) + out_dim * inter // 128
    for t in (t1, t2):
        assert t["selected_expert_count"] == 4
        assert t["logical_expert_bytes_requested"] == working == t["selected_working_set_bytes"]
        assert t["bytes_per_expert"] == single
        assert t["shared_fp8_bytes_loaded"] == sh_total and t["shared_fp8_bytes_reused"] == 0
        assert t["total_logical_bytes"] == working + sh_total
        assert t["total_loaded_bytes"] == t["routed_fp4_bytes_loaded"] + sh_total
        assert t["total_reused_bytes"] == t["routed_fp4_bytes_reused"]
        assert t["resident_cache_insert_attempt_count"] == 0 and t["dequantized_scratch_bytes"] == 0
        assert t["bytes_by_tensor_kind"] == {"gate": 0, "up": 0, "down": 0}
        assert t["shared_expert_ms"] > 0 and t["total_ms"] > 0
    # call 1: experts 3 and 1 miss, the repeated 3 hits; call 2: everything hits
    assert t1["actual_expert_bytes_loaded"] == 3 * single and t1["resident_cache_bytes_reused"] == single
    assert t1["resident_cache_miss_count"] == 18 and t1["resident_cache_hit_count"] == 6
    assert t2["actual_expert_bytes_loaded"] == 0 and t2["resident_cache_bytes_reused"] == 4 * single
    assert t2["resident_cache_hit_count"] == 6 + 24
    assert t1["weight_bytes_loaded"] + t1["scale_bytes_loaded"] == t1["routed_fp4_bytes_loaded"]
    cache.close()


def test_official_executor_without_cache_or_shared(backend):
    hidden, inter, out_dim = 256, 128, 256
    experts = [fp4_random_expert(hidden, inter, out_dim, 70 + e) for e in range(3)]
    sel = [(2, 0.7), (0, 0.3)]
    x = orc.gauss(hidden, 4, 1.0)
    moe = MoeExecutor(backend)
    out, t = moe.execute_selected_moe_official_routed_fp4(None, None, experts, sel, x, hidden, inter, out_dim, 0)
    dev, q, s = run_official(backend, experts, None, [sel], x[None, :], hidden, inter, out_dim)
    assert np.array_equal(out.view(np.uint32), dev[0].view(np.uint32))
    check_official(dev, q, s, experts, None, [sel], x[None, :], hidden, inter, out_dim)
    assert t["shared_fp8_bytes_loaded"] == 0 and t["shared_expert_ms"] == 0
    assert t["resident_cache_hit_count"] == 0 and t["routed_fp4_bytes_reused"] == 0
    with pytest.raises(HipError):  # expert index out of range
        moe.execute_selected_moe_official_routed_fp4(None, None, experts, [(3, 1.0)], x, hidden, inter, out_dim, 0)
