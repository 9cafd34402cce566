"""The oracle against library routines (numpy float16, numpy argsort) and against the
independent numpy formulation in tests/np_restatement.py."""
import numpy as np
import pytest

from oracle import oracle as orc
from tests import np_restatement as nps


def test_f16_to_f32_all_65536_against_numpy():
    # f16_to_f32_bits (quant.rs:1021-1044) is the IEEE widening; numpy's is too.
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = orc.f16_to_f32_bits(h)
    ref = h.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))
    # NaN payloads are carried (mant << 13), as the bit layout says
    assert np.all(np.isnan(got[nan]))
    assert np.array_equal(got[nan].view(np.uint32) & 0x7FFFFF, (h[nan].astype(np.uint32) & 0x3FF) << 13)


def _f32_to_f16_check(v):
    a = orc.f32_to_f16_bits(v)
    b = nps.f32_to_f16_bits(v)
    bad = np.nonzero(a != b)[0]
    assert bad.size == 0, f"{bad.size} mismatches, first {v[bad[:5]]} {a[bad[:5]]} {b[bad[:5]]}"


def test_f32_to_f16_exhaustive_mantissas_on_boundary_exponents():
    # every f32 mantissa for the exponents where f16 rounding changes regime:
    # underflow to zero, subnormal, first normal, mid range and overflow.
    mant = np.arange(1 << 23, dtype=np.uint32)
    for e in (101, 102, 103, 110, 112, 113, 114, 127, 140, 141, 142, 143):
        for sign in (0, 1):
            bits = (np.uint32(sign) << 31) | (np.uint32(e) << 23) | mant
            _f32_to_f16_check(bits.view(np.float32))


def test_f32_to_f16_random_and_ties():
    rng = np.random.default_rng(5)
    bits = rng.integers(0, 2 ** 32, size=4_000_000, dtype=np.uint64).astype(np.uint32)
    _f32_to_f16_check(bits.view(np.float32))
    # exact ties between f16 neighbours round away from zero (round-half-up on bit 12)
    h = rng.integers(0x0400, 0x7BFF, size=100_000).astype(np.uint16)
    lo = h.view(np.float16).astype(np.float64)
    hi = (h + 1).astype(np.uint16).view(np.float16).astype(np.float64)
    mid = ((lo + hi) / 2).astype(np.float32)
    got = orc.f32_to_f16_bits(mid)
    assert np.array_equal(got, (h + 1).astype(np.uint16))
    assert np.array_equal(orc.f32_to_f16_bits(-mid), ((h + 1) | 0x8000).astype(np.uint16))


def test_f32_to_f16_specials():
    v = np.array([np.inf, -np.inf, np.nan, 0.0, -0.0, 65504.0, 65519.0, 65520.0, 1e9, 2.0 ** -25,
                  2.0 ** -26, 1e-10], np.float32)
    got = orc.f32_to_f16_bits(v)
    assert list(got) == [0x7C00, 0xFC00, 0x7E00, 0x0000, 0x8000, 0x7BFF, 0x7BFF, 0x7C00, 0x7C00,
                         0x0001, 0x0000, 0x0000]


@pytest.mark.parametrize("fmt", [orc.Q4_0, orc.Q5_0, orc.IQ3_0, orc.FP4])
@pytest.mark.parametrize("seed", [0, 1, 123])
def test_quantize_bytes_match_numpy(fmt, seed):
    rows, cols = 64, 256
    m = orc.gauss(rows * cols, seed, 0.02)
    # sprinkle exact zeros, a zero block and a huge value
    m[5] = 0.0
    m[64:96] = 0.0
    m[300] = 3.0
    a = orc.quantize_matrix(fmt, m, rows, cols)
    b = nps.quantize(fmt, m, rows, cols)
    assert np.array_equal(a, b)


@pytest.mark.parametrize("fmt", [orc.Q4_0, orc.Q5_0, orc.IQ3_0])
def test_quantize_rounding_ties(fmt):
    # values landing exactly on .5 after v/scale + offset must round away from zero
    rows, cols = 8, 64
    div = {orc.Q4_0: 7.0, orc.Q5_0: 15.0, orc.IQ3_0: 4.0}[fmt]
    m = np.zeros(rows * cols, np.float32)
    blocks = m.reshape(-1, 32)
    for i, blk in enumerate(blocks):
        blk[0] = div  # amax = div -> scale = 1.0 exactly
        blk[1:] = np.linspace(-div + 0.5, div - 0.5, 31).astype(np.float32)
        blk[1:] = np.round(blk[1:] * 2) / 2 + (0.5 if i % 2 else 0.0)
        np.clip(blk, -div, div, out=blk)
    a = orc.quantize_matrix(fmt, m, rows, cols)
    assert np.array_equal(a, nps.quantize(fmt, m, rows, cols))


@pytest.mark.parametrize("fmt", [orc.Q4_0, orc.Q5_0, orc.IQ3_0])
@pytest.mark.parametrize("rows,cols", [(1, 32), (16, 32), (128, 256), (33, 2048)])
def test_gemv_matches_numpy_cumsum(fmt, rows, cols):
    m = orc.gauss(rows * cols, rows + cols, 0.02)
    x = orc.gauss(cols, 99, 1.0)
    q = orc.quantize_matrix(fmt, m, rows, cols)
    assert np.array_equal(orc.gemv(fmt, q, x, rows, cols), nps.gemv(fmt, q, x, rows, cols))


def test_dense_gemv_against_float64():
    rows, cols = 32, 512
    m = orc.gauss(rows * cols, 3, 0.02)
    x = orc.gauss(cols, 4, 1.0)
    y = orc.dense_gemv(m, x, rows, cols).astype(np.float64)
    ref = m.reshape(rows, cols).astype(np.float64) @ x.astype(np.float64)
    bound = cols * 2.0 ** -24 * (np.abs(m.reshape(rows, cols)) @ np.abs(x)).astype(np.float64)
    assert np.all(np.abs(y - ref) <= bound * 1.01)


def test_fp4_split_gemv_against_float64():
    rows, cols = 16, 256
    rng = np.random.default_rng(8)
    w = rng.integers(0, 256, size=rows * cols // 2, dtype=np.uint8)
    s = rng.integers(119, 128, size=rows * cols // 32, dtype=np.uint8)
    x = orc.gauss(cols, 5, 1.0)
    dec = orc.decode_fp4_split(w, s, rows, cols).reshape(rows, cols).astype(np.float64)
    y = orc.fp4_split_gemv(w, s, x, rows, cols)
    ref = dec @ x.astype(np.float64)
    bound = cols * 2.0 ** -24 * (np.abs(dec) @ np.abs(x.astype(np.float64)))
    assert np.all(np.abs(y - ref) <= bound * 1.01 + 1e-30)


def test_interleaved_fp4_gemv_equals_split_gemv_values():
    rows, cols = 8, 128
    m = orc.gauss(rows * cols, 21, 1.0)
    inter = orc.quantize_matrix(orc.FP4, m, rows, cols)
    w, s = orc.split_interleaved_fp4(inter, rows, cols)
    x = orc.gauss(cols, 22, 1.0)
    a = orc.gemv(orc.FP4, inter, x, rows, cols)
    b = orc.fp4_split_gemv(w, s, x, rows, cols)
    assert np.allclose(a, b, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("ne,k,hidden", [(8, 2, 64), (128, 8, 256), (256, 8, 128)])
def test_router_against_numpy(ne, k, hidden):
    w = orc.gauss(ne * hidden, ne, 0.5)
    x = orc.gauss(hidden, ne + 1, 1.0)
    ids, ws, logits, probs = orc.router(w, x, ne, hidden, k)
    prod = (w.reshape(ne, hidden) * x[None, :]).astype(np.float32)
    lg = np.cumsum(prod, axis=1, dtype=np.float32)[:, -1]
    assert np.array_equal(lg, logits)
    e = np.exp((lg - lg.max()).astype(np.float64))
    p = e / e.sum()
    order = np.argsort(-p, kind="stable")[:k]
    assert list(ids) == list(order)
    assert np.allclose(ws, p[order] / p[order].sum(), rtol=1e-5)
    assert abs(float(ws.astype(np.float64).sum()) - 1.0) < 1e-6


def test_router_ties_keep_lower_index():
    ne, hidden = 6, 8
    w = np.zeros(ne * hidden, np.float32)
    for e in (1, 2, 4):
        w[e * hidden:(e + 1) * hidden] = 1.0  # identical rows -> identical logits
    ids, _, _, _ = orc.router(w, np.ones(hidden, np.float32), ne, hidden, 3)
    assert list(ids) == [1, 2, 4]


def test_router_bias_shifts_selection():
    ne, hidden = 4, 8
    w = np.zeros(ne * hidden, np.float32)
    bias = np.array([0.0, 0.0, 5.0, 0.0], np.float32)
    ids, _, logits, _ = orc.router(w, np.ones(hidden, np.float32), ne, hidden, 1, bias=bias)
    assert ids[0] == 2 and logits[2] == 5.0


def test_gauss_generator_statistics_and_determinism():
    g = orc.gauss(1_000_000, 7, 1.0)
    assert abs(g.mean()) < 3e-3 and abs(g.std() - 1.0) < 3e-3
    assert np.array_equal(g[500:600], orc.gauss(100, 7, 1.0, first=500))
    s = orc.gauss(1000, 7, 0.02)
    assert np.array_equal(s, (g[:1000] * np.float32(0.02)).astype(np.float32))


_LIBM = None


def _expf(v: np.ndarray) -> np.ndarray:
    """glibc expf element-wise through its own symbol (Rust's f32::exp calls it on Linux)."""
    global _LIBM
    import ctypes
    if _LIBM is None:
        _LIBM = ctypes.CDLL("libm.so.6")
        _LIBM.expf.restype = ctypes.c_float
        _LIBM.expf.argtypes = [ctypes.c_float]
    return np.array([_LIBM.expf(float(a)) for a in np.asarray(v, np.float32)], np.float32)


def _np_split_fp4_gemv(w, s, x, rows, cols):
    """Dense sequential row sums over the decoded split FP4 matrix (table value * 2^(raw-127))."""
    table = np.array([0, .5, 1, 1.5, 2, 3, 4, 6, -0., -.5, -1, -1.5, -2, -3, -4, -6], np.float32)
    b = np.asarray(w, np.uint8).reshape(rows, cols // 2)
    nib = np.empty((rows, cols), np.uint8)
    nib[:, 0::2] = b & 15
    nib[:, 1::2] = b >> 4
    raw = np.asarray(s, np.uint8).reshape(rows, cols // 32).astype(np.uint32)
    scale = np.where(raw == 0, np.float32(2.0 ** -127), (raw << 23).view(np.float32)).astype(np.float32)
    dec = (table[nib] * np.repeat(scale, 32, axis=1)).astype(np.float32)
    prod = (dec * np.asarray(x, np.float32)[None, :]).astype(np.float32)
    return np.cumsum(prod, axis=1, dtype=np.float32)[:, -1]


def _np_selected_moe(fmt, experts, sel, x, hidden, inter, out_dim):
    """selected_moe_cpu (moe.rs:1283-1324) / selected_moe_cpu_native_fp4 (moe.rs:1665-1735)
    composed from independent numpy parts: gate and up GEMVs, act = g / (1 + exp(-g)) * u
    in float32 operations, down GEMV, out += w * down in selection order."""
    out = np.zeros(out_dim, np.float32)
    for e, wt in sel:
        ex = experts[e]
        if fmt == orc.FP4:
            g = _np_split_fp4_gemv(ex[0], ex[1], x, inter, hidden)
            u = _np_split_fp4_gemv(ex[2], ex[3], x, inter, hidden)
        else:
            g = nps.gemv(fmt, ex[0], x, inter, hidden)
            u = nps.gemv(fmt, ex[1], x, inter, hidden)
        act = ((g / (np.float32(1.0) + _expf(-g))).astype(np.float32) * u).astype(np.float32)
        if fmt == orc.FP4:
            d = _np_split_fp4_gemv(ex[4], ex[5], act, out_dim, inter)
        else:
            d = nps.gemv(fmt, ex[2], act, out_dim, inter)
        out = (out + (np.float32(wt) * d).astype(np.float32)).astype(np.float32)
    return out


@pytest.mark.parametrize("fmt", [orc.Q4_0, orc.Q5_0, orc.IQ3_0, orc.FP4])
@pytest.mark.parametrize("with_shared", [False, True])
def test_selected_moe_matches_numpy_composition(fmt, with_shared):
    """orc_selected_moe pinned on its own: expert indexing, gate/up order, SiLU, the
    slot-ordered combine and the shared expert (one more slot of weight 1.0 after the
    routed ones, moe.rs:1552-1600) against a numpy composition, bit for bit. A swapped
    gate/up, a dropped slot or a reordered combine changes the bits."""
    hidden, inter, out_dim, n = 128, 96, 64, 5
    experts = []
    for e in range(n):
        if fmt == orc.FP4:
            rng = np.random.default_rng(40 + e)
            mats = []
            for r, c in ((inter, hidden), (inter, hidden), (out_dim, inter)):
                mats += [rng.integers(0, 256, size=r * c // 2, dtype=np.uint8),
                         rng.integers(119, 128, size=r * c // 32, dtype=np.uint8)]
            experts.append(tuple(mats))
        else:
            experts.append(tuple(orc.quantize_matrix(fmt, orc.gauss(r * c, 100 * e + i, 0.05), r, c)
                                 for i, (r, c) in enumerate(((inter, hidden), (inter, hidden), (out_dim, inter)))))
    x = orc.gauss(hidden, 7, 1.0)
    sel = [(3, 0.4), (1, 0.35), (3, 0.15), (0, 0.1)]
    shared = experts[4] if with_shared else None
    got = orc.selected_moe(fmt, experts[:4], sel, x, hidden, inter, out_dim, shared=shared)
    want_sel = sel + ([(4, 1.0)] if with_shared else [])
    want = _np_selected_moe(fmt, experts, want_sel, x, hidden, inter, out_dim)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # a plausible mistake changes the bits: gate and up swapped
    swapped = [(ex[1], ex[0], ex[2]) if fmt != orc.FP4 else (ex[2], ex[3], ex[0], ex[1], ex[4], ex[5])
               for ex in experts]
    assert not np.array_equal(_np_selected_moe(fmt, swapped, want_sel, x, hidden, inter, out_dim), want)


def test_expf_restatement_matches_glibc_exhaustively_on_softmax_domain():
    """The router's softmax evaluates exp(l - max) with l - max in [-inf, 0]. The
    restatement of glibc's expf method (the device's form) agrees with glibc's expf on
    every float in [-110, 0]; exp in double rounded once to float does not (the
    disagreements exist, so a ranking built on it could break a probability tie
    differently from the reference)."""
    restated, dbl = orc.expf_range_check(0x80000000, 0xC2DC0000)  # -0 .. -110
    assert restated == 0
    assert dbl > 90000
    # below -110 glibc underflows to exactly 0 (from below log(2^-150) ~ -103.97)
    restated, _ = orc.expf_range_check(0xC2DC0001, 0xC3000000)  # -110 .. -128
    assert restated == 0


def test_expf_restatement_specials_and_positive_sample():
    x = np.array([0.0, -0.0, -np.inf, np.inf, 88.72, 88.73, -103.97, -103.98, 1e-30, -1e-30, 1.0, -1.0, 10.0, 50.5],
                 np.float32)
    rng = np.random.default_rng(3)
    x = np.concatenate([x, rng.uniform(-90, 88, 200000).astype(np.float32),
                        rng.uniform(-1e-3, 1e-3, 50000).astype(np.float32)])
    assert np.array_equal(orc.expf_restated(x).view(np.uint32), orc.expf_glibc(x).view(np.uint32))
    assert np.isnan(orc.expf_restated(np.array([np.nan], np.float32))[0])
