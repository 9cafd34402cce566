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
