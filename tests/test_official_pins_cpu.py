"""Pins of the oracle's official-arithmetic functions that do not reuse its code.

The oracle (oracle/oracle.c) restates cpu_fp8_act_fp4_weight_gemv_f32
(crates/objeta-parser/src/deepseek.rs:1528-1566), cpu_fp8_act_fp8_weight_gemv
(deepseek.rs:1630-1661) and the routed / shared expert compositions
(deepseek.rs:1664-1716). Each is checked here against:
  * a numpy restatement with its own decode tables, derived from the format
    definitions (E2M1: 1 sign, 2 exponent, 1 mantissa bit; E4M3 as the reference
    decodes it; E8M0 = 2^(raw - 127)), summed in the reference's order with
    numpy's sequential accumulate, compared bit for bit;
  * closed forms: one nonzero weight, so that the output names the nibble, the
    weight-scale byte r * cols / 32 + c / 32, the act-scale byte c / 128 and the
    128 x 128 tile byte (r / 128) * ceil(cols / 128) + c / 128 it used;
  * exact sums: integer-valued cases whose sum no order can round;
  * the composition with glibc's own expf (libm through ctypes) and a SwiGLU limit
    that the gate values exceed, so clamping the gate instead of the up projection
    fails;
  * the reference's FP4 fixture (quant.rs:1517-1540), as drawn and with finite
    scales.
act_quant is pinned on its own (tests/test_fp8_rules_cpu.py) and serves the
compositions here as a component."""
import ctypes
import ctypes.util

import numpy as np
import pytest

from oracle import oracle as orc
from tests.ref_fixtures import reference_fp4_fixture

F32, F64 = np.float32, np.float64


# ------------------------------------------------ decode tables from the formats
def e2m1_table() -> np.ndarray:
    """The 16 E2M1 values: code bit 3 the sign, bits 2..1 the exponent (bias 1), bit
    0 the mantissa; exponent 0 is the subnormal m * 0.5. The negative zero code is
    +0.0 in deepseek.rs:789-792 (and sums the same)."""
    out = np.empty(16, F32)
    for c in range(16):
        e, m = (c >> 1) & 3, c & 1
        mag = m * 0.5 if e == 0 else (1.0 + m / 2.0) * 2.0 ** (e - 1)
        out[c] = -mag if (c & 8) and mag != 0 else mag
    return out


def e4m3_table() -> np.ndarray:
    """The 256 E4M3 codes as the reference decodes them (deepseek.rs:799-829):
    exponent 0 is mant * 2^-5, exponent 15 is +-448, others (1 + m/8) * 2^(e-7)."""
    out = np.empty(256, F32)
    for c in range(256):
        s = -1.0 if c & 0x80 else 1.0
        e, m = (c >> 3) & 15, c & 7
        if e == 0:
            v = m * 2.0 ** -5
        elif e == 15:
            v = 448.0
        else:
            v = (1.0 + m / 8.0) * 2.0 ** (e - 7)
        out[c] = s * v
    return out


def e8m0_table() -> np.ndarray:
    """2^(raw - 127) in f32 (raw 0 is the subnormal 2^-127, raw 255 overflows to inf)."""
    with np.errstate(over="ignore"):
        return np.ldexp(np.ones(256, F64), np.arange(256) - 127).astype(F32)


E2M1, E4M3, E8M0 = e2m1_table(), e4m3_table(), e8m0_table()


def test_own_tables_against_known_values():
    assert E2M1.tolist() == [0, .5, 1, 1.5, 2, 3, 4, 6, 0, -.5, -1, -1.5, -2, -3, -4, -6]
    assert E4M3[[0x38, 0x40, 0x44, 0x48, 0x7E, 0xFE, 0x01, 0x77]].tolist() == [1, 2, 3, 4, 448, -448, 2 ** -5, 240]
    assert E8M0[127] == 1.0 and E8M0[0] == F32(2.0 ** -127) and np.isinf(E8M0[255])


# --------------------------------------------------------- numpy restatements
def np_fp8_act_fp4_gemv(av, asc, w, ws, rows, cols):
    """cpu_fp8_act_fp4_weight_gemv_f32: per row, element c = 2g (low nibble of byte
    g) then 2g + 1 (high nibble); product ((a_v * a_s) * fp4) * w_s in f32; f32 sum
    from 0.0 in element order."""
    phys = w.reshape(rows, cols // 2)
    nib = np.empty((rows, cols), np.uint8)
    nib[:, 0::2] = phys & 15
    nib[:, 1::2] = phys >> 4
    c = np.arange(cols)
    a = E4M3[av[:cols]] * E8M0[asc[c // 128]]
    wsv = E8M0[ws.reshape(rows, cols // 32)[:, c // 32]]
    with np.errstate(all="ignore"):
        prod = (a[None, :] * E2M1[nib]) * wsv
        acc = np.add.accumulate(np.concatenate([np.zeros((rows, 1), F32), prod], axis=1), axis=1, dtype=F32)
    return acc[:, -1]


def np_fp8_act_fp8_gemv(av, asc, w, ws, rows, cols):
    """cpu_fp8_act_fp8_weight_gemv: product ((a_v * a_s) * w_v) * w_s in f64, f64 sum
    from 0.0 in column order, rounded to f32; weight scales on the 128 x 128 tile
    grid [ceil(rows/128)][ceil(cols/128)]."""
    tcols = (cols + 127) // 128
    c, r = np.arange(cols), np.arange(rows)
    a = E4M3[av[:cols]].astype(F64) * E8M0[asc[c // 128]].astype(F64)
    wv = E4M3[w.reshape(rows, cols)].astype(F64)
    wsv = E8M0[ws[(r[:, None] // 128) * tcols + c[None, :] // 128]].astype(F64)
    with np.errstate(all="ignore"):
        prod = (a[None, :] * wv) * wsv
        acc = np.add.accumulate(np.concatenate([np.zeros((rows, 1), F64), prod], axis=1), axis=1)
    return acc[:, -1].astype(F32)


_LIBM = ctypes.CDLL(ctypes.util.find_library("m"))
_LIBM.expf.restype = ctypes.c_float
_LIBM.expf.argtypes = [ctypes.c_float]


def glibc_expf(v) -> np.ndarray:
    return np.array([_LIBM.expf(float(t)) for t in np.asarray(v, F32)], F32)


def np_swiglu(g, u, limit, clamp_gate=False):
    """act = g / (1 + exp(-g)) * clamp(u, -L, L) in f32, left to right, with glibc's
    expf (Rust's f32::exp on Linux); clamp_gate plants the wrong clamp side."""
    g, u = np.asarray(g, F32), np.asarray(u, F32)
    uc = np.clip(u, F32(-limit), F32(limit)).astype(F32)
    gg = np.clip(g, F32(-limit), F32(limit)).astype(F32) if clamp_gate else g
    e = glibc_expf(-gg)
    with np.errstate(all="ignore"):
        return ((gg / (F32(1.0) + e)).astype(F32) * uc).astype(F32)


def np_expert_official(fp8_weights, ex, x, dim, inter, limit, clamp_gate=False):
    gemv = np_fp8_act_fp8_gemv if fp8_weights else np_fp8_act_fp4_gemv
    gw, gs, uw, us, dw, ds = ex
    xq, xs = orc.act_quant(x)
    g = gemv(xq, xs, gw, gs, inter, dim)
    u = gemv(xq, xs, uw, us, inter, dim)
    act = np_swiglu(g, u, limit, clamp_gate)
    aq, asc = orc.act_quant(act)
    return gemv(aq, asc, dw, ds, dim, inter), act, aq, asc, g, u


def same_bits(a, b):
    a, b = np.asarray(a, F32), np.asarray(b, F32)
    return np.array_equal(a.view(np.uint32), b.view(np.uint32))


# ------------------------------------------------------------- FP8 x FP4 GEMV
@pytest.mark.parametrize("rows,cols,seed,lo,hi", [(5, 128, 1, 119, 127), (33, 512, 2, 100, 140),
                                                  (64, 2048, 3, 60, 200), (7, 7168, 4, 1, 254)])
def test_fp8_act_fp4_gemv_numpy_restatement(rows, cols, seed, lo, hi):
    """Random codes and scale bytes over [lo, hi] (subnormal act scales at the low end,
    products far from 1 at the high end)."""
    rng = np.random.default_rng(seed)
    w = rng.integers(0, 256, rows * cols // 2, dtype=np.uint8)
    ws = rng.integers(lo, hi + 1, rows * cols // 32).astype(np.uint8)
    av = rng.integers(0, 256, cols, dtype=np.uint8)
    asc = rng.integers(lo, hi + 1, cols // 128).astype(np.uint8)
    got = orc.fp8_act_fp4_gemv(av, asc, w, ws, rows, cols)
    assert same_bits(got, np_fp8_act_fp4_gemv(av, asc, w, ws, rows, cols))


def test_fp8_act_fp4_gemv_single_weight_closed_form():
    """One nonzero nibble at (r, c): out[r] = a_v[c] * a_s[c/128] * fp4 * w_s[r*cols/32 +
    c/32] exactly, every other row 0. Every scale byte differs from its neighbours and
    every activation code from its neighbour, so a swapped nibble order or a wrong
    scale index gives another value."""
    rows, cols = 6, 512
    rng = np.random.default_rng(11)
    av = (0x30 + (np.arange(cols) % 40)).astype(np.uint8)          # distinct neighbours, all normal
    asc = (120 + np.arange(cols // 128)).astype(np.uint8)          # 120..123
    ws = (100 + (np.arange(rows * cols // 32) * 7) % 50).astype(np.uint8)
    for _ in range(60):
        r, c, q = int(rng.integers(rows)), int(rng.integers(cols)), int(rng.integers(1, 16))
        if q == 8:
            q = 9
        w = np.zeros(rows * cols // 2, np.uint8)
        w[r * cols // 2 + c // 2] = q if c % 2 == 0 else q << 4
        got = orc.fp8_act_fp4_gemv(av, asc, w, ws, rows, cols)
        want = np.zeros(rows, F32)
        want[r] = ((E4M3[av[c]] * E8M0[asc[c // 128]]) * E2M1[q]) * E8M0[ws[r * (cols // 32) + c // 32]]
        assert same_bits(got, want), (r, c, q)


def test_fp8_act_fp4_gemv_exact_integer_sums():
    """Scales 1, integer activation codes (1..15) and half-integer weights: every
    partial sum is a multiple of 0.5 below 2^23, so the f32 sum is exact in any
    order and equals the integer dot product."""
    rows, cols = 16, 2048
    rng = np.random.default_rng(3)
    ints = np.array([1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15], F32)
    codes = np.array([int(np.nonzero(E4M3 == v)[0][0]) for v in ints], np.uint8)
    pick = rng.integers(0, ints.size, cols)
    av = codes[pick]
    w = rng.integers(0, 256, rows * cols // 2, dtype=np.uint8)
    got = orc.fp8_act_fp4_gemv(av, np.full(cols // 128, 127, np.uint8), w, np.full(rows * cols // 32, 127, np.uint8),
                               rows, cols)
    nib = np.empty((rows, cols), np.int64)
    nib[:, 0::2] = w.reshape(rows, -1) & 15
    nib[:, 1::2] = w.reshape(rows, -1) >> 4
    twice = (2 * E2M1[nib]).astype(np.int64)                       # exact: E2M1 values are halves
    exact = (twice * ints[pick].astype(np.int64)[None, :]).sum(axis=1)
    assert np.array_equal(got.astype(F64) * 2, exact.astype(F64))


@pytest.mark.parametrize("rows,cols,seed", [(1, 128, 42), (2, 256, 123), (64, 4096, 7), (96, 2048, 99)])
def test_fp8_act_fp4_gemv_reference_fixture_finite_scales(rows, cols, seed):
    """make_fp8_act_fp4_wt_fixture's draws (quant.rs:1517-1540) with every scale byte
    finite: all outputs finite, bit-equal to the restatement, and within the f32
    recursive-summation bound of the float64 sum."""
    av, asc, w, ws, _ = reference_fp4_fixture(rows, cols, seed, finite_scales=True)
    assert ws.min() >= 118 and ws.max() <= 136
    got = orc.fp8_act_fp4_gemv(av, asc, w, ws, rows, cols)
    assert np.isfinite(got).all()
    assert same_bits(got, np_fp8_act_fp4_gemv(av, asc, w, ws, rows, cols))
    # float64 sum of the same exact products and Higham's bound n * u * sum |p|
    phys = w.reshape(rows, cols // 2)
    nib = np.empty((rows, cols), np.uint8)
    nib[:, 0::2], nib[:, 1::2] = phys & 15, phys >> 4
    c = np.arange(cols)
    p = (E4M3[av].astype(F64) * E8M0[asc[c // 128]]) * E2M1[nib] * E8M0[ws.reshape(rows, -1)[:, c // 32]]
    bound = cols * 2.0 ** -24 * np.abs(p).sum(axis=1) * 1.01
    assert (np.abs(got.astype(F64) - p.sum(axis=1)) <= bound).all()


@pytest.mark.parametrize("rows,cols,seed", [(1, 128, 42), (2, 256, 123), (32, 4096, 7)])
def test_fp8_act_fp4_gemv_reference_fixture_as_drawn(rows, cols, seed):
    """The reference fixture as drawn (saturated 255 scale bytes, infinite scales):
    NaN / inf outputs in the same places and bit-equal values elsewhere."""
    av, asc, w, ws, _ = reference_fp4_fixture(rows, cols, seed)
    assert (ws == 255).any()
    got = orc.fp8_act_fp4_gemv(av, asc, w, ws, rows, cols)
    want = np_fp8_act_fp4_gemv(av, asc, w, ws, rows, cols)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    ok = ~np.isnan(want)
    assert same_bits(got[ok], want[ok])


# ------------------------------------------------------------- FP8 x FP8 GEMV
@pytest.mark.parametrize("rows,cols,seed", [(3, 128, 5), (300, 384, 6), (130, 1024, 7)])
def test_fp8_act_fp8_gemv_numpy_restatement(rows, cols, seed):
    rng = np.random.default_rng(seed)
    w = rng.integers(0, 256, rows * cols, dtype=np.uint8)
    ws = rng.integers(100, 150, ((rows + 127) // 128) * ((cols + 127) // 128)).astype(np.uint8)
    av = rng.integers(0, 256, cols, dtype=np.uint8)
    asc = rng.integers(100, 140, cols // 128).astype(np.uint8)
    got = orc.fp8_act_fp8_gemv(av, asc, w, ws, rows, cols)
    assert same_bits(got, np_fp8_act_fp8_gemv(av, asc, w, ws, rows, cols))


def test_fp8_act_fp8_gemv_single_weight_closed_form():
    """One nonzero code at (r, c) with every 128 x 128 tile's scale byte distinct:
    out[r] names the tile (r / 128, c / 128) of a 3 x 3 grid and the act block c / 128."""
    rows, cols = 300, 384
    tcols = 3
    av = (0x30 + (np.arange(cols) % 40)).astype(np.uint8)
    asc = np.array([121, 124, 126], np.uint8)
    ws = (110 + np.arange(9) * 2).astype(np.uint8)
    rng = np.random.default_rng(13)
    for _ in range(40):
        r, c = int(rng.integers(rows)), int(rng.integers(cols))
        code = int(rng.integers(0x08, 0x77))
        w = np.zeros(rows * cols, np.uint8)
        w[r * cols + c] = code
        got = orc.fp8_act_fp8_gemv(av, asc, w, ws, rows, cols)
        want = np.zeros(rows, F32)
        want[r] = F32(((F64(E4M3[av[c]]) * F64(E8M0[asc[c // 128]])) * F64(E4M3[code]))
                      * F64(E8M0[ws[(r // 128) * tcols + c // 128]]))
        assert same_bits(got, want), (r, c, code)


def test_fp8_act_fp8_gemv_exact_integer_sums():
    rows, cols = 9, 1024
    rng = np.random.default_rng(4)
    ints = np.array([1, 2, 3, 4, 6, 8, 12, 16], F32)
    codes = np.array([int(np.nonzero(E4M3 == v)[0][0]) for v in ints], np.uint8)
    ia, iw = rng.integers(0, ints.size, cols), rng.integers(0, ints.size, rows * cols)
    sign = np.where(rng.integers(0, 2, rows * cols) == 1, 0x80, 0).astype(np.uint8)
    w = (codes[iw] | sign).astype(np.uint8)
    got = orc.fp8_act_fp8_gemv(codes[ia], np.full(cols // 128, 127, np.uint8), w,
                               np.full(((rows + 127) // 128) * (cols // 128), 127, np.uint8), rows, cols)
    wv = (ints[iw].astype(np.int64) * np.where(sign == 0x80, -1, 1)).reshape(rows, cols)
    assert np.array_equal(got.astype(np.int64), (wv * ints[ia].astype(np.int64)[None, :]).sum(axis=1))


# ------------------------------------------------------- expert compositions
def _fp4_expert(dim, inter, seed, lo=118, hi=128):
    rng = np.random.default_rng(seed)
    mats = []
    for rows, cols in ((inter, dim), (inter, dim), (dim, inter)):
        mats.append(rng.integers(0, 256, rows * cols // 2, dtype=np.uint8))
        mats.append(rng.integers(lo, hi, rows * cols // 32).astype(np.uint8))
    return tuple(mats)


def _fp8_expert(dim, inter, seed):
    rng = np.random.default_rng(seed)
    mats = []
    for rows, cols in ((inter, dim), (inter, dim), (dim, inter)):
        mats.append(rng.integers(0, 256, rows * cols, dtype=np.uint8))
        mats.append(rng.integers(112, 122, ((rows + 127) // 128) * ((cols + 127) // 128)).astype(np.uint8))
    return tuple(mats)


@pytest.mark.parametrize("fp8_weights", [False, True])
@pytest.mark.parametrize("dim,inter,seed,limit", [(256, 384, 1, 7.0), (512, 256, 2, 0.75), (384, 128, 3, 1e6)])
def test_expert_official_numpy_composition(fp8_weights, dim, inter, seed, limit):
    """orc_expert_official against the composition restated here: act_quant(x), the
    numpy gate and up GEMVs, SwiGLU with the up projection alone clamped and glibc's
    expf, act_quant of the intermediate, the numpy down GEMV; bit for bit at every
    stage. The limits make gate values exceed them (and up values too, except in the
    unclamped case), so a restatement clamping the gate is shown to differ."""
    ex = _fp8_expert(dim, inter, seed) if fp8_weights else _fp4_expert(dim, inter, seed)
    x = orc.gauss(dim, 100 + seed, 1.0)
    out, pre, aq, asc = orc.expert_official(fp8_weights, ex, x, dim, inter, limit)
    nout, nact, naq, nasc, g, u = np_expert_official(fp8_weights, ex, x, dim, inter, limit)
    assert same_bits(pre, nact)
    assert np.array_equal(aq, naq) and np.array_equal(asc, nasc)
    assert same_bits(out, nout)
    assert np.isfinite(out).all() and np.abs(out).max() > 0
    if limit < 1e5:
        assert (g > limit).any() and (np.abs(u) > limit).any(), "the case must exercise both clamp sides"
        wrong = np_swiglu(g, u, limit, clamp_gate=True)
        assert not same_bits(pre, wrong)


def test_official_swiglu_clamps_only_up_closed_form():
    """x = 448 e_0 quantizes to code 0x7E at scale 1; with gate and up rows 0 holding
    1.0 at column 0 (every tile scale 1) g = u = 448 exactly. At limit 2 the
    oracle's intermediate must be silu(448) * 2 (up clamped, gate not), every other
    intermediate 0."""
    dim, inter = 128, 128
    x = np.zeros(dim, F32)
    x[0] = 448.0
    xq, xs = orc.act_quant(x)
    assert xq[0] == 0x7E and xs[0] == 127
    gw = np.zeros(inter * dim, np.uint8)
    uw = np.zeros(inter * dim, np.uint8)
    gw[0] = uw[0] = 0x38  # 1.0
    one = np.full(1, 127, np.uint8)
    dw = np.zeros(dim * inter, np.uint8)
    out, pre, _, _ = orc.expert_official(True, (gw, one, uw, one, dw, one), x, dim, inter, 2.0)
    g0 = F32(448.0)
    want = F32(g0 / (F32(1.0) + glibc_expf([-g0])[0])) * F32(2.0)
    assert same_bits(pre[:1], np.array([want], F32)) and want == F32(896.0)
    gate_clamped = F32(F32(2.0) / (F32(1.0) + glibc_expf([-2.0])[0])) * F32(2.0)
    assert not same_bits(pre[:1], np.array([gate_clamped], F32))
    assert (pre[1:] == 0).all() and (out == 0).all()
