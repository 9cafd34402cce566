"""The oracle against the reference's own known-answer tests and closed forms.

Each test names the reference test or code it pins (paths relative to the
reference repository)."""
import numpy as np
import pytest

from oracle import oracle as orc
from tests import np_restatement as nps


# --- exact-byte FP4 tests, crates/objeta-cuda/src/quant.rs:1860-1900
def test_fp4_nibble_order():
    b = np.zeros(32, np.float32)
    b[0], b[1], b[2] = 0.5, 1.5, 6.0
    q = orc.quantize_block(orc.FP4, b)
    assert q[0] == 127 and q[1] == (1 | (3 << 4))


def test_fp4_positive_negative_values():
    b = np.zeros(32, np.float32)
    b[:4] = [6.0, -6.0, 2.0, -2.0]
    q = orc.quantize_block(orc.FP4, b)
    assert q[0] == 127 and q[1] == (7 | (15 << 4)) and q[2] == (4 | (12 << 4))


def test_fp4_multiple_scale_blocks():
    m = np.zeros(128, np.float32)
    m[:32] = np.arange(32, dtype=np.float32) / 32 * 6.0
    m[32:64] = np.arange(32, dtype=np.float32) / 32 * 12.0
    q = orc.quantize_matrix(orc.FP4, m, 2, 64)
    assert q[0] == 127 and q[17] == 128


@pytest.mark.parametrize("fmt", [orc.Q4_0, orc.IQ3_0, orc.FP4])
def test_rejects_non_multiple_cols(fmt):
    # q4/iq3/fp4_rejects_non_multiple_cols, quant.rs:1665-1670,1802-1807,1903-1908
    with pytest.raises(orc.OracleError) as e:
        orc.quantize_matrix(fmt, np.zeros(4 * 33, np.float32), 4, 33)
    assert "multiple of block_size" in e.value.source_message
    assert e.value.kind == "InvalidInput"


# --- FP4 expert bytes, crates/objeta-cuda/src/moe.rs:2465-2469
def test_fp4_expert_bytes():
    h, i, o = 256, 512, 256
    total = 2 * (i * h // 2 + i * h // 32) + (o * i // 2 + o * i // 32)
    assert total == 208896


# --- cpu_router, crates/objeta-cuda/src/bin/deepseek_single_layer_moe.rs:3415-3445
def test_cpu_router_top_k_selection():
    hidden, ne = 4, 4
    w = np.zeros(ne * hidden, np.float32)
    w[1 * hidden:2 * hidden] = 1.0
    w[3 * hidden:4 * hidden] = 2.0
    ids, ws, _, _ = orc.router(w, np.full(hidden, 0.5, np.float32), ne, hidden, 2, renormalize=False)
    assert list(ids) == [3, 1]
    assert ws[0] > ws[1]


# --- smoke GEMV exact outputs, crates/objeta-cuda/src/lib.rs:157-185
def test_smoke_dense_gemv():
    m = np.array([1, 2, 3, 4, -1, .5, 0, 2, 3, -2, 1, .25], np.float32)
    v = np.array([.5, -1, 2, 1.5], np.float32)
    y = orc.dense_gemv(m, v, 3, 4)
    assert np.allclose(y, [1 * .5 - 2 + 6 + 6, -.5 - .5 + 0 + 3, 1.5 + 2 + 2 + .375], atol=1e-5)


# --- CPU round trips, quant.rs:1673-1712,1810-1828 (cosine vs dense)
@pytest.mark.parametrize("fmt,mseed,xseed,thr", [(orc.Q4_0, 42, 7, 0.995), (orc.Q5_0, 43, 8, 0.998),
                                                   (orc.IQ3_0, 44, 9, 0.970)])
def test_cpu_reference_roundtrip_small(fmt, mseed, xseed, thr):
    rows, cols = 16, 32
    m = orc.seeded_f32s(rows * cols, mseed)
    x = orc.seeded_f32s(cols, xseed)
    q = orc.quantize_matrix(fmt, m, rows, cols)
    y = orc.gemv(fmt, q, x, rows, cols)
    dense = orc.dense_gemv(m, x, rows, cols)
    assert orc.compare(dense, y)["cosine_similarity"] > thr


# --- q5_is_no_worse_than_q4_on_same_case, quant.rs:1773-1799
def test_q5_no_worse_than_q4():
    rows, cols, seed = 128, 256, 77
    m = orc.seeded_f32s(rows * cols, seed ^ 0x1234_5678_9ABC_DEF0)
    x = orc.seeded_f32s(cols, seed ^ 0x0BAD_F00D_1234_5678)
    dense = orc.dense_gemv(m, x, rows, cols)
    q4 = orc.gemv(orc.Q4_0, orc.quantize_matrix(orc.Q4_0, m, rows, cols), x, rows, cols)
    q5 = orc.gemv(orc.Q5_0, orc.quantize_matrix(orc.Q5_0, m, rows, cols), x, rows, cols)
    n4, n5 = orc.compare(dense, q4), orc.compare(dense, q5)
    assert n5["cosine_similarity"] >= n4["cosine_similarity"] - 1e-6
    assert n5["relative_l2_error"] <= n4["relative_l2_error"] + 1e-6


# --- closed forms
def test_zero_block_closed_form():
    # amax = 0 -> scale 1e-10, below the f16 range -> stored 0x0000; q = round(0 + 8) = 8
    q = orc.quantize_block(orc.Q4_0, np.zeros(32, np.float32))
    assert q[0] == 0 and q[1] == 0 and np.all(q[2:] == 0x88)
    q5 = orc.quantize_block(orc.Q5_0, np.zeros(32, np.float32))
    assert q5[0] == 0 and q5[1] == 0 and np.all(q5[2:6] == 0xFF) and np.all(q5[6:] == 0)  # q=16: hi=1, lo=0
    q3 = orc.quantize_block(orc.IQ3_0, np.zeros(32, np.float32))
    assert np.all(q3[2:10] == 0) and np.all(q3[10:14] == 0xFF)  # q=4: lo=0, hi=1


@pytest.mark.parametrize("a", [0.5, -3.25, 1e-3, 7.0, 123.456])
def test_single_value_block_closed_form(a):
    b = np.zeros(32, np.float32)
    b[0] = a
    q = orc.quantize_block(orc.Q4_0, b)
    scale = np.float32(abs(a)) / np.float32(7.0)
    hb = int(nps.f32_to_f16_bits(np.array([scale]))[0])
    assert (int(q[0]) | (int(q[1]) << 8)) == hb
    assert (q[2] & 15) == (15 if a > 0 else 1)  # round(+-7 + 8)
    assert np.all(q[3:] == 0x88) and (q[2] >> 4) == 8


def test_quantized_matrix_bytes_closed_form():
    for fmt, bb in orc.BLOCK_BYTES.items():
        rows, cols = 5, 96
        q = orc.quantize_matrix(fmt, np.ones(rows * cols, np.float32), rows, cols)
        assert q.size == rows * (cols // 32) * bb


def test_fp4_decode_all_codes_and_scales():
    # every FP4 decode is exact: table value * 2^(e-127)
    table = [0, .5, 1, 1.5, 2, 3, 4, 6, 0, -.5, -1, -1.5, -2, -3, -4, -6]
    for raw in range(256):
        s = orc.decode_f8_e8m0(raw)
        assert s == orc.f8e8m0_to_f32(raw)  # the two reference decodes agree on all bytes
        exp = 2.0 ** (raw - 127) if raw < 255 else np.inf
        assert np.float32(s) == np.float32(exp)
    w = np.arange(16, dtype=np.uint8)
    w = (w[0::2] | (w[1::2] << 4)).astype(np.uint8)  # 8 bytes, codes 0..15
    w = np.concatenate([w, w]).astype(np.uint8)  # one 32-wide row
    for raw in (1, 100, 127, 140, 254):
        dec = orc.decode_fp4_split(w, np.array([raw], np.uint8), 1, 32)
        with np.errstate(over="ignore"):
            expect = (np.array(table * 2, np.float64) * 2.0 ** (raw - 127)).astype(np.float32)
        assert np.array_equal(dec, expect)


def test_compare_outputs_definition():
    r = np.array([1, 2, 3], np.float32)
    a = np.array([1, 2, 4], np.float32)
    c = orc.compare(r, a)
    assert c["cosine_similarity"] == pytest.approx(17 / np.sqrt(14 * 21), rel=1e-6)
    assert c["relative_l2_error"] == pytest.approx(1 / np.sqrt(14), rel=1e-6)
    assert c["max_abs_error"] == 1.0
    z = orc.compare(np.zeros(3, np.float32), np.zeros(3, np.float32))
    assert z["cosine_similarity"] == 1.0 and z["relative_l2_error"] == 0.0


def test_seeded_f32s_matches_independent_lcg():
    for seed in (0, 1, 123, 0xDEADBEEF ^ 5):
        assert np.array_equal(orc.seeded_f32s(64, seed), nps.seeded_f32s(64, seed))
