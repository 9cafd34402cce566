"""The FP8 "official arithmetic" rules: the oracle against the reference's own
known-answer tests and against what the formats fix, and the device rules
(objeta_amd/csrc/quant_rules.hpp, compiled for the host) against glibc and the
oracle on every input.

Reference tests pinned: test_act_quant_fixture and test_f8e4m3_decode
(crates/objeta-parser/src/deepseek.rs:1351-1395)."""
import os
import shutil
import subprocess

import numpy as np
import pytest

from oracle import oracle as orc

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _decode_formula(c: int) -> float:
    """F8_E4M3 as the reference decodes it (deepseek.rs:799-829), from its definition:
    sign, 4 exponent bits (bias 7), 3 mantissa bits; exponent 0 is mant * 2^-5,
    exponent 15 is +-448."""
    sign = -1.0 if c & 0x80 else 1.0
    e, m = (c >> 3) & 15, c & 7
    if e == 0:
        return sign * m * 2.0 ** -5
    if e == 15:
        return sign * 448.0
    return sign * (1.0 + m / 8.0) * 2.0 ** (e - 7)


def test_f8e4m3_decode_reference_kat():
    # deepseek.rs:1351-1356 and the codes spelled out in test_fp8_gemv_tile_scaled
    d = orc.f8e4m3_to_f32(np.array([0x38, 0x00, 0x40, 0x44, 0x48], np.uint8))
    assert d.tolist() == [1.0, 0.0, 2.0, 3.0, 4.0]


def test_f8e4m3_decode_all_codes():
    d = orc.f8e4m3_to_f32(np.arange(256, dtype=np.uint8))
    want = np.array([_decode_formula(c) for c in range(256)], np.float32)
    assert np.array_equal(d.view(np.uint32), want.view(np.uint32))  # bit for bit, -0.0 at 0x80 included
    assert np.signbit(d[0x80]) and not np.signbit(d[0])


def test_act_quant_reference_fixture():
    # deepseek.rs:1382-1395: block 8; amax 448 -> scale byte 127, amax 2 -> 120
    x = np.array([1.0, 448.0, -448.0, 0.0, 100.0, 200.0, -100.0, -200.0,
                  1.0, 2.0, 0.5, -0.5, 0.0, 0.0, 0.0, 0.0], np.float32)
    y, s = orc.act_quant(x, 8)
    assert y.size == 16 and s.tolist() == [127, 120]
    # with scale 1 the codes are the encoder's: 448 saturates to 0x7E / 0xFE
    assert y[1] == 0x7E and y[2] == 0xFE and y[3] == 0x00 and y[0] == 0x38


def _normal_codes():
    return [c for c in range(256) if 1 <= ((c >> 3) & 15) <= 14]


def test_f8e4m3_encode_round_trips_every_normal_code():
    codes = np.array(_normal_codes(), np.uint8)
    assert np.array_equal(orc.f32_to_f8e4m3(orc.f8e4m3_to_f32(codes)), codes)


def test_f8e4m3_encode_rounds_half_away_at_every_midpoint():
    """Between consecutive normal codes of one sign the midpoint goes to the larger
    magnitude (mantissa rounded half up, deepseek.rs:1462-1467) and the float just
    below it to the smaller."""
    for sign in (0x00, 0x80):
        for c in range(0x08, 0x77):  # exponents 1..14, up to 0x76 -> 0x77
            lo, hi = _decode_formula(sign | c), _decode_formula(sign | (c + 1))
            mid = np.float32((lo + hi) / 2)  # exact: one more mantissa bit
            below = np.nextafter(mid, np.float32(0.0))
            got = orc.f32_to_f8e4m3(np.array([mid, below], np.float32))
            assert got.tolist() == [sign | (c + 1), sign | c], (hex(sign | c), float(mid))


def test_f8e4m3_encode_special_ranges():
    v = np.array([1 / 256, -1 / 256, 1 / 128 - 2 ** -30, 0.0, -0.0,  # below 1/128: signed zero
                  240.0, 255.9, 256.0, 447.9,                         # [240, 448): 0x77
                  448.0, 1e30, np.inf, -448.0, -np.inf,               # saturation
                  np.nan], np.float32)
    got = orc.f32_to_f8e4m3(v).tolist()
    assert got == [0x00, 0x80, 0x00, 0x00, 0x00,
                   0x77, 0x77, 0x77, 0x77,
                   0x7E, 0x7E, 0x7E, 0xFE, 0xFE,
                   0x77]
    # 1/128 itself takes the normal path with exponent field 0, which decodes as zero
    assert orc.f32_to_f8e4m3(np.array([1 / 128], np.float32))[0] == 0x00


def test_act_quant_closed_form_on_random_blocks():
    """Away from the power-of-two boundaries of amax / 448 the block scale is 2^k with
    k = ceil(log2(amax / 448)) exactly, its byte k + 127, and each code the encoding of
    clamp(x / 2^k)."""
    rng = np.random.default_rng(5)
    for sigma in (1e-3, 0.7, 30.0, 2e4):
        x = (rng.standard_normal(128 * 64) * sigma).astype(np.float32)
        y, s = orc.act_quant(x)
        for b in range(64):
            blk = x[128 * b:128 * (b + 1)]
            amax = max(float(np.max(np.abs(blk))), 1e-4)
            r = np.float32(amax) * np.float32(1 / 448)
            k = int(np.ceil(np.log2(np.float64(r))))
            if abs(np.log2(np.float64(r)) - round(np.log2(np.float64(r)))) < 1e-6:
                continue
            assert s[b] == k + 127
            v = np.clip(blk.astype(np.float64) / 2.0 ** k, -448, 448).astype(np.float32)
            assert np.array_equal(y[128 * b:128 * (b + 1)], orc.f32_to_f8e4m3(v))


def test_act_quant_small_and_nonfinite_blocks():
    z = np.zeros(128, np.float32)
    y, s = orc.act_quant(z)
    # amax floor 1e-4: ceil(log2(1e-4 / 448)) = -22
    assert s[0] == 127 - 22 and not y.any()
    nan_blk = np.full(128, np.nan, np.float32)
    nan_blk[3] = 2.0
    y, s = orc.act_quant(nan_blk)
    assert s[0] == 127 + int(np.ceil(np.log2(2.0 / 448)))  # NaN ignored by the maximum
    assert y[3] == orc.f32_to_f8e4m3(np.array([2.0 / 2.0 ** -7], np.float32))[0]
    assert (np.delete(y, 3) == 0x77).all()  # NaN encodes as 0x77
    inf_blk = np.linspace(-3, 3, 128).astype(np.float32)
    inf_blk[7], inf_blk[9] = np.inf, -np.inf
    y, s = orc.act_quant(inf_blk)
    # amax = inf: the saturated exponent wraps the byte to 0 and x / inf is +-0 (code 0)
    assert s[0] == 0
    assert y[7] == 0x77 and y[9] == 0x77  # inf / inf = NaN
    assert not np.delete(y, [7, 9]).any()


def test_quant_rules_match_glibc_and_oracle_on_every_input(tmp_path):
    """The device rules compiled for the host: ceil(log2f(.)) and the act_quant scale on
    every positive finite float, the encoder and an act_quant element on every float
    bit pattern, the decoder on every code."""
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("no host C++ compiler")
    libdir = os.path.join(ROOT, "oracle", "_build")
    orc.lib()  # builds the oracle when missing
    exe = str(tmp_path / "qrc")
    subprocess.run([gxx, "-O2", "-std=c++20", "-fopenmp", "-I", os.path.join(ROOT, "objeta_amd", "csrc"),
                    os.path.join(ROOT, "tests", "native", "quant_rules_check.cpp"), "-L", libdir, "-loracle",
                    f"-Wl,-rpath,{libdir}", "-o", exe], check=True)
    out = subprocess.run([exe], check=True, capture_output=True, text=True).stdout.split("\n")
    rows = [ln.split() for ln in out if ln.strip()]
    assert [r[0] for r in rows] == ["ceil_log2_and_act_scale", "f8e4m3_encode_and_act_code", "f8e4m3_decode"]
    for name, n, first in rows:
        assert int(n) == 0, f"{name}: {n} mismatches, first input bits 0x{first}"
