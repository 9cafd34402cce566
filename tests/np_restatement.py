"""Independent numpy formulation of the reference's CPU quantizers and GEMV, used to
cross-check the C oracle. It is written from the *definitions* rather than from the
bit-level code:

* f32 -> f16 is "round to nearest, ties away from zero" built on numpy's own
  float16 conversion (round to nearest even) with the ties moved, which is what
  f32_to_f16_bits (crates/objeta-cuda/src/quant.rs:1046-1079) computes;
* Rust's f32::round (half away from zero) is evaluated in float64;
* the sequential fp32 dot products of gemv_cpu (quant.rs:627-662, 928-1019) are
  np.cumsum in float32 over rounded products (numpy accumulates left to right).
"""
from __future__ import annotations

import numpy as np

BB = {0: 18, 1: 22, 2: 14, 3: 17}


def f32_to_f16_bits(v) -> np.ndarray:
    v = np.asarray(v, dtype=np.float32).ravel()
    with np.errstate(over="ignore", invalid="ignore"):
        h = v.astype(np.float16)
    hb = h.view(np.uint16).copy()
    finite = np.isfinite(v)
    # neighbours toward zero / away from zero in f16, as float64
    mag = np.abs(v.astype(np.float64))
    hmag = np.abs(h.astype(np.float64))
    down = np.where(hmag > mag, np.nextafter(np.abs(h), np.float16(0)).astype(np.float64), hmag)
    up = np.where(hmag > mag, hmag, np.nextafter(np.abs(h), np.float16(np.inf)).astype(np.float64))
    tie = finite & (mag == (down + up) / 2) & (mag > 0)
    # tie -> the larger magnitude neighbour
    big = np.where(tie, up, hmag).astype(np.float16)
    sign = np.signbit(v)
    fixed = np.where(sign, -big, big).astype(np.float16).view(np.uint16)
    hb = np.where(tie, fixed, hb)
    nan = np.isnan(v)
    hb = np.where(nan, np.where(sign, 0xFE00, 0x7E00), hb)
    return hb.astype(np.uint16)


def f16_bits_to_f32(h) -> np.ndarray:
    return np.asarray(h, dtype=np.uint16).view(np.float16).astype(np.float32)


def rust_round(x64: np.ndarray) -> np.ndarray:
    return np.trunc(x64 + np.copysign(0.5, x64))


def _q(v: np.ndarray, scale: np.ndarray, off: float, hi: float) -> np.ndarray:
    with np.errstate(divide="ignore", invalid="ignore"):
        t = (v / scale[:, None]).astype(np.float32) + np.float32(off)
    r = rust_round(t.astype(np.float64))
    r = np.where(np.isnan(r), 0.0, np.clip(r, 0.0, hi))
    return r.astype(np.uint8)


def quantize(fmt: int, m: np.ndarray, rows: int, cols: int) -> np.ndarray:
    blocks = np.asarray(m, dtype=np.float32).reshape(rows * cols // 32, 32)
    amax = np.max(np.abs(blocks), axis=1, initial=np.float32(0), where=~np.isnan(blocks))
    amax = amax.astype(np.float32)
    n = blocks.shape[0]
    if fmt == 3:
        out = np.zeros((n, 17), np.uint8)
        with np.errstate(divide="ignore"):
            k = np.ceil(np.log2((amax / np.float32(6)).astype(np.float32))).astype(np.float64)
        raw = np.where((amax > 0) & np.isfinite(amax),
                       np.clip(np.nan_to_num(k, neginf=-1e9) + 127, 0, 255), 0).astype(np.uint8)
        scale = np.where(raw == 0, np.float32(2.0 ** -127),
                         (raw.astype(np.uint32) << 23).view(np.float32)).astype(np.float32)
        table = np.array([0, .5, 1, 1.5, 2, 3, 4, 6, -0., -.5, -1, -1.5, -2, -3, -4, -6], np.float32)
        scaled = (blocks / scale[:, None]).astype(np.float32)
        diff = np.abs(scaled[:, :, None] - table[None, None, :])
        q = np.argmin(np.where(np.isnan(diff), np.inf, diff), axis=2).astype(np.uint8)
        out[:, 0] = raw
        out[:, 1:] = q[:, 0::2] | (q[:, 1::2] << 4)
        return out.ravel()
    div = {0: 7.0, 1: 15.0, 2: 4.0}[fmt]
    scale = np.where(amax > 0, (amax / np.float32(div)).astype(np.float32), np.float32(1e-10)).astype(np.float32)
    hb = f32_to_f16_bits(scale)
    out = np.zeros((n, BB[fmt]), np.uint8)
    out[:, 0] = hb & 0xFF
    out[:, 1] = hb >> 8
    if fmt == 0:
        q = _q(blocks, scale, 8.0, 15.0)
        out[:, 2:] = q[:, 0::2] | (q[:, 1::2] << 4)
    elif fmt == 1:
        q = _q(blocks, scale, 16.0, 31.0)
        lo = q & 15
        hi = (q >> 4) & 1
        out[:, 6:] = lo[:, 0::2] | (lo[:, 1::2] << 4)
        bits = hi.reshape(n, 4, 8).astype(np.uint32) << np.arange(8, dtype=np.uint32)
        out[:, 2:6] = bits.sum(axis=2).astype(np.uint8)
    else:
        q = _q(blocks, scale, 4.0, 7.0)
        lo = (q & 3).reshape(n, 8, 4).astype(np.uint32) << (2 * np.arange(4, dtype=np.uint32))
        hi = ((q >> 2) & 1).reshape(n, 4, 8).astype(np.uint32) << np.arange(8, dtype=np.uint32)
        out[:, 2:10] = lo.sum(axis=2).astype(np.uint8)
        out[:, 10:14] = hi.sum(axis=2).astype(np.uint8)
    return out.ravel()


def dequantize(fmt: int, q: np.ndarray, rows: int, cols: int) -> np.ndarray:
    """Dequantized weights w = value * scale as float32 (the reference's `w`)."""
    b = np.asarray(q, np.uint8).reshape(rows * cols // 32, BB[fmt])
    n = b.shape[0]
    if fmt == 3:
        raw = b[:, 0].astype(np.uint32)
        scale = np.where(raw == 0, np.float32(2.0 ** -127), (raw << 23).view(np.float32)).astype(np.float32)
        nib = np.empty((n, 32), np.uint8)
        nib[:, 0::2] = b[:, 1:] & 15
        nib[:, 1::2] = b[:, 1:] >> 4
        table = np.array([0, .5, 1, 1.5, 2, 3, 4, 6, -0., -.5, -1, -1.5, -2, -3, -4, -6], np.float32)
        return (table[nib] * scale[:, None]).astype(np.float32).reshape(rows, cols)
    scale = f16_bits_to_f32(b[:, 0].astype(np.uint16) | (b[:, 1].astype(np.uint16) << 8))
    if fmt == 0:
        q = np.empty((n, 32), np.int32)
        q[:, 0::2] = b[:, 2:] & 15
        q[:, 1::2] = b[:, 2:] >> 4
        v = q - 8
    elif fmt == 1:
        lo = np.empty((n, 32), np.int32)
        lo[:, 0::2] = b[:, 6:] & 15
        lo[:, 1::2] = b[:, 6:] >> 4
        hi = (b[:, 2:6, None] >> np.arange(8)) & 1
        v = (lo | (hi.reshape(n, 32).astype(np.int32) << 4)) - 16
    else:
        lo = (b[:, 2:10, None] >> (2 * np.arange(4))) & 3
        hi = (b[:, 10:14, None] >> np.arange(8)) & 1
        v = (lo.reshape(n, 32).astype(np.int32) | (hi.reshape(n, 32).astype(np.int32) << 2)) - 4
    return (v.astype(np.float32) * scale[:, None]).astype(np.float32).reshape(rows, cols)


def gemv(fmt: int, q: np.ndarray, x: np.ndarray, rows: int, cols: int) -> np.ndarray:
    w = dequantize(fmt, q, rows, cols)
    prod = (w * np.asarray(x, np.float32)[None, :]).astype(np.float32)
    return np.cumsum(prod, axis=1, dtype=np.float32)[:, -1]


def seeded_f32s(n: int, seed: int) -> np.ndarray:
    """seeded_f32s LCG (crates/objeta-cuda/src/bin/bench_qgemv.rs:39-49), in Python ints."""
    out = np.empty(n, np.float32)
    s = seed & 0xFFFFFFFFFFFFFFFF
    for i in range(n):
        s = (s * 6364136223846793005 + 1) & 0xFFFFFFFFFFFFFFFF
        bits = ((s >> 32) | 1) & 0xFFFFFFFF
        unit = np.float32(bits) / np.float32(4294967295.0)
        out[i] = unit * np.float32(2.0) - np.float32(1.0)
    return out
