"""Inputs of the reference's own FP8-activation GEMV tests, regenerated in numpy.

make_fp8_act_fp4_wt_fixture (crates/objeta-cuda/src/quant.rs:1517-1540) draws from the
tests' rand_next LCG. Its scale draw `127u8.saturating_add((r * 10) as i8 as u8)` sends
every negative draw to byte 255 (an infinite E8M0 scale), so most outputs of the
reference fixture are NaN or infinite; `finite_scales=True` gives the same draws with
the scale byte 127 + trunc(r * 10) taken as a signed offset (118..136, all finite)."""
from __future__ import annotations

import numpy as np

from oracle import oracle as orc

F32 = np.float32


def lcg_draws(n: int, seed: int) -> np.ndarray:
    """The reference tests' rand_next (quant.rs:1519-1524), n draws: state = state *
    6364136223846793005 + 1442695040888963407 (mod 2^64); (state >> 33) as f32 /
    u32::MAX as f32 * 2 - 1, all in f32. Vectorised with jump-ahead blocks."""
    a, c, mask = 6364136223846793005, 1442695040888963407, (1 << 64) - 1
    blk = 4096
    A, Cc = np.empty(blk, np.uint64), np.empty(blk, np.uint64)
    ak, ck = 1, 0
    for k in range(blk):  # state_{i+k+1} = A[k] * state_i + C[k]
        ak, ck = (ak * a) & mask, (ck * a + c) & mask
        A[k], Cc[k] = ak, ck
    out = np.empty(n, np.uint64)
    s = np.uint64(seed)
    with np.errstate(over="ignore"):
        for i in range(0, n, blk):
            m = min(blk, n - i)
            st = A[:m] * s + Cc[:m]
            out[i:i + m] = st
            s = st[m - 1]
    bits = (out >> np.uint64(33)).astype(np.uint32)
    return (bits.astype(F32) / F32(4294967295.0)) * F32(2.0) - F32(1.0)


def reference_fp4_fixture(rows: int, cols: int, seed: int, finite_scales: bool = False):
    """make_fp8_act_fp4_wt_fixture (quant.rs:1517-1540): the activation (cols draws *
    100, quantized by cpu_act_quant), packed nibbles ((|r| * 15) as u8 for lo then hi)
    and scales (127u8.saturating_add((r * 10) as i8 as u8), or the signed offset with
    finite_scales). Returns (act codes, act scales, packed weights, weight scales, x)."""
    r = lcg_draws(cols + rows * cols + rows * cols // 32, seed)
    x = r[:cols] * F32(100.0)
    nib = (np.abs(r[cols:cols + rows * cols]) * F32(15.0)).astype(np.uint8)
    packed = ((nib[1::2] << 4) | (nib[0::2] & 15)).astype(np.uint8)
    t = np.trunc(r[cols + rows * cols:] * F32(10.0)).astype(np.int64)
    if finite_scales:
        scales = (127 + t).astype(np.uint8)
    else:
        wrapped = (np.clip(t, -128, 127) & 0xFF).astype(np.int64)
        scales = np.minimum(127 + wrapped, 255).astype(np.uint8)
    av, asc = orc.act_quant(x)
    return av, asc, packed, scales, x
