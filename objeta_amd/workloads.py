"""Synthetic inputs of the benchmark configurations (no checkpoints are available).

- zipf_bias: router logit bias ln(Zipf(s) pmf) over a seeded rank permutation of the
  experts, so that expert popularity follows Zipf(s) (Qwen3-A3B-shaped stack).
- fp4_random_split: a DeepSeek split-layout FP4 matrix with nibbles uniform over the
  16 E2M1 codes and E8M0 block scales uniform over raw 119..127 (2^-8 .. 2^0), the
  layout of DeepSeekFp4ExpertWeights (crates/objeta-cuda/src/moe.rs:27-35); the
  same bytes as the device generator objeta_hip_fill_fp4_split_device.
"""
from __future__ import annotations

import numpy as np


def zipf_bias(n_experts: int, s: float, seed: int) -> np.ndarray:
    """ln of the Zipf(s) pmf over ranks 1..n, assigned to experts by a seeded permutation."""
    ranks = np.arange(1, n_experts + 1, dtype=np.float64)
    pmf = ranks ** (-s)
    pmf /= pmf.sum()
    perm = np.random.default_rng(seed).permutation(n_experts)
    bias = np.empty(n_experts, np.float64)
    bias[perm] = np.log(pmf)
    return bias.astype(np.float32)


_M64 = np.uint64(0xFFFFFFFFFFFFFFFF)


def splitmix64(z: np.ndarray) -> np.ndarray:
    """splitmix64 finaliser over uint64 arrays (wrapping arithmetic)."""
    z = np.asarray(z, np.uint64) + np.uint64(0x9E3779B97F4A7C15)
    z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
    z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return z ^ (z >> np.uint64(31))


def fp4_random_split(rows: int, cols: int, seed: int):
    """(weights [rows * cols / 2] u8, scales [rows * cols / 32] u8): the bytes
    objeta_hip_fill_fp4_split_device writes for the same seed. Weight byte i is byte
    i mod 8 of splitmix64(kw + i / 8); scale byte i is 119 + splitmix64(ks + i) mod 9,
    with kw = splitmix64(seed), ks = splitmix64(seed ^ 0x5CA1E5CA1E5CA1E5)."""
    with np.errstate(over="ignore"):
        kw = splitmix64(np.array([seed], np.uint64))[0]
        ks = splitmix64(np.array([seed ^ 0x5CA1E5CA1E5CA1E5], np.uint64))[0]
        n_w, n_s = rows * cols // 2, rows * cols // 32
        words = splitmix64(kw + np.arange((n_w + 7) // 8, dtype=np.uint64))
        w = words.view(np.uint8)[:n_w].copy()
        sc = (np.uint64(119) + splitmix64(ks + np.arange(n_s, dtype=np.uint64)) % np.uint64(9)).astype(np.uint8)
    return w, sc


def fp4_random_expert(hidden: int, inter: int, out_dim: int, seed: int):
    """(gate_w, gate_s, up_w, up_s, down_w, down_s) of one split FP4 expert."""
    gw, gs = fp4_random_split(inter, hidden, seed)
    uw, us = fp4_random_split(inter, hidden, seed + 1)
    dw, ds = fp4_random_split(out_dim, inter, seed + 2)
    return gw, gs, uw, us, dw, ds


def fp8_random_tiles(rows: int, cols: int, seed: int):
    """(weights [rows * cols] u8, scales [ceil(rows/128) * ceil(cols/128)] u8): random
    F8_E4M3 bytes with E8M0 128 x 128 tile scales in [119, 127], the layout of the
    DeepSeek FP8 shared expert. Weight byte i is byte i mod 8 of splitmix64(kw + i / 8)."""
    with np.errstate(over="ignore"):
        kw = splitmix64(np.array([seed ^ 0xF8F8F8F8], np.uint64))[0]
        ks = splitmix64(np.array([seed ^ 0x5CA1E5CA1E5CA1E5 ^ 0xF8], np.uint64))[0]
        n_w = rows * cols
        n_s = ((rows + 127) // 128) * ((cols + 127) // 128)
        words = splitmix64(kw + np.arange((n_w + 7) // 8, dtype=np.uint64))
        w = words.view(np.uint8)[:n_w].copy()
        sc = (np.uint64(119) + splitmix64(ks + np.arange(n_s, dtype=np.uint64)) % np.uint64(9)).astype(np.uint8)
    return w, sc


def fp8_random_expert(hidden: int, inter: int, out_dim: int, seed: int):
    """(gate_w, gate_s, up_w, up_s, down_w, down_s) of one FP8 shared expert."""
    gw, gs = fp8_random_tiles(inter, hidden, seed)
    uw, us = fp8_random_tiles(inter, hidden, seed + 1)
    dw, ds = fp8_random_tiles(out_dim, inter, seed + 2)
    return gw, gs, uw, us, dw, ds
