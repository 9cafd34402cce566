"""Synthetic inputs of the benchmark configurations (no checkpoints are available).

- zipf_bias: router logit bias ln(Zipf(s) pmf) over a seeded rank permutation of the
  experts, so that expert popularity follows Zipf(s) (Qwen3-A3B-shaped stack).
- fp4_random_split: a DeepSeek split-layout FP4 matrix with nibbles uniform over the
  16 E2M1 codes and E8M0 block scales uniform over raw 119..127 (2^-8 .. 2^0), the
  layout of DeepSeekFp4ExpertWeights (crates/objeta-cuda/src/moe.rs:27-35).
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


def fp4_random_split(rows: int, cols: int, seed: int):
    """(weights [rows * cols / 2] u8, scales [rows * cols / 32] u8) of one split FP4 matrix."""
    rng = np.random.default_rng(seed)
    w = rng.integers(0, 256, size=rows * cols // 2, dtype=np.uint8)
    sc = rng.integers(119, 128, size=rows * cols // 32, dtype=np.uint8)
    return w, sc


def fp4_random_expert(hidden: int, inter: int, out_dim: int, seed: int):
    """(gate_w, gate_s, up_w, up_s, down_w, down_s) of one split FP4 expert."""
    gw, gs = fp4_random_split(inter, hidden, seed)
    uw, us = fp4_random_split(inter, hidden, seed + 1)
    dw, ds = fp4_random_split(out_dim, inter, seed + 2)
    return gw, gs, uw, us, dw, ds
