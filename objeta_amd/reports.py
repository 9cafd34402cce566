"""Benchmark reports in the reference's JSON schemas, so that tooling written for the
reference's benches reads this build's results unchanged.

- QGemvStats / QGemvStatsTelemetry / QGemvStatsReport
  (crates/objeta-cuda/src/bin/bench_qgemv.rs:6-37), QGemvNumerics /
  QGemvNumericsSuite (crates/objeta-cuda/src/quant.rs:156-170);
- MoeStats / MoeStatsTelemetry / MoeStatsReport
  (crates/objeta-cuda/src/bin/bench_selected_moe.rs:19-101), with MoeTelemetry and
  BytesByTensorKind (crates/objeta-cuda/src/moe.rs:229-276).

Field names and their order are the reference's (serde serialises struct fields in
declaration order, and QuantFormat as its variant name). The functions only format
values measured elsewhere; `numerics` is a QGemvNumericsSuite dict or None (then
every comparison field is NaN, which serialises as the JSON token NaN: no check ran).
"""
from __future__ import annotations

import math

import numpy as np

FORMAT_NAMES = ("Q4_0", "Q5_0", "IQ3_0", "DeepSeekFp4E2M1")
BLOCK_BYTES = {"Q4_0": 18, "Q5_0": 22, "IQ3_0": 14, "DeepSeekFp4E2M1": 17}


def percentile_index(p: float, n: int) -> int:
    """(p * (n - 1) as f32).round() as usize: the product in f32, rounded half away
    from zero as Rust's f32::round does (bench_qgemv.rs:59-65)."""
    v = np.float32(p) * np.float32(n - 1)
    r = np.floor(v)
    return int(r) + (1 if v - r >= np.float32(0.5) else 0)


def stats(values) -> dict:
    """QGemvStats / MoeStats: avg, min, max, p50, p95 with compute_stats' percentile
    rule over the sorted values (bench_qgemv.rs:59-100)."""
    v = sorted(float(x) for x in values)
    if not v:
        return {"avg": 0.0, "min": 0.0, "max": 0.0, "p50": 0.0, "p95": 0.0}
    return {"avg": sum(v) / len(v), "min": v[0], "max": v[-1], "p50": v[percentile_index(0.50, len(v))],
            "p95": v[percentile_index(0.95, len(v))]}


def numerics_suite(cuda_vs_cpu_quant: dict | None, quant_vs_fp32: dict | None) -> dict:
    """QGemvNumericsSuite (quant.rs:163-170): the top-level fields repeat cuda_vs_cpu_quant."""
    nan = {"cosine_similarity": math.nan, "relative_l2_error": math.nan, "max_abs_error": math.nan}
    a = dict(cuda_vs_cpu_quant or nan)
    b = dict(quant_vs_fp32 or nan)
    keys = ("cosine_similarity", "relative_l2_error", "max_abs_error")
    return {"cosine_similarity": a[keys[0]], "relative_l2_error": a[keys[1]], "max_abs_error": a[keys[2]],
            "cuda_vs_cpu_quant": {k: a[k] for k in keys}, "quant_vs_fp32": {k: b[k] for k in keys}}


def qgemv_stats_report(backend: str, kernel: str, fmt: str, rows: int, cols: int, kernel_ms, bytes_read: int,
                       numerics: dict | None, h2d_ms=None, d2h_ms=None, unaccounted_ms=None,
                       total_ms=None) -> dict:
    """QGemvStatsReport (bench_qgemv.rs:27-37). Per-iteration millisecond samples;
    missing phases (device-resident runs have no copies) are zeros; total defaults to
    the kernel samples. effective_gbps = bytes_read / average kernel time, as
    run_benchmark_for_shape computes it (bench_qgemv.rs:164-170)."""
    if fmt not in FORMAT_NAMES:
        raise ValueError(f"unknown format {fmt}")
    k = list(kernel_ms)
    zeros = [0.0] * len(k)
    ks = stats(k)
    tel = {"h2d_ms": stats(h2d_ms if h2d_ms is not None else zeros),
           "kernel_ms": ks,
           "d2h_ms": stats(d2h_ms if d2h_ms is not None else zeros),
           "unaccounted_ms": stats(unaccounted_ms if unaccounted_ms is not None else zeros),
           "total_ms": stats(total_ms if total_ms is not None else k),
           "bytes_read": int(bytes_read),
           "effective_gbps": (bytes_read / (ks["avg"] / 1000.0) / 1e9) if ks["avg"] > 0 else 0.0}
    return {"backend": backend, "kernel": kernel, "format": fmt, "rows": int(rows), "cols": int(cols),
            "block_size": 32, "block_bytes": BLOCK_BYTES[fmt], "telemetry": tel,
            "numerics": numerics if numerics is not None else numerics_suite(None, None)}


_MOE_TEL_FIELDS = (
    "selected_expert_count", "logical_expert_bytes_requested", "actual_expert_bytes_loaded",
    "resident_cache_bytes_reused", "weight_bytes_loaded", "weight_bytes_reused", "scale_bytes_loaded",
    "scale_bytes_reused", "resident_cache_resident_bytes", "resident_cache_capacity_bytes",
    "resident_cache_hit_count", "resident_cache_miss_count", "resident_cache_eviction_count",
    "resident_cache_insert_attempt_count", "resident_cache_insert_accept_count",
    "resident_cache_insert_bypass_count", "resident_cache_oversized_tensor_bypass_count",
    "resident_cache_oversized_expert_bypass_count", "resident_cache_self_eviction_risk_count",
    "dequantized_scratch_bytes", "h2d_ms", "gate_up_qgemv_ms", "activation_ms", "down_qgemv_ms", "accum_ms",
    "unaccounted_ms", "total_ms", "shared_expert_ms", "bytes_by_tensor_kind", "bytes_per_expert",
    "selected_working_set_bytes", "routed_fp4_bytes_loaded", "routed_fp4_bytes_reused", "shared_fp8_bytes_loaded",
    "shared_fp8_bytes_reused", "total_logical_bytes", "total_loaded_bytes", "total_reused_bytes")
_MOE_PHASES = ("h2d_ms", "gate_up_qgemv_ms", "activation_ms", "down_qgemv_ms", "accum_ms", "unaccounted_ms",
               "total_ms")


def moe_telemetry(tel: dict) -> dict:
    """MoeTelemetry (moe.rs:236-276) in field order, from an executor telemetry dict."""
    out = {}
    for f in _MOE_TEL_FIELDS:
        v = tel.get(f, 0)
        out[f] = dict(v) if f == "bytes_by_tensor_kind" else v
    return out


def _hit_rate(t: dict) -> float:
    ops = t["resident_cache_hit_count"] + t["resident_cache_miss_count"]
    return t["resident_cache_hit_count"] / ops if ops else 0.0


def moe_stats_report(source: str, backend: str, fmt: str, hidden: int, intermediate: int, out: int,
                     telemetries, numerics: dict | None) -> dict:
    """MoeStatsReport (bench_selected_moe.rs:79-101) over executor calls: the byte and
    cache fields from the first call, as run_benchmark_for_shape keeps its first
    iteration's telemetry (bench_selected_moe.rs:381-393), the phase statistics over
    all calls, cache_hit_rate = hits / (hits + misses) of the cache counters
    (bench_selected_moe.rs:525-530)."""
    if fmt not in FORMAT_NAMES:
        raise ValueError(f"unknown format {fmt}")
    tels = list(telemetries)
    if not tels:
        raise ValueError("no telemetry")
    t0 = moe_telemetry(tels[0])
    logical = t0["logical_expert_bytes_requested"]
    rep = {"source": source, "backend": backend, "format": fmt, "hidden": int(hidden),
           "intermediate": int(intermediate), "out": int(out), "selected_experts": t0["selected_expert_count"],
           "logical_expert_bytes_requested": logical,
           "actual_expert_bytes_loaded": t0["actual_expert_bytes_loaded"],
           "resident_cache_bytes_reused": t0["resident_cache_bytes_reused"],
           "dequantized_scratch_bytes": t0["dequantized_scratch_bytes"],
           "resident_cache_capacity_bytes": t0["resident_cache_capacity_bytes"],
           "resident_cache_resident_bytes": t0["resident_cache_resident_bytes"],
           "resident_cache_hit_count": t0["resident_cache_hit_count"],
           "resident_cache_miss_count": t0["resident_cache_miss_count"],
           "resident_cache_eviction_count": t0["resident_cache_eviction_count"],
           "cache_insert_attempt_count": t0["resident_cache_insert_attempt_count"],
           "cache_insert_accept_count": t0["resident_cache_insert_accept_count"],
           "cache_insert_bypass_count": t0["resident_cache_insert_bypass_count"],
           "oversized_tensor_bypass_count": t0["resident_cache_oversized_tensor_bypass_count"],
           "oversized_expert_bypass_count": t0["resident_cache_oversized_expert_bypass_count"],
           "self_eviction_risk_count": t0["resident_cache_self_eviction_risk_count"],
           "bytes_by_tensor_kind": t0["bytes_by_tensor_kind"], "bytes_per_expert": t0["bytes_per_expert"],
           "selected_working_set_bytes": t0["selected_working_set_bytes"],
           "cache_hit_rate": _hit_rate(t0),
           "telemetry": {p: stats([t[p] for t in tels]) for p in _MOE_PHASES},
           "numerics": numerics if numerics is not None else numerics_suite(None, None)}
    return rep
