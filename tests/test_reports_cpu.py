"""The benchmark reports follow the reference's report structs field for field and
in declaration order (tests/golden/report_schema.json, extracted from
bench_qgemv.rs, bench_selected_moe.rs, quant.rs and moe.rs by
tests/golden/make_report_schema.py), and their statistics follow compute_stats."""
import json
import os

from objeta_amd import reports

SCHEMA = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "report_schema.json")))


def _tel(i):
    t = {f: i for f in reports._MOE_TEL_FIELDS}
    t["bytes_by_tensor_kind"] = {"gate": 1, "up": 2, "down": 3}
    for p in reports._MOE_PHASES:
        t[p] = float(i)
    t["resident_cache_hit_count"], t["resident_cache_miss_count"] = 3, 1
    return t


def test_qgemv_stats_report_schema():
    r = reports.qgemv_stats_report("hip", "q4_gemv", "Q4_0", 1024, 4096, [0.003, 0.001, 0.002], 2375680,
                                   reports.numerics_suite({"cosine_similarity": 1.0, "relative_l2_error": 0.0,
                                                           "max_abs_error": 0.0}, None))
    assert list(r) == SCHEMA["QGemvStatsReport"]
    assert list(r["telemetry"]) == SCHEMA["QGemvStatsTelemetry"]
    for k in ("h2d_ms", "kernel_ms", "d2h_ms", "unaccounted_ms", "total_ms"):
        assert list(r["telemetry"][k]) == SCHEMA["QGemvStats"]
    assert list(r["numerics"]) == SCHEMA["QGemvNumericsSuite"]
    assert list(r["numerics"]["cuda_vs_cpu_quant"]) == SCHEMA["QGemvNumerics"]
    assert r["block_bytes"] == 18 and r["format"] == "Q4_0"
    # effective_gbps = bytes_read / avg kernel seconds (bench_qgemv.rs:164-170)
    assert abs(r["telemetry"]["effective_gbps"] - 2375680 / 0.002e-3 / 1e9) < 1e-6


def test_moe_stats_report_schema():
    r = reports.moe_stats_report("synthetic", "hip", "Q4_0", 2048, 768, 2048, [_tel(1), _tel(2), _tel(3)], None)
    assert list(r) == SCHEMA["MoeStatsReport"]
    assert list(r["telemetry"]) == SCHEMA["MoeStatsTelemetry"]
    assert list(r["telemetry"]["total_ms"]) == SCHEMA["MoeStats"]
    assert list(r["bytes_by_tensor_kind"]) == SCHEMA["BytesByTensorKind"]
    assert r["cache_hit_rate"] == 0.75
    assert list(reports.moe_telemetry(_tel(1))) == SCHEMA["MoeTelemetry"]


def test_stats_percentile_rule():
    """compute_stats: sorted values, index round(p * (n - 1)) (bench_qgemv.rs:59-100)."""
    s = reports.stats([5.0, 1.0, 4.0, 2.0, 3.0, 10.0, 7.0, 8.0, 6.0, 9.0])
    assert s == {"avg": 5.5, "min": 1.0, "max": 10.0, "p50": 6.0, "p95": 10.0}
    # 0.5 * 1 = 0.5 rounds half away from zero (Rust's f32::round) to index 1, where
    # Python's round() would give 0
    assert reports.stats([1.0, 2.0])["p50"] == 2.0
    # 0.95f32 * 10 rounds to exactly 9.5 in f32, then away from zero to 10
    assert [reports.percentile_index(0.95, n) for n in (1, 2, 10, 11, 21)] == [0, 1, 9, 10, 19]
