"""Reference-schema reports made from HIP runs.

The two benches the reference's tooling reads run here on the device, as their
run_benchmark_for_shape functions do, and their reports are written as JSON and read
back:
  * bench_qgemv (crates/objeta-cuda/src/bin/bench_qgemv.rs:102-181): QuantBackend::gemv
    host-in/host-out over seeded_f32s inputs, warmup 5 and 10 timed iterations (its
    --matrix defaults), QGemvStatsReport (bench_qgemv.rs:6-37);
  * bench_selected_moe (crates/objeta-cuda/src/bin/bench_selected_moe.rs:243-420): the
    executor over its synthetic experts (seed ^ e ^ 0x1111 / 0x2222 / 0x3333, x from
    seed ^ 0xDEADBEEF, selection (seed + idx) % n with weights 0.4, 0.3, ...) with and
    without a cache, MoeStatsReport (bench_selected_moe.rs:19-101).
Each report's field names and order must equal the reference structs'
(tests/golden/report_schema.json), its numerics must come from this run (cosine of the
device result against the CPU oracle at least 0.9999, the reference benches' bar) and
its byte accounting must follow the reference's formulas."""
import json
import os

import numpy as np
import pytest

from objeta_amd import ExpertCache, MoeExecutor, QGemvShape, QuantFormat, reports
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

SCHEMA = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "report_schema.json")))
KERNEL = {0: "q4_gemv", 1: "q5_gemv", 2: "iq3_gemv"}
NAME = {0: "Q4_0", 1: "Q5_0", 2: "IQ3_0"}
BB = {0: 18, 1: 22, 2: 14}


def _roundtrip(tmp_path, name, rep):
    p = tmp_path / name
    p.write_text(json.dumps(rep) + "\n")
    return json.loads(p.read_text())


@pytest.mark.parametrize("fmt,rows,cols", [(0, 1024, 4096), (1, 4096, 4096), (2, 11008, 4096)])
def test_qgemv_stats_report_from_device_runs(quant, tmp_path, fmt, rows, cols):
    seed = 123  # bench_qgemv's default --seed
    matrix = orc.seeded_f32s(rows * cols, seed ^ 0xABCD_EF01_2345_6789)
    x = orc.seeded_f32s(cols, seed ^ 0x1020_3040_5060_7080)
    q = orc.quantize_matrix(fmt, matrix, rows, cols)
    shape = QGemvShape.new(QuantFormat(fmt), rows, cols)  # QGemvShape::new (quant.rs:108)
    for _ in range(5):
        quant.gemv(fmt, None, q, x, shape)
    tels, first = [], None
    for i in range(10):
        y, tel = quant.gemv(fmt, None, q, x, shape)
        tels.append(tel)
        if i == 0:
            first = y
    num = reports.numerics_suite(orc.compare(orc.gemv(fmt, q, x, rows, cols), first),
                                 orc.compare(orc.dense_gemv(matrix, x, rows, cols), first))
    rep = reports.qgemv_stats_report("hip", KERNEL[fmt], NAME[fmt], rows, cols, [t["kernel_ms"] for t in tels],
                                     tels[0]["bytes_read"], num, h2d_ms=[t["h2d_ms"] for t in tels],
                                     d2h_ms=[t["d2h_ms"] for t in tels],
                                     unaccounted_ms=[t["unaccounted_ms"] for t in tels],
                                     total_ms=[t["total_ms"] for t in tels])
    back = _roundtrip(tmp_path, "qgemv_stats_report.json", rep)
    assert list(back) == SCHEMA["QGemvStatsReport"]
    assert list(back["telemetry"]) == SCHEMA["QGemvStatsTelemetry"]
    for k in ("h2d_ms", "kernel_ms", "d2h_ms", "unaccounted_ms", "total_ms"):
        assert list(back["telemetry"][k]) == SCHEMA["QGemvStats"]
    assert list(back["numerics"]) == SCHEMA["QGemvNumericsSuite"]
    assert list(back["numerics"]["cuda_vs_cpu_quant"]) == SCHEMA["QGemvNumerics"]
    # bytes_read = quantized matrix + x (quant.rs:282, bench_qgemv.rs:164)
    assert back["telemetry"]["bytes_read"] == rows * (cols // 32) * BB[fmt] + 4 * cols
    assert back["block_bytes"] == BB[fmt] and back["format"] == NAME[fmt]
    assert back["numerics"]["cuda_vs_cpu_quant"]["cosine_similarity"] >= 0.9999
    assert back["numerics"]["cosine_similarity"] == back["numerics"]["cuda_vs_cpu_quant"]["cosine_similarity"]
    # quantization error, not the device's: the reference's round-trip bars (quant.rs:1689, 1710, 1826)
    assert back["numerics"]["quant_vs_fp32"]["cosine_similarity"] > {0: 0.995, 1: 0.998, 2: 0.970}[fmt]
    k = back["telemetry"]["kernel_ms"]
    assert 0 < k["min"] <= k["p50"] <= k["p95"] <= k["max"] and k["avg"] > 0
    assert back["telemetry"]["h2d_ms"]["avg"] > 0 and back["telemetry"]["total_ms"]["avg"] >= k["avg"]
    assert back["telemetry"]["effective_gbps"] > 0


def _bench_moe_experts(hidden, inter, out_dim, n, seed):
    """bench_selected_moe's synthetic experts (bench_selected_moe.rs:258-276)."""
    q, f = [], []
    for e in range(n):
        g = orc.seeded_f32s(inter * hidden, seed ^ e ^ 0x1111)
        u = orc.seeded_f32s(inter * hidden, seed ^ e ^ 0x2222)
        d = orc.seeded_f32s(out_dim * inter, seed ^ e ^ 0x3333)
        q.append((orc.quantize_matrix(0, g, inter, hidden), orc.quantize_matrix(0, u, inter, hidden),
                  orc.quantize_matrix(0, d, out_dim, inter)))
        f.append((g, u, d))
    return q, f


@pytest.mark.parametrize("cache_bytes", [0, 64 << 20])
def test_moe_stats_report_from_executor_runs(backend, tmp_path, cache_bytes):
    """bench_selected_moe's defaults (hidden 256, intermediate 512, out 256, 2 experts,
    seed 123) and its --matrix iteration counts (warmup 5, 10 timed), with and without a
    device cache (counters reset after warmup, so every timed call hits)."""
    hidden, inter, out_dim, n_sel, seed = 256, 512, 256, 2, 123
    n = max(n_sel, 8)
    experts, experts32 = _bench_moe_experts(hidden, inter, out_dim, n, seed)
    x = orc.seeded_f32s(hidden, seed ^ 0xDEADBEEF)
    wts = [0.4, 0.3, 0.2, 0.1]
    sel = [((seed + i) % n, wts[i % 4]) for i in range(n_sel)]
    moe = MoeExecutor(backend)
    cache = ExpertCache(cache_bytes, backend) if cache_bytes else None
    for _ in range(5):
        moe.execute_selected_moe_cuda(None, None, experts, sel, x, hidden, inter, out_dim, 0, cache)
    if cache is not None:
        cache.reset_counters()
    tels, first = [], None
    for i in range(10):
        y, tel = moe.execute_selected_moe_cuda(None, None, experts, sel, x, hidden, inter, out_dim, 0, cache)
        tels.append(tel)
        if i == 0:
            first = y
    ref = orc.selected_moe(0, experts, sel, x, hidden, inter, out_dim)
    ref32 = orc.selected_moe(-1, experts32, sel, x, hidden, inter, out_dim)
    num = reports.numerics_suite(orc.compare(ref, first), orc.compare(ref32, first))
    rep = reports.moe_stats_report("synthetic", "hip", "Q4_0", hidden, inter, out_dim, tels, num)
    back = _roundtrip(tmp_path, "moe_stats_report.json", rep)
    assert list(back) == SCHEMA["MoeStatsReport"]
    assert list(back["telemetry"]) == SCHEMA["MoeStatsTelemetry"]
    for k in back["telemetry"]:
        assert list(back["telemetry"][k]) == SCHEMA["MoeStats"]
    assert list(back["bytes_by_tensor_kind"]) == SCHEMA["BytesByTensorKind"]
    assert list(reports.moe_telemetry(tels[0])) == SCHEMA["MoeTelemetry"]
    assert back["numerics"]["cuda_vs_cpu_quant"]["cosine_similarity"] >= 0.9999
    assert back["numerics"]["quant_vs_fp32"]["cosine_similarity"] > 0.99
    per_expert = 2 * inter * (hidden // 32) * 18 + out_dim * (inter // 32) * 18
    assert back["selected_experts"] == n_sel and back["bytes_per_expert"] == per_expert
    assert back["logical_expert_bytes_requested"] == n_sel * per_expert
    # the byte invariant of moe.rs:743-748
    assert back["logical_expert_bytes_requested"] == (back["actual_expert_bytes_loaded"]
                                                      + back["resident_cache_bytes_reused"])
    if cache is None:
        assert back["actual_expert_bytes_loaded"] == n_sel * per_expert and back["cache_hit_rate"] == 0.0
    else:
        assert back["resident_cache_bytes_reused"] == n_sel * per_expert and back["cache_hit_rate"] == 1.0
        assert back["resident_cache_capacity_bytes"] == cache_bytes
        cache.close()
    assert back["telemetry"]["total_ms"]["avg"] > 0
    assert moe.device_error() == 0
