"""Host-in/host-out executor (execute_selected_moe_cuda / _native_fp4_cuda) with the
VRAM expert cache on the GPU: outputs against the CPU oracle (moe.rs:1283-1324,
1665-1735) and every telemetry byte/counter field against the oracle's cache model
(oracle/cache_model.py, itself pinned to the reference's asserted values in
tests/test_cache_cpu.py)."""
import ctypes as C

import numpy as np
import pytest

from objeta_amd import ExpertCache, ExpertCacheKey, ExpertTensorKind, HipError, MoeExecutor, QuantFormat
from oracle import cache_model as cm
from oracle import oracle as orc
from tests.test_gpu_moe import assert_moe_close, make_experts, oracle_experts

pytestmark = pytest.mark.gpu

H, I, OUT = 256, 512, 256
FIELDS = ("selected_expert_count", "logical_expert_bytes_requested", "actual_expert_bytes_loaded",
          "resident_cache_bytes_reused", "weight_bytes_loaded", "weight_bytes_reused", "scale_bytes_loaded",
          "scale_bytes_reused")


def host_experts(fmt, experts):
    if fmt == 3:
        return [(g[0], g[1], u[0], u[1], d[0], d[1]) for g, u, d in experts]
    return [(g[0], u[0], d[0]) for g, u, d in experts]


def check_telemetry(tel, model_tel, model_cache, fmt):
    for f in FIELDS:
        assert tel[f] == model_tel[f], f
    assert tel["bytes_by_tensor_kind"] == {"gate": model_tel["bytes_by_tensor_kind_gate"],
                                           "up": model_tel["bytes_by_tensor_kind_up"],
                                           "down": model_tel["bytes_by_tensor_kind_down"]}
    assert tel["logical_expert_bytes_requested"] == (tel["actual_expert_bytes_loaded"]
                                                     + tel["resident_cache_bytes_reused"])
    if model_cache is not None:
        for f, v in model_cache.counters().items():
            if f == "pinned_bytes":
                continue
            name = {"capacity_bytes": "resident_cache_capacity_bytes",
                    "resident_bytes": "resident_cache_resident_bytes",
                    "hit_count": "resident_cache_hit_count", "miss_count": "resident_cache_miss_count",
                    "eviction_count": "resident_cache_eviction_count",
                    "cache_insert_attempt_count": "resident_cache_insert_attempt_count",
                    "cache_insert_accept_count": "resident_cache_insert_accept_count",
                    "cache_insert_bypass_count": "resident_cache_insert_bypass_count",
                    "oversized_tensor_bypass_count": "resident_cache_oversized_tensor_bypass_count",
                    "oversized_expert_bypass_count": "resident_cache_oversized_expert_bypass_count",
                    "self_eviction_risk_count": "resident_cache_self_eviction_risk_count"}[f]
            assert tel[name] == v, f
    assert tel["dequantized_scratch_bytes"] == 0 and tel["total_ms"] > 0.0


@pytest.fixture(scope="module")
def q4_experts():
    return make_experts(0, 4, H, I, OUT, 42)


@pytest.fixture(scope="module")
def fp4_experts():
    return make_experts(3, 4, H, I, OUT, 42)


def _lens(fmt, experts):
    return [tuple(int(np.asarray(a).size) for a in he) for he in host_experts(fmt, experts)]


def run_sequence(backend, fmt, experts, seq, capacity, bypass=False):
    """Runs the executor over `seq` (list of selections) with one cache, checking each
    call's output and telemetry."""
    moe = MoeExecutor(backend)
    cache = ExpertCache(capacity, backend) if capacity is not None else None
    model = cm.CacheModel(capacity) if capacity is not None else None
    if cache is not None:
        cache.bypass_oversized_experts = bypass
        model.bypass_oversized_experts = bypass
    x = orc.seeded_f32s(H, 42 ^ 0xDEADBEEF)
    hx = host_experts(fmt, experts)
    for sel in seq:
        if fmt == 3:
            out, tel = moe.execute_selected_moe_native_fp4_cuda(None, None, hx, sel, x, H, I, OUT, 0, cache)
        else:
            out, tel = moe.execute_selected_moe_cuda(None, None, hx, sel, x, H, I, OUT, 0, cache,
                                                     fmt=QuantFormat(fmt))
        mt = cm.execute_accounting(model, fmt, _lens(fmt, experts), sel, 0)
        check_telemetry(tel, mt, model, fmt)
        ref = orc.selected_moe(fmt, oracle_experts(fmt, experts), sel, x, H, I, OUT)
        assert_moe_close(out, ref)
    if cache is not None:
        cache.close()


def test_executor_cache_disabled(backend, q4_experts):
    run_sequence(backend, 0, q4_experts, [[(0, .5), (1, .5)]], None)


def test_executor_warm_then_hits(backend, q4_experts):
    run_sequence(backend, 0, q4_experts, [[(0, .5), (1, .5)], [(0, .5), (1, .5)]], 1000 * 1024)


def test_executor_eviction_and_lru_touch(backend, q4_experts):
    eb = sum(_lens(0, q4_experts)[0])
    run_sequence(backend, 0, q4_experts, [[(0, .5), (1, .5), (2, .5), (3, .5)]], 4 * eb)
    run_sequence(backend, 0, q4_experts, [[(0, 1.0)], [(1, 1.0)], [(0, 1.0)]], eb)
    run_sequence(backend, 0, q4_experts, [[(0, 1.0)], [(1, 1.0)], [(0, 1.0)], [(2, 1.0)], [(0, 1.0)], [(1, 1.0)]],
                 2 * eb)


def test_executor_oversized_tensor_and_expert(backend, q4_experts):
    lens = _lens(0, q4_experts)[0]
    run_sequence(backend, 0, q4_experts[:1], [[(0, 1.0)]], lens[0] - 1)
    run_sequence(backend, 0, q4_experts[:1], [[(0, 1.0)], [(0, 1.0)]], sum(lens) - 100, bypass=True)
    run_sequence(backend, 0, q4_experts[:1], [[(0, 1.0)], [(0, 1.0)]], sum(lens) - 100, bypass=False)


def test_executor_fp4_cache_sequence(backend, fp4_experts):
    eb = sum(_lens(3, fp4_experts)[0])
    assert eb == 208896
    run_sequence(backend, 3, fp4_experts, [[(0, 1.0)], [(0, 1.0)], [(1, 1.0)], [(2, 1.0)], [(0, 1.0)],
                                           [(0, .4), (2, .6)]], 2 * eb)


def test_executor_random_mixed_hits_and_misses(backend):
    """Repeated experts in one selection, hits mixed with misses, evictions inside a
    call (self-eviction risk) on Q5_0."""
    experts = make_experts(1, 6, H, I, OUT, 5)
    eb = sum(_lens(1, experts)[0])
    rng = np.random.default_rng(3)
    seq = [[(int(rng.integers(6)), float(rng.random())) for _ in range(int(rng.integers(1, 5)))] for _ in range(8)]
    run_sequence(backend, 1, experts, seq, int(2.5 * eb))


def test_executor_validation_messages(backend, q4_experts):
    moe = MoeExecutor(backend)
    hx = host_experts(0, q4_experts)
    x = orc.seeded_f32s(H, 1)
    with pytest.raises(HipError) as e:
        moe.execute_selected_moe_cuda(None, None, hx, [(9, 1.0)], x, H, I, OUT, 0)
    assert e.value.kind == "InvalidInput" and "expert index 9 out of bounds (len=4)" in e.value.source_message
    with pytest.raises(HipError) as e:
        moe.execute_selected_moe_cuda(None, None, hx, [(0, 1.0)], x[:-1], H, I, OUT, 0)
    assert "x len 255 != hidden 256" in e.value.source_message
    bad = [(hx[0][0][:-1], hx[0][1], hx[0][2])]
    with pytest.raises(HipError) as e:
        moe.execute_selected_moe_cuda(None, None, bad, [(0, 1.0)], x, H, I, OUT, 0)
    assert e.value.action == "validate expert w_gate size" and "w_gate len" in e.value.source_message


def test_cache_device_copies_and_pinned(backend):
    """insert / get_or_insert / insert_pinned put the host bytes in device memory."""
    cache = ExpertCache(1 << 20, backend)
    data = np.arange(5000, dtype=np.uint32).view(np.uint8)
    k = ExpertCacheKey(3, 7, ExpertTensorKind.Gate, QuantFormat.Q4_0)
    p, hit, cached = cache.get_or_insert(k, data)
    assert not hit and cached
    backend.synchronize()
    out = np.empty_like(data)
    backend.L.objeta_hip_copy_d2h(backend.ctx, None, out.ctypes.data_as(C.c_void_p), C.c_void_p(p), data.nbytes)
    backend.synchronize()
    assert np.array_equal(out, data)
    p2, hit, _ = cache.get_or_insert(k, data)
    assert hit and p2 == p
    kp = ExpertCacheKey(3, 8, ExpertTensorKind.Up, QuantFormat.Q4_0)
    pp = cache.insert_pinned(kp, data[::-1].copy())
    assert cache.pinned_bytes == data.nbytes
    assert cache.evict_lru() == k  # the pinned entry is skipped
    assert cache.evict_lru() is None
    backend.synchronize()
    backend.L.objeta_hip_copy_d2h(backend.ctx, None, out.ctypes.data_as(C.c_void_p), C.c_void_p(pp), data.nbytes)
    backend.synchronize()
    assert np.array_equal(out, data[::-1])
    big = np.zeros((1 << 20) + 1, np.uint8)
    pt, cached = cache.insert(ExpertCacheKey(0, 0, ExpertTensorKind.Down, QuantFormat.Q4_0), big)
    assert not cached and pt
    cache.release_transient(pt)
    cache.close()


def test_executor_pinned_host_weights_overlap_path(backend):
    """Expert weights in pinned host memory, a cache smaller than the working set:
    every call misses, so the per-expert copy/compute overlap path runs."""
    experts = make_experts(0, 4, H, I, OUT, 9)
    hx = host_experts(0, experts)
    L = backend.L
    pinned, keep = [], []
    for tensors in hx:
        row = []
        for a in tensors:
            a = np.ascontiguousarray(a)
            hp = C.c_void_p()
            assert L.objeta_hip_alloc_pinned_host(backend.ctx, a.nbytes, C.byref(hp)) == 0
            buf = (C.c_uint8 * a.nbytes).from_address(hp.value)
            arr = np.frombuffer(buf, dtype=np.uint8)
            arr[:] = a
            keep.append(hp)
            row.append(arr)
        pinned.append(tuple(row))
    moe = MoeExecutor(backend)
    eb = sum(_lens(0, experts)[0])
    cache = ExpertCache(eb, backend)
    x = orc.seeded_f32s(H, 77)
    for sel in ([(0, .3), (1, .7)], [(2, .5), (3, .25), (0, .25)], [(1, 1.0)]):
        out, tel = moe.execute_selected_moe_cuda(None, None, pinned, sel, x, H, I, OUT, 4, cache)
        ref = orc.selected_moe(0, oracle_experts(0, experts), sel, x, H, I, OUT)
        assert_moe_close(out, ref)
        assert tel["actual_expert_bytes_loaded"] > 0 and tel["h2d_ms"] > 0.0
    cache.close()
    backend.synchronize()
    for hp in keep:
        L.objeta_hip_free_pinned_host(backend.ctx, hp)
