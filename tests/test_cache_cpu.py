"""Expert cache semantics on the CPU.

1. The oracle's cache model (oracle/cache_model.py) against the exact counter values
   the reference's own tests assert (moe.rs:1892-2316, 2422-2559): this pins the
   model.
2. The library's cache (accounting mode: no device memory, same code path for the
   LRU order and counters) against the model over random operation sequences.
"""
import numpy as np
import pytest

from objeta_amd import ExpertCache, ExpertCacheKey, ExpertTensorKind, QuantFormat
from oracle import cache_model as cm

H, I, OUT = 256, 512, 256
Q4_LENS = (I * (H // 32) * 18, I * (H // 32) * 18, OUT * (I // 32) * 18)   # gate, up, down
FP4_LENS = (I * H // 2, I * H // 32, I * H // 2, I * H // 32, OUT * I // 2, OUT * I // 32)
EXPERT = sum(Q4_LENS)


def run(cache, sel, fmt=cm.Q4_0, n=4, layer=0):
    lens = [FP4_LENS if fmt == cm.FP4 else Q4_LENS] * n
    return cm.execute_accounting(cache, fmt, lens, sel, layer)


def test_model_cache_disabled():
    t = run(None, [(0, .5), (1, .5)])
    assert t["resident_cache_bytes_reused"] == 0
    assert t["actual_expert_bytes_loaded"] == t["logical_expert_bytes_requested"]


def test_model_warm_then_hits():
    c = cm.CacheModel(1000 * 1024)
    t1 = run(c, [(0, .5), (1, .5)])
    assert t1["resident_cache_bytes_reused"] == 0 and c.miss_count == 6 and c.hit_count == 0
    assert c.eviction_count == 0
    t2 = run(c, [(0, .5), (1, .5)])
    assert t2["resident_cache_bytes_reused"] == t2["logical_expert_bytes_requested"]
    assert t2["actual_expert_bytes_loaded"] == 0
    assert (c.hit_count, c.miss_count, c.eviction_count) == (6, 6, 0)


def test_model_fits_all_and_single_slot_eviction():
    c = cm.CacheModel(4 * EXPERT)
    run(c, [(0, .5), (1, .5), (2, .5), (3, .5)])
    assert c.eviction_count == 0 and c.resident_bytes == 4 * EXPERT
    c = cm.CacheModel(EXPERT)
    run(c, [(0, 1.0)])
    assert c.eviction_count == 0 and c.resident_bytes == EXPERT
    run(c, [(1, 1.0)])
    assert c.eviction_count > 0 and c.resident_bytes == EXPERT
    t3 = run(c, [(0, 1.0)])
    assert t3["actual_expert_bytes_loaded"] == EXPERT and t3["resident_cache_bytes_reused"] == 0


def test_model_lru_touch_order():
    c = cm.CacheModel(2 * EXPERT)
    for e in (0, 1, 0, 2):
        run(c, [(e, 1.0)])
    assert run(c, [(0, 1.0)])["resident_cache_bytes_reused"] == EXPERT
    t = run(c, [(1, 1.0)])
    assert t["resident_cache_bytes_reused"] == 0 and t["actual_expert_bytes_loaded"] == EXPERT


def test_model_oversized_tensor_bypass():
    c = cm.CacheModel(Q4_LENS[0] - 1)
    t = run(c, [(0, 1.0)], n=1)
    assert (c.cache_insert_attempt_count, c.cache_insert_accept_count, c.cache_insert_bypass_count) == (3, 0, 3)
    assert (c.oversized_tensor_bypass_count, c.oversized_expert_bypass_count) == (3, 0)
    assert c.resident_bytes == 0
    assert t["actual_expert_bytes_loaded"] == t["logical_expert_bytes_requested"]


def test_model_oversized_expert_bypass_and_self_eviction():
    c = cm.CacheModel(EXPERT - 100)
    c.bypass_oversized_experts = True
    t = run(c, [(0, 1.0)], n=1)
    assert (c.cache_insert_attempt_count, c.cache_insert_accept_count, c.cache_insert_bypass_count) == (3, 0, 3)
    assert (c.oversized_tensor_bypass_count, c.oversized_expert_bypass_count, c.self_eviction_risk_count) == (0, 1, 0)
    assert c.resident_bytes == 0 and c.miss_count == 0  # the bypass path never calls get
    assert t["actual_expert_bytes_loaded"] == t["logical_expert_bytes_requested"]
    c = cm.CacheModel(EXPERT - 100)
    run(c, [(0, 1.0)], n=1)
    assert c.self_eviction_risk_count == 1 and c.oversized_expert_bypass_count == 0
    assert c.cache_insert_accept_count > 0


def test_model_fp4_cache_sequence():
    fp4_expert = sum(FP4_LENS)
    assert fp4_expert == 208896  # moe.rs:2465-2469
    c = cm.CacheModel(2 * fp4_expert)
    expect = [(0, 0, fp4_expert, 1), (0, fp4_expert, 0, 1), (1, 0, fp4_expert, 2), (2, 0, fp4_expert, 2),
              (0, 0, fp4_expert, 2)]
    for e, reused, loaded, resident in expect:
        t = run(c, [(e, 1.0)], fmt=cm.FP4)
        assert t["resident_cache_bytes_reused"] == reused and t["actual_expert_bytes_loaded"] == loaded
        assert c.resident_bytes == resident * fp4_expert


# ---------------------------------------------------------------- library vs model
def _key(k):
    return ExpertCacheKey(k[0], k[1], ExpertTensorKind(k[2]), QuantFormat(k[3]))


@pytest.mark.parametrize("seed", range(6))
def test_library_cache_matches_model_on_random_sequences(seed):
    rng = np.random.default_rng(seed)
    cap = int(rng.integers(200, 2000))
    lib = ExpertCache(cap)
    model = cm.CacheModel(cap)
    keys = [(int(rng.integers(0, 2)), int(rng.integers(0, 6)), int(rng.integers(0, 3)), 0) for _ in range(12)]
    sizes = {k: int(rng.integers(1, cap // 2 + 50)) for k in keys}
    for step in range(400):
        op = rng.choice(["get", "insert", "get_or_insert", "pin", "insert_pinned", "touch", "evict", "clear",
                         "reset", "prefetch"], p=[.2, .2, .25, .05, .02, .1, .08, .02, .03, .05])
        k = keys[int(rng.integers(len(keys)))]
        if op == "get":
            assert (lib.get(_key(k)) is not None) == model.get(k)
        elif op == "insert":
            _, cached = lib.insert(_key(k), np.zeros(sizes[k], np.uint8))
            assert cached == model.insert(k, sizes[k])
        elif op == "get_or_insert":
            _, hit, cached = lib.get_or_insert(_key(k), np.zeros(sizes[k], np.uint8))
            mh = model.get(k)
            assert hit == mh
            if not mh:
                assert cached == model.insert(k, sizes[k])
        elif op == "pin":
            lib.pin(_key(k))
            model.pin(k)
        elif op == "insert_pinned":
            lib.insert_pinned(_key(k), np.zeros(sizes[k] // 4 + 1, np.uint8))
            model.insert_pinned(k, sizes[k] // 4 + 1)
        elif op == "touch":
            lib.touch(_key(k))
            model.touch(k)
        elif op == "evict":
            got = lib.evict_lru()
            exp = model.evict_lru()
            assert (None if got is None else (got.layer_id, got.expert_id, int(got.tensor_kind),
                                              int(got.quant_format))) == exp
        elif op == "clear":
            lib.clear()
            model.clear()
        elif op == "prefetch":
            # an insert of absent keys that fit, never a get (no hit or miss counted)
            k2 = keys[int(rng.integers(len(keys)))]
            arrs = [np.zeros(sizes[k], np.uint8), np.zeros(sizes[k2], np.uint8)]
            n = lib.prefetch([(_key(k), arrs[0]), (_key(k2), arrs[1])])
            want = 0
            for kk in dict.fromkeys([k, k2]):
                if kk not in model.sizes and sizes[kk] <= cap:
                    model.insert(kk, sizes[kk])
                    want += 1
            assert n == want
        else:
            lib.reset_counters()
            model.reset_counters()
        st = lib.stats()
        for name, v in model.counters().items():
            assert st[name] == v, (step, op, name)
        assert lib.order() == model.order, (step, op)
    lib.close()


def test_library_cache_insert_stops_when_only_pinned_remain():
    """moe.rs:145-147 would loop forever here; the library admits over capacity."""
    lib = ExpertCache(100)
    a = ExpertCacheKey(0, 0, ExpertTensorKind.Gate, QuantFormat.Q4_0)
    b = ExpertCacheKey(0, 1, ExpertTensorKind.Gate, QuantFormat.Q4_0)
    lib.insert_pinned(a, np.zeros(80, np.uint8))
    _, cached = lib.insert(b, np.zeros(50, np.uint8))
    assert cached and lib.resident_bytes == 130 and lib.eviction_count == 0


def test_library_preload_shared_pins_six_tensors_per_layer():
    """The shared-expert preload (deepseek_single_layer_moe.rs:1698-1730): insert_pinned of
    the six shared tensors per layer under (layer, 0, Shared*, FP4); eviction skips them."""
    lens = (3000, 100, 3000, 100, 2500, 80)
    shared = [tuple(np.zeros(n, np.uint8) for n in lens) for _ in range(3)]
    lib = ExpertCache(50_000)
    nbytes, ms = lib.preload_shared(shared, first_layer=5)
    assert nbytes == 3 * sum(lens) and ms >= 0
    st = lib.stats()
    assert st["pinned_bytes"] == st["resident_bytes"] == nbytes
    kinds = [ExpertTensorKind.SharedGateWeight, ExpertTensorKind.SharedGateScale, ExpertTensorKind.SharedUpWeight,
             ExpertTensorKind.SharedUpScale, ExpertTensorKind.SharedDownWeight, ExpertTensorKind.SharedDownScale]
    assert lib.order() == [(5 + l, 0, int(k), int(QuantFormat.DeepSeekFp4E2M1)) for l in range(3) for k in kinds]
    assert lib.evict_lru() is None
    # a regular insert that needs room evicts around the pinned entries
    big = ExpertCacheKey(9, 1, ExpertTensorKind.GateWeight, QuantFormat.DeepSeekFp4E2M1)
    _, cached = lib.insert(big, np.zeros(50_000 - nbytes + 1, np.uint8))
    assert cached and lib.stats()["pinned_bytes"] == nbytes
    lib.close()
