"""Shared-expert residency and cross-layer prefetch on the GPU.

* objeta_hip_cache_preload_shared: the pinned shared-expert preload of
  deepseek_single_layer_moe.rs:1698-1730, and the official executor resolving the
  shared expert from those entries (the sketch in crates/objeta-cuda/src/moe_tmp.txt).
* objeta_hip_cache_prefetch: copies started ahead of the call that uses them; the
  executor and cache_get must order themselves after copies still in flight, so the
  tests start a prefetch and use its entries at once, then compare with the oracle
  and with runs that copy nothing ahead."""
import ctypes as C

import numpy as np
import pytest

from objeta_amd import (ExpertCache, ExpertCacheKey, ExpertTensorKind, HostExpertSet, MoeExecutor,
                        PinnedHostBuffer, QuantFormat, check)
from objeta_amd.workloads import fp4_random_expert, fp8_random_expert
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

F32 = np.float32


def q4_random(rows: int, cols: int, rng) -> np.ndarray:
    """Random Q4_0 bytes: f16 block scales in [2^-9, 2^-6), uniform nibbles."""
    nb = rows * cols // 32
    b = rng.integers(0, 256, (nb, 18), dtype=np.uint8)
    scale = rng.uniform(2.0 ** -9, 2.0 ** -6, nb).astype(np.float16).view(np.uint8).reshape(nb, 2)
    b[:, :2] = scale
    return b.ravel()


def pinned_experts(backend, n, hidden, inter, out_dim, seed):
    """n Q4_0 experts whose bytes live in one pinned host buffer (copies from it run
    asynchronously)."""
    rng = np.random.default_rng(seed)
    gu = inter * (hidden // 32) * 18
    dn = out_dim * (inter // 32) * 18
    pin = PinnedHostBuffer(backend, n * (2 * gu + dn))
    host = pin.array(np.uint8)
    experts = []
    for e in range(n):
        base = e * (2 * gu + dn)
        host[base:base + gu] = q4_random(inter, hidden, rng)
        host[base + gu:base + 2 * gu] = q4_random(inter, hidden, rng)
        host[base + 2 * gu:base + 2 * gu + dn] = q4_random(out_dim, inter, rng)
        experts.append((host[base:base + gu], host[base + gu:base + 2 * gu], host[base + 2 * gu:base + 2 * gu + dn]))
    return pin, experts


def q4_keys(layer, e):
    return [ExpertCacheKey(layer, e, k, QuantFormat.Q4_0)
            for k in (ExpertTensorKind.Gate, ExpertTensorKind.Up, ExpertTensorKind.Down)]


def assert_close(out, ref):
    c = orc.compare(ref, out)
    assert c["cosine_similarity"] >= 0.9999 and c["relative_l2_error"] <= 1e-4, c
    scale = max(float(np.max(np.abs(ref))), 1e-30)
    assert float(np.max(np.abs(out.astype(np.float64) - ref))) <= 1e-4 * scale


def test_prefetch_then_execute_uses_entries_in_flight(backend):
    hidden, inter, out_dim, n = 2048, 768, 2048, 12
    pin, experts = pinned_experts(backend, n, hidden, inter, out_dim, 7)
    moe = MoeExecutor(backend)
    hx = HostExpertSet(experts)
    x = orc.gauss(hidden, 3, 1.0)
    sel = [(3, 0.3), (9, 0.25), (0, 0.2), (11, 0.1), (5, 0.08), (2, 0.04), (7, 0.02), (4, 0.01)]
    ref = orc.selected_moe(orc.Q4_0, experts, sel, x, hidden, inter, out_dim)
    for rep in range(3):  # the copies race the call differently on each repetition
        cache = ExpertCache(64 * sum(a.nbytes for a in experts[0]), backend)
        started = cache.prefetch([(k, a) for e, _ in sel for k, a in zip(q4_keys(0, e), experts[e])])
        assert started == 3 * len(sel)
        st0 = cache.stats()
        assert st0["hit_count"] == 0 and st0["miss_count"] == 0 and st0["cache_insert_accept_count"] == 3 * len(sel)
        out, tel = moe.execute_selected_moe_cuda(None, None, hx, sel, x, hidden, inter, out_dim, 0, cache)
        assert tel["actual_expert_bytes_loaded"] == 0
        assert tel["resident_cache_bytes_reused"] == tel["logical_expert_bytes_requested"]
        assert cache.stats()["hit_count"] == 3 * len(sel)
        assert_close(out, ref)
        # a second prefetch of resident keys starts nothing
        assert cache.prefetch([(k, a) for k, a in zip(q4_keys(0, 3), experts[3])]) == 0
        cache.close()
    out_nc, _ = moe.execute_selected_moe_cuda(None, None, hx, sel, x, hidden, inter, out_dim, 0, None)
    assert_close(out_nc, ref)
    pin.free()


def test_prefetch_then_cache_get_waits_for_the_copy(backend):
    nbytes = 64 << 20
    pin = PinnedHostBuffer(backend, nbytes)
    host = pin.array(np.uint8)
    host[:] = np.random.default_rng(5).integers(0, 256, nbytes, dtype=np.uint8)
    cache = ExpertCache(2 * nbytes, backend)
    key = ExpertCacheKey(3, 1, ExpertTensorKind.DownWeight, QuantFormat.DeepSeekFp4E2M1)
    assert cache.prefetch([(key, host)]) == 1
    ptr = cache.get(key)  # waits on the host for the copy in flight
    assert ptr
    out = np.empty(nbytes, np.uint8)
    check(backend.L.objeta_hip_copy_d2h(backend.ctx, None, out.ctypes.data_as(C.c_void_p), C.c_void_p(ptr), nbytes))
    backend.synchronize()
    assert np.array_equal(out, host)
    cache.close()
    pin.free()


def test_prefetch_with_evictions_keeps_outputs_right(backend):
    """Capacity for three experts: prefetching the next call's experts evicts entries the
    current call has just used; fences keep the recycled blocks from being overwritten
    while a launch may still read them."""
    hidden, inter, out_dim, n = 1024, 512, 1024, 10
    pin, experts = pinned_experts(backend, n, hidden, inter, out_dim, 21)
    one = sum(a.nbytes for a in experts[0])
    cache = ExpertCache(3 * one, backend)
    moe = MoeExecutor(backend)
    hx = HostExpertSet(experts)
    rng = np.random.default_rng(8)
    h = orc.gauss(hidden, 9, 1.0)
    for layer in range(6):
        sel = [(int(e), float(w)) for e, w in zip(rng.choice(n, 2, replace=False), (0.6, 0.4))]
        nxt = [int(e) for e in rng.choice(n, 2, replace=False)]
        out, _ = moe.execute_selected_moe_cuda(None, None, hx, sel, h, hidden, inter, out_dim, 0, cache)
        cache.prefetch([(k, a) for e in nxt for k, a in zip(q4_keys(0, e), experts[e])])
        ref = orc.selected_moe(orc.Q4_0, experts, sel, h, hidden, inter, out_dim)
        assert_close(out, ref)
        h = (h + F32(0.1) * out / max(1.0, float(np.max(np.abs(out))))).astype(F32)
    assert cache.stats()["eviction_count"] > 0
    cache.close()
    pin.free()


def ptr_order(t):
    return (t[0], t[2], t[4], t[1], t[3], t[5])


def test_preload_shared_and_official_executor_from_cache(backend):
    hidden, inter, out_dim, n_layers = 512, 256, 512, 3
    experts = [fp4_random_expert(hidden, inter, out_dim, 300 + e) for e in range(4)]
    shared = [fp8_random_expert(hidden, inter, out_dim, 77 + l) for l in range(n_layers)]
    cache = ExpertCache(1 << 30, backend)
    nbytes, ms = cache.preload_shared(shared)
    sizes = sum(a.nbytes for a in shared[0])
    assert nbytes == n_layers * sizes and cache.stats()["pinned_bytes"] == nbytes
    moe = MoeExecutor(backend)
    x = orc.gauss(hidden, 12, 1.0)
    sel = [(1, 0.5), (3, 0.5)]
    for layer in range(n_layers):
        sh_dev = [backend.to_device(a) for a in shared[layer]]
        want, tw = moe.execute_selected_moe_official_routed_fp4(None, None, experts, sel, x, hidden, inter, out_dim,
                                                                layer, None, ptr_order(sh_dev), 10.0)
        h0 = cache.stats()["hit_count"]
        got, tg = moe.execute_selected_moe_official_routed_fp4(None, None, experts, sel, x, hidden, inter, out_dim,
                                                               layer, cache, None, 10.0, shared_from_cache=True)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
        assert cache.stats()["hit_count"] - h0 == 6  # the six shared tensors (routed: first call, all misses)
        assert tg["shared_fp8_bytes_reused"] == sizes and tg["shared_fp8_bytes_loaded"] == 0
        assert tg["total_reused_bytes"] == tg["routed_fp4_bytes_reused"] + sizes
        assert tw["shared_fp8_bytes_loaded"] > 0 and tw["shared_fp8_bytes_reused"] == 0
    # a layer without preloaded entries falls back to the argument (one miss counted)
    sh_dev = [backend.to_device(a) for a in shared[0]]
    m0 = cache.stats()["miss_count"]
    got, tg = moe.execute_selected_moe_official_routed_fp4(None, None, experts, sel, x, hidden, inter, out_dim, 9,
                                                           cache, ptr_order(sh_dev), 10.0, shared_from_cache=True)
    want, _ = moe.execute_selected_moe_official_routed_fp4(None, None, experts, sel, x, hidden, inter, out_dim, 0,
                                                           None, ptr_order(sh_dev), 10.0)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert cache.stats()["miss_count"] - m0 == 12 + 1  # two routed experts' six tensors, then one shared key
    assert tg["shared_fp8_bytes_reused"] == 0 and tg["shared_fp8_bytes_loaded"] > 0
    cache.close()


def test_official_executor_rejects_cached_shared_expert_of_another_shape(backend):
    """Shared entries preloaded for intermediate 256 and an executor call at 384: the
    cached blocks are shorter than the kernels would read, so the call fails with
    InvalidInput before any launch, and a call at the preloaded shape still works."""
    from objeta_amd import HipError

    hidden, inter, out_dim = 512, 256, 512
    cache = ExpertCache(1 << 30, backend)
    cache.preload_shared([fp8_random_expert(hidden, inter, out_dim, 91)])
    moe = MoeExecutor(backend)
    x = orc.gauss(hidden, 13, 1.0)
    wide = [fp4_random_expert(hidden, 384, out_dim, 400 + e) for e in range(2)]
    with pytest.raises(HipError) as e:
        moe.execute_selected_moe_official_routed_fp4(None, None, wide, [(0, 0.5), (1, 0.5)], x, hidden, 384, out_dim,
                                                     0, cache, None, 10.0, shared_from_cache=True)
    assert e.value.status == 5 and "shared gate weight holds 131072 bytes, expected 196608" in str(e.value)
    narrow = [fp4_random_expert(hidden, inter, out_dim, 500 + e) for e in range(2)]
    got, _ = moe.execute_selected_moe_official_routed_fp4(None, None, narrow, [(0, 0.5), (1, 0.5)], x, hidden, inter,
                                                          out_dim, 0, cache, None, 10.0, shared_from_cache=True)
    assert np.isfinite(got).all()
    assert moe.device_error() == 0
    cache.close()
