"""objeta_hip_moe_stack_cached: a decode stack with the experts behind the expert
cache (the loop the reference's drivers run over execute_selected_moe_cuda,
crates/objeta-cuda/src/moe.rs:352-751, with the hidden state on the device).

Each layer of each call is checked against the oracle on the device's own input to
that layer (the trace of hidden states): router ids bit-exact (cpu_router followed
by renormalisation), outputs within 1e-4 of the oracle's selected_moe_cpu. The
cache must not change a single bit of the result (no cache, a cache at 25% of the
expert bytes with evictions, and the same with next-layer prefetch), and the byte
accounting keeps logical == loaded + reused (moe.rs:743-748)."""
import numpy as np
import pytest

from objeta_amd import ExpertCache, HipError, MoeExecutor, PinnedHostBuffer
from objeta_amd.workloads import zipf_bias
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

Q4 = 0
F32 = np.float32


@pytest.fixture(scope="module")
def stack(backend):
    """4 layers of 16 Q4_0 experts (hidden 512, intermediate 256) in one pinned host
    buffer, Zipf-biased routers on the device."""
    L, E, H, I = 4, 16, 512, 256
    gu, dn = I * (H // 32) * 18, H * (I // 32) * 18
    eb = 2 * gu + dn
    pin = PinnedHostBuffer(backend, L * E * eb)
    host = pin.array(np.uint8)
    layers_host = []
    for l in range(L):
        ex = []
        for e in range(E):
            base = (l * E + e) * eb
            for j, (r, c, off, n) in enumerate(((I, H, 0, gu), (I, H, gu, gu), (H, I, 2 * gu, dn))):
                host[base + off:base + off + n] = orc.quantize_matrix(
                    Q4, orc.gauss(r * c, 900 + 3 * (l * E + e) + j, 0.02), r, c)
            ex.append((host[base:base + gu], host[base + gu:base + 2 * gu], host[base + 2 * gu:base + eb]))
        layers_host.append(ex)
    wrs = [orc.gauss(E * H, 950 + l, 0.02) for l in range(L)]
    biases = [zipf_bias(E, 1.1, 960 + l) for l in range(L)]
    d_wr = [backend.to_device(w) for w in wrs]
    d_b = [backend.to_device(b) for b in biases]
    yield dict(L=L, E=E, H=H, I=I, eb=eb, host=layers_host, wrs=wrs, biases=biases,
               layers=[(layers_host[l], d_wr[l], d_b[l], l) for l in range(L)])
    pin.free()


def run(backend, st, T, k, cache=None, prefetch=False, seed=970, stream=None):
    H = st["H"]
    x = orc.gauss(T * H, seed + T, 1.0)
    d_h = backend.to_device(x)
    d_trace = backend.alloc(4 * st["L"] * T * H)
    moe = MoeExecutor(backend)
    ids, ws, tel = moe.stack_cached(Q4, st["layers"], k, T, d_h, H, st["I"], cache=cache, prefetch_next=prefetch,
                                    d_trace=d_trace, stream=stream)
    backend.synchronize(stream)
    trace = d_trace.download(F32, st["L"] * T * H).reshape(st["L"], T, H)
    assert np.array_equal(d_h.download(F32, T * H).reshape(T, H), trace[-1])
    assert moe.device_error() == 0
    return x.reshape(T, H), ids, ws, trace, tel


def check_against_oracle(st, x, ids, ws, trace, k, tokens=None):
    L, E, H, I = st["L"], st["E"], st["H"], st["I"]
    T = x.shape[0]
    for l in range(L):
        hin = x if l == 0 else trace[l - 1]
        for t in (range(T) if tokens is None else tokens):
            rid, rw, _, _ = orc.router(st["wrs"][l], hin[t], E, H, k, bias=st["biases"][l], renormalize=True)
            assert np.array_equal(ids[l, t], rid), (l, t)
            np.testing.assert_allclose(ws[l, t], rw, rtol=1e-4, atol=1e-7)
            ref = orc.selected_moe(Q4, st["host"][l], [(int(i), float(v)) for i, v in zip(rid, rw)], hin[t], H, I, H)
            got = trace[l, t].astype(np.float64) - hin[t]
            scale = max(float(np.max(np.abs(ref))), 1e-30)
            assert float(np.max(np.abs(got - ref))) <= 1e-4 * scale, (l, t)


def check_accounting(st, tel, T, k):
    assert tel["layers"] == st["L"] and tel["tokens"] == T
    assert tel["logical_expert_bytes_requested"] == (tel["actual_expert_bytes_loaded"]
                                                     + tel["resident_cache_bytes_reused"])
    assert tel["logical_expert_bytes_requested"] == tel["distinct_experts"] * st["eb"]
    assert st["L"] <= tel["distinct_experts"] <= st["L"] * min(st["E"], T * k)
    assert tel["total_ms"] > 0 and tel["host_wait_ms"] >= 0


@pytest.mark.parametrize("T", [1, 5, 20])
def test_stack_cached_matches_oracle_layer_by_layer(backend, stack, T):
    """T = 20 runs the grouped-token products, 1 and 5 the per-assignment kernels."""
    k = 4
    cache = ExpertCache(stack["L"] * stack["E"] * stack["eb"] // 4, backend)
    x, ids, ws, trace, tel = run(backend, stack, T, k, cache=cache)
    check_accounting(stack, tel, T, k)
    check_against_oracle(stack, x, ids, ws, trace, k, tokens=None if T <= 5 else [0, 7, 19])
    cache.close()


def test_stack_cached_result_independent_of_cache(backend, stack):
    """No cache, a quarter-size cache (evictions), a cache of every expert twice (all
    misses, then all hits) and the quarter-size cache with prefetch: bit-identical
    hidden states, the same ids, consistent counters."""
    T, k = 3, 4
    L, E, eb = stack["L"], stack["E"], stack["eb"]
    _, ids0, _, tr0, tel0 = run(backend, stack, T, k, cache=None)
    assert tel0["resident_cache_bytes_reused"] == 0
    assert tel0["actual_expert_bytes_loaded"] == tel0["logical_expert_bytes_requested"]
    cache = ExpertCache(L * E * eb // 4, backend)
    _, ids1, _, tr1, tel1 = run(backend, stack, T, k, cache=cache)
    st = cache.stats()
    assert st["eviction_count"] > 0 and st["resident_bytes"] <= L * E * eb // 4
    cache.close()
    # a cache holding every expert: the second pass hits on every tensor
    cache = ExpertCache(L * E * eb, backend)
    _, ids_a, _, tr_a, tel_a = run(backend, stack, T, k, cache=cache)
    _, ids2, _, tr2, tel2 = run(backend, stack, T, k, cache=cache)
    assert tel_a["actual_expert_bytes_loaded"] == tel_a["logical_expert_bytes_requested"]
    assert tel2["actual_expert_bytes_loaded"] == 0
    assert tel2["resident_cache_bytes_reused"] == tel2["logical_expert_bytes_requested"]
    assert cache.stats()["eviction_count"] == 0
    cache.close()
    cache = ExpertCache(L * E * eb // 4, backend)
    _, ids3, _, tr3, tel3 = run(backend, stack, T, k, cache=cache, prefetch=True)
    assert tel3["prefetch_experts_predicted"] == (L - 1) * T * k
    assert 0 <= tel3["prefetch_experts_correct"] <= tel3["prefetch_experts_predicted"]
    assert tel3["prefetch_tensors_issued"] > 0 and tel3["prefetch_bytes_issued"] > 0
    cache.close()
    for ids, tr, tel in ((ids1, tr1, tel1), (ids_a, tr_a, tel_a), (ids2, tr2, tel2), (ids3, tr3, tel3)):
        assert np.array_equal(ids, ids0)
        assert np.array_equal(tr.view(np.uint32), tr0.view(np.uint32))
        check_accounting(stack, tel, T, k)


def test_stack_cached_rejects_a_wrong_expert_before_any_launch(backend, stack):
    layers = list(stack["layers"])
    bad = list(stack["host"][2])
    g, u, d = bad[5]
    bad[5] = (g, u[:-18], d)
    layers[2] = (bad, *layers[2][1:])
    d_h = backend.to_device(orc.gauss(stack["H"], 5, 1.0))
    before = d_h.download(F32, stack["H"])
    moe = MoeExecutor(backend)
    with pytest.raises(HipError) as e:
        moe.stack_cached(Q4, layers, 4, 1, d_h, stack["H"], stack["I"])
    assert e.value.status == 5 and "w_up len" in str(e.value)
    assert np.array_equal(d_h.download(F32, stack["H"]), before)  # nothing ran


def test_stack_cached_streams_in_turn_share_the_cache(backend, stack):
    """Calls on the context's two streams in turn through one quarter-size cache: blocks
    that a call on one stream read are evicted and refilled for a call on the other, their
    reuse ordered by the calls' end marks (or fences while those are pending). Every
    hidden state equals the no-cache run's bit for bit, with and without prefetch."""
    T, k = 3, 4
    L, E, eb = stack["L"], stack["E"], stack["eb"]
    _, ids0, _, tr0, _ = run(backend, stack, T, k, cache=None)
    cache = ExpertCache(L * E * eb // 4, backend)
    for rep in range(6):
        _, ids, _, tr, tel = run(backend, stack, T, k, cache=cache, prefetch=rep >= 3, stream=backend.stream(rep % 2))
        assert np.array_equal(ids, ids0), rep
        assert np.array_equal(tr.view(np.uint32), tr0.view(np.uint32)), rep
        check_accounting(stack, tel, T, k)
    assert cache.stats()["eviction_count"] > 0
    cache.close()
