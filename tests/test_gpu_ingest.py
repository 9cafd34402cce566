"""A DeepSeek-layout checkpoint from disk through the GPU path: experts, shared
expert and router read by the memory-mapped safetensors reader go straight (as
zero-copy host views) into the executors and the cache, and the results match the
oracle on the same bytes."""
import numpy as np
import pytest

from objeta_amd import ExpertCache, MoeExecutor
from objeta_amd.safetensors import ModelWeights
from oracle import oracle as orc
from tests.test_safetensors_cpu import deepseek_checkpoint

pytestmark = pytest.mark.gpu


def assert_close(out, ref):
    c = orc.compare(ref, out)
    assert c["cosine_similarity"] >= 0.9999 and c["relative_l2_error"] <= 1e-4, c
    scale = max(float(np.max(np.abs(ref))), 1e-30)
    assert float(np.max(np.abs(out.astype(np.float64) - ref))) <= 1e-4 * scale


def test_checkpoint_experts_through_the_native_fp4_executor(backend, tmp_path):
    hidden, inter = 512, 256
    p = tmp_path / "ds.safetensors"
    deepseek_checkpoint(p, hidden=hidden, inter=inter, experts=4, layers=(0, 1), mtp=False, seed=4)
    m = ModelWeights(p)
    moe = MoeExecutor(backend)
    x = orc.gauss(hidden, 17, 1.0)
    for layer in (0, 1):
        experts = [m.deepseek_expert(layer, e)[0] for e in range(4)]
        name, w_r = m.deepseek_router(layer)
        ids, wts, _, _ = orc.router(w_r.ravel(), x, 4, hidden, 2)
        sel = [(int(i), float(w)) for i, w in zip(ids, wts)]
        cache = ExpertCache(1 << 28, backend)
        out, tel = moe.execute_selected_moe_native_fp4_cuda(None, None, experts, sel, x, hidden, inter, hidden, layer,
                                                            cache)
        ref = orc.selected_moe(orc.FP4, [(e[0], e[1], e[2], e[3], e[4], e[5]) for e in experts], sel, x, hidden,
                               inter, hidden)
        assert_close(out, ref)
        assert tel["logical_expert_bytes_requested"] == sum(sum(a.nbytes for a in experts[e]) for e, _ in sel)
        cache.close()


def test_checkpoint_shared_expert_preloaded_for_the_official_executor(backend, tmp_path):
    hidden, inter = 512, 256
    p = tmp_path / "ds.safetensors"
    deepseek_checkpoint(p, hidden=hidden, inter=inter, experts=3, layers=(0, 1, 2), mtp=False, seed=9)
    m = ModelWeights(p)
    moe = MoeExecutor(backend)
    shared = [m.deepseek_shared_expert(l)[0] for l in range(3)]
    cache = ExpertCache(1 << 28, backend)
    nbytes, _ = cache.preload_shared(shared)
    assert nbytes == 3 * sum(a.nbytes for a in shared[0])
    x = orc.gauss(hidden, 5, 1.0)
    sel = [(2, 0.6), (0, 0.4)]
    for layer in range(3):
        experts = [m.deepseek_expert(layer, e)[0] for e in range(3)]
        sh_dev = [backend.to_device(np.ascontiguousarray(a)) for a in shared[layer]]
        want, _ = moe.execute_selected_moe_official_routed_fp4(
            None, None, experts, sel, x, hidden, inter, hidden, layer, None,
            (sh_dev[0], sh_dev[2], sh_dev[4], sh_dev[1], sh_dev[3], sh_dev[5]), 10.0)
        got, tel = moe.execute_selected_moe_official_routed_fp4(None, None, experts, sel, x, hidden, inter, hidden,
                                                                layer, cache, None, 10.0, shared_from_cache=True)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
        assert tel["shared_fp8_bytes_reused"] == sum(a.nbytes for a in shared[layer])
        # the official composition of the same bytes (routed experts plus the shared one)
        ref = np.zeros(hidden, np.float32)
        for e, w in sel:
            o, _, _, _ = orc.expert_official(False, experts[e], x, hidden, inter, 10.0)
            ref = (ref + np.float32(w) * o).astype(np.float32)
        o, _, _, _ = orc.expert_official(True, shared[layer], x, hidden, inter, 10.0)
        ref = (ref + o).astype(np.float32)
        c = orc.compare(ref, got)
        assert c["cosine_similarity"] >= 0.999, c  # intermediate FP8 codes may move (see test_gpu_official)
    cache.close()
