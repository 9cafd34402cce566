"""Persistent decode-stack kernel (objeta_hip_moe_stack_*) on the GPU.

Each case builds a small stack (device-generated Q formats or random split-FP4
bytes), runs it, and checks:
  * per layer, the expert ids equal the CPU oracle's router on the oracle's own
    hidden state (bit-exact), and the weights within rtol 2e-5;
  * the final hidden state equals the oracle's layer-by-layer
    h <- h + selected_moe(h) within 1e-4 * max|h| (plus the reference's cosine /
    rel-L2 bars);
  * the stack agrees with the same layers run through objeta_hip_moe_layer_device.
"""
import ctypes as C

import numpy as np
import pytest

from objeta_amd import ExpertTable, HipError, MoeExecutor, MoeStack, QuantFormat, check
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

BB = {0: 18, 1: 22, 2: 14}


def make_stack(backend, fmt, L, E, K, H, I, seed, pool=6, bias=True, tie_layer=None):
    """Per layer: a pool of distinct experts (table entry e -> pool[e % pool]), a router
    W_r [E][H] ~N(0, 0.02) and a bias. Returns device objects and host copies."""
    L_ = backend.L
    layers, host, keep = [], [], []
    for l in range(L):
        experts_h, entries = [], []
        for p in range(pool):
            if fmt == 3:
                rng = np.random.default_rng(seed * 1000 + l * 31 + p)
                tens = []
                for rows, cols in ((I, H), (I, H), (H, I)):
                    tens.append(rng.integers(0, 256, rows * cols // 2, dtype=np.uint8))
                    tens.append(rng.integers(119, 128, rows * cols // 32, dtype=np.uint8))
                g, gs, u, us, d, ds = tens
                bufs = [backend.to_device(a) for a in (g, u, d, gs, us, ds)]
                experts_h.append((g, gs, u, us, d, ds))
                entries.append(tuple(bufs))
            else:
                bb = BB[fmt]
                sizes = (I * (H // 32) * bb, I * (H // 32) * bb, H * (I // 32) * bb)
                bufs = []
                for t, (rows, cols) in enumerate(((I, H), (I, H), (H, I))):
                    b = backend.alloc(sizes[t])
                    check(L_.objeta_hip_fill_gauss_quantized_device(backend.ctx, fmt, None, b.addr(), rows, cols,
                                                                    seed * 100000 + l * 1000 + p * 3 + t,
                                                                    C.c_float(0.02)))
                    bufs.append(b)
                backend.synchronize()
                experts_h.append(tuple(b.download(np.uint8, b.nbytes) for b in bufs))
                entries.append(tuple(bufs))
            keep += bufs
        table = ExpertTable(backend, [entries[e % pool] for e in range(E)])
        w_r = orc.gauss(E * H, seed * 7 + l, 0.02).reshape(E, H).copy()
        if tie_layer == l:
            # rows that differ by one ulp in one element: only the sequential order decides
            base = w_r[0].copy()
            rng = np.random.default_rng(l)
            for e in range(E):
                w_r[e] = base
                j = rng.integers(0, H)
                w_r[e, j] = np.nextafter(base[j], np.float32(np.inf) if e % 2 else np.float32(-np.inf))
        b = orc.gauss(E, seed * 7 + 100 + l, 1.0) if bias and tie_layer != l else None
        d_w, d_b = backend.to_device(w_r.ravel()), (backend.to_device(b) if b is not None else None)
        ids, wts = backend.alloc(4 * K), backend.alloc(4 * K)
        layers.append((table, d_w, d_b, ids, wts))
        host.append((experts_h, w_r.ravel(), b))
        keep += [d_w, ids, wts] + ([d_b] if d_b is not None else [])
    return layers, host, keep


def oracle_stack(fmt, host, x, E, K, H, I, pool, renormalize=True):
    h = np.asarray(x, np.float32).copy()
    ids_all, ws_all = [], []
    for experts_h, w_r, b in host:
        rid, rw, _, _ = orc.router(w_r, h, E, H, K, bias=b, renormalize=renormalize)
        ids_all.append(rid)
        ws_all.append(rw)
        sel = [(int(e) % pool, float(w)) for e, w in zip(rid, rw)]
        out = orc.selected_moe(fmt, experts_h, sel, h, H, I, H)
        h = (h + out).astype(np.float32)
    return h, ids_all, ws_all


def check_close(out, ref):
    out, ref = np.asarray(out, np.float64), np.asarray(ref, np.float64)
    scale = max(float(np.max(np.abs(ref))), 1e-30)
    err = float(np.max(np.abs(out - ref)))
    assert err <= 1e-4 * scale, f"max rel err {err / scale:.3e}"
    c = orc.compare(ref.astype(np.float32), out.astype(np.float32))
    assert c["cosine_similarity"] >= 0.9999 and c["relative_l2_error"] <= 1e-4, c


def run_case(backend, fmt, L, E, K, H, I, seed, pool=6, bias=True, renormalize=True, tie_layer=None, runs=2):
    layers, host, keep = make_stack(backend, fmt, L, E, K, H, I, seed, pool, bias, tie_layer)
    st = MoeStack(backend, fmt, layers, E, K, H, I, renormalize=renormalize)
    moe = MoeExecutor(backend)
    for r in range(runs):
        x = orc.gauss(H, seed * 13 + r, 1.0)
        d_x = backend.to_device(x)
        d_out = backend.alloc(4 * H)
        st.run(d_x, d_out)
        backend.synchronize()
        assert moe.device_error() == 0
        out = d_out.download(np.float32, H)
        ref, rids, rws = oracle_stack(fmt, host, x, E, K, H, I, pool, renormalize)
        for l, (table, d_w, d_b, ids, wts) in enumerate(layers):
            got = ids.download(np.uint32, K)
            assert np.array_equal(got, rids[l]), f"run {r} layer {l}: {got} vs {rids[l]}"
            np.testing.assert_allclose(wts.download(np.float32, K), rws[l], rtol=2e-5, atol=1e-7)
        check_close(out, ref)
        # the same layers, one objeta_hip_moe_layer_device call each
        h = backend.to_device(x)
        for table, d_w, d_b, ids, wts in layers:
            moe.layer_device(fmt, table, d_w, d_b, K, 1, h, h, h, ids, wts, H, I, H, renormalize=renormalize)
        backend.synchronize()
        chained = h.download(np.float32, H)
        np.testing.assert_allclose(out, chained, rtol=0, atol=1e-5 * max(1.0, float(np.max(np.abs(chained)))))
    info = st.info()
    st.close()
    del keep
    return info


def test_stack_qwen3_a3b_shape(backend):
    """hidden 2048, 128 experts, top-8, intermediate 768 (4 layers of the Qwen3-A3B stack)."""
    info = run_case(backend, 0, L=4, E=128, K=8, H=2048, I=768, seed=1)
    assert info["grid"] > 32


def test_stack_eight_expert_top2(backend):
    run_case(backend, 0, L=3, E=8, K=2, H=2048, I=1024, seed=2, bias=False)


@pytest.mark.parametrize("fmt,E,K,H,I", [(1, 32, 4, 512, 256), (2, 16, 3, 256, 128), (3, 16, 4, 1024, 512)])
def test_stack_formats(backend, fmt, E, K, H, I):
    run_case(backend, fmt, L=2, E=E, K=K, H=H, I=I, seed=3)


def test_stack_raw_probabilities(backend):
    run_case(backend, 0, L=2, E=16, K=4, H=512, I=256, seed=4, renormalize=False)


def test_stack_near_ties_take_the_sequential_path(backend):
    """A layer whose router rows differ by one ulp: the publisher workgroup recomputes
    in the reference's order and every other workgroup waits for its selection."""
    run_case(backend, 0, L=3, E=32, K=4, H=512, I=256, seed=5, tie_layer=0, runs=1)


def test_stack_rejects_unsupported_shapes(backend):
    layers, host, keep = make_stack(backend, 0, 1, 8, 2, 256, 64, 6, pool=1)
    with pytest.raises(HipError) as e:
        MoeStack(backend, 0, layers, 8, 2, 7168, 64)
    assert e.value.kind == "Unsupported"
    with pytest.raises(HipError) as e:
        MoeStack(backend, 0, layers, 8, 9, 256, 64)
    assert e.value.kind in ("Unsupported", "InvalidInput")
    del keep


def test_stack_close_calls_are_settled_exactly(backend):
    """Layer 0's router has adjacent selected experts 2-3e-5 apart for the run's token:
    every workgroup recomputes those logits and the stack must match the oracle."""
    from test_gpu_quantize_router import _close_calls
    E, K, H, I = 64, 8, 512, 256
    layers, host, keep = make_stack(backend, 0, 2, E, K, H, I, seed=7, bias=False)
    w, x = _close_calls(E, H, 41, [(1, 3e-5), (4, 2e-5), (7, 3e-5)])
    table, d_w, d_b, ids, wts = layers[0]
    layers[0] = (table, backend.to_device(w.ravel()), d_b, ids, wts)
    keep.append(layers[0][1])
    experts_h, _, b = host[0]
    host[0] = (experts_h, w.ravel(), b)
    st = MoeStack(backend, 0, layers, E, K, H, I)
    d_x = backend.to_device(x)
    d_out = backend.alloc(4 * H)
    st.run(d_x, d_out)
    backend.synchronize()
    assert MoeExecutor(backend).device_error() == 0
    ref, rids, rws = oracle_stack(0, host, x, E, K, H, I, 6)
    for l, (_, _, _, ids_l, wts_l) in enumerate(layers):
        assert np.array_equal(ids_l.download(np.uint32, K), rids[l]), f"layer {l}"
        np.testing.assert_allclose(wts_l.download(np.float32, K), rws[l], rtol=2e-5, atol=1e-7)
    check_close(d_out.download(np.float32, H), ref)
    st.close()
    del keep
