"""Parity at the benchmark configurations, on the GPU through the C ABI, against the
CPU oracle:

- the format sweep: Q4_0 / Q5_0 / IQ3_0 GEMV at [4096 x 4096] and [14336 x 4096],
  batch 1 and 8 (every output element against orc_gemv);
- the 4-layer x 8-expert top-2 stack (H 2048, I 1024), layer after layer;
- the Qwen3-A3B-shaped layer (H 2048, I 768, 128 experts, top-8, Zipf(1.1) router
  bias) through the host-in/host-out executor from pinned host memory, with the
  expert cache capped at 25% of the expert bytes of two layers so that LRU
  eviction runs; outputs against selected_moe_cpu and every telemetry counter
  against the oracle's cache model;
- the DeepSeek-V3-class FP4 layer (H 7168, 256 routed experts + 1 shared, top-8,
  I 2048) at batch 1 and 32, through the layer entry point and through the router
  plus the grouped-token product.

Bars: expert ids bit-exact with cpu_router (softmax -> stable top-k ->
renormalise); outputs within 1e-4 * max|ref| plus the reference's own cosine /
rel-L2 / max-abs thresholds (assert_moe_close; the FP4 layer's outputs are of
order 1e6, where only the relative bars are meaningful)."""
import ctypes as C

import numpy as np
import pytest

from objeta_amd import (ExpertCache, ExpertTable, MoeExecutor, PinnedHostBuffer, QGemvShape, QuantFormat,
                        check)
from objeta_amd.workloads import fp4_random_expert, zipf_bias
from oracle import cache_model as cm
from oracle import oracle as orc
from tests.test_gpu_executor import check_telemetry
from tests.test_gpu_moe import assert_moe_close

pytestmark = pytest.mark.gpu

Q4, Q5, IQ3, FP4 = 0, 1, 2, 3


def _fill_quantized(backend, fmt, rows, cols, seed, sigma=0.02):
    buf = backend.alloc(rows * (cols // 32) * orc.BLOCK_BYTES[fmt])
    check(backend.L.objeta_hip_fill_gauss_quantized_device(backend.ctx, fmt, None, buf.addr(), rows, cols, seed,
                                                           C.c_float(sigma)))
    return buf


def _bb(fmt):
    return orc.BLOCK_BYTES[fmt]


# ------------------------------------------------------------------ format sweep
@pytest.mark.parametrize("fmt", [Q4, Q5, IQ3])
@pytest.mark.parametrize("rows", [4096, 14336])
def test_format_sweep_gemv(backend, quant, fmt, rows):
    cols = 4096
    dq = _fill_quantized(backend, fmt, rows, cols, 9000 + 10 * fmt + rows)
    q = dq.download(np.uint8, rows * (cols // 32) * _bb(fmt))
    xs = orc.gauss(8 * cols, 9100 + fmt, 1.0)
    dx = backend.to_device(xs)
    shape = QGemvShape.new(QuantFormat(fmt), rows, cols)
    for B in (1, 8):
        dy = backend.alloc(4 * B * rows)
        quant.launch_kernel(QuantFormat(fmt), None, dq, dx, dy, shape, batch=B)
        y = dy.download(np.float32, B * rows).reshape(B, rows)
        for t in range(B):
            ref = orc.gemv(fmt, q, xs[t * cols:(t + 1) * cols], rows, cols)
            scale = float(np.max(np.abs(ref)))
            err = float(np.max(np.abs(y[t].astype(np.float64) - ref)))
            assert err <= 1e-4 * scale, f"B={B} t={t}: rel err {err / scale:.3e}"
            assert orc.compare(ref, y[t])["cosine_similarity"] >= 0.9999


# ------------------------------------------------- 4-layer x 8-expert top-2 stack
def test_four_layer_eight_expert_stack(backend):
    H, I, E, K, L = 2048, 1024, 8, 2, 4
    moe = MoeExecutor(backend)
    gu, dn = I * (H // 32) * 18, H * (I // 32) * 18
    keep, tables, host, wrs = [], [], [], []
    for l in range(L):
        entries, hexp = [], []
        for e in range(E):
            key = 5000 + 3 * (l * E + e)
            g = _fill_quantized(backend, Q4, I, H, key)
            u = _fill_quantized(backend, Q4, I, H, key + 1)
            d = _fill_quantized(backend, Q4, H, I, key + 2)
            keep += [g, u, d]
            entries.append((g, u, d))
            hexp.append((g.download(np.uint8, gu), u.download(np.uint8, gu), d.download(np.uint8, dn)))
        tables.append(ExpertTable(backend, entries))
        host.append(hexp)
        wrs.append(orc.gauss(E * H, 5900 + l, 0.02))
    d_wr = [backend.to_device(w) for w in wrs]
    hs = [backend.to_device(orc.gauss(H, 5999, 1.0))] + [backend.alloc(4 * H) for _ in range(L)]
    d_ids, d_w = backend.alloc(4 * L * K), backend.alloc(4 * L * K)
    for l in range(L):
        moe.layer_device(Q4, tables[l], d_wr[l], None, K, 1, hs[l], hs[l], hs[l + 1], d_ids.addr(4 * l * K),
                         d_w.addr(4 * l * K), H, I, H)
    backend.synchronize()
    ids = d_ids.download(np.uint32, L * K).reshape(L, K)
    for l in range(L):
        hin = hs[l].download(np.float32, H)
        hout = hs[l + 1].download(np.float32, H)
        rid, rw, _, _ = orc.router(wrs[l], hin, E, H, K, renormalize=True)
        assert np.array_equal(ids[l], rid), l
        ref = orc.selected_moe(Q4, host[l], [(int(i), float(v)) for i, v in zip(rid, rw)], hin, H, I, H)
        assert_moe_close(hout - hin, ref)
    assert moe.device_error() == 0
    del keep


# ------------------------------------- Qwen3-A3B layer, cache at 25% of expert bytes
def test_qwen3_a3b_cache_quarter_capacity(backend):
    H, I, E, K, L, T, POOL = 2048, 768, 128, 8, 2, 40, 16
    gu, dn = I * (H // 32) * 18, H * (I // 32) * 18
    eb = 2 * gu + dn
    assert eb == 2654208
    pin = PinnedHostBuffer(backend, POOL * eb)
    arr = pin.array(np.uint8)
    pool = []
    for p in range(POOL):
        for j, (r, c) in enumerate(((I, H), (I, H), (H, I))):
            buf = _fill_quantized(backend, Q4, r, c, 7000 + 3 * p + j)
            off = p * eb + (0, gu, 2 * gu)[j]
            n = gu if j < 2 else dn
            arr[off:off + n] = buf.download(np.uint8, n)
            buf.free()
        base = p * eb
        pool.append((arr[base:base + gu], arr[base + gu:base + 2 * gu], arr[base + 2 * gu:base + eb]))
    experts = [pool[e % POOL] for e in range(E)]  # host tensors of expert e (pinned)
    lens = [(gu, gu, dn)] * E
    capacity = (L * E * eb) // 4
    cache = ExpertCache(capacity, backend)
    model = cm.CacheModel(capacity)
    moe = MoeExecutor(backend)
    wrs = [orc.gauss(E * H, 7500 + l, 0.02) for l in range(L)]
    biases = [zipf_bias(E, 1.1, 7600 + l) for l in range(L)]
    for t in range(T):
        h = orc.gauss(H, 7700 + t, 1.0)
        for l in range(L):
            rid, rw, _, _ = orc.router(wrs[l], h, E, H, K, bias=biases[l], renormalize=True)
            sel = [(int(i), float(v)) for i, v in zip(rid, rw)]
            out, tel = moe.execute_selected_moe_cuda(None, None, experts, sel, h, H, I, H, l, cache)
            mt = cm.execute_accounting(model, Q4, lens, sel, l)
            check_telemetry(tel, mt, model, Q4)
            ref = orc.selected_moe(Q4, experts, sel, h, H, I, H)
            assert_moe_close(out, ref)
            h = (h + out).astype(np.float32)
    st = cache.stats()
    assert st["eviction_count"] > 0 and st["hit_count"] > 0, st
    assert st["resident_bytes"] <= capacity
    cache.close()
    pin.free()


# ------------------------------------ DeepSeek-V3-class FP4 layer, 256 + 1 shared
@pytest.fixture(scope="module")
def ds_layer(backend):
    H, I, E, K, POOL = 7168, 2048, 256, 8, 10
    pool = [fp4_random_expert(H, I, H, 8000 + 3 * p) for p in range(POOL)]
    shared_host = fp4_random_expert(H, I, H, 8999)
    keep = []

    def dev(e):
        gw, gs, uw, us, dw, ds = (backend.to_device(a) for a in e)
        keep.extend([gw, gs, uw, us, dw, ds])
        return (gw, uw, dw, gs, us, ds)

    pool_dev = [dev(e) for e in pool]
    table = ExpertTable(backend, [pool_dev[e % POOL] for e in range(E)])
    shared = ExpertTable(backend, [dev(shared_host)])
    w_r = orc.gauss(E * H, 8100, 0.02)
    return dict(H=H, I=I, E=E, K=K, table=table, shared=shared, host=[pool[e % POOL] for e in range(E)],
                shared_host=shared_host, w_r=w_r, d_wr=backend.to_device(w_r), keep=keep)


@pytest.fixture
def oracle_threads():
    """The oracle's row loops on 16 host threads while a test checks every token."""
    orc.set_threads(16)
    yield
    orc.set_threads(1)


# 4 tokens: the grouped path, which the layer entry takes from 2 tokens at this shape
@pytest.mark.parametrize("T", [1, 4, 32])
def test_deepseek_fp4_layer_with_shared_expert(backend, ds_layer, oracle_threads, T):
    d = ds_layer
    H, I, E, K = d["H"], d["I"], d["E"], d["K"]
    xs = orc.gauss(T * H, 8200 + T, 1.0).reshape(T, H)
    d_x = backend.to_device(xs.ravel())
    d_out = backend.alloc(4 * T * H)
    d_ids, d_w = backend.alloc(4 * T * K), backend.alloc(4 * T * K)
    moe = MoeExecutor(backend)
    moe.layer_device(FP4, d["table"], d["d_wr"], None, K, T, d_x, None, d_out, d_ids, d_w, H, I, H,
                     shared=d["shared"])
    backend.synchronize()
    ids = d_ids.download(np.uint32, T * K).reshape(T, K)
    ws = d_w.download(np.float32, T * K).reshape(T, K)
    out = d_out.download(np.float32, T * H).reshape(T, H)
    sels = []
    for t in range(T):
        rid, rw, _, _ = orc.router(d["w_r"], xs[t], E, H, K, renormalize=True)
        assert np.array_equal(ids[t], rid), t
        # the device weights come from the exact logit sums, the reference's from its
        # sequential fp32 sums (7168 terms): they agree to the path's 1e-4 bar
        np.testing.assert_allclose(ws[t], rw, rtol=1e-4, atol=1e-7)
        sels.append([(int(i), float(v)) for i, v in zip(rid, rw)])
    for t in range(T):
        ref = orc.selected_moe(FP4, d["host"], sels[t], xs[t], H, I, H, shared=d["shared_host"])
        # uniform E2M1 codes with scales up to 2^0 give outputs of order 1e6: the
        # absolute 1e-2 bar of the reference's small test shapes does not apply
        assert_moe_close(out[t], ref, abs_bar=None)
    assert moe.device_error() == 0


def test_deepseek_fp4_batch32_grouped(backend, ds_layer, oracle_threads):
    """Batch 32 through the router and the grouped-token product (routed experts)."""
    d = ds_layer
    H, I, E, K, T = d["H"], d["I"], d["E"], d["K"], 32
    xs = orc.gauss(T * H, 8300, 1.0).reshape(T, H)
    d_x = backend.to_device(xs.ravel())
    d_out = backend.alloc(4 * T * H)
    d_ids, d_w = backend.alloc(4 * T * K), backend.alloc(4 * T * K)
    check(backend.L.objeta_hip_router_topk_device(backend.ctx, None, d["d_wr"].addr(), None, d_x.addr(), T, E, H, K,
                                                   1, d_ids.addr(), d_w.addr()))
    moe = MoeExecutor(backend)
    moe.grouped_device(FP4, d["table"], d_ids, d_w, T, K, d_x, d_x, d_out, H, I, H)
    backend.synchronize()
    ids = d_ids.download(np.uint32, T * K).reshape(T, K)
    out = d_out.download(np.float32, T * H).reshape(T, H)
    for t in range(T):
        rid, rw, _, _ = orc.router(d["w_r"], xs[t], E, H, K, renormalize=True)
        assert np.array_equal(ids[t], rid), t
        ref = orc.selected_moe(FP4, d["host"], [(int(i), float(v)) for i, v in zip(rid, rw)], xs[t], H, I, H)
        assert_moe_close(out[t] - xs[t], ref, abs_bar=None)
    assert moe.device_error() == 0
