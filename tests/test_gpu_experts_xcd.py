"""One token through objeta_hip_moe_layer_device with top-8 routing on a context
created with OBJETA_HIP_EXPERTS_XCD=1: the router kernel, then the selected
experts in one launch laid out over the XCDs
(gate/up + SiLU and down + combine; selection slot j on XCD j). The three-kernel
form (objeta_hip_moe_selected_device on the same ids and weights) and the CPU
oracle are the references.

Each case checks:
  * the expert ids equal cpu_router's (deepseek_single_layer_moe.rs:687-743,
    renormalised as moe_dispatch.rs:403-435) bit for bit, the weights within rtol 2e-5;
  * out = resid + selected_moe(x) (moe.rs:1283-1324 / 1665-1735) within
    1e-4 * max|ref| plus the reference's cosine / relative-L2 bars;
  * out within 1e-5 * max|out| of the three-kernel form (only the order of the
    fp32 sums inside a row differs).
The launch takes its epoch from a device counter, so consecutive calls, in-place
updates (x, resid and out one buffer), other launches in between and replays of a
captured graph are covered too."""
import ctypes as C

import numpy as np
import pytest

from objeta_amd import MoeExecutor, check
from oracle import oracle as orc
from test_gpu_stack import check_close, make_stack, oracle_stack

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def backend():
    """A context created with OBJETA_HIP_EXPERTS_XCD=1, so that one-token top-8
    layers take the XCD-aligned expert launch (off by default)."""
    import os
    from objeta_amd import HipBackend
    old = os.environ.get("OBJETA_HIP_EXPERTS_XCD")
    os.environ["OBJETA_HIP_EXPERTS_XCD"] = "1"
    try:
        be = HipBackend(0, 2)
    finally:
        if old is None:
            del os.environ["OBJETA_HIP_EXPERTS_XCD"]
        else:
            os.environ["OBJETA_HIP_EXPERTS_XCD"] = old
    yield be
    be.close()


def xcd_shape(backend, fmt, E, K, H, I):
    # the expert kernel takes the fused layer's shapes (its router limits aside)
    return MoeExecutor(backend).layer_fused_supported(fmt, E, K, H, I, H)


def layer_call(moe, fmt, layer, d_x, d_res, d_out, K, H, I, renormalize=True, stream=None):
    table, d_w, d_b, ids, wts = layer
    moe.layer_device(fmt, table, d_w, d_b, K, 1, d_x, d_res, d_out, ids, wts, H, I, H, renormalize=renormalize,
                     stream=stream)


def check_layer(backend, moe, fmt, layer, host_layer, x, out, E, K, H, I, pool=6, renormalize=True, what=""):
    ref, rids, rws = oracle_stack(fmt, [host_layer], x, E, K, H, I, pool, renormalize)
    table, _, _, ids, wts = layer
    got = ids.download(np.uint32, K)
    assert np.array_equal(got, rids[0]), f"{what}: ids {got} vs {rids[0]}"
    np.testing.assert_allclose(wts.download(np.float32, K), rws[0], rtol=2e-5, atol=1e-7)
    check_close(out, ref)
    # the three-kernel form on the same routing
    d_x, d_o = backend.to_device(np.asarray(x, np.float32)), backend.alloc(4 * H)
    moe.selected_device(fmt, table, ids, wts, 1, K, d_x, d_x, d_o, H, I, H)
    backend.synchronize()
    three = d_o.download(np.float32, H).astype(np.float64)
    err = float(np.max(np.abs(np.asarray(out, np.float64) - three)))
    assert err <= 1e-5 * max(float(np.max(np.abs(three))), 1e-30), f"{what}: vs three kernels {err:.3e}"


@pytest.mark.parametrize("fmt,E,K,H,I,bias", [
    (0, 128, 8, 2048, 768, True),   # Qwen3-A3B layer
    (1, 32, 8, 1024, 256, True),
    (2, 16, 8, 512, 512, True),
    (3, 16, 8, 1024, 512, False),
    (0, 256, 8, 1024, 128, True),
    (1, 64, 8, 256, 1024, False),
])
def test_experts_xcd_matches_oracle_and_three_kernels(backend, fmt, E, K, H, I, bias):
    assert xcd_shape(backend, fmt, E, K, H, I)
    layers, host, keep = make_stack(backend, fmt, 1, E, K, H, I, seed=31 + fmt, bias=bias)
    moe = MoeExecutor(backend)
    for r in range(3):
        x = orc.gauss(H, 600 + r, 1.0)
        d_x, d_out = backend.to_device(x), backend.alloc(4 * H)
        layer_call(moe, fmt, layers[0], d_x, d_x, d_out, K, H, I)
        backend.synchronize()
        assert moe.device_error() == 0
        check_layer(backend, moe, fmt, layers[0], host[0], x, d_out.download(np.float32, H), E, K, H, I,
                    what=f"call {r}")
    del keep


def test_experts_xcd_in_place_chain(backend):
    """h <- h + moe_l(h) for four layers with x, resid and out one buffer: no
    workgroup may overwrite h while another still reads it."""
    E, K, H, I = 128, 8, 2048, 768
    layers, host, keep = make_stack(backend, 0, 4, E, K, H, I, seed=32)
    moe = MoeExecutor(backend)
    x = orc.gauss(H, 78, 1.0)
    h = backend.to_device(x)
    ref = x.copy()
    for l in range(4):
        layer_call(moe, 0, layers[l], h, h, h, K, H, I)
        backend.synchronize()
        assert moe.device_error() == 0
        out = h.download(np.float32, H)
        check_layer(backend, moe, 0, layers[l], host[l], ref, out, E, K, H, I, what=f"layer {l}")
        ref = out.copy()
    del keep


def test_experts_xcd_between_other_launches(backend):
    """Calls of another shape, of the single-launch layer and of a two-token batch
    between calls: the shared epoch counter keeps every call's words apart."""
    a = dict(E=32, K=8, H=1024, I=256)
    b = dict(E=128, K=8, H=2048, I=768)
    la, ha, ka = make_stack(backend, 0, 1, seed=33, **a)
    lb, hb, kb = make_stack(backend, 0, 1, seed=34, **b)
    moe = MoeExecutor(backend)
    for r, (lay, hst, sh) in enumerate([(la, ha, a), (lb, hb, b), (la, ha, a), (lb, hb, b), (la, ha, a)]):
        x = orc.gauss(sh["H"], 910 + r, 1.0)
        d_x, d_out = backend.to_device(x), backend.alloc(4 * sh["H"])
        layer_call(moe, 0, lay[0], d_x, d_x, d_out, sh["K"], sh["H"], sh["I"])
        table, d_w, d_b, _, _ = lay[0]
        if r == 1:  # the single-launch layer on the same context
            i1, w1, o1 = backend.alloc(4 * sh["K"]), backend.alloc(4 * sh["K"]), backend.alloc(4 * sh["H"])
            moe.layer_fused_device(0, table, d_w, d_b, sh["K"], d_x, d_x, o1, i1, w1, sh["H"], sh["I"], sh["H"])
        if r == 2:  # a two-token call (router + per-assignment kernels)
            x2 = np.stack([orc.gauss(sh["H"], 960, 1.0), orc.gauss(sh["H"], 961, 1.0)])
            d2, o2 = backend.to_device(x2.ravel()), backend.alloc(8 * sh["H"])
            ids2, w2 = backend.alloc(8 * sh["K"]), backend.alloc(8 * sh["K"])
            moe.layer_device(0, table, d_w, d_b, sh["K"], 2, d2, d2, o2, ids2, w2, sh["H"], sh["I"], sh["H"])
        backend.synchronize()
        assert moe.device_error() == 0
        check_layer(backend, moe, 0, lay[0], hst[0], x, d_out.download(np.float32, sh["H"]), sh["E"], sh["K"],
                    sh["H"], sh["I"], what=f"call {r}")
    del ka, kb


def test_experts_xcd_raw_probabilities(backend):
    E, K, H, I = 32, 8, 1024, 256
    layers, host, keep = make_stack(backend, 0, 1, E, K, H, I, seed=35)
    moe = MoeExecutor(backend)
    x = orc.gauss(H, 35, 1.0)
    d_x, d_out = backend.to_device(x), backend.alloc(4 * H)
    layer_call(moe, 0, layers[0], d_x, d_x, d_out, K, H, I, renormalize=False)
    backend.synchronize()
    assert moe.device_error() == 0
    ref, rids, _ = oracle_stack(0, host, x, E, K, H, I, 6, renormalize=False)
    assert np.array_equal(layers[0][3].download(np.uint32, K), rids[0])
    check_close(d_out.download(np.float32, H), ref)
    del keep


def test_experts_xcd_graph_replays(backend):
    """Three chained layers captured in a graph and replayed with new inputs copied
    in between, eager work and synchronisation between replays: every replay
    equals the oracle."""
    E, K, H, I = 128, 8, 2048, 768
    layers, host, keep = make_stack(backend, 0, 3, E, K, H, I, seed=36)
    moe = MoeExecutor(backend)
    lib, ctx = backend.L, backend.ctx
    stream = backend.stream(0)
    h = backend.alloc(4 * H)
    h.upload(orc.gauss(H, 190, 1.0))
    for l in range(3):  # eager first: workspaces and the XCD probe outside capture
        layer_call(moe, 0, layers[l], h, h, h, K, H, I, stream=stream)
    backend.synchronize(stream)
    check(lib.objeta_hip_graph_begin_capture(ctx, stream))
    for l in range(3):
        layer_call(moe, 0, layers[l], h, h, h, K, H, I, stream=stream)
    g = C.c_void_p()
    check(lib.objeta_hip_graph_end_capture(ctx, stream, C.byref(g)))
    try:
        for r in range(4):
            x = orc.gauss(H, 191 + r, 1.0)
            h.upload(x, stream=stream)
            backend.synchronize(stream)
            check(lib.objeta_hip_graph_launch(ctx, g, stream))
            backend.synchronize(stream)
            assert moe.device_error() == 0
            ref, rids, _ = oracle_stack(0, host, x, E, K, H, I, 6)
            for l in range(3):
                assert np.array_equal(layers[l][3].download(np.uint32, K), rids[l]), f"replay {r} layer {l}"
            check_close(h.download(np.float32, H), ref)
            # eager work between replays
            d_x, d_o = backend.to_device(x), backend.alloc(4 * H)
            layer_call(moe, 0, layers[0], d_x, d_x, d_o, K, H, I, stream=stream)
            backend.synchronize(stream)
    finally:
        check(lib.objeta_hip_graph_destroy(ctx, g))
    del keep
