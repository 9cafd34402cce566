"""One MoE layer of one token in a single launch: objeta_hip_moe_layer_fused_device
(top-8 routing, one selection slot per XCD; objeta_hip_moe_layer_fused_supported
says which shapes it takes, others are refused as Unsupported).

Each case checks, against the CPU oracle:
  * the expert ids equal cpu_router's (deepseek_single_layer_moe.rs:687-743,
    renormalised as moe_dispatch.rs:403-435) bit for bit, the weights within rtol 2e-5;
  * out = resid + selected_moe(x) (moe.rs:1283-1324 / 1665-1735) within
    1e-4 * max|ref| plus the reference's cosine / relative-L2 bars.
Consecutive calls, calls of other shapes in between, in-place updates, close calls
in the router, and replays of a captured graph are covered, since the launch takes
its epoch from a device counter rather than from the host."""
import ctypes as C

import numpy as np
import pytest

from objeta_amd import HipError, MoeExecutor, check
from oracle import oracle as orc
from test_gpu_stack import check_close, make_stack, oracle_stack

pytestmark = pytest.mark.gpu


def layer_call(backend, moe, fmt, layer, d_x, d_res, d_out, K, H, I, renormalize=True, stream=None):
    table, d_w, d_b, ids, wts = layer
    moe.layer_fused_device(fmt, table, d_w, d_b, K, d_x, d_res, d_out, ids, wts, H, I, H, renormalize=renormalize,
                           stream=stream)


def check_layer(fmt, layer, host_layer, x, out, E, K, H, I, pool, renormalize=True, what=""):
    ref, rids, rws = oracle_stack(fmt, [host_layer], x, E, K, H, I, pool, renormalize)
    _, _, _, ids, wts = layer
    got = ids.download(np.uint32, K)
    assert np.array_equal(got, rids[0]), f"{what}: ids {got} vs {rids[0]}"
    np.testing.assert_allclose(wts.download(np.float32, K), rws[0], rtol=2e-5, atol=1e-7)
    check_close(out, ref)


def fused(backend, fmt, E, K, H, I):
    return MoeExecutor(backend).layer_fused_supported(fmt, E, K, H, I, H)


@pytest.mark.parametrize("fmt,E,K,H,I,bias,expect_fused", [
    (0, 128, 8, 2048, 768, True, True),   # Qwen3-A3B layer
    (1, 32, 8, 1024, 256, True, True),
    (2, 16, 8, 512, 512, True, True),
    (3, 16, 8, 1024, 512, False, True),
    (0, 256, 8, 1024, 128, True, True),   # more router workgroups than gate/up ones
    (0, 8, 2, 2048, 1024, False, False),  # top-2
    (0, 64, 8, 4096, 512, True, False),   # hidden above the router's 2048
])
def test_fused_layer_matches_oracle(backend, fmt, E, K, H, I, bias, expect_fused):
    assert fused(backend, fmt, E, K, H, I) == expect_fused
    layers, host, keep = make_stack(backend, fmt, 1, E, K, H, I, seed=11 + fmt, bias=bias)
    moe = MoeExecutor(backend)
    if not expect_fused:
        d_x = backend.to_device(orc.gauss(H, 499, 1.0))
        with pytest.raises(HipError) as e:
            layer_call(backend, moe, fmt, layers[0], d_x, d_x, backend.alloc(4 * H), K, H, I)
        assert e.value.kind == "Unsupported"
        del keep
        return
    for r in range(3):
        x = orc.gauss(H, 500 + r, 1.0)
        d_x, d_out = backend.to_device(x), backend.alloc(4 * H)
        layer_call(backend, moe, fmt, layers[0], d_x, d_x, d_out, K, H, I)
        backend.synchronize()
        assert moe.device_error() == 0
        check_layer(fmt, layers[0], host[0], x, d_out.download(np.float32, H), E, K, H, I, 6, what=f"call {r}")
    del keep


def test_fused_layer_in_place_chain(backend):
    """h <- h + moe_l(h) for four layers, x, resid and out the same buffer."""
    E, K, H, I = 64, 8, 2048, 512
    assert fused(backend, 0, E, K, H, I)
    layers, host, keep = make_stack(backend, 0, 4, E, K, H, I, seed=12)
    moe = MoeExecutor(backend)
    x = orc.gauss(H, 77, 1.0)
    h = backend.to_device(x)
    ref = x.copy()
    for l in range(4):
        layer_call(backend, moe, 0, layers[l], h, h, h, K, H, I)
        backend.synchronize()
        assert moe.device_error() == 0
        out = h.download(np.float32, H)
        check_layer(0, layers[l], host[l], ref, out, E, K, H, I, 6, what=f"layer {l}")
        ref = out.copy()  # the next layer's oracle input is the device state
    del keep


def test_fused_layer_between_other_shapes(backend):
    """Launches of other grid shapes (another fused shape, the multi-token path)
    between calls must not disturb the epochs of the next call."""
    a = dict(E=32, K=8, H=1024, I=256)
    b = dict(E=128, K=8, H=2048, I=768)
    assert fused(backend, 0, **a) and fused(backend, 0, **b)
    la, ha, ka = make_stack(backend, 0, 1, seed=13, **a)
    lb, hb, kb = make_stack(backend, 0, 1, seed=14, **b)
    moe = MoeExecutor(backend)
    for r, (lay, hst, sh) in enumerate([(la, ha, a), (lb, hb, b), (la, ha, a), (la, ha, a), (lb, hb, b)]):
        x = orc.gauss(sh["H"], 900 + r, 1.0)
        d_x, d_out = backend.to_device(x), backend.alloc(4 * sh["H"])
        layer_call(backend, moe, 0, lay[0], d_x, d_x, d_out, sh["K"], sh["H"], sh["I"])
        if r == 2:  # a two-token call in between (router + per-assignment kernels)
            x2 = np.stack([orc.gauss(sh["H"], 950, 1.0), orc.gauss(sh["H"], 951, 1.0)])
            d2, o2 = backend.to_device(x2.ravel()), backend.alloc(8 * sh["H"])
            ids2, w2 = backend.alloc(8 * sh["K"]), backend.alloc(8 * sh["K"])
            table, d_w, d_b, _, _ = lay[0]
            moe.layer_device(0, table, d_w, d_b, sh["K"], 2, d2, d2, o2, ids2, w2, sh["H"], sh["I"], sh["H"])
        backend.synchronize()
        assert moe.device_error() == 0
        check_layer(0, lay[0], hst[0], x, d_out.download(np.float32, sh["H"]), sh["E"], sh["K"], sh["H"], sh["I"],
                    6, what=f"call {r}")
    del ka, kb


def test_fused_layer_raw_probabilities(backend):
    E, K, H, I = 32, 8, 1024, 256
    layers, host, keep = make_stack(backend, 0, 1, E, K, H, I, seed=15)
    moe = MoeExecutor(backend)
    x = orc.gauss(H, 15, 1.0)
    d_x, d_out = backend.to_device(x), backend.alloc(4 * H)
    layer_call(backend, moe, 0, layers[0], d_x, d_x, d_out, K, H, I, renormalize=False)
    backend.synchronize()
    assert moe.device_error() == 0
    check_layer(0, layers[0], host[0], x, d_out.download(np.float32, H), E, K, H, I, 6, renormalize=False)
    del keep


def test_fused_layer_close_calls_are_settled_exactly(backend):
    """Selected experts 2-3e-5 apart: the gate/up workgroups recompute the logits
    involved, workgroup 0 of each XCD hands the selection to its down workgroups."""
    from test_gpu_quantize_router import _close_calls
    E, K, H, I = 64, 8, 1024, 256
    assert fused(backend, 0, E, K, H, I)
    layers, host, keep = make_stack(backend, 0, 1, E, K, H, I, seed=16, bias=False)
    w, x = _close_calls(E, H, 43, [(1, 3e-5), (4, 2e-5), (7, 3e-5)])
    table, _, d_b, ids, wts = layers[0]
    d_w = backend.to_device(w.ravel())
    keep.append(d_w)
    layer = (table, d_w, d_b, ids, wts)
    host_layer = (host[0][0], w.ravel(), host[0][2])
    moe = MoeExecutor(backend)
    d_x, d_out = backend.to_device(x), backend.alloc(4 * H)
    layer_call(backend, moe, 0, layer, d_x, d_x, d_out, K, H, I)
    backend.synchronize()
    assert moe.device_error() == 0
    check_layer(0, layer, host_layer, x, d_out.download(np.float32, H), E, K, H, I, 6)
    del keep


def test_fused_layer_near_ties_take_the_sequential_path(backend):
    """Router rows that differ by one ulp: only the reference's sequential order
    decides, which workgroup 0 of each XCD computes and hands to the others."""
    E, K, H, I = 32, 8, 1024, 256
    assert fused(backend, 0, E, K, H, I)
    layers, host, keep = make_stack(backend, 0, 1, E, K, H, I, seed=17, tie_layer=0)
    moe = MoeExecutor(backend)
    for r in range(2):
        x = orc.gauss(H, 170 + r, 1.0)
        d_x, d_out = backend.to_device(x), backend.alloc(4 * H)
        layer_call(backend, moe, 0, layers[0], d_x, d_x, d_out, K, H, I)
        backend.synchronize()
        assert moe.device_error() == 0
        check_layer(0, layers[0], host[0], x, d_out.download(np.float32, H), E, K, H, I, 6, what=f"call {r}")
    del keep


def test_fused_layer_graph_replays(backend):
    """Two chained layers captured in a graph, replayed with new inputs copied in
    between: every replay equals the oracle (the epoch advances on the device)."""
    E, K, H, I = 64, 8, 2048, 768
    assert fused(backend, 0, E, K, H, I)
    layers, host, keep = make_stack(backend, 0, 2, E, K, H, I, seed=18)
    moe = MoeExecutor(backend)
    lib, ctx = backend.L, backend.ctx
    stream = backend.stream(0)
    h = backend.alloc(4 * H)
    x0 = orc.gauss(H, 180, 1.0)
    h.upload(x0)
    for l in range(2):  # eager first: workspaces are allocated outside capture
        layer_call(backend, moe, 0, layers[l], h, h, h, K, H, I, stream=stream)
    backend.synchronize(stream)
    check(lib.objeta_hip_graph_begin_capture(ctx, stream))
    for l in range(2):
        layer_call(backend, moe, 0, layers[l], h, h, h, K, H, I, stream=stream)
    g = C.c_void_p()
    check(lib.objeta_hip_graph_end_capture(ctx, stream, C.byref(g)))
    for r in range(4):
        x = orc.gauss(H, 181 + r, 1.0)
        h.upload(x, stream=stream)
        backend.synchronize(stream)
        check(lib.objeta_hip_graph_launch(ctx, g, stream))
        backend.synchronize(stream)
        assert moe.device_error() == 0
        ref, rids, _ = oracle_stack(0, host, x, E, K, H, I, 6)
        for l in range(2):
            assert np.array_equal(layers[l][3].download(np.uint32, K), rids[l]), f"replay {r} layer {l}"
        check_close(h.download(np.float32, H), ref)
    check(lib.objeta_hip_graph_destroy(ctx, g))
    del keep
