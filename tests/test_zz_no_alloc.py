"""objeta_hip_moe_selected_device_noalloc (no allocation; activations in a static
device array) against objeta_hip_moe_selected_device through the C ABI: the two
entry points run the same kernels, so their outputs must be bit-identical. Two
calls in a row, the second with a smaller input, so that the static array carries
the first call's contents into the second; plus the size limit."""
import ctypes as C

import numpy as np
import pytest

from objeta_amd import ExpertTable, HipError, MoeExecutor, QuantFormat, check
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

Q4 = int(QuantFormat.Q4_0)
LIMIT = 1 << 20  # floats of the static activation array


def _experts(backend, n, hidden, inter, out_dim, seed):
    keep, entries, host = [], [], []
    for e in range(n):
        mats = [orc.quantize_matrix(Q4, orc.gauss(r * c, seed + 3 * e + i, 0.02), r, c)
                for i, (r, c) in enumerate(((inter, hidden), (inter, hidden), (out_dim, inter)))]
        bufs = [backend.to_device(m) for m in mats]
        host.append(tuple(mats))
        keep += bufs
        entries.append(tuple(bufs))
    return ExpertTable(backend, entries), keep, host


def _run(backend, fn, table, d_ids, d_w, T, k, d_x, d_res, hidden, inter, out_dim):
    d_out = backend.alloc(4 * T * out_dim)
    check(fn(backend.ctx, Q4, None, table.addr(), C.c_uint64(table.n), d_ids.addr(), d_w.addr(), C.c_uint64(T),
             C.c_uint64(k), d_x.addr(), None if d_res is None else d_res.addr(), d_out.addr(), C.c_uint64(hidden),
             C.c_uint64(inter), C.c_uint64(out_dim), C.c_float(0.0)))
    backend.synchronize()
    return d_out.download(np.float32, T * out_dim).reshape(T, out_dim)


@pytest.mark.parametrize("calls", [[(16, 8, 2048, 768, 2048, 32), (3, 4, 1024, 512, 1024, 12)],
                                   [(1, 8, 2048, 768, 2048, 128), (1, 2, 256, 128, 512, 4)]])
def test_noalloc_matches_selected_device(backend, calls):
    L = backend.L
    moe = MoeExecutor(backend)
    for ci, (T, k, hidden, inter, out_dim, n) in enumerate(calls):
        table, keep, host = _experts(backend, n, hidden, inter, out_dim, 100 * ci + 1)
        rng = np.random.default_rng(ci)
        ids = rng.integers(0, n, size=T * k).astype(np.uint32)
        w = rng.random(T * k).astype(np.float32)
        xs = orc.gauss(T * hidden, 50 + ci, 1.0)
        res = orc.gauss(T * out_dim, 60 + ci, 1.0)
        d_ids, d_w, d_x, d_res = (backend.to_device(a) for a in (ids, w, xs, res))
        ref = _run(backend, L.objeta_hip_moe_selected_device, table, d_ids, d_w, T, k, d_x, d_res, hidden, inter,
                   out_dim)
        got = _run(backend, L.objeta_hip_moe_selected_device_noalloc, table, d_ids, d_w, T, k, d_x, d_res, hidden,
                   inter, out_dim)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), f"call {ci}: outputs differ"
        # and both within the oracle's bar for the first token
        sel = [(int(ids[j]), float(w[j])) for j in range(k)]
        oref = orc.selected_moe(Q4, host, sel, xs[:hidden], hidden, inter, out_dim)
        err = np.max(np.abs((got[0] - res[:out_dim]).astype(np.float64) - oref))
        assert err <= 1e-4 * max(1e-30, float(np.max(np.abs(oref))))
        assert moe.device_error() == 0
        del keep


def test_noalloc_rejects_oversized(backend):
    L = backend.L
    table, keep, _ = _experts(backend, 1, 256, 128, 256, 7)
    T, k, inter = 1025, 8, 128  # 1025 * 8 * 128 > 2^20
    assert T * k * inter > LIMIT
    d_ids = backend.to_device(np.zeros(T * k, np.uint32))
    d_w = backend.to_device(np.ones(T * k, np.float32))
    d_x = backend.to_device(np.zeros(T * 256, np.float32))
    d_out = backend.alloc(4 * T * 256)
    with pytest.raises(HipError) as ei:
        check(L.objeta_hip_moe_selected_device_noalloc(backend.ctx, Q4, None, table.addr(), C.c_uint64(1),
                                                         d_ids.addr(), d_w.addr(), C.c_uint64(T), C.c_uint64(k),
                                                         d_x.addr(), None, d_out.addr(), C.c_uint64(256),
                                                         C.c_uint64(inter), C.c_uint64(256), C.c_float(0.0)))
    assert ei.value.kind == "InvalidInput" and "static scratch" in ei.value.source_message
    del keep
