"""Host-to-device copies (objeta_hip_copy_h2d, the cache's miss copies): a pinned,
16-byte aligned source is copied by a kernel reading it through its device mapping,
anything else by HIP's copy. Every byte must arrive, whatever the path: sizes from
one 16-byte unit to several MiB, offsets that are and are not 16-byte aligned,
sizes that are not multiples of 16, and pageable numpy memory."""
import ctypes as C

import numpy as np
import pytest

from objeta_amd import PinnedHostBuffer, check

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("offset,size", [(0, 16), (0, 4096), (16, 1 << 20), (48, (3 << 20) + 80), (0, 884736),
                                         (8, 4096), (0, 4100), (4, 1 << 20), (0, 17)])
def test_copy_h2d_from_pinned_memory(backend, offset, size):
    L = backend.L
    pin = PinnedHostBuffer(backend, offset + size + 64)
    host = pin.array(np.uint8)
    rng = np.random.default_rng(size + offset)
    host[:] = rng.integers(0, 256, size=host.size, dtype=np.uint8)
    dst = backend.alloc(size + 64)
    dst.upload(np.zeros(size + 64, np.uint8))
    check(L.objeta_hip_copy_h2d(backend.ctx, None, dst.addr(), C.c_void_p(pin.ptr + offset), size))
    backend.synchronize()
    got = dst.download(np.uint8, size + 64)
    assert np.array_equal(got[:size], host[offset:offset + size])
    assert not got[size:].any()  # nothing written past the end
    pin.free()


def test_copy_h2d_from_pageable_memory(backend):
    src = np.random.default_rng(5).integers(0, 256, size=(1 << 20) + 32, dtype=np.uint8)
    dst = backend.alloc(src.size)
    check(backend.L.objeta_hip_copy_h2d(backend.ctx, None, dst.addr(), src.ctypes.data_as(C.c_void_p), src.size))
    backend.synchronize()
    assert np.array_equal(dst.download(np.uint8, src.size), src)
