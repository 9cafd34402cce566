"""GEMV parity on the GPU through the C ABI against the CPU oracle.

Tolerance: GPU and CPU sum the same products in different orders, so results
differ by fp32 rounding only. Per element we require
    |y - ref| <= 1e-4 * max|ref|     (the path's 1e-4 relative bound)
and, tighter, |y - ref| <= 2^-18 * sum_j |w_j x_j| + 1e-30 (a few hundred ulps of
the dot product's magnitude)."""
import ctypes as C

import numpy as np
import pytest

from objeta_amd import QGemvShape, QuantFormat
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

FORMATS = [QuantFormat.Q4_0, QuantFormat.Q5_0, QuantFormat.IQ3_0, QuantFormat.DeepSeekFp4E2M1]


def _assert_close(y, ref, q, x, fmt, rows, cols):
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    assert y.shape == ref.shape
    scale = max(float(np.max(np.abs(ref))), 1e-30)
    err = np.abs(y - ref)
    assert float(err.max()) <= 1e-4 * scale, f"rel err {err.max() / scale:.3e}"
    if fmt != QuantFormat.DeepSeekFp4E2M1:
        from tests import np_restatement as nps
        w = nps.dequantize(int(fmt), q, rows, cols).astype(np.float64)
        mag = np.abs(w) @ np.abs(np.asarray(x, np.float64))
        assert np.all(err <= 2.0 ** -18 * mag + 1e-30)


def _case(fmt, rows, cols, seed):
    m = orc.seeded_f32s(rows * cols, seed ^ 0xA5A5_5A5A_1234_5678)
    x = orc.seeded_f32s(cols, seed ^ 0xD00D_F00D_1234_5678)
    q = orc.quantize_matrix(int(fmt), m, rows, cols)
    return m, x, q


# q4/q5/iq3 correctness_and_seed_sweep and test_fp4_cuda_vs_cpu (quant.rs:1715-1770,1831-1857,1911-1937)
@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("rows,cols", [(1, 32), (16, 32), (128, 256), (1024, 4096)])
@pytest.mark.parametrize("seed", [0, 1, 2, 3, 4, 123])
def test_gemv_reference_sweep(quant, fmt, rows, cols, seed):
    m, x, q = _case(fmt, rows, cols, seed)
    shape = QGemvShape.new(fmt, rows, cols)
    y, tel = quant.gemv(fmt, None, q, x, shape)
    ref = orc.gemv(int(fmt), q, x, rows, cols)
    _assert_close(y, ref, q, x, fmt, rows, cols)
    # the reference's own thresholds (device vs CPU-quantized reference cosine)
    thr = {0: 0.990, 1: 0.995, 2: 0.970, 3: 0.9999}[int(fmt)]
    assert orc.compare(ref, y)["cosine_similarity"] > thr
    assert tel["bytes_read"] == shape.quantized_matrix_bytes() + 4 * cols
    assert tel["kernel_ms"] >= 0.0 and tel["total_ms"] >= tel["kernel_ms"]


@pytest.mark.parametrize("fmt", FORMATS[:3])
@pytest.mark.parametrize("rows,cols", [(768, 2048), (2048, 768), (37, 4096), (5, 64), (64, 1024), (300, 192)])
def test_gemv_fast_path_shapes(quant, fmt, rows, cols):
    m = orc.gauss(rows * cols, rows * 7 + cols, 0.02)
    x = orc.gauss(cols, 3, 1.0)
    q = orc.quantize_matrix(int(fmt), m, rows, cols)
    y, _ = quant.gemv(fmt, None, q, x, QGemvShape.new(fmt, rows, cols))
    _assert_close(y, orc.gemv(int(fmt), q, x, rows, cols), q, x, fmt, rows, cols)


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("batch", [1, 2, 3, 5, 8, 11])
def test_gemv_device_batched(backend, quant, fmt, batch):
    rows, cols = 200, 512
    m = orc.gauss(rows * cols, 17, 0.02)
    q = orc.quantize_matrix(int(fmt), m, rows, cols)
    xs = orc.gauss(batch * cols, 18, 1.0)
    dq = backend.to_device(q)
    dx = backend.to_device(xs)
    dy = backend.alloc(batch * rows * 4)
    quant.launch_kernel(fmt, None, dq, dx, dy, QGemvShape.new(fmt, rows, cols), batch=batch)
    y = dy.download(np.float32, batch * rows).reshape(batch, rows)
    for t in range(batch):
        xt = xs[t * cols:(t + 1) * cols]
        _assert_close(y[t], orc.gemv(int(fmt), q, xt, rows, cols), q, xt, fmt, rows, cols)


def test_gemv_unaligned_weights_take_generic_path(backend, quant):
    rows, cols = 64, 256
    fmt = QuantFormat.Q4_0
    m = orc.gauss(rows * cols, 9, 0.02)
    x = orc.gauss(cols, 10, 1.0)
    q = orc.quantize_matrix(0, m, rows, cols)
    buf = backend.alloc(q.size + 16)
    buf.upload(q, offset=2)  # 2-byte aligned weights
    dx = backend.to_device(x)
    dy = backend.alloc(rows * 4)
    quant.launch_kernel(fmt, None, buf.addr(2), dx, dy, QGemvShape.new(fmt, rows, cols))
    _assert_close(dy.download(np.float32, rows), orc.gemv(0, q, x, rows, cols), q, x, fmt, rows, cols)


@pytest.mark.parametrize("cols", [64, 32])
def test_every_f16_scale_through_q4_gemv(backend, quant, cols):
    """All 65,536 f16 scale bit patterns decoded by the GEMV kernels (fast path at
    cols=64, generic at cols=32): every block has q-8 = 1 on lane 0, x = e_0."""
    rows = 65536 if cols == 32 else 32768
    nb = cols // 32
    blocks = np.zeros((rows * nb, 18), np.uint8)
    blocks[:, 2:] = 0x88
    blocks[:, 2] = 0x89  # lane 0 -> q = 9 -> value 1
    scales = np.arange(rows * nb, dtype=np.uint32).astype(np.uint16)
    blocks[:, 0] = scales & 0xFF
    blocks[:, 1] = scales >> 8
    x = np.zeros(cols, np.float32)
    x[0] = 1.0
    if nb == 2:
        x[32] = 1.0
    q = blocks.ravel()
    y, _ = quant.gemv(QuantFormat.Q4_0, None, q, x, QGemvShape.new(QuantFormat.Q4_0, rows, cols))
    ref = orc.gemv(0, q, x, rows, cols)
    finite = np.isfinite(ref)
    assert np.array_equal(y[finite], ref[finite])
    assert np.array_equal(np.isnan(y), np.isnan(ref))
    assert np.array_equal(y[np.isinf(ref)], ref[np.isinf(ref)])


@pytest.mark.parametrize("rows,cols", [(64, 256), (2048, 7168), (7168, 2048), (33, 96)])
@pytest.mark.parametrize("batch", [1, 4])
def test_fp4_split_gemv(backend, quant, rows, cols, batch):
    rng = np.random.default_rng(rows + cols)
    w = rng.integers(0, 256, size=rows * cols // 2, dtype=np.uint8)
    s = rng.integers(119, 128, size=rows * cols // 32, dtype=np.uint8)
    xs = orc.gauss(batch * cols, 4, 1.0)
    dw, ds, dx = backend.to_device(w), backend.to_device(s), backend.to_device(xs)
    dy = backend.alloc(batch * rows * 4)
    quant.launch_kernel_split_fp4(None, dw, ds, dx, dy, rows, cols, batch=batch)
    y = dy.download(np.float32, batch * rows).reshape(batch, rows)
    check_rows = np.arange(rows) if rows <= 2048 else np.arange(0, rows, 7)
    for t in range(batch):
        xt = xs[t * cols:(t + 1) * cols]
        ws_ = w.reshape(rows, cols // 2)[check_rows].ravel()
        ss_ = s.reshape(rows, cols // 32)[check_rows].ravel()
        ref = orc.fp4_split_gemv(ws_, ss_, xt, len(check_rows), cols)
        scale = float(np.max(np.abs(ref)))
        assert float(np.max(np.abs(y[t][check_rows] - ref))) <= 1e-4 * scale


def test_fp4_interleaved_vs_split_on_reference_test_data(backend, quant):
    # the reference's test_native_fp4 data path: fp4_quantize_matrix_cpu then split
    rows, cols = 512, 256
    m = orc.seeded_f32s(rows * cols, 42 ^ 0x1111)
    inter = orc.quantize_matrix(orc.FP4, m, rows, cols)
    w, s = orc.split_interleaved_fp4(inter, rows, cols)
    x = orc.seeded_f32s(cols, 42 ^ 0xDEADBEEF)
    y_int, _ = quant.gemv(QuantFormat.DeepSeekFp4E2M1, None, inter, x,
                          QGemvShape.new(QuantFormat.DeepSeekFp4E2M1, rows, cols))
    dw, ds, dx = backend.to_device(w), backend.to_device(s), backend.to_device(x)
    dy = backend.alloc(rows * 4)
    quant.launch_kernel_split_fp4(None, dw, ds, dx, dy, rows, cols)
    y_split = dy.download(np.float32, rows)
    ref = orc.fp4_split_gemv(w, s, x, rows, cols)
    scale = float(np.max(np.abs(ref)))
    assert float(np.max(np.abs(y_int - ref))) <= 1e-4 * scale
    assert float(np.max(np.abs(y_split - ref))) <= 1e-4 * scale


def test_gemv_validation_messages(quant):
    from objeta_amd import HipError
    shape = QGemvShape.new(QuantFormat.Q4_0, 4, 33)
    with pytest.raises(HipError) as e:
        quant.gemv(QuantFormat.Q4_0, None, np.zeros(10, np.uint8), np.zeros(33, np.float32), shape)
    assert e.value.kind == "InvalidInput" and "multiple of block_size" in e.value.source_message
    shape = QGemvShape.new(QuantFormat.Q4_0, 4, 64)
    with pytest.raises(HipError) as e:
        quant.gemv(QuantFormat.Q4_0, None, np.zeros(10, np.uint8), np.zeros(64, np.float32), shape)
    assert "qweights len 10 != expected 144" in e.value.source_message
    with pytest.raises(HipError) as e:
        quant.gemv(QuantFormat.Q4_0, None, np.zeros(144, np.uint8), np.zeros(63, np.float32), shape)
    assert "x len 63 != cols 64" in e.value.source_message


@pytest.mark.parametrize("fmt", FORMATS[:3])
def test_gemv_full_size_linearity(backend, quant, fmt):
    """[14336 x 4096]: linearity in x, and exact parity on a sample of rows."""
    rows, cols = 14336, 4096
    L = backend.L
    dq = backend.alloc(rows * cols // 32 * fmt.block_bytes())
    from objeta_amd import check
    check(L.objeta_hip_fill_gauss_quantized_device(backend.ctx, int(fmt), None, dq.addr(), rows, cols, 777, C.c_float(0.02)))
    x1 = orc.gauss(cols, 1, 1.0)
    x2 = orc.gauss(cols, 2, 1.0)
    xs = np.concatenate([x1, x2, (np.float32(0.5) * x1 + np.float32(2.0) * x2).astype(np.float32)])
    dx = backend.to_device(xs)
    dy = backend.alloc(3 * rows * 4)
    quant.launch_kernel(fmt, None, dq, dx, dy, QGemvShape.new(fmt, rows, cols), batch=3)
    y = dy.download(np.float32, 3 * rows).reshape(3, rows).astype(np.float64)
    lin = 0.5 * y[0] + 2.0 * y[1]
    assert float(np.max(np.abs(y[2] - lin))) <= 1e-4 * float(np.max(np.abs(y[2])))
    sample = np.arange(0, rows, 97)
    rb = cols // 32 * fmt.block_bytes()
    qall = dq.download(np.uint8, rows * rb).reshape(rows, rb)
    ref = orc.gemv(int(fmt), qall[sample].ravel(), x1, len(sample), cols)
    assert float(np.max(np.abs(y[0][sample] - ref))) <= 1e-4 * float(np.max(np.abs(ref)))


# ---------------------------------------------------- batched GEMV on the matrix cores
@pytest.mark.parametrize("fmt", FORMATS[:3])
@pytest.mark.parametrize("rows,cols,batch", [(200, 704, 6), (37, 1536, 9), (1000, 64, 5)])
def test_gemv_batched_mfma_column_ranges(backend, quant, fmt, rows, cols, batch):
    """From five vectors the batched GEMV runs on MFMA, each workgroup over a range of
    512 columns (the last one partial here) whose partial sums are added in range
    order; every vector is checked against the oracle with the tight bound."""
    m = orc.gauss(rows * cols, 40 + rows, 0.02)
    q = orc.quantize_matrix(int(fmt), m, rows, cols)
    xs = orc.gauss(batch * cols, 41 + cols, 1.0)
    dy = backend.alloc(batch * rows * 4)
    quant.launch_kernel(fmt, None, backend.to_device(q), backend.to_device(xs), dy, QGemvShape.new(fmt, rows, cols),
                        batch=batch)
    y = dy.download(np.float32, batch * rows).reshape(batch, rows)
    for t in range(batch):
        xt = xs[t * cols:(t + 1) * cols]
        _assert_close(y[t], orc.gemv(int(fmt), q, xt, rows, cols), q, xt, fmt, rows, cols)


@pytest.mark.parametrize("fmt", FORMATS[:3])
@pytest.mark.parametrize("cols", [4096, 4160])
def test_gemv_batched_mfma_wide_tiles(backend, quant, fmt, cols):
    """8200 rows over 8 or 9 column ranges give enough workgroups for 128-row tiles
    (8 slabs per workgroup, the last tile 8 rows deep) for Q4_0 and Q5_0; IQ3_0 keeps
    64-row tiles: 16-byte weight units when every range is full (4096 columns), dword
    units with a 64-column last range (4160)."""
    rows, batch = 8200, 8
    m = orc.gauss(rows * cols, 50 + cols, 0.02)
    q = orc.quantize_matrix(int(fmt), m, rows, cols)
    xs = orc.gauss(batch * cols, 51 + cols, 1.0)
    dy = backend.alloc(batch * rows * 4)
    quant.launch_kernel(fmt, None, backend.to_device(q), backend.to_device(xs), dy, QGemvShape.new(fmt, rows, cols),
                        batch=batch)
    y = dy.download(np.float32, batch * rows).reshape(batch, rows)
    for t in range(batch):
        xt = xs[t * cols:(t + 1) * cols]
        _assert_close(y[t], orc.gemv(int(fmt), q, xt, rows, cols), q, xt, fmt, rows, cols)


@pytest.mark.parametrize("rows,cols,batch", [(100, 640, 5), (48, 1024, 8), (8200, 4096, 8), (8200, 4224, 7)])
def test_fp4_split_gemv_batched_mfma(backend, quant, rows, cols, batch):
    rng = np.random.default_rng(rows * cols)
    w = rng.integers(0, 256, size=rows * cols // 2, dtype=np.uint8)
    s = rng.integers(112, 132, size=rows * cols // 32, dtype=np.uint8)
    xs = orc.gauss(batch * cols, 6, 1.0)
    dy = backend.alloc(batch * rows * 4)
    quant.launch_kernel_split_fp4(None, backend.to_device(w), backend.to_device(s), backend.to_device(xs), dy, rows,
                                  cols, batch=batch)
    y = dy.download(np.float32, batch * rows).reshape(batch, rows)
    for t in range(batch):
        ref = orc.fp4_split_gemv(w, s, xs[t * cols:(t + 1) * cols], rows, cols)
        assert float(np.max(np.abs(y[t] - ref))) <= 1e-4 * float(np.max(np.abs(ref)))


def test_gemv_batched_mfma_non_finite_scales(backend, quant):
    """Rows with an inf or NaN block scale give non-finite outputs on the MFMA path as
    in the reference (not necessarily the same special value: the block sum is
    scaled once); the other rows stay within the bar."""
    fmt, rows, cols, batch = QuantFormat.Q4_0, 64, 1024, 8
    q = orc.quantize_matrix(0, orc.gauss(rows * cols, 7, 0.02), rows, cols).reshape(rows, cols // 32, 18).copy()
    q[5, 3, :2] = np.array([0x7C00], np.uint16).view(np.uint8)   # +inf scale
    q[17, 30, :2] = np.array([0x7E00], np.uint16).view(np.uint8)  # NaN scale
    q = q.ravel()
    xs = orc.gauss(batch * cols, 8, 1.0)
    dy = backend.alloc(batch * rows * 4)
    quant.launch_kernel(fmt, None, backend.to_device(q), backend.to_device(xs), dy, QGemvShape.new(fmt, rows, cols),
                        batch=batch)
    y = dy.download(np.float32, batch * rows).reshape(batch, rows)
    for t in range(batch):
        ref = orc.gemv(0, q, xs[t * cols:(t + 1) * cols], rows, cols)
        bad = ~np.isfinite(ref)
        assert bad[5] and bad[17]
        assert np.array_equal(~np.isfinite(y[t]), bad)
        scale = float(np.max(np.abs(ref[~bad])))
        assert float(np.max(np.abs(y[t][~bad] - ref[~bad]))) <= 1e-4 * scale
