"""Python mirror of the reference's objeta-cuda API over the C ABI.

Names, argument meaning and error behaviour follow crates/objeta-cuda/src:
QuantFormat / QGemvShape (quant.rs:25-143), CudaError (lib.rs:50-79),
CudaBackendBuilder / CudaBackend (context.rs:37-165), CudaStreamPool
(stream.rs:9-51), QuantBackend (quant.rs:192-408). Every call goes through
libobjeta_hip.so; nothing here computes on the CPU.
"""
from __future__ import annotations

import ctypes as C
import enum
from dataclasses import dataclass

import numpy as np

from . import _lib
from ._lib import DeviceInfo, Error, ExpertPtrs, InitOptions, QGemvTelemetry

KIND_NAMES = ["Driver", "Runtime", "Nvrtc", "Io", "InvalidInput", "Unsupported", "Internal"]


class HipError(Exception):
    """CudaError (lib.rs:50-79): kind, action, file, line, module, source_message."""

    def __init__(self, status: int, rec: Error):
        self.status = status
        self.kind = KIND_NAMES[rec.kind] if 0 <= rec.kind < len(KIND_NAMES) else "Internal"
        self.action = rec.action.decode(errors="replace")
        self.file = rec.file.decode(errors="replace")
        self.line = rec.line
        self.module = rec.module.decode(errors="replace")
        self.source_message = rec.source_message.decode(errors="replace")
        super().__init__(f"{self.kind} error during {self.action} at {self.module}:{self.line} "
                         f"({self.file}): {self.source_message}")


def check(status: int) -> None:
    if status != 0:
        rec = Error()
        _lib.load().objeta_hip_last_error(C.byref(rec))
        raise HipError(status, rec)


class QuantFormat(enum.IntEnum):
    """QuantFormat (quant.rs:25-96)."""
    Q4_0 = 0
    Q5_0 = 1
    IQ3_0 = 2
    DeepSeekFp4E2M1 = 3

    def block_size(self) -> int:
        return 32

    def block_bytes(self) -> int:
        return {0: 18, 1: 22, 2: 14, 3: 17}[int(self)]

    def kernel_name(self) -> str:
        return {0: "q4_gemv", 1: "q5_gemv", 2: "iq3_gemv", 3: "fp4_e2m1_gemv"}[int(self)]

    def format_label(self) -> str:
        return {0: "q4_0", 1: "q5_0", 2: "iq3_0", 3: "deepseek_fp4_e2m1"}[int(self)]

    def scale_dtype(self) -> str:
        return "F8_E8M0" if self == QuantFormat.DeepSeekFp4E2M1 else "F16"


@dataclass(frozen=True)
class QGemvShape:
    """QGemvShape (quant.rs:98-143)."""
    rows: int
    cols: int
    block_size: int = 32
    block_bytes: int = 18

    @staticmethod
    def new(fmt: QuantFormat, rows: int, cols: int) -> "QGemvShape":
        fmt = QuantFormat(fmt)
        return QGemvShape(rows, cols, fmt.block_size(), fmt.block_bytes())

    def blocks_per_row(self) -> int:
        return self.cols // self.block_size

    def quantized_row_bytes(self) -> int:
        return self.blocks_per_row() * self.block_bytes

    def quantized_matrix_bytes(self) -> int:
        return self.rows * self.quantized_row_bytes()


def discover_devices() -> list:
    """CudaBackend::discover_devices (context.rs:73-104)."""
    L = _lib.load()
    n = C.c_int32(0)
    check(L.objeta_hip_device_count(C.byref(n)))
    out = []
    for i in range(n.value):
        info = DeviceInfo()
        check(L.objeta_hip_discover_device(i, C.byref(info)))
        out.append(_info_dict(info))
    return out


def _info_dict(info: DeviceInfo) -> dict:
    d = {k: getattr(info, k) for k, _ in DeviceInfo._fields_ if k != "reserved"}
    d["name"] = info.name.decode()
    d["arch"] = info.arch.decode()
    return d


class DeviceBuffer:
    """Device allocation owned by the backend (memory.rs:8-28)."""

    def __init__(self, backend: "HipBackend", nbytes: int):
        self.backend = backend
        self.nbytes = int(nbytes)
        p = C.c_void_p()
        check(backend.L.objeta_hip_malloc(backend.ctx, self.nbytes, C.byref(p)))
        self.ptr = p.value or 0

    def free(self):
        if self.ptr:
            check(self.backend.L.objeta_hip_free(self.backend.ctx, C.c_void_p(self.ptr)))
            self.ptr = 0

    def __del__(self):
        try:
            if self.ptr and self.backend.ctx:
                self.backend.L.objeta_hip_free(self.backend.ctx, C.c_void_p(self.ptr))
        except Exception:
            pass

    def addr(self, offset: int = 0):
        return C.c_void_p(self.ptr + offset)

    def upload(self, arr: np.ndarray, stream=None, offset: int = 0) -> "DeviceBuffer":
        a = np.ascontiguousarray(arr)
        assert offset + a.nbytes <= self.nbytes, "upload exceeds buffer"
        check(self.backend.L.objeta_hip_copy_h2d(self.backend.ctx, stream, self.addr(offset),
                                                 a.ctypes.data_as(C.c_void_p), a.nbytes))
        self.backend.synchronize(stream)
        return self

    def download(self, dtype, count: int, stream=None, offset: int = 0) -> np.ndarray:
        out = np.empty(count, dtype=dtype)
        assert offset + out.nbytes <= self.nbytes, "download exceeds buffer"
        check(self.backend.L.objeta_hip_copy_d2h(self.backend.ctx, stream,
                                                 out.ctypes.data_as(C.c_void_p), self.addr(offset),
                                                 out.nbytes))
        self.backend.synchronize(stream)
        return out


class HipBackend:
    """CudaBackend (context.rs:72-165): one device, a pool of streams."""

    def __init__(self, device_ordinal: int = 0, stream_count: int = 1):
        self.L = _lib.load()
        opts = InitOptions(device_ordinal, max(1, stream_count))
        ctx = C.c_void_p()
        check(self.L.objeta_hip_init(C.byref(opts), C.byref(ctx)))
        self.ctx = ctx
        info = DeviceInfo()
        check(self.L.objeta_hip_device_info_get(self.ctx, C.byref(info)))
        self.device_info = _info_dict(info)
        self.streams = []
        for i in range(max(1, stream_count)):
            s = C.c_void_p()
            check(self.L.objeta_hip_stream_get(self.ctx, i, C.byref(s)))
            self.streams.append(s)

    def stream(self, index: int = 0):
        if index >= len(self.streams):
            s = C.c_void_p()
            check(self.L.objeta_hip_stream_get(self.ctx, index, C.byref(s)))
        return self.streams[index]

    def synchronize(self, stream=None) -> None:
        check(self.L.objeta_hip_stream_synchronize(self.ctx, stream))

    def alloc(self, nbytes: int) -> DeviceBuffer:
        return DeviceBuffer(self, nbytes)

    def to_device(self, arr: np.ndarray, stream=None) -> DeviceBuffer:
        a = np.ascontiguousarray(arr)
        return DeviceBuffer(self, max(a.nbytes, 4)).upload(a, stream)

    def close(self) -> None:
        if self.ctx:
            check(self.L.objeta_hip_destroy(self.ctx))
            self.ctx = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


class HipBackendBuilder:
    """CudaBackendBuilder (context.rs:37-70)."""

    def __init__(self):
        self._ordinal = 0
        self._streams = 1

    def device_ordinal(self, n: int) -> "HipBackendBuilder":
        self._ordinal = n
        return self

    def stream_count(self, n: int) -> "HipBackendBuilder":
        self._streams = max(1, n)
        return self

    def build(self) -> HipBackend:
        return HipBackend(self._ordinal, self._streams)


def _telemetry_dict(t: QGemvTelemetry) -> dict:
    return {k: getattr(t, k) for k, _ in QGemvTelemetry._fields_}


class QuantBackend:
    """QuantBackend (quant.rs:192-408). Kernels are compiled ahead of time, so
    compile_format only validates the format."""

    def __init__(self, backend: HipBackend):
        self.backend = backend
        self.L = backend.L

    def compile_format(self, fmt) -> None:
        QuantFormat(fmt)

    def quantize_matrix(self, fmt, matrix: np.ndarray, shape: QGemvShape) -> np.ndarray:
        """quantize_matrix (quant.rs:239-246), evaluated by the device quantizer."""
        fmt = QuantFormat(fmt)
        m = np.ascontiguousarray(matrix, dtype=np.float32).ravel()
        if m.size != shape.rows * shape.cols:
            raise ValueError(f"matrix len {m.size} != rows*cols {shape.rows * shape.cols}")
        nbytes = int(self.L.objeta_hip_quantized_matrix_bytes(int(fmt), shape.rows, shape.cols))
        if nbytes < 0:
            raise ValueError(f"cols {shape.cols} must be a multiple of block_size 32")
        dm = self.backend.to_device(m)
        dq = self.backend.alloc(max(nbytes, 4))
        check(self.L.objeta_hip_quantize_matrix_device(self.backend.ctx, int(fmt), None, dm.addr(),
                                                       shape.rows, shape.cols, dq.addr()))
        return dq.download(np.uint8, nbytes)

    def gemv(self, fmt, stream, qweights: np.ndarray, x: np.ndarray, shape: QGemvShape):
        """QuantBackend::gemv (quant.rs:256-302): returns (y, telemetry)."""
        q = np.ascontiguousarray(qweights, dtype=np.uint8).ravel()
        xv = np.ascontiguousarray(x, dtype=np.float32).ravel()
        y = np.zeros(max(shape.rows, 1), np.float32)
        tel = QGemvTelemetry()
        check(self.L.objeta_hip_qgemv(self.backend.ctx, int(QuantFormat(fmt)), stream,
                                      q.ctypes.data_as(C.c_void_p), q.size,
                                      xv.ctypes.data_as(C.c_void_p), xv.size, shape.rows, shape.cols,
                                      y.ctypes.data_as(C.c_void_p), C.byref(tel)))
        return y[:shape.rows], _telemetry_dict(tel)

    def q4_gemv(self, stream, qweights, x, shape):
        return self.gemv(QuantFormat.Q4_0, stream, qweights, x, shape)

    def q5_gemv(self, stream, qweights, x, shape):
        return self.gemv(QuantFormat.Q5_0, stream, qweights, x, shape)

    def launch_kernel(self, fmt, stream, d_q, d_x, d_y, shape: QGemvShape, batch: int = 1) -> None:
        """QuantBackend::launch_kernel (quant.rs:324-366); device pointers, `batch` vectors."""
        check(self.L.objeta_hip_qgemv_device(self.backend.ctx, int(QuantFormat(fmt)), stream,
                                             _addr(d_q), _addr(d_x), _addr(d_y), shape.rows,
                                             shape.cols, batch))

    def launch_kernel_split_fp4(self, stream, d_w, d_s, d_x, d_y, rows: int, cols: int,
                                batch: int = 1) -> None:
        """QuantBackend::launch_kernel_split_fp4 (quant.rs:368-408)."""
        check(self.L.objeta_hip_fp4_gemv_split_device(self.backend.ctx, stream, _addr(d_w), _addr(d_s),
                                                      _addr(d_x), _addr(d_y), rows, cols, batch))


def _addr(v):
    if isinstance(v, DeviceBuffer):
        return v.addr()
    if isinstance(v, int):
        return C.c_void_p(v)
    return v


class ExpertTable:
    """Device array of objeta_hip_expert_ptrs: one entry per expert, pointing at
    device-resident gate/up/down matrices (and E8M0 scales for split FP4)."""

    def __init__(self, backend: HipBackend, entries):
        """entries: list of (gate, up, down) or (gate, up, down, gate_s, up_s, down_s)
        device addresses (ints or DeviceBuffers)."""
        self.backend = backend
        self.n = len(entries)
        arr = (ExpertPtrs * max(1, self.n))()
        for i, e in enumerate(entries):
            v = [_ptr_int(p) for p in e] + [0] * (6 - len(e))
            arr[i] = ExpertPtrs(*v)
        raw = np.frombuffer(bytes(arr), dtype=np.uint8)
        self.buf = backend.to_device(raw)

    def addr(self):
        return self.buf.addr()


def _ptr_int(p) -> int:
    if isinstance(p, DeviceBuffer):
        return p.ptr
    if isinstance(p, C.c_void_p):
        return p.value or 0
    return int(p or 0)


class MoeExecutor:
    """MoeExecutor (moe.rs:285-1280): the selected-expert MoE on the device."""

    def __init__(self, backend: HipBackend):
        self.backend = backend
        self.L = backend.L

    def compile(self) -> None:
        """Kernels are compiled ahead of time (moe.rs:304-307 compiles NVRTC modules)."""

    def selected_device(self, fmt, table: ExpertTable, d_ids, d_weights, n_tokens: int, k: int, d_x,
                        d_residual, d_out, hidden: int, inter: int, out_dim: int,
                        swiglu_limit: float = 0.0, stream=None) -> None:
        check(self.L.objeta_hip_moe_selected_device(
            self.backend.ctx, int(fmt), stream, table.addr(), table.n, _addr_or_none(d_ids),
            _addr(d_weights), n_tokens, k, _addr(d_x), _addr_or_none(d_residual), _addr(d_out), hidden,
            inter, out_dim, swiglu_limit))

    def layer_device(self, fmt, table: ExpertTable, d_router_w, d_router_bias, k: int, n_tokens: int,
                     d_x, d_residual, d_out, d_ids_out, d_weights_out, hidden: int, inter: int,
                     out_dim: int, renormalize: bool = True, swiglu_limit: float = 0.0,
                     stream=None) -> None:
        check(self.L.objeta_hip_moe_layer_device(
            self.backend.ctx, int(fmt), stream, table.addr(), table.n, _addr(d_router_w),
            _addr_or_none(d_router_bias), k, 1 if renormalize else 0, n_tokens, _addr(d_x),
            _addr_or_none(d_residual), _addr(d_out), _addr(d_ids_out), _addr(d_weights_out), hidden,
            inter, out_dim, swiglu_limit))

    def device_error(self) -> int:
        v = C.c_uint32(0)
        check(self.L.objeta_hip_device_error(self.backend.ctx, C.byref(v)))
        return v.value


def _addr_or_none(v):
    return None if v is None else _addr(v)
