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
from ._lib import (CacheKey, CacheStats, DeviceInfo, Error, ExpertPtrs, HostExpert, InitOptions, MoeTelemetry,
                   QGemvTelemetry)

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


class PinnedHostBuffer:
    """PinnedHostBuffer (memory.rs:31-80): page-locked host memory of the backend's
    device, so that copies from it run asynchronously at PCIe rate. `array(dtype)`
    views it as a numpy array; free it (or let it be collected) before the backend
    closes."""

    def __init__(self, backend: "HipBackend", nbytes: int):
        self.backend = backend
        self.nbytes = int(nbytes)
        p = C.c_void_p()
        check(backend.L.objeta_hip_alloc_pinned_host(backend.ctx, self.nbytes, C.byref(p)))
        self.ptr = p.value or 0

    def array(self, dtype=np.uint8, count: int | None = None, offset: int = 0) -> np.ndarray:
        dt = np.dtype(dtype)
        n = (self.nbytes - offset) // dt.itemsize if count is None else int(count)
        assert offset + n * dt.itemsize <= self.nbytes
        buf = (C.c_uint8 * (n * dt.itemsize)).from_address(self.ptr + offset)
        return np.frombuffer(buf, dtype=dt, count=n)

    def free(self) -> None:
        if self.ptr and self.backend.ctx:
            check(self.backend.L.objeta_hip_free_pinned_host(self.backend.ctx, C.c_void_p(self.ptr)))
        self.ptr = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


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

    # ---- FP8-activation ("official arithmetic") kernels
    def act_quant_device(self, stream, d_x, rows: int, cols: int, d_values=None, d_scales=None,
                         d_dequant=None) -> None:
        """cuda_act_quant_device (quant.rs:1229-1281) with cpu_act_quant's bytes: FP8 E4M3
        values [rows][cols], E8M0 scales [rows][cols/128], optionally the dequantized floats."""
        check(self.L.objeta_hip_act_quant_fp8_device(self.backend.ctx, stream, _addr(d_x), rows, cols,
                                                     _addr_or_none(d_values), _addr_or_none(d_scales),
                                                     _addr_or_none(d_dequant)))

    def act_quant(self, stream, x: np.ndarray, rows: int, cols: int):
        """cuda_act_quant (quant.rs:1119-1216): host floats in, (values, scales) bytes out."""
        xv = np.ascontiguousarray(x, dtype=np.float32).ravel()
        if cols % 128 != 0:
            raise ValueError(f"cuda_act_quant: cols {cols} not divisible by 128")
        if xv.size != rows * cols:
            raise ValueError(f"cuda_act_quant: input len {xv.size} != rows {rows} * cols {cols}")
        dx = self.backend.to_device(xv)
        dv, ds = self.backend.alloc(max(1, rows * cols)), self.backend.alloc(max(1, rows * cols // 128))
        self.act_quant_device(stream, dx, rows, cols, dv, ds)
        return dv.download(np.uint8, rows * cols, stream), ds.download(np.uint8, rows * cols // 128, stream)

    def fp8_act_fp4_weight_gemv_device(self, stream, d_act_values, d_act_scales, d_weight, d_weight_scales,
                                       d_out, rows: int, k_logical: int, batch: int = 1) -> None:
        """cuda_fp8_act_fp4_weight_gemv_device (quant.rs:1284-1325), `batch` activation vectors."""
        check(self.L.objeta_hip_fp8_act_fp4_weight_gemv_device(
            self.backend.ctx, stream, _addr(d_act_values), _addr(d_act_scales), _addr(d_weight),
            _addr(d_weight_scales), _addr(d_out), rows, k_logical, batch))

    def fp8_act_fp8_weight_gemv_device(self, stream, d_act_values, d_act_scales, d_weight, d_weight_scales,
                                       d_out, rows: int, k_logical: int, batch: int = 1) -> None:
        """cuda_fp8_act_fp8_weight_gemv_device (quant.rs:1328-1362): FP8 weights, 128 x 128 scale tiles."""
        check(self.L.objeta_hip_fp8_act_fp8_weight_gemv_device(
            self.backend.ctx, stream, _addr(d_act_values), _addr(d_act_scales), _addr(d_weight),
            _addr(d_weight_scales), _addr(d_out), rows, k_logical, batch))


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
                        swiglu_limit: float = 0.0, stream=None, shared: "ExpertTable | None" = None) -> None:
        """shared: a one-entry ExpertTable applied to every token with weight 1.0 after
        the routed sum (moe.rs:1552-1600)."""
        check(self.L.objeta_hip_moe_selected_shared_device(
            self.backend.ctx, int(fmt), stream, table.addr(), table.n, None if shared is None else shared.addr(),
            _addr_or_none(d_ids), _addr(d_weights), n_tokens, k, _addr(d_x), _addr_or_none(d_residual),
            _addr(d_out), hidden, inter, out_dim, swiglu_limit))

    def grouped_device(self, fmt, table: ExpertTable, d_ids, d_weights, n_tokens: int, k: int, d_x,
                       d_residual, d_out, hidden: int, inter: int, out_dim: int,
                       swiglu_limit: float = 0.0, stream=None) -> None:
        """selected_device for a batch: assignments grouped by expert, each expert's
        matrices read once for all its tokens, products on the matrix cores."""
        check(self.L.objeta_hip_moe_grouped_device(
            self.backend.ctx, int(fmt), stream, table.addr(), table.n, _addr(d_ids), _addr(d_weights), n_tokens,
            k, _addr(d_x), _addr_or_none(d_residual), _addr(d_out), hidden, inter, out_dim, swiglu_limit))

    def gate_up_device(self, fmt, table: ExpertTable, d_ids, n_tokens: int, k: int, d_x, d_act,
                       hidden: int, inter: int, swiglu_limit: float = 0.0, stream=None) -> None:
        """The fused gate/up + SiLU phase alone: act[t*k + j] = silu(gate_e x_t) * up_e x_t."""
        check(self.L.objeta_hip_moe_gate_up_device(
            self.backend.ctx, int(fmt), stream, table.addr(), table.n, _addr_or_none(d_ids), n_tokens, k,
            _addr(d_x), _addr(d_act), hidden, inter, swiglu_limit))

    def down_device(self, fmt, table: ExpertTable, d_ids, d_weights, n_tokens: int, k: int, d_act,
                    d_residual, d_out, inter: int, out_dim: int, stream=None) -> None:
        """The down + weighted-combine phase alone: out = residual + sum_j w_j down_e act_j."""
        check(self.L.objeta_hip_moe_down_device(
            self.backend.ctx, int(fmt), stream, table.addr(), table.n, _addr_or_none(d_ids), _addr(d_weights),
            n_tokens, k, _addr(d_act), _addr_or_none(d_residual), _addr(d_out), inter, out_dim))

    def layer_device(self, fmt, table: ExpertTable, d_router_w, d_router_bias, k: int, n_tokens: int,
                     d_x, d_residual, d_out, d_ids_out, d_weights_out, hidden: int, inter: int,
                     out_dim: int, renormalize: bool = True, swiglu_limit: float = 0.0,
                     stream=None, shared: "ExpertTable | None" = None) -> None:
        check(self.L.objeta_hip_moe_layer_shared_device(
            self.backend.ctx, int(fmt), stream, table.addr(), table.n, None if shared is None else shared.addr(),
            _addr(d_router_w), _addr_or_none(d_router_bias), k, 1 if renormalize else 0, n_tokens, _addr(d_x),
            _addr_or_none(d_residual), _addr(d_out), _addr(d_ids_out), _addr(d_weights_out), hidden,
            inter, out_dim, swiglu_limit))

    def official_fp4_device(self, table: ExpertTable, d_ids, d_weights, n_tokens: int, k: int, d_x, d_out,
                            hidden: int, inter: int, out_dim: int, swiglu_limit: float = 10.0, stream=None,
                            shared_fp8: "ExpertTable | None" = None, d_inter_values=None,
                            d_inter_scales=None) -> None:
        """The device part of execute_selected_moe_official_routed_fp4_cuda (moe.rs:1393-1663),
        batched over tokens: FP8 activations, FP4 split routed experts, an optional FP8
        shared expert (a one-entry ExpertTable with 128 x 128 scale tiles)."""
        check(self.L.objeta_hip_moe_official_fp4_device(
            self.backend.ctx, stream, table.addr(), table.n, None if shared_fp8 is None else shared_fp8.addr(),
            _addr(d_ids), _addr(d_weights), n_tokens, k, _addr(d_x), _addr(d_out), hidden, inter, out_dim,
            swiglu_limit, _addr_or_none(d_inter_values), _addr_or_none(d_inter_scales)))

    def device_error(self) -> int:
        v = C.c_uint32(0)
        check(self.L.objeta_hip_device_error(self.backend.ctx, C.byref(v)))
        return v.value


def _addr_or_none(v):
    return None if v is None else _addr(v)


class ExpertTensorKind(enum.IntEnum):
    """ExpertTensorKind (moe.rs:37-54)."""
    Gate = 0
    Up = 1
    Down = 2
    GateWeight = 3
    GateScale = 4
    UpWeight = 5
    UpScale = 6
    DownWeight = 7
    DownScale = 8
    SharedGateWeight = 9
    SharedGateScale = 10
    SharedUpWeight = 11
    SharedUpScale = 12
    SharedDownWeight = 13
    SharedDownScale = 14


@dataclass(frozen=True)
class ExpertCacheKey:
    """ExpertCacheKey (moe.rs:56-62)."""
    layer_id: int
    expert_id: int
    tensor_kind: ExpertTensorKind
    quant_format: QuantFormat

    def c(self) -> CacheKey:
        return CacheKey(self.layer_id, self.expert_id, int(self.tensor_kind), int(self.quant_format))


_CACHE_FIELDS = [n for n, _ in CacheStats._fields_ if n not in ("reserved", "bypass_oversized_experts")]


class ExpertCache:
    """CudaExpertCache (moe.rs:70-226) over the library's cache. Counter fields are
    read-only attributes with the reference's names; `backend=None` keeps the
    accounting only (no device memory)."""

    def __init__(self, capacity_bytes: int, backend: HipBackend | None = None):
        self.backend = backend
        self.L = _lib.load()
        h = C.c_void_p()
        check(self.L.objeta_hip_cache_create(backend.ctx if backend else None, capacity_bytes, C.byref(h)))
        self.h = h

    def close(self) -> None:
        if self.h:
            check(self.L.objeta_hip_cache_destroy(self.h))
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def stats(self) -> dict:
        st = CacheStats()
        check(self.L.objeta_hip_cache_stats_get(self.h, C.byref(st)))
        d = {n: getattr(st, n) for n in _CACHE_FIELDS}
        d["bypass_oversized_experts"] = bool(st.bypass_oversized_experts)
        return d

    def __getattr__(self, name):
        if name in _CACHE_FIELDS or name == "bypass_oversized_experts":
            return self.stats()[name]
        raise AttributeError(name)

    def __setattr__(self, name, value):
        if name == "bypass_oversized_experts":
            check(self.L.objeta_hip_cache_set_bypass_oversized_experts(self.h, 1 if value else 0))
        else:
            object.__setattr__(self, name, value)

    def get(self, key: ExpertCacheKey):
        """get (moe.rs:113-122): device address on a hit, None on a miss."""
        hit, ptr, n = C.c_int32(), C.c_void_p(), C.c_uint64()
        k = key.c()
        check(self.L.objeta_hip_cache_get(self.h, C.byref(k), C.byref(hit), C.byref(ptr), C.byref(n)))
        return (ptr.value or 0) if hit.value else None

    def insert(self, key: ExpertCacheKey, data: np.ndarray, stream=None):
        """insert (moe.rs:124-158) of host bytes; returns (device address, cached)."""
        a = np.ascontiguousarray(data).view(np.uint8).ravel()
        ptr, cached = C.c_void_p(), C.c_int32()
        k = key.c()
        check(self.L.objeta_hip_cache_insert(self.h, C.byref(k), a.ctypes.data_as(C.c_void_p), a.nbytes, stream,
                                             C.byref(ptr), C.byref(cached)))
        return ptr.value or 0, bool(cached.value)

    def get_or_insert(self, key: ExpertCacheKey, data: np.ndarray, stream=None):
        """get, then insert on a miss (README.md:123); returns (address, hit, cached)."""
        a = np.ascontiguousarray(data).view(np.uint8).ravel()
        ptr, hit, cached = C.c_void_p(), C.c_int32(), C.c_int32()
        k = key.c()
        check(self.L.objeta_hip_cache_get_or_insert(self.h, C.byref(k), a.ctypes.data_as(C.c_void_p), a.nbytes,
                                                    stream, C.byref(ptr), C.byref(hit), C.byref(cached)))
        return ptr.value or 0, bool(hit.value), bool(cached.value)

    def insert_pinned(self, key: ExpertCacheKey, data: np.ndarray, stream=None) -> int:
        a = np.ascontiguousarray(data).view(np.uint8).ravel()
        ptr = C.c_void_p()
        k = key.c()
        check(self.L.objeta_hip_cache_insert_pinned(self.h, C.byref(k), a.ctypes.data_as(C.c_void_p), a.nbytes,
                                                    stream, C.byref(ptr)))
        return ptr.value or 0

    def release_transient(self, ptr: int) -> None:
        check(self.L.objeta_hip_cache_release_transient(self.h, C.c_void_p(ptr)))

    def prefetch(self, items) -> int:
        """Cross-layer prefetch: items = [(ExpertCacheKey, host array)]; starts the copies
        of the absent ones on the copy stream and returns the number started. The host
        arrays must stay alive until the copies end (pinned memory lets them overlap)."""
        items = list(items)
        n = len(items)
        keys = (CacheKey * max(1, n))()
        srcs = (C.c_void_p * max(1, n))()
        sizes = (C.c_uint64 * max(1, n))()
        for i, (k, a) in enumerate(items):
            a = np.asarray(a)
            if not a.flags.c_contiguous:
                raise ValueError("prefetch needs contiguous host arrays (they are read after the call returns)")
            keys[i] = k.c()
            srcs[i] = a.ctypes.data
            sizes[i] = a.nbytes
        issued = C.c_uint64(0)
        check(self.L.objeta_hip_cache_prefetch(self.h, keys, srcs, sizes, n, C.byref(issued)))
        return issued.value

    def preload_shared(self, shared_experts, first_layer: int = 0, stream=None):
        """The shared-expert preload (deepseek_single_layer_moe.rs:1698-1730): insert_pinned of
        every layer's six FP8 shared tensors, shared_experts = [(gate_w, gate_s, up_w, up_s,
        down_w, down_s)] per layer. Returns (bytes, ms)."""
        arr, keep = _host_experts(shared_experts)
        nbytes, ms = C.c_uint64(0), C.c_float(0)
        check(self.L.objeta_hip_cache_preload_shared(self.h, arr, len(shared_experts), first_layer, stream,
                                                     C.byref(nbytes), C.byref(ms)))
        del keep
        return nbytes.value, ms.value

    def pin(self, key: ExpertCacheKey) -> None:
        k = key.c()
        check(self.L.objeta_hip_cache_pin(self.h, C.byref(k)))

    def touch(self, key: ExpertCacheKey) -> None:
        k = key.c()
        check(self.L.objeta_hip_cache_touch(self.h, C.byref(k)))

    def evict_lru(self):
        ev, k = C.c_int32(), CacheKey()
        check(self.L.objeta_hip_cache_evict_lru(self.h, C.byref(ev), C.byref(k)))
        if not ev.value:
            return None
        return ExpertCacheKey(k.layer_id, k.expert_id, ExpertTensorKind(k.tensor_kind), QuantFormat(k.quant_format))

    def clear(self) -> None:
        check(self.L.objeta_hip_cache_clear(self.h))

    def reset_counters(self) -> None:
        check(self.L.objeta_hip_cache_reset_counters(self.h))

    def order(self) -> list:
        n = C.c_uint64()
        check(self.L.objeta_hip_cache_order(self.h, None, 0, C.byref(n)))
        arr = (CacheKey * max(1, n.value))()
        check(self.L.objeta_hip_cache_order(self.h, arr, n.value, C.byref(n)))
        return [(k.layer_id, k.expert_id, k.tensor_kind, k.quant_format) for k in arr[:n.value]]


def _telemetry_moe(t: MoeTelemetry) -> dict:
    d = {k: getattr(t, k) for k, _ in MoeTelemetry._fields_}
    d["bytes_by_tensor_kind"] = {"gate": d.pop("bytes_by_tensor_kind_gate"), "up": d.pop("bytes_by_tensor_kind_up"),
                                 "down": d.pop("bytes_by_tensor_kind_down")}
    return d


def _moe_stack_cached(self, fmt, layers, k: int, n_tokens: int, d_h, hidden: int, inter: int,
                      cache: "ExpertCache | None" = None, prefetch_next: bool = False, renormalize: bool = True,
                      d_trace=None, stream=None):
    """objeta_hip_moe_stack_cached: n_tokens tokens through len(layers) layers with the
    experts behind the cache, the hidden state d_h updated in place. layers = [(host
    experts or HostExpertSet, d_router_w, d_router_bias or None, layer_id)]. Returns
    (ids [L][T][k], weights [L][T][k], telemetry dict)."""
    from ._lib import CachedLayer, StackTelemetry
    sets = [lay[0] if isinstance(lay[0], HostExpertSet) else HostExpertSet(lay[0]) for lay in layers]
    arr = (CachedLayer * len(layers))()
    for i, (lay, hs) in enumerate(zip(layers, sets)):
        _, w, b, lid = lay
        arr[i] = CachedLayer(C.cast(hs.arr, C.c_void_p), hs.n, _addr(w).value, None if b is None else _addr(b).value,
                             lid)
    L = len(layers)
    ids = np.zeros((L, n_tokens, k), np.uint32)
    ws = np.zeros((L, n_tokens, k), np.float32)
    tel = StackTelemetry()
    check(self.L.objeta_hip_moe_stack_cached(
        self.backend.ctx, int(fmt), stream, arr, L, k, 1 if renormalize else 0, n_tokens, _addr(d_h), hidden, inter,
        cache.h if cache is not None else None, 1 if prefetch_next else 0, ids.ctypes.data_as(C.c_void_p),
        ws.ctypes.data_as(C.c_void_p), _addr_or_none(d_trace), C.byref(tel)))
    return ids, ws, {n: getattr(tel, n) for n, _ in StackTelemetry._fields_ if n != "reserved"}


class HostExpertSet:
    """A layer's host expert tensors marshalled once for the executor entry points
    (the reference passes &[ExpertWeights]; rebuilding the C array on every call costs
    about a millisecond of Python at 128 experts). Keeps the arrays alive."""

    def __init__(self, experts):
        self.arr, self.keep = _host_experts(experts)
        self.n = len(experts)

    def __len__(self) -> int:
        return self.n


def _host_experts(experts):
    """(HostExpert array, kept arrays) for [(gate, up, down)] or
    [(gate_w, gate_s, up_w, up_s, down_w, down_s)] host tensors."""
    if isinstance(experts, HostExpertSet):
        return experts.arr, experts.keep
    keep = []
    arr = (HostExpert * max(1, len(experts)))()
    for i, e in enumerate(experts):
        parts = [np.ascontiguousarray(p).view(np.uint8).ravel() for p in e]
        keep += parts
        v = []
        for p in parts:
            v += [p.ctypes.data, p.nbytes]
        v += [0] * (12 - len(v))
        if len(parts) == 6:  # (gate_w, gate_s, up_w, up_s, down_w, down_s)
            g, gs, u, us, d, ds = parts
            v = [g.ctypes.data, g.nbytes, u.ctypes.data, u.nbytes, d.ctypes.data, d.nbytes,
                 gs.ctypes.data, gs.nbytes, us.ctypes.data, us.nbytes, ds.ctypes.data, ds.nbytes]
        arr[i] = HostExpert(*v)
    return arr, keep


def _execute(backend: HipBackend, fmt: int, stream, experts, selected, x, hidden, inter, out_dim, layer_id,
             cache: ExpertCache | None):
    arr, keep = _host_experts(experts)
    ids = np.array([s[0] for s in selected], np.uint64)
    ws = np.array([s[1] for s in selected], np.float32)
    xv = np.ascontiguousarray(x, dtype=np.float32).ravel()
    out = np.zeros(max(out_dim, 1), np.float32)
    tel = MoeTelemetry()
    check(backend.L.objeta_hip_moe_execute_selected(
        backend.ctx, int(fmt), stream, arr, len(experts), ids.ctypes.data_as(C.c_void_p),
        ws.ctypes.data_as(C.c_void_p), ids.size, xv.ctypes.data_as(C.c_void_p), xv.size, hidden, inter, out_dim,
        layer_id, cache.h if cache is not None else None, out.ctypes.data_as(C.c_void_p), C.byref(tel)))
    return out[:out_dim], _telemetry_moe(tel)


def _moe_execute_selected(self, quant, stream, experts, selected_experts, x, hidden: int, intermediate: int,
                          out_dim: int, layer_id: int, cache: ExpertCache | None = None, fmt=QuantFormat.Q4_0):
    """execute_selected_moe_cuda (moe.rs:352-751): experts = [(w_gate, w_up, w_down)] host
    bytes; selected_experts = [(expert_id, weight)]. Returns (out, telemetry)."""
    return _execute(self.backend, int(fmt), stream, experts, selected_experts, x, hidden, intermediate, out_dim,
                    layer_id, cache)


def _moe_execute_native_fp4(self, quant, stream, experts, selected_experts, x, hidden: int, intermediate: int,
                            out_dim: int, layer_id: int, cache: ExpertCache | None = None):
    """execute_selected_moe_native_fp4_cuda (moe.rs:816-1280): experts =
    [(gate_w, gate_s, up_w, up_s, down_w, down_s)] split-FP4 host bytes."""
    return _execute(self.backend, int(QuantFormat.DeepSeekFp4E2M1), stream, experts, selected_experts, x, hidden,
                    intermediate, out_dim, layer_id, cache)


def _moe_execute_official_fp4(self, quant, stream, experts, selected_experts, hidden_state, hidden_size: int,
                              intermediate_size: int, out_dim: int, layer_id: int,
                              cache: ExpertCache | None = None, shared_expert=None, swiglu_limit: float = 10.0,
                              shared_from_cache: bool = False):
    """execute_selected_moe_official_routed_fp4_cuda (moe.rs:1393-1663): experts =
    [(gate_w, gate_s, up_w, up_s, down_w, down_s)] split-FP4 host bytes (or a
    HostExpertSet); shared_expert = (gate_w, up_w, down_w, gate_s, up_s, down_s) device
    addresses of the FP8 shared expert, or None; shared_from_cache resolves the shared
    expert from the cache's preloaded entries first. Returns (out, telemetry)."""
    arr, keep = _host_experts(experts)
    ids = np.array([s[0] for s in selected_experts], np.uint64)
    ws = np.array([s[1] for s in selected_experts], np.float32)
    xv = np.ascontiguousarray(hidden_state, dtype=np.float32).ravel()
    out = np.zeros(max(out_dim, 1), np.float32)
    tel = MoeTelemetry()
    sh = None
    if shared_expert is not None:
        sh = ExpertPtrs(*[_ptr_int(p) for p in shared_expert])
    check(self.L.objeta_hip_moe_execute_official_fp4(
        self.backend.ctx, stream, arr, len(experts), ids.ctypes.data_as(C.c_void_p), ws.ctypes.data_as(C.c_void_p),
        ids.size, xv.ctypes.data_as(C.c_void_p), xv.size, hidden_size, intermediate_size, out_dim, layer_id,
        cache.h if cache is not None else None, None if sh is None else C.byref(sh), 1 if shared_from_cache else 0,
        swiglu_limit, out.ctypes.data_as(C.c_void_p), C.byref(tel)))
    del keep
    return out[:out_dim], _telemetry_moe(tel)


MoeExecutor.execute_selected_moe_official_routed_fp4 = _moe_execute_official_fp4
MoeExecutor.execute_selected_moe_official_routed_fp4_cuda = _moe_execute_official_fp4
MoeExecutor.execute_selected_moe = _moe_execute_selected
MoeExecutor.execute_selected_moe_cuda = _moe_execute_selected
MoeExecutor.stack_cached = _moe_stack_cached
MoeExecutor.execute_selected_moe_native_fp4 = _moe_execute_native_fp4
MoeExecutor.execute_selected_moe_native_fp4_cuda = _moe_execute_native_fp4
