"""Checkpoint ingest for the expert path: the Python mirror of ModelWeights
(crates/objeta-parser/src/lib.rs:88-293) and of the DeepSeek tensor lookups of
crates/objeta-cuda/src/bin/deepseek_single_layer_moe.rs, over libobjeta_hip.so's
memory-mapped safetensors reader (objeta_amd/csrc/safetensors.cpp).

Arrays returned by get_raw and the DeepSeek lookups are zero-copy views of the
mapping; each keeps the model open while it is alive."""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

from . import _lib
from .api import HostExpert, check

DTYPES = ("F32", "F16", "BF16", "I64", "I32", "I8", "U8", "F8_E8M0", "F8_E4M3", "BOOL")
_NP = {"F32": np.float32, "F16": np.float16, "I64": np.int64, "I32": np.int32, "I8": np.int8, "U8": np.uint8,
       "BOOL": np.bool_}


class StInfo(C.Structure):
    _fields_ = [("dtype", C.c_int32), ("ndim", C.c_uint32), ("shape", C.c_uint64 * 8), ("nbytes", C.c_uint64),
                ("nelem", C.c_uint64), ("file", C.c_uint32), ("reserved", C.c_uint32)]


class TensorInfo:
    """TensorInfo (lib.rs:20-28): dtype name, shape, byte count, element count and shard."""

    def __init__(self, s: StInfo):
        self.dtype = DTYPES[s.dtype]
        self.shape = tuple(int(s.shape[i]) for i in range(s.ndim))
        self.nbytes = int(s.nbytes)
        self.nelem = int(s.nelem)
        self.file = int(s.file)

    def __repr__(self):
        return f"TensorInfo(dtype={self.dtype}, shape={self.shape}, nbytes={self.nbytes})"


class ModelWeights:
    """ModelWeights::open (lib.rs:104-178) of one .safetensors file or a directory of
    shards (taken in file-name order)."""

    def __init__(self, path: str | os.PathLike):
        self.L = _lib.load()
        h = C.c_void_p()
        check(self.L.objeta_hip_st_open(os.fsencode(path), C.byref(h)))
        self.h = h

    @classmethod
    def open(cls, path) -> "ModelWeights":
        return cls(path)

    def close(self) -> None:
        if self.h:
            self.L.objeta_hip_st_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __len__(self) -> int:
        n = C.c_uint64()
        check(self.L.objeta_hip_st_len(self.h, C.byref(n)))
        return n.value

    def is_empty(self) -> bool:
        return len(self) == 0

    def keys(self) -> list:
        out = []
        for i in range(len(self)):
            n = C.c_uint64()
            check(self.L.objeta_hip_st_key(self.h, i, None, 0, C.byref(n)))
            buf = C.create_string_buffer(n.value + 1)
            check(self.L.objeta_hip_st_key(self.h, i, buf, n.value + 1, C.byref(n)))
            out.append(buf.value.decode("utf-8"))
        return out

    def info(self, name: str) -> TensorInfo | None:
        found, st = C.c_int32(), StInfo()
        check(self.L.objeta_hip_st_info_get(self.h, name.encode(), C.byref(found), C.byref(st)))
        return TensorInfo(st) if found.value else None

    def contains(self, name: str) -> bool:
        return self.info(name) is not None

    def _view(self, ptr: int, nbytes: int) -> np.ndarray:
        buf = (C.c_uint8 * max(1, nbytes)).from_address(ptr)
        buf._owner = self  # the mapping stays while a view is alive
        return np.frombuffer(buf, dtype=np.uint8, count=nbytes)

    def get_raw(self, name: str) -> np.ndarray:
        """get_raw (lib.rs:232-241): the tensor's bytes, a view of the mapping."""
        p, n = C.c_void_p(), C.c_uint64()
        check(self.L.objeta_hip_st_get_raw(self.h, name.encode(), C.byref(p), C.byref(n)))
        return self._view(p.value or 0, n.value)

    def get_typed(self, name: str) -> np.ndarray:
        """The raw bytes viewed in the tensor's numpy dtype and shape (dtypes numpy has)."""
        info = self.info(name)
        raw = self.get_raw(name)
        dt = _NP.get(info.dtype, np.uint8) if info.dtype not in ("BF16", "F8_E8M0", "F8_E4M3") else np.uint8
        if info.dtype == "BF16":
            dt = np.uint16
        return raw.view(dt).reshape(info.shape)

    def get_f32(self, name: str) -> np.ndarray:
        """get_f32 (lib.rs:243-276): F32 copied, F16 / BF16 converted."""
        n = C.c_uint64()
        check(self.L.objeta_hip_st_get_f32(self.h, name.encode(), None, 0, C.byref(n)))
        out = np.empty(n.value, np.float32)
        check(self.L.objeta_hip_st_get_f32(self.h, name.encode(), out.ctypes.data_as(C.c_void_p), n.value,
                                           C.byref(n)))
        return out

    def get_matrix(self, name: str):
        """get_matrix (lib.rs:278-296): (rows, cols, row-major f32) of a 2-D tensor."""
        info = self.info(name)
        if info is None:
            self.get_raw(name)  # raises the missing-tensor error
        if len(info.shape) != 2:
            raise ValueError(f"expected 2D tensor for {name}, got shape {list(info.shape)}")
        return info.shape[0], info.shape[1], self.get_f32(name).reshape(info.shape)

    # ---- DeepSeek naming
    def _expert(self, fn, *args):
        he = HostExpert()
        hid, inter, out = C.c_uint64(), C.c_uint64(), C.c_uint64()
        check(fn(self.h, *args, C.byref(he), C.byref(hid), C.byref(inter), C.byref(out)))
        parts = [self._view(he.gate or 0, he.gate_len), self._view(he.gate_scale or 0, he.gate_scale_len),
                 self._view(he.up or 0, he.up_len), self._view(he.up_scale or 0, he.up_scale_len),
                 self._view(he.down or 0, he.down_len), self._view(he.down_scale or 0, he.down_scale_len)]
        return tuple(parts), (hid.value, inter.value, out.value)

    def deepseek_expert(self, layer: int, expert: int, mtp: bool = False):
        """find_fp4_expert_tensors (deepseek_single_layer_moe.rs:410-520) by classify_tensor's
        rules: ((gate_w, gate_s, up_w, up_s, down_w, down_s) split-FP4 byte views,
        (hidden, intermediate, out_dim))."""
        return self._expert(self.L.objeta_hip_st_deepseek_expert, layer, expert, 1 if mtp else 0)

    def deepseek_shared_expert(self, layer: int, mtp: bool = False):
        """load_shared_expert_fp8 (deepseek_single_layer_moe.rs:1034-1080): the FP8 shared
        expert's (gate_w, gate_s, up_w, up_s, down_w, down_s) byte views and dims."""
        return self._expert(self.L.objeta_hip_st_deepseek_shared_expert, layer, 1 if mtp else 0)

    def deepseek_router(self, layer: int, mtp: bool = False):
        """find_router_tensor (deepseek_single_layer_moe.rs:226-330): (name, [E][H] f32)."""
        buf = C.create_string_buffer(512)
        st = StInfo()
        check(self.L.objeta_hip_st_deepseek_router(self.h, layer, 1 if mtp else 0, buf, 512, C.byref(st)))
        name = buf.value.decode("utf-8")
        _, _, m = self.get_matrix(name)
        return name, m
