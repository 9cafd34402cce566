"""ctypes binding of the CPU oracle (oracle/oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, always as the checker (or the timed CPU baseline),
never by the product package. Builds oracle/_build/liboracle.so on first use when
it is missing and a C compiler is present.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "liboracle.so")

Q4_0, Q5_0, IQ3_0, FP4 = 0, 1, 2, 3
BLOCK_BYTES = {Q4_0: 18, Q5_0: 22, IQ3_0: 14, FP4: 17}

_lib = None


def build() -> str:
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = C.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


P = C.c_void_p
SZ = C.c_size_t


def _declare(L):
    L.orc_block_bytes.argtypes = [C.c_int]
    L.orc_f32_to_f16_bits.argtypes = [C.c_float]
    L.orc_f32_to_f16_bits.restype = C.c_uint16
    L.orc_f16_to_f32_bits.argtypes = [C.c_uint16]
    L.orc_f16_to_f32_bits.restype = C.c_float
    L.orc_f32_to_f16_bits_n.argtypes = [P, P, SZ]
    L.orc_f16_to_f32_bits_n.argtypes = [P, P, SZ]
    L.orc_decode_f8_e8m0.argtypes = [C.c_uint8]
    L.orc_decode_f8_e8m0.restype = C.c_float
    L.orc_f8e8m0_to_f32.argtypes = [C.c_uint8]
    L.orc_f8e8m0_to_f32.restype = C.c_float
    L.orc_fp4_scale_raw.argtypes = [C.c_float]
    L.orc_fp4_scale_raw.restype = C.c_uint8
    L.orc_fp4_scale_raw_n.argtypes = [P, P, SZ]
    for n in ("orc_q4_quantize_block", "orc_q5_quantize_block", "orc_iq3_quantize_block",
              "orc_fp4_quantize_block"):
        getattr(L, n).argtypes = [P, P]
    L.orc_quantize_matrix.argtypes = [C.c_int, P, SZ, SZ, SZ, P, SZ, C.c_char_p, SZ]
    L.orc_dot_row.argtypes = [C.c_int, P, P, SZ]
    L.orc_dot_row.restype = C.c_float
    L.orc_gemv.argtypes = [C.c_int, P, SZ, P, SZ, SZ, SZ, P, C.c_char_p, SZ]
    L.orc_dense_gemv.argtypes = [P, SZ, P, SZ, SZ, SZ, P, C.c_char_p, SZ]
    L.orc_decode_fp4_split.argtypes = [P, P, SZ, SZ, P]
    L.orc_fp4_split_gemv.argtypes = [P, P, P, SZ, SZ, P]
    L.orc_selected_moe.argtypes = [C.c_int, SZ, P, P, P, P, P, P, P, P, SZ, P, SZ, SZ, SZ, P,
                                   C.c_char_p, SZ]
    L.orc_router.argtypes = [P, P, P, SZ, SZ, SZ, C.c_int, P, P, P, P, C.c_char_p, SZ]
    L.orc_compare.argtypes = [P, P, SZ, P]
    L.orc_seeded_f32s.argtypes = [C.c_uint64, P, SZ]
    L.orc_gauss.argtypes = [C.c_uint64, C.c_uint64, C.c_float]
    L.orc_gauss.restype = C.c_float
    L.orc_gauss_fill.argtypes = [C.c_uint64, C.c_uint64, C.c_float, P, SZ]
    L.orc_splitmix64.argtypes = [C.c_uint64]
    L.orc_splitmix64.restype = C.c_uint64
    L.orc_f8e4m3_to_f32.argtypes = [C.c_uint8]
    L.orc_f8e4m3_to_f32.restype = C.c_float
    L.orc_f32_to_f8e4m3_exact.argtypes = [C.c_float]
    L.orc_f32_to_f8e4m3_exact.restype = C.c_uint8
    L.orc_f8e4m3_to_f32_n.argtypes = [P, P, SZ]
    L.orc_f32_to_f8e4m3_exact_n.argtypes = [P, P, SZ]
    L.orc_act_quant.argtypes = [P, SZ, SZ, P, P]
    L.orc_fp8_act_fp4_weight_gemv_f32.argtypes = [P, P, P, P, SZ, SZ, P]
    L.orc_fp8_act_fp8_weight_gemv.argtypes = [P, P, P, P, SZ, SZ, P]
    L.orc_expert_official.argtypes = [C.c_int, P, P, P, P, P, P, P, SZ, SZ, C.c_float, P, P, P, P, C.c_char_p,
                                      SZ]
    L.orc_set_threads.argtypes = [C.c_int]
    L.orc_get_threads.restype = C.c_int
    L.orc_expf_glibc.argtypes = [P, P, SZ]
    L.orc_expf_restated.argtypes = [C.c_float]
    L.orc_expf_restated.restype = C.c_float
    L.orc_expf_range_check.argtypes = [C.c_uint32, C.c_uint32, C.POINTER(C.c_uint64), C.POINTER(C.c_uint64)]
    L.orc_expf_double_disagreements.argtypes = [C.c_uint32, C.c_uint32, P, SZ]
    L.orc_expf_double_disagreements.restype = SZ


class OracleError(Exception):
    """Error raised by an oracle function; `kind` is the CudaErrorKind ordinal."""

    KINDS = ["Driver", "Runtime", "Nvrtc", "Io", "InvalidInput", "Unsupported", "Internal"]

    def __init__(self, rc: int, msg: str):
        self.kind = self.KINDS[rc - 1] if 0 < rc <= len(self.KINDS) else "Internal"
        self.source_message = msg
        super().__init__(f"{self.kind}: {msg}")


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


def _check(rc: int, err) -> None:
    if rc != 0:
        raise OracleError(rc, err.value.decode())


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _u8(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.uint8)


# ---------------------------------------------------------------- conversions
def f32_to_f16_bits(v) -> np.ndarray:
    v = _f32(v).ravel()
    out = np.empty(v.size, np.uint16)
    lib().orc_f32_to_f16_bits_n(_ptr(v), _ptr(out), v.size)
    return out


def f16_to_f32_bits(h) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16).ravel()
    out = np.empty(h.size, np.float32)
    lib().orc_f16_to_f32_bits_n(_ptr(h), _ptr(out), h.size)
    return out


def decode_f8_e8m0(raw: int) -> float:
    return lib().orc_decode_f8_e8m0(raw)


def f8e8m0_to_f32(raw: int) -> float:
    return lib().orc_f8e8m0_to_f32(raw)


def fp4_scale_raw(amax: float) -> int:
    return lib().orc_fp4_scale_raw(amax)


# ---------------------------------------------------------------- quantizers
def quantize_block(fmt: int, src) -> np.ndarray:
    src = _f32(src)
    assert src.size == 32
    out = np.zeros(BLOCK_BYTES[fmt], np.uint8)
    fn = {Q4_0: "orc_q4_quantize_block", Q5_0: "orc_q5_quantize_block",
          IQ3_0: "orc_iq3_quantize_block", FP4: "orc_fp4_quantize_block"}[fmt]
    getattr(lib(), fn)(_ptr(src), _ptr(out))
    return out


def quantize_matrix(fmt: int, matrix, rows: int, cols: int) -> np.ndarray:
    m = _f32(matrix).ravel()
    nbytes = rows * (cols // 32) * BLOCK_BYTES[fmt] if cols % 32 == 0 else 0
    out = np.zeros(max(nbytes, 1), np.uint8)
    err = C.create_string_buffer(256)
    rc = lib().orc_quantize_matrix(fmt, _ptr(m), m.size, rows, cols, _ptr(out), nbytes, err, 256)
    _check(rc, err)
    return out[:nbytes]


def gemv(fmt: int, q, x, rows: int, cols: int) -> np.ndarray:
    q = _u8(q).ravel()
    x = _f32(x).ravel()
    y = np.zeros(max(rows, 1), np.float32)
    err = C.create_string_buffer(256)
    rc = lib().orc_gemv(fmt, _ptr(q), q.size, _ptr(x), x.size, rows, cols, _ptr(y), err, 256)
    _check(rc, err)
    return y[:rows]


def dense_gemv(m, x, rows: int, cols: int) -> np.ndarray:
    m = _f32(m).ravel()
    x = _f32(x).ravel()
    y = np.zeros(max(rows, 1), np.float32)
    err = C.create_string_buffer(256)
    rc = lib().orc_dense_gemv(_ptr(m), m.size, _ptr(x), x.size, rows, cols, _ptr(y), err, 256)
    _check(rc, err)
    return y[:rows]


def decode_fp4_split(w, s, rows: int, cols: int) -> np.ndarray:
    w = _u8(w).ravel()
    s = _u8(s).ravel()
    assert w.size == rows * cols // 2 and s.size == rows * cols // 32
    out = np.empty(rows * cols, np.float32)
    lib().orc_decode_fp4_split(_ptr(w), _ptr(s), rows, cols, _ptr(out))
    return out


def fp4_split_gemv(w, s, x, rows: int, cols: int) -> np.ndarray:
    w, s, x = _u8(w).ravel(), _u8(s).ravel(), _f32(x).ravel()
    assert w.size == rows * cols // 2 and s.size == rows * cols // 32 and x.size == cols
    y = np.empty(rows, np.float32)
    lib().orc_fp4_split_gemv(_ptr(w), _ptr(s), _ptr(x), rows, cols, _ptr(y))
    return y


def split_interleaved_fp4(interleaved, rows: int, cols: int):
    """Interleaved 17-byte FP4 blocks -> (weights [rows, cols/2], scales [rows, cols/32]),
    as the reference's test helper split_interleaved_fp4 (moe.rs:2318-2331)."""
    b = _u8(interleaved).reshape(rows, cols // 32, 17)
    return np.ascontiguousarray(b[:, :, 1:]).ravel(), np.ascontiguousarray(b[:, :, 0]).ravel()


# ---------------------------------------------------------------- MoE
def selected_moe(fmt: int, experts, selected, x, hidden: int, inter: int, out_dim: int, shared=None):
    """experts: list of (gate, up, down) arrays (bytes for block formats / f32 for
    fmt=-1) or, for FP4, (gate_w, gate_s, up_w, up_s, down_w, down_s).
    selected: list of (expert_id, weight). shared: one more expert in the same form,
    added with weight 1.0 after the routed sum, as execute_selected_moe_official_routed_fp4_cuda
    does (moe.rs:1552-1600: weighted_accum(shared_down, out, 1.0) after the routed loop),
    which is the routed loop of orc_selected_moe run over one more slot."""
    if shared is not None:
        experts = list(experts) + [shared]
        selected = list(selected) + [(len(experts) - 1, 1.0)]
    n = len(experts)
    keep = []

    def arr(a, f32):
        a = _f32(a) if f32 else _u8(a)
        keep.append(a)
        return a.ctypes.data

    PA = C.c_void_p * n
    if fmt == FP4:
        g = PA(*[arr(e[0], False) for e in experts])
        gs = PA(*[arr(e[1], False) for e in experts])
        u = PA(*[arr(e[2], False) for e in experts])
        us = PA(*[arr(e[3], False) for e in experts])
        d = PA(*[arr(e[4], False) for e in experts])
        ds = PA(*[arr(e[5], False) for e in experts])
    else:
        f32 = fmt == -1
        g = PA(*[arr(e[0], f32) for e in experts])
        u = PA(*[arr(e[1], f32) for e in experts])
        d = PA(*[arr(e[2], f32) for e in experts])
        gs = us = ds = None
    ids = np.array([s[0] for s in selected], np.uint32)
    ws = np.array([s[1] for s in selected], np.float32)
    x = _f32(x).ravel()
    out = np.zeros(out_dim, np.float32)
    err = C.create_string_buffer(256)
    rc = lib().orc_selected_moe(fmt, n, g, u, d, gs, us, ds, _ptr(ids), _ptr(ws), ids.size,
                                _ptr(x), hidden, inter, out_dim, _ptr(out), err, 256)
    _check(rc, err)
    return out


def router(w_r, x, n_experts: int, hidden: int, k: int, bias=None, renormalize=True):
    w_r, x = _f32(w_r).ravel(), _f32(x).ravel()
    b = None if bias is None else _f32(bias).ravel()
    ids = np.zeros(k, np.uint32)
    ws = np.zeros(k, np.float32)
    logits = np.zeros(n_experts, np.float32)
    probs = np.zeros(n_experts, np.float32)
    err = C.create_string_buffer(256)
    rc = lib().orc_router(_ptr(w_r), None if b is None else _ptr(b), _ptr(x), n_experts, hidden,
                          k, 1 if renormalize else 0, _ptr(ids), _ptr(ws), _ptr(logits),
                          _ptr(probs), err, 256)
    _check(rc, err)
    return ids, ws, logits, probs


# ------------------------------------------------------ FP8 official arithmetic
def f8e4m3_to_f32(raw) -> np.ndarray:
    """f8e4m3_to_f32 (deepseek.rs:799-829) element-wise."""
    r = _u8(raw).ravel()
    out = np.empty(r.size, np.float32)
    lib().orc_f8e4m3_to_f32_n(_ptr(r), _ptr(out), r.size)
    return out


def f32_to_f8e4m3(v) -> np.ndarray:
    """f32_to_f8e4m3_exact (deepseek.rs:1444-1473) element-wise."""
    x = _f32(v).ravel()
    out = np.empty(x.size, np.uint8)
    lib().orc_f32_to_f8e4m3_exact_n(_ptr(x), _ptr(out), x.size)
    return out


def act_quant(x, block: int = 128):
    """cpu_act_quant (deepseek.rs:1484-1525): (F8_E4M3 bytes, F8_E8M0 scales)."""
    x = _f32(x).ravel()
    assert x.size % block == 0
    y = np.empty(x.size, np.uint8)
    sc = np.empty(x.size // block, np.uint8)
    lib().orc_act_quant(_ptr(x), x.size, block, _ptr(y), _ptr(sc))
    return y, sc


def fp8_act_fp4_gemv(act_v, act_s, w, ws, rows: int, cols: int) -> np.ndarray:
    """cpu_fp8_act_fp4_weight_gemv_f32 (deepseek.rs:1528-1566)."""
    a, s_, w, ws = _u8(act_v), _u8(act_s), _u8(w), _u8(ws)
    out = np.empty(rows, np.float32)
    lib().orc_fp8_act_fp4_weight_gemv_f32(_ptr(a), _ptr(s_), _ptr(w), _ptr(ws), rows, cols, _ptr(out))
    return out


def fp8_act_fp8_gemv(act_v, act_s, w, ws, rows: int, cols: int) -> np.ndarray:
    """cpu_fp8_act_fp8_weight_gemv (deepseek.rs:1630-1661), f64 sums."""
    a, s_, w, ws = _u8(act_v), _u8(act_s), _u8(w), _u8(ws)
    out = np.empty(rows, np.float32)
    lib().orc_fp8_act_fp8_weight_gemv(_ptr(a), _ptr(s_), _ptr(w), _ptr(ws), rows, cols, _ptr(out))
    return out


def expert_official(fp8_weights: bool, ex, x, dim: int, inter: int, swiglu_limit: float = 10.0):
    """One expert of the official composition: cpu_routed_expert_fp4_official_f32
    (deepseek.rs:1694-1716; ex = FP4 split (gw, gs, uw, us, dw, ds)) or
    cpu_shared_expert_fp8_official (deepseek.rs:1664-1692; ex = FP8 weights with
    128 x 128 tile scales). dim is both the input and the output length, as in the
    reference's compositions. Returns (out, act before its act_quant, act bytes, act
    scales)."""
    parts = [_u8(a) for a in ex]
    x = _f32(x).ravel()
    out = np.empty(dim, np.float32)
    pre = np.empty(inter, np.float32)
    aq = np.empty(inter, np.uint8)
    asc = np.empty(inter // 128, np.uint8)
    err = C.create_string_buffer(256)
    rc = lib().orc_expert_official(1 if fp8_weights else 0, *[_ptr(p) for p in parts], _ptr(x), dim, inter,
                                   swiglu_limit, _ptr(out), _ptr(pre), _ptr(aq), _ptr(asc), err, 256)
    _check(rc, err)
    return out, pre, aq, asc


def set_threads(n: int) -> None:
    """Threads of the oracle's row loops (1 = the reference's single thread)."""
    lib().orc_set_threads(int(n))


def expf_glibc(x) -> np.ndarray:
    """glibc's expf element-wise (the f32::exp of the reference's softmax)."""
    x = _f32(x).ravel()
    out = np.empty_like(x)
    lib().orc_expf_glibc(_ptr(x), _ptr(out), x.size)
    return out


def expf_restated(x) -> np.ndarray:
    """The oracle's restatement of glibc's expf method (the device router's form)."""
    x = _f32(x).ravel()
    return np.array([lib().orc_expf_restated(float(v)) for v in x], np.float32)


def expf_range_check(lo_bits: int, hi_bits: int):
    """(restated mismatches, double-rounded mismatches) against glibc's expf over every
    float with bits in [lo_bits, hi_bits]."""
    a, b = C.c_uint64(), C.c_uint64()
    lib().orc_expf_range_check(lo_bits, hi_bits, C.byref(a), C.byref(b))
    return a.value, b.value


def expf_double_disagreements(lo_bits: int, hi_bits: int, cap: int = 1 << 18) -> np.ndarray:
    """Sorted arguments in [lo_bits, hi_bits] where double exp rounded to float != glibc expf."""
    out = np.empty(cap, np.float32)
    n = lib().orc_expf_double_disagreements(lo_bits, hi_bits, _ptr(out), cap)
    return np.sort(out[:min(n, cap)])


def compare(ref, act):
    ref, act = _f32(ref).ravel(), _f32(act).ravel()
    assert ref.size == act.size
    out = np.zeros(3, np.float32)
    lib().orc_compare(_ptr(ref), _ptr(act), ref.size, _ptr(out))
    return {"cosine_similarity": float(out[0]), "relative_l2_error": float(out[1]),
            "max_abs_error": float(out[2])}


# ---------------------------------------------------------------- generators
def seeded_f32s(n: int, seed: int) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().orc_seeded_f32s(seed & 0xFFFFFFFFFFFFFFFF, _ptr(out), n)
    return out


def gauss(n: int, seed: int, sigma: float, first: int = 0) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().orc_gauss_fill(seed & 0xFFFFFFFFFFFFFFFF, first, sigma, _ptr(out), n)
    return out


def splitmix64(z: int) -> int:
    return lib().orc_splitmix64(z & 0xFFFFFFFFFFFFFFFF)
