"""CPU oracle for the Q4_K / Q6_K x Q8 projection path -- TEST INFRASTRUCTURE.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline leg
may import this package, and only as the checker (or the timed CPU baseline).
The product (``qw38_amd``) never imports it and has no CPU fallback.

The arithmetic lives in ``oracle.c`` (plain C, built with -ffp-contract=off);
this module wraps it with numpy. ``ref()`` loads ``_ref/libref_llama_q4k.so``,
the reference's own pinned llama.cpp Q4_K header compiled in place, used to pin
the oracle's quantizer. The header of ``oracle.c`` states how every function is
pinned; the Q6_K quantizer (no reference code or vectors exist) is pinned by
exact-block round trips and closed-form properties of its last steps.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libref_llama_q4k.so")

LAYOUT_Q4K_SEQ = 0x020D     # reference CudaQ4KCandidateV2
LAYOUT_Q4K_W64 = 0x0240     # wave64 nibble order (this build)
LAYOUT_Q6K_W64 = 0x0241     # Q6_K wave64 layout (this build)

_lib = None
_ref = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def _p(a):
    return a.ctypes.data_as(C.c_void_p) if a is not None else None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        V, U16, U32, U64, I = C.c_void_p, C.c_uint16, C.c_uint32, C.c_uint64, C.c_int
        sig = {
            "orc_fp16_to_fp32": (C.c_float, [U16]),
            "orc_fp32_to_fp16": (U16, [C.c_float]),
            "orc_fp32_to_bf16_rne": (U16, [C.c_float]),
            "orc_nearest_int": (I, [C.c_float]),
            "orc_expf": (C.c_float, [C.c_float]),
            "orc_pack_q8": (I, [V, U32, U32, U32, V, V, V]),
            "orc_pack_q8_f32": (I, [V, U32, U32, U32, V, V, V]),
            "orc_rms_q8": (I, [V, V, C.c_float, U32, V, V, V, V]),
            "orc_swiglu_q8": (I, [V, V, U32, U32, V, V, V, V]),
            "orc_quantize_q4k_block": (I, [V, V, V]),
            "orc_quantize_q4k_rows": (I, [V, U64, U64, V, V, I]),
            "orc_q4k_logical_to_ggml": (None, [V, V, U64, V]),
            "orc_q4k_ggml_to_logical": (None, [V, U64, V, V]),
            "orc_pack_q4k_layout": (I, [U16, V, V, U32, U32, V, V]),
            "orc_unpack_q4k_layout": (I, [U16, V, V, U32, U32, V, V]),
            "orc_quantize_q6k_block": (None, [V, V, V, V]),
            "orc_q6k_fit_subblock": (C.c_float, [V, V]),
            "orc_quantize_q6k_rows": (I, [V, U64, U64, V, V, V, I]),
            "orc_q6k_logical_to_ggml": (None, [V, V, V, U64, V]),
            "orc_q6k_ggml_to_logical": (None, [V, U64, V, V, V]),
            "orc_pack_q6k_layout": (I, [V, V, V, U32, U32, V, V]),
            "orc_unpack_q6k_layout": (I, [V, V, U32, U32, V, V, V]),
            "orc_q4k_q8_contract": (None, [V, V, U32, U32, V, V, V, U32, V, V, V, I]),
            "orc_q6k_q8_contract": (None, [V, V, V, U32, U32, V, V, V, U32, V, V, V, I]),
            "orc_q4k_bf16_weight": (C.c_float, [V, C.c_uint, C.c_uint]),
            "orc_q4k_bf16_gemv": (None, [V, V, U32, U32, U32, V, V, I]),
            "orc_pack_dense_layout": (I, [U16, V, V, U32, U32, V, V]),
            "orc_pack_bf16_tile": (I, [V, U32, U32, V]),
            "orc_dense_operands": (None, [U16, V, V, U32, U32, V]),
            "orc_e4m3_to_fp32": (C.c_float, [C.c_uint8]),
            "orc_fp32_to_e4m3": (C.c_uint8, [C.c_float]),
            "orc_pack_fp8": (None, [V, U32, U32, V, V]),
            "orc_fp8_gemv": (None, [V, V, U32, U32, V, V, V]),
            "orc_fp8_gemm": (None, [V, V, U32, U32, V, V, U32, V, V]),
            "orc_e2m1_value": (C.c_float, [C.c_uint8]),
            "orc_ue4m3_value": (C.c_float, [C.c_uint8]),
            "orc_nvfp4_nearest": (C.c_uint8, [C.c_float, I]),
            "orc_nvfp4_sf_index": (U64, [U64, U64, U64]),
            "orc_pack_nvfp4": (None, [V, U32, U32, V, V]),
            "orc_quantize_nvfp4": (I, [V, U32, U32, V, V]),
            "orc_nvfp4_gemv": (None, [V, V, U32, U32, V, U32, V, V]),
            "orc_nvfp4_gemm": (None, [V, V, U32, U32, V, V, U32, V, V]),
        }
        for name, (res, args) in sig.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def ref():
    """The pinned llama.cpp header compiled in place (None when unavailable)."""
    global _ref
    if _ref is None:
        if not os.path.exists(REF_PATH):
            return None
        R = C.CDLL(REF_PATH)
        R.ref_quantize_row_q4_K.argtypes = [C.c_void_p, C.c_void_p, C.c_longlong]
        R.ref_dequantize_row_q4_K.argtypes = [C.c_void_p, C.c_void_p, C.c_longlong]
        R.ref_fp16_to_fp32.restype = C.c_float
        R.ref_fp16_to_fp32.argtypes = [C.c_ushort]
        R.ref_fp32_to_fp16.restype = C.c_ushort
        R.ref_fp32_to_fp16.argtypes = [C.c_float]
        R.ref_nearest_int.restype = C.c_int
        R.ref_nearest_int.argtypes = [C.c_float]
        _ref = R
    return _ref


def _threads():
    return int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))


# ---- conversions ----------------------------------------------------------
def fp32_to_bf16(x: np.ndarray) -> np.ndarray:
    """Vectorised restatement of orc_fp32_to_bf16_rne (floatcvt.hpp:82-95)."""
    b = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    nan = ((b >> 23) & 0xFF) == 0xFF
    rounded = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)
    special = (b >> 16).astype(np.uint16) | np.where((b & 0x7FFFFF) != 0, 0x40, 0).astype(np.uint16)
    return np.where(nan, special, rounded).astype(np.uint16)


def bf16_to_fp32(h: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def pad256(k: int) -> int:
    return (k + 255) // 256 * 256


def pad8(n: int) -> int:
    return (n + 7) // 8 * 8


# ---- Q8 producers -----------------------------------------------------------
class Q8:
    def __init__(self, codes, scales, sums, m, k, pk, failed=False):
        self.codes, self.scales, self.sums = codes, scales, sums
        self.m, self.k, self.pk, self.failed = m, k, pk, failed


def pack_q8(bf16: np.ndarray, m: int, k: int) -> Q8:
    pk = pad256(k)
    bf16 = np.ascontiguousarray(bf16, dtype=np.uint16).reshape(m, k)
    codes = np.zeros((m, pk), np.int8)
    scales = np.zeros((m, pk // 32), np.float32)
    sums = np.zeros((m, pk // 32), np.int32)
    f = lib().orc_pack_q8(_p(bf16), m, k, pk, _p(codes), _p(scales), _p(sums))
    return Q8(codes, scales, sums, m, k, pk, bool(f))


def rms_q8(residual: np.ndarray, gamma: np.ndarray, eps: float):
    residual = np.ascontiguousarray(residual, dtype=np.float32)
    m = residual.shape[0]
    codes = np.zeros((m, 5120), np.int8)
    scales = np.zeros((m, 160), np.float32)
    sums = np.zeros((m, 160), np.int32)
    bf = np.zeros((m, 5120), np.uint16)
    gamma = np.ascontiguousarray(gamma, dtype=np.uint16)
    f = lib().orc_rms_q8(_p(residual), _p(gamma), eps, m, _p(codes), _p(scales), _p(sums), _p(bf))
    return Q8(codes, scales, sums, m, 5120, 5120, bool(f)), bf


def swiglu_q8(gate: np.ndarray, up: np.ndarray):
    gate = np.ascontiguousarray(gate, dtype=np.float32)
    up = np.ascontiguousarray(up, dtype=np.float32)
    m, n = gate.shape
    codes = np.zeros((m, n), np.int8)
    scales = np.zeros((m, n // 32), np.float32)
    sums = np.zeros((m, n // 32), np.int32)
    bf = np.zeros((m, n), np.uint16)
    f = lib().orc_swiglu_q8(_p(gate), _p(up), m, n, _p(codes), _p(scales), _p(sums), _p(bf))
    return Q8(codes, scales, sums, m, n, n, bool(f)), bf


# ---- Q4_K weights ---------------------------------------------------------
class Q4K:
    """Logical Q4_K matrix: codes uint8 [n][pk] in 0..15, meta uint8 [n][pk/256][16]."""

    def __init__(self, codes, meta, n, k):
        self.codes, self.meta, self.n, self.k = codes, meta, n, k
        self.pk = codes.shape[1]

    def physical(self, layout=LAYOUT_Q4K_SEQ):
        pn = pad8(self.n)
        co = np.zeros(pn * self.pk // 2, np.uint8)
        mo = np.zeros(pn * (self.pk // 256) * 16, np.uint8)
        rc = lib().orc_pack_q4k_layout(layout, _p(self.codes), _p(self.meta), self.n, self.pk, _p(co), _p(mo))
        assert rc == 0
        return co, mo

    @staticmethod
    def from_physical(layout, co, mo, n, k):
        pk = pad256(k)
        codes = np.zeros((n, pk), np.uint8)
        meta = np.zeros((n, pk // 256, 16), np.uint8)
        rc = lib().orc_unpack_q4k_layout(layout, _p(np.ascontiguousarray(co)), _p(np.ascontiguousarray(mo)),
                                         n, pk, _p(codes), _p(meta))
        assert rc == 0
        return Q4K(codes, meta, n, k)

    def ggml(self):
        blocks = self.n * self.pk // 256
        out = np.zeros(blocks * 144, np.uint8)
        lib().orc_q4k_logical_to_ggml(_p(self.codes), _p(self.meta), blocks, _p(out))
        return out

    @staticmethod
    def from_ggml(buf, n, k):
        pk = pad256(k)
        codes = np.zeros((n, pk), np.uint8)
        meta = np.zeros((n, pk // 256, 16), np.uint8)
        lib().orc_q4k_ggml_to_logical(_p(np.ascontiguousarray(buf, np.uint8)), n * pk // 256, _p(codes), _p(meta))
        return Q4K(codes, meta, n, k)


def quantize_q4k(w: np.ndarray, threads=None) -> Q4K:
    """Row-major fp32 [n][k] (k % 256 == 0) -> logical Q4_K."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    n, k = w.shape
    assert k % 256 == 0
    codes = np.zeros((n, k), np.uint8)
    meta = np.zeros((n, k // 256, 16), np.uint8)
    rc = lib().orc_quantize_q4k_rows(_p(w), n, k, _p(codes), _p(meta), threads or _threads())
    if rc:
        raise ValueError(f"Q4_K quantizer rejected input ({rc})")
    return Q4K(codes, meta, n, k)


def quantize_q4k_block(x: np.ndarray):
    x = np.ascontiguousarray(x, dtype=np.float32)
    codes = np.zeros(256, np.uint8)
    meta = np.zeros(16, np.uint8)
    rc = lib().orc_quantize_q4k_block(_p(x), _p(codes), _p(meta))
    return rc, codes, meta


# ---- Q6_K weights ---------------------------------------------------------
class Q6K:
    """Logical Q6_K: q uint8 [n][pk] in 0..63, sc int8 [n][pk/16], d uint16 [n][pk/256]."""

    def __init__(self, q, sc, d, n, k):
        self.q, self.sc, self.d, self.n, self.k = q, sc, d, n, k
        self.pk = q.shape[1]

    def physical(self):
        pn = pad8(self.n)
        kbs = self.pk // 256
        co = np.zeros(pn * kbs * 192, np.uint8)
        mo = np.zeros(pn * kbs * 18, np.uint8)
        rc = lib().orc_pack_q6k_layout(_p(self.q), _p(self.sc), _p(self.d), self.n, self.pk, _p(co), _p(mo))
        assert rc == 0
        return co, mo

    @staticmethod
    def from_physical(co, mo, n, k):
        pk = pad256(k)
        q = np.zeros((n, pk), np.uint8)
        sc = np.zeros((n, pk // 16), np.int8)
        d = np.zeros((n, pk // 256), np.uint16)
        rc = lib().orc_unpack_q6k_layout(_p(np.ascontiguousarray(co)), _p(np.ascontiguousarray(mo)), n, pk,
                                         _p(q), _p(sc), _p(d))
        assert rc == 0
        return Q6K(q, sc, d, n, k)

    def ggml(self):
        blocks = self.n * self.pk // 256
        out = np.zeros(blocks * 210, np.uint8)
        lib().orc_q6k_logical_to_ggml(_p(self.q), _p(self.sc), _p(self.d), blocks, _p(out))
        return out

    @staticmethod
    def from_ggml(buf, n, k):
        pk = pad256(k)
        q = np.zeros((n, pk), np.uint8)
        sc = np.zeros((n, pk // 16), np.int8)
        d = np.zeros((n, pk // 256), np.uint16)
        lib().orc_q6k_ggml_to_logical(_p(np.ascontiguousarray(buf, np.uint8)), n * pk // 256, _p(q), _p(sc), _p(d))
        return Q6K(q, sc, d, n, k)

    def dequantize(self) -> np.ndarray:
        dd = np.array([lib().orc_fp16_to_fp32(int(v)) for v in self.d.ravel()], np.float64).reshape(self.d.shape)
        sc = self.sc.astype(np.float64)
        q = self.q.astype(np.float64) - 32
        return q * np.repeat(sc, 16, axis=1) * np.repeat(dd, 256, axis=1)


def quantize_q6k(w: np.ndarray, threads=None) -> Q6K:
    w = np.ascontiguousarray(w, dtype=np.float32)
    n, k = w.shape
    assert k % 256 == 0
    q = np.zeros((n, k), np.uint8)
    sc = np.zeros((n, k // 16), np.int8)
    d = np.zeros((n, k // 256), np.uint16)
    lib().orc_quantize_q6k_rows(_p(w), n, k, _p(q), _p(sc), _p(d), threads or _threads())
    return Q6K(q, sc, d, n, k)


# ---- contractions ---------------------------------------------------------
def q4k_q8_contract(w: Q4K, x: Q8, want_dots=False, threads=None):
    assert w.pk == x.pk
    out64 = np.zeros((x.m, w.n), np.float64)
    out32 = np.zeros((x.m, w.n), np.float32)
    dots = np.zeros((x.m, w.n, w.pk // 32), np.int32) if want_dots else None
    lib().orc_q4k_q8_contract(_p(w.codes), _p(w.meta), w.n, w.pk, _p(x.codes), _p(x.scales), _p(x.sums),
                              x.m, _p(out64), _p(out32), _p(dots), threads or _threads())
    return out64, out32, dots


def q6k_q8_contract(w: Q6K, x: Q8, want_dots=False, threads=None):
    assert w.pk == x.pk
    out64 = np.zeros((x.m, w.n), np.float64)
    out32 = np.zeros((x.m, w.n), np.float32)
    dots = np.zeros((x.m, w.n, w.pk // 32), np.int32) if want_dots else None
    lib().orc_q6k_q8_contract(_p(w.q), _p(w.sc), _p(w.d), w.n, w.pk, _p(x.codes), _p(x.scales), _p(x.sums),
                              x.m, _p(out64), _p(out32), _p(dots), threads or _threads())
    return out64, out32, dots


def q4k_bf16_gemv(w: Q4K, x_bf16: np.ndarray, threads=None):
    out = np.zeros(w.n, np.float64)
    x = np.ascontiguousarray(x_bf16, np.uint16)
    lib().orc_q4k_bf16_gemv(_p(w.codes), _p(w.meta), w.n, w.pk, w.k, _p(x), _p(out), threads or _threads())
    return out


# ---- decode_mmv dense layouts (Q4G64, Q8G32, BF16 dense tile) ---------------
LAYOUT_Q4G64, LAYOUT_Q8G32, LAYOUT_BF16_TILE = 0x0201, 0x0202, 0x0203
LAYOUT_Q4G64_CAND, LAYOUT_Q8G32_CAND = 0x020B, 0x020C


def dense_group(layout: int) -> int:
    return 64 if layout in (LAYOUT_Q4G64, LAYOUT_Q4G64_CAND) else 32


def pack_dense(layout: int, codes: np.ndarray, scales: np.ndarray, n: int, k: int):
    """Logical int8 codes [n][k] + FP16 scale bits [n][k/group] -> (codes, scales)
    in the reference tile layout (src/format/pack.cpp:143-215)."""
    pn, pk = pad8(n), pad256(k)
    q4 = layout in (LAYOUT_Q4G64, LAYOUT_Q4G64_CAND)
    co = np.zeros(pn * pk // (2 if q4 else 1), np.uint8)
    so = np.zeros(pn * (pk // dense_group(layout)) * 2, np.uint8)
    c = np.ascontiguousarray(codes, np.int8)
    sc = np.ascontiguousarray(scales, np.uint16)
    assert c.size == n * k and sc.size == n * (k // dense_group(layout))
    st = lib().orc_pack_dense_layout(layout, _p(c), _p(sc), n, k, _p(co), _p(so))
    assert st == 0, "unsupported dense layout/shape"
    return co, so


def pack_bf16_tile(w_bf16: np.ndarray, n: int, k: int) -> np.ndarray:
    """Row-major BF16 bits [n][k] -> BF16 dense tiles (src/format/pack.cpp:247-290)."""
    w = np.ascontiguousarray(w_bf16, np.uint16)
    co = np.zeros(n * k * 2, np.uint8)
    assert lib().orc_pack_bf16_tile(_p(w), n, k, _p(co)) == 0
    return co


def dense_operands(layout: int, co: np.ndarray, so, pn: int, pk: int) -> np.ndarray:
    """BF16 operand bits [pn][pk] as decode_mmv rebuilds them (cuda/decode_mmv.cu:92-180)."""
    out = np.zeros((pn, pk), np.uint16)
    so = np.zeros(1, np.uint8) if so is None else np.ascontiguousarray(so, np.uint8)
    lib().orc_dense_operands(layout, _p(np.ascontiguousarray(co, np.uint8)), _p(so), pn, pk, _p(out))
    return out


def bf16_gemv(w_bf16: np.ndarray, x_bf16: np.ndarray) -> np.ndarray:
    """y = W x in double for BF16 operand bits W [n][k] and x [k]."""
    w = bf16_to_fp32(np.ascontiguousarray(w_bf16, np.uint16)).astype(np.float64)
    x = bf16_to_fp32(np.ascontiguousarray(x_bf16, np.uint16)).astype(np.float64)
    return w @ x


# ---- FP8 (OCP E4M3FN) path (cuda/fp8.cu) ------------------------------------
def pad128(v: int) -> int:
    return (v + 127) // 128 * 128


def e4m3_to_fp32(codes) -> np.ndarray:
    """Values of E4M3FN codes (NaN for 0x7F / 0xFF)."""
    table = np.array([lib().orc_e4m3_to_fp32(c) for c in range(256)], np.float32)
    return table[np.asarray(codes, np.uint8)]


def fp32_to_e4m3(x) -> np.ndarray:
    """Round to nearest even E4M3FN, saturating finite values at +-448."""
    f = lib().orc_fp32_to_e4m3
    a = np.asarray(x, np.float32)
    return np.array([f(float(v)) for v in a.ravel()], np.uint8).reshape(a.shape)


def pack_fp8(x_bf16: np.ndarray, m: int, k: int):
    """pack_fp8 (cuda/fp8.cu:64-81): codes [pm][pk], scales [pk/128][pm]."""
    pm, pk = pad128(m), pad128(k)
    codes = np.zeros((pm, pk), np.uint8)
    scales = np.zeros((pk // 128, pm), np.float32)
    x = np.ascontiguousarray(x_bf16, np.uint16)
    lib().orc_pack_fp8(_p(x), m, k, _p(codes), _p(scales))
    return codes, scales


def fp8_gemv(codes, wscales, n: int, k: int, x_bf16):
    """(y, l1) in double: y[r] = sum_c value(code) * scale * x."""
    y = np.zeros(n, np.float64)
    l1 = np.zeros(n, np.float64)
    lib().orc_fp8_gemv(_p(np.ascontiguousarray(codes, np.uint8)), _p(np.ascontiguousarray(wscales, np.float32)),
                       n, k, _p(np.ascontiguousarray(x_bf16, np.uint16)), _p(y), _p(l1))
    return y, l1


def fp8_gemm(wc, ws, n: int, k: int, xc, xs, m: int):
    """(y [m][n], l1) in double for packed FP8 operands (xs is [k/128][m])."""
    y = np.zeros((m, n), np.float64)
    l1 = np.zeros((m, n), np.float64)
    lib().orc_fp8_gemm(_p(np.ascontiguousarray(wc, np.uint8)), _p(np.ascontiguousarray(ws, np.float32)), n, k,
                       _p(np.ascontiguousarray(xc, np.uint8)), _p(np.ascontiguousarray(xs, np.float32)), m,
                       _p(y), _p(l1))
    return y, l1


# ---- NVFP4 path (cuda/nvfp4.cu, src/format/nvfp4.cpp) -----------------------
def nvfp4_scale_bytes(rows: int, pk: int) -> int:
    return pad128(rows) * (pk // 16)


def pad_k256(k: int) -> int:
    return (k + 255) // 256 * 256


def e2m1_value(c) -> np.ndarray:
    table = np.array([lib().orc_e2m1_value(i) for i in range(16)], np.float32)
    return table[np.asarray(c, np.uint8) & 15]


def ue4m3_value(c) -> np.ndarray:
    table = np.array([lib().orc_ue4m3_value(i) for i in range(128)], np.float32)
    return table[np.asarray(c, np.uint8) & 127]


def nvfp4_nearest(v: float, scale: bool) -> int:
    return int(lib().orc_nvfp4_nearest(float(v), 1 if scale else 0))


def nvfp4_sf_index(row: int, block: int, pk: int) -> int:
    return int(lib().orc_nvfp4_sf_index(row, block, pk))


def pack_nvfp4(x_bf16: np.ndarray, m: int, k: int):
    """launch_pack_nvfp4 (cuda/nvfp4.cu:72-82): (codes [m][pk/2], scales)."""
    pk = pad_k256(k)
    codes = np.zeros((m, pk // 2), np.uint8)
    scales = np.zeros(nvfp4_scale_bytes(m, pk), np.uint8)
    x = np.ascontiguousarray(x_bf16, np.uint16)
    lib().orc_pack_nvfp4(_p(x), m, k, _p(codes), _p(scales))
    return codes, scales


def quantize_nvfp4(w_bf16: np.ndarray, n: int, k: int):
    """quantize_nvfp4 (src/compiler/quantization/nvfp4.cpp:12-61): (codes
    [pn][pk/2], scales with the 256-byte factor header), pn = pad8(n)."""
    pk, pn = pad_k256(k), pad8(n)
    codes = np.zeros((pn, pk // 2), np.uint8)
    scales = np.zeros(256 + nvfp4_scale_bytes(pn, pk), np.uint8)
    w = np.ascontiguousarray(w_bf16, np.uint16)
    if lib().orc_quantize_nvfp4(_p(w), n, k, _p(codes), _p(scales)) != 0:
        raise ValueError("nonfinite BF16 weight")
    return codes, scales


def nvfp4_gemv(codes, scales, n: int, pk: int, x_bf16, k: int):
    y = np.zeros(n, np.float64)
    l1 = np.zeros(n, np.float64)
    lib().orc_nvfp4_gemv(_p(np.ascontiguousarray(codes, np.uint8)), _p(np.ascontiguousarray(scales, np.uint8)),
                         n, pk, _p(np.ascontiguousarray(x_bf16, np.uint16)), k, _p(y), _p(l1))
    return y, l1


def nvfp4_gemm(wc, ws, n: int, pk: int, xc, xs, m: int):
    y = np.zeros((m, n), np.float64)
    l1 = np.zeros((m, n), np.float64)
    lib().orc_nvfp4_gemm(_p(np.ascontiguousarray(wc, np.uint8)), _p(np.ascontiguousarray(ws, np.uint8)), n, pk,
                         _p(np.ascontiguousarray(xc, np.uint8)), _p(np.ascontiguousarray(xs, np.uint8)), m,
                         _p(y), _p(l1))
    return y, l1


# ---- parity metrics -------------------------------------------------------
def parity_ok(y: np.ndarray, ref: np.ndarray, max_abs_rms=1e-3, mean_rel=1e-5):
    """max|y-ref| <= 1e-3*rms(ref) and
    mean|y-ref| / mean|ref| <= 1e-5. Returns (ok, max_abs/rms, mean_rel)."""
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    if not np.all(np.isfinite(y)):
        return False, float("inf"), float("inf")
    err = np.abs(y - ref)
    rms = float(np.sqrt(np.mean(ref * ref))) or 1.0
    ma = float(err.max()) / rms if err.size else 0.0
    mabs = float(np.mean(np.abs(ref))) or 1.0
    mr = float(err.mean()) / mabs if err.size else 0.0
    return (ma <= max_abs_rms and mr <= mean_rel), ma, mr
