"""ctypes binding of the C-ABI in ``include/qw38_hip.h``.

Loads ``qw38_amd/libqw38_hip.so`` built in-tree. There is no fallback: a
missing library raises immediately, naming the build step.
"""
from __future__ import annotations

import ctypes as C
import os
import re

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
LIB_PATH = os.path.join(PKG, "libqw38_hip.so")
HEADER = os.path.join(ROOT, "include", "qw38_hip.h")

QW38_OK, QW38_STATUS, QW38_INVALID_ARGUMENT, QW38_OVERFLOW = 0, 1, 2, 3
LAYOUT_Q4K_SEQ = 0x020D
LAYOUT_Q4K_W64 = 0x0240
LAYOUT_Q6K_W64 = 0x0241
QUANTIZER_Q4K = 0x0105
QUANTIZER_Q6K = 0x0140
CODE_NAMES = {1: "Status", 2: "InvalidArgument", 3: "Overflow"}


class Weight(C.Structure):
    """qw38_weight == cuda::PrefillWeight (cuda/prefill.hpp:33-44)."""
    _fields_ = [("codes", C.c_void_p), ("scales", C.c_void_p), ("layout", C.c_uint16),
                ("quantizer", C.c_uint16), ("n", C.c_uint32), ("k", C.c_uint32),
                ("padded_n", C.c_uint32), ("padded_k", C.c_uint32),
                ("codes_bytes", C.c_uint64), ("scales_bytes", C.c_uint64)]


class Q8Input(C.Structure):
    """qw38_q8_input == cuda::Q8Input (cuda/q4k_q8.hpp:16-21)."""
    _fields_ = [("codes", C.c_void_p), ("codes_len", C.c_uint64), ("scales", C.c_void_p),
                ("scales_len", C.c_uint64), ("sums", C.c_void_p), ("sums_len", C.c_uint64),
                ("m", C.c_uint32), ("k", C.c_uint32), ("padded_k", C.c_uint32)]


class DecodeView(C.Structure):
    """qw38_decode_view == cuda::DecodeOperandView (cuda/decode_mmv.hpp:80-93)."""
    _fields_ = [("pointer", C.c_void_p), ("space", C.c_uint8), ("dtype", C.c_uint8),
                ("layout", C.c_uint16), ("logical_n", C.c_uint32), ("logical_k", C.c_uint32),
                ("padded_n", C.c_uint32), ("padded_k", C.c_uint32), ("bytes", C.c_uint64),
                ("alignment", C.c_uint32), ("writable", C.c_uint8)]


class DecodeDesc(C.Structure):
    """qw38_decode_desc == cuda::DecodeMmvDesc (cuda/decode_mmv.hpp:117-134)."""
    _fields_ = [("layout", C.c_uint16), ("quantizer", C.c_uint16),
                ("activation_policy", C.c_uint8), ("n", C.c_uint32), ("k", C.c_uint32),
                ("padded_n", C.c_uint32), ("padded_k", C.c_uint32), ("codes", DecodeView),
                ("scales", DecodeView), ("input", DecodeView), ("output", DecodeView),
                ("residual", DecodeView), ("epilogue", C.c_uint8)]


class Fp8Weight(C.Structure):
    """qw38_fp8_weight == cuda::Fp8Weight (cuda/fp8.hpp:18-22)."""
    _fields_ = [("codes", C.c_void_p), ("codes_len", C.c_uint64), ("scales", C.c_void_p),
                ("scales_len", C.c_uint64), ("n", C.c_uint32), ("k", C.c_uint32)]


class Fp8Input(C.Structure):
    """qw38_fp8_input == cuda::Fp8Input (cuda/fp8.hpp:13-17)."""
    _fields_ = [("codes", C.c_void_p), ("codes_len", C.c_uint64), ("scales", C.c_void_p),
                ("scales_len", C.c_uint64), ("m", C.c_uint32), ("k", C.c_uint32)]


class Qw38Error(RuntimeError):
    def __init__(self, status, hip_status, operation, detail):
        self.status, self.hip_status = status, hip_status
        self.operation, self.detail = operation, detail
        super().__init__(f"{CODE_NAMES.get(status, status)} in {operation}: {detail}"
                         + (f" (hip {hip_status})" if hip_status else ""))


_lib = None

_V, _U16, _U32, _U64, _I, _F = C.c_void_p, C.c_uint16, C.c_uint32, C.c_uint64, C.c_int, C.c_float
_P = C.POINTER
SIGNATURES = {
    "qw38_last_error": (_I, [_P(_I), C.c_char_p, C.c_size_t, C.c_char_p, C.c_size_t]),
    "qw38_pack_q8": (_I, [_V, _U64, _P(Q8Input), _V, _U64, _V]),
    "qw38_q4k_q8_project": (_I, [_P(Weight), _P(Q8Input), _V, _U64, _V, _U64, _V]),
    "qw38_q4k_q8_gate_up_swiglu": (_I, [_P(Weight), _P(Weight), _P(Q8Input), _P(Q8Input), _V, _U64, _V]),
    "qw38_q8_mlp_workspace_bytes": (_U64, [_U32]),
    "qw38_q4k_q8_mlp": (_I, [_P(Weight), _P(Weight), _P(Weight), _V, _V, _F, _V, _U32, _V, _U64,
                             _V, _P(_I), _V]),
    "qw38_q8_mlp_static_scratch_bytes": (_U64, []),
    "qw38_q4k_q8_mlp_static": (_I, [_P(Weight), _P(Weight), _P(Weight), _V, _V, _F, _V, _U32, _V,
                                    _P(_I), _V]),
    "qw38_hidden_rms_q8": (_I, [_V, _V, _F, _U32, _V, _V, _V, _V, _V]),
    "qw38_swiglu_q8": (_I, [_V, _V, _U32, _U32, _V, _V, _V, _V, _V]),
    "qw38_q8_group_dots": (_I, [_P(Weight), _P(Q8Input), _V, _U64, _V]),
    "qw38_repack_q4k_blocks": (_I, [_V, _U64, _U32, _U32, _U16, _V, _U64, _V, _U64, _V]),
    "qw38_repack_q6k_blocks": (_I, [_V, _U64, _U32, _U32, _V, _U64, _V, _U64, _V]),
    "qw38_quantize_q4k_blocks": (_I, [_V, _U64, _U32, _U32, _V, _U64, _V, _V]),
    "qw38_quantize_q6k_blocks": (_I, [_V, _U64, _U32, _U32, _V, _U64, _V]),
    "qw38_decode_mmv": (_I, [_P(DecodeDesc), _V]),
    "qw38_decode_mmv_paired": (_I, [_P(DecodeDesc), _P(DecodeDesc), _V]),
    "qw38_decode_mmv_ranges": (_I, [_P(DecodeDesc), _U32, _V]),
    "qw38_decode_ab_bf16": (_I, [_P(DecodeDesc), _P(DecodeDesc), _V]),
    "qw38_pack_fp8": (_I, [_V, _U64, _U32, _U32, _V, _U64, _V, _U64, _V]),
    "qw38_fp8_gemv": (_I, [_P(Fp8Weight), _V, _U64, _V, _U64, _V]),
    "qw38_fp8_gemm": (_I, [_P(Fp8Weight), _P(Fp8Input), _V, _U64, _V, _U64, _I, _V]),
    "qw38_fp8_store_bf16": (_I, [_V, _V, _U64, _V]),
    "qw38_fp8_project": (_I, [_P(Fp8Weight), _P(Fp8Input), _U32, _V, _V, _I, _V]),
    "qw38_pack_nvfp4": (_I, [_V, _U32, _U32, _V, _U64, _V, _U64, _V]),
    "qw38_hidden_rms_nvfp4": (_I, [_V, _V, _F, _U32, _V, _V, _V]),
    "qw38_hidden_rms_fp8": (_I, [_V, _V, _F, _U32, _V, _V, _V, _V]),
    "qw38_nvfp4_gemm_tile": (_I, [_V, _V, _V, _V, _U32, _U32, _U32, _U32, _V, _V]),
    "qw38_nvfp4_workspace_bytes": (_U64, [_U32]),
    "qw38_nvfp4_project": (_I, [_P(Weight), _V, _U32, _V, _V, _I, _V, _U64, _V]),
    "qw38_nvfp4_paired_swiglu": (_I, [_P(Weight), _P(Weight), _V, _V, _U32, _V, _U64, _V]),
    "qw38_fp8_prepare": (_I, [_V, _P(_I)]),
    "qw38_prefill_project": (_I, [_P(Weight), _V, _U32, _V, _V, _I, _V]),
    "qw38_prefill_paired_swiglu": (_I, [_P(Weight), _P(Weight), _V, _V, _U32, _V]),
    "qw38_hidden_rms_bf16": (_I, [_V, _V, _F, _U32, _V, _V]),
    "qw38_prefill_mlp_workspace_bytes": (_U64, [_U32]),
    "qw38_prefill_mlp": (_I, [_P(Weight), _P(Weight), _P(Weight), _V, _V, _F, _V, _U32, _V, _U64,
                              _V]),
    "qw38_mfma_clock_probe": (_I, [_U32, _V, _P(_U32), _V]),
    "qw38_read_probe": (_I, [_V, _U64, _U32, _U32, _V, _U64, _V]),
    "qw38_issue_probe": (_I, [_U32, _U32, _V, _V, _V]),
    "qw38_scratch_stats": (_I, [_V]),
    "qw38_set_profiling": (None, [_I]),
    "qw38_code_bytes": (_U64, [_U16, _U32, _U32]),
    "qw38_scale_bytes": (_U64, [_U16, _U32, _U32]),
    "qw38_device_malloc": (_I, [_P(_V), _U64]),
    "qw38_device_free": (_I, [_V, _U64]),
    "qw38_malloc_count": (_U64, []),
    "qw38_free_count": (_U64, []),
    "qw38_live_bytes": (_U64, []),
    "qw38_peak_live_bytes": (_U64, []),
    "qw38_record_malloc": (None, [_U64]),
    "qw38_record_free": (None, [_U64]),
}


def header_symbols() -> list[str]:
    """Every function the C header declares."""
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int|uint64_t|void)\s+(qw38_\w+)\s*\(", text, re.M)))


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: run __graft_entry__.build() "
                               "(hipcc for gfx950) first; there is no CPU fallback")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            f = getattr(L, name)
            f.restype, f.argtypes = res, args
        _lib = L
    return _lib


def last_error() -> Qw38Error:
    hip = C.c_int(0)
    op = C.create_string_buffer(96)
    detail = C.create_string_buffer(256)
    st = lib().qw38_last_error(C.byref(hip), op, 96, detail, 256)
    return Qw38Error(st, hip.value, op.value.decode(), detail.value.decode())


def check(status: int) -> None:
    if status != QW38_OK:
        raise last_error()
