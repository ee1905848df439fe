"""C-ABI surface on the CPU: the library loads, exports every symbol the header
declares, sizes agree with the layout definitions, and contract violations are
rejected before any device work (no GPU needed for those paths)."""
import ctypes as C
import re

import pytest

import qw38_amd
from qw38_amd import _lib


def test_library_exports_every_header_symbol():
    L = qw38_amd.lib()
    syms = _lib.header_symbols()
    assert len(syms) >= 18
    missing = [s for s in syms if not hasattr(L, s)]
    assert not missing, missing
    # and the ctypes binding covers exactly the header
    assert set(_lib.SIGNATURES) == set(syms)


def test_header_is_plain_c():
    text = open(_lib.HEADER).read()
    assert 'extern "C"' in text
    code = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    code = re.sub(r"//[^\n]*", "", code)
    for bad in ("torch", "std::", "hip_runtime", "namespace", "template", "class "):
        assert bad not in code


def test_layout_sizes():
    L = qw38_amd.lib()
    assert L.qw38_code_bytes(0x020D, 5120, 5120) == 5120 * 5120 // 2
    assert L.qw38_scale_bytes(0x020D, 5120, 5120) == 5120 * 20 * 16
    assert L.qw38_code_bytes(0x0240, 34816, 5120) == 34816 * 5120 // 2
    assert L.qw38_code_bytes(0x0241, 5120, 17408) == 5120 * 68 * 192
    assert L.qw38_scale_bytes(0x0241, 5120, 17408) == 5120 * 68 * 18
    assert L.qw38_code_bytes(0x0123, 8, 256) == 0
    # Q4_K: 144 B per 256 weights; Q6_K: 210 B per 256 weights
    assert (L.qw38_code_bytes(0x0240, 8, 256) + L.qw38_scale_bytes(0x0240, 8, 256)) == 8 * 144
    assert (L.qw38_code_bytes(0x0241, 8, 256) + L.qw38_scale_bytes(0x0241, 8, 256)) == 8 * 210
    # workspace formula of cuda/q4k_q8.hpp:28-30
    for m in (1, 7, 512):
        assert L.qw38_q8_mlp_workspace_bytes(m) == m * (17408 + 17408 // 32 * 8 + 2 * 17408 * 4) + 4


def _q8(m, k, pk, n_codes=None):
    return _lib.Q8Input(0x1000, m * pk if n_codes is None else n_codes, 0x2000, m * pk // 32,
                        0x3000, m * pk // 32, m, k, pk)


def test_prelaunch_rejections_without_device():
    L = qw38_amd.lib()
    q = _q8(3, 259, 512)
    bad_pk = _q8(3, 259, 256)
    flag = C.c_int(0)
    assert L.qw38_pack_q8(None, 3 * 259, C.byref(bad_pk), C.addressof(flag), 1, None) == 2
    assert L.qw38_pack_q8(None, 3 * 258, C.byref(q), C.addressof(flag), 1, None) == 2
    assert L.qw38_pack_q8(None, 3 * 259, C.byref(q), C.addressof(flag), 2, None) == 2
    err = _lib.last_error()
    assert err.status == 2 and err.operation == "q8.pack" and "geometry" in err.detail
    w = _lib.Weight(0x4000, 0x5000, 0x020D, 0x0105, 137, 259, 144, 512, 144 * 256, 144 * 2 * 16 - 1)
    assert L.qw38_q4k_q8_project(C.byref(w), C.byref(q), 0x6000, 3 * 137, None, 0, None) == 2
    assert _lib.last_error().operation == "q8.weight"
    w.scales_bytes += 1
    w.quantizer = 0x0140  # Q6_K quantizer with a Q4_K layout
    assert L.qw38_q4k_q8_project(C.byref(w), C.byref(q), 0x6000, 3 * 137, None, 0, None) == 2
    w.quantizer = 0x0105
    assert L.qw38_q4k_q8_project(C.byref(w), C.byref(q), 0x6000, 3 * 138, None, 0, None) == 2
    assert L.qw38_q4k_q8_project(C.byref(w), C.byref(q), 0x6000, 3 * 137, 0x7000, 1, None) == 2
    too_many = _q8(4097, 256, 256)
    w2 = _lib.Weight(0x4000, 0x5000, 0x020D, 0x0105, 8, 256, 8, 256, 8 * 128, 8 * 16)
    assert L.qw38_q4k_q8_project(C.byref(w2), C.byref(too_many), 0x6000, 4097 * 8, None, 0, None) == 2
    sub = C.c_int(7)
    g = _lib.Weight(0x4000, 0x5000, 0x020D, 0x0105, 17408, 5120, 17408, 5120, 0, 0)
    # pending_failure supplied: internal submission skips the capture query
    assert L.qw38_q4k_q8_mlp(C.byref(g), C.byref(g), C.byref(g), None, None, 1e-6, None, 0,
                             None, 0, None, C.byref(sub), C.addressof(flag)) == 2
    assert sub.value == 0, "submitted stays false on prelaunch rejection"
    assert L.qw38_hidden_rms_q8(None, None, float("nan"), 1, None, None, None, None, None) == 2
    assert L.qw38_swiglu_q8(None, None, 1, 300, None, None, None, None, None) == 2


def test_no_cpu_fallback_symbols():
    """The product library has no host compute path: no exported symbol names a
    CPU/host implementation of the contraction."""
    L = qw38_amd.lib()
    import subprocess
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True,
                         text=True).stdout
    exported = re.findall(r" T (qw38_\w+)", out)
    assert exported and all(not re.search(r"cpu|host|oracle", s) for s in exported)
    assert "orc_" not in out


def _decode_desc(n=40, k=512, epi=2):
    """A decode_mmv descriptor over fake (never dereferenced) addresses; only
    ever passed with one field broken, so validation rejects it before any
    device call."""
    pn, pk = (n + 7) // 8 * 8, (k + 255) // 256 * 256
    V = _lib.DecodeView
    d = _lib.DecodeDesc()
    d.layout, d.quantizer, d.activation_policy = 0x020D, 0x0105, 1
    d.n, d.k, d.padded_n, d.padded_k = n, k, pn, pk
    d.codes = V(0x100000, 1, 1, 0x020D, n, k, pn, pk, pn * pk // 2, 16, 0)
    units = pk // 256 * 8
    d.scales = V(0x200000, 1, 4, 0x020D, pn, units, pn, units, pn * pk // 256 * 16, 2, 0)
    d.input = V(0x300000, 1, 3, 0x0205, k, 1, k, 1, 2 * k, 2, 0)
    d.output = V(0x400000, 1, 5 if epi == 2 else 3, 0x020A if epi == 2 else 0x0205, n, 1, n, 1,
                 n * (4 if epi == 2 else 2), 4 if epi == 2 else 2, 1)
    d.epilogue = epi
    return d


def test_decode_rejections_without_device():
    L = qw38_amd.lib()
    cases = []
    d = _decode_desc(); d.quantizer = 0x0101; cases.append((d, "layout/quantizer"))
    d = _decode_desc(); d.scales.bytes //= 2; cases.append((d, "scales typed view"))
    d = _decode_desc(); d.padded_k = 768; cases.append((d, "padded N/K"))
    d = _decode_desc(k=300); cases.append((d, "quantizer group"))
    d = _decode_desc(k=17664); cases.append((d, "staging limit"))
    d = _decode_desc(); d.codes.alignment = 8; cases.append((d, "codes typed view"))
    d = _decode_desc(); d.output.writable = 0; cases.append((d, "output typed view"))
    d = _decode_desc(); d.input.pointer = 0x100010; cases.append((d, "overlap"))
    d = _decode_desc(); d.epilogue = 4; cases.append((d, "paired gate/up"))
    d = _decode_desc(); d.epilogue = 9; cases.append((d, "unknown epilogue"))
    d = _decode_desc(); d.activation_policy = 2; cases.append((d, "activation policy"))
    d = _decode_desc(); d.residual = d.output; cases.append((d, "must not supply residual"))
    for desc, needle in cases:
        assert L.qw38_decode_mmv(C.byref(desc), None) == 2, needle
        err = _lib.last_error()
        assert err.operation.startswith("decode_mmv") and needle in err.detail, (needle, err.detail)
    # NVFP4 V1 (4-bit codes, FP16-typed opaque scale span of 256 + 128-row
    # blocks x K/16 bytes): N beyond the model geometry is rejected
    # (cuda/decode_mmv.cu:391-393)
    n = 248328
    d = _decode_desc(n=n, k=256)
    d.layout, d.quantizer = 0x020E, 0x0106
    d.codes.layout, d.codes.dtype, d.codes.bytes = 0x020E, 6, n * 256 // 2
    units = (256 + (n + 127) // 128 * 128 * (256 // 16)) // 2
    d.scales = _lib.DecodeView(0x200000, 1, 4, 0x020E, 1, units, 1, units, 2 * units, 16, 0)
    assert L.qw38_decode_mmv(C.byref(d), None) == 2
    assert "NVFP4 N exceeds model geometry" in _lib.last_error().detail
    # FP8 V1 geometry contract (cuda/decode_mmv.cu:331-332)
    d = _decode_desc(n=120, k=256)
    d.layout, d.quantizer = 0x020F, 0x0107
    d.codes.layout, d.codes.dtype, d.codes.bytes = 0x020F, 7, 120 * 256
    assert L.qw38_decode_mmv(C.byref(d), None) == 2
    assert "FP8 requires aligned mixer geometry" in _lib.last_error().detail
    # FP8 entries reject bad geometry before touching memory
    fw = _lib.Fp8Weight(0x100000, 100, 0x200000, 1, 128, 128)  # codes_len != n*k
    assert L.qw38_fp8_gemv(C.byref(fw), C.c_void_p(0x300000), 128, C.c_void_p(0x400000), 128,
                           C.c_void_p(0x1)) == 2
    assert L.qw38_pack_fp8(C.c_void_p(0x100000), 10, 1, 11, C.c_void_p(0x200000), 0,
                           C.c_void_p(0x300000), 0, C.c_void_p(0x1)) == 2
    # FP8 prefill projection: prefill geometry (k % 256, cuda/prefill.cu:218-219),
    # operand m = tokens rounded up to 128, epilogue/residual pairing
    fw = _lib.Fp8Weight(0x100000, 128 * 128, 0x200000, 1, 128, 128)
    fx = _lib.Fp8Input(0x300000, 128 * 128, 0x400000, 128, 128, 128)
    assert L.qw38_fp8_project(C.byref(fw), C.byref(fx), 5, C.c_void_p(0x500000), None, 1, None) == 2
    assert "invalid geometry" in _lib.last_error().detail
    fw = _lib.Fp8Weight(0x100000, 128 * 256, 0x200000, 2, 128, 256)
    fx = _lib.Fp8Input(0x300000, 128 * 256, 0x400000, 256, 128, 256)
    assert L.qw38_fp8_project(C.byref(fw), C.byref(fx), 129, C.c_void_p(0x500000), None, 1, None) == 2
    assert L.qw38_fp8_project(C.byref(fw), C.byref(fx), 5, C.c_void_p(0x500000), None, 3, None) == 2
    assert "epilogue contract" in _lib.last_error().detail
    assert L.qw38_fp8_project(C.byref(fw), C.byref(fx), 5, C.c_void_p(0x500000),
                              C.c_void_p(0x600000), 2, None) == 2
    assert "epilogue contract" in _lib.last_error().detail
    # NVFP4 entries reject before touching memory
    # (cuda/nvfp4.cu:74-75, 87-90; cuda/prefill.cu:220-221)
    assert L.qw38_pack_nvfp4(C.c_void_p(0x100000), 0, 16, C.c_void_p(0x200000), 8,
                             C.c_void_p(0x300000), 2048, None) == 2
    assert L.qw38_pack_nvfp4(C.c_void_p(0x100000), 2, 256, C.c_void_p(0x200000), 255,
                             C.c_void_p(0x300000), 2048, None) == 2
    assert L.qw38_nvfp4_gemm_tile(C.c_void_p(0x100000), C.c_void_p(0x200000), C.c_void_p(0x300000),
                                  C.c_void_p(0x400000), 4, 12, 256, 0, C.c_void_p(0x500000), None) == 2
    assert "invalid tile" in _lib.last_error().detail
    assert L.qw38_nvfp4_gemm_tile(C.c_void_p(0x100000), C.c_void_p(0x200000), C.c_void_p(0x300000),
                                  C.c_void_p(0x400000), 4, 16, 256, 64, C.c_void_p(0x500000), None) == 2
    nw = _lib.Weight(0x100000, 0x200000, 0x020E, 0x0106, 16, 6144, 16, 6144, 16 * 6144 // 2,
                     256 + 128 * 6144 // 16)
    assert L.qw38_nvfp4_project(C.byref(nw), C.c_void_p(0x300000), 4, C.c_void_p(0x400000), None, 2,
                                C.c_void_p(0x500000), 1 << 20, None) == 2
    assert "weight, layout or token contract" in _lib.last_error().detail
    assert L.qw38_hidden_rms_nvfp4(C.c_void_p(0x100000), C.c_void_p(0x200000), -1.0, 4,
                                   C.c_void_p(0x300000), C.c_void_p(0x400000), None) == 2
    assert L.qw38_hidden_rms_fp8(C.c_void_p(0x100000), C.c_void_p(0x200000), 1e-6, 1025, None,
                                 C.c_void_p(0x300000), C.c_void_p(0x400000), None) == 2
    # a/b contraction: BF16 dense tiles with FP32 output only
    a, b = _decode_desc(), _decode_desc()
    assert L.qw38_decode_ab_bf16(C.byref(a), C.byref(b), None) == 2
    assert "cuda_bf16_dense_tile_v0" in _lib.last_error().detail
    # paired: B must match A; SwiGLU B declares no output
    a, b = _decode_desc(), _decode_desc()
    b.codes.pointer, b.scales.pointer, b.output.pointer = 0x500000, 0x600000, 0x700000
    b.k = 256
    assert L.qw38_decode_mmv_paired(C.byref(a), C.byref(b), None) == 2
    a, b = _decode_desc(epi=4), _decode_desc(epi=4)
    b.codes.pointer, b.scales.pointer = 0x500000, 0x600000
    assert L.qw38_decode_mmv_paired(C.byref(a), C.byref(b), None) == 2
    assert "separately materialized" in _lib.last_error().detail
    # ranges: count and BF16 store contract
    arr = (_lib.DecodeDesc * 1)(_decode_desc(epi=1))
    assert L.qw38_decode_mmv_ranges(arr, 1, None) == 2
    arr = (_lib.DecodeDesc * 2)(_decode_desc(epi=2), _decode_desc(epi=2))
    assert L.qw38_decode_mmv_ranges(arr, 2, None) == 2
    assert "store BF16" in _lib.last_error().detail
