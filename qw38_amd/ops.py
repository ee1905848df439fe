"""Python mirror of the reference operator interface for the Q4_K_M x Q8 path.

Names, argument meaning and error behaviour follow ``cuda/q4k_q8.hpp`` (pack_q8,
q4k_q8_project, q4k_q8_mlp) and ``cuda/activation.hpp`` (launch_hidden_rms_q8)
of the reference; device memory and streams come from torch (plumbing only).
Every call goes through the C-ABI of ``libqw38_hip.so``; errors raise
``Qw38Error`` carrying the reference's error code names.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import torch

from ._lib import (LAYOUT_Q4K_SEQ, LAYOUT_Q4K_W64, LAYOUT_Q6K_W64, QUANTIZER_Q4K, QUANTIZER_Q6K,
                   Q8Input as _Q8, Weight as _W, check, lib)

__all__ = ["PrefillWeight", "Q8Input", "pack_q8", "q4k_q8_project", "q4k_q8_mlp", "q4k_q8_gate_up_swiglu",
           "hidden_rms_q8", "swiglu_q8", "group_dots", "quantize_q4k_blocks", "quantize_q6k_blocks", "upload_q4k_blocks", "upload_q6k_blocks",
           "q8_mlp_workspace_bytes", "code_bytes", "scale_bytes", "pad_k", "pad_n",
           "decode_view", "decode_desc", "decode_mmv", "decode_mmv_paired", "decode_mmv_ranges",
           "prefill_project", "prefill_paired_swiglu", "hidden_rms_bf16", "prefill_mlp",
           "prefill_mlp_workspace_bytes"]


def pad_k(k: int) -> int:
    return (k + 255) // 256 * 256


def pad_n(n: int) -> int:
    return (n + 7) // 8 * 8


def code_bytes(layout: int, padded_n: int, padded_k: int) -> int:
    return int(lib().qw38_code_bytes(layout, padded_n, padded_k))


def scale_bytes(layout: int, padded_n: int, padded_k: int) -> int:
    return int(lib().qw38_scale_bytes(layout, padded_n, padded_k))


def _stream(stream) -> int:
    if stream is None:
        return torch.cuda.current_stream().cuda_stream
    if isinstance(stream, torch.cuda.Stream):
        return stream.cuda_stream
    return int(stream)


def _ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


@dataclass
class PrefillWeight:
    """Device-resident tiled weight: cuda::PrefillWeight (cuda/prefill.hpp:33-44)."""
    codes: torch.Tensor
    scales: torch.Tensor
    layout: int
    quantizer: int
    n: int
    k: int
    padded_n: int
    padded_k: int
    codes_bytes: int = -1
    scales_bytes: int = -1
    codes_ptr: int | None = None  # explicit (possibly offset) pointer override

    def __post_init__(self):
        if self.codes_bytes < 0:
            self.codes_bytes = self.codes.numel() * self.codes.element_size()
        if self.scales_bytes < 0:
            self.scales_bytes = (0 if self.scales is None else
                                 self.scales.numel() * self.scales.element_size())

    @staticmethod
    def from_bytes(codes, scales, layout, n, k, device="cuda"):
        """From host byte arrays (numpy uint8) of an already tiled layout."""
        q = QUANTIZER_Q6K if layout == LAYOUT_Q6K_W64 else QUANTIZER_Q4K
        c = torch.from_numpy(codes).to(device)
        s = torch.from_numpy(scales).to(device)
        return PrefillWeight(c, s, layout, q, n, k, pad_n(n), pad_k(k))

    def struct(self) -> _W:
        return _W(self.codes_ptr if self.codes_ptr is not None else self.codes.data_ptr(),
                  self.scales.data_ptr(), self.layout, self.quantizer, self.n, self.k,
                  self.padded_n, self.padded_k, self.codes_bytes, self.scales_bytes)


@dataclass
class Q8Input:
    """Q8 K32 activation pack: cuda::Q8Input (cuda/q4k_q8.hpp:16-21)."""
    codes: torch.Tensor   # int8 [m][padded_k]
    scales: torch.Tensor  # float32 [m][padded_k/32]
    sums: torch.Tensor    # int32 [m][padded_k/32]
    m: int
    k: int
    padded_k: int
    codes_ptr: int | None = None
    codes_len: int | None = None

    @staticmethod
    def empty(m: int, k: int, device="cuda") -> "Q8Input":
        pk = pad_k(k)
        return Q8Input(torch.zeros(m, pk, dtype=torch.int8, device=device),
                       torch.zeros(m, pk // 32, dtype=torch.float32, device=device),
                       torch.zeros(m, pk // 32, dtype=torch.int32, device=device), m, k, pk)

    def struct(self) -> _Q8:
        n = self.codes_len if self.codes_len is not None else self.codes.numel()
        return _Q8(self.codes_ptr if self.codes_ptr is not None else self.codes.data_ptr(), n,
                   self.scales.data_ptr(), self.scales.numel(), self.sums.data_ptr(),
                   self.sums.numel(), self.m, self.k, self.padded_k)


def pack_q8(input_bf16: torch.Tensor, output: Q8Input, failure: torch.Tensor, stream=None):
    """cuda::pack_q8 (cuda/q4k_q8.cu:318-330). input_bf16: int16/uint16 bits [m][k]."""
    q = output.struct()
    check(lib().qw38_pack_q8(_ptr(input_bf16), input_bf16.numel(), C.byref(q), _ptr(failure),
                             failure.numel(), _stream(stream)))


def q4k_q8_project(weight: PrefillWeight, x: Q8Input, output: torch.Tensor, stream=None,
                   residual: torch.Tensor | None = None, output_ptr=None, output_len=None):
    """cuda::q4k_q8_project (cuda/q4k_q8.cu:332-345)."""
    w, q = weight.struct(), x.struct()
    optr = output_ptr if output_ptr is not None else output.data_ptr()
    olen = output_len if output_len is not None else output.numel()
    check(lib().qw38_q4k_q8_project(C.byref(w), C.byref(q), optr, olen, _ptr(residual),
                                    0 if residual is None else residual.numel(), _stream(stream)))


def q4k_q8_gate_up_swiglu(gate: PrefillWeight, up: PrefillWeight, x: Q8Input, out: Q8Input,
                          failure: torch.Tensor, stream=None):
    """Fused gate + up projections with the SwiGLU->Q8 epilogue: ``out`` is the
    down projection's Q8 operand (cuda/q4k_q8.cu:378-385 as one launch)."""
    g, u, q, o = gate.struct(), up.struct(), x.struct(), out.struct()
    check(lib().qw38_q4k_q8_gate_up_swiglu(C.byref(g), C.byref(u), C.byref(q), C.byref(o),
                                           _ptr(failure), failure.numel(), _stream(stream)))


def scratch_stats() -> tuple[int, int, int]:
    """Library scratch requests on the current device since the process
    started: (granted, refused for size, refused because in use)."""
    st = (C.c_uint64 * 3)()
    check(lib().qw38_scratch_stats(st))
    return int(st[0]), int(st[1]), int(st[2])


def q8_mlp_workspace_bytes(m: int) -> int:
    return int(lib().qw38_q8_mlp_workspace_bytes(m))


def q4k_q8_mlp(gate: PrefillWeight, up: PrefillWeight, down: PrefillWeight,
               residual: torch.Tensor, gamma: torch.Tensor, eps: float, output: torch.Tensor,
               m: int, workspace: torch.Tensor, stream=None, pending_failure=None) -> bool:
    """cuda::q4k_q8_mlp (cuda/q4k_q8.cu:347-398). Returns ``submitted``."""
    g, u, d = gate.struct(), up.struct(), down.struct()
    submitted = C.c_int(0)
    st = lib().qw38_q4k_q8_mlp(C.byref(g), C.byref(u), C.byref(d), _ptr(residual), _ptr(gamma),
                               eps, _ptr(output), m, _ptr(workspace), workspace.numel(),
                               _stream(stream), C.byref(submitted), _ptr(pending_failure))
    if st:
        err = __import__("qw38_amd._lib", fromlist=["last_error"]).last_error()
        err.submitted = bool(submitted.value)
        raise err
    return bool(submitted.value)


def hidden_rms_q8(residual, gamma, eps, m, out: Q8Input, failure, stream=None):
    """launch_hidden_rms_q8 (cuda/activation.cu:536-548)."""
    check(lib().qw38_hidden_rms_q8(_ptr(residual), _ptr(gamma), eps, m, _ptr(out.codes),
                                   _ptr(out.scales), _ptr(out.sums), _ptr(failure),
                                   _stream(stream)))


def swiglu_q8(gate, up, m, n, out: Q8Input, failure, stream=None):
    """The SwiGLU->Q8 producer of q4k_q8_mlp (cuda/q4k_q8.cu:52-61)."""
    check(lib().qw38_swiglu_q8(_ptr(gate), _ptr(up), m, n, _ptr(out.codes), _ptr(out.scales),
                               _ptr(out.sums), _ptr(failure), _stream(stream)))


def group_dots(weight: PrefillWeight, x: Q8Input, dots: torch.Tensor, stream=None):
    w, q = weight.struct(), x.struct()
    check(lib().qw38_q8_group_dots(C.byref(w), C.byref(q), _ptr(dots), dots.numel(),
                                   _stream(stream)))


def upload_q4k_blocks(blocks: torch.Tensor, n: int, k: int, layout=LAYOUT_Q4K_W64,
                      stream=None) -> PrefillWeight:
    """Load-time repack of GGML Q4_K super-blocks (uint8 device tensor)."""
    pn, pk = pad_n(n), pad_k(k)
    codes = torch.empty(code_bytes(layout, pn, pk), dtype=torch.uint8, device=blocks.device)
    scales = torch.empty(scale_bytes(layout, pn, pk), dtype=torch.uint8, device=blocks.device)
    check(lib().qw38_repack_q4k_blocks(_ptr(blocks), blocks.numel(), n, k, layout, _ptr(codes),
                                       codes.numel(), _ptr(scales), scales.numel(),
                                       _stream(stream)))
    return PrefillWeight(codes, scales, layout, QUANTIZER_Q4K, n, k, pn, pk)


def quantize_q4k_blocks(x: torch.Tensor, n: int, k: int, failure: torch.Tensor,
                        stream=None) -> torch.Tensor:
    """FP32 rows [n][k] on the device -> GGML Q4_K super-blocks (uint8)."""
    blocks = torch.empty(n * (k // 256) * 144, dtype=torch.uint8, device=x.device)
    check(lib().qw38_quantize_q4k_blocks(_ptr(x), x.numel(), n, k, _ptr(blocks), blocks.numel(),
                                         _ptr(failure), _stream(stream)))
    return blocks


def quantize_q6k_blocks(x: torch.Tensor, n: int, k: int, stream=None) -> torch.Tensor:
    """FP32 rows [n][k] on the device -> GGML Q6_K super-blocks (uint8)."""
    blocks = torch.empty(n * (k // 256) * 210, dtype=torch.uint8, device=x.device)
    check(lib().qw38_quantize_q6k_blocks(_ptr(x), x.numel(), n, k, _ptr(blocks), blocks.numel(),
                                         _stream(stream)))
    return blocks


def upload_q6k_blocks(blocks: torch.Tensor, n: int, k: int, stream=None) -> PrefillWeight:
    """Load-time repack of GGML Q6_K super-blocks (uint8 device tensor)."""
    pn, pk = pad_n(n), pad_k(k)
    codes = torch.empty(code_bytes(LAYOUT_Q6K_W64, pn, pk), dtype=torch.uint8, device=blocks.device)
    scales = torch.empty(scale_bytes(LAYOUT_Q6K_W64, pn, pk), dtype=torch.uint8, device=blocks.device)
    check(lib().qw38_repack_q6k_blocks(_ptr(blocks), blocks.numel(), n, k, _ptr(codes),
                                       codes.numel(), _ptr(scales), scales.numel(),
                                       _stream(stream)))
    return PrefillWeight(codes, scales, LAYOUT_Q6K_W64, QUANTIZER_Q6K, n, k, pn, pk)


# ---- BF16-activation decode GEMV (cuda/decode_mmv.hpp) ----------------------
DECODE_STORE_BF16, DECODE_STORE_FP32, DECODE_RESIDUAL_ADD_FP32, DECODE_SWIGLU_BF16 = 1, 2, 3, 4
DTYPE_Q4, DTYPE_Q8, DTYPE_BF16, DTYPE_FP16, DTYPE_FP32 = 1, 2, 3, 4, 5
LAYOUT_BF16_VECTOR, LAYOUT_FP32_VECTOR = 0x0205, 0x020A


def decode_view(t, dtype, layout, logical_n, logical_k, padded_n, padded_k, alignment,
                writable, nbytes=None):
    """cuda::decode_matrix_view / decode_vector_view (cuda/decode_mmv.hpp:95-112)."""
    from ._lib import DecodeView
    if t is None:
        return DecodeView()
    b = t.numel() * t.element_size() if nbytes is None else nbytes
    return DecodeView(t.data_ptr(), 1, dtype, layout, logical_n, logical_k, padded_n, padded_k,
                      b, alignment, 1 if writable else 0)


DECODE_LAYOUT_Q4G64, DECODE_LAYOUT_Q8G32, DECODE_LAYOUT_BF16_TILE = 0x0201, 0x0202, 0x0203
DECODE_LAYOUT_Q4G64_CAND, DECODE_LAYOUT_Q8G32_CAND = 0x020B, 0x020C
_DENSE_QUANTIZER = {0x0201: 0x0101, 0x0202: 0x0102, 0x0203: 0x0100, 0x020B: 0x0103, 0x020C: 0x0104}


def dense_weight(layout: int, codes: torch.Tensor, scales, n: int, k: int) -> PrefillWeight:
    """A decode_mmv weight in one of the reference's dense tile layouts
    (Q4G64, Q8G32, BF16 dense tile; cuda/decode_mmv.hpp:25-35): device byte
    tensors already in the tile order, scales None for BF16."""
    return PrefillWeight(codes, scales, layout, _DENSE_QUANTIZER[layout], n, k, pad_n(n), pad_k(k))


def _weight_dtype(layout: int) -> int:
    if layout in (0x0202, 0x020C):
        return DTYPE_Q8
    if layout == 0x0203:
        return DTYPE_BF16
    return DTYPE_Q4


def decode_desc(w: PrefillWeight, x, output, epilogue=DECODE_STORE_FP32, residual=None,
                output_view=True):
    """A DecodeMmvDesc for a decode weight (Q4_K 0x020D or a dense layout), BF16
    input x [k] (int16 tensor of BF16 bits), output [n] (FP32, or BF16 bits
    for the BF16 epilogues) and residual [n] FP32 for the residual epilogue.
    With output=None and the residual epilogue the update is in place."""
    from ._lib import DecodeDesc
    d = DecodeDesc()
    d.layout, d.quantizer, d.activation_policy = w.layout, w.quantizer, 1
    d.n, d.k, d.padded_n, d.padded_k = w.n, w.k, w.padded_n, w.padded_k
    d.codes = decode_view(w.codes, _weight_dtype(w.layout), w.layout, w.n, w.k, w.padded_n,
                          w.padded_k, 16, False)
    if w.scales is not None:
        units = w.scales.numel() * w.scales.element_size() // w.padded_n // 2
        d.scales = decode_view(w.scales, DTYPE_FP16, w.layout, w.padded_n, units, w.padded_n,
                               units, 2, False)
    d.input = decode_view(x, DTYPE_BF16, LAYOUT_BF16_VECTOR, w.k, 1, w.k, 1, 2, False)
    bf16_out = epilogue in (DECODE_STORE_BF16, DECODE_SWIGLU_BF16)
    if output is not None and output_view:
        d.output = decode_view(output, DTYPE_BF16 if bf16_out else DTYPE_FP32,
                               LAYOUT_BF16_VECTOR if bf16_out else LAYOUT_FP32_VECTOR, w.n, 1, w.n,
                               1, 2 if bf16_out else 4, True)
    if residual is not None:
        d.residual = decode_view(residual, DTYPE_FP32, LAYOUT_FP32_VECTOR, w.n, 1, w.n, 1, 4,
                                 output is None)
    d.epilogue = epilogue
    d._tensors = (w.codes, w.scales, x, output, residual)  # the views hold raw pointers
    return d


def decode_mmv(desc, stream=None) -> None:
    """cuda::launch_decode_mmv (cuda/decode_mmv.hpp:205-206)."""
    check(lib().qw38_decode_mmv(C.byref(desc), _stream(stream)))


def decode_mmv_paired(a, b, stream=None) -> None:
    """cuda::launch_decode_mmv_paired (cuda/decode_mmv.hpp:208-209)."""
    check(lib().qw38_decode_mmv_paired(C.byref(a), C.byref(b), _stream(stream)))


def decode_ab_bf16(a, b, stream=None) -> None:
    """cuda::launch_decode_ab_bf16 (cuda/decode_mmv.hpp:211-213)."""
    check(lib().qw38_decode_ab_bf16(C.byref(a), C.byref(b), _stream(stream)))


def decode_mmv_ranges(descs, stream=None) -> None:
    """cuda::launch_decode_mmv_ranges (cuda/decode_mmv.hpp:216-217)."""
    from ._lib import DecodeDesc
    arr = (DecodeDesc * len(descs))(*descs)
    check(lib().qw38_decode_mmv_ranges(arr, len(descs), _stream(stream)))


# ---- FP8 (OCP E4M3FN) projections (cuda/fp8.hpp) ----------------------------
DECODE_LAYOUT_FP8, DECODE_QUANTIZER_FP8, DTYPE_FP8 = 0x020F, 0x0107, 7


def _pad128(v: int) -> int:
    return (v + 127) // 128 * 128


def fp8_weight_struct(codes, scales, n: int, k: int):
    """cuda::Fp8Weight over device tensors: codes uint8 [n][k], scales FP32 [k/128][n/128]."""
    from ._lib import Fp8Weight
    w = Fp8Weight(codes.data_ptr(), codes.numel(), scales.data_ptr(), scales.numel(), n, k)
    w._tensors = (codes, scales)  # the struct holds raw pointers: keep the storage alive with it
    return w


def fp8_input_struct(codes, scales, m: int, k: int):
    """cuda::Fp8Input over device tensors: codes uint8 [m][k], scales FP32 [k/128][m]."""
    from ._lib import Fp8Input
    x = Fp8Input(codes.data_ptr(), codes.numel(), scales.data_ptr(), scales.numel(), m, k)
    x._tensors = (codes, scales)
    return x


def pack_fp8(x, m: int, k: int, codes=None, scales=None, stream=None):
    """cuda::pack_fp8: BF16 bits [m][k] (int16 tensor) -> (codes [pm][pk], scales [pk/128][pm])."""
    pm, pk = _pad128(m), _pad128(k)
    if codes is None:
        codes = torch.empty(pm, pk, dtype=torch.uint8, device=x.device)
    if scales is None:
        scales = torch.empty(pk // 128, pm, dtype=torch.float32, device=x.device)
    check(lib().qw38_pack_fp8(x.data_ptr(), x.numel(), m, k, codes.data_ptr(), codes.numel(),
                              scales.data_ptr(), scales.numel(), _stream(stream)))
    return codes, scales


def fp8_gemv(w, x, y, stream=None) -> None:
    """cuda::fp8_gemv: w a qw38_fp8_weight, x BF16 bits [k], y FP32 [n]."""
    check(lib().qw38_fp8_gemv(C.byref(w), x.data_ptr(), x.numel(), y.data_ptr(), y.numel(),
                              _stream(stream)))


def fp8_gemm(w, xin, y, workspace, sm_count: int, stream=None) -> None:
    """cuda::fp8_gemm: y FP32 [m][n] from packed operands."""
    check(lib().qw38_fp8_gemm(C.byref(w), C.byref(xin), y.data_ptr(), y.numel(), workspace.data_ptr(),
                              workspace.numel() * workspace.element_size(), sm_count, _stream(stream)))


def fp8_project(w, xin, tokens: int, output, epilogue=DECODE_STORE_BF16, residual=None,
                stream=None) -> None:
    """PrefillEngine::project FP8 branch for M > 1 (cuda/prefill.cu:565-593):
    output [tokens][n] through the fused GEMM epilogue."""
    check(lib().qw38_fp8_project(C.byref(w), C.byref(xin), tokens, output.data_ptr(),
                                 _ptr(residual), epilogue, _stream(stream)))


def fp8_store_bf16(x, y, stream=None) -> None:
    """cuda::fp8_store_bf16: FP32 -> BF16 bits, round to nearest even."""
    check(lib().qw38_fp8_store_bf16(x.data_ptr(), y.data_ptr(), x.numel(), _stream(stream)))


def fp8_prepare(stream=None) -> int:
    """cuda::prepare_fp8_gemm: compute units of the stream's device."""
    v = C.c_int(0)
    check(lib().qw38_fp8_prepare(_stream(stream), C.byref(v)))
    return v.value


def fp8_decode_desc(codes, scales, n: int, k: int, x, output, epilogue=DECODE_STORE_FP32,
                    residual=None):
    """A DecodeMmvDesc over an FP8 weight (layout 0x020F): codes uint8 [n][k],
    scales FP32 [k/128][n/128] (cuda/prefill.cu:236-246)."""
    from ._lib import DecodeDesc
    d = DecodeDesc()
    d.layout, d.quantizer, d.activation_policy = DECODE_LAYOUT_FP8, DECODE_QUANTIZER_FP8, 1
    d.n, d.k, d.padded_n, d.padded_k = n, k, pad_n(n), pad_k(k)
    d.codes = decode_view(codes, DTYPE_FP8, DECODE_LAYOUT_FP8, n, k, pad_n(n), pad_k(k), 16, False)
    units = scales.numel()
    d.scales = decode_view(scales, DTYPE_FP32, DECODE_LAYOUT_FP8, 1, units, 1, units, 16, False)
    d.input = decode_view(x, DTYPE_BF16, LAYOUT_BF16_VECTOR, k, 1, k, 1, 2, False)
    bf16_out = epilogue == DECODE_STORE_BF16
    if output is not None:
        d.output = decode_view(output, DTYPE_BF16 if bf16_out else DTYPE_FP32,
                               LAYOUT_BF16_VECTOR if bf16_out else LAYOUT_FP32_VECTOR, n, 1, n, 1,
                               2 if bf16_out else 4, True)
    if residual is not None:
        d.residual = decode_view(residual, DTYPE_FP32, LAYOUT_FP32_VECTOR, n, 1, n, 1, 4,
                                 output is None)
    d.epilogue = epilogue
    d._tensors = (codes, scales, x, output, residual)  # the views hold raw pointers
    return d


# ---- NVFP4 (cuda/nvfp4.hpp) ---------------------------------------------------
DECODE_LAYOUT_NVFP4, DECODE_QUANTIZER_NVFP4, DTYPE_NVFP4 = 0x020E, 0x0106, 6


def nvfp4_scale_count(rows: int, pk: int) -> int:
    """Swizzled scale bytes of `rows` rows (src/format/nvfp4.hpp:12-14)."""
    return _pad128(rows) * (pk // 16)


def pack_nvfp4(x, m: int, k: int, codes=None, scales=None, stream=None):
    """launch_pack_nvfp4: BF16 bits [m][k] -> (codes uint8 [m][pk/2], swizzled scales)."""
    pk = pad_k(k)
    if codes is None:
        codes = torch.zeros(m, pk // 2, dtype=torch.uint8, device=x.device)
    if scales is None:
        scales = torch.zeros(nvfp4_scale_count(m, pk), dtype=torch.uint8, device=x.device)
    check(lib().qw38_pack_nvfp4(x.data_ptr(), m, k, codes.data_ptr(), codes.numel(),
                                scales.data_ptr(), scales.numel(), _stream(stream)))
    return codes, scales


def hidden_rms_nvfp4(residual, gamma, eps, m, codes, scales, stream=None) -> None:
    """launch_hidden_rms_nvfp4 (cuda/activation.cu:507-520)."""
    check(lib().qw38_hidden_rms_nvfp4(residual.data_ptr(), gamma.data_ptr(), eps, m,
                                      codes.data_ptr(), scales.data_ptr(), _stream(stream)))


def hidden_rms_fp8(residual, gamma, eps, m, codes, scales, companion=None, stream=None) -> None:
    """launch_hidden_rms_fp8 (cuda/activation.cu:522-534)."""
    check(lib().qw38_hidden_rms_fp8(residual.data_ptr(), gamma.data_ptr(), eps, m, _ptr(companion),
                                    codes.data_ptr(), scales.data_ptr(), _stream(stream)))


def nvfp4_gemm_tile(codes, scales, act, act_scales, m, n, k, row_start, out, stream=None) -> None:
    """nvfp4_gemm_tile (cuda/nvfp4.cu:83-116): out FP32 [m][n]."""
    check(lib().qw38_nvfp4_gemm_tile(codes.data_ptr(), scales.data_ptr(), act.data_ptr(),
                                     act_scales.data_ptr(), m, n, k, row_start, out.data_ptr(),
                                     _stream(stream)))


def nvfp4_weight(codes, scales, n: int, k: int) -> PrefillWeight:
    """A PrefillWeight over an NVFP4 payload (layout 0x020E)."""
    return PrefillWeight(codes, scales, DECODE_LAYOUT_NVFP4, DECODE_QUANTIZER_NVFP4, n, k,
                         pad_n(n), pad_k(k))


def nvfp4_workspace_bytes(tokens: int) -> int:
    return int(lib().qw38_nvfp4_workspace_bytes(tokens))


def nvfp4_project(w: PrefillWeight, x, tokens: int, output, workspace, epilogue=DECODE_STORE_FP32,
                  residual=None, stream=None) -> None:
    """NVFP4 branch of PrefillEngine::project (cuda/prefill.cu:598-628)."""
    ws = w.struct()
    check(lib().qw38_nvfp4_project(C.byref(ws), x.data_ptr(), tokens, output.data_ptr(),
                                   _ptr(residual), epilogue, workspace.data_ptr(), workspace.numel(),
                                   _stream(stream)))


def nvfp4_paired_swiglu(gate: PrefillWeight, up: PrefillWeight, x, swiglu, tokens: int, workspace,
                        stream=None) -> None:
    """NVFP4 branch of PrefillEngine::paired_swiglu (cuda/prefill.cu:680-715)."""
    g, u = gate.struct(), up.struct()
    check(lib().qw38_nvfp4_paired_swiglu(C.byref(g), C.byref(u), x.data_ptr(), swiglu.data_ptr(),
                                         tokens, workspace.data_ptr(), workspace.numel(),
                                         _stream(stream)))


def nvfp4_decode_desc(w: PrefillWeight, x, output, epilogue=DECODE_STORE_FP32, residual=None):
    """A DecodeMmvDesc over an NVFP4 weight (cuda/prefill.cu:236-246): scales
    are an FP16-typed opaque span of one row."""
    from ._lib import DecodeDesc
    d = DecodeDesc()
    d.layout, d.quantizer, d.activation_policy = DECODE_LAYOUT_NVFP4, DECODE_QUANTIZER_NVFP4, 1
    d.n, d.k, d.padded_n, d.padded_k = w.n, w.k, w.padded_n, w.padded_k
    d.codes = decode_view(w.codes, DTYPE_NVFP4, DECODE_LAYOUT_NVFP4, w.n, w.k, w.padded_n,
                          w.padded_k, 16, False)
    units = w.scales.numel() // 2
    d.scales = decode_view(w.scales, DTYPE_FP16, DECODE_LAYOUT_NVFP4, 1, units, 1, units, 16, False)
    d.input = decode_view(x, DTYPE_BF16, LAYOUT_BF16_VECTOR, w.k, 1, w.k, 1, 2, False)
    bf16_out = epilogue in (DECODE_STORE_BF16, DECODE_SWIGLU_BF16)
    if output is not None:
        d.output = decode_view(output, DTYPE_BF16 if bf16_out else DTYPE_FP32,
                               LAYOUT_BF16_VECTOR if bf16_out else LAYOUT_FP32_VECTOR, w.n, 1, w.n,
                               1, 2 if bf16_out else 4, True)
    if residual is not None:
        d.residual = decode_view(residual, DTYPE_FP32, LAYOUT_FP32_VECTOR, w.n, 1, w.n, 1, 4,
                                 output is None)
    d.epilogue = epilogue
    d._tensors = (w.codes, w.scales, x, output, residual)
    return d


# ---- BF16 prefill projections (cuda/prefill.hpp) ----------------------------
def prefill_project(w: PrefillWeight, x, tokens: int, output, epilogue=DECODE_STORE_FP32,
                    residual=None, stream=None) -> None:
    """PrefillEngine::project for Q4_K: x BF16 bits [tokens][k] -> output."""
    check(lib().qw38_prefill_project(C.byref(w.struct()), x.data_ptr(), tokens, output.data_ptr(),
                                     _ptr(residual), epilogue, _stream(stream)))


def prefill_paired_swiglu(gate: PrefillWeight, up: PrefillWeight, normalized, swiglu, tokens,
                          stream=None) -> None:
    """PrefillEngine::paired_swiglu: BF16(SiLU(X gate^T) * (X up^T))."""
    check(lib().qw38_prefill_paired_swiglu(C.byref(gate.struct()), C.byref(up.struct()),
                                           normalized.data_ptr(), swiglu.data_ptr(), tokens,
                                           _stream(stream)))


def hidden_rms_bf16(residual, gamma, eps, m, output, stream=None) -> None:
    """launch_hidden_rms: RMS over hidden 5120 -> BF16 [m][5120]."""
    check(lib().qw38_hidden_rms_bf16(residual.data_ptr(), gamma.data_ptr(), float(eps), m,
                                     output.data_ptr(), _stream(stream)))


def prefill_mlp_workspace_bytes(tokens: int) -> int:
    return int(lib().qw38_prefill_mlp_workspace_bytes(tokens))


def prefill_mlp(gate, up, down, h_mid, gamma, eps, next_h, tokens, workspace, stream=None):
    """PrefillEngine::mlp: RMS -> BF16 -> paired SwiGLU -> down + residual."""
    check(lib().qw38_prefill_mlp(C.byref(gate.struct()), C.byref(up.struct()), C.byref(down.struct()),
                                 h_mid.data_ptr(), gamma.data_ptr(), float(eps), next_h.data_ptr(),
                                 tokens, workspace.data_ptr(), workspace.numel(), _stream(stream)))
