"""qw38_amd: MI355X (gfx950) Q4_K_M x Q8 projection path of qw38.

The compute lives in ``libqw38_hip.so`` (hand-written HIP kernels behind the
C-ABI declared in ``include/qw38_hip.h``); ``qw38_amd.ops`` mirrors the
reference's operator interface over that ABI with torch device tensors.
"""
from ._lib import (LAYOUT_Q4K_SEQ, LAYOUT_Q4K_W64, LAYOUT_Q6K_W64, QUANTIZER_Q4K,  # noqa: F401
                   QUANTIZER_Q6K, Qw38Error, header_symbols, lib)
