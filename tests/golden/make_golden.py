"""Writes the committed golden fixtures under tests/golden/.

Run in a container where the reference tree is mounted and oracle/_ref is
built (``make -C oracle``): the expected bytes come from the reference's own
pinned llama.cpp Q4_K header compiled in place (oracle/_ref), never from the
oracle under test.

    python tests/golden/make_golden.py

Fixtures (numpy .npz, no pickles):
  q4k_ref_blocks.npz  inputs of tests/q4k_reference_test.cpp:126-165 (zero,
                      constants, asymmetric groups, outliers, subnormal scales,
                      256 heterogeneous BF16 blocks) and the pinned fitter's
                      144-byte blocks and dequantized values.
  fp16_ref.npz        FP32 -> FP16 encodings of an edge + random sweep and the
                      pinned nearest_int of a random sweep.
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402


def ref_blocks() -> np.ndarray:
    """The block inputs of tests/q4k_reference_test.cpp:126-165, restated."""
    cases = [np.zeros(256, np.float32)]
    for c in [1.0, -1.0, 0.03125, -0.03125, 1.0e-5, -1.0e-5, 1.0e-20, -1.0e-20, 1.0e-30, -1.0e-30]:
        cases.append(np.full(256, c, np.float32))
    i = np.arange(256)
    cases.append(((i % 32 - 7) * (1 + i // 32) / np.float32(19.0)).astype(np.float32))
    x = np.full(256, 0.01, np.float32)
    x[0], x[37], x[255] = -99.0, 127.0, -1.7
    cases.append(x)
    cases.append(((i % 32 - 9) * (1 + i // 32) * np.float32(2.0 ** -22)).astype(np.float32))
    state = 0x912782AC
    for block in range(256):
        x = np.zeros(256, np.float32)
        for j in range(256):
            state = (state * 1664525 + 1013904223) & 0xFFFFFFFF
            v = np.float32(((state >> 16) - 30000) / 16000.0)
            v = np.float32(np.ldexp(v, (j // 32 + block) % 16 - 12))
            x[j] = oracle.bf16_to_fp32(oracle.fp32_to_bf16(np.array([v], np.float32)))[0]
        cases.append(x)
    return np.stack(cases)


def main():
    R = oracle.ref()
    if R is None:
        raise SystemExit("oracle/_ref is not built (needs the reference tree): make -C oracle")
    x = ref_blocks()
    blocks = np.zeros((len(x), 144), np.uint8)
    deq = np.zeros_like(x)
    for b in range(len(x)):
        xb = np.ascontiguousarray(x[b])
        R.ref_quantize_row_q4_K(xb.ctypes.data, blocks[b].ctypes.data, 256)
        R.ref_dequantize_row_q4_K(blocks[b].ctypes.data, deq[b].ctypes.data, 256)
    np.savez_compressed(os.path.join(HERE, "q4k_ref_blocks.npz"), x=x, blocks=blocks, dequant=deq)

    rng = np.random.Generator(np.random.PCG64(2024))
    vals = (rng.standard_normal(4096) * np.float32(10.0) ** rng.integers(-9, 6, 4096)).astype(np.float32)
    edges = np.array([0.0, -0.0, 65504, 65519, 65520, 65536, 1e-8, 6e-8, 3e-8, 2.98e-8, 5.96e-8,
                      6.1035e-5, 6.1e-5, np.inf, -np.inf, np.nan, 1.0, -1.0, 0.5, 2049, 4097],
                     np.float32)
    allv = np.concatenate([edges, vals]).astype(np.float32)
    enc = np.array([R.ref_fp32_to_fp16(float(v)) for v in allv], np.uint16)
    ni_in = (rng.standard_normal(4096) * 1000).astype(np.float32)
    ni_in = np.concatenate([ni_in, np.array([0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 4194303.0], np.float32)])
    ni = np.array([R.ref_nearest_int(float(v)) for v in ni_in], np.int32)
    np.savez_compressed(os.path.join(HERE, "fp16_ref.npz"), f32=allv, f16=enc, ni_in=ni_in, ni=ni)
    print("wrote", os.listdir(HERE))


if __name__ == "__main__":
    main()
