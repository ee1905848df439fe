"""GPU fitter and load-time repack: bytes equal the oracle's (which is pinned to
the reference's llama.cpp Q4_K fitter), repack is lossless for every layout."""
import numpy as np
import pytest

import oracle
from _fix import ggml_q6k_decode, normal

pytestmark = pytest.mark.gpu


def test_gpu_q4k_fitter_bit_exact(torch_gpu):
    torch = torch_gpu
    import qw38_amd.ops as ops
    for (n, k, seed, scale) in [(64, 512, 3, 0.02), (40, 1024, 4, 1.0), (8, 256, 5, 1e-3)]:
        print(f"fit q4k n={n} k={k}", flush=True)
        x = normal((n, k), seed, scale)
        x[0, :256] = 0.0                   # zero block
        x[1, :256] = 0.03125               # constant block
        fail = torch.zeros(1, dtype=torch.int32, device="cuda")
        blocks = ops.quantize_q4k_blocks(torch.from_numpy(x).cuda(), n, k, fail)
        torch.cuda.synchronize()
        assert int(fail.item()) == 0
        ref = oracle.quantize_q4k(x).ggml()
        assert np.array_equal(blocks.cpu().numpy(), ref)


def test_gpu_q4k_fitter_rejects_nonfinite(torch_gpu):
    torch = torch_gpu
    import qw38_amd.ops as ops
    x = normal((8, 256), 9)
    x[3, 7] = np.inf
    fail = torch.zeros(1, dtype=torch.int32, device="cuda")
    ops.quantize_q4k_blocks(torch.from_numpy(x).cuda(), 8, 256, fail)
    torch.cuda.synchronize()
    assert int(fail.item()) == 1


def test_gpu_q6k_fitter_matches_oracle(torch_gpu):
    torch = torch_gpu
    import qw38_amd.ops as ops
    n, k = 48, 768
    x = normal((n, k), 13, 0.02)
    x[0, :256] = 0.0
    blocks = ops.quantize_q6k_blocks(torch.from_numpy(x).cuda(), n, k)
    torch.cuda.synchronize()
    assert np.array_equal(blocks.cpu().numpy(), oracle.quantize_q6k(x).ggml())


@pytest.mark.parametrize("layout", [oracle.LAYOUT_Q4K_SEQ, oracle.LAYOUT_Q4K_W64])
def test_repack_q4k(torch_gpu, layout):
    torch = torch_gpu
    import qw38_amd.ops as ops
    n, k = 37, 768                      # ragged N: padding rows must be zero
    w = oracle.quantize_q4k(normal((n, k), 17, 0.02))
    dblk = torch.from_numpy(w.ggml()).cuda()
    dw = ops.upload_q4k_blocks(dblk, n, k, layout=layout)
    torch.cuda.synchronize()
    co, mo = w.physical(layout)
    assert np.array_equal(dw.codes.cpu().numpy(), co)
    assert np.array_equal(dw.scales.cpu().numpy(), mo)


def test_repack_q6k(torch_gpu):
    torch = torch_gpu
    import qw38_amd.ops as ops
    n, k = 21, 512
    w = oracle.quantize_q6k(normal((n, k), 19, 0.02))
    dw = ops.upload_q6k_blocks(torch.from_numpy(w.ggml()).cuda(), n, k)
    torch.cuda.synchronize()
    co, mo = w.physical()
    assert np.array_equal(dw.codes.cpu().numpy(), co)
    assert np.array_equal(dw.scales.cpu().numpy(), mo)


def test_repack_q6k_against_published_ggml_coordinates(torch_gpu):
    """The device repack of arbitrary GGML Q6_K bytes, read back through the
    coordinate-pinned 0x0241 unpacker, equals the weights that ggml's published
    dequantize_row_q6_K index expressions read from those bytes
    (tests/_fix.py ggml_q6k_decode), not the oracle's own GGML converter."""
    torch = torch_gpu
    import qw38_amd.ops as ops
    n, k = 13, 768
    rng = np.random.Generator(np.random.PCG64(41))
    blk = rng.integers(0, 256, size=(n * k // 256, 210), dtype=np.uint8)
    blk[:, 209] &= 0x3B  # finite fp16 d
    dw = ops.upload_q6k_blocks(torch.from_numpy(blk.reshape(-1)).cuda(), n, k)
    torch.cuda.synchronize()
    got = oracle.Q6K.from_physical(dw.codes.cpu().numpy(), dw.scales.cpu().numpy(), n, k)
    q, sc, d = ggml_q6k_decode(blk)
    assert np.array_equal(got.q.reshape(-1, 256), q)
    assert np.array_equal(got.sc.reshape(-1, 16), sc)
    assert np.array_equal(got.d.reshape(-1), d)
