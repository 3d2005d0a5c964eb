"""W8A8 parity on the GPU: int32 accumulators bit-exact against exact integer matmul, the
fp32 epilogue and bf16 output bit-exact against the oracle's operation order, the per-token
quantizer bit-exact against the oracle."""
import numpy as np
import pytest
import torch

from oracle import qlinear_oracle as orc
from tests.gpu_util import to_np_f32

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _lib():
    from comfy_ui_gfx906_tools_amd import _lib
    return _lib


# K % 8 == 0 and K <= 16384 take the register-resident vector kernel; (5, 1004) and (3, 16392)
# the element-wise one
@pytest.mark.parametrize("M,K,dt", [(1, 64, torch.bfloat16), (7, 3072, torch.bfloat16), (300, 1000, torch.float16),
                                    (64, 4096, torch.float32), (5, 1004, torch.float16), (3, 16392, torch.bfloat16),
                                    (2, 16384, torch.float32), (9, 2088, torch.bfloat16), (6, 1536, torch.float32),
                                    (4, 8192, torch.float16)])
def test_quantize_int8_per_token_matches_oracle(M, K, dt):
    print(f"case quant8 M={M} K={K} {dt}", flush=True)
    g = torch.Generator().manual_seed(M + K)
    x = (torch.randn(M, K, generator=g) * torch.rand(M, 1, generator=g) * 10).to(dt)
    if M > 1:
        x[1] = 0  # all-zero row: scale 1e-8/127, codes 0
    q, s = _lib().quantize_int8_per_token(x.to(DEV))
    q_ref, s_ref = orc.quantize_int8_rows(to_np_f32(x))
    assert np.array_equal(s.cpu().numpy().view(np.uint32), s_ref.view(np.uint32))
    assert np.array_equal(q.cpu().numpy(), q_ref)


# M <= 128 runs the 16 / 64 / 128-row kernel, M > 128 the 256 x 256-tile kernel (ragged M and N,
# K of 1, 3, 4 and 5 stages of 64, 64-row and 16-row remainders of a tile)
SHAPES = [(1, 256, 64), (5, 300, 192), (64, 512, 3072), (200, 1000, 4096), (257, 256, 256), (129, 17, 64),
          (300, 520, 192), (513, 257, 320), (256, 768, 4224)]


@pytest.mark.parametrize("M,N,K", SHAPES)
def test_w8a8_accumulators_bit_exact(M, N, K):
    print(f"case w8a8 acc M={M} N={N} K={K}", flush=True)
    rng = np.random.default_rng(M * 3 + N + K)
    a = rng.integers(-127, 128, (M, K), dtype=np.int8)
    b = rng.integers(-127, 128, (N, K), dtype=np.int8)
    acc = _lib().w8a8_gemm(torch.from_numpy(a).to(DEV), None, torch.from_numpy(b).to(DEV), None,
                           out_dtype=torch.int32)
    ref = orc.int8_matmul_exact(a, b)
    assert np.array_equal(acc.cpu().numpy().astype(np.int64), ref)


@pytest.mark.parametrize("M", [32, 300])
def test_w8a8_extreme_values_bit_exact(M):
    """All +-127 / -128 operands: the largest-magnitude accumulators the format allows."""
    N, K = 64, 12288
    print(f"case w8a8 extreme M={M}", flush=True)
    a = np.full((M, K), -128, np.int8)
    a[1::2] = 127
    b = np.full((N, K), -128, np.int8)
    b[::3] = 127
    acc = _lib().w8a8_gemm(torch.from_numpy(a).to(DEV), None, torch.from_numpy(b).to(DEV), None,
                           out_dtype=torch.int32)
    assert np.array_equal(acc.cpu().numpy().astype(np.int64), orc.int8_matmul_exact(a, b))


@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("with_bias", [False, True])
@pytest.mark.parametrize("M,N", [(100, 320), (130, 320), (300, 261)])
def test_w8a8_epilogue_bit_exact(out_dtype, with_bias, M, N):
    K = 1024
    print(f"case w8a8 epilogue M={M} N={N} {out_dtype} bias={with_bias}", flush=True)
    g = torch.Generator().manual_seed(4)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    w = torch.randn(N, K, generator=g) * 0.02
    xq, sx = orc.quantize_int8_rows(to_np_f32(x))
    wq, sw = orc.quantize_int8_rows(w.numpy())
    bias = (torch.randn(N, generator=g) * 0.1).to(out_dtype) if with_bias else None
    y = _lib().w8a8_gemm(torch.from_numpy(xq).to(DEV), torch.from_numpy(sx).to(DEV), torch.from_numpy(wq).to(DEV),
                         torch.from_numpy(sw).to(DEV), None if bias is None else bias.to(DEV), out_dtype=out_dtype)
    ref = orc.w8a8_epilogue(orc.int8_matmul_exact(xq, wq), sx, sw, None if bias is None else to_np_f32(bias))
    name = {torch.float32: "float32", torch.bfloat16: "bfloat16", torch.float16: "float16"}[out_dtype]
    assert np.array_equal(to_np_f32(y), orc.round_to_dtype(ref, name))


def test_w8a8_c3_full_size():
    """C3: 3072 -> 21504, M = 4608. Accumulators vs float64 torch matmul on the GPU (exact: every
    partial sum is an integer below 2^53); bf16 output vs torch's fp32 ops in the same order."""
    M, K, N = 4608, 3072, 21504
    g = torch.Generator().manual_seed(3)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16).to(DEV)
    w = (torch.randn(N, K, generator=g) * 0.02).to(DEV)
    lib = _lib()
    xq, sx = lib.quantize_int8_per_token(x)
    wq, sw = lib.quantize_int8_per_token(w)
    acc = lib.w8a8_gemm(xq, None, wq, None, out_dtype=torch.int32)
    exact = (xq.double() @ wq.double().t())
    assert torch.equal(acc.double(), exact)
    y = lib.w8a8_gemm(xq, sx, wq, sw, out_dtype=torch.bfloat16)
    ref = (acc.float() * (sx[:, None] * sw[None, :])).to(torch.bfloat16)
    assert torch.equal(y, ref)
