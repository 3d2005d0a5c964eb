"""224-row tiles of the 256-column kernel (configuration 5, automatic plan): taken where 256-row
tiles would make a single round that leaves CUs idle and 224-row tiles still fit one round (the C2
fc2 shape: 216 -> 252 tiles on 256 CUs).

Every output element is accumulated over K in the same MFMA order whichever row block holds it,
so the 224-row plan must equal the 256-row whole tiles (splits=1) bit for bit, for every
epilogue: fp32 / bf16 / fp16 out with bias, GELU, the row-scaled fp16 output, the gated residual,
bf16-MFMA mode, and ragged M / N (the second half of a 224-row tile holds 96 rows). Pinned to the
float64 oracle (gate) and exactly on an integer grid.
"""
import numpy as np
import pytest
import torch

from oracle import qlinear_oracle as orc
from tests.gpu_util import rel_max_err, seeded_linear, to_np_f32

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
TOL = 2e-3


def _lib():
    from comfy_ui_gfx906_tools_amd import _lib
    return _lib


def _plan(M, N, K, **kw):
    d = _lib().w4a16_describe_plan(M, N, K, cus=256, **kw)
    print(f"plan M={M} N={N} K={K} {kw}: {d}", flush=True)
    return d


# M, N, K: the C2 fc2 shape, C1, a C5 img shape, ragged M and N
SHAPES = [(4608, 3072, 12288), (4608, 3072, 3072), (4096, 3072, 3072), (4000, 3000, 1024)]


@pytest.mark.parametrize("M,N,K", SHAPES)
def test_tile224_equals_256_row_tiles(M, N, K):
    L = _lib()
    if L.w4a16_describe_plan(M, N, K)["tile_rows"] != 224:
        pytest.skip("this GPU's CU count plans no 224-row tiles for the shape")
    assert _plan(M, N, K)["tile_rows"] == 224 and _plan(M, N, K, splits=1)["tile_rows"] == 256
    x, wq, ws = seeded_linear(M, N, K, seed=M + N + K)
    x, wq, ws = x.to(DEV), wq.to(DEV), ws.to(DEV)
    g = torch.Generator().manual_seed(N)
    for odt in (torch.float32, torch.bfloat16, torch.float16):
        bias = (torch.randn(N, generator=g) * 0.1).to(odt).to(DEV)
        for gelu in (False, True):
            a = L.w4a16_gemm(x, wq, ws, bias, out_dtype=odt, gelu=gelu)
            b = L.w4a16_gemm(x, wq, ws, bias, out_dtype=odt, gelu=gelu, splits=1)
            assert torch.equal(a, b), f"out {odt} gelu {gelu}"
    bias = (torch.randn(N, generator=g) * 0.1).to(torch.bfloat16).to(DEV)
    a = L.w4a16_gemm(x, wq, ws, bias, out_dtype=torch.bfloat16, gelu=True, f16_rowscaled=True)
    b = L.w4a16_gemm(x, wq, ws, bias, out_dtype=torch.bfloat16, gelu=True, f16_rowscaled=True, splits=1)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
    res = torch.randn(M, N, generator=g).to(torch.bfloat16).to(DEV)
    gate = torch.randn(2, N, generator=g).to(torch.bfloat16).to(DEV)
    a = L.w4a16_gemm(x, wq, ws, bias, out_dtype=torch.bfloat16, residual=res, gate=gate)
    b = L.w4a16_gemm(x, wq, ws, bias, out_dtype=torch.bfloat16, residual=res, gate=gate, splits=1)
    assert torch.equal(a, b)
    a = L.w4a16_gemm(x, wq, ws, None, out_dtype=torch.float32, bf16_mfma=True)
    b = L.w4a16_gemm(x, wq, ws, None, out_dtype=torch.float32, bf16_mfma=True, splits=1)
    assert torch.equal(a, b)


@pytest.mark.parametrize("M,N,K", [(4608, 3072, 3072), (4000, 3000, 1024)])
def test_tile224_vs_oracle(M, N, K):
    """fp32 out with bias against the float64 dequant-then-matmul (gate), output pre-filled with
    NaN so a row the 224-row tiles miss would show."""
    L = _lib()
    if L.w4a16_describe_plan(M, N, K)["tile_rows"] != 224:
        pytest.skip("this GPU's CU count plans no 224-row tiles for the shape")
    x, wq, ws = seeded_linear(M, N, K, seed=M + K)
    bias = torch.randn(N, generator=torch.Generator().manual_seed(M))
    out = torch.full((M, N), float("nan"), device=DEV)
    y = L.w4a16_gemm(x.to(DEV), wq.to(DEV), ws.to(DEV), bias.to(DEV), out_dtype=torch.float32, out=out)
    assert not torch.isnan(y).any()
    ref = orc.w4a16_reference(to_np_f32(x), wq.numpy(), ws.numpy(), bias.numpy())
    assert rel_max_err(to_np_f32(y), ref) <= TOL


def test_tile224_exact_on_integer_grid():
    """Integer activations, int4 codes and power-of-two group scales: exact in fp32, equal to the
    oracle bit for bit (ragged M: the last tile's second half holds a few rows)."""
    M, N, K = 4500, 3072, 1024
    L = _lib()
    if L.w4a16_describe_plan(M, N, K)["tile_rows"] != 224:
        pytest.skip("this GPU's CU count plans no 224-row tiles for the shape")
    gen = np.random.default_rng(3)
    x = torch.from_numpy(gen.integers(-4, 5, (M, K)).astype(np.float32)).to(torch.bfloat16)
    codes = gen.integers(-8, 8, (N, K))
    nib = (codes & 0xF).astype(np.uint8)
    packed = (nib[:, 0::2] | (nib[:, 1::2] << 4)).view(np.int8)
    scale = (2.0 ** gen.integers(-6, 0, (N, K // 32))).astype(np.float32)
    y = L.w4a16_gemm(x.to(DEV), torch.from_numpy(packed).to(DEV), torch.from_numpy(scale).to(DEV),
                     out_dtype=torch.float32)
    ref = orc.w4a16_reference(to_np_f32(x), packed, scale)
    assert np.array_equal(to_np_f32(y).astype(np.float64), ref)
