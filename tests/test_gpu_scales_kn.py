"""Group-major scales (qlinear_w4a16_scales_kn, the w_scale_kn argument of qlinear_w4a16_gemm).

The copy must be the exact transpose of w_scale, and a GEMM given it must return the same bits as
the same GEMM reading w_scale: the kernels read the same scale values, only from other addresses.
That is checked for every kernel configuration (the direct kernels 7 and 8 ignore the copy), whole
tiles and K pieces, ragged N (the last tile's columns past N read scales of the next group row,
which must never reach a stored output), K tails of the 4-wave kernel, fp32 / 16-bit outputs, the
GELU and row-scaled fp16 epilogues, and weights whose columns carry power-of-two factors.
"""
import numpy as np
import pytest
import torch

from tests.gpu_util import seeded_linear

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _lib():
    from comfy_ui_gfx906_tools_amd import _lib
    return _lib


@pytest.mark.parametrize("N,K", [(1, 32), (31, 96), (33, 1024), (777, 640), (3072, 3072), (130, 4160)])
def test_scales_kn_is_the_transpose(N, K):
    ws = torch.randn(N, K // 32, generator=torch.Generator().manual_seed(N + K)).to(DEV)
    kn = _lib().w4a16_scales_kn(ws)
    assert kn.shape == (K // 32, N) and torch.equal(kn, ws.t().contiguous())


CASES = [
    # M, N, K, config, splits
    (300, 777, 640, None, 0), (300, 777, 640, 0, 0), (257, 300, 1024, 1, 0), (200, 520, 1024, 1, 3),
    (64, 1040, 512, 2, 0), (40, 600, 512, 3, 0), (16, 300, 160, 3, 0), (130, 777, 96, 1, 0),
    (513, 777, 640, 4, 0), (300, 1300, 1024, 5, 0), (300, 1300, 1024, 5, 1), (100, 2600, 4096, 5, 0),
    (64, 777, 2048, 5, 3), (513, 520, 1024, 6, 0), (3, 777, 1024, 7, 0), (12, 777, 1024, 8, 0),
    (1, 10240, 4096, None, 0), (16, 10240, 4096, None, 0), (64, 10240, 4096, None, 0),
]


@pytest.mark.parametrize("M,N,K,cfg,splits", CASES)
@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
def test_gemm_with_scales_kn_is_bit_identical(M, N, K, cfg, splits, out_dtype):
    L = _lib()
    print(f"case scales_kn M={M} N={N} K={K} cfg={cfg} splits={splits} out={out_dtype}", flush=True)
    x, wq, ws = seeded_linear(M, N, K, seed=M + N + K)
    x, wq, ws = x.to(DEV), wq.to(DEV), ws.to(DEV)
    bias = (torch.randn(N, generator=torch.Generator().manual_seed(3)) * 0.1).to(out_dtype).to(DEV)
    kn = L.w4a16_scales_kn(ws)
    kw = dict(out_dtype=out_dtype, config=cfg, splits=splits)
    assert torch.equal(L.w4a16_gemm(x, wq, ws, bias, scales_kn=kn, **kw), L.w4a16_gemm(x, wq, ws, bias, **kw))
    if cfg not in (7, 8):  # 16-bit x on the fp16 route's staged operand, GELU epilogue
        x16, rs = L.rows_to_f16(x)
        kw = dict(out_dtype=out_dtype, config=cfg, splits=splits, gelu=True, row_scale=rs)
        assert torch.equal(L.w4a16_gemm(x16, wq, ws, bias, scales_kn=kn, **kw), L.w4a16_gemm(x16, wq, ws, bias, **kw))
    if out_dtype == torch.bfloat16 and cfg in (None, 0, 1, 2, 3, 5):
        a = L.w4a16_gemm(x, wq, ws, bias, out_dtype=out_dtype, config=cfg, splits=splits, f16_rowscaled=True,
                         scales_kn=kn)
        b = L.w4a16_gemm(x, wq, ws, bias, out_dtype=out_dtype, config=cfg, splits=splits, f16_rowscaled=True)
        assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
    if cfg not in (7, 8):  # the reference's bf16 dequant numerics (bf16 MFMA)
        kw = dict(out_dtype=out_dtype, config=cfg, splits=splits, bf16_mfma=True)
        assert torch.equal(L.w4a16_gemm(x, wq, ws, bias, scales_kn=kn, **kw), L.w4a16_gemm(x, wq, ws, bias, **kw))


@pytest.mark.parametrize("cfg", [None, 1, 3, 5])
def test_scales_kn_with_column_factors(cfg):
    """Scales far outside fp16's range (every column its own exponent in [-24, 14]): the column
    factors and the group-major copy together, same bits as without the copy."""
    L = _lib()
    M, N, K = 300, 264, 640
    rng = np.random.default_rng(9)
    x = torch.from_numpy(rng.normal(0.0, 1.0, (M, K)).astype(np.float32)).to(torch.bfloat16).to(DEV)
    codes = rng.integers(-8, 8, (N, K))
    nib = (codes & 0xF).astype(np.uint8)
    wq = torch.from_numpy((nib[:, 0::2] | (nib[:, 1::2] << 4)).view(np.int8)).to(DEV)
    s = np.exp(rng.normal(0.0, 0.3, (N, K // 32))) * 2.0 ** rng.integers(-24, 15, (N, 1))
    ws = torch.from_numpy(s.astype(np.float32)).to(DEV)
    cs = L.w4a16_col_scales(ws)
    assert not torch.equal(cs, torch.ones_like(cs))
    kn = L.w4a16_scales_kn(ws)
    for out_dtype in (torch.float32, torch.bfloat16):
        a = L.w4a16_gemm(x, wq, ws, out_dtype=out_dtype, config=cfg, col_scale=cs, scales_kn=kn)
        b = L.w4a16_gemm(x, wq, ws, out_dtype=out_dtype, config=cfg, col_scale=cs)
        assert torch.equal(a, b)


def test_scales_kn_noalloc_and_argument_checks():
    L = _lib()
    x, wq, ws = seeded_linear(200, 520, 1024, seed=1)
    x, wq, ws = x.to(DEV), wq.to(DEV), ws.to(DEV)
    kn = L.w4a16_scales_kn(ws)
    assert torch.equal(L.w4a16_gemm(x, wq, ws, out_dtype=torch.float32, scales_kn=kn, noalloc=True),
                       L.w4a16_gemm(x, wq, ws, out_dtype=torch.float32))
    with pytest.raises(RuntimeError, match="scales_kn must be"):
        L.w4a16_gemm(x, wq, ws, out_dtype=torch.float32, scales_kn=ws)  # [N, K/32], not [K/32, N]


def test_cached_scales_kn_follow_in_place_updates():
    L = _lib()
    ws = torch.rand(40, 8, device=DEV)
    k1 = L.cached_scales_kn(ws)
    assert L.cached_scales_kn(ws) is k1 and torch.equal(k1, ws.t().contiguous())
    ws.mul_(3.0)
    k2 = L.cached_scales_kn(ws)
    assert k2 is not k1 and torch.equal(k2, ws.t().contiguous())
