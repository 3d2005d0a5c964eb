"""QL_W4A16_F16_ROWSCALED: a W4A16 GEMM whose bf16 result is stored as the next GEMM's row-scaled
fp16 operand (the staging pass between two linears folded into the first one's epilogue).

Pinned against the unfused sequence on the same GPU: the same GEMM with bf16 output gives the
logical values, and y16 * 2^e_m must equal them bit for bit wherever |value| >= 2^(e_m - 16)
(which is at least the documented floor of 2^-31 of the row bound B_m, since B_m 2^-e_m < 2^15);
below that floor a bf16 value -- only GELU's negative tail gets there -- lands in fp16's subnormals
and is rounded there, within half a subnormal step, 2^(e_m - 25). fc1 -> fc2 chained through
(y16, row_scale) equals fc1 (bf16) -> fc2 (bf16 x, staged inside the call) to 1 bf16 ulp: the two
fp16 operands differ per row only by a power of two, except for those tail values. The weight
bound is checked against float64.
"""
import numpy as np
import pytest
import torch

from oracle import qlinear_oracle as orc
from tests.gpu_util import seeded_linear

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _lib():
    from comfy_ui_gfx906_tools_amd import _lib
    return _lib


def _layer(M, N, K, seed):
    x, wq, ws = seeded_linear(M, N, K, seed=seed)
    bias = (torch.randn(N, generator=torch.Generator().manual_seed(seed + 1)) * 0.1).to(torch.bfloat16)
    return x.to(DEV), wq.to(DEV), ws.to(DEV), bias.to(DEV)


def test_out_bound_matches_float64():
    L = _lib()
    x, wq, ws, bias = _layer(8, 333, 640, seed=3)
    b = L.w4a16_out_bound(wq, ws, bias).cpu().numpy().astype(np.float64)
    w = orc.dequant_int4(wq.cpu().numpy(), ws.cpu().numpy()).astype(np.float64)
    l1 = np.abs(w).sum(axis=1).max()
    assert l1 <= b[0] <= l1 * (1 + 2.0 ** -9)
    assert b[1] == float(bias.float().abs().max())
    assert L.w4a16_out_bound(wq, ws, None)[1].item() == 0.0


@pytest.mark.parametrize("M,N,K,cfg,splits", [(300, 1040, 1024, None, 0), (300, 1040, 1024, 5, 0),
                                              (513, 777, 640, 5, 0), (257, 520, 512, 1, 3), (200, 700, 512, 2, 0),
                                              (40, 600, 512, 3, 0), (600, 256, 3072, None, 0),
                                              (64, 1040, 1024, 5, 0), (100, 777, 640, 5, 1), (128, 520, 2048, 5, 3)])
@pytest.mark.parametrize("gelu", [False, True])
def test_rowscaled_output_equals_bf16_output(M, N, K, cfg, splits, gelu):
    L = _lib()
    print(f"case rowscaled M={M} N={N} K={K} cfg={cfg} splits={splits} gelu={gelu}", flush=True)
    x, wq, ws, bias = _layer(M, N, K, seed=M + N + K)
    kw = dict(config=cfg, splits=splits, gelu=gelu)
    yb = L.w4a16_gemm(x, wq, ws, bias, out_dtype=torch.bfloat16, **kw)
    y16, rs = L.w4a16_gemm(x, wq, ws, bias, out_dtype=torch.bfloat16, f16_rowscaled=True, **kw)
    torch.cuda.synchronize()
    assert y16.dtype == torch.float16 and rs.shape == (M,)
    assert bool(torch.isfinite(y16).all()) and float(y16.abs().max()) <= 2.0 ** 15 * (1 + 2.0 ** -8)
    m, _ = np.frexp(rs.cpu().numpy())
    assert np.all(m == 0.5), "row factors must be powers of two"
    got, want, up = y16.double() * rs.double()[:, None], yb.double(), rs.double()[:, None]
    exact = want.abs() >= up * 2.0 ** -16
    assert exact.double().mean().item() > 0.99
    assert torch.equal(got[exact], want[exact]), f"max diff {(got - want)[exact].abs().max().item()}"
    assert bool(((got - want).abs() <= up * 2.0 ** -25).all())
    # the bound holds: every row's largest value fits below 2^15 after scaling, with room to spare
    assert float((yb.double().abs().amax(dim=1) / rs.double()).max()) < 2.0 ** 15


def test_chained_mlp_equals_unfused():
    """fc1 (+ GELU) writing row-scaled fp16, fc2 reading it: within 1 bf16 ulp of the bf16
    pipeline (fc1 bf16 out, fc2 staging the bf16 activation itself), and equal in almost every
    element (only GELU tail values below the exactness floor are rounded differently)."""
    L = _lib()
    M, H, F = 515, 768, 3072
    x, w1q, w1s, b1 = _layer(M, F, H, seed=41)
    _, w2q, w2s, b2 = _layer(M, H, F, seed=42)
    hb = L.w4a16_gemm(x, w1q, w1s, b1, out_dtype=torch.bfloat16, gelu=True)
    y_ref = L.w4a16_gemm(hb, w2q, w2s, b2, out_dtype=torch.bfloat16)
    h16, rs = L.w4a16_gemm(x, w1q, w1s, b1, out_dtype=torch.bfloat16, gelu=True, f16_rowscaled=True)
    y = L.w4a16_gemm(h16, w2q, w2s, b2, out_dtype=torch.bfloat16, row_scale=rs)
    torch.cuda.synchronize()
    d = (y.double() - y_ref.double()).abs()
    ulp = 2.0 ** (torch.floor(torch.log2(y_ref.double().abs().clamp_min(2.0 ** -126))) - 7)
    assert bool((d <= ulp).all()), f"max diff {d.max().item()}"
    assert (d == 0).double().mean().item() > 0.999


def test_rowscaled_argument_checks():
    L = _lib()
    x, wq, ws, bias = _layer(64, 256, 512, seed=5)
    with pytest.raises(RuntimeError, match="bfloat16"):
        L.w4a16_gemm(x, wq, ws, None, out_dtype=torch.float32, f16_rowscaled=True)
    with pytest.raises(RuntimeError, match="configurations 0-3"):
        L.w4a16_gemm(x, wq, ws, None, out_dtype=torch.bfloat16, f16_rowscaled=True, config=4)
    with pytest.raises(RuntimeError, match="row_scale"):
        L.w4a16_gemm(x.half(), wq, ws, None, out_dtype=torch.bfloat16, f16_rowscaled=True)
    # skinny M goes to the tile kernels instead of the direct ones
    y16, rs = L.w4a16_gemm(x[:3], wq, ws, bias, out_dtype=torch.bfloat16, f16_rowscaled=True)
    assert torch.equal(y16.double() * rs.double()[:, None],
                       L.w4a16_gemm(x[:3], wq, ws, bias, out_dtype=torch.bfloat16, config=3).double())
