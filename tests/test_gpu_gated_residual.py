"""The gated residual epilogue (QL_W4A16_GATED_RESIDUAL): y = residual + gate * linear(x) in the
GEMM's epilogue, the DiT block's "x = x + gate * proj(h)" without the separate elementwise pass.

Pinned bit for bit against the unfused sequence on the same GPU: the same GEMM storing its
output, then residual + gate * y evaluated by torch in fp32 (the product of two 16-bit numbers is
exact in fp32, then one rounding of the sum in fp32 and one to the output dtype -- what the
epilogue computes; for fp32 outputs the product rounds too, as in torch's two ops) and by the
library's standalone elementwise kernel (qlinear_gated_residual). Every tile configuration that
takes it (0-5), whole tiles and K pieces with their reduce, ragged M and N, per-batch gates, GELU
before the residual, in place, and the allocation-free entry point.
"""
import pytest
import torch

from tests.gpu_util import seeded_linear

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _lib():
    from comfy_ui_gfx906_tools_amd import _lib
    return _lib


def _unfused(y, res, gate2, rows_per_gate):
    g = gate2.float().repeat_interleave(rows_per_gate, dim=0)
    if y.dtype == torch.float32:
        return res + g * y
    return (res.float() + g * y.float()).to(y.dtype)


CASES = [
    # M, N, K, config, splits
    (300, 777, 640, None, 0), (300, 777, 640, 0, 0), (257, 300, 1024, 1, 0), (200, 520, 1024, 1, 3),
    (64, 1040, 512, 2, 0), (40, 600, 512, 3, 0), (9, 300, 256, None, 0), (513, 777, 640, 4, 0),
    (300, 1300, 1024, 5, 0), (300, 1300, 1024, 5, 1), (64, 777, 2048, 5, 3), (4096, 2048, 256, None, 0),
    (3840, 5120, 256, 5, 0),  # 300 tiles: whole 256 x 256 tiles, then the last round as 128-row halves
]


@pytest.mark.parametrize("M,N,K,cfg,splits", CASES)
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_fused_equals_unfused(M, N, K, cfg, splits, out_dtype):
    L = _lib()
    print(f"case gated residual M={M} N={N} K={K} cfg={cfg} splits={splits} out={out_dtype}", flush=True)
    x, wq, ws = seeded_linear(M, N, K, seed=M + N + K)
    x, wq, ws = x.to(DEV), wq.to(DEV), ws.to(DEV)
    g = torch.Generator().manual_seed(M)
    bias = torch.randn(N, generator=g).to(out_dtype).to(DEV)
    res = torch.randn(M, N, generator=g).to(out_dtype).to(DEV)
    G = 3 if M % 3 == 0 else 1  # per-batch gates: rows [b M/G, (b+1) M/G) take gate row b
    gate = (torch.randn(G, N, generator=g) * 0.5).to(out_dtype).to(DEV)
    # the unfused output from the kernel the fused call runs on: up to 16 rows the automatic plan
    # would otherwise take a direct kernel (exact codes, other rounding), which has no such epilogue
    ycfg = 3 if cfg is None and M <= 16 else cfg
    for gelu in (False, True):
        kw = dict(out_dtype=out_dtype, config=cfg, splits=splits, gelu=gelu)
        y = L.w4a16_gemm(x, wq, ws, bias, **{**kw, "config": ycfg})
        want = _unfused(y, res, gate, M // G)
        got = L.w4a16_gemm(x, wq, ws, bias, residual=res, gate=gate, **kw)
        assert torch.equal(got, want), f"gelu={gelu}: max diff {(got.float() - want.float()).abs().max().item()}"
        if G == 1 and out_dtype != torch.float32 and N % 8 == 0:  # the library's elementwise kernel agrees
            assert torch.equal(got, L.gated_residual(res, gate.reshape(-1), y))
    # in place: y written over the residual
    r2 = res.clone()
    out = L.w4a16_gemm(x, wq, ws, bias, out_dtype=out_dtype, config=cfg, splits=splits, residual=r2, gate=gate,
                       out=r2)
    assert out.data_ptr() == r2.data_ptr()
    assert torch.equal(r2, _unfused(L.w4a16_gemm(x, wq, ws, bias, out_dtype=out_dtype, config=ycfg, splits=splits),
                                    res, gate, M // G))


def test_fused_noalloc_and_scales_kn():
    L = _lib()
    M, N, K = 200, 520, 1024
    x, wq, ws = seeded_linear(M, N, K, seed=7)
    x, wq, ws = x.to(DEV), wq.to(DEV), ws.to(DEV)
    res = torch.randn(M, N, device=DEV).to(torch.bfloat16)
    gate = torch.randn(1, N, device=DEV).to(torch.bfloat16)
    want = L.w4a16_gemm(x, wq, ws, out_dtype=torch.bfloat16, residual=res, gate=gate)
    assert torch.equal(L.w4a16_gemm(x, wq, ws, out_dtype=torch.bfloat16, residual=res, gate=gate, noalloc=True), want)
    assert torch.equal(L.w4a16_gemm(x, wq, ws, out_dtype=torch.bfloat16, residual=res, gate=gate,
                                    scales_kn=L.w4a16_scales_kn(ws)), want)


def test_fused_argument_checks():
    L = _lib()
    x, wq, ws = seeded_linear(64, 256, 512, seed=5)
    x, wq, ws = x.to(DEV), wq.to(DEV), ws.to(DEV)
    res = torch.zeros(64, 256, device=DEV, dtype=torch.bfloat16)
    gate = torch.ones(256, device=DEV, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="configurations 0-5"):
        L.w4a16_gemm(x, wq, ws, out_dtype=torch.bfloat16, residual=res, gate=gate, config=6)
    with pytest.raises(RuntimeError, match="do not combine"):
        L.w4a16_gemm(x, wq, ws, out_dtype=torch.bfloat16, residual=res, gate=gate, f16_rowscaled=True)
    with pytest.raises(RuntimeError, match="gate must be"):
        L.w4a16_gemm(x, wq, ws, out_dtype=torch.bfloat16, residual=res, gate=torch.ones(5, 256, device=DEV,
                                                                                        dtype=torch.bfloat16))
    with pytest.raises(RuntimeError, match="residual must be"):
        L.w4a16_gemm(x, wq, ws, out_dtype=torch.bfloat16, residual=res.float(), gate=gate)
    # skinny M: the planner keeps the tile kernels (the direct kernels have no such epilogue)
    y = L.w4a16_gemm(x[:4], wq, ws, out_dtype=torch.bfloat16, residual=res[:4], gate=gate)
    ref = L.w4a16_gemm(x[:4], wq, ws, out_dtype=torch.bfloat16, config=3)
    assert torch.equal(y, (res[:4].float() + gate.float() * ref.float()).to(torch.bfloat16))
