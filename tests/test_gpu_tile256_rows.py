"""The 256-column kernel's variant 1 (configuration 5) at small M: tiles of 64, 128 or 256 rows,
whole or cut into K pieces whose fp32 partials the ordered reduce sums (the few-tile shapes where
whole tiles would leave most CUs idle).

Pinned against the float64 dequant-then-matmul oracle (2e-3 of max|ref|, fp32 out), bit-exact on
an integer grid (every partial and sum exact in fp32), 16-bit outputs within 1 ulp + gate, the
bf16-MFMA mode against the reference's bf16 dequant, and K pieces against whole tiles of the same
height on the same inputs (the same products, summed in another order: within the gate).
"""
import numpy as np
import pytest
import torch

from oracle import qlinear_oracle as orc
from tests.gpu_util import bf16_ulp, f16_ulp, rel_max_err, seeded_linear, to_np_f32

pytestmark = pytest.mark.gpu
TOL = 2e-3
DEV = "cuda:0"
CFG = 5


def _lib():
    from comfy_ui_gfx906_tools_amd import _lib
    return _lib


def _run(x, wq, ws, bias=None, out_dtype=torch.float32, splits=0, bf16_mfma=False, gelu=False):
    return _lib().w4a16_gemm(x.to(DEV), wq.to(DEV), ws.to(DEV), None if bias is None else bias.to(DEV),
                             out_dtype=out_dtype, splits=splits, bf16_mfma=bf16_mfma, config=CFG, gelu=gelu)


CASES = [
    # M, N, K, x dtype: tile heights 64 (M <= 64), 128 (M <= 128), 256; ragged M and N
    (1, 300, 640, torch.bfloat16),
    (17, 777, 1024, torch.float16),
    (64, 2600, 3072, torch.bfloat16),
    (65, 520, 512, torch.float16),
    (100, 1040, 4096, torch.bfloat16),
    (128, 256, 256, torch.bfloat16),
    (129, 777, 1024, torch.float16),
    (256, 1300, 2048, torch.bfloat16),
]


@pytest.mark.parametrize("splits", [0, 1, 3])
@pytest.mark.parametrize("M,N,K,xdt", CASES)
def test_rows_vs_oracle(M, N, K, xdt, splits):
    """fp32 out with bias within the gate; the plan's tile height is the shortest covering M; two
    runs bit-identical (fixed reduction order)."""
    L = _lib()
    plan = L.w4a16_describe_plan(M, N, K, x_dtype=xdt, splits=splits, config=CFG)
    assert plan["tile_rows"] == (64 if M <= 64 else 128 if M <= 128 else 256)
    assert plan["k_pieces"] == (1 if splits == 1 else min(3, K // 64) if splits == 3 else plan["k_pieces"])
    print(f"case rows M={M} N={N} K={K} x={xdt} splits={splits} plan={plan}", flush=True)
    x, wq, ws = seeded_linear(M, N, K, seed=M + N + K + splits, x_dtype=xdt)
    bias = torch.randn(N, generator=torch.Generator().manual_seed(M))
    y1 = _run(x, wq, ws, bias, splits=splits)
    y2 = _run(x, wq, ws, bias, splits=splits)
    assert torch.equal(y1, y2), "not deterministic"
    ref = orc.w4a16_reference(to_np_f32(x), wq.numpy(), ws.numpy(), bias.numpy())
    err = rel_max_err(to_np_f32(y1), ref)
    assert err <= TOL, f"max rel err {err:.3e} > {TOL}"


@pytest.mark.parametrize("M", [40, 120, 250])
@pytest.mark.parametrize("splits", [0, 1, 5])
def test_rows_exact_on_integer_grid(M, splits):
    """Integer activations, int4 codes and power-of-two group scales: every product, partial and
    sum is exact in fp32, so whole tiles and every K-piece count equal the oracle bit for bit."""
    N, K = 300, 1280
    g = np.random.default_rng(7 + M + splits)
    x = torch.from_numpy(g.integers(-4, 5, (M, K)).astype(np.float32)).to(torch.bfloat16)
    codes = g.integers(-8, 8, (N, K))
    nib = (codes & 0xF).astype(np.uint8)
    packed = (nib[:, 0::2] | (nib[:, 1::2] << 4)).view(np.int8)
    scale = (2.0 ** g.integers(-6, 0, (N, K // 32))).astype(np.float32)
    print(f"case rows exact M={M} splits={splits}", flush=True)
    y = to_np_f32(_run(x, torch.from_numpy(packed), torch.from_numpy(scale), splits=splits))
    ref = orc.w4a16_reference(to_np_f32(x), packed, scale)
    assert np.array_equal(y.astype(np.float64), ref), f"max abs diff {np.abs(y - ref).max()}"


@pytest.mark.parametrize("M", [33, 100, 200])
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16])
def test_rows_16bit_out_and_bf16_mfma(M, out_dtype):
    """16-bit outputs with bias (1 ulp + gate of the rounded oracle) through the reduce's epilogue,
    and the bf16-MFMA mode within 2e-5 of the reference's bf16 dequant-then-matmul."""
    N, K = 520, 2048
    print(f"case rows 16-bit M={M} out={out_dtype}", flush=True)
    x, wq, ws = seeded_linear(M, N, K, seed=M + 11)
    y = to_np_f32(_run(x, wq, ws, bf16_mfma=True))
    w_bf16 = orc.round_to_bf16(orc.dequant_int4(wq.numpy(), ws.numpy())).astype(np.float64)
    assert rel_max_err(y, to_np_f32(x).astype(np.float64) @ w_bf16.T) <= 2e-5
    bias = torch.randn(N, generator=torch.Generator().manual_seed(4)).to(out_dtype)
    y = to_np_f32(_run(x, wq, ws, bias, out_dtype=out_dtype))
    ref = orc.w4a16_reference(to_np_f32(x), wq.numpy(), ws.numpy(), to_np_f32(bias)).astype(np.float32)
    name = "bfloat16" if out_dtype == torch.bfloat16 else "float16"
    ref_r = orc.round_to_dtype(ref, name)
    ulp = bf16_ulp(ref_r) if out_dtype == torch.bfloat16 else f16_ulp(ref_r)
    bound = ulp + TOL * np.abs(ref).max()
    assert (np.abs(y - ref_r) <= bound).all(), f"max excess {(np.abs(y - ref_r) - bound).max():.3e}"


@pytest.mark.parametrize("M", [64, 128, 256])
def test_rows_k_pieces_vs_whole_tiles(M):
    """The automatic K pieces against whole tiles of the same height (splits=1), bf16 x, GELU
    epilogue, bf16 out: the same products summed in another order, within 1 ulp + gate."""
    L = _lib()
    N, K = 2560, 4096
    assert L.w4a16_describe_plan(M, N, K, config=CFG, cus=256)["k_pieces"] > 1
    print(f"case rows pieces vs whole M={M}", flush=True)
    x, wq, ws = seeded_linear(M, N, K, seed=M + 5)
    bias = torch.randn(N, generator=torch.Generator().manual_seed(9)).to(torch.bfloat16)
    cut = to_np_f32(_run(x, wq, ws, bias, out_dtype=torch.bfloat16, gelu=True))
    whole = to_np_f32(_run(x, wq, ws, bias, out_dtype=torch.bfloat16, gelu=True, splits=1))
    bound = bf16_ulp(whole) + TOL * np.abs(whole).max()
    assert (np.abs(cut - whole) <= bound).all()


@pytest.mark.parametrize("M,N,K,cfg", [(768, 3072, 12288, 5), (1024, 3072, 12288, 5), (1000, 2600, 8192, 5),
                                       (1024, 3072, 3072, 1), (768, 3072, 3072, 1), (128, 18432, 3072, 1),
                                       (40, 18432, 3072, 2)])
def test_auto_plan_one_round_of_k_pieces(M, N, K, cfg):
    """Fewer 256 x 256 tiles than a quarter of the CUs: the automatic plan cuts K into pieces that
    fit one round of workgroups, on the 128- or 64-row tiles, or on the 256 x 256 tiles where the
    128-row round leaves CUs idle and the 256 x 256 pieces stay long (K = 8192, 12288); against
    the float64 oracle (gate), fp32 and bf16 out with bias."""
    L = _lib()
    plan = L.w4a16_describe_plan(M, N, K, cus=256)
    assert plan["config"] == cfg and plan["k_pieces"] > 1
    assert plan["whole_tiles"] + (plan["tiles"] - plan["whole_tiles"]) * plan["k_pieces"] <= 256
    print(f"case auto one-round M={M} N={N} K={K} plan={plan}", flush=True)
    x, wq, ws = seeded_linear(M, N, K, seed=M + N + K)
    bias = torch.randn(N, generator=torch.Generator().manual_seed(M))
    xd, wqd, wsd = x.to(DEV), wq.to(DEV), ws.to(DEV)
    y = L.w4a16_gemm(xd, wqd, wsd, bias.to(DEV), out_dtype=torch.float32)
    ref = orc.w4a16_reference(to_np_f32(x), wq.numpy(), ws.numpy(), bias.numpy())
    assert rel_max_err(to_np_f32(y), ref) <= TOL
    yb = to_np_f32(L.w4a16_gemm(xd, wqd, wsd, bias.to(torch.bfloat16).to(DEV), out_dtype=torch.bfloat16))
    refb = orc.w4a16_reference(to_np_f32(x), wq.numpy(), ws.numpy(), to_np_f32(bias.to(torch.bfloat16))).astype(np.float32)
    ref_r = orc.round_to_dtype(refb, "bfloat16")
    assert (np.abs(yb - ref_r) <= bf16_ulp(ref_r) + TOL * np.abs(refb).max()).all()
