"""W4A16 parity on the GPU: the gfx950 kernel vs the CPU oracle (small shapes, golden fixture)
and vs an fp32 torch GEMM of the dequantized weight (the BASELINE configs at full size).

Tolerance: max|y - ref| / max|ref| <= 2e-3 against the fp32-dequant
reference with fp32 output. With 16-bit output the kernel's value is rounded once more, so
bf16/fp16 outputs are gated elementwise at |y - round(ref)| <= 1 ulp(round(ref)) + 2e-3*max|ref|.
"""
import numpy as np
import pytest
import torch

from oracle import qlinear_oracle as orc
from tests.conftest import golden_path
from tests.gpu_util import bf16_ulp, dequant_torch, f16_ulp, rel_max_err, seeded_linear, to_np_f32

pytestmark = pytest.mark.gpu
TOL = 2e-3
DEV = "cuda:0"


def _lib():
    from comfy_ui_gfx906_tools_amd import _lib
    return _lib


def _run(x, wq, ws, bias=None, out_dtype=torch.float32, splits=0, bf16_mfma=False):
    return _lib().w4a16_gemm(x.to(DEV), wq.to(DEV), ws.to(DEV), None if bias is None else bias.to(DEV),
                             out_dtype=out_dtype, splits=splits, bf16_mfma=bf16_mfma)


SMALL = [
    # M, N, K, x dtype, bias
    (1, 256, 256, torch.bfloat16, False),
    (5, 300, 96, torch.bfloat16, True),
    (16, 512, 1024, torch.float16, False),
    (17, 512, 1024, torch.float16, True),
    (64, 256, 512, torch.bfloat16, True),
    (100, 700, 160, torch.bfloat16, False),
    (300, 1000, 4096, torch.bfloat16, True),
    (513, 384, 3072, torch.float16, False),
]


@pytest.mark.parametrize("M,N,K,xdt,with_bias", SMALL)
def test_w4a16_vs_oracle_fp32_out(M, N, K, xdt, with_bias):
    print(f"case M={M} N={N} K={K} x={xdt} bias={with_bias}", flush=True)
    x, wq, ws = seeded_linear(M, N, K, seed=M * 7 + N + K, x_dtype=xdt)
    bias = torch.randn(N, generator=torch.Generator().manual_seed(1)) if with_bias else None
    y = to_np_f32(_run(x, wq, ws, bias))
    ref = orc.w4a16_reference(to_np_f32(x), wq.numpy(), ws.numpy(), None if bias is None else bias.numpy())
    assert y.shape == (M, N)
    assert np.isfinite(y).all()
    err = rel_max_err(y, ref)
    assert err <= TOL, f"max rel err {err:.3e} > {TOL}"


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("xdt", [torch.bfloat16, torch.float16])
def test_w4a16_16bit_out(out_dtype, xdt):
    M, N, K = 96, 640, 2048
    print(f"case 16-bit out {out_dtype} x={xdt}", flush=True)
    x, wq, ws = seeded_linear(M, N, K, seed=11, x_dtype=xdt)
    bias = torch.randn(N, generator=torch.Generator().manual_seed(2)).to(out_dtype)
    y = to_np_f32(_run(x, wq, ws, bias, out_dtype=out_dtype))
    ref = orc.w4a16_reference(to_np_f32(x), wq.numpy(), ws.numpy(), to_np_f32(bias)).astype(np.float32)
    name = "bfloat16" if out_dtype == torch.bfloat16 else "float16"
    ref_r = orc.round_to_dtype(ref, name)
    ulp = bf16_ulp(ref_r) if out_dtype == torch.bfloat16 else f16_ulp(ref_r)
    bound = ulp + TOL * np.abs(ref).max()
    assert (np.abs(y - ref_r) <= bound).all(), f"max excess {(np.abs(y - ref_r) - bound).max():.3e}"


@pytest.mark.parametrize("splits", [1, 2, 3, 7])
def test_w4a16_split_k_and_determinism(splits):
    M, N, K = 200, 512, 2048
    print(f"case splits={splits}", flush=True)
    x, wq, ws = seeded_linear(M, N, K, seed=5)
    bias = torch.randn(N, generator=torch.Generator().manual_seed(3))
    y1 = _run(x, wq, ws, bias, splits=splits)
    y2 = _run(x, wq, ws, bias, splits=splits)
    assert torch.equal(y1, y2), "split-K result is not deterministic"
    ref = orc.w4a16_reference(to_np_f32(x), wq.numpy(), ws.numpy(), bias.numpy())
    assert rel_max_err(to_np_f32(y1), ref) <= TOL


@pytest.mark.parametrize("M,N,K", [(7, 300, 512), (130, 640, 3072)])
def test_w4a16_bf16_mfma_matches_reference_bf16_path(M, N, K):
    """bf16 MFMA mode against the reference's own W4A16 path for a bf16 model: the dequantized
    weight cast back to bf16 (nodes.py:52, 116), then the matmul with fp32 accumulation. Only the
    fp32 summation order differs, so the gate is tight."""
    x, wq, ws = seeded_linear(M, N, K, seed=21)
    y = to_np_f32(_run(x, wq, ws, bf16_mfma=True))
    w_bf16 = orc.round_to_bf16(orc.dequant_int4(wq.numpy(), ws.numpy())).astype(np.float64)
    ref = to_np_f32(x).astype(np.float64) @ w_bf16.T
    assert rel_max_err(y, ref) <= 2e-5


def test_w4a16_fp32_activations():
    """fp32 x (the rotated path of int4_linear) goes through the fp16 staging: gate as fp32-dequant."""
    M, N, K = 33, 256, 1024
    g = torch.Generator().manual_seed(12)
    x = torch.randn(M, K, generator=g)
    _, wq, ws = seeded_linear(M, N, K, seed=13)
    y = to_np_f32(_run(x, wq, ws))
    ref = orc.w4a16_reference(x.numpy(), wq.numpy(), ws.numpy())
    assert rel_max_err(y, ref) <= TOL


def test_w4a16_exact_on_integer_grid():
    """Integer x in [-4, 4], codes in [-8, 7], power-of-two scales >= 2^-6, K = 256: every
    dequantized weight is exact in bf16 and every partial sum is a multiple of 2^-6 below 2^12,
    exact in fp32. The kernel must then equal the float64 oracle exactly."""
    M, N, K = 40, 300, 256
    g = np.random.default_rng(9)
    x = torch.from_numpy(g.integers(-4, 5, (M, K)).astype(np.float32)).to(torch.bfloat16)
    codes = g.integers(-8, 8, (N, K))
    nib = (codes & 0xF).astype(np.uint8)
    packed = (nib[:, 0::2] | (nib[:, 1::2] << 4)).view(np.int8)
    scale = (2.0 ** g.integers(-6, 0, (N, K // 32))).astype(np.float32)
    y = to_np_f32(_run(x, torch.from_numpy(packed), torch.from_numpy(scale)))
    ref = orc.w4a16_reference(to_np_f32(x), packed, scale)
    assert np.array_equal(y.astype(np.float64), ref), f"max abs diff {np.abs(y - ref).max()}"


def test_w4a16_golden_fixture():
    """Committed seeded case (tests/golden/w4a16_small.npz, written by make_golden.py from the
    oracle): the kernel must reproduce the stored fp64 reference within the gate."""
    d = np.load(golden_path("w4a16_small.npz"))
    x = torch.from_numpy(orc.bf16_bits_to_f32(d["x_bf16_bits"])).to(torch.bfloat16)
    y = to_np_f32(_run(x, torch.from_numpy(d["w_q4"]), torch.from_numpy(d["w_scale"]),
                       torch.from_numpy(d["bias"])))
    assert rel_max_err(y, d["y_ref"]) <= TOL


@pytest.mark.parametrize("M,K,N,xdt", [
    (4608, 3072, 3072, torch.float16),    # C1 shape
    (4608, 3072, 12288, torch.bfloat16),  # C2 fc1
    (4608, 12288, 3072, torch.bfloat16),  # C2 fc2
    (1, 4096, 10240, torch.bfloat16),     # C4 skinny
    (16, 4096, 10240, torch.bfloat16),
    (64, 4096, 10240, torch.bfloat16),
    (256, 4096, 10240, torch.bfloat16),
    (1, 3072, 18432, torch.bfloat16),     # C4 modulation
])
def test_w4a16_baseline_shapes_vs_torch_fp32(M, K, N, xdt):
    """Full-size BASELINE shapes against torch's fp32 GEMM of the fp32-dequantized weight (GPU)."""
    print(f"case full-size M={M} K={K} N={N}", flush=True)
    g = torch.Generator().manual_seed(0)
    x = torch.randn(M, K, generator=g).to(xdt).to(DEV)
    w = (torch.randn(N, K, generator=g) * 0.02).to(DEV)
    from comfy_ui_gfx906_tools_amd import ops
    wq, ws = ops.quantize_pack_int4(w)
    y = _lib().w4a16_gemm(x, wq, ws, out_dtype=torch.float32)
    ref = x.float() @ dequant_torch(wq, ws).t()
    err = ((y - ref).abs().max() / ref.abs().max()).item()
    del w
    assert err <= TOL, f"max rel err {err:.3e}"


# Every kernel configuration, forced through the flags field (QL_W4A16_CFG): 0-3 are the
# 4-wave kernel's 256/128/64/16-row tiles, 4-6 the 256 x 256 kernel's wave layouts.
ALL_CFGS = list(range(7))
TILE256_CFGS = [4, 5, 6]


def _run_cfg(x, wq, ws, bias=None, out_dtype=torch.float32, cfg=None, bf16_mfma=False):
    return _lib().w4a16_gemm(x.to(DEV), wq.to(DEV), ws.to(DEV), None if bias is None else bias.to(DEV),
                             out_dtype=out_dtype, bf16_mfma=bf16_mfma, config=cfg)


@pytest.mark.parametrize("cfg", ALL_CFGS)
@pytest.mark.parametrize("M,N,K,xdt", [(300, 200, 192, torch.bfloat16), (513, 777, 640, torch.float16),
                                       (256, 512, 3072, torch.bfloat16), (257, 300, 1024, torch.float16)])
def test_w4a16_every_config_vs_oracle(cfg, M, N, K, xdt):
    """Ragged M and N (tiles past the edges), bias, fp32 out: each configuration within the gate,
    and two runs bit-identical. M = 513 and 257 leave one row in the last 256-row tile, so on the
    256 x 256 kernel the second 128-row half of that tile lies wholly past M (regression: its
    activation descriptor once took a wrapped range past the end of x and faulted the GPU)."""
    print(f"case cfg={cfg} M={M} N={N} K={K} x={xdt}", flush=True)
    x, wq, ws = seeded_linear(M, N, K, seed=M + 3 * N + K + cfg, x_dtype=xdt)
    bias = torch.randn(N, generator=torch.Generator().manual_seed(cfg))
    y1 = _run_cfg(x, wq, ws, bias, cfg=cfg)
    y2 = _run_cfg(x, wq, ws, bias, cfg=cfg)
    assert torch.equal(y1, y2), "not deterministic"
    ref = orc.w4a16_reference(to_np_f32(x), wq.numpy(), ws.numpy(), bias.numpy())
    err = rel_max_err(to_np_f32(y1), ref)
    assert err <= TOL, f"cfg {cfg}: max rel err {err:.3e} > {TOL}"


@pytest.mark.parametrize("cfg", ALL_CFGS)
def test_w4a16_every_config_exact_on_integer_grid(cfg):
    """The exact-grid case of test_w4a16_exact_on_integer_grid through each configuration."""
    M, N, K = 290, 300, 256
    print(f"case exact grid cfg={cfg}", flush=True)
    g = np.random.default_rng(19 + cfg)
    x = torch.from_numpy(g.integers(-4, 5, (M, K)).astype(np.float32)).to(torch.bfloat16)
    codes = g.integers(-8, 8, (N, K))
    nib = (codes & 0xF).astype(np.uint8)
    packed = (nib[:, 0::2] | (nib[:, 1::2] << 4)).view(np.int8)
    scale = (2.0 ** g.integers(-6, 0, (N, K // 32))).astype(np.float32)
    y = to_np_f32(_run_cfg(x, torch.from_numpy(packed), torch.from_numpy(scale), cfg=cfg))
    ref = orc.w4a16_reference(to_np_f32(x), packed, scale)
    assert np.array_equal(y.astype(np.float64), ref), f"cfg {cfg}: max abs diff {np.abs(y - ref).max()}"


@pytest.mark.parametrize("cfg", TILE256_CFGS)
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16])
def test_w4a16_tile256_bf16_mfma_and_16bit_out(cfg, out_dtype):
    """bf16 MFMA mode (tight gate against the reference's bf16 dequant-then-matmul) and 16-bit
    outputs with bias (1 ulp + gate) on the 256 x 256 kernel."""
    M, N, K = 300, 520, 1024
    print(f"case tile256 cfg={cfg} out={out_dtype}", flush=True)
    x, wq, ws = seeded_linear(M, N, K, seed=23 + cfg)
    y = to_np_f32(_run_cfg(x, wq, ws, cfg=cfg, bf16_mfma=True))
    w_bf16 = orc.round_to_bf16(orc.dequant_int4(wq.numpy(), ws.numpy())).astype(np.float64)
    assert rel_max_err(y, to_np_f32(x).astype(np.float64) @ w_bf16.T) <= 2e-5
    bias = torch.randn(N, generator=torch.Generator().manual_seed(4)).to(out_dtype)
    y = to_np_f32(_run_cfg(x, wq, ws, bias, out_dtype=out_dtype, cfg=cfg))
    ref = orc.w4a16_reference(to_np_f32(x), wq.numpy(), ws.numpy(), to_np_f32(bias)).astype(np.float32)
    name = "bfloat16" if out_dtype == torch.bfloat16 else "float16"
    ref_r = orc.round_to_dtype(ref, name)
    ulp = bf16_ulp(ref_r) if out_dtype == torch.bfloat16 else f16_ulp(ref_r)
    bound = ulp + TOL * np.abs(ref).max()
    assert (np.abs(y - ref_r) <= bound).all(), f"max excess {(np.abs(y - ref_r) - bound).max():.3e}"


@pytest.mark.parametrize("cfg", TILE256_CFGS)
def test_w4a16_tile256_rejects_k_not_multiple_of_64(cfg):
    x, wq, ws = seeded_linear(64, 256, 96, seed=1)
    with pytest.raises(RuntimeError, match="K % 64"):
        _run_cfg(x, wq, ws, cfg=cfg)


def _gelu_tanh_f64(v: np.ndarray) -> np.ndarray:
    """GELU, tanh approximation, in float64 (the formula of torch.nn.functional.gelu(approximate="tanh"))."""
    v = v.astype(np.float64)
    return 0.5 * v * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (v + 0.044715 * v ** 3)))


@pytest.mark.parametrize("cfg", [None, 1, 3, 5])
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
def test_w4a16_fused_gelu_matches_unfused(cfg, out_dtype):
    """QL_W4A16_GELU_TANH: gelu_tanh(round(y)) in the epilogue. `plain` is the same kernel's output
    without the epilogue (the linear rounded to out_dtype); the fused result must equal the float64
    GELU of `plain`, rounded to out_dtype, within 1 ulp (16-bit) or 1e-5 relative + 1e-6 absolute
    (fp32: the epilogue evaluates 0.5 (1 + tanh(u)) as 1 / (1 + exp(-2u)) with the hardware exp2 and
    reciprocal). torch's unfused gelu on `plain` is also checked, within 2 ulp + 1e-6 absolute: its
    0.5 x (1 + tanh(u)) cancels in the negative tail (absolute error ~1e-7 there). M = 300 with cfg None takes the automatic plan,
    including K-cut tiles and their reduction for the 4-wave kernel."""
    M, N, K = (300, 1040, 1024) if cfg != 3 else (9, 700, 512)
    print(f"case gelu cfg={cfg} out={out_dtype}", flush=True)
    x, wq, ws = seeded_linear(M, N, K, seed=31, x_dtype=torch.bfloat16)
    bias = torch.randn(N, generator=torch.Generator().manual_seed(5)).to(out_dtype)
    plain = _run_cfg(x, wq, ws, bias, out_dtype=out_dtype, cfg=cfg)
    fused = _lib().w4a16_gemm(x.to(DEV), wq.to(DEV), ws.to(DEV), bias.to(DEV), out_dtype=out_dtype, config=cfg,
                              gelu=True)
    f = to_np_f32(fused)
    exact = _gelu_tanh_f64(to_np_f32(plain))
    r_torch = to_np_f32(torch.nn.functional.gelu(plain, approximate="tanh"))
    if out_dtype == torch.bfloat16:
        e = orc.round_to_dtype(exact.astype(np.float32), "bfloat16")
        ulp = bf16_ulp(e)
        assert (np.abs(f - e) <= ulp).all(), f"max diff vs exact {np.abs(f - e).max():.3e}"
        assert (np.abs(f - r_torch) <= 2 * bf16_ulp(r_torch) + 1e-6).all()
    else:
        assert (np.abs(f - exact) <= 1e-5 * np.abs(exact) + 1e-6).all(), f"max diff {np.abs(f - exact).max():.3e}"
        assert (np.abs(f - r_torch) <= 1e-5 * np.abs(r_torch) + 1e-6).all()


GEMV_CFG = 7


@pytest.mark.parametrize("M", [1, 2, 3, 4])
@pytest.mark.parametrize("N,K", [(1, 32), (3, 96), (17, 2048), (100, 4096), (257, 3072), (64, 8192)])
@pytest.mark.parametrize("xdt", [torch.bfloat16, torch.float16])
def test_w4a16_gemv_vs_oracle(M, N, K, xdt):
    """Configuration 7 (M <= 4, VALU dot products on exact codes): ragged N (wave columns past N),
    K with partial last groups-per-lane rounds (K = 3072: 96 groups over 64 lanes), bias, fp32 out;
    within the gate against the fp64 oracle, deterministic. The codes and x enter exactly and the
    scale is applied in fp32, so the error is far below the gate (checked at 2e-4)."""
    print(f"case gemv M={M} N={N} K={K} x={xdt}", flush=True)
    x, wq, ws = seeded_linear(M, N, K, seed=7 * M + N + K, x_dtype=xdt)
    bias = torch.randn(N, generator=torch.Generator().manual_seed(M))
    if M > 2 and K > 4096:  # the kernel keeps M x K activations in registers: M * K <= 16384
        with pytest.raises(RuntimeError, match="K <= 4096 for M > 2"):
            _run_cfg(x, wq, ws, bias, cfg=GEMV_CFG)
        return
    y1 = _run_cfg(x, wq, ws, bias, cfg=GEMV_CFG)
    y2 = _run_cfg(x, wq, ws, bias, cfg=GEMV_CFG)
    assert torch.equal(y1, y2), "not deterministic"
    ref = orc.w4a16_reference(to_np_f32(x), wq.numpy(), ws.numpy(), bias.numpy())
    err = rel_max_err(to_np_f32(y1), ref)
    assert err <= 2e-4, f"max rel err {err:.3e}"


def test_w4a16_gemv_exact_on_integer_grid():
    """Integer x, codes in [-8, 7], power-of-two scales: every partial sum is exact in fp32, so the
    VALU kernel must equal the fp64 oracle exactly (both dtypes)."""
    M, N, K = 4, 70, 2048
    g = np.random.default_rng(41)
    codes = g.integers(-8, 8, (N, K))
    nib = (codes & 0xF).astype(np.uint8)
    packed = (nib[:, 0::2] | (nib[:, 1::2] << 4)).view(np.int8)
    scale = (2.0 ** g.integers(-6, 0, (N, K // 32))).astype(np.float32)
    for xdt in (torch.bfloat16, torch.float16):
        x = torch.from_numpy(g.integers(-4, 5, (M, K)).astype(np.float32)).to(xdt)
        y = to_np_f32(_run_cfg(x, torch.from_numpy(packed), torch.from_numpy(scale), cfg=GEMV_CFG))
        ref = orc.w4a16_reference(to_np_f32(x), packed, scale)
        assert np.array_equal(y.astype(np.float64), ref), f"{xdt}: max abs diff {np.abs(y - ref).max()}"


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16])
def test_w4a16_gemv_16bit_out_gelu_and_row_scale(out_dtype):
    """16-bit outputs (1 ulp + gate), the fused GELU (1 ulp of the exact GELU of the plain output),
    and fp16 x staged by rows_to_f16 with its row scale, through configuration 7 and the automatic
    choice."""
    from comfy_ui_gfx906_tools_amd import _lib as L
    M, N, K = 3, 300, 3072
    x, wq, ws = seeded_linear(M, N, K, seed=51)
    bias = torch.randn(N, generator=torch.Generator().manual_seed(6)).to(out_dtype)
    ref = orc.w4a16_reference(to_np_f32(x), wq.numpy(), ws.numpy(), to_np_f32(bias)).astype(np.float32)
    name = "bfloat16" if out_dtype == torch.bfloat16 else "float16"
    ref_r = orc.round_to_dtype(ref, name)
    ulp = bf16_ulp(ref_r) if out_dtype == torch.bfloat16 else f16_ulp(ref_r)
    for cfg in (GEMV_CFG, None):
        y = to_np_f32(_run_cfg(x, wq, ws, bias, out_dtype=out_dtype, cfg=cfg))
        assert (np.abs(y - ref_r) <= ulp + 2e-4 * np.abs(ref).max()).all()
    plain = _run_cfg(x, wq, ws, bias, out_dtype=out_dtype, cfg=GEMV_CFG)
    fused = L.w4a16_gemm(x.to(DEV), wq.to(DEV), ws.to(DEV), bias.to(DEV), out_dtype=out_dtype, config=GEMV_CFG,
                         gelu=True)
    e = orc.round_to_dtype(_gelu_tanh_f64(to_np_f32(plain)).astype(np.float32), name)
    ue = bf16_ulp(e) if out_dtype == torch.bfloat16 else f16_ulp(e)
    assert (np.abs(to_np_f32(fused) - e) <= ue).all()
    x16, rs = L.rows_to_f16(x.to(DEV))
    y = to_np_f32(L.w4a16_gemm(x16, wq.to(DEV), ws.to(DEV), bias.to(DEV), out_dtype=out_dtype, row_scale=rs,
                               config=GEMV_CFG))
    assert (np.abs(y - ref_r) <= ulp + 2e-4 * np.abs(ref).max()).all()


SKINNY_CFG = 8


@pytest.mark.parametrize("M", [1, 5, 8, 9, 16])
@pytest.mark.parametrize("N,K", [(1, 128), (33, 256), (100, 4096), (257, 3072), (64, 384)])
@pytest.mark.parametrize("xdt", [torch.bfloat16, torch.float16])
def test_w4a16_skinny_vs_oracle(M, N, K, xdt):
    """Configuration 8 (M <= 16, MFMA on exact codes, K split over 8 waves; one 16-column block per
    workgroup up to M = 8, two above): ragged N (columns past N in the last workgroup), K slices of 4 to 16 groups with idle waves (K = 128: one slice), bias,
    fp32 out; deterministic and within 2e-4 of the fp64 oracle (exact products, fp32 sums)."""
    print(f"case skinny M={M} N={N} K={K} x={xdt}", flush=True)
    x, wq, ws = seeded_linear(M, N, K, seed=11 * M + N + K, x_dtype=xdt)
    bias = torch.randn(N, generator=torch.Generator().manual_seed(M))
    y1 = _run_cfg(x, wq, ws, bias, cfg=SKINNY_CFG)
    y2 = _run_cfg(x, wq, ws, bias, cfg=SKINNY_CFG)
    assert torch.equal(y1, y2), "not deterministic"
    ref = orc.w4a16_reference(to_np_f32(x), wq.numpy(), ws.numpy(), bias.numpy())
    err = rel_max_err(to_np_f32(y1), ref)
    assert err <= 2e-4, f"max rel err {err:.3e}"


@pytest.mark.parametrize("M,N,K", [(4, 5000, 1024), (16, 5000, 1024), (3, 6200, 3072), (16, 6200, 3072),
                                   (9, 12288, 4096), (16, 18432, 3072), (2, 3072, 3072)])
def test_w4a16_skinny_block_counts_vs_oracle(M, N, K):
    """The planner's choice of 16-column blocks per workgroup (on a 256-CU device: N = 5000 -> 2
    blocks, 157 workgroups; 6200 and 12288 -> 3 blocks, 130 and 256 workgroups; 18432 -> 2 above 8
    rows; 3072 -> 1), ragged last workgroups included: deterministic and within 2e-4 of the fp64
    oracle, as for the other skinny shapes."""
    print(f"case skinny blocks M={M} N={N} K={K}", flush=True)
    x, wq, ws = seeded_linear(M, N, K, seed=5 * M + N + K)
    bias = torch.randn(N, generator=torch.Generator().manual_seed(N))
    y1 = _run_cfg(x, wq, ws, bias, cfg=SKINNY_CFG)
    y2 = _run_cfg(x, wq, ws, bias)
    assert torch.equal(y1, y2), "automatic choice differs from configuration 8, or not deterministic"
    ref = orc.w4a16_reference(to_np_f32(x), wq.numpy(), ws.numpy(), bias.numpy())
    err = rel_max_err(to_np_f32(y1), ref)
    assert err <= 2e-4, f"max rel err {err:.3e}"


@pytest.mark.parametrize("M,K,msg", [(17, 256, "M <= 16"), (4, 160, "K % 128 == 0"), (4, 8192, "K <= 4096")])
def test_w4a16_skinny_rejects_unsupported_shapes(M, K, msg):
    x, wq, ws = seeded_linear(M, 8, K, seed=3)
    with pytest.raises(RuntimeError, match=msg):
        _run_cfg(x, wq, ws, cfg=SKINNY_CFG)


def test_w4a16_skinny_exact_on_integer_grid():
    """Integer x, codes in [-8, 7], power-of-two scales: every partial sum is exact in fp32, so the
    MFMA kernel must equal the fp64 oracle exactly (both dtypes; on a 256-CU device N = 70 runs on
    one-block workgroups at 8 rows and two-block ones at 16, N = 6200 on three-block ones)."""
    K = 1024
    g = np.random.default_rng(43)
    for M, N in ((8, 70), (16, 70), (16, 6200)):
        codes = g.integers(-8, 8, (N, K))
        nib = (codes & 0xF).astype(np.uint8)
        packed = (nib[:, 0::2] | (nib[:, 1::2] << 4)).view(np.int8)
        scale = (2.0 ** g.integers(-6, 0, (N, K // 32))).astype(np.float32)
        for xdt in (torch.bfloat16, torch.float16):
            x = torch.from_numpy(g.integers(-4, 5, (M, K)).astype(np.float32)).to(xdt)
            y = to_np_f32(_run_cfg(x, torch.from_numpy(packed), torch.from_numpy(scale), cfg=SKINNY_CFG))
            ref = orc.w4a16_reference(to_np_f32(x), packed, scale)
            assert np.array_equal(y.astype(np.float64), ref), f"M={M} {xdt}: max abs diff {np.abs(y - ref).max()}"


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16])
def test_w4a16_skinny_16bit_out_gelu_and_row_scale(out_dtype):
    """16-bit outputs (1 ulp + gate), the fused GELU (1 ulp of the exact GELU of the plain output),
    and fp16 x staged by rows_to_f16 with its row scale, through configuration 8 and the automatic
    choice (which takes configuration 8 for 2 <= M <= 16)."""
    from comfy_ui_gfx906_tools_amd import _lib as L
    M, N, K = 12, 300, 3072
    x, wq, ws = seeded_linear(M, N, K, seed=53)
    bias = torch.randn(N, generator=torch.Generator().manual_seed(7)).to(out_dtype)
    ref = orc.w4a16_reference(to_np_f32(x), wq.numpy(), ws.numpy(), to_np_f32(bias)).astype(np.float32)
    name = "bfloat16" if out_dtype == torch.bfloat16 else "float16"
    ref_r = orc.round_to_dtype(ref, name)
    ulp = bf16_ulp(ref_r) if out_dtype == torch.bfloat16 else f16_ulp(ref_r)
    for cfg in (SKINNY_CFG, None):
        y = to_np_f32(_run_cfg(x, wq, ws, bias, out_dtype=out_dtype, cfg=cfg))
        assert (np.abs(y - ref_r) <= ulp + 2e-4 * np.abs(ref).max()).all()
    plain = _run_cfg(x, wq, ws, bias, out_dtype=out_dtype, cfg=SKINNY_CFG)
    fused = L.w4a16_gemm(x.to(DEV), wq.to(DEV), ws.to(DEV), bias.to(DEV), out_dtype=out_dtype, config=SKINNY_CFG,
                         gelu=True)
    e = orc.round_to_dtype(_gelu_tanh_f64(to_np_f32(plain)).astype(np.float32), name)
    ue = bf16_ulp(e) if out_dtype == torch.bfloat16 else f16_ulp(e)
    assert (np.abs(to_np_f32(fused) - e) <= ue).all()
    x16, rs = L.rows_to_f16(x.to(DEV))
    y = to_np_f32(L.w4a16_gemm(x16, wq.to(DEV), ws.to(DEV), bias.to(DEV), out_dtype=out_dtype, row_scale=rs,
                               config=SKINNY_CFG))
    assert (np.abs(y - ref_r) <= ulp + 2e-4 * np.abs(ref).max()).all()

