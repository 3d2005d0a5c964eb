"""Weight dynamic range of the W4A16 tile kernels (configurations 0-6, the fp16 dequant route).

The reference dequantizes to the model's dtype (bf16, nodes/ComfyUI-Gfx906Int4/nodes.py:116),
which keeps fp32's exponent range. The tile kernels round q * s to fp16 instead, so without
help a group scale above ~8188 overflows (8 * 8188 > 65504) and one below ~2^-14 / 8 puts its
small codes into fp16's subnormals. Each output column therefore carries a power-of-two factor
(qlinear_w4a16_col_scales): these tests pin that every configuration meets the 2e-3 gate against
the float64 dequant-then-matmul oracle with group scales anywhere in [2^-24, 2^14], and that the
factors change nothing where the plain fp16 dequant was already exact in range.
"""
import numpy as np
import pytest
import torch

from oracle import qlinear_oracle as orc
from tests.gpu_util import rel_max_err, to_np_f32

pytestmark = pytest.mark.gpu
TOL = 2e-3
DEV = "cuda:0"


def _lib():
    from comfy_ui_gfx906_tools_amd import _lib
    return _lib


def _pack(codes: np.ndarray) -> np.ndarray:
    nib = (codes & 0xF).astype(np.uint8)
    return (nib[:, 0::2] | (nib[:, 1::2] << 4)).view(np.int8)


def _scales(pattern: str, N: int, G: int, rng: np.random.Generator) -> np.ndarray:
    """Group scales [N, G] spanning fp32 ranges that fp16 cannot hold unscaled."""
    base = np.exp(rng.normal(0.0, 0.3, (N, G)))  # within-column spread of a few tens of percent
    if pattern == "tiny":        # the whole layer at 2^-24 .. 2^-18: q * s below fp16's normal range
        e = rng.integers(-24, -17, (N, 1))
    elif pattern == "huge":      # 2^10 .. 2^14: 8 s above fp16's maximum for most groups
        e = rng.integers(10, 15, (N, 1))
    elif pattern == "one_huge_column":  # a normal layer (s ~ 0.01) with one column at 2^14
        e = np.full((N, 1), -7)
        e[N // 3] = 14
    elif pattern == "mixed_columns":    # every column its own exponent in [-24, 14]
        e = rng.integers(-24, 15, (N, 1))
    elif pattern == "wide_groups":      # exponents per group: 2^12 of range inside each column
        e = rng.integers(-6, 7, (N, G)) + rng.integers(-18, 8, (N, 1))
    else:
        raise ValueError(pattern)
    return (base * 2.0 ** e).astype(np.float32)


def _layer(pattern: str, M: int, N: int, K: int, seed: int, xdt=torch.bfloat16):
    rng = np.random.default_rng(seed)
    x = torch.from_numpy(rng.normal(0.0, 1.0, (M, K)).astype(np.float32)).to(xdt)
    codes = rng.integers(-8, 8, (N, K))
    return x, _pack(codes), _scales(pattern, N, K // 32, rng)


PATTERNS = ["tiny", "huge", "one_huge_column", "mixed_columns", "wide_groups"]


@pytest.mark.parametrize("cfg", [None, 0, 1, 2, 3, 4, 5, 6])
@pytest.mark.parametrize("pattern", PATTERNS)
def test_w4a16_weight_range_every_config(pattern, cfg):
    """Ragged M and N, fp32 out: every tile configuration within the gate for scales of any
    magnitude, finite everywhere, and the per-column error bounded by the column's own magnitude
    (a tiny column next to a huge one keeps its precision)."""
    M, N, K = 300, 264, 640
    print(f"case weight range {pattern} cfg={cfg}", flush=True)
    x, packed, scale = _layer(pattern, M, N, K, seed=PATTERNS.index(pattern) * 10 + (cfg or 0))
    y = to_np_f32(_lib().w4a16_gemm(x.to(DEV), torch.from_numpy(packed).to(DEV), torch.from_numpy(scale).to(DEV),
                                    out_dtype=torch.float32, config=cfg))
    ref = orc.w4a16_reference(to_np_f32(x), packed, scale)
    assert np.isfinite(y).all(), f"{pattern} cfg {cfg}: non-finite outputs"
    err = rel_max_err(y, ref)
    assert err <= TOL, f"{pattern} cfg {cfg}: max rel err {err:.3e} > {TOL}"
    col_err = np.abs(y - ref).max(axis=0) / np.maximum(np.abs(ref).max(axis=0), 1e-300)
    if pattern != "wide_groups":  # there the column's small groups may sit below fp16 after scaling
        assert col_err.max() <= TOL, f"{pattern} cfg {cfg}: worst column rel err {col_err.max():.3e}"


@pytest.mark.parametrize("pattern", ["tiny", "huge", "mixed_columns"])
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16])
def test_w4a16_weight_range_16bit_out(pattern, out_dtype):
    """16-bit outputs of the default route: within 1 ulp + gate of the rounded oracle where the
    oracle's value is representable (fp16 outputs above 65504 are inf there too)."""
    M, N, K = 200, 320, 512
    x, packed, scale = _layer(pattern, M, N, K, seed=77)
    if out_dtype == torch.float16:  # keep the outputs inside fp16's range (a power-of-two rescale)
        top = np.abs(orc.w4a16_reference(to_np_f32(x), packed, scale)).max()
        scale = (scale * 2.0 ** -max(0, int(np.ceil(np.log2(top))) - 14)).astype(np.float32)
    y = to_np_f32(_lib().w4a16_gemm(x.to(DEV), torch.from_numpy(packed).to(DEV), torch.from_numpy(scale).to(DEV),
                                    out_dtype=out_dtype))
    ref = orc.w4a16_reference(to_np_f32(x), packed, scale).astype(np.float32)
    name = "bfloat16" if out_dtype == torch.bfloat16 else "float16"
    ref_r = orc.round_to_dtype(ref, name).astype(np.float64)
    a = np.abs(ref_r)
    if out_dtype == torch.bfloat16:
        ulp = 2.0 ** (np.floor(np.log2(np.maximum(a, 2.0 ** -126))) - 7)
    else:
        ulp = 2.0 ** (np.floor(np.log2(np.maximum(a, 2.0 ** -14))) - 10)
    bound = ulp + TOL * np.abs(ref).max()
    assert np.isfinite(y).all()
    assert (np.abs(y - ref_r) <= bound).all(), f"max excess {(np.abs(y - ref_r) - bound).max():.3e}"


def test_w4a16_col_scales_properties():
    """qlinear_w4a16_col_scales: 1 where every code's q * s is already a normal fp16 number
    (nonzero |s| >= 2^-14 and 8 max|s| <= 65504), else a power of two c with 8 max|s| / c in
    [2^14, 2^15); 1 for an all-zero column; independent of the scales' signs (Q4_0 d may be
    negative)."""
    rng = np.random.default_rng(5)
    N, G = 40, 24
    s = (np.exp(rng.normal(0, 2, (N, G))) * 2.0 ** rng.integers(-30, 30, (N, 1))).astype(np.float32)
    s[3] = 0.0
    s[4] = -np.abs(s[4])
    s[5, 7] = 3.0e38  # near fp32's top: 2^116, finite
    s[6] = np.float32(2.0 ** -130)  # fp32 subnormal scales: the factor stops at 2^-126
    s[7] = 0.01  # ordinary scales: in range, factor 1
    s[8] = 0.01
    s[8, 3] = 2.0 ** -15  # one tiny group takes the column out of range
    s[9] = 8188.0  # 8 s = 65504: still in range
    s[10] = 8189.0  # just above
    c = _lib().w4a16_col_scales(torch.from_numpy(s).to(DEV)).cpu().numpy().astype(np.float64)
    m, e = np.frexp(c)
    assert np.all(m == 0.5), "factors must be powers of two"
    assert c[3] == 1.0 and c[5] == 2.0 ** 116 and c[6] == 2.0 ** -126 and c[7] == 1.0 and c[9] == 1.0
    a = np.abs(s).astype(np.float64)
    amax = a.max(axis=1)
    amin = np.where(a > 0, a, np.inf).min(axis=1)
    in_range = (amin >= 2.0 ** -14) & (8.0 * amax <= 65504.0)
    assert not in_range[8] and not in_range[10] and in_range[7] and in_range[9]
    assert np.all(c[in_range] == 1.0)
    ok = ~in_range
    ok[[6]] = False
    r = 8.0 * amax[ok] / c[ok]
    assert np.all((r >= 2.0 ** 14) & (r < 2.0 ** 15)), r


def test_w4a16_col_scales_change_nothing_in_range():
    """Normal weights (N(0, 0.02), the reference's own quantizer): every factor is 1, and the
    GEMM equals, bit for bit, the same GEMM given explicit factors of 1 or factors of 2^-3 (rounding
    to fp16 commutes with a power-of-two scale while q * s stays a normal fp16 number; 2^-3 keeps
    8 max|s| * 8 far below 65504), for whole tiles, K-cut tiles and the 256 x 256 kernel, on the
    plain and on the column-scaled epilogue; the cached factors equal the computed ones."""
    L = _lib()
    g = torch.Generator().manual_seed(3)
    M, N, K = 330, 640, 1536
    x = torch.randn(M, K, generator=g).to(torch.bfloat16).to(DEV)
    w = torch.randn(N, K, generator=g) * 0.02
    packed, scale = orc.quantize_pack_int4(w.numpy())
    wq, ws = torch.from_numpy(packed).to(DEV), torch.from_numpy(scale).to(DEV)
    ones = torch.ones(N, dtype=torch.float32, device=DEV)
    assert torch.equal(L.w4a16_col_scales(ws), ones)
    eighth = torch.full((N,), 0.125, dtype=torch.float32, device=DEV)
    half_eighth = ones.clone()
    half_eighth[N // 2:] = 0.125  # tiles with both kinds of columns
    for cfg, splits in [(None, 0), (1, 0), (1, 3), (2, 0), (4, 0), (5, 0), (6, 0)]:
        for out_dtype in (torch.float32, torch.bfloat16):
            y_auto = L.w4a16_gemm(x, wq, ws, out_dtype=out_dtype, config=cfg, splits=splits)
            for cs in (ones, eighth, half_eighth, L.cached_col_scales(ws)):
                y = L.w4a16_gemm(x, wq, ws, out_dtype=out_dtype, config=cfg, splits=splits, col_scale=cs)
                assert torch.equal(y_auto, y), f"cfg {cfg} splits {splits} {out_dtype} factors {cs[0].item()}"


def test_cached_col_scales_follow_in_place_updates():
    """The cache kept on the scale tensor is recomputed after an in-place change."""
    L = _lib()
    ws = torch.full((8, 4), 0.01, dtype=torch.float32, device=DEV)
    c1 = L.cached_col_scales(ws).clone()
    assert L.cached_col_scales(ws) is L.cached_col_scales(ws)
    assert torch.equal(c1, torch.ones(8, device=DEV))
    ws.mul_(2.0 ** 20)  # 8 * 10485.76 > 65504: out of fp16's range now
    c2 = L.cached_col_scales(ws)
    assert torch.equal(c2, L.w4a16_col_scales(ws)) and not torch.equal(c2, c1)
