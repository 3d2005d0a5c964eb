"""The W4A4 GEMM (the reference's production numerics, csrc/w4a4_gemm.hip) through the C ABI,
bit-exact against the oracle's restatement of gemm_int4 (per-block int32 dot, fmaf(float(ip),
as * bs, acc) in K order, + bias; oracle/qlinear_oracle.py gemm_int4_w4a4, pinned on the CPU), and
the reference's whole int4_linear (quantize_int4 + gemm_int4) through the extension surface."""
import numpy as np
import pytest
import torch

from comfy_ui_gfx906_tools_amd import _lib, ext, ops
from oracle import qlinear_oracle as orc

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _operands(M, N, K, qblock, seed):
    g = np.random.default_rng(seed)
    a = g.integers(-8, 8, (M, K))
    b = g.integers(-8, 8, (N, K))
    pack = lambda c: ((c[:, 0::2] & 0xF) | ((c[:, 1::2] & 0xF) << 4)).astype(np.uint8).view(np.int8)
    sa = (2.0 ** g.uniform(-12, -2, (M, K // qblock))).astype(np.float32)
    sb = (2.0 ** g.uniform(-12, -2, (N, K // qblock))).astype(np.float32)
    sa[0, 0] = 0.0  # an all-zero activation block (scale 0)
    return pack(a), sa, pack(b), sb


def _ref(ap, sa, bp, sb, bias, qblock):
    return orc.gemm_int8_block32(orc.unpack_int4(ap), sa, orc.unpack_int4(bp), sb, bias, qblock)


@pytest.mark.parametrize("M,N,K", [(1, 64, 32), (37, 100, 96), (130, 257, 640), (300, 520, 1024), (129, 128, 160)])
@pytest.mark.parametrize("qblock", [32, 16])
def test_w4a4_bit_exact_fp32(M, N, K, qblock):
    print(f"w4a4 M={M} N={N} K={K} qblock={qblock}", flush=True)
    ap, sa, bp, sb = _operands(M, N, K, qblock, seed=M * 7 + N + K + qblock)
    bias = np.random.default_rng(1).standard_normal(N).astype(np.float32)
    y = _lib.w4a4_gemm(*(torch.from_numpy(t).to(DEV) for t in (ap, sa, bp, sb)), torch.from_numpy(bias).to(DEV),
                       out_dtype=torch.float32, qblock=qblock)
    ref = _ref(ap, sa, bp, sb, bias, qblock)
    assert np.array_equal(y.cpu().numpy(), ref), f"max abs diff {np.abs(y.cpu().numpy() - ref).max()}"
    y0 = _lib.w4a4_gemm(*(torch.from_numpy(t).to(DEV) for t in (ap, sa, bp, sb)), None, qblock=qblock)
    assert np.array_equal(y0.cpu().numpy(), _ref(ap, sa, bp, sb, None, qblock))


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16])
def test_w4a4_16bit_out_is_the_rounded_fp32_result(out_dtype):
    M, N, K = 77, 200, 256
    ap, sa, bp, sb = _operands(M, N, K, 32, seed=5)
    bias = torch.randn(N, generator=torch.Generator().manual_seed(2)).to(out_dtype)
    y = _lib.w4a4_gemm(*(torch.from_numpy(t).to(DEV) for t in (ap, sa, bp, sb)), bias.to(DEV), out_dtype=out_dtype)
    ref = torch.from_numpy(_ref(ap, sa, bp, sb, bias.float().numpy(), 32)).to(out_dtype)
    assert torch.equal(y.cpu(), ref)


@pytest.mark.parametrize("M,K,N", [(64, 3072, 96), (300, 512, 520)])
def test_reference_int4_linear_w4a4_bit_exact(M, K, N):
    """ops.int4_linear_w4a4 = the reference's int4_linear: activation quantize by the reference
    kernel's rule (amax * fl(1/7), rint), W4A4 GEMM, bias in x.dtype, output in x.dtype."""
    g = torch.Generator().manual_seed(M + K)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    w = torch.randn(N, K, generator=g) * 0.02
    bias = (torch.randn(N, generator=g) * 0.1).to(torch.bfloat16)
    wp, ws = orc.quantize_pack_int4(w.numpy(), rule="div")
    y = ops.int4_linear_w4a4(x.to(DEV), torch.from_numpy(wp).to(DEV), torch.from_numpy(ws).to(DEV), bias.to(DEV))
    xp, xs = orc.quantize_pack_int4(x.float().numpy(), rule="recip")
    # gemm_int4's default splits = 0: the reference's auto_splits for this GPU's CU count
    cus = torch.cuda.get_device_properties(DEV).multi_processor_count
    splits = orc.reference_auto_splits(M, N, K, cus)
    assert ext.gemm_int4_auto_splits(M, N, K) == splits
    ref = torch.from_numpy(orc.gemm_int4_w4a4(xp, xs, wp, ws, bias.float().numpy(), splits=splits)).to(torch.bfloat16)
    assert y.dtype == torch.bfloat16 and torch.equal(y.cpu(), ref)


@pytest.mark.parametrize("M,N,K,splits", [(37, 100, 1024, 2), (130, 257, 640, 3), (1, 64, 32, 8), (64, 96, 3072, 0),
                                          (200, 130, 4096, 8), (300, 520, 1024, 5)])
@pytest.mark.parametrize("qblock", [32, 16])
@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
def test_w4a4_split_k_bit_exact(M, N, K, splits, qblock, out_dtype):
    """gemm_int4 with split-K: per-split fp32 partials from 0, summed in split order, + bias -- the
    reference's association (oracle gemm_split_k), bit for bit; splits = 0 resolves to the
    reference's auto_splits; K = 32 with 8 splits leaves seven splits empty."""
    print(f"w4a4 split M={M} N={N} K={K} splits={splits} qblock={qblock} out={out_dtype}", flush=True)
    ap, sa, bp, sb = _operands(M, N, K, qblock, seed=M + N + K + splits + qblock)
    bias = np.random.default_rng(3).standard_normal(N).astype(np.float32)
    bias_t = torch.from_numpy(bias).to(out_dtype)
    y = ext.gemm_int4(*(torch.from_numpy(t).to(DEV) for t in (ap, sa, bp, sb)), bias_t.to(DEV), out_dtype,
                      splits=splits, qblock=qblock)
    eff = splits or orc.reference_auto_splits(M, N, K, torch.cuda.get_device_properties(DEV).multi_processor_count)
    ref = orc.gemm_split_k(orc.unpack_int4(ap), sa, orc.unpack_int4(bp), sb, bias_t.float().numpy(), qblock, eff)
    assert torch.equal(y.cpu(), torch.from_numpy(ref).to(out_dtype)), \
        f"max abs diff {np.abs(y.float().cpu().numpy() - ref).max()}"


def test_w4a4_c1_shape_rows_match():
    """C1 shape (x [4608, 3072], W [3072, 3072]): every row is independent, so rows at both ends
    are checked against the oracle."""
    M, K, N = 4608, 3072, 3072
    ap, sa, bp, sb = _operands(M, N, K, 32, seed=11)
    y = _lib.w4a4_gemm(*(torch.from_numpy(t).to(DEV) for t in (ap, sa, bp, sb)), None).cpu().numpy()
    for rows in (slice(0, 40), slice(M - 40, M)):
        assert np.array_equal(y[rows], _ref(ap[rows], sa[rows], bp, sb, None, 32))


def test_ext_surface_errors():
    a = torch.zeros(4, 16, dtype=torch.int8, device=DEV)
    s = torch.ones(4, 1, device=DEV)
    with pytest.raises(RuntimeError, match="qblock"):
        ext.gemm_int4(a, s, a, s, None, torch.float32, qblock=8)
    with pytest.raises(RuntimeError, match="splits"):
        ext.gemm_int4(a, s, a, s, None, torch.float32, splits=9)
    with pytest.raises(RuntimeError, match="bias dtype"):
        ext.gemm_int4(a, s, a, s, torch.zeros(4, device=DEV), torch.bfloat16)
    with pytest.raises(RuntimeError, match="scales must be"):
        ext.gemm_int4(a, torch.ones(4, 2, device=DEV), a, s, None, torch.float32)
    assert ext.gemm_int4_auto_splits(4608, 3072, 3072) == 1


@pytest.mark.parametrize("M,K", [(1, 32), (7, 96), (300, 3072)])
@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16, torch.float32])
def test_quantize_int8_block32_bit_exact(M, K, dt):
    x = (torch.randn(M, K, generator=torch.Generator().manual_seed(M + K)) * 4).to(dt)
    x[0, :32] = 0.0
    q, s = ext.quantize_int8(x.to(DEV))
    q_ref, s_ref = orc.quantize_int8_rows(x.float().numpy(), block=32)
    assert np.array_equal(q.cpu().numpy(), q_ref) and np.array_equal(s.cpu().numpy(), s_ref)


@pytest.mark.parametrize("M,N,K", [(1, 64, 32), (37, 100, 96), (130, 257, 640), (300, 520, 1056)])
@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
def test_gemm_int8_block32_bit_exact(M, N, K, out_dtype):
    """The reference's gemm_int8 (block-32 scales both sides, per-block fmaf in K order, + bias)."""
    print(f"gemm_int8 M={M} N={N} K={K} {out_dtype}", flush=True)
    g = np.random.default_rng(M + N + K)
    a = g.integers(-127, 128, (M, K)).astype(np.int8)
    b = g.integers(-127, 128, (N, K)).astype(np.int8)
    sa = (2.0 ** g.uniform(-14, -4, (M, K // 32))).astype(np.float32)
    sb = (2.0 ** g.uniform(-14, -4, (N, K // 32))).astype(np.float32)
    bias = torch.randn(N, generator=torch.Generator().manual_seed(3)).to(out_dtype)
    y = ext.gemm_int8(*(torch.from_numpy(t).to(DEV) for t in (a, sa, b, sb)), bias.to(DEV), out_dtype)
    ref = torch.from_numpy(orc.gemm_int8_block32(a, sa, b, sb, bias.float().numpy(), 32)).to(out_dtype)
    assert torch.equal(y.cpu(), ref)


def test_reference_int8_linear_pipeline_bit_exact():
    """quantize_int8 of x and W, then gemm_int8: the reference's int8 linear, bit-exact."""
    M, N, K = 200, 300, 1024
    g = torch.Generator().manual_seed(9)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    w = torch.randn(N, K, generator=g) * 0.02
    qa, sa = ext.quantize_int8(x.to(DEV))
    qb, sb = ext.quantize_int8(w.to(DEV))
    y = ext.gemm_int8(qa, sa, qb, sb, None, torch.float32)
    a_ref, sa_ref = orc.quantize_int8_rows(x.float().numpy(), block=32)
    b_ref, sb_ref = orc.quantize_int8_rows(w.numpy(), block=32)
    assert np.array_equal(y.cpu().numpy(), orc.gemm_int8_block32(a_ref, sa_ref, b_ref, sb_ref, None, 32))
