"""The per-token int8 quantize fused into its producers (qlinear_adaln_modulate and
qlinear_heads_gather with QL_OPERAND_I8_PER_TOKEN): the adaLN row that feeds a W8A8 linear, and the
attention output gathered for the next linear, are written straight as the W8A8 GEMM's operand.

Pinned bit for bit against the unfused pair on the same GPU -- the plain adaLN output (x's dtype)
followed by qlinear_quantize_int8_per_token, the reference's per-token int8 rule (csrc/
int8_gemm.hip:215-246 widened to the row) -- codes and scales, for bf16 / fp16 / fp32 rows of
every register-tile width (K up to 16384), constant and large-magnitude rows; the plain output is
checked against a float64 LayerNorm + modulate within one rounding, and the W8A8 GEMM on the fused
operand against the GEMM on the unfused one (same bits).
"""
import pytest
import torch

from comfy_ui_gfx906_tools_amd import _lib

pytestmark = pytest.mark.gpu


def _adaln_ref(x, shift, scale, eps=1e-6):
    xd = x.double()
    mu = xd.mean(-1, keepdim=True)
    var = ((xd - mu) ** 2).mean(-1, keepdim=True)
    return (xd - mu) / torch.sqrt(var + eps) * (1 + scale.double()) + shift.double()


@pytest.mark.parametrize("M,K", [(1, 64), (7, 256), (300, 3072), (33, 4104), (5, 12288), (2, 16384)])
@pytest.mark.parametrize("xdt,mdt", [(torch.bfloat16, torch.bfloat16), (torch.float16, torch.float32),
                                     (torch.float32, torch.bfloat16)])
def test_adaln_i8_equals_plain_then_quantize(M, K, xdt, mdt):
    print(f"adaln i8 M={M} K={K} {xdt} {mdt}", flush=True)
    g = torch.Generator().manual_seed(M * 5 + K)
    x = (torch.randn(M, K, generator=g) * 3 + 0.5).to(xdt)
    if M >= 3:
        x[1] = 2.0  # constant row: LayerNorm gives 0, y = shift
        x[2] *= 1e3
    shift = (torch.randn(K, generator=g) * 0.5).to(mdt).cuda()
    scale = (torch.randn(K, generator=g) * 0.5).to(mdt).cuda()
    xc = x.cuda()
    plain = _lib.adaln_modulate(xc, shift, scale, out="plain")
    q, s = _lib.adaln_modulate(xc, shift, scale, out="i8")
    q_ref, s_ref = _lib.quantize_int8_per_token(plain)
    torch.cuda.synchronize()
    assert plain.dtype == xdt and q.dtype == torch.int8
    assert torch.equal(s, s_ref), f"scales differ: {(s - s_ref).abs().max().item()}"
    assert torch.equal(q, q_ref), f"{(q != q_ref).sum().item()} codes differ"
    # the plain row: one rounding to x's dtype of the fp32 computation
    ref = _adaln_ref(x.float(), shift.float().cpu(), scale.float().cpu())
    got = plain.cpu().double()
    tol = {torch.bfloat16: 2.0 ** -8, torch.float16: 2.0 ** -11, torch.float32: 2.0 ** -20}[xdt]
    assert bool(((got - ref).abs() <= tol * ref.abs() + 1e-4 * ref.abs().amax(-1, keepdim=True)).all())


def test_w8a8_on_fused_operand():
    """The W8A8 GEMM fed by the fused producer equals the GEMM fed by adaLN -> quantize."""
    M, K, N = 300, 3072, 1000
    g = torch.Generator(device="cuda").manual_seed(3)
    x = torch.randn(M, K, device="cuda", generator=g).to(torch.bfloat16)
    shift = (torch.randn(K, device="cuda", generator=g) * 0.3).to(torch.bfloat16)
    scale = (torch.randn(K, device="cuda", generator=g) * 0.3).to(torch.bfloat16)
    wq, sw = _lib.quantize_int8_per_token(torch.randn(N, K, device="cuda", generator=g) * 0.02)
    q, s = _lib.adaln_modulate(x, shift, scale, out="i8")
    q2, s2 = _lib.quantize_int8_per_token(_lib.adaln_modulate(x, shift, scale, out="plain"))
    y = _lib.w8a8_gemm(q, s, wq, sw, out_dtype=torch.bfloat16)
    assert torch.equal(y, _lib.w8a8_gemm(q2, s2, wq, sw, out_dtype=torch.bfloat16))


def test_adaln_modulate_argument_checks():
    x = torch.zeros(4, 64, device="cuda", dtype=torch.bfloat16)
    sh = torch.zeros(64, device="cuda", dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="out must be"):
        _lib.adaln_modulate(x, sh, sh, out="int4")
    lib = _lib.load_library()
    assert lib.qlinear_adaln_modulate(7, 2, x.data_ptr(), 2, sh.data_ptr(), sh.data_ptr(), x.data_ptr(), None, 4, 64,
                                      1e-6, None) != 0
    assert "out_kind" in lib.qlinear_last_error().decode()
    # int8 output needs its scales
    assert lib.qlinear_adaln_modulate(2, 2, x.data_ptr(), 2, sh.data_ptr(), sh.data_ptr(), x.data_ptr(), None, 4, 64,
                                      1e-6, None) != 0


@pytest.mark.parametrize("H,L,l0,rows,E,dt", [(24, 700, 100, 512, 0, torch.bfloat16), (24, 300, 0, 300, 256, torch.float16),
                                             (8, 64, 3, 17, 8, torch.bfloat16)])
def test_heads_gather_i8_equals_plain_then_quantize(H, L, l0, rows, E, dt):
    """The attention-output gather: the plain rows equal torch's transpose + concatenation, and the
    int8 operand equals qlinear_quantize_int8_per_token of them bit for bit."""
    print(f"heads gather i8 H={H} L={L} l0={l0} rows={rows} E={E} {dt}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(H + L + E)
    o = torch.randn(H, L, 128, device="cuda", generator=g).to(dt)
    extra = torch.randn(rows, E, device="cuda", generator=g).to(dt) if E else None
    plain = _lib.heads_gather(o, l_offset=l0, rows=rows, extra=extra, out="plain")
    ref = o[:, l0:l0 + rows].permute(1, 0, 2).reshape(rows, H * 128)
    if extra is not None:
        ref = torch.cat([ref, extra], dim=1)
    assert torch.equal(plain, ref)
    q, s = _lib.heads_gather(o, l_offset=l0, rows=rows, extra=extra, out="i8")
    q_ref, s_ref = _lib.quantize_int8_per_token(plain)
    assert torch.equal(s, s_ref) and torch.equal(q, q_ref)
    x16, rs = _lib.heads_gather(o, l_offset=l0, rows=rows, extra=extra, out="f16")
    x16b, rsb = _lib.heads_to_f16(o, l_offset=l0, rows=rows, extra=extra)
    assert torch.equal(x16, x16b) and torch.equal(rs, rsb)
