"""The fused DiT glue kernels (csrc/dit_fused.hip) through the C ABI, against float64 torch
restatements of the ops they replace (the torch path of comfy_ui_gfx906_tools_amd/flux_dit.py):
adaLN modulate into the row-scaled fp16 GEMM operand, QK RMSNorm + RoPE + head split, gated
residual. Bounds: one rounding to the output type plus fp32 arithmetic."""
import numpy as np
import pytest
import torch

from comfy_ui_gfx906_tools_amd import _lib, flux_dit as fd

pytestmark = pytest.mark.gpu


def _adaln_ref(x, shift, scale, eps=1e-6):
    xd = x.double()
    mu = xd.mean(-1, keepdim=True)
    var = ((xd - mu) ** 2).mean(-1, keepdim=True)
    return (xd - mu) / torch.sqrt(var + eps) * (1 + scale.double()) + shift.double()


@pytest.mark.parametrize("M,K", [(1, 64), (7, 256), (300, 3072), (33, 4104), (5, 12288), (2, 16384)])
@pytest.mark.parametrize("xdt,mdt", [(torch.bfloat16, torch.bfloat16), (torch.float16, torch.float32),
                                     (torch.float32, torch.bfloat16)])
def test_adaln_modulate_f16(M, K, xdt, mdt):
    print(f"adaln M={M} K={K} {xdt} {mdt}", flush=True)
    g = torch.Generator().manual_seed(M * 7 + K)
    x = (torch.randn(M, K, generator=g) * 3 + 0.5).to(xdt)
    if M >= 3:
        x[1] = 2.0  # constant row: LayerNorm gives 0, y = shift
        x[2] *= 1e3
    shift = (torch.randn(K, generator=g) * 0.5).to(mdt)
    scale = (torch.randn(K, generator=g) * 0.5).to(mdt)
    x16, rs = _lib.adaln_modulate_f16(x.cuda(), shift.cuda(), scale.cuda())
    torch.cuda.synchronize()
    x16, rs = x16.cpu().double(), rs.cpu().double()
    ref = _adaln_ref(x.float(), shift.float(), scale.float())
    # row factors are powers of two putting each row's max into [2^14, 2^15] (2^15 only when the
    # fp16 rounding of a value just below it carries up)
    assert torch.all(torch.log2(rs) == torch.round(torch.log2(rs)))
    amax = x16.abs().amax(-1)
    assert torch.all((amax >= 2.0 ** 14) & (amax <= 2.0 ** 15)), amax
    y = x16 * rs[:, None]
    rowmax = ref.abs().amax(-1, keepdim=True)
    bound = 2.0 ** -11 * ref.abs() + 2.0 ** -24 * rs[:, None] + 1e-5 * rowmax
    assert torch.all((y - ref).abs() <= bound), float(((y - ref).abs() - bound).max())


@pytest.mark.parametrize("L,H,L_out,l0", [(1, 1, 1, 0), (5, 3, 12, 4), (130, 24, 130, 0), (77, 2, 100, 23)])
@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
def test_qk_norm_rope(L, H, L_out, l0, dt):
    print(f"qk_norm_rope L={L} H={H} L_out={L_out} l0={l0} {dt}", flush=True)
    D = 128
    g = torch.Generator().manual_seed(L * 31 + H)
    qkv = (torch.randn(L, 3 * H * D, generator=g) * 2).to(dt)
    qn = (1 + 0.3 * torch.randn(D, generator=g)).to(dt)
    kn = (1 + 0.3 * torch.randn(D, generator=g)).to(dt)
    ids = torch.stack([torch.zeros(L_out), torch.arange(L_out) % 7, torch.arange(L_out) // 7], -1)[None].float()
    cos, sin = fd.rope_cos_sin(ids, (16, 56, 56), 10000.0)
    cos, sin = cos[0, 0], sin[0, 0]
    sentinel = torch.full((H, L_out, D), 7.0, dtype=dt)
    out = tuple(sentinel.clone().cuda() for _ in range(3))
    _lib.qk_norm_rope(qkv.cuda(), qn.cuda(), kn.cuda(), cos.cuda(), sin.cuda(), H, out=out, l_offset=l0)
    torch.cuda.synchronize()
    q, k, v = (t.cpu() for t in out)
    t = qkv.double().view(L, 3, H, D).permute(1, 2, 0, 3)  # [3, H, L, D]
    cd, sd = cos[l0:l0 + L].double(), sin[l0:l0 + L].double()
    for got, x, w in ((q, t[0], qn), (k, t[1], kn)):
        y = x / torch.sqrt((x ** 2).mean(-1, keepdim=True) + 1e-6) * w.double()
        y0, y1 = y[..., 0::2], y[..., 1::2]
        ref = torch.stack([cd * y0 - sd * y1, sd * y0 + cd * y1], -1).flatten(-2)
        gd = got[:, l0:l0 + L].double()
        bound = 2.0 ** -8 * ref.abs() + 1e-5 * ref.abs().amax(-1, keepdim=True)
        assert torch.all((gd - ref).abs() <= bound)
    assert torch.equal(v[:, l0:l0 + L], t[2].to(dt))
    for got in (q, k, v):  # rows outside [l0, l0 + L) untouched
        assert torch.equal(got[:, :l0], sentinel[:, :l0]) and torch.equal(got[:, l0 + L:], sentinel[:, l0 + L:])


@pytest.mark.parametrize("M,K", [(1, 8), (3, 3072), (4608, 3072), (1000, 15360)])
@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16, torch.float32])
def test_gated_residual_bit_exact(M, K, dt):
    """out = x + gate * y, each op rounded in fp32 (torch's fp32 composition), then once to dt."""
    print(f"gated_residual M={M} K={K} {dt}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(M + K)
    x = torch.randn(M, K, device="cuda", generator=g).to(dt)
    y = torch.randn(M, K, device="cuda", generator=g).to(dt)
    gate = torch.randn(K, device="cuda", generator=g).to(dt)
    ref = (x.float() + gate.float() * y.float()).to(dt)
    out = _lib.gated_residual(x, gate, y)
    assert torch.equal(out, ref)
    x2 = x.clone()
    assert _lib.gated_residual(x2, gate, y, out=x2).data_ptr() == x2.data_ptr()
    torch.cuda.synchronize()
    assert torch.equal(x2, ref)


def test_engine_blocks_leave_inputs_unchanged():
    cfg = fd.FluxDiTConfig.tiny()
    with torch.no_grad():
        m = fd.FluxDiT(cfg, device="cuda", dtype=torch.bfloat16)
        fd.init_random_(m, seed=2)
        img = torch.randn(1, 64, cfg.hidden, device="cuda").to(torch.bfloat16)
        txt = torch.randn(1, 16, cfg.hidden, device="cuda").to(torch.bfloat16)
        vec = torch.randn(1, cfg.hidden, device="cuda").to(torch.bfloat16)
        ids = torch.zeros(1, 80, 3, device="cuda")
        cos, sin = fd.rope_cos_sin(ids, cfg.axes_dim, cfg.theta)
        i0, t0 = img.clone(), txt.clone()
        m.double_blocks[0](img, txt, vec, cos, sin)
        x = torch.cat([txt, img], 1)
        x0 = x.clone()
        m.single_blocks[0](x, vec, cos, sin)
        torch.cuda.synchronize()
    assert torch.equal(img, i0) and torch.equal(txt, t0) and torch.equal(x, x0)


@pytest.mark.parametrize("H,L,l0,rows,E", [(1, 5, 0, 5, 0), (24, 300, 40, 260, 0), (2, 64, 0, 64, 512),
                                           (24, 130, 0, 130, 12288)])
@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
def test_heads_to_f16(H, L, l0, rows, E, dt):
    """Head-major attention rows (+ a second source) into the row-scaled fp16 GEMM operand: the
    values are the exact inputs (16-bit values scale into fp16 without rounding unless they fall
    below the row's range), the layout is [heads | extra]."""
    print(f"heads_to_f16 H={H} L={L} l0={l0} rows={rows} E={E} {dt}", flush=True)
    g = torch.Generator().manual_seed(H + L + E)
    o = torch.randn(H, L, 128, generator=g).to(dt)
    extra = (torch.randn(rows, E, generator=g) * 5).to(dt) if E else None
    x16, rs = _lib.heads_to_f16(o.cuda(), l0, rows, extra.cuda() if extra is not None else None)
    torch.cuda.synchronize()
    ref = o[:, l0:l0 + rows].transpose(0, 1).reshape(rows, H * 128).double()
    if E:
        ref = torch.cat([ref, extra.double()], 1)
    y = x16.cpu().double() * rs.cpu().double()[:, None]
    amax = x16.cpu().double().abs().amax(-1)
    assert torch.all((amax >= 2.0 ** 14) & (amax <= 2.0 ** 15))
    rowmax = ref.abs().amax(-1, keepdim=True)
    assert torch.all((y - ref).abs() <= 2.0 ** -11 * ref.abs() + 2.0 ** -24 * rs.cpu().double()[:, None])
    assert torch.all(rowmax > 0)
