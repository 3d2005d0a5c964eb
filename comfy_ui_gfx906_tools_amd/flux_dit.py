"""A Flux-style DiT (double-stream + single-stream blocks) whose every Linear is a
``Gfx906Int4Ops.Linear``: the C5 workload, one denoise step of a 12B model on the W4A16 engine.

The reference patches the Linears of ComfyUI's Flux model (nodes/ComfyUI-Gfx906Int4/nodes.py:71-124,
447-599 build it with ``custom_operations``); ComfyUI is not part of this package, so this module
is the model those operations plug into, with ComfyUI's parameter names (``double_blocks.N.img_attn.qkv``,
``single_blocks.N.linear1``, ...) so a Flux state dict loads through ``make_load_quantizing_ops``.
The architecture is the public Flux one: hidden 3072, 24 heads of 128, 19 double-stream and 38
single-stream blocks, adaLN modulation from the timestep / guidance / pooled-text vector, QK
RMSNorm, 3-axis RoPE (16 + 56 + 56), GELU-tanh MLPs. Attention is PyTorch SDPA (flash or
memory-efficient backends only); every projection runs on libqlinear.so.

``ops`` is any namespace with a ``Linear(in, out, bias=True, device=None, dtype=None)`` class:
``Gfx906Int4Ops`` for the engine, ``torch.nn`` for a float model (the tests' CPU reference, whose
weights are the dequantized codes of the engine model).
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import NamedTuple

import torch
import torch.nn.functional as F

from . import _lib
from .ops import (ROTATE_FUSED_MAX_K, Gfx906Int4Ops, apply_group_rotation, get_group_rotation, get_group_signs,
                  quantize_pack_int4)


@dataclass(frozen=True)
class FluxDiTConfig:
    hidden: int = 3072
    heads: int = 24
    mlp_ratio: int = 4
    depth_double: int = 19
    depth_single: int = 38
    in_channels: int = 64          # 2x2 patches of a 16-channel latent
    context_in: int = 4096         # T5-XXL hidden size
    vec_in: int = 768              # CLIP-L pooled
    time_dim: int = 256
    axes_dim: tuple = (16, 56, 56)
    theta: float = 10000.0
    guidance_embed: bool = True

    @property
    def head_dim(self) -> int:
        return self.hidden // self.heads

    @property
    def mlp_hidden(self) -> int:
        return self.hidden * self.mlp_ratio

    @staticmethod
    def flux12b() -> "FluxDiTConfig":
        return FluxDiTConfig()

    @staticmethod
    def tiny() -> "FluxDiTConfig":
        """Two blocks of each kind at hidden 256 (2 heads of 128): the parity-test model."""
        return FluxDiTConfig(hidden=256, heads=2, depth_double=2, depth_single=2, context_in=128, vec_in=64)

    def linear_flops(self, n_img: int, n_txt: int) -> float:
        """2*M*N*K summed over the token-wise linears of the blocks (modulation and embedders left
        out): each block does 36864 * hidden multiply-adds per token."""
        per_tok = 2.0 * self.hidden * (3 * self.hidden + self.hidden + 2 * self.mlp_hidden)
        return per_tok * (n_img + n_txt) * (self.depth_double + self.depth_single)

    def attention_flops(self, n_img: int, n_txt: int) -> float:
        L = n_img + n_txt
        return 4.0 * L * L * self.hidden * (self.depth_double + self.depth_single)


# ---------------------------------------------------------------------------------------------
# building blocks
# ---------------------------------------------------------------------------------------------
def _is_engine_linear(layer) -> bool:
    return isinstance(layer, Gfx906Int4Ops.Linear) and layer.quantized


def _fusable(layer) -> bool:
    """Engine layer without activation rotation: it can take the fused adaLN operand."""
    return _is_engine_linear(layer) and not layer.rotation_group


class Staged(NamedTuple):
    """A GEMM operand already in the W4A16 kernel's fp16 form: x16 [rows, K] fp16 with per-row
    power-of-two factors row_scale [rows]; `lead` are the leading dims of the logical tensor and
    `dtype` its activation dtype (the GEMM's output dtype)."""
    x16: torch.Tensor
    row_scale: torch.Tensor
    lead: tuple
    dtype: torch.dtype


def _scales_kn(layer, ws: torch.Tensor, rows: slice | None):
    """The group-major copy of ws (or of its rows `rows`), computed once and kept: on ws for the
    whole weight, on the layer per row slice (a column slice of the whole copy would not be
    contiguous). Recomputed after an in-place change of ws or on another stream; None off the GPU
    or for tensors without a version counter."""
    if not ws.is_cuda:
        return None
    if rows is None:
        return _lib.cached_scales_kn(ws)
    try:
        key = (rows.start, rows.stop, ws._version, torch.cuda.current_stream(ws.device).cuda_stream)
    except RuntimeError:
        return None
    cache = layer.__dict__.setdefault("_qlinear_scales_kn_rows", {})
    hit = cache.get(key[:2])
    if hit is not None and hit[0] == key:
        return hit[1]
    kn = _lib.w4a16_scales_kn(ws[rows])
    cache[key[:2]] = (key, kn)
    return kn


def _linear(layer, x, gelu: bool = False, rows: slice | None = None, staged_out: bool = False,
            residual: tuple | None = None):
    """layer(x), optionally followed by GELU-tanh, optionally restricted to output rows `rows`
    of the weight. Engine layers fuse the GELU into the GEMM epilogue, take row slices of
    weight_q4 / weight_scale / bias as views (rows of the packed layout are contiguous) and
    accept a Staged operand. staged_out: return the bf16 result as the next GEMM's Staged operand
    (row-scaled fp16 written by this GEMM's epilogue, no staging pass) where the engine can: an
    engine layer without rotation or row slice, a Staged bf16 input; otherwise a plain tensor.
    residual = (r, gate, inplace): return r + gate * layer(x) for r [B, L, N] and gate [B, 1, N]
    (into r itself when inplace), fused into the GEMM epilogue on engine layers."""
    if _is_engine_linear(layer):
        wq, ws, b = layer.weight_q4, layer.weight_scale, layer.bias
        # the fp16 dequant's per-column factors, kept with the whole weight (rows slice them), and
        # the group-major scale copy of the rows used
        cs = _lib.cached_col_scales(ws) if ws.is_cuda else None
        kn = _scales_kn(layer, ws, rows)
        if rows is not None:
            wq, ws = wq[rows], ws[rows]
            b = b[rows] if b is not None else None
            cs = cs[rows] if cs is not None else None
        N = wq.shape[0]
        rk, lead = {}, None
        if residual is not None:  # the gated residual in the epilogue: y = r + gate * linear
            r, gate, inplace = residual
            lead = r.shape[:-1]
            r2 = r.reshape(-1, N)
            rk = dict(residual=r2, gate=gate.reshape(-1, N), out=r2 if inplace else None)
        if isinstance(x, Staged):
            if layer.rotation_group:
                raise RuntimeError("a layer with activation rotation takes a plain activation tensor")
            bias = b.to(x.dtype) if b is not None else None
            if staged_out and rows is None and x.dtype == torch.bfloat16 and residual is None:
                y16, rs = _lib.w4a16_gemm(x.x16, wq, ws, bias, out_dtype=x.dtype, row_scale=x.row_scale, gelu=gelu,
                                          col_scale=cs, scales_kn=kn, f16_rowscaled=True,
                                          out_bound=_lib.cached_out_bound(wq, ws, bias))
                return Staged(y16, rs, x.lead, x.dtype)
            y = _lib.w4a16_gemm(x.x16, wq, ws, bias, out_dtype=x.dtype, row_scale=x.row_scale, gelu=gelu,
                                col_scale=cs, scales_kn=kn, **rk)
            return y.reshape(*(lead if lead is not None else x.lead), N)
        shape = x.shape
        x2 = x.reshape(-1, shape[-1])
        bias = b.to(x.dtype) if b is not None else None
        if layer.rotation_group:  # the weight was folded through the rotation (as int4_linear does)
            g = layer.rotation_group
            if shape[-1] <= ROTATE_FUSED_MAX_K:
                x16, rs = _lib.rotate_rows_to_f16(x2, get_group_signs(g, x2.device), g)
                y = _lib.w4a16_gemm(x16, wq, ws, bias, out_dtype=x.dtype, row_scale=rs, gelu=gelu, col_scale=cs,
                                    scales_kn=kn, **rk)
                return y.reshape(*shape[:-1], N)
            x2 = apply_group_rotation(x2.float(), get_group_rotation(shape[-1], g, x2.device), g)
        y = _lib.w4a16_gemm(x2, wq, ws, bias, out_dtype=x.dtype, gelu=gelu, col_scale=cs, scales_kn=kn, **rk)
        return y.reshape(*shape[:-1], N)
    w, b = layer.weight, layer.bias
    if rows is not None:
        w = w[rows]
        b = b[rows] if b is not None else None
    y = F.linear(x, w.to(x.dtype), b.to(x.dtype) if b is not None else None)
    y = F.gelu(y, approximate="tanh") if gelu else y
    if residual is not None:
        r, gate, inplace = residual
        return r.add_(gate * y) if inplace else r + gate * y
    return y


def timestep_embedding(t: torch.Tensor, dim: int, max_period: float = 10000.0, time_factor: float = 1000.0):
    """Sinusoidal embedding [B, dim] of t in [0, 1] (cos half first), in fp32."""
    t = time_factor * t.float()
    half = dim // 2
    freqs = torch.exp(-math.log(max_period) * torch.arange(half, dtype=torch.float32, device=t.device) / half)
    args = t[:, None] * freqs[None]
    return torch.cat([torch.cos(args), torch.sin(args)], dim=-1)


def rope_cos_sin(ids: torch.Tensor, axes_dim, theta: float):
    """ids [B, L, n_axes] positions -> (cos, sin) [B, 1, L, head_dim/2] in fp32: axis i rotates
    axes_dim[i]/2 pairs with frequencies theta^(-2j/axes_dim[i])."""
    parts = []
    for i, d in enumerate(axes_dim):
        omega = 1.0 / theta ** (torch.arange(0, d, 2, dtype=torch.float64, device=ids.device) / d)
        parts.append(ids[..., i].double()[..., None] * omega)
    ang = torch.cat(parts, dim=-1).float()[:, None]
    return torch.cos(ang), torch.sin(ang)


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Rotate consecutive pairs (x0, x1) of the head dim by the position angle, in fp32."""
    xf = x.float().unflatten(-1, (-1, 2))
    x0, x1 = xf[..., 0], xf[..., 1]
    out = torch.stack([cos * x0 - sin * x1, sin * x0 + cos * x1], dim=-1)
    return out.flatten(-2).to(x.dtype)


def attention(q, k, v, cos, sin) -> torch.Tensor:
    """RoPE on q, k, then SDPA; [B, H, L, D] -> [B, L, H*D]. On the GPU only the flash and
    memory-efficient kernels are allowed (no silent fallback to the unfused math path)."""
    q, k = apply_rope(q, cos, sin), apply_rope(k, cos, sin)
    if q.is_cuda:
        from torch.nn.attention import SDPBackend, sdpa_kernel
        with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
            o = F.scaled_dot_product_attention(q.contiguous(), k.contiguous(), v.contiguous())
    else:
        o = F.scaled_dot_product_attention(q, k, v)
    return o.transpose(1, 2).flatten(2)


class RMSNorm(torch.nn.Module):
    def __init__(self, dim, device=None, dtype=None):
        super().__init__()
        self.scale = torch.nn.Parameter(torch.ones(dim, device=device, dtype=dtype))

    def forward(self, x):
        xf = x.float()
        y = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6)
        return (y * self.scale.float()).to(x.dtype)


class QKNorm(torch.nn.Module):
    def __init__(self, dim, device=None, dtype=None):
        super().__init__()
        self.query_norm = RMSNorm(dim, device, dtype)
        self.key_norm = RMSNorm(dim, device, dtype)

    def forward(self, q, k):
        return self.query_norm(q), self.key_norm(k)


def _layer_norm(x: torch.Tensor) -> torch.Tensor:
    return F.layer_norm(x, (x.shape[-1],), eps=1e-6)


def _modulate(x, shift, scale):
    return _layer_norm(x) * (1 + scale) + shift


# ---- the engine path's fused glue (csrc/dit_fused.hip); batch items one call each -----------
def _adaln(x: torch.Tensor, shift: torch.Tensor, scale: torch.Tensor) -> Staged:
    """_modulate(x, shift, scale) for x [B, L, K], shift / scale [B, 1, K], as the fp16 GEMM operand."""
    B, L, K = x.shape
    parts = [_lib.adaln_modulate_f16(x[b], shift[b].reshape(-1), scale[b].reshape(-1)) for b in range(B)]
    if B == 1:
        x16, rs = parts[0]
    else:
        x16, rs = torch.cat([p[0] for p in parts]), torch.cat([p[1] for p in parts])
    return Staged(x16, rs, (B, L), x.dtype)


def _heads_into(attn: "SelfAttention", qkv: torch.Tensor, cos, sin, q, k, v, l_offset: int) -> None:
    """QK-norm + RoPE of qkv [B, Lx, 3 H D] into rows [l_offset, l_offset + Lx) of q, k, v [B, H, L, D]."""
    for b in range(qkv.shape[0]):
        _lib.qk_norm_rope(qkv[b], attn.norm.query_norm.scale, attn.norm.key_norm.scale, cos[b, 0], sin[b, 0],
                          attn.heads, out=(q[b], k[b], v[b]), l_offset=l_offset)


def _sdpa_heads(q, k, v) -> torch.Tensor:
    """SDPA on [B, H, L, D] (flash / memory-efficient kernels only), output kept head-major."""
    from torch.nn.attention import SDPBackend, sdpa_kernel
    with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
        return F.scaled_dot_product_attention(q, k, v).contiguous()


def _heads_staged(o: torch.Tensor, l_offset: int, rows: int, extra: torch.Tensor | None = None) -> Staged:
    """Rows [l_offset, l_offset + rows) of o [B, H, L, D] flattened over heads (followed by
    extra [B, rows, E]) as the next GEMM's fp16 operand: the head transpose, the concatenation
    and the staging pass in one kernel per batch item."""
    B = o.shape[0]
    parts = [_lib.heads_to_f16(o[b], l_offset, rows, extra[b] if extra is not None else None) for b in range(B)]
    if B == 1:
        x16, rs = parts[0]
    else:
        x16, rs = torch.cat([p[0] for p in parts]), torch.cat([p[1] for p in parts])
    return Staged(x16, rs, (B, rows), o.dtype)


class MLPEmbedder(torch.nn.Module):
    def __init__(self, in_dim, hidden, ops, device=None, dtype=None):
        super().__init__()
        self.in_layer = ops.Linear(in_dim, hidden, bias=True, device=device, dtype=dtype)
        self.out_layer = ops.Linear(hidden, hidden, bias=True, device=device, dtype=dtype)

    def forward(self, x):
        return _linear(self.out_layer, F.silu(_linear(self.in_layer, x)))


class Modulation(torch.nn.Module):
    """lin(silu(vec)) split into 3 (single) or 6 (double) chunks of (shift, scale, gate)."""

    def __init__(self, dim, double, ops, device=None, dtype=None):
        super().__init__()
        self.multiplier = 6 if double else 3
        self.lin = ops.Linear(dim, self.multiplier * dim, bias=True, device=device, dtype=dtype)

    def forward(self, vec):
        out = _linear(self.lin, F.silu(vec))[:, None, :].chunk(self.multiplier, dim=-1)
        return out


class SelfAttention(torch.nn.Module):
    def __init__(self, dim, heads, ops, device=None, dtype=None):
        super().__init__()
        self.heads = heads
        self.qkv = ops.Linear(dim, 3 * dim, bias=True, device=device, dtype=dtype)
        self.norm = QKNorm(dim // heads, device, dtype)
        self.proj = ops.Linear(dim, dim, bias=True, device=device, dtype=dtype)


def _split_heads(qkv: torch.Tensor, heads: int):
    """[B, L, 3*H*D] -> q, k, v each [B, H, L, D]."""
    B, L, _ = qkv.shape
    t = qkv.view(B, L, 3, heads, -1).permute(2, 0, 3, 1, 4)
    return t[0], t[1], t[2]


class DoubleStreamBlock(torch.nn.Module):
    def __init__(self, cfg: FluxDiTConfig, ops, device=None, dtype=None):
        super().__init__()
        h, m = cfg.hidden, cfg.mlp_hidden
        self.heads = cfg.heads
        for s in ("img", "txt"):
            setattr(self, f"{s}_mod", Modulation(h, True, ops, device, dtype))
            setattr(self, f"{s}_attn", SelfAttention(h, cfg.heads, ops, device, dtype))
            setattr(self, f"{s}_mlp", torch.nn.Sequential(ops.Linear(h, m, bias=True, device=device, dtype=dtype),
                                                          torch.nn.GELU(approximate="tanh"),
                                                          ops.Linear(m, h, bias=True, device=device, dtype=dtype)))

    def forward(self, img, txt, vec, cos, sin):
        if img.is_cuda and all(_fusable(m) for m in self.modules() if isinstance(m, Gfx906Int4Ops.Linear)):
            return self._forward_engine(img, txt, vec, cos, sin)
        i_sh1, i_sc1, i_g1, i_sh2, i_sc2, i_g2 = self.img_mod(vec)
        t_sh1, t_sc1, t_g1, t_sh2, t_sc2, t_g2 = self.txt_mod(vec)
        qs, ks, vs = [], [], []
        for x, attn, sh, sc in ((txt, self.txt_attn, t_sh1, t_sc1), (img, self.img_attn, i_sh1, i_sc1)):
            q, k, v = _split_heads(_linear(attn.qkv, _modulate(x, sh, sc)), self.heads)
            q, k = attn.norm(q, k)
            qs.append(q), ks.append(k), vs.append(v)
        o = attention(torch.cat(qs, 2), torch.cat(ks, 2), torch.cat(vs, 2), cos, sin)
        n_txt = txt.shape[1]
        txt_o, img_o = o[:, :n_txt], o[:, n_txt:]
        img = img + i_g1 * _linear(self.img_attn.proj, img_o)
        img = img + i_g2 * _linear(self.img_mlp[2], _linear(self.img_mlp[0], _modulate(img, i_sh2, i_sc2), gelu=True))
        txt = txt + t_g1 * _linear(self.txt_attn.proj, txt_o)
        txt = txt + t_g2 * _linear(self.txt_mlp[2], _linear(self.txt_mlp[0], _modulate(txt, t_sh2, t_sc2), gelu=True))
        return img, txt

    def _forward_engine(self, img, txt, vec, cos, sin):
        """forward() with the fused kernels: adaLN straight into the GEMM operand, QK-norm + RoPE
        written into the joint [txt | img] q / k / v, gated residuals in one pass each."""
        i_sh1, i_sc1, i_g1, i_sh2, i_sc2, i_g2 = self.img_mod(vec)
        t_sh1, t_sc1, t_g1, t_sh2, t_sc2, t_g2 = self.txt_mod(vec)
        B, n_img, _ = img.shape
        n_txt = txt.shape[1]
        D = self.img_attn.qkv.in_features // self.heads
        q, k, v = (torch.empty(B, self.heads, n_txt + n_img, D, dtype=img.dtype, device=img.device) for _ in range(3))
        _heads_into(self.txt_attn, _linear(self.txt_attn.qkv, _adaln(txt, t_sh1, t_sc1)), cos, sin, q, k, v, 0)
        _heads_into(self.img_attn, _linear(self.img_attn.qkv, _adaln(img, i_sh1, i_sc1)), cos, sin, q, k, v, n_txt)
        o = _sdpa_heads(q, k, v)
        # gated residuals in the proj / fc2 epilogues; the block's inputs stay untouched
        img = _linear(self.img_attn.proj, _heads_staged(o, n_txt, n_img), residual=(img, i_g1, False))
        # fc1 writes its GELU output straight as fc2's fp16 operand (no staging pass between them)
        h = _linear(self.img_mlp[0], _adaln(img, i_sh2, i_sc2), gelu=True, staged_out=True)
        img = _linear(self.img_mlp[2], h, residual=(img, i_g2, True))
        txt = _linear(self.txt_attn.proj, _heads_staged(o, 0, n_txt), residual=(txt, t_g1, False))
        h = _linear(self.txt_mlp[0], _adaln(txt, t_sh2, t_sc2), gelu=True, staged_out=True)
        txt = _linear(self.txt_mlp[2], h, residual=(txt, t_g2, True))
        return img, txt


class SingleStreamBlock(torch.nn.Module):
    def __init__(self, cfg: FluxDiTConfig, ops, device=None, dtype=None):
        super().__init__()
        h, m = cfg.hidden, cfg.mlp_hidden
        self.heads, self.hidden = cfg.heads, h
        self.linear1 = ops.Linear(h, 3 * h + m, bias=True, device=device, dtype=dtype)
        self.linear2 = ops.Linear(h + m, h, bias=True, device=device, dtype=dtype)
        self.norm = QKNorm(cfg.head_dim, device, dtype)
        self.modulation = Modulation(h, False, ops, device, dtype)

    def forward(self, x, vec, cos, sin):
        if x.is_cuda and all(_fusable(m) for m in self.modules() if isinstance(m, Gfx906Int4Ops.Linear)):
            return self._forward_engine(x, vec, cos, sin)
        shift, scale, gate = self.modulation(vec)
        xm = _modulate(x, shift, scale)
        h3 = 3 * self.hidden
        # linear1 = [qkv | mlp]: two GEMMs on row slices of the packed weight, GELU fused into the second
        qkv = _linear(self.linear1, xm, rows=slice(0, h3))
        mlp = _linear(self.linear1, xm, gelu=True, rows=slice(h3, None))
        q, k, v = _split_heads(qkv, self.heads)
        q, k = self.norm(q, k)
        o = attention(q, k, v, cos, sin)
        return x + gate * _linear(self.linear2, torch.cat([o, mlp], dim=-1))

    def _forward_engine(self, x, vec, cos, sin):
        shift, scale, gate = self.modulation(vec)
        st = _adaln(x, shift, scale)
        h3 = 3 * self.hidden
        B, L, _ = x.shape
        D = self.hidden // self.heads
        q, k, v = (torch.empty(B, self.heads, L, D, dtype=x.dtype, device=x.device) for _ in range(3))
        for b in range(B):
            _lib.qk_norm_rope(_linear(self.linear1, Staged(st.x16[b * L:(b + 1) * L], st.row_scale[b * L:(b + 1) * L],
                                                           (L,), x.dtype), rows=slice(0, h3)),
                              self.norm.query_norm.scale, self.norm.key_norm.scale, cos[b, 0], sin[b, 0], self.heads,
                              out=(q[b], k[b], v[b]))
        mlp = _linear(self.linear1, st, gelu=True, rows=slice(h3, None))
        # linear2's input [attention | gelu(mlp)] gathered straight into its fp16 operand, the gated
        # residual in its epilogue
        return _linear(self.linear2, _heads_staged(_sdpa_heads(q, k, v), 0, L, mlp), residual=(x, gate, False))


class LastLayer(torch.nn.Module):
    def __init__(self, hidden, out_channels, ops, device=None, dtype=None):
        super().__init__()
        self.linear = ops.Linear(hidden, out_channels, bias=True, device=device, dtype=dtype)
        self.adaLN_modulation = torch.nn.Sequential(torch.nn.SiLU(),
                                                    ops.Linear(hidden, 2 * hidden, bias=True, device=device,
                                                               dtype=dtype))

    def forward(self, x, vec):
        shift, scale = _linear(self.adaLN_modulation[1], F.silu(vec)).chunk(2, dim=-1)
        if _fusable(self.linear) and x.is_cuda:
            return _linear(self.linear, _adaln(x.contiguous(), shift[:, None], scale[:, None]))
        return _linear(self.linear, _modulate(x, shift[:, None], scale[:, None]))


class FluxDiT(torch.nn.Module):
    def __init__(self, cfg: FluxDiTConfig, ops=Gfx906Int4Ops, device=None, dtype=torch.bfloat16):
        super().__init__()
        if sum(cfg.axes_dim) != cfg.head_dim:
            raise ValueError(f"axes_dim {cfg.axes_dim} must sum to head_dim {cfg.head_dim}")
        self.cfg = cfg
        h = cfg.hidden
        self.img_in = ops.Linear(cfg.in_channels, h, bias=True, device=device, dtype=dtype)
        self.time_in = MLPEmbedder(cfg.time_dim, h, ops, device, dtype)
        self.vector_in = MLPEmbedder(cfg.vec_in, h, ops, device, dtype)
        self.guidance_in = MLPEmbedder(cfg.time_dim, h, ops, device, dtype) if cfg.guidance_embed else None
        self.txt_in = ops.Linear(cfg.context_in, h, bias=True, device=device, dtype=dtype)
        self.double_blocks = torch.nn.ModuleList(DoubleStreamBlock(cfg, ops, device, dtype)
                                                 for _ in range(cfg.depth_double))
        self.single_blocks = torch.nn.ModuleList(SingleStreamBlock(cfg, ops, device, dtype)
                                                 for _ in range(cfg.depth_single))
        self.final_layer = LastLayer(h, cfg.in_channels, ops, device, dtype)

    def forward(self, img, img_ids, txt, txt_ids, timesteps, y, guidance=None):
        """img [B, L_img, in_channels], img_ids [B, L_img, 3], txt [B, L_txt, context_in],
        txt_ids [B, L_txt, 3], timesteps [B] in [0, 1], y [B, vec_in], guidance [B] -> the
        velocity prediction [B, L_img, in_channels]."""
        dt = img.dtype
        img = _linear(self.img_in, img)
        vec = _linear(self.time_in.in_layer, timestep_embedding(timesteps, self.cfg.time_dim).to(dt))
        vec = _linear(self.time_in.out_layer, F.silu(vec))
        if self.guidance_in is not None:
            vec = vec + self.guidance_in(timestep_embedding(guidance, self.cfg.time_dim).to(dt))
        vec = vec + self.vector_in(y)
        txt = _linear(self.txt_in, txt)
        cos, sin = rope_cos_sin(torch.cat([txt_ids, img_ids], dim=1), self.cfg.axes_dim, self.cfg.theta)
        for blk in self.double_blocks:
            img, txt = blk(img, txt, vec, cos, sin)
        x = torch.cat([txt, img], dim=1)
        for blk in self.single_blocks:
            x = blk(x, vec, cos, sin)
        return self.final_layer(x[:, txt.shape[1]:], vec)


# ---------------------------------------------------------------------------------------------
# synthetic weights and inputs
# ---------------------------------------------------------------------------------------------
@torch.no_grad()
def init_random_(model: FluxDiT, seed: int, w_std: float = 0.02) -> None:
    """Random-init in place on the model's device: every Linear weight ~ N(0, w_std) in fp32,
    quantized to int4 group-32 by quantize_pack_int4 (the HIP quantizer for device weights),
    one layer at a time so no full-precision copy of the model exists; biases ~ N(0, w_std);
    RMSNorm scales stay 1."""
    gens = {}
    for name, mod in model.named_modules():
        if not hasattr(mod, "in_features") or not hasattr(mod, "out_features"):
            continue
        dev = mod.bias.device if mod.bias is not None else next(mod.buffers()).device
        g = gens.get(dev)
        if g is None:
            g = gens[dev] = torch.Generator(device=dev).manual_seed(seed)
        w = torch.randn(mod.out_features, mod.in_features, generator=g, device=dev) * w_std
        if _is_engine_linear(mod):
            q, s = quantize_pack_int4(w)
            mod.weight_q4.copy_(q)
            mod.weight_scale.copy_(s)
        else:
            mod.weight.copy_(w)
        del w
        if mod.bias is not None:
            mod.bias.copy_(torch.randn(mod.out_features, generator=g, device=dev) * w_std)


def synthetic_inputs(cfg: FluxDiTConfig, n_img_side: int, n_txt: int, seed: int, device, dtype=torch.bfloat16,
                     batch: int = 1):
    """Inputs of one denoise step: an n_img_side x n_img_side grid of latent patches (4096 tokens
    for a 1024x1024 image), n_txt text tokens, t = 0.5, guidance 3.5; activations ~ N(0, 1)."""
    g = torch.Generator().manual_seed(seed)
    L = n_img_side * n_img_side
    img = torch.randn(batch, L, cfg.in_channels, generator=g).to(dtype)
    txt = torch.randn(batch, n_txt, cfg.context_in, generator=g).to(dtype)
    y = torch.randn(batch, cfg.vec_in, generator=g).to(dtype)
    rr, cc = torch.meshgrid(torch.arange(n_img_side), torch.arange(n_img_side), indexing="ij")
    img_ids = torch.stack([torch.zeros_like(rr), rr, cc], dim=-1).reshape(1, L, 3).expand(batch, L, 3).float()
    txt_ids = torch.zeros(batch, n_txt, 3)
    t = torch.full((batch,), 0.5)
    gd = torch.full((batch,), 3.5)
    return tuple(v.to(device) for v in (img, img_ids, txt, txt_ids, t, y, gd))
