"""Quantized Linear for ComfyUI on MI355X (gfx950): the reference's Gfx906Int4Ops API
(nodes/ComfyUI-Gfx906Int4/ops.py) with a W4A16 engine underneath.

Kept as in the reference, so packed checkpoints and workflows are a drop-in:
  * weight format: buffers ``weight_q4`` int8 [N, K/2] (two's-complement nibbles, byte j =
    code[2j] | code[2j+1] << 4) and ``weight_scale`` fp32 [N, K/32] (ops.py:108-126, 214-215);
  * ``quantize_pack_int4`` / ``repack_q4_0_native`` / rotation helpers with the same
    signatures and results (ops.py:43-164);
  * ``int4_linear(x, w_packed, w_scale, bias=None, rotation_group=0)`` as a module-level name
    (instrumented by monkeypatching in the reference's harness, bench_model.py:119-121);
  * ``Gfx906Int4Ops.Linear`` / ``make_load_quantizing_ops`` (ops.py:199-276), including the
    K % 32 float fallback, lowvram per-call device moves and quantize-on-load.
Changed: ``int4_linear`` computes x @ dequant(W)^T with bf16/fp16 activations (W4A16) on the
gfx950 kernels of libqlinear.so instead of quantizing x to int4 (the reference's W4A4,
ops.py:181-182). There is no CPU fallback for the forward: CPU tensors raise.
"""
from __future__ import annotations

import torch

from . import _lib

BLOCK = 32  # ops.py:196
ROTATION_SEED = 0  # ops.py:39: weight-fold time and forward time must agree
ROTATE_FUSED_MAX_K = 16384  # the fused rotation + staging kernel keeps a row in registers

# Which scale rule torch's own `amax / 7.0` follows on each device (see _lib.RULE_*): the HIP
# quantizer reproduces torch's result on the device the weight lives on.
_TORCH_RULE = {"cpu": _lib.RULE_DIV, "cuda": _lib.RULE_RECIP}

_HADAMARD_CACHE: dict = {}
_ROTATION_CACHE: dict = {}


def _get_ext():
    """The extension module of the int4 path (quantize_int4 / gemm_int4 / gemm_int4_auto_splits,
    comfy_ui_gfx906_tools_amd.ext) with libqlinear.so loaded; raises if the library was not built.
    Mirrors ops.py:14-34, which JIT-built a pybind11 extension instead."""
    _lib.load_library()
    from . import ext
    return ext


# ---------------------------------------------------------------------------------------------
# Hadamard group rotation (ops.py:43-105)
# ---------------------------------------------------------------------------------------------
def _hadamard(n: int, device, dtype=torch.float32) -> torch.Tensor:
    """Orthonormal Sylvester-Hadamard matrix of order n (power of two)."""
    key = (n, torch.device(device), dtype)
    h = _HADAMARD_CACHE.get(key)
    if h is None:
        if n <= 0 or n & (n - 1):
            raise ValueError(f"Hadamard order {n} must be a power of two")
        base = torch.tensor([[1.0, 1.0], [1.0, -1.0]], dtype=torch.float64)
        h = torch.ones(1, 1, dtype=torch.float64)
        while h.shape[0] < n:
            h = torch.kron(base, h)
        h = (h / n ** 0.5).to(device=device, dtype=dtype)
        _HADAMARD_CACHE[key] = h
    return h


def choose_rotation_group(in_features: int, max_group: int = 128, min_group: int = 32) -> int | None:
    """Largest power of two <= max_group (and >= min_group) dividing in_features, else None."""
    g = max_group
    while g >= min_group:
        if in_features % g == 0:
            return g
        g //= 2
    return None


def get_group_rotation(in_features: int, group: int, device) -> torch.Tensor:
    """R = H * diag(signs) for one `group`-sized block; signs from torch's CPU generator seeded
    with ROTATION_SEED ^ group, so the weight fold and the activation rotation agree."""
    key = (in_features, group, torch.device(device))
    r = _ROTATION_CACHE.get(key)
    if r is None:
        gen = torch.Generator(device="cpu").manual_seed(ROTATION_SEED ^ group)
        signs = torch.randint(0, 2, (group,), generator=gen).float() * 2 - 1
        r = _hadamard(group, device) * signs.to(device)
        _ROTATION_CACHE[key] = r
    return r


def get_group_signs(group: int, device) -> torch.Tensor:
    """The +-1 column signs of get_group_rotation (fp32 [group]): R = H * signs, and the first
    row of the Sylvester H is all ones, so they are R's first row times sqrt(group)."""
    key = ("signs", group, torch.device(device))
    s = _ROTATION_CACHE.get(key)
    if s is None:
        s = torch.sign(get_group_rotation(group, group, device)[0]).contiguous()
        _ROTATION_CACHE[key] = s
    return s


def apply_group_rotation(t: torch.Tensor, R: torch.Tensor, group: int) -> torch.Tensor:
    """Rotate every `group`-sized chunk of the last dim: chunk v -> v @ R^T. One 2-D matmul over
    rows*groups; CPU-resident tensors are rotated on the GPU when one is present (ops.py:85-105)."""
    shape = t.shape
    flat = t.reshape(-1, group)
    if flat.device.type == "cpu" and torch.cuda.is_available():
        out = (flat.cuda() @ R.t().to("cuda")).to("cpu")
    else:
        out = flat @ R.t().to(flat.device)
    return out.reshape(shape)


# ---------------------------------------------------------------------------------------------
# Weight format
# ---------------------------------------------------------------------------------------------
def quantize_pack_int4(t: torch.Tensor, block: int = BLOCK, rule: int | None = None):
    """t [..., K] float -> (packed int8 [..., K/2], scale fp32 [..., K/block]) (ops.py:108-126).
    Device tensors are quantized by the HIP kernel with the scale rule torch itself uses on that
    device, so results equal the reference's torch expression on the same device; CPU tensors use
    that torch expression directly (load-time code, not the forward path). `rule` (_lib.RULE_DIV /
    RULE_RECIP) overrides the device's rule: a weight the reference would quantize on the CPU can
    then be quantized on the GPU with the CPU's result."""
    K = t.shape[-1]
    if K % block != 0:
        raise AssertionError(f"last dim {K} not divisible by block {block}")
    rule = _TORCH_RULE["cuda" if t.device.type == "cuda" else "cpu"] if rule is None else rule
    if t.device.type == "cuda" and block == BLOCK and t.dtype in (torch.float32, torch.float16, torch.bfloat16):
        return _lib.quantize_int4(t, rule)
    shape = t.shape
    tb = t.reshape(-1, K // block, block).float()
    amax = tb.abs().amax(dim=-1, keepdim=True).clamp_min(1e-8)
    scale = amax / 7.0 if rule == _lib.RULE_DIV else amax * torch.tensor(1.0 / 7.0, dtype=torch.float32)
    codes = torch.round(tb / scale).clamp(-8, 7).to(torch.int32).reshape(-1, K)
    packed = ((codes[:, 0::2] & 0xF) | ((codes[:, 1::2] & 0xF) << 4)).to(torch.uint8).view(torch.int8)
    return (packed.reshape(*shape[:-1], K // 2).contiguous(),
            scale.reshape(*shape[:-1], K // block).contiguous())


def repack_q4_0_native(raw_bytes: torch.Tensor, out_features: int, in_features: int, block: int = BLOCK):
    """Lossless ggml Q4_0 (18-byte blocks: fp16 d, 16 bytes of offset-binary nibbles in
    split-half order) -> native two's-complement interleaved int4 + fp32 scales (ops.py:129-164).
    Device tensors go through the HIP repack kernel; CPU tensors through the torch expression."""
    if raw_bytes.device.type == "cuda" and block == BLOCK:
        return _lib.repack_q4_0(raw_bytes, out_features, in_features)
    n_blocks = out_features * (in_features // block)
    blocks = raw_bytes.reshape(-1).view(torch.uint8).reshape(n_blocks, 18)
    scale = blocks[:, :2].contiguous().view(torch.float16).reshape(n_blocks).float()
    qs = blocks[:, 2:].to(torch.int32)
    elems = torch.cat([((qs & 0xF) - 8) & 0xF, (((qs >> 4) & 0xF) - 8) & 0xF], dim=1)  # order 0..31
    packed = (elems[:, 0::2] | (elems[:, 1::2] << 4)).to(torch.uint8).view(torch.int8)
    return (packed.reshape(out_features, in_features // 2).contiguous(),
            scale.reshape(out_features, in_features // block).contiguous())


# ---------------------------------------------------------------------------------------------
# Forward
# ---------------------------------------------------------------------------------------------
def int4_linear(x: torch.Tensor, w_packed: torch.Tensor, w_scale: torch.Tensor, bias: torch.Tensor | None = None,
                rotation_group: int = 0) -> torch.Tensor:
    """x [..., K] -> [..., N] in x.dtype: x @ dequant(w_packed, w_scale)^T (+ bias) on the gfx950
    W4A16 kernel. w_packed/w_scale come from quantize_pack_int4 of the weight, folded through the
    same rotation when rotation_group != 0; bias, if given, is already x.dtype (ops.py:167-183).
    bf16 and fp32 activations (the rotated path is fp32) are staged as exactly row-scaled fp16,
    so the weights dequantize to fp16 (11-bit mantissa) rather than bf16."""
    shape = x.shape
    K = shape[-1]
    x2d = x.reshape(-1, K)
    # the fp16 dequant's per-column factors, computed once per weight and kept with it, and the
    # group-major copy of the scales that the tile kernels (more than 16 rows) read
    cs = _lib.cached_col_scales(w_scale) if w_scale.is_cuda else None
    kn = _lib.cached_scales_kn(w_scale) if w_scale.is_cuda and x2d.shape[0] > 16 else None
    if rotation_group and x2d.is_cuda and K <= ROTATE_FUSED_MAX_K:
        # rotation and fp16 staging in one pass, then the GEMM on the staged operand
        x16, rs = _lib.rotate_rows_to_f16(x2d, get_group_signs(rotation_group, x2d.device), rotation_group)
        out = _lib.w4a16_gemm(x16, w_packed, w_scale, bias, out_dtype=x.dtype, row_scale=rs, col_scale=cs,
                              scales_kn=kn)
        return out.reshape(*shape[:-1], w_packed.shape[0])
    if rotation_group:
        R = get_group_rotation(K, rotation_group, x2d.device)
        x2d = apply_group_rotation(x2d.float(), R, rotation_group)
    out = _lib.w4a16_gemm(x2d, w_packed, w_scale, bias, out_dtype=x.dtype, col_scale=cs, scales_kn=kn)
    return out.reshape(*shape[:-1], w_packed.shape[0])


def int4_linear_w4a4(x: torch.Tensor, w_packed: torch.Tensor, w_scale: torch.Tensor, bias: torch.Tensor | None = None,
                     rotation_group: int = 0) -> torch.Tensor:
    """The reference's own int4_linear (ops.py:167-183): x is quantized to block-32 int4 as well
    (W4A4) and multiplied by the block-scaled int4 GEMM; bit-identical to the reference's unsplit
    run on the same inputs. int4_linear (W4A16) is the engine's default path."""
    ext = _get_ext()
    shape = x.shape
    K = shape[-1]
    x2d = x.reshape(-1, K)
    if rotation_group:
        R = get_group_rotation(K, rotation_group, x2d.device)
        x2d = apply_group_rotation(x2d.float(), R, rotation_group)
    qa, sa = ext.quantize_int4(x2d.contiguous())
    out = ext.gemm_int4(qa, sa, w_packed, w_scale, bias, x.dtype)
    return out.reshape(*shape[:-1], w_packed.shape[0])


# ---------------------------------------------------------------------------------------------
# custom_operations integration (ops.py:186-276)
# ---------------------------------------------------------------------------------------------
try:  # inside ComfyUI the ops class extends comfy's, so every other layer type is unchanged
    import comfy.ops as _comfy_ops  # type: ignore

    _OpsBase = _comfy_ops.disable_weight_init
except ImportError:  # standalone use (tests, benchmarks): only Linear is provided
    class _OpsBase:  # noqa: D401 - a namespace like comfy.ops.disable_weight_init
        pass


class Gfx906Int4Ops(_OpsBase):
    class Linear(torch.nn.Module):
        # Device plain float weights are quantized on while loading; set by make_load_quantizing_ops.
        quantize_device = None
        quantized_on_load = 0

        def __init__(self, in_features, out_features, bias=True, device=None, dtype=None, rotation_group=0):
            super().__init__()
            self.in_features = in_features
            self.out_features = out_features
            self.rotation_group = rotation_group
            # layers too narrow for a 32-wide group stay plain float Linears (ops.py:206-212)
            self.quantized = in_features % BLOCK == 0 and in_features >= BLOCK
            if self.quantized:
                self.register_buffer("weight_q4", torch.empty(out_features, in_features // 2, dtype=torch.int8,
                                                              device=device))
                self.register_buffer("weight_scale", torch.empty(out_features, in_features // BLOCK,
                                                                 dtype=torch.float32, device=device))
            else:
                self.weight = torch.nn.Parameter(torch.empty(out_features, in_features, device=device, dtype=dtype))
            if bias:
                self.bias = torch.nn.Parameter(torch.empty(out_features, device=device, dtype=dtype))
            else:
                self.register_parameter("bias", None)

        def _load_from_state_dict(self, state_dict, prefix, local_metadata, strict, missing_keys, unexpected_keys,
                                  error_msgs):
            key = prefix + "weight"
            if self.quantized and self.quantize_device is not None and key in state_dict:
                # a plain float checkpoint weight, quantized here one layer at a time
                w = state_dict.pop(key)
                if w.dtype not in (torch.float32, torch.float16, torch.bfloat16) or \
                        tuple(w.shape) != (self.out_features, self.in_features):
                    raise RuntimeError(f"{key}: expected a float [{self.out_features}, {self.in_features}] weight, "
                                       f"got {w.dtype} {tuple(w.shape)}")
                w_float = w.to(self.quantize_device).float()
                if self.rotation_group:
                    R = get_group_rotation(self.in_features, self.rotation_group, w_float.device)
                    w_float = apply_group_rotation(w_float, R, self.rotation_group)
                packed, scale = quantize_pack_int4(w_float, BLOCK)
                state_dict[prefix + "weight_q4"] = packed.to(w.device)
                state_dict[prefix + "weight_scale"] = scale.to(w.device)
                type(self).quantized_on_load += 1
            super()._load_from_state_dict(state_dict, prefix, local_metadata, strict, missing_keys, unexpected_keys,
                                          error_msgs)

        def forward(self, x):
            if not self.quantized:
                bias = self.bias.to(x.device, x.dtype) if self.bias is not None else None
                return torch.nn.functional.linear(x, self.weight.to(x.device, x.dtype), bias)
            # lowvram: weights may be CPU-resident and moved per call (ops.py:252-259)
            weight_q4 = self.weight_q4.to(x.device)
            weight_scale = self.weight_scale.to(x.device)
            bias = self.bias.to(x.device, x.dtype) if self.bias is not None else None
            return int4_linear(x, weight_q4, weight_scale, bias, self.rotation_group)


def make_load_quantizing_ops(base_ops, quantize_device, rotate):
    """custom_operations that quantize plain float Linear weights while the state dict loads, on
    quantize_device; every other layer comes from base_ops (ops.py:263-276)."""
    class Linear(Gfx906Int4Ops.Linear):
        quantized_on_load = 0

        def __init__(self, in_features, out_features, bias=True, device=None, dtype=None):
            group = (choose_rotation_group(in_features) or 0) if rotate else 0
            super().__init__(in_features, out_features, bias, device, dtype, rotation_group=group)

    Linear.quantize_device = torch.device(quantize_device)
    return type("Gfx906Int4LoadOps", (base_ops,), {"Linear": Linear})
