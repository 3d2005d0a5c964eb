"""The reference extension's Python surface for the int4 path (nodes/ComfyUI-Gfx906Int4/csrc/
binding.cpp:52-112, 359-372: the module `_get_ext()` returns in ops.py:14-34), on libqlinear.so.

    quantize_int4(x) -> (packed int8 [M, K/2], scale fp32 [M, K/32])
    gemm_int4(A_packed, A_scale, B_packed, B_scale, bias, out_dtype, splits=0, qblock=32)
    gemm_int4_auto_splits(M, N, K)

Same argument meaning, shapes and error behaviour (RuntimeError naming expected vs actual), so
the reference's own `int4_linear` -- ext.quantize_int4 then ext.gemm_int4 (ops.py:181-182), its
W4A4 production path -- runs unchanged on MI355X with bit-identical results: the activation
quantizer follows the reference kernel's rule (scale = amax * (1/7), rint), the GEMM its
per-block fmaf order, and split-K (splits > 1, or splits = 0 resolved by the reference's
auto_splits rule for this GPU's CU count) its per-split fp32 partials summed in split order.
Also provided: the block-32 int8 pair quantize_int8 / gemm_int8 (csrc/binding.cpp:173-217,
bit-identical to its kernel for every tile config) and the engine's own entry points
w4a16_linear, quantize_int8_per_token and w8a8_linear. The reference's conv_int8 and attention
functions (VAE, attention nodes) are outside this package.
"""
from __future__ import annotations

import torch

from . import _lib

MAX_SPLITS = 8  # binding.cpp: splits in [0, MAX_SPLITS]


def quantize_int4(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """x [M, K] float32/16/bf16 on the GPU, K % 32 == 0 -> (packed int8 [M, K/2], scale fp32 [M, K/32])."""
    if not (isinstance(x, torch.Tensor) and x.is_cuda):
        raise RuntimeError("x must be on device")
    if x.dim() != 2 or x.shape[1] % 32 != 0:
        raise RuntimeError(f"x must be [M, K] with K % 32 == 0, got {list(x.shape)}")
    return _lib.quantize_int4(x, rule=_lib.RULE_RECIP)


def gemm_int4(A_packed: torch.Tensor, A_scale: torch.Tensor, B_packed: torch.Tensor, B_scale: torch.Tensor,
              bias: torch.Tensor | None, out_dtype: torch.dtype, splits: int = 0, qblock: int = 32) -> torch.Tensor:
    """[M, N] in out_dtype = block-scaled int4 A [M, K/2] x B [N, K/2]^T (+ bias in out_dtype)."""
    if not (A_packed.is_cuda and B_packed.is_cuda):
        raise RuntimeError("inputs must be on device")
    if not 0 <= int(splits) <= MAX_SPLITS:
        raise RuntimeError(f"splits must be in [0, {MAX_SPLITS}], got {splits}")
    return _lib.w4a4_gemm(A_packed, A_scale, B_packed, B_scale, bias, out_dtype=out_dtype, qblock=int(qblock),
                          splits=int(splits))


def gemm_int4_auto_splits(M: int, N: int, K: int) -> int:
    """Split-K count gemm_int4 picks for [M, K] x [N, K]^T (the reference's rule, binding.cpp:36-43,
    with the current GPU's CU count)."""
    return _lib.w4a4_auto_splits(int(M), int(N), int(K))


def quantize_int8(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """x [M, K] float32/16/bf16 on the GPU, K % 32 == 0 -> (int8 [M, K], scale fp32 [M, K/32])."""
    if not (isinstance(x, torch.Tensor) and x.is_cuda):
        raise RuntimeError("x must be on device")
    if x.dim() != 2 or x.shape[1] % 32 != 0:
        raise RuntimeError(f"x must be [M, K] with K % 32 == 0, got {list(x.shape)}")
    return _lib.quantize_int8_block32(x)


def gemm_int8(A: torch.Tensor, A_scale: torch.Tensor, B: torch.Tensor, B_scale: torch.Tensor,
              bias: torch.Tensor | None, out_dtype: torch.dtype, config: int = 0) -> torch.Tensor:
    """[M, N] in out_dtype = block-32 int8 A [M, K] x B [N, K]^T (+ bias in out_dtype)."""
    if not (A.is_cuda and B.is_cuda):
        raise RuntimeError("inputs must be on device")
    if not 0 <= int(config) <= 3:
        raise RuntimeError(f"config must be in [0, 3], got {config}")
    return _lib.gemm_int8_block32(A, A_scale, B, B_scale, bias, out_dtype=out_dtype)


def w4a16_linear(x: torch.Tensor, w_q4: torch.Tensor, w_scale: torch.Tensor, bias: torch.Tensor | None = None,
                 out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """x [M, K] @ dequant(w_q4, w_scale)^T (+ bias) on the W4A16 engine."""
    return _lib.w4a16_gemm(x, w_q4, w_scale, bias, out_dtype=out_dtype)


def quantize_int8_per_token(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """x [M, K] -> (int8 [M, K], fp32 [M]): the int8 rule with one block per row."""
    return _lib.quantize_int8_per_token(x)


def w8a8_linear(xq: torch.Tensor, s_x: torch.Tensor, wq: torch.Tensor, s_w: torch.Tensor,
                bias: torch.Tensor | None = None, out_dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """float(xq @ wq^T in int32) * (s_x[m] * s_w[n]) (+ bias) in out_dtype."""
    return _lib.w8a8_gemm(xq, s_x, wq, s_w, bias, out_dtype=out_dtype)
