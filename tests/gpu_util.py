"""Helpers shared by the GPU parity tests (seeded inputs, torch <-> numpy, error metrics)."""
from __future__ import annotations

import numpy as np
import torch

from oracle import qlinear_oracle as orc


def seeded_linear(M: int, N: int, K: int, seed: int, x_dtype=torch.bfloat16, w_std: float = 0.02,
                  rule: str = "div"):
    """x ~ N(0,1) [M, K] in x_dtype; W ~ N(0, w_std) [N, K] quantized by the reference rule (numpy
    oracle, ops.py:108-126). Returns torch CPU tensors (x, w_q4, w_scale) plus numpy copies."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g).to(x_dtype)
    w = torch.randn(N, K, generator=g) * w_std
    packed, scale = orc.quantize_pack_int4(w.numpy(), rule=rule)
    return x, torch.from_numpy(packed), torch.from_numpy(scale)


def to_np_f32(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def rel_max_err(y: np.ndarray, ref: np.ndarray) -> float:
    """The reference's error metric: max|y - ref| / max|ref| (bench_int8.py:44, bench_linear.py:81)."""
    denom = float(np.abs(ref).max())
    return float(np.abs(y.astype(np.float64) - ref.astype(np.float64)).max() / (denom if denom else 1.0))


def bf16_ulp(a: np.ndarray) -> np.ndarray:
    """Spacing of bf16 numbers at |a| (a already bf16-representable)."""
    a = np.abs(np.asarray(a, np.float32))
    e = np.floor(np.log2(np.maximum(a, np.float32(2.0 ** -126))))
    return (2.0 ** (e - 7)).astype(np.float32)


def f16_ulp(a: np.ndarray) -> np.ndarray:
    a = np.abs(np.asarray(a, np.float32))
    e = np.floor(np.log2(np.maximum(a, np.float32(2.0 ** -14))))
    return (2.0 ** (e - 10)).astype(np.float32)


def dequant_torch(w_q4: torch.Tensor, w_scale: torch.Tensor) -> torch.Tensor:
    """fp32 dequant of the packed layout on w_q4's device (decode as int4_train_test.py:46-52)."""
    b = w_q4.view(torch.uint8).to(torch.int16)
    lo = b & 0xF
    hi = b >> 4
    codes = torch.stack([lo, hi], dim=-1).reshape(w_q4.shape[0], -1)
    codes = torch.where(codes > 7, codes - 16, codes).float()
    return codes * w_scale.float().repeat_interleave(32, dim=1)
