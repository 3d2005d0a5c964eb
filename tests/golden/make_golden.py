"""Writes the small committed fixtures under tests/golden/.

The reference holds no golden vectors for this path (no tests/, captured tensors are
gitignored: develop/.gitignore:1-5). These fixtures are therefore seeded cases computed by the
CPU oracle (oracle/qlinear_oracle.py) -- after the oracle itself was pinned by the closed-form
tests in tests/test_oracle.py -- plus the Hadamard sign vectors from torch's CPU generator,
which is the exact call the reference makes (nodes/ComfyUI-Gfx906Int4/ops.py:79-80).

Usage: python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import qlinear_oracle as orc  # noqa: E402


def rotation_signs():
    out = {}
    for g in (32, 64, 128):
        gen = torch.Generator(device="cpu").manual_seed(0 ^ g)
        out[f"signs_{g}"] = (torch.randint(0, 2, (g,), generator=gen).float() * 2 - 1).numpy()
    np.savez(os.path.join(HERE, "rotation_signs.npz"), **out)


def w4a16_small():
    g = torch.Generator().manual_seed(0)
    M, N, K = 48, 96, 320
    x = torch.randn(M, K, generator=g).to(torch.bfloat16).float().numpy()
    w = (torch.randn(N, K, generator=g) * 0.02).numpy()
    bias = torch.randn(N, generator=g).numpy().astype(np.float32)
    packed, scale = orc.quantize_pack_int4(w, rule="div")
    y = orc.w4a16_reference(x, packed, scale, bias)
    np.savez(os.path.join(HERE, "w4a16_small.npz"), x_bf16_bits=orc.f32_to_bf16_bits(x), w_q4=packed,
             w_scale=scale, bias=bias, y_ref=y, w_float=w)


def w8a8_small():
    g = torch.Generator().manual_seed(1)
    M, N, K = 24, 40, 192
    x = torch.randn(M, K, generator=g).to(torch.bfloat16).float().numpy()
    w = (torch.randn(N, K, generator=g) * 0.02).numpy()
    xq, sx = orc.quantize_int8_rows(x)
    wq, sw = orc.quantize_int8_rows(w)
    acc = orc.int8_matmul_exact(xq, wq)
    y = orc.round_to_dtype(orc.w8a8_epilogue(acc, sx, sw), "bfloat16")
    np.savez(os.path.join(HERE, "w8a8_small.npz"), x_bf16_bits=orc.f32_to_bf16_bits(x), w_float=w, xq=xq, sx=sx,
             wq=wq, sw=sw, acc=acc, y_bf16=y)


if __name__ == "__main__":
    rotation_signs()
    w4a16_small()
    w8a8_small()
    print("fixtures written to", HERE)
