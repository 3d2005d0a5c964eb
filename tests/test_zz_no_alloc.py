"""qlinear_w4a16_gemm_noalloc (the allocation-free W4A16 entry point) against qlinear_w4a16_gemm.

Both run the same plan and kernels; only the workspace differs (the library's static scratch vs
a buffer from torch's allocator), so results must be bit-identical. Two calls in a row, the
second with a smaller input, catch stale scratch contents; a call that needs more scratch than
the static array holds must fail before launching anything.
"""
import numpy as np
import pytest
import torch

from oracle import qlinear_oracle as orc
from tests.gpu_util import rel_max_err, to_np_f32

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _lib():
    from comfy_ui_gfx906_tools_amd import _lib
    return _lib


def _layer(M, N, K, seed, xdt=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g).to(xdt)
    w = torch.randn(N, K, generator=g) * 0.02
    packed, scale = orc.quantize_pack_int4(w.numpy())
    bias = (torch.randn(N, generator=g) * 0.1)
    return x, packed, scale, bias


# (M, N, K, x dtype, splits, config, out dtype, gelu): the first of each pair is the larger call.
# bf16 x goes through the fp16 staging pass (scratch: row scales + staged x + column factors);
# splits > 1 adds split-K partial tiles; config 5 is the 256 x 256 kernel; M <= 16 the direct
# kernels (no scratch at all).
PAIRS = [
    ((300, 640, 1536, torch.bfloat16, 3, None, torch.float32, False),
     (40, 256, 512, torch.bfloat16, 3, None, torch.float32, False)),
    ((513, 777, 640, torch.float16, 0, 5, torch.bfloat16, True),
     (257, 300, 1024, torch.float16, 0, 5, torch.bfloat16, True)),
    ((200, 1000, 4096, torch.float32, 0, None, torch.bfloat16, False),
     (17, 512, 1024, torch.bfloat16, 0, None, torch.float16, False)),
    ((16, 512, 1024, torch.bfloat16, 0, None, torch.bfloat16, False),
     (1, 256, 256, torch.bfloat16, 0, None, torch.bfloat16, False)),
]


@pytest.mark.parametrize("pair", PAIRS, ids=[f"pair{i}" for i in range(len(PAIRS))])
def test_noalloc_matches_workspace_entry_point(pair):
    L = _lib()
    for i, (M, N, K, xdt, splits, cfg, odt, gelu) in enumerate(pair):
        print(f"case noalloc call {i}: M={M} N={N} K={K} x={xdt} splits={splits} cfg={cfg} out={odt}", flush=True)
        x, packed, scale, bias = _layer(M, N, K, seed=M + N + K + i, xdt=xdt)
        args = (x.to(DEV), torch.from_numpy(packed).to(DEV), torch.from_numpy(scale).to(DEV), bias.to(odt).to(DEV))
        kw = dict(out_dtype=odt, splits=splits, config=cfg, gelu=gelu)
        y_ws = L.w4a16_gemm(*args, **kw)
        y_na = L.w4a16_gemm(*args, noalloc=True, **kw)
        torch.cuda.synchronize()
        assert torch.equal(y_ws, y_na), f"call {i}: noalloc differs from the workspace entry point"
        if odt == torch.float32 and not gelu:
            ref = orc.w4a16_reference(to_np_f32(x), packed, scale, to_np_f32(bias.to(odt)))
            assert rel_max_err(to_np_f32(y_na), ref) <= 2e-3


def test_noalloc_rejects_calls_beyond_the_scratch():
    """bf16 x of 4608 x 12288 needs a 113 MB staged copy: more than the 32 MiB scratch."""
    L = _lib()
    M, N, K = 4608, 256, 12288
    assert L.load_library().qlinear_w4a16_workspace_bytes(2, M, N, K, 0, 0, 0) > L.W4A16_NOALLOC_SCRATCH_BYTES
    x = torch.zeros(M, K, dtype=torch.bfloat16, device=DEV)
    wq = torch.zeros(N, K // 2, dtype=torch.int8, device=DEV)
    ws = torch.ones(N, K // 32, dtype=torch.float32, device=DEV)
    with pytest.raises(RuntimeError, match="static scratch"):
        L.w4a16_gemm(x, wq, ws, out_dtype=torch.bfloat16, noalloc=True)
    # the same call with the fp16 operand staged by the caller and no K split needs only the
    # column factors
    x16, rs = L.rows_to_f16(x)
    y = L.w4a16_gemm(x16, wq, ws, out_dtype=torch.bfloat16, row_scale=rs, splits=1, noalloc=True)
    torch.cuda.synchronize()
    assert not torch.isnan(y).any() and float(y.float().abs().max()) == 0.0
