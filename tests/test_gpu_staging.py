"""The row-scaled fp16 staging pass of the tile kernels (rows_to_scaled_f16_kernel, through
qlinear_rows_to_f16) against its defining arithmetic: row_scale = 2^e with e = E - 15, amax =
f * 2^E (f in [0.5, 1)) the row's max |x|, and x16 = fp16(x * 2^-e) rounded to nearest even.
Every step is an IEEE operation that numpy performs the same way, so the comparison is bit-exact.
K covers each register-resident instance (K <= 2048, 4096, 8192, 16384; ragged last chunks) and
the strided two-pass loop above 16384."""
import numpy as np
import pytest
import torch

from comfy_ui_gfx906_tools_amd import _lib

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _staging_reference(x: np.ndarray):
    x = x.astype(np.float32)
    amax = np.abs(x).max(axis=1)
    _, E = np.frexp(amax)
    e = np.where(amax > 0, E - 15, 0).astype(np.int32)
    scale = np.ldexp(np.float32(1.0), e).astype(np.float32)
    x16 = (x * np.ldexp(np.float32(1.0), -e)[:, None].astype(np.float32)).astype(np.float16)
    return x16, scale


@pytest.mark.parametrize("K", [32, 1024, 1056, 2048, 2080, 3072, 3104, 4096, 6144, 8192, 12288, 16384, 16416, 20480])
@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16, torch.float32])
def test_rows_to_f16_bit_exact(K, dt):
    print(f"case staging K={K} dt={dt}", flush=True)
    g = torch.Generator().manual_seed(K)
    M = 6
    x = torch.randn(M, K, generator=g)
    x[1] *= 1e-3   # small row: scaled up
    x[2] *= 300.0  # large row: scaled down
    x[3] = 0.0     # zero row: scale 1
    x[4, K - 1] = 50.0  # the max in the last element (the ragged chunk for K % 2048 != 0)
    x = x.to(dt)
    x16, rs = _lib.rows_to_f16(x.to(DEV))
    torch.cuda.synchronize()
    ref16, refs = _staging_reference(x.float().numpy())
    assert np.array_equal(rs.cpu().numpy(), refs)
    assert np.array_equal(x16.cpu().numpy().view(np.uint16), ref16.view(np.uint16))
    amax16 = np.abs(x16.float().cpu().numpy()).max(axis=1)
    nonzero = np.abs(x.float().numpy()).max(axis=1) > 0
    assert (amax16[nonzero] >= 2.0 ** 14).all() and (amax16 <= 2.0 ** 15).all()
    assert (refs[~nonzero] == 1.0).all()
    if dt != torch.float32:  # 16-bit inputs map exactly
        back = x16.float().cpu().numpy() * rs.cpu().numpy()[:, None]
        assert np.array_equal(back, x.float().numpy())
