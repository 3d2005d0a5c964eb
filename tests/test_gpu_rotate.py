"""The fused activation rotation + fp16 staging kernel (csrc/rotate.hip) through the C ABI against
a float64 restatement of the reference's rotation (x_g R^T, R = H diag(signs) / sqrt(g), signs from
the committed fixture of torch's generator; oracle/qlinear_oracle.py group_rotation), and the
rotated W4A16 linear (ops.int4_linear with rotation_group) against the fp32 dequant reference of
the rotated problem."""
import numpy as np
import pytest
import torch

from comfy_ui_gfx906_tools_amd import _lib, ops
from oracle import qlinear_oracle as orc
from tests.conftest import golden_path
from tests.gpu_util import rel_max_err

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _rotate64(x: np.ndarray, g: int) -> np.ndarray:
    signs = np.load(golden_path("rotation_signs.npz"))[f"signs_{g}"].astype(np.float64)
    # exact H diag(signs) / sqrt(g): the +-1 pattern of the oracle's Sylvester matrix, scaled in float64
    R = np.sign(orc.hadamard(g)).astype(np.float64) * signs[None, :] / np.sqrt(g)
    return (x.astype(np.float64).reshape(-1, g) @ R.T).reshape(x.shape)


def test_signs_match_the_fixture():
    for g in (32, 64, 128):
        s = ops.get_group_signs(g, DEV).cpu().numpy()
        assert np.array_equal(s, np.load(golden_path("rotation_signs.npz"))[f"signs_{g}"].astype(np.float32))


@pytest.mark.parametrize("M,K,g", [(1, 128, 128), (5, 3072, 128), (33, 96, 32), (17, 4160, 64), (3, 16384, 128),
                                   (64, 12288, 128)])
@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16, torch.float32])
def test_rotate_rows_to_f16(M, K, g, dt):
    print(f"rotate M={M} K={K} g={g} {dt}", flush=True)
    x = (torch.randn(M, K, generator=torch.Generator().manual_seed(M + K + g)) * 3).to(dt)
    if M > 2:
        x[1, : K // 2] *= 1e3  # an outlier half-row
    x16, rs = _lib.rotate_rows_to_f16(x.to(DEV), ops.get_group_signs(g, DEV), g)
    torch.cuda.synchronize()
    y = x16.cpu().double() * rs.cpu().double()[:, None]
    ref = _rotate64(x.float().numpy(), g)
    amax = x16.cpu().double().abs().amax(-1)
    assert torch.all((amax >= 2.0 ** 14) & (amax <= 2.0 ** 15))
    rowmax = np.abs(ref).max(-1, keepdims=True)
    # one fp16 rounding of each value, plus fp32 butterflies (log2(g) additions) relative to the row
    bound = 2.0 ** -11 * np.abs(ref) + 2.0 ** -24 * rs.cpu().double().numpy()[:, None] + 4e-6 * rowmax
    assert np.all(np.abs(y.numpy() - ref) <= bound), float((np.abs(y.numpy() - ref) - bound).max())


@pytest.mark.parametrize("M,N,K", [(1, 256, 3072), (8, 320, 1024), (300, 520, 3072), (4608, 1024, 3072)])
def test_rotated_int4_linear(M, N, K):
    """y = int4_linear(x, W_rot) with W_rot the int4 quantization of the rotated weight: equal to
    rotate(x) @ dequant(W_rot)^T within the 2e-3 gate (fp32 output)."""
    print(f"rotated linear M={M} N={N} K={K}", flush=True)
    g = ops.choose_rotation_group(K)
    gen = torch.Generator().manual_seed(M + N)
    x = torch.randn(M, K, generator=gen).to(torch.bfloat16)
    w = torch.randn(N, K, generator=gen) * 0.02
    wr = _rotate64(w.numpy(), g).astype(np.float32)
    wp, ws = orc.quantize_pack_int4(wr, rule="div")
    y = ops.int4_linear(x.to(DEV).float(), torch.from_numpy(wp).to(DEV), torch.from_numpy(ws).to(DEV),
                        rotation_group=g)
    ref = _rotate64(x.float().numpy(), g) @ orc.dequant_int4(wp, ws).astype(np.float64).T
    assert rel_max_err(y.cpu().numpy(), ref) <= 2e-3
    # bf16 activations: the same within one bf16 rounding of the output
    yb = ops.int4_linear(x.to(DEV), torch.from_numpy(wp).to(DEV), torch.from_numpy(ws).to(DEV), rotation_group=g)
    assert yb.dtype == torch.bfloat16 and rel_max_err(yb.float().cpu().numpy(), ref) <= 2e-3 + 2.0 ** -8
