"""Host-side logic of the ops mirror (comfy_ui_gfx906_tools_amd/ops.py) on the CPU: the weight
format helpers against the oracle, the rotation against the committed sign fixture, the Linear
module's state handling (float fallback, quantize-on-load, load errors) and the loud failure of
the forward on CPU tensors (there is no CPU fallback)."""
import numpy as np
import pytest
import torch

from comfy_ui_gfx906_tools_amd import _lib, ops
from oracle import qlinear_oracle as orc
from tests.conftest import golden_path


def test_quantize_pack_int4_cpu_matches_oracle():
    g = torch.Generator().manual_seed(0)
    w = torch.randn(64, 256, generator=g) * 0.02
    w[3, :32] = 0.0  # zero block
    w[5, 32:64] *= 1e4
    packed, scale = ops.quantize_pack_int4(w)
    p_ref, s_ref = orc.quantize_pack_int4(w.numpy(), rule="div")
    assert packed.dtype == torch.int8 and scale.dtype == torch.float32
    assert np.array_equal(packed.numpy(), p_ref) and np.array_equal(scale.numpy(), s_ref)
    # leading dims are kept
    p3, s3 = ops.quantize_pack_int4(w.reshape(4, 16, 256))
    assert p3.shape == (4, 16, 128) and s3.shape == (4, 16, 8)
    with pytest.raises(AssertionError):
        ops.quantize_pack_int4(torch.zeros(2, 48))


def test_quantize_pack_int4_16bit_inputs():
    w = (torch.randn(8, 64, generator=torch.Generator().manual_seed(1)) * 0.1).to(torch.bfloat16)
    packed, scale = ops.quantize_pack_int4(w)
    p_ref, s_ref = orc.quantize_pack_int4(w.float().numpy(), rule="div")
    assert np.array_equal(packed.numpy(), p_ref) and np.array_equal(scale.numpy(), s_ref)


def test_repack_q4_0_native_matches_oracle():
    rng = np.random.default_rng(2)
    out_f, in_f = 5, 96
    n = out_f * in_f // 32
    d = (rng.standard_normal(n) * 0.01).astype(np.float16)
    raw = np.concatenate([d.view(np.uint8).reshape(n, 2), rng.integers(0, 256, (n, 16)).astype(np.uint8)], axis=1)
    packed, scale = ops.repack_q4_0_native(torch.from_numpy(raw.reshape(-1)), out_f, in_f)
    p_ref, s_ref = orc.repack_q4_0_native(raw, out_f, in_f)
    assert np.array_equal(packed.numpy(), p_ref) and np.array_equal(scale.numpy(), s_ref)
    assert np.array_equal(orc.dequant_int4(packed.numpy(), scale.numpy()), orc.ggml_q4_0_dequant(raw, out_f, in_f))


def test_rotation_matches_fixture_and_oracle():
    f = np.load(golden_path("rotation_signs.npz"))
    for g in (32, 64, 128):
        R = ops.get_group_rotation(4 * g, g, "cpu")
        assert np.allclose(R.numpy(), orc.group_rotation(f[f"signs_{g}"]), atol=0, rtol=0)
    t = torch.randn(3, 384, generator=torch.Generator().manual_seed(3))
    R = ops.get_group_rotation(384, 128, "cpu")
    got = ops.apply_group_rotation(t, R, 128).numpy()
    assert np.allclose(got, orc.apply_group_rotation(t.numpy(), R.numpy()), atol=1e-5)
    assert ops.choose_rotation_group(3072) == 128 and ops.choose_rotation_group(48) is None
    with pytest.raises(ValueError):
        ops._hadamard(48, "cpu")


def test_linear_float_fallback_for_narrow_k():
    lin = ops.Gfx906Int4Ops.Linear(40, 8, bias=True)
    assert not lin.quantized and not hasattr(lin, "weight_q4")
    torch.nn.init.normal_(lin.weight)
    torch.nn.init.normal_(lin.bias)
    x = torch.randn(3, 40)
    assert torch.equal(lin(x), torch.nn.functional.linear(x, lin.weight, lin.bias))


def test_linear_buffers_and_state_dict_roundtrip():
    lin = ops.Gfx906Int4Ops.Linear(64, 16, bias=False)
    assert lin.quantized and lin.bias is None
    assert lin.weight_q4.shape == (16, 32) and lin.weight_q4.dtype == torch.int8
    assert lin.weight_scale.shape == (16, 2) and lin.weight_scale.dtype == torch.float32
    p, s = orc.quantize_pack_int4(np.random.default_rng(4).standard_normal((16, 64)).astype(np.float32))
    lin.load_state_dict({"weight_q4": torch.from_numpy(p), "weight_scale": torch.from_numpy(s)})
    assert np.array_equal(lin.weight_q4.numpy(), p)
    assert set(lin.state_dict()) == {"weight_q4", "weight_scale"}


def test_quantize_on_load_and_rotation_fold():
    base = type("Base", (), {})
    Ops = ops.make_load_quantizing_ops(base, "cpu", rotate=True)
    lin = Ops.Linear(256, 8, bias=True)
    assert lin.rotation_group == 128 and issubclass(Ops, base)
    w = torch.randn(8, 256, generator=torch.Generator().manual_seed(5)) * 0.02
    b = torch.randn(8)
    lin.load_state_dict({"weight": w.clone(), "bias": b})
    R = ops.get_group_rotation(256, 128, "cpu")
    w_rot = ops.apply_group_rotation(w, R, 128)
    assert np.allclose(w_rot.numpy(), orc.apply_group_rotation(w.numpy(), R.numpy()), atol=1e-6)
    p_ref, s_ref = orc.quantize_pack_int4(w_rot.numpy(), rule="div")
    assert np.array_equal(lin.weight_q4.numpy(), p_ref) and np.array_equal(lin.weight_scale.numpy(), s_ref)
    assert Ops.Linear.quantized_on_load == 1
    # no rotation when rotate=False
    Plain = ops.make_load_quantizing_ops(base, "cpu", rotate=False)
    lin2 = Plain.Linear(256, 8, bias=False)
    lin2.load_state_dict({"weight": w.clone()})
    p2, s2 = orc.quantize_pack_int4(w.numpy(), rule="div")
    assert lin2.rotation_group == 0 and np.array_equal(lin2.weight_q4.numpy(), p2)


def test_quantize_on_load_rejects_bad_weight():
    Ops = ops.make_load_quantizing_ops(type("Base", (), {}), "cpu", rotate=False)
    lin = Ops.Linear(64, 8, bias=False)
    with pytest.raises(RuntimeError, match=r"expected a float \[8, 64\] weight"):
        lin.load_state_dict({"weight": torch.zeros(8, 32)})
    with pytest.raises(RuntimeError, match="torch.int32"):
        lin.load_state_dict({"weight": torch.zeros(8, 64, dtype=torch.int32)})


def test_forward_on_cpu_fails_loudly():
    lin = ops.Gfx906Int4Ops.Linear(64, 16, bias=False)
    p, s = orc.quantize_pack_int4(np.ones((16, 64), np.float32))
    lin.load_state_dict({"weight_q4": torch.from_numpy(p), "weight_scale": torch.from_numpy(s)})
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        lin(torch.randn(2, 64))
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        _lib.w8a8_gemm(torch.zeros(2, 64, dtype=torch.int8), None, torch.zeros(2, 64, dtype=torch.int8), None,
                       out_dtype=torch.int32)


def test_missing_library_is_an_error(tmp_path, monkeypatch):
    monkeypatch.setattr(_lib, "_lib", None)
    with pytest.raises(RuntimeError, match="missing"):
        _lib.load_library(str(tmp_path / "libqlinear.so"))
