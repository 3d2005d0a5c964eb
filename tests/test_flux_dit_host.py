"""The Flux-style DiT caller (comfy_ui_gfx906_tools_amd/flux_dit.py) on the CPU: its layer set
and parameter names, the per-step work the C5 bench reports, the RoPE and timestep embedding
against their closed forms, and the loud failure of the engine model on CPU tensors."""
import math

import numpy as np
import pytest
import torch

from comfy_ui_gfx906_tools_amd import flux_dit as fd
from comfy_ui_gfx906_tools_amd.ops import Gfx906Int4Ops


def test_flux12b_size_and_work():
    cfg = fd.FluxDiTConfig.flux12b()
    # 19 double blocks (per stream: mod 6h, qkv 3h, proj h, mlp 4h + 4h) and 38 single blocks
    # (mod 3h, linear1 3h + 4h, linear2 from h + 4h); weights only, biases left out
    h = 3072
    per_double = 2 * (h * 6 * h + h * 3 * h + h * h + 2 * h * 4 * h)
    per_single = h * 3 * h + h * 7 * h + 5 * h * h
    assert 19 * per_double + 38 * per_single == pytest.approx(11.83e9, rel=1e-3)
    # the blocks' token-wise linears: 2 * 36864 * h flops per token per block
    assert cfg.linear_flops(4096, 512) == 2 * 36864 * h * 4608 * 57
    assert cfg.linear_flops(4096, 512) / 1e12 == pytest.approx(59.49, abs=0.01)
    assert cfg.attention_flops(4096, 512) / 1e12 == pytest.approx(14.87, abs=0.01)


def test_parameter_names_follow_flux():
    m = fd.FluxDiT(fd.FluxDiTConfig.tiny(), ops=torch.nn, dtype=torch.float32)
    names = {n for n, _ in m.named_parameters()}
    for n in ("img_in.weight", "time_in.in_layer.weight", "vector_in.out_layer.bias", "guidance_in.in_layer.weight",
              "txt_in.weight", "double_blocks.0.img_mod.lin.weight", "double_blocks.1.txt_attn.qkv.weight",
              "double_blocks.0.img_attn.norm.query_norm.scale", "double_blocks.0.img_attn.proj.bias",
              "double_blocks.0.txt_mlp.0.weight", "double_blocks.0.txt_mlp.2.weight",
              "single_blocks.1.linear1.weight", "single_blocks.0.linear2.weight",
              "single_blocks.0.norm.key_norm.scale", "single_blocks.0.modulation.lin.weight",
              "final_layer.linear.weight", "final_layer.adaLN_modulation.1.weight"):
        assert n in names, n


def test_engine_model_state_is_packed():
    cfg = fd.FluxDiTConfig.tiny()
    m = fd.FluxDiT(cfg, device="cpu", dtype=torch.bfloat16)
    sd = m.state_dict()
    assert sd["single_blocks.0.linear1.weight_q4"].shape == (3 * 256 + 1024, 128)
    assert sd["single_blocks.0.linear1.weight_scale"].shape == (3 * 256 + 1024, 8)
    assert sd["single_blocks.0.linear1.weight_q4"].dtype == torch.int8
    assert not any(k.endswith("linear1.weight") for k in sd)


def test_float_model_forward_shape_and_determinism():
    cfg = fd.FluxDiTConfig.tiny()
    m = fd.FluxDiT(cfg, ops=torch.nn, dtype=torch.float32)
    fd.init_random_(m, seed=3)
    inp = fd.synthetic_inputs(cfg, 4, 8, seed=0, device="cpu", dtype=torch.float32)
    with torch.no_grad():
        y1 = m(*inp)
        y2 = m(*inp)
    assert y1.shape == (1, 16, cfg.in_channels)
    assert torch.isfinite(y1).all() and torch.equal(y1, y2)


def test_engine_forward_refuses_cpu_tensors():
    cfg = fd.FluxDiTConfig.tiny()
    m = fd.FluxDiT(cfg, device="cpu", dtype=torch.bfloat16)
    for mod in m.modules():
        if isinstance(mod, Gfx906Int4Ops.Linear) and mod.quantized:
            mod.weight_q4.zero_()
            mod.weight_scale.fill_(1.0)
            mod.bias.data.zero_()
    inp = fd.synthetic_inputs(cfg, 4, 8, seed=0, device="cpu")
    with pytest.raises(RuntimeError):
        m(*inp)


def test_rope_is_a_rotation_by_position_angles():
    axes = (16, 56, 56)
    ids = torch.tensor([[[0.0, 3.0, 5.0], [0.0, 0.0, 0.0]]])
    cos, sin = fd.rope_cos_sin(ids, axes, 10000.0)
    assert cos.shape == (1, 1, 2, 64)
    # position 0 -> identity
    assert torch.equal(cos[0, 0, 1], torch.ones(64)) and torch.equal(sin[0, 0, 1], torch.zeros(64))
    # axis 1 pair j at position 3: angle 3 * 10000^(-2j/56)
    j = 4
    ang = 3.0 * 10000.0 ** (-2 * j / 56)
    assert float(cos[0, 0, 0, 8 + j]) == pytest.approx(math.cos(ang), abs=1e-6)
    assert float(sin[0, 0, 0, 8 + j]) == pytest.approx(math.sin(ang), abs=1e-6)
    # rotation keeps pair norms; a unit x0 goes to (cos, sin)
    x = torch.zeros(1, 1, 2, 128)
    x[..., 0::2] = 1.0
    r = fd.apply_rope(x, cos, sin)
    assert torch.allclose(r[..., 0::2], cos, atol=1e-7) and torch.allclose(r[..., 1::2], sin, atol=1e-7)


def test_timestep_embedding_closed_form():
    t = torch.tensor([0.25])
    e = fd.timestep_embedding(t, 8).numpy()[0]
    f = np.exp(-np.log(10000.0) * np.arange(4) / 4)
    ref = np.concatenate([np.cos(250.0 * f), np.sin(250.0 * f)])
    assert np.allclose(e, ref, atol=1e-4)
