"""The ComfyUI node surface (comfy_ui_gfx906_tools_amd/nodes.py) on the CPU, without ComfyUI:
node names and widgets, the int4 weight emulation of the test patch against the oracle, the
patch / transcode nodes on stand-in MODEL / CLIP objects, the state-dict quantizer of the UNet
loader (plain, pass-through and ConvRot layers) and its agreement with the transcode."""
import json

import numpy as np
import pytest
import torch

from comfy_ui_gfx906_tools_amd import NODE_CLASS_MAPPINGS, NODE_DISPLAY_NAME_MAPPINGS, flux_dit as fd, nodes
from comfy_ui_gfx906_tools_amd.ops import Gfx906Int4Ops
from oracle import qlinear_oracle as orc
from tests.conftest import golden_path


class _Model:
    """What the nodes touch of a ComfyUI ModelPatcher / CLIP: clone() and the wrapped module."""

    def __init__(self, root, attr="diffusion_model"):
        self.model = type("Inner", (), {})()
        setattr(self.model, attr, root)
        self.cond_stage_model = root

    def clone(self):
        return self  # ModelPatcher.clone shares the module; the nodes patch it in place


def test_node_mappings_match_the_reference_names():
    assert set(NODE_CLASS_MAPPINGS) == {"Gfx906Int4Patch", "Gfx906Int4UnetLoader", "Gfx906Int4Transcode",
                                        "Gfx906Int4TranscodeCLIP", "Gfx906Int4CLIPLoader"}
    assert NODE_DISPLAY_NAME_MAPPINGS["Gfx906Int4Transcode"] == "Gfx906 Int4 Transcode (native kernel, any source)"
    for cls in NODE_CLASS_MAPPINGS.values():
        assert cls.CATEGORY == "gfx906" and hasattr(cls, cls.FUNCTION)
    req = nodes.Gfx906Int4Patch.INPUT_TYPES()["required"]
    assert req["mode"][0] == ["w4a16", "w4a4_naive"] and req["block_size"][1]["default"] == 32
    assert nodes.Gfx906Int4Transcode.INPUT_TYPES()["required"]["activation_rotation"][1]["default"] is False
    assert nodes.Gfx906Int4TranscodeCLIP.RETURN_TYPES == ("CLIP",)
    assert nodes.Gfx906Int4UnetLoader.RETURN_TYPES == ("MODEL",)


def test_quantize_dequantize_matches_oracle():
    g = torch.Generator().manual_seed(0)
    w = torch.randn(24, 96, generator=g) * 0.05
    w[1, :32] = 0.0
    got = nodes.quantize_dequantize_int4(w)
    assert np.array_equal(got.numpy(), orc.quantize_dequantize_int4(w.numpy(), rule="div"))
    assert torch.equal(nodes.quantize_dequantize_int4(torch.ones(3, 40)), torch.ones(3, 40))  # K % 32 != 0
    wb = w.to(torch.bfloat16)
    assert nodes.quantize_dequantize_int4(wb).dtype == torch.bfloat16


def _block(k, n):
    b = torch.nn.Module()
    b.proj = torch.nn.Linear(k, n)
    return b


def test_find_max_layer_index():
    root = torch.nn.Module()
    root.layers = torch.nn.ModuleList(_block(4, 4) for _ in range(6))
    assert nodes.find_max_layer_index(root) == 5
    flat = torch.nn.Module()
    flat.layers = torch.nn.ModuleList(torch.nn.Linear(4, 4) for _ in range(3))  # "layers.N" has no child
    assert nodes.find_max_layer_index(flat) == -1
    assert nodes.find_max_layer_index(torch.nn.Linear(2, 2)) == -1


def _layered_model():
    torch.manual_seed(1)
    root = torch.nn.Module()
    root.layers = torch.nn.ModuleList(_block(64, 32) for _ in range(3))
    root.final_layer = torch.nn.Linear(64, 16)
    root.odd = torch.nn.Linear(40, 8)  # K % 32 != 0: untouched
    return root


@pytest.mark.parametrize("mode", ["w4a16", "w4a4_naive"])
def test_patch_node(mode):
    root = _layered_model()
    before = {n: p.detach().clone() for n, p in root.named_parameters()}
    (out,) = nodes.Gfx906Int4Patch().patch(_Model(root), mode, True, 32)
    m = out.model.diffusion_model
    for spared in ("layers.0.proj.weight", "layers.2.proj.weight", "final_layer.weight", "odd.weight"):
        assert torch.equal(dict(m.named_parameters())[spared], before[spared]), spared
    w1 = dict(m.named_parameters())["layers.1.proj.weight"]
    assert np.array_equal(w1.detach().numpy(), orc.quantize_dequantize_int4(before["layers.1.proj.weight"].numpy()))
    x = torch.randn(5, 64)
    y = m.layers[1].proj(x)
    xin = nodes.quantize_dequantize_int4(x) if mode == "w4a4_naive" else x
    assert torch.allclose(y, torch.nn.functional.linear(xin, w1, m.layers[1].proj.bias), atol=1e-6)
    # spare_first_last_layers=False rounds every eligible weight
    root2 = _layered_model()
    nodes.Gfx906Int4Patch().patch(_Model(root2), "w4a16", False, 32)
    assert np.array_equal(root2.layers[0].proj.weight.detach().numpy(),
                          orc.quantize_dequantize_int4(before["layers.0.proj.weight"].numpy()))


def _float_dit(dtype=torch.float32, device="cpu"):
    cfg = fd.FluxDiTConfig.tiny()
    m = fd.FluxDiT(cfg, ops=torch.nn, dtype=dtype, device=device)
    fd.init_random_(m, seed=11)
    return m


def test_transcode_node_swaps_every_linear():
    m = _float_dit()
    m.extra = torch.nn.Linear(48, 8)  # K % 32 != 0: skipped
    ref = {n: (mod.weight.detach().clone(), mod.bias.detach().clone()) for n, mod in m.named_modules()
           if isinstance(mod, torch.nn.Linear)}
    (out,) = nodes.Gfx906Int4Transcode().transcode(_Model(m), False)
    assert out.model.diffusion_model is m
    swapped = {n: mod for n, mod in m.named_modules() if isinstance(mod, Gfx906Int4Ops.Linear)}
    assert set(swapped) == set(ref) - {"extra"} and isinstance(m.extra, torch.nn.Linear)
    for n, mod in swapped.items():
        p, s = orc.quantize_pack_int4(ref[n][0].numpy(), rule="div")
        assert np.array_equal(mod.weight_q4.numpy(), p) and np.array_equal(mod.weight_scale.numpy(), s), n
        assert torch.equal(mod.bias, ref[n][1]) and mod.rotation_group == 0


def test_transcode_with_rotation_folds_the_weights():
    """activation_rotation=True: group = largest power of two <= 128 dividing K; the packed weight
    is the int4 quantization of W rotated per group (W R^T, R = H diag(signs), signs from the
    committed fixture of torch's generator)."""
    torch.manual_seed(3)
    root = torch.nn.Module()
    root.lin = torch.nn.Linear(192, 16)
    w = root.lin.weight.detach().numpy().copy()
    c, s, src = nodes.transcode_linears(root, rotate=True)
    assert (c, s) == (1, 0) and src == {"plain_rotated": 1}
    assert root.lin.rotation_group == 64  # 192 = 3 * 64
    R = orc.group_rotation(np.load(golden_path("rotation_signs.npz"))["signs_64"])
    wr = orc.apply_group_rotation(w, R)
    _, s_ref = orc.quantize_pack_int4(wr, rule="div")
    assert np.allclose(root.lin.weight_scale.numpy(), s_ref, rtol=1e-6, atol=0)
    deq = orc.dequant_int4(root.lin.weight_q4.numpy(), root.lin.weight_scale.numpy())
    assert np.all(np.abs(deq - wr) <= np.repeat(s_ref, 32, axis=1) * (0.5 + 1e-4))


def test_clip_transcode_node():
    enc = torch.nn.Sequential(torch.nn.Linear(64, 64), torch.nn.GELU(), torch.nn.Linear(64, 32))
    (clip,) = nodes.Gfx906Int4TranscodeCLIP().transcode(_Model(enc), False)
    assert all(isinstance(clip.cond_stage_model[i], Gfx906Int4Ops.Linear) for i in (0, 2))


def test_parse_convrot_layers():
    meta = {"_quantization_metadata": json.dumps({"layers": {
        "model.diffusion_model.a.weight": {"format": "convrot_w4a4", "convrot_groupsize": 64, "quant_group_size": 32},
        "model.diffusion_model.b.weight": {"format": "fp8"}}})}
    assert nodes.parse_convrot_layers(meta, "model.diffusion_model.") == {
        "a.weight": {"format": "convrot_w4a4", "convrot_groupsize": 64, "quant_group_size": 32}}
    assert nodes.parse_convrot_layers(None) == {} and nodes.parse_convrot_layers({"x": 1}) == {}


def test_quantize_state_dict_plain_passthrough_and_convrot():
    g = torch.Generator().manual_seed(5)
    w = torch.randn(16, 64, generator=g) * 0.02
    sd = {"blk.lin.weight": w.to(torch.bfloat16), "blk.lin.bias": torch.zeros(16),
          "blk.norm.scale": torch.ones(64), "blk.odd.weight": torch.randn(8, 40, generator=g),
          "blk.cr.weight": torch.randint(-8, 8, (16, 32), dtype=torch.int8, generator=g),
          "blk.cr.weight_scale": torch.rand(16, generator=g)}
    meta = {"_quantization_metadata": json.dumps({"layers": {
        "blk.cr": {"format": "convrot_w4a4", "convrot_groupsize": 64, "quant_group_size": 64}}})}
    calls = []

    def decoder(t, scale, convrot_groupsize, quant_group_size, output_dtype):
        calls.append((convrot_groupsize, quant_group_size, output_dtype))
        lo = (t.to(torch.int16) & 0xF) - ((t.to(torch.int16) & 0x8) << 1)
        hi = (t.to(torch.int16) >> 4)
        return torch.stack([lo, hi], -1).reshape(t.shape[0], -1).float() * scale[:, None]

    q, counts = nodes.quantize_state_dict(sd, "cpu", meta, convrot_decoder=decoder)
    assert counts == {"quantized": 1, "convrot_repacked": 1, "passthrough": 3}
    assert calls == [(64, 64, torch.float32)]
    assert set(q) == {"blk.lin.weight_q4", "blk.lin.weight_scale", "blk.lin.bias", "blk.norm.scale",
                      "blk.odd.weight", "blk.cr.weight_q4", "blk.cr.weight_scale"}
    p, s = orc.quantize_pack_int4(w.to(torch.bfloat16).float().numpy(), rule="div")
    assert np.array_equal(q["blk.lin.weight_q4"].numpy(), p) and np.array_equal(q["blk.lin.weight_scale"].numpy(), s)
    dec = decoder(sd["blk.cr.weight"], sd["blk.cr.weight_scale"], 64, 64, torch.float32)
    p2, s2 = orc.quantize_pack_int4(dec.numpy(), rule="div")
    assert np.array_equal(q["blk.cr.weight_q4"].numpy(), p2) and np.array_equal(q["blk.cr.weight_scale"].numpy(), s2)
    with pytest.raises(RuntimeError, match="comfy_kitchen"):
        nodes.quantize_state_dict(sd, "cpu", meta)


def test_loader_state_dict_loads_into_engine_model_like_transcode():
    """The UNet loader's quantized state dict, loaded into a model built with Gfx906Int4Ops, holds
    the same buffers as transcoding the float model."""
    float_model = _float_dit()
    qsd, counts = nodes.quantize_state_dict(float_model.state_dict(), "cpu")
    assert counts["passthrough"] > 0 and counts["convrot_repacked"] == 0
    engine = fd.FluxDiT(fd.FluxDiTConfig.tiny(), device="cpu", dtype=torch.float32)
    engine.load_state_dict(qsd)
    nodes.transcode_linears(float_model)
    a, b = engine.state_dict(), float_model.state_dict()
    assert set(a) == set(b)
    for k in a:
        assert torch.equal(a[k], b[k]), k


def test_default_device():
    assert nodes._default_device(["cpu"]) == "cpu"
    assert nodes._default_device(["cpu", "cuda:0"]) == "cuda:0"
    assert nodes._default_device(["cpu", "cuda:0", "cuda:1"]) == "cuda:1"
