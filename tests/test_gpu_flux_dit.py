"""The Flux-style DiT on the W4A16 engine (every Linear through libqlinear.so, attention on
SDPA) against the same model in fp32 on the host whose weights are the dequantized int4 codes
(the reference's dequantize-then-matmul numerics, nodes/ComfyUI-Gfx906Int4/nodes.py:43-52).
The engine model keeps bf16 activations between ops, so the gate is on the whole output:
max|y - ref| / max|ref| <= 2e-2."""
import numpy as np
import pytest
import torch

from comfy_ui_gfx906_tools_amd import flux_dit as fd
from tests.conftest import golden_path
from tests.gpu_util import dequant_torch, rel_max_err

pytestmark = pytest.mark.gpu

GATE = 2e-2


def _float_twin(model: fd.FluxDiT) -> fd.FluxDiT:
    ref = fd.FluxDiT(model.cfg, ops=torch.nn, dtype=torch.float32)
    sd = {}
    for name, mod in model.named_modules():
        if fd._is_engine_linear(mod):
            sd[f"{name}.weight"] = dequant_torch(mod.weight_q4, mod.weight_scale).cpu()
            sd[f"{name}.bias"] = mod.bias.float().cpu()
    for name, p in model.named_parameters():
        if name.endswith(".scale"):
            sd[name] = p.float().cpu()
    ref.load_state_dict(sd)
    return ref


@pytest.mark.parametrize("n_side,n_txt", [(8, 16), (16, 40)])
def test_tiny_dit_matches_fp32_dequant_model(n_side, n_txt):
    cfg = fd.FluxDiTConfig.tiny()
    print(f"tiny DiT n_side={n_side} n_txt={n_txt}", flush=True)
    with torch.no_grad():
        m = fd.FluxDiT(cfg, device="cuda", dtype=torch.bfloat16)
        fd.init_random_(m, seed=3)
        inp = fd.synthetic_inputs(cfg, n_side, n_txt, seed=0, device="cuda")
        y = m(*inp)
        y2 = m(*inp)
        torch.cuda.synchronize()
        ref = _float_twin(m)(*[t.float().cpu() for t in inp])
    assert torch.equal(y, y2), "two forwards on the same inputs differ"
    err = rel_max_err(y.float().cpu().numpy(), ref.numpy())
    assert np.isfinite(err) and err <= GATE, f"max rel err {err:.3e}"


def test_single_block_split_linear1_matches_whole():
    """linear1 run as two GEMMs on row slices of the packed weight ([qkv | mlp]) gives the whole
    GEMM's columns (to one bf16 rounding: the planner may cut K differently at another N), with
    the GELU of the second half fused."""
    cfg = fd.FluxDiTConfig.tiny()
    with torch.no_grad():
        m = fd.FluxDiT(cfg, device="cuda", dtype=torch.bfloat16)
        fd.init_random_(m, seed=7)
        lin = m.single_blocks[0].linear1
        x = torch.randn(100, cfg.hidden, device="cuda").to(torch.bfloat16)
        whole = lin(x)
        h3 = 3 * cfg.hidden
        qkv = fd._linear(lin, x, rows=slice(0, h3))
        mlp = fd._linear(lin, x, gelu=True, rows=slice(h3, None))
        torch.cuda.synchronize()
    w = whole[:, :h3].float()
    assert ((qkv.float() - w).abs() <= 2.0 ** -8 * w.abs() + 1e-6).all()
    ref = torch.nn.functional.gelu(whole[:, h3:].float(), approximate="tanh")
    err = (mlp.float() - ref).abs().max().item()
    assert err <= 2.0 ** -7 * max(1.0, ref.abs().max().item()), err


@pytest.mark.parametrize("rotate", [False, True])
def test_transcoded_float_dit_matches_twin(rotate):
    """A float DiT on the GPU, transcoded in place by the Transcode node's code (HIP quantizer,
    optional Hadamard rotation folded into the weights), against the fp32 host twin whose weights
    are the dequantized codes -- times the group rotation R when rotated, since
    rotate(x) @ Wq^T = x @ (Wq R)^T per group."""
    from comfy_ui_gfx906_tools_amd import nodes
    from oracle import qlinear_oracle as orc
    cfg = fd.FluxDiTConfig.tiny()
    print(f"transcoded tiny DiT rotate={rotate}", flush=True)
    with torch.no_grad():
        m = fd.FluxDiT(cfg, ops=torch.nn, device="cuda", dtype=torch.bfloat16)
        fd.init_random_(m, seed=13)
        converted, skipped, _ = nodes.transcode_linears(m, rotate=rotate)
        assert skipped == 0 and converted == sum(1 for x in m.modules() if isinstance(x, fd.Gfx906Int4Ops.Linear))
        inp = fd.synthetic_inputs(cfg, 8, 16, seed=1, device="cuda")
        y = m(*inp)
        torch.cuda.synchronize()
        ref_model = fd.FluxDiT(cfg, ops=torch.nn, dtype=torch.float32)
        sd = {}
        signs = np.load(golden_path("rotation_signs.npz"))
        for name, mod in m.named_modules():
            if fd._is_engine_linear(mod):
                w = dequant_torch(mod.weight_q4, mod.weight_scale).cpu().double().numpy()
                g = mod.rotation_group
                assert bool(g) == rotate
                if g:
                    R = orc.group_rotation(signs[f"signs_{g}"]).astype(np.float64)
                    w = (w.reshape(w.shape[0], -1, g) @ R).reshape(w.shape)
                sd[f"{name}.weight"] = torch.from_numpy(w).float()
                sd[f"{name}.bias"] = mod.bias.float().cpu()
        for name, p in m.named_parameters():
            if name.endswith(".scale"):
                sd[name] = p.float().cpu()
        ref_model.load_state_dict(sd)
        ref = ref_model(*[t.float().cpu() for t in inp])
    err = rel_max_err(y.float().cpu().numpy(), ref.numpy())
    assert np.isfinite(err) and err <= GATE, f"max rel err {err:.3e}"
