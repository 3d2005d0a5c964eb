"""The full-size C5 configuration on the GPU: the 12B Flux-style DiT (hidden 3072, 24 heads x 128,
19 double + 38 single blocks) at 1024 x 1024 (4096 image + 512 text tokens, batch 1), random
weights quantized on the device by the HIP quantizer, every Linear on the W4A16 engine.

* Double block 0 (image and text streams) and single block 0, run by the engine on the real
  activations entering them, against the same blocks in fp32 on the host with the dequantized
  int4 weights: max|d| / max|ref| <= 2% (the engine keeps bf16 activations between the block's
  operations; the GEMMs themselves are within 2e-3 of their fp32 dequant reference).
* The whole 57-block step, twice: finite and bit-identical (every kernel on the path is
  deterministic: no atomics, fixed reduction orders).
"""
import numpy as np
import pytest
import torch

from tests.gpu_util import dequant_torch

pytestmark = pytest.mark.gpu
GATE = 2e-2


def _host_block(gpu_block, cls, cfg, fd):
    """The block in fp32 on the host: weights = the dequantized int4 codes, same biases and norms."""
    blk = cls(cfg, torch.nn, dtype=torch.float32)
    sd = {}
    for name, mod in gpu_block.named_modules():
        if fd._is_engine_linear(mod):
            sd[f"{name}.weight"] = dequant_torch(mod.weight_q4, mod.weight_scale).cpu()
            sd[f"{name}.bias"] = mod.bias.float().cpu()
    for name, p in gpu_block.named_parameters():
        if name.endswith(".scale"):
            sd[name] = p.float().cpu()
    blk.load_state_dict(sd)
    return blk


def _rel(a: torch.Tensor, b: torch.Tensor) -> float:
    a, b = a.float().cpu().double(), b.double()
    return float((a - b).abs().max() / b.abs().max())


def test_c5_full_size_blocks_vs_host_fp32_and_deterministic_step():
    from comfy_ui_gfx906_tools_amd import flux_dit as fd
    cfg = fd.FluxDiTConfig.flux12b()
    assert (cfg.hidden, cfg.heads, cfg.depth_double, cfg.depth_single) == (3072, 24, 19, 38)
    n_side, n_txt = 64, 512
    print("case C5 full size: building the 12B DiT on cuda:0", flush=True)
    with torch.no_grad():
        model = fd.FluxDiT(cfg, device="cuda", dtype=torch.bfloat16)
        fd.init_random_(model, seed=4)
        inp = fd.synthetic_inputs(cfg, n_side, n_txt, seed=4, device="cuda")
        print("case C5 full size: two whole steps", flush=True)
        y1 = model(*inp)
        y2 = model(*inp)
        torch.cuda.synchronize()
        assert y1.shape == (1, n_side * n_side, cfg.in_channels)
        assert bool(torch.isfinite(y1).all()), "non-finite step output"
        assert torch.equal(y1, y2), "two runs of the step differ"

        print("case C5 full size: block 0 inputs", flush=True)
        img, img_ids, txt, txt_ids, ts, yv, gd = inp
        dt = torch.bfloat16
        h_img = fd._linear(model.img_in, img)
        vec = fd._linear(model.time_in.in_layer, fd.timestep_embedding(ts, cfg.time_dim).to(dt))
        vec = fd._linear(model.time_in.out_layer, torch.nn.functional.silu(vec))
        vec = vec + model.guidance_in(fd.timestep_embedding(gd, cfg.time_dim).to(dt)) + model.vector_in(yv)
        h_txt = fd._linear(model.txt_in, txt)
        cos, sin = fd.rope_cos_sin(torch.cat([txt_ids, img_ids], 1), cfg.axes_dim, cfg.theta)
        dblk, sblk = model.double_blocks[0], model.single_blocks[0]
        g_img, g_txt = dblk(h_img, h_txt, vec, cos, sin)
        x_cat = torch.cat([g_txt, g_img], 1)
        g_single = sblk(x_cat, vec, cos, sin)
        torch.cuda.synchronize()

        print("case C5 full size: host fp32 double block 0", flush=True)
        c_cos, c_sin, c_vec = cos.cpu(), sin.cpu(), vec.float().cpu()
        hd = _host_block(dblk, fd.DoubleStreamBlock, cfg, fd)
        r_img, r_txt = hd(h_img.float().cpu(), h_txt.float().cpu(), c_vec, c_cos, c_sin)
        del hd
        print("case C5 full size: host fp32 single block 0", flush=True)
        hs = _host_block(sblk, fd.SingleStreamBlock, cfg, fd)
        r_single = hs(x_cat.float().cpu(), c_vec, c_cos, c_sin)
        del hs
    errs = {"double0_img": _rel(g_img, r_img), "double0_txt": _rel(g_txt, r_txt), "single0": _rel(g_single, r_single)}
    print(f"C5 block parity (max|d|/max|ref|): {errs}", flush=True)
    for k, e in errs.items():
        assert np.isfinite(e) and e <= GATE, f"{k}: {e:.3e} > {GATE}"
