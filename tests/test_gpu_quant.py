"""Device-side int4 quantize + pack (quantize_pack_int4 for GPU-resident weights): bit-exact
against the oracle for both scale rules, and against the reference's own torch expression
(ops.py:108-126) evaluated by torch on the same GPU."""
import numpy as np
import pytest
import torch

from oracle import qlinear_oracle as orc
from tests.gpu_util import to_np_f32

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _lib():
    from comfy_ui_gfx906_tools_amd import _lib
    return _lib


def _reference_torch_expression(t: torch.Tensor):
    """ops.py:108-126 verbatim in its arithmetic (the reference's quantizer), run by torch."""
    K = t.shape[-1]
    tb = t.reshape(-1, K // 32, 32).float()
    amax = tb.abs().amax(dim=-1, keepdim=True).clamp_min(1e-8)
    scale = amax / 7.0
    codes = torch.round(tb / scale).clamp(-8, 7).to(torch.int32).reshape(-1, K)
    packed = ((codes[:, 0::2] & 0xF) | ((codes[:, 1::2] & 0xF) << 4)).to(torch.uint8).view(torch.int8)
    return packed.reshape(*t.shape[:-1], K // 2), scale.reshape(*t.shape[:-1], K // 32)


@pytest.mark.parametrize("rule,rname", [(0, "div"), (1, "recip")])
@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16, torch.float16])
def test_quantize_int4_matches_oracle(rule, rname, dt):
    print(f"case quant4 rule={rname} {dt}", flush=True)
    g = torch.Generator().manual_seed(7)
    x = (torch.randn(67, 1024, generator=g) * torch.rand(67, 1, generator=g) * 3).to(dt)
    x[3] = 0
    p, s = _lib().quantize_int4(x.to(DEV), rule)
    p_ref, s_ref = orc.quantize_pack_int4(to_np_f32(x), rule=rname)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), s_ref.view(np.uint32))
    assert np.array_equal(p.cpu().numpy(), p_ref)


def test_quantize_pack_int4_gpu_equals_reference_torch_on_gpu():
    """ops.quantize_pack_int4 of a device tensor must equal the reference's torch expression
    evaluated on the same device, bit for bit (packed bytes and scales)."""
    from comfy_ui_gfx906_tools_amd import ops
    g = torch.Generator().manual_seed(8)
    w = (torch.randn(512, 3072, generator=g) * 0.02).to(DEV)
    p, s = ops.quantize_pack_int4(w)
    p_ref, s_ref = _reference_torch_expression(w)
    same_scale = torch.equal(s, s_ref)
    # report which rule torch used on this device if the HIP rule disagrees
    if not same_scale:
        p0, s0 = _lib().quantize_int4(w, 0)
        p1, s1 = _lib().quantize_int4(w, 1)
        pytest.fail(f"scale mismatch: torch-GPU == rule0? {torch.equal(s0, s_ref)}; == rule1? {torch.equal(s1, s_ref)}")
    assert torch.equal(p, p_ref)


@pytest.mark.parametrize("out_f,in_f,offset", [(1, 32, 0), (5, 96, 2), (300, 4096, 0), (7, 3072, 2)])
def test_repack_q4_0_matches_oracle(out_f, in_f, offset):
    """HIP Q4_0 -> native repack (ops.py:129-164): bit-exact against the oracle's restatement, and
    dequantized equal to the ggml Q4_0 definition; fp16 d of every class (zero, -0, subnormal,
    max), a block with every nibble 0 (code -8), and a source only 2-byte aligned (offset 2)."""
    print(f"case q4_0 {out_f}x{in_f} offset={offset}", flush=True)
    rng = np.random.default_rng(out_f + in_f)
    n = out_f * in_f // 32
    d = (rng.standard_normal(n) * 0.01).astype(np.float16)
    special = np.array([0.0, -0.0, 6e-8, 65504.0, -2.0 ** -14], dtype=np.float16)
    d[: min(n, len(special))] = special[: min(n, len(special))]
    qs = rng.integers(0, 256, (n, 16)).astype(np.uint8)
    qs[-1] = 0  # every element at code -8
    raw = np.concatenate([d.view(np.uint8).reshape(n, 2), qs], axis=1).reshape(-1)
    buf = torch.zeros(raw.size + offset, dtype=torch.uint8)
    buf[offset:] = torch.from_numpy(raw)
    dev = buf.to(DEV)[offset:]
    packed, scale = _lib().repack_q4_0(dev, out_f, in_f)
    p_ref, s_ref = orc.repack_q4_0_native(raw, out_f, in_f)
    assert np.array_equal(packed.cpu().numpy(), p_ref)
    assert np.array_equal(scale.cpu().numpy().view(np.uint32), s_ref.view(np.uint32))
    deq = orc.dequant_int4(packed.cpu().numpy(), scale.cpu().numpy())
    assert np.array_equal(deq, orc.ggml_q4_0_dequant(raw, out_f, in_f))


def test_repack_q4_0_through_ops_on_device():
    """ops.repack_q4_0_native takes the HIP kernel for device tensors and returns the same as on CPU."""
    from comfy_ui_gfx906_tools_amd import ops
    rng = np.random.default_rng(9)
    out_f, in_f = 16, 256
    n = out_f * in_f // 32
    d = (rng.standard_normal(n) * 0.01).astype(np.float16)
    raw = np.concatenate([d.view(np.uint8).reshape(n, 2), rng.integers(0, 256, (n, 16)).astype(np.uint8)], axis=1)
    t = torch.from_numpy(raw.reshape(-1))
    p_cpu, s_cpu = ops.repack_q4_0_native(t, out_f, in_f)
    p_dev, s_dev = ops.repack_q4_0_native(t.to(DEV), out_f, in_f)
    assert p_dev.is_cuda and torch.equal(p_dev.cpu(), p_cpu) and torch.equal(s_dev.cpu(), s_cpu)


def test_unet_loader_quantizes_cpu_loaded_weights_with_the_cpu_rule():
    """The reference's UNet loader quantizes a plain float weight where load_torch_file put it, the
    CPU (nodes.py:557-561 -> quantize_pack_int4 on a CPU tensor: a true `amax / 7.0`). The engine's
    loader computes on the GPU but must produce the same bytes: nodes.quantize_state_dict(sd, cuda)
    against the reference's torch expression on the CPU tensors, bit for bit (the GPU's own rule
    differs from it in the last bit of about half the scales on random data)."""
    from comfy_ui_gfx906_tools_amd import nodes
    g = torch.Generator().manual_seed(31)
    sd = {"a.weight": torch.randn(300, 1024, generator=g) * 0.02,
          "b.weight": (torch.randn(64, 3072, generator=g) * 0.05).to(torch.bfloat16),
          "c.weight": (torch.randn(40, 96, generator=g) * 3.0).to(torch.float16)}
    q, counts = nodes.quantize_state_dict(sd, DEV)
    assert counts["quantized"] == 3
    for base in ("a", "b", "c"):
        p_ref, s_ref = _reference_torch_expression(sd[base + ".weight"])
        assert q[base + ".weight_q4"].device.type == "cpu"
        assert torch.equal(q[base + ".weight_scale"], s_ref), base
        assert torch.equal(q[base + ".weight_q4"], p_ref), base
    # the GPU rule on the same data does differ somewhere (so the test distinguishes the rules)
    _, s_gpu = _lib().quantize_int4(sd["a.weight"].to(DEV), 1)
    assert not torch.equal(s_gpu.cpu(), q["a.weight_scale"])
