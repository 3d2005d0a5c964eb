"""The two loader nodes executed end to end on the CPU against stand-in ComfyUI modules.

ComfyUI is not installed here, so `folder_paths`, `comfy.utils`, `comfy.model_detection`,
`comfy.model_management`, `comfy.model_patcher`, `comfy.storage`, `comfy.ops`, `comfy.sd` and
ComfyUI-GGUF's loader are replaced by small recording stand-ins with ComfyUI's call signatures.
The tests pin what the node bodies do with them, against the reference's loaders
(nodes/ComfyUI-Gfx906Int4/nodes.py:382-398 CLIP, :483-599 UNet): which ComfyUI calls are made
with which arguments and in which order, that architecture detection sees the float state dict
while the model is built from and loaded with the quantized one, the quantized buffers (the
reference's CPU quantizer rule for a CPU-loaded checkpoint, bit for bit against the oracle), the
printed counts and the error paths.
"""
import sys
import types

import numpy as np
import pytest
import torch

from comfy_ui_gfx906_tools_amd import flux_dit as fd, nodes
from comfy_ui_gfx906_tools_amd.ops import Gfx906Int4Ops
from oracle import qlinear_oracle as orc
from tests.conftest import golden_path

PREFIX = "model.diffusion_model."


class _Calls(list):
    def add(self, call, **kw):
        self.append((call, kw))

    def names(self):
        return [n for n, _ in self]

    def get(self, name):
        return [kw for n, kw in self if n == name]


def _float_dit_sd():
    m = fd.FluxDiT(fd.FluxDiTConfig.tiny(), ops=torch.nn, dtype=torch.float32, device="cpu")
    fd.init_random_(m, seed=17)
    return {k: v.detach().to(torch.bfloat16).clone() for k, v in m.state_dict().items()}


class _BaseModel:
    """What get_model returns: ComfyUI's BaseModel wrapper around the diffusion model."""

    def __init__(self, ops, calls):
        self.diffusion_model = fd.FluxDiT(fd.FluxDiTConfig.tiny(), ops=ops, dtype=torch.float32, device="cpu")
        self.calls = calls

    def to(self, device):
        self.calls.add("model.to", device=device)
        return self

    def load_model_weights(self, sd, prefix):
        self.calls.add("load_model_weights", sd=sd, prefix=prefix)
        self.diffusion_model.load_state_dict(sd, strict=True)


class _ModelConfig:
    supported_inference_dtypes = [torch.bfloat16, torch.float32]

    def __init__(self, calls):
        self.calls = calls
        self.custom_operations = None

    def set_inference_dtype(self, dtype, manual_cast_dtype, device=None):
        self.calls.add("set_inference_dtype", dtype=dtype, manual_cast_dtype=manual_cast_dtype, device=device)

    def get_model(self, sd, prefix):
        self.calls.add("get_model", sd=sd, prefix=prefix, ops=self.custom_operations)
        return _BaseModel(self.custom_operations, self.calls)


@pytest.fixture
def comfy(monkeypatch):
    """Install the stand-in ComfyUI modules; yields (calls, files) where files maps a model path
    to (state dict, metadata) for load_torch_file / the GGUF loader / load_clip."""
    calls, files = _Calls(), {}
    fp = types.ModuleType("folder_paths")

    def get_full_path_or_raise(kind, name):
        calls.add("get_full_path_or_raise", kind=kind, name=name)
        return f"/models/{kind}/{name}"

    fp.get_full_path_or_raise = get_full_path_or_raise
    fp.get_folder_paths = lambda kind: (calls.add("get_folder_paths", kind=kind), [f"/models/{kind}"])[1]
    fp.get_filename_list = lambda kind: sorted(p.rsplit("/", 1)[1] for p in files if f"/{kind}/" in p)
    fp.folder_names_and_paths = {}

    comfy_pkg = types.ModuleType("comfy")
    comfy_pkg.__path__ = []
    utils = types.ModuleType("comfy.utils")

    def load_torch_file(path, return_metadata=False):
        calls.add("load_torch_file", path=path, return_metadata=return_metadata)
        sd, meta = files[path]
        return (dict(sd), meta) if return_metadata else dict(sd)

    def state_dict_prefix_replace(sd, replace, filter_keys=False):
        calls.add("state_dict_prefix_replace", replace=replace, filter_keys=filter_keys)
        out = {} if filter_keys else dict(sd)
        for old, new in replace.items():
            for k in [k for k in sd if k.startswith(old)]:
                out[new + k[len(old):]] = sd[k]
                if not filter_keys:
                    out.pop(k)
        return out

    utils.load_torch_file = load_torch_file
    utils.state_dict_prefix_replace = state_dict_prefix_replace
    utils.calculate_parameters = lambda sd: (calls.add("calculate_parameters", sd=sd),
                                             sum(v.numel() for v in sd.values()))[1]
    utils.weight_dtype = lambda sd: (calls.add("weight_dtype", sd=sd), torch.bfloat16)[1]

    md = types.ModuleType("comfy.model_detection")
    md.unet_prefix_from_state_dict = lambda sd: (calls.add("unet_prefix_from_state_dict"),
                                                 PREFIX if any(k.startswith(PREFIX) for k in sd) else "")[1]

    def model_config_from_unet(sd, prefix, metadata=None):
        calls.add("model_config_from_unet", sd=sd, prefix=prefix, metadata=metadata)
        return None if "img_in.weight" not in sd else _ModelConfig(calls)

    md.model_config_from_unet = model_config_from_unet

    mm = types.ModuleType("comfy.model_management")
    mm.unet_dtype = lambda model_params, supported_dtypes, weight_dtype: (
        calls.add("unet_dtype", model_params=model_params, supported_dtypes=supported_dtypes,
                  weight_dtype=weight_dtype), torch.bfloat16)[1]
    mm.unet_manual_cast = lambda dtype, device, supported: (
        calls.add("unet_manual_cast", dtype=dtype, device=device, supported=supported), None)[1]
    mm.unet_offload_device = lambda: (calls.add("unet_offload_device"), torch.device("cpu"))[1]
    mm.is_device_cpu = lambda d: (calls.add("is_device_cpu", device=d), torch.device(d).type == "cpu")[1]

    mp = types.ModuleType("comfy.model_patcher")

    class ModelPatcher:
        def __init__(self, model, load_device, offload_device, fast_disk=False):
            calls.add("ModelPatcher", model=model, load_device=load_device, offload_device=offload_device,
                      fast_disk=fast_disk)
            self.model = model

    mp.ModelPatcher = ModelPatcher
    storage = types.ModuleType("comfy.storage")
    storage.state_dict_fast_disk = lambda sd: (calls.add("state_dict_fast_disk", sd=sd), False)[1]

    cops = types.ModuleType("comfy.ops")

    class manual_cast:  # noqa: N801 - ComfyUI's name
        Linear = torch.nn.Linear
        LayerNorm = torch.nn.LayerNorm

    cops.manual_cast = manual_cast

    csd = types.ModuleType("comfy.sd")

    class CLIPType:
        STABLE_DIFFUSION = "sd"
        KREA2 = "krea2"
        FLUX = "flux"

    class _Encoder(torch.nn.Module):
        """A text encoder built with the model_options' custom_operations, as ComfyUI's do."""

        def __init__(self, ops):
            super().__init__()
            self.norm = ops.LayerNorm(256)
            self.fc1 = ops.Linear(256, 512)
            self.fc2 = ops.Linear(512, 256)
            self.head = ops.Linear(256, 40)  # K % 32 == 0: quantized
            self.odd = ops.Linear(40, 8)     # K % 32 != 0: stays float

    class CLIP:
        def __init__(self, model):
            self.cond_stage_model = model

    def load_clip(ckpt_paths, embedding_directory=None, clip_type=None, model_options=None):
        calls.add("load_clip", ckpt_paths=ckpt_paths, embedding_directory=embedding_directory, clip_type=clip_type,
                  model_options=model_options)
        enc = _Encoder(model_options["custom_operations"])
        sd, _ = files[ckpt_paths[0]]
        enc.load_state_dict(dict(sd), strict=True)
        return CLIP(enc)

    csd.CLIPType = CLIPType
    csd.load_clip = load_clip
    comfy_pkg.utils, comfy_pkg.model_detection, comfy_pkg.model_management = utils, md, mm
    comfy_pkg.model_patcher, comfy_pkg.storage, comfy_pkg.ops, comfy_pkg.sd = mp, storage, cops, csd
    for name, mod in {"folder_paths": fp, "comfy": comfy_pkg, "comfy.utils": utils, "comfy.model_detection": md,
                      "comfy.model_management": mm, "comfy.model_patcher": mp, "comfy.storage": storage,
                      "comfy.ops": cops, "comfy.sd": csd}.items():
        monkeypatch.setitem(sys.modules, name, mod)
    calls.encoder_type = _Encoder
    yield calls, files


def _quantized_like_reference(w: torch.Tensor):
    """The reference UNet loader's quantizer on a CPU-loaded weight: torch's CPU `amax / 7.0`."""
    return orc.quantize_pack_int4(w.float().numpy(), rule="div")


def test_unet_loader_runs_the_reference_sequence(comfy, capsys):
    calls, files = comfy
    float_sd = _float_dit_sd()
    path = "/models/diffusion_models/tiny.safetensors"
    files[path] = ({PREFIX + k: v for k, v in float_sd.items()}, {"format": "pt"})
    (patcher,) = nodes.Gfx906Int4UnetLoader().load_unet("tiny.safetensors", "cpu")

    names = calls.names()
    # order constraints of the reference (nodes.py:483-599): read, strip the prefix, quantize,
    # detect on the float dict, dtype selection, build with the int4 ops, wrap, load the weights
    for a, b in [("load_torch_file", "unet_prefix_from_state_dict"),
                 ("unet_prefix_from_state_dict", "state_dict_prefix_replace"),
                 ("state_dict_prefix_replace", "model_config_from_unet"),
                 ("model_config_from_unet", "unet_dtype"), ("unet_dtype", "unet_manual_cast"),
                 ("unet_manual_cast", "set_inference_dtype"), ("set_inference_dtype", "get_model"),
                 ("get_model", "ModelPatcher"), ("ModelPatcher", "load_model_weights")]:
        assert names.index(a) < names.index(b), (a, b, names)
    assert calls.get("get_full_path_or_raise") == [{"kind": "diffusion_models", "name": "tiny.safetensors"}]
    assert calls.get("load_torch_file") == [{"path": path, "return_metadata": True}]
    assert calls.get("state_dict_prefix_replace") == [{"replace": {PREFIX: ""}, "filter_keys": True}]
    det = calls.get("model_config_from_unet")[0]
    assert det["prefix"] == "" and det["metadata"] == {"format": "pt"}
    assert set(det["sd"]) == set(float_sd)  # the float, prefix-stripped dict
    assert calls.get("calculate_parameters")[0]["sd"] is det["sd"]
    assert calls.get("unet_dtype")[0]["supported_dtypes"] == [torch.bfloat16, torch.float32]
    assert calls.get("set_inference_dtype") == [{"dtype": torch.bfloat16, "manual_cast_dtype": None,
                                                 "device": torch.device("cpu")}]
    built = calls.get("get_model")[0]
    assert built["ops"] is Gfx906Int4Ops and built["prefix"] == ""
    qsd = built["sd"]
    assert calls.get("load_model_weights")[0]["sd"] is qsd and calls.get("state_dict_fast_disk")[0]["sd"] is qsd
    mp_call = calls.get("ModelPatcher")[0]
    assert mp_call["load_device"] == torch.device("cpu") and mp_call["offload_device"] == torch.device("cpu")
    assert "model.to" not in names  # the offload device is the CPU: no move (nodes.py:596-597)
    assert patcher.model is mp_call["model"]

    # the quantized dict: every eligible 2-D weight as weight_q4 / weight_scale, the rest as is
    n_q = n_p = 0
    for k, v in float_sd.items():
        base = k[:-len(".weight")] if k.endswith(".weight") else None
        if base is not None and v.ndim == 2 and v.shape[1] % 32 == 0:
            p, s = _quantized_like_reference(v)
            assert np.array_equal(qsd[base + ".weight_q4"].numpy(), p), base
            assert np.array_equal(qsd[base + ".weight_scale"].numpy(), s), base
            assert k not in qsd
            n_q += 1
        else:
            assert torch.equal(qsd[k], v), k
            n_p += 1
    out = capsys.readouterr().out
    assert f"[Gfx906Int4UnetLoader] quantized={n_q} convrot_repacked=0 passthrough_tensors={n_p} device=cpu" in out
    # the built model holds those buffers
    dm = patcher.model.diffusion_model
    lin = dm.double_blocks[0].img_attn.qkv
    assert isinstance(lin, Gfx906Int4Ops.Linear)
    assert torch.equal(lin.weight_q4, qsd["double_blocks.0.img_attn.qkv.weight_q4"])


def test_unet_loader_gguf_and_errors(comfy, monkeypatch):
    calls, files = comfy
    float_sd = _float_dit_sd()
    loader = nodes.Gfx906Int4UnetLoader()
    files["/models/diffusion_models/tiny.gguf"] = (float_sd, None)
    with pytest.raises(RuntimeError, match="requires ComfyUI-GGUF"):
        loader.load_unet("tiny.gguf", "cpu")
    gguf_loader = types.ModuleType("ComfyUI-GGUF.loader")
    gguf_loader.gguf_sd_loader = lambda path: (calls.add("gguf_sd_loader", path=path), (dict(files[path][0]), {}))[1]
    monkeypatch.setitem(sys.modules, "ComfyUI-GGUF.loader", gguf_loader)
    loader.load_unet("tiny.gguf", "cpu")
    assert calls.get("gguf_sd_loader") == [{"path": "/models/diffusion_models/tiny.gguf"}]
    assert "load_torch_file" not in calls.names() and "state_dict_prefix_replace" not in calls.names()
    assert calls.get("model_config_from_unet")[-1]["metadata"] is None
    # an undetectable architecture
    files["/models/diffusion_models/bad.safetensors"] = ({"w.weight": torch.zeros(4, 32)}, {})
    with pytest.raises(RuntimeError, match="Could not detect model type"):
        loader.load_unet("bad.safetensors", "cpu")


@pytest.mark.parametrize("rotation", [False, True])
def test_clip_loader_quantizes_while_loading(comfy, capsys, rotation):
    calls, files = comfy
    g = torch.Generator().manual_seed(23)
    sd = {"norm.weight": torch.ones(256), "norm.bias": torch.zeros(256),
          "fc1.weight": torch.randn(512, 256, generator=g) * 0.02, "fc1.bias": torch.randn(512, generator=g),
          "fc2.weight": torch.randn(256, 512, generator=g) * 0.02, "fc2.bias": torch.randn(256, generator=g),
          "head.weight": torch.randn(40, 256, generator=g) * 0.02, "head.bias": torch.zeros(40),
          "odd.weight": torch.randn(8, 40, generator=g), "odd.bias": torch.zeros(8)}
    files["/models/text_encoders/enc.safetensors"] = (sd, None)
    (clip,) = nodes.Gfx906Int4CLIPLoader().load_clip("enc.safetensors", "krea2", "cpu", rotation)
    assert calls.get("get_full_path_or_raise") == [{"kind": "text_encoders", "name": "enc.safetensors"}]
    lc = calls.get("load_clip")[0]
    assert lc["ckpt_paths"] == ["/models/text_encoders/enc.safetensors"]
    assert lc["embedding_directory"] == ["/models/embeddings"] and lc["clip_type"] == "krea2"
    ops = lc["model_options"]["custom_operations"]
    assert lc["model_options"]["load_device"] == torch.device("cpu")
    assert issubclass(ops, sys.modules["comfy.ops"].manual_cast) and ops.Linear.quantize_device == torch.device("cpu")
    enc = clip.cond_stage_model
    assert ops.Linear.quantized_on_load == 3 and not enc.odd.quantized
    signs = np.load(golden_path("rotation_signs.npz"))
    for name in ("fc1", "fc2", "head"):
        lin = getattr(enc, name)
        w = sd[f"{name}.weight"].float().numpy()
        g_rot = lin.rotation_group
        assert bool(g_rot) == rotation
        if g_rot:  # the rotation folded into the weight before quantizing (ops.py:228-246)
            # the reference's fold is torch's fp32 matmul t.reshape(-1, g) @ R^T (ops.py:85-105); R from
            # the committed signs fixture and the float64 Hadamard (its own accuracy is pinned in
            # tests/test_oracle.py and tests/test_gpu_rotate.py)
            R = torch.from_numpy(orc.group_rotation(signs[f"signs_{g_rot}"]).astype(np.float32))
            w = (torch.from_numpy(w).reshape(-1, g_rot) @ R.t()).reshape(w.shape).numpy()
        p, s = orc.quantize_pack_int4(w, rule="div")  # quantized on the CPU device here
        assert np.array_equal(lin.weight_q4.numpy(), p), name
        assert np.array_equal(lin.weight_scale.numpy(), s), name
        assert torch.equal(lin.bias, sd[f"{name}.bias"])
    assert f"[Gfx906Int4CLIPLoader] quantized=3 rotation={rotation} device=cpu" in capsys.readouterr().out


def test_clip_loader_errors(comfy):
    calls, files = comfy
    loader = nodes.Gfx906Int4CLIPLoader()
    with pytest.raises(ValueError, match="expected a safetensors text encoder"):
        loader.load_clip("enc.gguf", "krea2", "cpu", False)
    # a checkpoint whose Linears arrive already packed: none is quantized while loading
    enc = calls.encoder_type(nodes.make_load_quantizing_ops(sys.modules["comfy.ops"].manual_cast, "cpu", False))
    files["/models/text_encoders/packed.safetensors"] = (enc.state_dict(), None)
    with pytest.raises(RuntimeError, match="expected all 3 int4 Linears quantized from float weights, got 0"):
        loader.load_clip("packed.safetensors", "krea2", "cpu", False)
