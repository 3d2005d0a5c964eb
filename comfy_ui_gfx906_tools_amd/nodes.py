"""ComfyUI nodes of the quantized-linear path: the reference's linear-related node set
(nodes/ComfyUI-Gfx906Int4/nodes.py:602-622) with the same class names, widgets, return types and
CATEGORY, so saved workflows resolve to these classes. Each node ends in the same module state as
the reference (``weight_q4`` / ``weight_scale`` Linears from ops.py); the forward those Linears
run is the gfx950 W4A16 engine.

ComfyUI itself (``folder_paths``, ``comfy.*``, ``nodes``) is imported inside the node methods
that need it, so this module -- and the format dispatch, the Linear swap and the state-dict
quantizer below, which are plain functions over torch modules and tensors -- also load and run
without ComfyUI. Third-party decoders are reached the way the reference reaches them: ComfyUI-GGUF
through ``sys.modules`` (nodes.py:127-142), comfy_kitchen's QuantizedTensor / ConvRot decoder by
import when installed (nodes.py:33-36, 195-207). Not included: the row-split, attention and VAE
nodes (not on the quantized-linear path).
"""
from __future__ import annotations

import json
import re
import sys

import torch

from . import _lib
from .ops import (BLOCK, Gfx906Int4Ops, apply_group_rotation, choose_rotation_group, get_group_rotation,
                  make_load_quantizing_ops, quantize_pack_int4, repack_q4_0_native)

CATEGORY = "gfx906"
# module-name prefixes the test patch leaves in full precision (nodes.py:40)
SPARED_PREFIXES = ("x_embedder", "final_layer", "cap_embedder", "t_embedder")
_ROTATION_TOOLTIP = ("Randomized Hadamard rotation of weight+activation before quantizing (SpinQuant / QuIP# "
                     "style): spreads outlier energy without calibration data; a GGUF Q4_0 weight then takes "
                     "the dequantize + requantize path instead of the lossless repack.")


# ---------------------------------------------------------------------------------------------
# weight emulation and format dispatch
# ---------------------------------------------------------------------------------------------
def quantize_dequantize_int4(t: torch.Tensor, block: int = BLOCK) -> torch.Tensor:
    """Round trip of the int4 rule, in t's dtype: per `block` elements along the last dim,
    s = max(amax, 1e-8) / 7, q = clamp(round(t / s), -8, 7), t' = q * s (nodes.py:43-52).
    Tensors whose last dim is not a multiple of `block` are returned unchanged."""
    K = t.shape[-1]
    if K % block != 0:
        return t
    tb = t.float().reshape(-1, K // block, block)
    s = tb.abs().amax(dim=-1, keepdim=True).clamp_min(1e-8) / 7.0
    return (torch.round(tb / s).clamp(-8, 7) * s).reshape(t.shape).to(t.dtype)


def find_max_layer_index(root: torch.nn.Module, prefix: str = "layers.") -> int:
    """Largest N of any submodule named `<prefix>N.…` (-1 if none)."""
    pat = re.compile(re.escape(prefix) + r"(\d+)\.")
    found = [int(m.group(1)) for name, _ in root.named_modules() if (m := pat.match(name))]
    return max(found, default=-1)


def _activation_round_trip_hook(module, inputs):
    return (quantize_dequantize_int4(inputs[0]),) + tuple(inputs[1:])


class RawWeight:
    """A state-dict tensor presented as a Linear-shaped object (weight, out_features,
    in_features), so loader and transcode share quantize_module_weight (nodes.py:145-155)."""

    def __init__(self, weight: torch.Tensor, out_features: int, in_features: int):
        self.weight = weight
        self.out_features = out_features
        self.in_features = in_features


def _gguf_module(name: str):
    # ComfyUI-GGUF lives in a folder with a dash in its name: reachable only via sys.modules
    return sys.modules.get(f"ComfyUI-GGUF.{name}")


def _is_gguf_q4_0(tensor_type) -> bool:
    try:
        import gguf  # type: ignore
    except ImportError:
        return False
    return tensor_type == gguf.GGMLQuantizationType.Q4_0


def _float_weight(w) -> tuple[torch.Tensor, str]:
    """fp32 copy of a Linear weight in whatever format it arrived, and the source tag."""
    if getattr(w, "tensor_type", None) is not None:
        dq = _gguf_module("dequant")
        if dq is None:
            raise RuntimeError("GGUF-quantized weight but ComfyUI-GGUF is not loaded: it is needed to "
                               "dequantize the weight before requantizing it to int4")
        return dq.dequantize_tensor(w, dtype=torch.float32), "gguf_dequant_requant"
    try:
        from comfy_kitchen.tensor import QuantizedTensor  # type: ignore
    except ImportError:
        QuantizedTensor = None
    if QuantizedTensor is not None and isinstance(w, QuantizedTensor):
        if w.device.type == "cpu" and torch.cuda.is_available():
            w = w.cuda()  # some layouts run a rotation-undo matmul inside dequantize()
        return w.dequantize().float(), "comfy_quantized_dequant_requant"
    if w.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        raise RuntimeError(f"weight of dtype {w.dtype} is neither a plain float weight, a GGUF tensor nor a known "
                           "QuantizedTensor: no decoder for this quantization format")
    return w.detach().float(), "plain"


def quantize_module_weight(module, block_size: int = BLOCK, rotation_group: int = 0, rule: int | None = None):
    """(weight_q4 int8 [N, K/2], weight_scale fp32 [N, K/32], source tag) for a Linear-like
    object (nodes.py:157-223): a GGUF Q4_0 weight is repacked losslessly (unless a rotation must
    be folded in); any other format is decoded to fp32, optionally rotated, and quantized by
    quantize_pack_int4 (the HIP quantizer for device tensors; `rule` as there)."""
    if block_size != BLOCK:
        raise ValueError(f"the packed layout has groups of {BLOCK}, got block_size={block_size}")
    w = module.weight
    tensor_type = getattr(w, "tensor_type", None)
    if tensor_type is not None and not rotation_group and _is_gguf_q4_0(tensor_type):
        data = w.data if isinstance(w, torch.Tensor) else w
        packed, scale = repack_q4_0_native(torch.as_tensor(data), module.out_features, module.in_features)
        return packed, scale, "gguf_q4_0_repack"
    w_float, tag = _float_weight(w)
    if rotation_group:
        R = get_group_rotation(module.in_features, rotation_group, w_float.device)
        w_float = apply_group_rotation(w_float, R, rotation_group)
        tag += "_rotated"
    packed, scale = quantize_pack_int4(w_float, block_size, rule)
    return packed, scale, tag


def _mixed_precision_op_type():
    try:
        import comfy.ops  # type: ignore
        return getattr(comfy.ops, "MixedPrecisionOp", None)
    except ImportError:
        return None


def transcode_linears(root: torch.nn.Module, block_size: int = BLOCK, rotate: bool = False):
    """Replace every 2-D Linear of `root` whose in_features is a multiple of block_size (plain
    torch.nn.Linear, and ComfyUI's MixedPrecisionOp when ComfyUI is present) in place by a
    Gfx906Int4Ops.Linear on the same device and dtype (nodes.py:226-287). Returns (converted,
    skipped, {source tag: count})."""
    mixed = _mixed_precision_op_type()
    converted, skipped, sources = 0, 0, {}
    candidates = [(name, mod) for name, mod in root.named_modules()
                  if isinstance(mod, torch.nn.Linear)
                  or (mixed is not None and isinstance(mod, mixed) and getattr(mod, "weight", None) is not None)]
    with torch.no_grad():
        for name, mod in candidates:
            K, N = mod.in_features, mod.out_features
            if getattr(mod.weight, "ndim", 2) != 2 or K % block_size != 0 or K < block_size:
                skipped += 1
                continue
            group = (choose_rotation_group(K) or 0) if rotate else 0
            dev, dt = mod.weight.device, mod.weight.dtype
            packed, scale, tag = quantize_module_weight(mod, block_size, group)
            sources[tag] = sources.get(tag, 0) + 1
            new = Gfx906Int4Ops.Linear(K, N, bias=mod.bias is not None, device=dev, dtype=dt, rotation_group=group)
            new.weight_q4.copy_(packed.to(dev))
            new.weight_scale.copy_(scale.to(dev))
            if mod.bias is not None:
                new.bias.copy_(mod.bias.detach().float().to(dt))
            parent_name, _, attr = name.rpartition(".")
            setattr(root.get_submodule(parent_name) if parent_name else root, attr, new)
            converted += 1
    del candidates
    if torch.cuda.is_available():
        torch.cuda.empty_cache()  # hand the replaced float weights back to the device
    return converted, skipped, sources


def parse_convrot_layers(metadata: dict | None, prefix: str = "") -> dict:
    """{layer key without `prefix`: config} of the layers a checkpoint's
    `_quantization_metadata` JSON marks as format "convrot_w4a4" (nodes.py:419-444)."""
    raw = (metadata or {}).get("_quantization_metadata")
    if not raw:
        return {}
    out = {}
    for key, cfg in json.loads(raw).get("layers", {}).items():
        if cfg.get("format") == "convrot_w4a4":
            out[key[len(prefix):] if prefix and key.startswith(prefix) else key] = cfg
    return out


def quantize_state_dict(sd: dict, device, metadata: dict | None = None, prefix: str = "",
                        block_size: int = BLOCK, convrot_decoder=None):
    """The load-time quantizer of Gfx906Int4UnetLoader (nodes.py:508-573): every 2-D `<base>.weight`
    whose last dim is a multiple of block_size becomes `<base>.weight_q4` / `<base>.weight_scale`
    (quantized on `device`, stored on the CPU); ConvRot W4A4 layers (named by the metadata, or any
    int8 2-D weight with an fp32 per-row `.weight_scale` sidecar once the file has ConvRot layers)
    are decoded by `convrot_decoder` (comfy_kitchen's dequantize_convrot_w4a4_weight when None)
    first; every other tensor passes through. Returns (quantized state dict, counts).
    The reference quantizes a plain float weight where the state dict holds it (the CPU, after
    load_torch_file: torch's `amax / 7.0` there is a true division) and a decoded ConvRot weight on
    `device` (torch's GPU rule, amax * fl(1/7)); the same rules are used here, whichever device
    computes, so the packed weights equal the reference's bit for bit."""
    device = torch.device(device)
    layers = parse_convrot_layers(metadata, prefix)
    shared_cfg = next(iter(layers.values()), None)
    convrot = {}
    for key, t in sd.items():
        if not key.endswith(".weight"):
            continue
        base = key[:-len(".weight")]
        cfg = layers.get(base)
        side = sd.get(base + ".weight_scale")
        if cfg is None and shared_cfg is not None and t.dtype == torch.int8 and t.ndim == 2 and side is not None \
                and side.dtype == torch.float32 and tuple(side.shape) == (t.shape[0],):
            cfg = shared_cfg
        if cfg is not None:
            convrot[base] = cfg
    sidecars = {b + ".weight_scale" for b in convrot}
    out, counts = {}, {"quantized": 0, "convrot_repacked": 0, "passthrough": 0}
    for key, t in sd.items():
        if key in sidecars:
            continue
        base = key[:-len(".weight")] if key.endswith(".weight") else None
        rule = None  # the rule of the device the weight is quantized on
        if base is not None and base in convrot:
            if convrot_decoder is None:
                try:
                    from comfy_kitchen.tensor.convrot_w4a4 import dequantize_convrot_w4a4_weight as convrot_decoder
                except ImportError:
                    raise RuntimeError(f"{key} is ConvRot-quantized but comfy_kitchen is not available to decode it")
            cfg = convrot[base]
            w = convrot_decoder(t.to(device), sd[base + ".weight_scale"].to(device),
                                convrot_groupsize=cfg["convrot_groupsize"], quant_group_size=cfg["quant_group_size"],
                                output_dtype=torch.float32)
            src = RawWeight(w, w.shape[0], w.shape[1])
            counts["convrot_repacked"] += 1
        elif base is not None and t.ndim == 2 and t.shape[1] % block_size == 0 and t.shape[1] >= block_size:
            plain = getattr(t, "tensor_type", None) is None and t.is_floating_point()
            src = RawWeight(t.to(device) if plain else t, t.shape[0], t.shape[1])
            if plain:  # computed on `device`, with the rule of the device the tensor was loaded on
                rule = _lib.RULE_RECIP if t.device.type == "cuda" else _lib.RULE_DIV
            counts["quantized"] += 1
        else:
            out[key] = t
            counts["passthrough"] += 1
            continue
        packed, scale, _ = quantize_module_weight(src, block_size, rule=rule)
        out[base + ".weight_q4"] = packed.cpu()
        out[base + ".weight_scale"] = scale.cpu()
    return out, counts


def _device_list():
    return ["cpu"] + [f"cuda:{i}" for i in range(torch.cuda.device_count())]


def _default_device(devices):
    """The second GPU when there are several (the first usually drives the desktop), else the
    only one, else cpu (nodes.py:405-411)."""
    gpus = [d for d in devices if d != "cpu"]
    return gpus[1] if len(gpus) > 1 else (gpus[0] if gpus else "cpu")


# ---------------------------------------------------------------------------------------------
# nodes
# ---------------------------------------------------------------------------------------------
class Gfx906Int4Patch:
    """MODEL -> MODEL: rounds the diffusion model's Linear weights through int4 in place (and,
    in w4a4_naive mode, each such layer's input activation) for accuracy tests with the stock
    matmul; no kernel involved (nodes.py:71-124)."""

    @classmethod
    def INPUT_TYPES(cls):
        return {"required": {"model": ("MODEL",),
                             "mode": (["w4a16", "w4a4_naive"], {"default": "w4a16"}),
                             "spare_first_last_layers": ("BOOLEAN", {"default": True}),
                             "block_size": ("INT", {"default": 32, "min": 16, "max": 256, "step": 16})}}

    RETURN_TYPES = ("MODEL",)
    FUNCTION = "patch"
    CATEGORY = CATEGORY
    TITLE = "Gfx906 Int4 Quantize (test)"

    def patch(self, model, mode, spare_first_last_layers, block_size):
        model = model.clone()
        root = model.model.diffusion_model
        spared = ()
        if spare_first_last_layers:
            last = find_max_layer_index(root)
            spared = SPARED_PREFIXES + (("layers.0.", f"layers.{last}.") if last >= 0 else ())
        modules = dict(root.named_modules())
        n_q = n_spared = n_hooks = 0
        with torch.no_grad():
            for name, p in root.named_parameters():
                if not name.endswith(".weight") or p.ndim != 2 or p.shape[1] < block_size or p.shape[1] % block_size:
                    continue
                owner = name[:-len(".weight")]
                if owner.startswith(spared):
                    n_spared += 1
                    continue
                p.data.copy_(quantize_dequantize_int4(p.data.float(), block_size).to(p.dtype))
                n_q += 1
                if mode == "w4a4_naive" and owner in modules:
                    modules[owner].register_forward_pre_hook(_activation_round_trip_hook)
                    n_hooks += 1
        print(f"[Gfx906Int4Patch] mode={mode} quantized={n_q} spared={n_spared} activation_hooks={n_hooks}")
        return (model,)


class Gfx906Int4Transcode:
    """MODEL -> MODEL: every eligible Linear of the loaded diffusion model becomes an int4 engine
    Linear, whatever format it arrived in (nodes.py:290-323)."""

    @classmethod
    def INPUT_TYPES(cls):
        return {"required": {"model": ("MODEL",),
                             "activation_rotation": ("BOOLEAN", {"default": False, "tooltip": _ROTATION_TOOLTIP})}}

    RETURN_TYPES = ("MODEL",)
    FUNCTION = "transcode"
    CATEGORY = CATEGORY
    TITLE = "Gfx906 Int4 Transcode (native kernel, any source)"

    def transcode(self, model, activation_rotation):
        model = model.clone()
        c, s, src = transcode_linears(model.model.diffusion_model, BLOCK, activation_rotation)
        print(f"[Gfx906Int4Transcode] converted={c} skipped={s} sources={src}")
        return (model,)


class Gfx906Int4TranscodeCLIP:
    """CLIP -> CLIP: the same transcode on a loaded text encoder (nodes.py:326-350)."""

    @classmethod
    def INPUT_TYPES(cls):
        return {"required": {"clip": ("CLIP",),
                             "activation_rotation": ("BOOLEAN", {"default": False, "tooltip": _ROTATION_TOOLTIP})}}

    RETURN_TYPES = ("CLIP",)
    FUNCTION = "transcode"
    CATEGORY = CATEGORY
    TITLE = "Gfx906 Int4 Transcode CLIP (native kernel, any source)"

    def transcode(self, clip, activation_rotation):
        clip = clip.clone()
        c, s, src = transcode_linears(clip.cond_stage_model, BLOCK, activation_rotation)
        print(f"[Gfx906Int4TranscodeCLIP] converted={c} skipped={s} sources={src}")
        return (clip,)


class Gfx906Int4CLIPLoader:
    """Loads a float safetensors text encoder with each Linear quantized on the target GPU while
    the state dict loads (make_load_quantizing_ops), so the float encoder never sits in device
    memory (nodes.py:353-398)."""

    @classmethod
    def INPUT_TYPES(cls):
        import folder_paths  # type: ignore
        import nodes as comfy_nodes  # type: ignore
        devices = [d for d in _device_list() if d != "cpu"]
        return {"required": {
            "clip_name": (folder_paths.get_filename_list("text_encoders"),),
            "type": (comfy_nodes.CLIPLoader.INPUT_TYPES()["required"]["type"][0], {"default": "krea2"}),
            "device": (devices, {"default": _default_device(devices)}),
            "activation_rotation": ("BOOLEAN", {"default": True, "tooltip": _ROTATION_TOOLTIP})}}

    RETURN_TYPES = ("CLIP",)
    FUNCTION = "load_clip"
    CATEGORY = CATEGORY
    TITLE = "Gfx906 Int4 CLIP Loader (native kernel)"

    def load_clip(self, clip_name, type, device, activation_rotation):
        import comfy.ops  # type: ignore
        import comfy.sd  # type: ignore
        import folder_paths  # type: ignore
        path = folder_paths.get_full_path_or_raise("text_encoders", clip_name)
        if path.endswith(".gguf"):
            raise ValueError(f"Gfx906 Int4 CLIP Loader: expected a safetensors text encoder, got {clip_name}; load "
                             ".gguf files with the GGUF CLIP loader followed by Gfx906 Int4 Transcode CLIP")
        dev = torch.device(device)
        ops = make_load_quantizing_ops(comfy.ops.manual_cast, dev, activation_rotation)
        clip = comfy.sd.load_clip(ckpt_paths=[path], embedding_directory=folder_paths.get_folder_paths("embeddings"),
                                  clip_type=getattr(comfy.sd.CLIPType, type.upper()),
                                  model_options={"custom_operations": ops, "load_device": dev})
        eligible = sum(isinstance(m, ops.Linear) and m.quantized for m in clip.cond_stage_model.modules())
        if ops.Linear.quantized_on_load != eligible:
            raise RuntimeError(f"Gfx906 Int4 CLIP Loader: expected all {eligible} int4 Linears quantized from float "
                               f"weights, got {ops.Linear.quantized_on_load} (pre-quantized or missing weights?)")
        torch.cuda.empty_cache()
        print(f"[Gfx906Int4CLIPLoader] quantized={eligible} rotation={activation_rotation} device={device}")
        return (clip,)


class Gfx906Int4UnetLoader:
    """Loads a diffusion model (float safetensors, .gguf through ComfyUI-GGUF's reader, or a
    ConvRot W4A4 checkpoint) with its Linear weights quantized at load time into the packed
    layout, then builds the model with Gfx906Int4Ops as custom_operations (nodes.py:447-599)."""

    @classmethod
    def INPUT_TYPES(cls):
        import folder_paths  # type: ignore
        names = list(folder_paths.get_filename_list("diffusion_models"))
        if "unet_gguf" in folder_paths.folder_names_and_paths:
            names += [n for n in folder_paths.get_filename_list("unet_gguf") if n not in names]
        devices = _device_list()
        return {"required": {"unet_name": (names,), "device": (devices, {"default": _default_device(devices)})}}

    RETURN_TYPES = ("MODEL",)
    FUNCTION = "load_unet"
    CATEGORY = CATEGORY
    TITLE = "Gfx906 Int4 UNet Loader (native kernel)"

    def load_unet(self, unet_name, device):
        import comfy.model_detection  # type: ignore
        import comfy.model_management as mm  # type: ignore
        import comfy.model_patcher  # type: ignore
        import comfy.storage  # type: ignore
        import comfy.utils  # type: ignore
        import folder_paths  # type: ignore
        path = folder_paths.get_full_path_or_raise("diffusion_models", unet_name)
        dev = torch.device(device)
        metadata, prefix = None, ""
        if path.endswith(".gguf"):
            loader = _gguf_module("loader")
            if loader is None:
                raise RuntimeError("Loading a .gguf model requires ComfyUI-GGUF to be loaded (for gguf_sd_loader)")
            sd, _ = loader.gguf_sd_loader(path)
        else:
            sd, metadata = comfy.utils.load_torch_file(path, return_metadata=True)
            prefix = comfy.model_detection.unet_prefix_from_state_dict(sd)
            stripped = comfy.utils.state_dict_prefix_replace(sd, {prefix: ""}, filter_keys=True)
            if stripped:
                sd = stripped
        qsd, counts = quantize_state_dict(sd, dev, metadata, prefix)
        print(f"[Gfx906Int4UnetLoader] quantized={counts['quantized']} convrot_repacked={counts['convrot_repacked']} "
              f"passthrough_tensors={counts['passthrough']} device={device}")
        # architecture detection reads the float ".weight" shapes, so it gets the original dict
        cfg = comfy.model_detection.model_config_from_unet(sd, "", metadata=metadata)
        if cfg is None:
            raise RuntimeError(f"Could not detect model type of: {path}")
        params = comfy.utils.calculate_parameters(sd)
        unet_dtype = mm.unet_dtype(model_params=params, supported_dtypes=list(cfg.supported_inference_dtypes),
                                   weight_dtype=comfy.utils.weight_dtype(sd))
        cfg.set_inference_dtype(unet_dtype, mm.unet_manual_cast(unet_dtype, dev, cfg.supported_inference_dtypes),
                                device=dev)
        cfg.custom_operations = Gfx906Int4Ops
        model = cfg.get_model(qsd, "")
        offload = mm.unet_offload_device()
        patcher = comfy.model_patcher.ModelPatcher(model, load_device=dev, offload_device=offload,
                                                   fast_disk=comfy.storage.state_dict_fast_disk(qsd))
        if not mm.is_device_cpu(offload):
            model.to(offload)
        model.load_model_weights(qsd, "")
        return (patcher,)


NODE_CLASS_MAPPINGS = {
    "Gfx906Int4Patch": Gfx906Int4Patch,
    "Gfx906Int4UnetLoader": Gfx906Int4UnetLoader,
    "Gfx906Int4Transcode": Gfx906Int4Transcode,
    "Gfx906Int4TranscodeCLIP": Gfx906Int4TranscodeCLIP,
    "Gfx906Int4CLIPLoader": Gfx906Int4CLIPLoader,
}

NODE_DISPLAY_NAME_MAPPINGS = {k: v.TITLE for k, v in NODE_CLASS_MAPPINGS.items()}
