"""Quantised-checkpoint loading for the VGGT aggregator and camera head.

The host-side half of "loads the same quantised checkpoints unchanged": the
selection logic of the reference loader (qvggt/inference/loader.py), applied
to ``qvggt_amd.aggregator.Aggregator``, whose module tree uses the same names
as the checkpoint (``aggregator.frame_blocks.{i}.attn.qkv.qweight`` ...).

* ``checkpoint_is_self_contained``   loader.py:164-176
* ``infer_quantization_layout``      loader.py:178-222
* ``extract_cict_token``             loader.py:224-232
* ``should_quantize_layer``          loader.py:320-362
* ``quantize_specified_blocks``      loader.py:364-400 (nn.Linear -> WQLinear(init_only))
* ``merge_state_dicts``              loader.py:466-548
* ``load_model_config``              loader.py:146-162 (config.json, read as JSON)
* ``load_quantized_aggregator``      loader.py:550-600 for the aggregator part
* ``load_quantized_camera_head``     the same for ``camera_head.*`` (W4 trunk)

Files are read with loaders that execute nothing from the file: safetensors,
or ``torch.load(..., weights_only=True)`` (the reference unpickles).
"""
from __future__ import annotations

from collections import OrderedDict
from pathlib import Path

import torch
import torch.nn as nn

from .awq.qmodule import WQLinear

AUX_KEYS = ("cict_token", "cict_topk", "unquantized_patch_start_idx")
LAYER_TYPES = ("qkv", "proj", "fc1", "fc2")
PREFIX = "aggregator."


def _block_index(key: str, kind: str) -> int:
    return int(key.split(f".{kind}.", 1)[1].split(".", 1)[0])


def checkpoint_is_self_contained(state_dict) -> bool:
    """True when the checkpoint carries the unquantised weights too (loader.py:164-176)."""
    required = ("aggregator.patch_embed.patch_embed.proj.weight", "aggregator.camera_token",
                "camera_head.pose_branch.fc1.weight")
    return all(k in state_dict for k in required)


def infer_quantization_layout(state_dict) -> dict:
    """Which frame / global blocks, layer types and camera-head trunk the
    checkpoint quantises, read off its ``.qweight`` keys (loader.py:178-222)."""
    frame, glob, types = set(), set(), set()
    camera = False
    for key in state_dict.keys():
        if not key.endswith(".qweight"):
            continue
        if ".frame_blocks." in key:
            frame.add(_block_index(key, "frame_blocks"))
        elif ".global_blocks." in key:
            glob.add(_block_index(key, "global_blocks"))
        elif "camera_head.trunk." in key:
            camera = True
        for t in LAYER_TYPES:
            if f".{t}." in key:
                types.add(t)
    return {"frame_blocks": sorted(frame) or None, "global_blocks": sorted(glob) or None,
            "quantize_camera_head": camera, "layer_types": sorted(types) or None}


def extract_cict_token(state_dict):
    """The camera head's CICT token, if the checkpoint carries one (loader.py:224-232)."""
    for key in ("camera_head.cict_token", "model.camera_head.cict_token", "cict_token"):
        if key in state_dict and torch.is_tensor(state_dict[key]):
            return state_dict[key].detach().cpu().view(-1)
    return None


def _layer_type(name: str) -> str:
    for t in LAYER_TYPES:
        if f".{t}" in name:
            return t
    return "unknown"


def should_quantize_layer(name: str, quantize_type: str, frame_blocks, global_blocks, layer_types,
                          quantize_camera_head: bool) -> bool:
    """Whether the linear called ``name`` (full model path) is a W4 layer
    (loader.py:320-362): camera-head trunk linears when that is quantised,
    otherwise only aggregator frame/global block linears of the selected types
    and blocks; the DINOv2 patch embed always stays in floating point."""
    if quantize_camera_head and "camera_head" in name:
        return "trunk." in name and not any(
            n in name for n in ("norm", "bn", "ln", "layernorm", "batchnorm", "groupnorm"))
    if not name.startswith(PREFIX) or "patch_embed" in name:
        return False
    if layer_types is not None and _layer_type(name) not in layer_types:
        return False
    for kind, blocks in ((".frame_blocks.", frame_blocks), (".global_blocks.", global_blocks)):
        if kind in name:
            idx = _block_index(name, kind.strip("."))
            if quantize_type == "all":
                return True
            if quantize_type == "specific_blocks":
                return blocks is not None and idx in blocks
            return False
    return False


def quantize_specified_blocks(model: nn.Module, w_bit: int = 4, group_size: int = 128,
                              quantize_type: str = "specific_blocks", frame_blocks=None, global_blocks=None,
                              layer_types=None, quantize_camera_head: bool = False, prefix: str = PREFIX):
    """Replace the selected ``nn.Linear`` modules by empty ``WQLinear`` buffers
    (``from_linear(init_only=True)``, loader.py:364-400); returns their names.
    ``prefix`` is the model's own path in the checkpoint (the aggregator is
    ``aggregator.`` inside VGGT)."""
    replaced = []
    for name, mod in list(model.named_modules()):
        if not isinstance(mod, nn.Linear):
            continue
        full = prefix + name
        if not should_quantize_layer(full, quantize_type, frame_blocks, global_blocks, layer_types,
                                     quantize_camera_head):
            continue
        *parents, attr = name.split(".")
        parent = model
        for p in parents:
            parent = getattr(parent, p)
        setattr(parent, attr, WQLinear.from_linear(mod, w_bit, group_size, init_only=True))
        replaced.append(full)
    return replaced


def merge_state_dicts(quantized_sd, original_sd=None, quantize_type: str = "specific_blocks",
                      frame_blocks=None, global_blocks=None, quantized_layer_types=None,
                      quantize_camera_head: bool = False):
    """Overlay the quantised entries of the selected blocks on the original
    weights and drop each replaced ``.weight`` (loader.py:466-548).  Returns
    (merged state dict, CICT token or None)."""
    q = OrderedDict(quantized_sd)
    cict = extract_cict_token(q)
    for k in AUX_KEYS:
        q.pop(k, None)
    if checkpoint_is_self_contained(q):
        merged = OrderedDict(q)
    else:
        if original_sd is None:
            raise ValueError("Checkpoint is not self-contained. Please provide an original FP16 model "
                             "checkpoint via model_path.")
        merged = OrderedDict(original_sd)

    def selected(key):
        if quantize_camera_head and "camera_head" in key:
            return True
        for kind, blocks in ((".frame_blocks.", frame_blocks), (".global_blocks.", global_blocks)):
            if kind in key:
                idx = _block_index(key, kind.strip("."))
                return quantize_type == "all" or (quantize_type == "specific_blocks" and blocks is not None
                                                  and idx in blocks)
        return False

    drop = set()
    for key, value in q.items():
        if not selected(key):
            continue
        t = _layer_type(key)
        if t == "unknown" and "camera_head" in key:
            t = "linear"
        if quantized_layer_types is not None and t not in quantized_layer_types:
            continue
        merged[key] = value
        for suffix in (".qweight", ".scales", ".scaled_zeros"):
            if key.endswith(suffix):
                orig = key[: -len(suffix)] + ".weight"
                if orig in merged and orig != key:
                    drop.add(orig)
    for key in drop:
        merged.pop(key, None)
    return merged, cict


def read_state_dict(path) -> dict:
    """Tensors of a ``.safetensors`` file, or of a torch checkpoint read with
    ``weights_only=True`` (a file that needs unpickling is refused)."""
    path = Path(path)
    if path.suffix == ".safetensors":
        from safetensors.torch import load_file
        return load_file(str(path), device="cpu")
    sd = torch.load(str(path), map_location="cpu", weights_only=True)
    if not isinstance(sd, dict):
        raise ValueError(f"{path}: expected a state dict, got {type(sd).__name__}")
    return sd


def aggregator_state_dict(sd, prefix: str = PREFIX) -> OrderedDict:
    """The ``aggregator.*`` (or other ``prefix``) entries of a VGGT state dict, prefix stripped."""
    return OrderedDict((k[len(prefix):], v) for k, v in sd.items() if k.startswith(prefix))


def _copy_into(model: nn.Module, sd, strict: bool, what: str):
    """Copy a prefix-stripped state dict into ``model``; returns (missing, unused)."""
    own = model.state_dict()
    missing = [k for k in own if k not in sd and not k.startswith("img_")]
    unused = [k for k in sd if k not in own]
    if strict and missing:
        raise KeyError(f"checkpoint lacks {len(missing)} {what} tensors, e.g. {missing[:4]}")
    for k, v in sd.items():
        if k in own:
            if own[k].shape != v.shape:
                raise ValueError(f"{k}: checkpoint shape {tuple(v.shape)} != model {tuple(own[k].shape)}")
            own[k].copy_(v.to(own[k].dtype) if not k.endswith(".qweight") else v)
    return missing, unused


def _merged(quantized_path, model_path, quantize_type, frame_blocks, global_blocks, layer_types,
            quantize_camera_head):
    qsd = read_state_dict(quantized_path)
    if checkpoint_is_self_contained(qsd):
        lay = infer_quantization_layout(qsd)
        frame_blocks, global_blocks, layer_types = lay["frame_blocks"], lay["global_blocks"], lay["layer_types"]
        quantize_camera_head = lay["quantize_camera_head"]
    osd = read_state_dict(model_path) if model_path is not None else None
    merged, cict = merge_state_dicts(qsd, osd, quantize_type, frame_blocks, global_blocks, layer_types,
                                     quantize_camera_head)
    return merged, cict, frame_blocks, global_blocks, layer_types, quantize_camera_head


def load_model_config(quantized_path, model_path=None):
    """The aggregator's model config (``AggregatorConfig``), found as the
    reference finds its ``VGGTConfig`` (loader.py:146-162): the ``config.json``
    in the directory of the original fp16 model when one is given; otherwise,
    unlike the reference (which then takes the config class defaults), a
    ``config.json`` beside the quantised checkpoint; otherwise the defaults.
    The file is read as JSON only."""
    from .aggregator import AggregatorConfig

    for p in (model_path, quantized_path):
        if p is None:
            continue
        d = Path(p)
        if ((d if d.is_dir() else d.parent) / "config.json").exists():
            return AggregatorConfig.from_pretrained(p)
        if p is model_path:
            break
    return AggregatorConfig()


@torch.no_grad()
def load_quantized_aggregator(quantized_path, model_path=None, device="cuda", depth: int | None = None,
                              w_bit: int = 4, group_size: int = 128, quantize_type: str = "specific_blocks",
                              frame_blocks=None, global_blocks=None, layer_types=None, strict: bool = True,
                              config=None):
    """Build the aggregator for a QVGGT quantised checkpoint: fp16 model,
    selected linears swapped for ``WQLinear``, merged weights loaded.

    The model parameters (LayerNorm eps, depth, RoPE base) come from
    ``config`` or, when that is None, from ``load_model_config``; ``depth``
    overrides the config's depths.  For a self-contained checkpoint the layout
    (blocks, layer types) is inferred from its ``.qweight`` keys, as
    loader.py:600-612 does.  Returns (aggregator, report) with the replaced
    layer names, the checkpoint keys the aggregator does not use (``strict``
    raises on missing ones) and the config used."""
    from .aggregator import Aggregator

    cfg = config if config is not None else load_model_config(quantized_path, model_path)
    merged, cict, frame_blocks, global_blocks, layer_types, _ = _merged(
        quantized_path, model_path, quantize_type, frame_blocks, global_blocks, layer_types, False)
    agg = Aggregator.empty(device=device, depth=depth, config=cfg)
    replaced = quantize_specified_blocks(agg, w_bit, group_size, quantize_type, frame_blocks, global_blocks,
                                         layer_types)
    missing, unused = _copy_into(agg, aggregator_state_dict(merged), strict, "aggregator")
    return agg, {"replaced": replaced, "unused": unused, "missing": missing, "cict_token": cict,
                 "config": agg.config}


@torch.no_grad()
def load_quantized_camera_head(quantized_path, model_path=None, device="cuda", w_bit: int = 4,
                               group_size: int = 128, quantize_camera_head: bool = True, strict: bool = True):
    """Build the VGGT camera head for a QVGGT checkpoint: fp16 head, trunk
    linears swapped for ``WQLinear`` when the checkpoint quantises them
    (``camera_head.trunk.*.qweight``, loader.py:204-206, 338-344), merged
    ``camera_head.*`` weights loaded.  Returns (head, report) like
    ``load_quantized_aggregator``; ``report["cict_token"]`` carries the CICT
    token if the checkpoint has one (the head does not use it)."""
    from .camera_head import CameraHead

    merged, cict, _, _, _, quantize_camera_head = _merged(
        quantized_path, model_path, "specific_blocks", None, None, None, quantize_camera_head)
    head = CameraHead.empty(device=device)
    replaced = (quantize_specified_blocks(head, w_bit, group_size, quantize_camera_head=True,
                                          prefix="camera_head.") if quantize_camera_head else [])
    missing, unused = _copy_into(head, aggregator_state_dict(merged, "camera_head."), strict, "camera head")
    return head, {"replaced": replaced, "unused": unused, "missing": missing, "cict_token": cict}
