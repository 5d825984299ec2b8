"""The reference's INT2 export format for hip models.

Mirrors ``tesm_ssm/utils/int2_quantization.py`` (WANGLILIN360/tesm):

* ``export_model_to_int2(model)`` (:196-217) -- one entry per BitLinear:
  ``{'packed_weight': uint8 (out, ceil(in/4)), 'weight_scale': 0-d tensor,
  'bias': tensor or None, 'in_features', 'out_features'}``, tensors on the CPU.
  The scale is ``1 / mean|w|.clamp_min(1e-8)`` in the weight's dtype and the
  codes ``round(w * scale).clamp(-1, 1)`` (:32-36), computed and packed on the
  device; an INT2-backed layer exports the entry it was loaded from.
* ``load_int2_weights_to_model(model, exported)`` (:220-245) -- installs each
  entry into the BitLinear of the same name.  The reference replaces the layer
  with an ``Int2Linear`` whose forward multiplies the unquantized input by the
  dequantized weight (:158-174); here the layer stays a BitLinear and keeps its
  forward (int8 activations x ternary codes), now with the loaded codes and
  scale, so that a loaded model computes what the exported BitLinear model
  computes.  No float weight is read.
* ``save_int2_model`` / ``load_int2_model`` (:248-279) -- the dict through
  ``torch.save`` / ``torch.load(weights_only=True)``.

The canonical byte layout (code = q + 1, four 2-bit fields per byte, low bits
first, pad code 1) is the reference's (:10-13, :38-58); the device caches rows
padded to the products' 128-code K tile.
"""
from __future__ import annotations

from typing import Dict, List

import torch
import torch.nn as nn

from . import hip_ops
from .bitlinear import BitLinear

EXPORT_EPS = 1e-8  # int2_quantization.py:32


def quantize_weight_to_int2(weight: torch.Tensor):
    """(packed uint8 (N, ceil(K/4)), scale 0-d tensor of the weight's dtype) on the weight's device
    (int2_quantization.py:96-107)."""
    w = weight.detach()
    if w.dim() != 2:
        raise ValueError(f"expected a 2-D weight, got shape {tuple(w.shape)}")
    hip_ops.require_device(w)
    s_w, _ = hip_ops.absmean_scale(w, EXPORT_EPS)
    packed = hip_ops.pack_weight(w, s_w, ldp=(w.shape[1] + 3) // 4)
    return packed, s_w.reshape(()).to(w.dtype)


def export_model_to_int2(model: nn.Module) -> Dict[str, Dict]:
    """Every BitLinear of ``model`` as an INT2 entry (int2_quantization.py:196-217)."""
    exported = {}
    for name, module in model.named_modules():
        if not isinstance(module, BitLinear):
            continue
        if module.is_int2:
            packed = module.int2_packed.cpu().clone()
            scale = torch.tensor(module.int2_scale, dtype=torch.float32).to(module.weight.dtype)
        else:
            with torch.no_grad():
                packed, scale = quantize_weight_to_int2(module.weight)
            packed, scale = packed.cpu(), scale.cpu()
        exported[name] = {
            "packed_weight": packed,
            "weight_scale": scale,
            "bias": module.bias.data.cpu() if module.bias is not None else None,
            "in_features": module.in_features,
            "out_features": module.out_features,
        }
    return exported


def load_int2_weights_to_model(model: nn.Module, exported: Dict[str, Dict],
                               keep_float_weights: bool = True) -> List[str]:
    """Install the entries of ``exported`` into the BitLinear layers of the same name
    (int2_quantization.py:220-245); names that are not BitLinear layers of ``model`` are skipped,
    as in the reference.  Returns the names loaded.  ``keep_float_weights=False`` releases the
    float weights of the loaded layers."""
    loaded = []
    for name, module in model.named_modules():
        if name in exported and isinstance(module, BitLinear):
            e = exported[name]
            module.load_int2(e["packed_weight"], e["weight_scale"], bias=e.get("bias"),
                             in_features=e.get("in_features"), out_features=e.get("out_features"),
                             keep_float_weight=keep_float_weights)
            loaded.append(name)
    return loaded


def save_int2_model(model: nn.Module, path: str) -> Dict[str, Dict]:
    """``torch.save`` of ``export_model_to_int2(model)`` (int2_quantization.py:248-266)."""
    exported = export_model_to_int2(model)
    torch.save(exported, path)
    total = sum(e["packed_weight"].numel() for e in exported.values())
    print(f"INT2 model saved to {path}")
    print(f"packed weight size: {total / (1024 * 1024):.2f} MB (INT2)")
    return exported


def load_int2_model(model: nn.Module, path: str, keep_float_weights: bool = True) -> List[str]:
    """Load a saved export into ``model`` (int2_quantization.py:269-279), with the loader that
    executes nothing from the file."""
    exported = torch.load(path, map_location="cpu", weights_only=True)
    loaded = load_int2_weights_to_model(model, exported, keep_float_weights=keep_float_weights)
    print(f"INT2 model loaded from {path}")
    return loaded
