"""Restatement of the reference's INT2 export format -- TEST INFRASTRUCTURE ONLY.

The checker for ``tesm_amd.int2``: what ``export_model_to_int2`` writes for each
BitLinear (WANGLILIN360/tesm, tesm_ssm/utils/int2_quantization.py:196-217) and
what a BitLinear whose weight quantizes to those codes computes.

* ``pack_int2_to_uint8`` (int2_quantization.py:21-58): scale =
  ``1 / mean|w|.clamp_min(1e-8)`` in the weight's dtype (torch evaluates
  ``1.0 / t`` as ``t.reciprocal() * 1.0``), codes ``round(w * scale).clamp(-1, 1)``,
  packed by ``oracle.int_ref.pack_i2`` (code + 1, four 2-bit fields per byte,
  low bits first, pad code 1).
* ``unpack_uint8_to_int2`` (int2_quantization.py:61-93): field - 1, divided by
  the scale in float32.
* ``export_model_to_int2`` (int2_quantization.py:196-217): one entry per
  BitLinear of an ``oracle.tesm_torch`` model, tensors on the CPU.

Pinned by tests/test_oracle_int2.py: the reference's own known answer
``[-1, 0, +1, 0] -> 0x64`` (int2_quantization.py:12-13), a hand-computed scale
and byte, the shape assertion of the reference's test (16 x 64 -> 16 x 16,
tests/test_torch_only.py:398-403), unpack(pack) = codes, and agreement of the
export codes with the codes of ``BitLinear.quantized_weight`` (tesm.py:211-215)
wherever ``mean|w| >= bit_eps``.
"""
from __future__ import annotations

from typing import Dict, Tuple

import numpy as np
import torch
import torch.nn as nn

from . import int_ref


def export_scale(w: torch.Tensor) -> torch.Tensor:
    """``1.0 / w.abs().mean().clamp_min(1e-8)`` (int2_quantization.py:32), a 0-d tensor of w's dtype."""
    return 1.0 / w.detach().abs().mean().clamp_min(1e-8)


def export_codes(w: torch.Tensor, scale: torch.Tensor) -> np.ndarray:
    """``(w * scale).round().clamp(-1, 1)`` as int8 (int2_quantization.py:35-36)."""
    return (w.detach() * scale).round().clamp(-1, 1).to(torch.int8).cpu().numpy()


def pack_int2_to_uint8(w: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """(packed uint8 (N, ceil(K/4)), scale) of a 2-D weight (int2_quantization.py:21-58)."""
    scale = export_scale(w)
    packed = int_ref.pack_i2(export_codes(w, scale))
    return torch.from_numpy(packed), scale.detach().clone()


def unpack_uint8_to_int2(packed: torch.Tensor, scale: float) -> torch.Tensor:
    """Dequantized float32 weight (N, 4 * packed.shape[1]) (int2_quantization.py:61-93)."""
    p = packed.cpu().numpy()
    codes = int_ref.unpack_i2(p, 4 * p.shape[1])
    return torch.from_numpy(codes).float() / scale


def export_model_to_int2(model: nn.Module) -> Dict[str, Dict]:
    """{module name: {'packed_weight', 'weight_scale', 'bias', 'in_features', 'out_features'}}
    for every ``oracle.tesm_torch.BitLinear`` in ``model`` (int2_quantization.py:196-217)."""
    from .tesm_torch import BitLinear

    exported = {}
    for name, module in model.named_modules():
        if isinstance(module, BitLinear):
            packed, scale = pack_int2_to_uint8(module.weight.data)
            exported[name] = {
                "packed_weight": packed.cpu(),
                "weight_scale": scale.cpu(),
                "bias": module.bias.data.cpu() if module.bias is not None else None,
                "in_features": module.in_features,
                "out_features": module.out_features,
            }
    return exported
