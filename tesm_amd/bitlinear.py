"""BitLinear with ``kernel_backend='hip'``.

Same constructor, parameters and initialisation as the reference's BitLinear
(tesm_ssm/modules/tesm.py:124-204), so checkpoints and seeded construction carry
over.  The forward pass is eval-only (no autograd), like the reference's
``cuda`` eval path: it quantizes activations per token to int8, multiplies
against the ternary weights packed four per byte, and scales the exact int32
accumulators once (tesm.py:206-215, 238-290).

The packed weight, its scale and the dequantized +1 value are cached per
``weight._version`` like the reference's eval cache (tesm.py:226-236).
"""
from __future__ import annotations

import math

import torch
import torch.nn as nn

from . import hip_ops

HIP_BACKENDS = ("hip", "auto")


def backend_error(backend: str, what: str, detail: str = "") -> RuntimeError:
    """The reference's strict-backend error shape (tesm.py:278-285)."""
    msg = (f"kernel_backend='{backend}' specified but {what} kernel not available. "
           f"Available backends: hip=True (eval mode, torch.no_grad(), tensors on a ROCm device). "
           f"Use kernel_backend='hip' or 'auto'.")
    if detail:
        msg += f" ({detail})"
    return RuntimeError(msg)


def check_hip_call(backend: str, what: str, module: nn.Module, x: torch.Tensor) -> None:
    if backend not in HIP_BACKENDS:
        raise backend_error(backend, what, "this package implements only the hip backend")
    if module.training or torch.is_grad_enabled():
        raise backend_error(backend, what, "the hip kernels are forward-only: call module.eval() under torch.no_grad()")
    if not x.is_cuda:
        raise backend_error(backend, what, f"input is on {x.device}")


class PackedWeight:
    """Device-resident INT2 weight: packed codes (N, kpad(K)/4), s_w and c_w scalars."""

    def __init__(self, packed, s_w, c_w, N, K):
        self.packed, self.s_w, self.c_w, self.N, self.K = packed, s_w, c_w, N, K


class BitLinear(nn.Module):
    def __init__(self, in_features, out_features, bias=False, bit_eps=1e-5, bit_threshold=0.5, kernel_backend="hip",
                 kernel_mode="fast", device=None, dtype=None):
        super().__init__()
        factory_kwargs = {"device": device, "dtype": dtype}
        self.in_features = in_features
        self.out_features = out_features
        self.bit_eps = bit_eps
        self.bit_threshold = bit_threshold
        self.kernel_backend = str(kernel_backend)
        self.kernel_mode = "precise" if str(kernel_mode) == "precise" else "fast"
        self.weight = nn.Parameter(torch.empty(out_features, in_features, **factory_kwargs))
        if bias:
            self.bias = nn.Parameter(torch.zeros(out_features, **factory_kwargs))
        else:
            self.bias = None
        self._packed = None
        self._packed_key = None
        self.reset_parameters()

    def reset_parameters(self):  # tesm.py:200-204
        nn.init.kaiming_uniform_(self.weight, a=math.sqrt(5))
        if self.bias is not None:
            bound = 1 / math.sqrt(self.in_features)
            nn.init.uniform_(self.bias, -bound, bound)

    # -- packed weight cache ---------------------------------------------------
    def packed_weight(self) -> PackedWeight:
        """Pack the ternary weight once per weight version (tesm.py:226-236)."""
        w = self.weight
        key = (w._version, w.data_ptr(), w.dtype, w.device)
        if self._packed is None or self._packed_key != key:
            with torch.no_grad():
                s_w, c_w = hip_ops.absmean_scale(w.detach(), self.bit_eps)
                packed = hip_ops.pack_weight(w.detach(), s_w)
            self._packed = PackedWeight(packed, s_w, c_w, self.out_features, self.in_features)
            self._packed_key = key
        return self._packed

    def linear_desc(self):
        """The ``tesm_hip_linear`` descriptor of this layer (for the fused layer drivers)."""
        from ._lib import Linear
        pw = self.packed_weight()
        return Linear(pw.packed.data_ptr(), pw.packed.stride(0), pw.c_w.data_ptr(), 0)

    # -- forward ----------------------------------------------------------------
    def forward(self, x):
        check_hip_call(self.kernel_backend, "BitLinear", self, x)
        if x.dtype != self.weight.dtype:
            # F.linear in the reference raises for mixed operand dtypes
            raise RuntimeError(f"expected both operands to have the same dtype, got {x.dtype} and {self.weight.dtype}")
        pw = self.packed_weight()
        lead = x.shape[:-1]
        x2 = x.reshape(-1, self.in_features)
        q, s, rs = hip_ops.quant_act(x2, self.bit_eps)
        out = hip_ops.bitlinear(q, s, rs, pw.packed, pw.c_w, self.out_features, self.in_features, x.dtype,
                                bias=self.bias)
        return out.reshape(*lead, self.out_features)

    def extra_repr(self):
        return (f"in_features={self.in_features}, out_features={self.out_features}, bias={self.bias is not None}, "
                f"kernel_backend={self.kernel_backend}")
