"""BitLinear with ``kernel_backend='hip'``.

Same constructor, parameters and initialisation as the reference's BitLinear
(tesm_ssm/modules/tesm.py:124-204), so checkpoints and seeded construction carry
over.  The forward pass is eval-only (no autograd), like the reference's
``cuda`` eval path: it quantizes activations per token to int8, multiplies
against the ternary weights packed four per byte, and scales the exact int32
accumulators once (tesm.py:206-215, 238-290).

The packed weight, its scale and the dequantized +1 value are cached per
``weight._version`` like the reference's eval cache (tesm.py:226-236).

``load_int2`` makes a module INT2-backed: its codes and scale then come from an
export entry of the reference's INT2 format (tesm_ssm/utils/int2_quantization.py:
196-217) instead of from the float weight, which is no longer read.
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
        # INT2-backed state: canonical packed codes (N, ceil(K/4)) and the exported scale.
        self.register_buffer("int2_packed", None, persistent=False)
        self.int2_scale = None
        self._int2_gen = 0
        self.reset_parameters()

    def reset_parameters(self):  # tesm.py:200-204
        nn.init.kaiming_uniform_(self.weight, a=math.sqrt(5))
        if self.bias is not None:
            bound = 1 / math.sqrt(self.in_features)
            nn.init.uniform_(self.bias, -bound, bound)

    # -- packed weight cache ---------------------------------------------------
    def cache_key(self):
        """Changes whenever the packed cache must be rebuilt: a new weight version, storage or dtype,
        or a new INT2 load."""
        w = self._parameters["weight"]
        return (w._version, w.data_ptr(), w.dtype, w.device, self._int2_gen)

    def packed_weight(self) -> PackedWeight:
        """Pack the ternary weight once per weight version (tesm.py:226-236), or lay out the loaded
        INT2 codes once per load, dtype and device."""
        key = self.cache_key()
        if self._packed is None or self._packed_key != key:
            w = self.weight
            with torch.no_grad():
                if self.int2_packed is not None:
                    self._packed = self._int2_cache(w.dtype, w.device)
                else:
                    s_w, c_w = hip_ops.absmean_scale(w.detach(), self.bit_eps)
                    packed = hip_ops.pack_weight(w.detach(), s_w)
                    self._packed = PackedWeight(packed, s_w, c_w, self.out_features, self.in_features)
            self._packed_key = key
        return self._packed

    # -- INT2 export entries (tesm_ssm/utils/int2_quantization.py:196-245) ------
    @property
    def is_int2(self) -> bool:
        return self.int2_packed is not None

    def load_int2(self, packed_weight, weight_scale, bias=None, in_features=None, out_features=None,
                  keep_float_weight=True):
        """Take this layer's codes and scale from one ``export_model_to_int2`` entry.

        ``packed_weight`` is the canonical uint8 (out_features, ceil(in_features/4)) array (code =
        q + 1, four 2-bit fields per byte, low bits first; int2_quantization.py:21-58) and
        ``weight_scale`` the exported ``1 / mean|w|`` (:32).  The forward keeps BitLinear's
        semantics (tesm.py:206-215, 287-290): the output is that of a BitLinear whose weight
        quantizes to these codes at this scale, i.e. int8 activations times ``code / scale`` with
        ``1 / scale`` rounded to the module dtype.  (The reference instead swaps in an
        ``Int2Linear``, which multiplies the unquantized input, int2_quantization.py:158-174.)
        ``bias`` replaces the layer's bias, ``None`` removing it, as the swap does.

        Raises ``ValueError`` for a shape that does not match the layer, a scale that is not a
        positive finite number, or a 2-bit field holding 3 (no ternary value).  With
        ``keep_float_weight=False`` the float weight's storage is released (the parameter keeps
        its dtype and device, with no elements); ``clear_int2`` goes back to the float weight.
        """
        N, K = self.out_features, self.in_features
        if in_features is not None and int(in_features) != K or out_features is not None and int(out_features) != N:
            raise ValueError(f"INT2 entry is {in_features} -> {out_features}, the layer is {K} -> {N}")
        p = torch.as_tensor(packed_weight)
        kb = (K + 3) // 4
        if p.dtype != torch.uint8 or p.dim() != 2 or tuple(p.shape) != (N, kb):
            raise ValueError(f"packed_weight must be uint8 of shape ({N}, {kb}), got {p.dtype} {tuple(p.shape)}")
        scale = torch.as_tensor(weight_scale)
        if scale.numel() != 1:
            raise ValueError(f"weight_scale must hold one value, got shape {tuple(scale.shape)}")
        sv = float(scale.reshape(()).item())
        if not (math.isfinite(sv) and sv > 0.0):
            raise ValueError(f"weight_scale must be a positive finite number, got {sv}")
        if bool(((p >> 1) & p & 0x55).any()):
            raise ValueError("packed_weight holds a 2-bit field equal to 3, which encodes no ternary value")
        dev = self.weight.device
        p = p.to(device=dev, copy=True).contiguous()
        if K % 4:
            # fields past in_features hold code 1 (value 0), as the exporter pads them (int2_quantization.py:42-45)
            keep = (1 << (2 * (K % 4))) - 1
            p[:, kb - 1] = (p[:, kb - 1] & keep) | (0x55 & ~keep & 0xFF)
        with torch.no_grad():
            if bias is None:
                self.bias = None
            else:
                b = torch.as_tensor(bias)
                if b.numel() != N:
                    raise ValueError(f"bias must have {N} elements, got {b.numel()}")
                self.bias = nn.Parameter(b.detach().reshape(N).to(device=dev, dtype=self.weight.dtype).clone())
            if not keep_float_weight:
                self.weight.data = torch.empty((0,), dtype=self.weight.dtype, device=dev)
        self.int2_packed = p
        self.int2_scale = sv
        self._int2_gen += 1
        self._packed = None

    def clear_int2(self):
        """Forget the loaded INT2 codes; the packed cache follows the float weight again."""
        if self.weight.numel() != self.out_features * self.in_features:
            raise RuntimeError("the float weight was released by load_int2(keep_float_weight=False)")
        self.int2_packed = None
        self.int2_scale = None
        self._int2_gen += 1
        self._packed = None

    def _int2_cache(self, dtype, device) -> PackedWeight:
        """Loaded codes in the products' layout: rows padded to kpad(K)/4 bytes with code 1.  The
        scale is rounded to the module dtype and the +1 value is ``1 / scale`` divided in that
        dtype, as BitLinear's dequantization ``q / scale`` (tesm.py:215) rounds it."""
        N, K = self.out_features, self.in_features
        src = self.int2_packed.to(device)
        packed = torch.full((N, hip_ops.kpad(K) // 4), 0x55, dtype=torch.uint8, device=device)
        packed[:, :src.shape[1]].copy_(src)
        s = torch.tensor(self.int2_scale, dtype=torch.float32).to(dtype)
        c = torch.ones((), dtype=dtype) / s
        sc = torch.stack([s.float(), c.float()]).to(device)
        return PackedWeight(packed, sc[0:1], sc[1:2], N, K)

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
        # quantized_input + _project_quantized (tesm.py:206-209, 287-290) in one C-ABI call
        out = hip_ops.bitlinear_fwd(x2, pw.packed, pw.c_w, self.out_features, self.bit_eps, bias=self.bias)
        return out.reshape(*lead, self.out_features)

    def extra_repr(self):
        return (f"in_features={self.in_features}, out_features={self.out_features}, bias={self.bias is not None}, "
                f"kernel_backend={self.kernel_backend}")
