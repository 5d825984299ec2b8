"""RMSNorm and Block with ``kernel_backend='hip'``.

Same parameters, construction order and forward contract as the reference's
``tesm_ssm/modules/block.py`` (RMSNorm :7-16, Block :19-47).  The residual add
and the norm run as one kernel (``tesm_hip_add_rmsnorm``); after the mixer the
second norm also emits the per-token int8 codes that the feed-forward's gate /
up products read, so its normalised output is never written.  Eval only, like
every module of this package.
"""
from __future__ import annotations

import ctypes
from typing import Optional

import torch
import torch.nn as nn

from . import _lib, hip_ops
from .bitlinear import backend_error


def _check(t: torch.Tensor, what: str) -> None:
    if not t.is_cuda:
        raise backend_error("hip", what, f"input is on {t.device}")
    if torch.is_grad_enabled():
        raise backend_error("hip", what, "the hip kernels are forward-only: run under torch.no_grad()")


class RMSNorm(nn.Module):
    """``x * rsqrt(mean(x^2) + eps) * weight`` in the input dtype (block.py:7-16)."""

    def __init__(self, dim: int, eps: float = 1e-5, device=None, dtype=None):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim, device=device, dtype=dtype))

    def fused(self, x: torch.Tensor, residual: Optional[torch.Tensor] = None, residual_dtype=None,
              want_y: bool = True, codes_eps: Optional[float] = None):
        """``s = x + residual`` (promoted dtype), ``y = self(s.to(weight dtype))``; returns
        ``(y or None, s in residual_dtype or None, codes or None)`` where ``codes = (q, s_x, rowsum)``
        are y's per-token int8 codes in the product layout (computed when ``codes_eps`` is given)."""
        _check(x, "RMSNorm")
        dt = self.weight.dtype
        if x.dtype != dt:
            raise RuntimeError(f"RMSNorm: input is {x.dtype} but the weight is {dt}")
        D = x.shape[-1]
        lead = x.shape[:-1]
        x2 = x.reshape(-1, D)
        if x2.stride(-1) != 1:
            x2 = x2.contiguous()
        M = x2.shape[0]
        dev = x.device
        desc = _lib.RmsNorm()
        desc.dt = hip_ops.dt_code(dt)
        desc.M, desc.D = M, D
        desc.eps = float(self.eps)
        desc.x, desc.ld_x = x2.data_ptr(), x2.stride(0)
        r2 = None
        if residual is not None:
            r2 = residual.reshape(-1, D)
            if r2.stride(-1) != 1:
                r2 = r2.contiguous()
            desc.residual, desc.residual_dt, desc.ld_res = r2.data_ptr(), hip_ops.dt_code(r2.dtype), r2.stride(0)
        res_out = None
        if residual_dtype is not None:
            res_out = torch.empty((M, D), dtype=residual_dtype, device=dev)
            desc.residual_out, desc.residual_out_dt, desc.ld_res_out = (res_out.data_ptr(),
                                                                        hip_ops.dt_code(residual_dtype), D)
        w = self.weight.detach()
        desc.weight = w.data_ptr()
        y = None
        if want_y:
            y = torch.empty((M, D), dtype=dt, device=dev)
            desc.y, desc.ld_y = y.data_ptr(), D
        codes = None
        if codes_eps is not None:
            ldq = hip_ops.kpad(D)
            q = torch.empty((M, ldq), dtype=torch.int8, device=dev)
            s = torch.empty((M,), dtype=torch.float32, device=dev)
            rs = torch.empty((M,), dtype=torch.int32, device=dev)
            desc.q, desc.ldq, desc.s_x, desc.rowsum, desc.bit_eps = (q.data_ptr(), ldq, s.data_ptr(), rs.data_ptr(),
                                                                     float(codes_eps))
            codes = (q, s, rs)
        hip_ops.require_device(x2, r2, w, res_out, y, *(codes or ()))
        with torch.cuda.device(dev):
            _lib.check(_lib.load().tesm_hip_add_rmsnorm(ctypes.byref(desc),
                                                         ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)))
        return (y.reshape(*lead, D) if y is not None else None,
                res_out.reshape(*lead, D) if res_out is not None else None, codes)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.fused(x)[0]

    def extra_repr(self):
        return f"{self.weight.shape[0]}, eps={self.eps}"


class Block(nn.Module):
    """Pre-norm residual block: norm -> mixer -> residual add -> norm2 -> mlp (block.py:19-47)."""

    def __init__(self, dim, mixer_cls, mlp_cls, norm_cls=RMSNorm, residual_in_fp32=False):
        super().__init__()
        self.residual_in_fp32 = residual_in_fp32
        self.norm = norm_cls(dim)
        self.mixer = mixer_cls(dim)
        self.norm2 = norm_cls(dim)
        self.mlp = mlp_cls(dim)
        if not isinstance(self.norm, RMSNorm) or not isinstance(self.norm2, RMSNorm):
            raise backend_error("hip", "Block norm", "only RMSNorm (config.rms_norm=True) is implemented")

    def _residual_dtype(self, hidden: torch.Tensor, residual: Optional[torch.Tensor]):
        if self.residual_in_fp32:
            return torch.float32
        return torch.promote_types(hidden.dtype, residual.dtype) if residual is not None else hidden.dtype

    def forward(self, hidden_states, residual=None, inference_params=None, prev_state=None, **mixer_kwargs):
        # residual = hidden + residual; hidden = norm(residual.to(dtype)); residual.to(f32) (block.py:28-31)
        res_dt = self._residual_dtype(hidden_states, residual)
        hidden, residual, _ = self.norm.fused(hidden_states, residual, residual_dtype=res_dt)
        out = self.mixer(hidden, inference_params=inference_params, prev_state=prev_state, **mixer_kwargs)
        hidden, final_state = out if isinstance(out, tuple) else (out, None)
        # residual = hidden + residual; the mlp reads norm2's output as int8 codes (block.py:37-44)
        res_dt = self._residual_dtype(hidden, residual)
        mlp = self.mlp
        eps = getattr(getattr(mlp, "gate_proj", None), "bit_eps", None)
        if hasattr(mlp, "forward_codes") and eps is not None:
            _, residual, codes = self.norm2.fused(hidden, residual, residual_dtype=res_dt, want_y=False, codes_eps=eps)
            hidden = mlp.forward_codes(codes, hidden.shape)
        else:
            hidden, residual, _ = self.norm2.fused(hidden, residual, residual_dtype=res_dt)
            hidden = mlp(hidden)
        return hidden, residual, final_state

    def allocate_inference_cache(self, batch_size, max_seqlen, dtype=None, **kwargs):
        if hasattr(self.mixer, "allocate_inference_cache"):
            return self.mixer.allocate_inference_cache(batch_size, max_seqlen, dtype=dtype, **kwargs)
        return None
