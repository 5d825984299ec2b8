"""MI355X-native (gfx950) forward hot path of the TESM layer: ``kernel_backend='hip'``.

Public API mirrors the reference package ``tesm_ssm`` for this path:
``BitLinear``, ``TESM_SISO`` (alias ``TESM``), ``TESMMIMO_Optimized`` and ``TESMConfig``.
Kernels live in ``tesm_amd/csrc`` and are reached through the C-ABI library
``libtesm_hip.so`` (``include/tesm_hip.h``).
"""
from .bitlinear import BitLinear
from .config import TESMConfig
from .tesm import TESM, TESM_SISO
from .tesm_mimo import TESMMIMO_Optimized

__all__ = ["BitLinear", "TESM", "TESM_SISO", "TESMMIMO_Optimized", "TESMConfig"]
