"""MI355X-native (gfx950) forward hot path of the TESM layer: ``kernel_backend='hip'``.

Public API mirrors the reference package ``tesm_ssm`` for this path:
``BitLinear``, ``TESM_SISO`` (alias ``TESM``), ``TESMMIMO_Optimized`` and ``TESMConfig``, plus the
block and model around the layers (``RMSNorm``, ``Block``, ``FeedForward``, ``MixerModel``,
``TESMLMHeadModel``) and the INT2 export format (``tesm_amd.int2``).  Kernels live in
``tesm_amd/csrc`` and are reached through the C-ABI library ``libtesm_hip.so``
(``include/tesm_hip.h``).
"""
from .bitlinear import BitLinear
from .block import Block, RMSNorm
from .config import TESMConfig
from .lm import FeedForward, MixerModel, TESMCausalLMOutput, TESMLMHeadModel
from .tesm import TESM, TESM_SISO
from .tesm_mimo import TESMMIMO_Optimized

__all__ = ["BitLinear", "Block", "FeedForward", "MixerModel", "RMSNorm", "TESM", "TESMCausalLMOutput", "TESMConfig",
           "TESMLMHeadModel", "TESM_SISO", "TESMMIMO_Optimized"]
