"""TESMConfig: the reference's configuration dataclass, with ``'hip'`` accepted.

Field names, defaults and preset values are the reference's
(``tesm_ssm/models/config_tesm.py:18-480``) so that configs round-trip between
the two packages; presets are written here as overrides of the defaults.
``kernel_backend`` accepts ``'hip'`` (and ``'auto'``, which this package
resolves to ``'hip'``).
"""
from __future__ import annotations

from dataclasses import asdict, dataclass, replace
from typing import Dict, Optional


@dataclass
class TESMConfig:
    d_model: int = 768
    n_layer: int = 24
    d_intermediate: int = 2048
    vocab_size: int = 151936
    max_seq_len: int = 2048
    pad_token_id: int = 0
    eos_token_id: Optional[int] = None
    label_ignore_index: int = -100
    gradient_checkpointing: bool = False
    tie_embeddings: bool = True
    dropout: float = 0.0
    rms_norm: bool = True
    residual_in_fp32: bool = True
    norm_epsilon: float = 1e-5
    initializer_range: float = 0.02
    rescale_prenorm_residual: bool = True
    bit_eps: float = 1e-5
    bit_threshold: float = 0.5
    vocab_suppression: bool = False
    suppression_bias: float = -10.0
    semantic_activation: bool = True
    semantic_activation_strength: float = 0.5
    semantic_activation_threshold: float = 0.1
    use_mimo: bool = False
    n_heads: int = 4
    d_state: int = 256
    expand: int = 2
    ent_rank: int = 64
    entanglement_scale: float = 0.2
    entanglement_threshold: float = 0.1
    entanglement_init: float = 0.3
    entanglement_window: int = 16
    entanglement_block_size: int = 256
    state_scan_chunk_size: int = 16
    use_triton_kernels: bool = True
    kernel_backend: str = "auto"
    kernel_mode: str = "fast"
    decay_init_bias: float = 3.0
    rope_base: float = 10000.0
    global_rel_pos_dim: int = 64
    annealing_enabled: bool = True
    T_start: float = 10.0
    T_end: float = 0.1
    annealing_steps: int = 1000
    annealing_schedule: str = "cosine"
    quantum_tunneling_enabled: bool = False
    tunneling_strength: float = 0.1
    num_tunnel_paths: int = 4
    energy_landscape: str = "entropy"
    tunneling_schedule: str = "adaptive"

    # -- presets (config_tesm.py:195-473) -------------------------------------
    @classmethod
    def _preset(cls, **over) -> "TESMConfig":
        return replace(cls(), **over)

    @classmethod
    def tiny(cls):
        return cls._preset(n_layer=12, d_intermediate=3072, max_seq_len=1024, d_state=384, ent_rank=96,
                           entanglement_scale=0.25, entanglement_threshold=0.05, decay_init_bias=1.0,
                           annealing_steps=500)

    @classmethod
    def small(cls):
        return cls._preset(d_model=512, n_layer=16, d_intermediate=1536, max_seq_len=512, ent_rank=48,
                           entanglement_threshold=0.08, entanglement_window=0, decay_init_bias=1.0,
                           annealing_steps=2000)

    @classmethod
    def small_short(cls):
        return cls._preset(d_model=512, n_layer=16, d_intermediate=1536, max_seq_len=256, ent_rank=48,
                           entanglement_scale=0.25, entanglement_threshold=0.05, decay_init_bias=0.0)

    @classmethod
    def base(cls):
        return cls._preset(d_state=384, entanglement_threshold=0.08, entanglement_window=32,
                           decay_init_bias=2.0, annealing_steps=5000)

    @classmethod
    def medium(cls):
        return cls._preset(d_model=1024, n_layer=32, d_intermediate=2816, d_state=512, ent_rank=80,
                           entanglement_scale=0.25, entanglement_threshold=0.08, entanglement_init=0.35,
                           entanglement_window=32, decay_init_bias=2.0, annealing_steps=10000)

    @classmethod
    def long_context(cls):
        return cls._preset(d_model=256, n_layer=8, d_intermediate=512, max_seq_len=16384, d_state=512,
                           ent_rank=32, entanglement_scale=0.25, entanglement_threshold=0.08,
                           entanglement_window=32, decay_init_bias=6.0, annealing_steps=10000)

    @classmethod
    def exp_decay_comparison(cls, decay_bias: float):
        return cls._exp(decay_init_bias=decay_bias)

    @classmethod
    def exp_threshold_comparison(cls, threshold: float):
        return cls._exp(entanglement_threshold=threshold, decay_init_bias=0.0)

    @classmethod
    def exp_scale_comparison(cls, scale: float):
        return cls._exp(entanglement_scale=scale, decay_init_bias=0.0)

    @classmethod
    def _exp(cls, **over):
        base = dict(d_model=256, n_layer=6, d_intermediate=1024, max_seq_len=256, ent_rank=32,
                    entanglement_scale=0.25, entanglement_threshold=0.05, annealing_steps=500)
        base.update(over)
        return cls._preset(**base)

    @classmethod
    def _large(cls, d_model, n_layer, max_seq_len, window, steps):
        return cls._preset(d_model=d_model, n_layer=n_layer, d_intermediate=4 * d_model, max_seq_len=max_seq_len,
                           d_state=d_model // 2, ent_rank=d_model // 16, entanglement_threshold=0.05,
                           entanglement_window=window, entanglement_block_size=512, state_scan_chunk_size=32,
                           decay_init_bias=6.0, annealing_steps=steps)

    @classmethod
    def large_40b(cls):
        return cls._large(4096, 48, 131072, 64, 20000)

    @classmethod
    def large_70b(cls):
        return cls._large(6144, 48, 131072, 64, 30000)

    @classmethod
    def large_100b(cls):
        return cls._large(8192, 56, 204800, 64, 50000)

    @classmethod
    def large_200b(cls):
        return cls._large(10240, 72, 204800, 128, 100000)

    @classmethod
    def large_400b(cls):
        return cls._large(12288, 96, 204800, 128, 200000)

    def to_dict(self) -> Dict:
        return asdict(self)

    @classmethod
    def from_dict(cls, config_dict: Dict) -> "TESMConfig":
        return cls(**{k: v for k, v in config_dict.items() if k in cls.__dataclass_fields__})
