"""FeedForward, MixerModel and TESMLMHeadModel with ``kernel_backend='hip'``.

Mirrors ``tesm_ssm/models/mixer_seq_simple.py`` (FeedForward :25-67, MixerModel :69-239,
TESMLMHeadModel :242-345, _merge_stats :761-787, _init_weights :790-803): same constructor
arguments, parameter names and creation order, so ``torch.manual_seed(s)`` before construction
gives the reference's weights and a reference ``state_dict`` loads unchanged.  The feed-forward is
one C-ABI call (``tesm_hip_ffn_forward``): gate and up share one int8 quantization of the input
(the reference's grouped projection, :45-57), both products and ``silu(gate) * up`` come out of one
pass, and down_proj follows.  Embeddings and the tied LM head are torch ops (a gather and a plain
library GEMM).  Eval forward only; the vocabulary-suppression branch of the LM head (off by
default) is not provided.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from functools import partial
from typing import Dict, List, Optional

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _lib, hip_ops
from .bitlinear import BitLinear, backend_error, check_hip_call
from .block import Block, RMSNorm
from .config import TESMConfig
from .tesm import TESM_SISO, workspace
from .tesm_mimo import TESMMIMO_Optimized


@dataclass
class TESMCausalLMOutput:
    loss: Optional[torch.Tensor] = None
    logits: Optional[torch.Tensor] = None
    hidden_states: Optional[torch.Tensor] = None
    entanglement_maps: Optional[List[torch.Tensor]] = None
    entanglement_stats: Optional[Dict[str, float]] = None


class FeedForward(nn.Module):
    """``down_proj(silu(gate_proj(x)) * up_proj(x))`` on INT2 BitLinears (mixer_seq_simple.py:25-67)."""

    def __init__(self, config: TESMConfig, device=None, dtype=None):
        super().__init__()
        bl = dict(bias=False, bit_eps=config.bit_eps, bit_threshold=config.bit_threshold,
                  kernel_backend=config.kernel_backend, kernel_mode=config.kernel_mode, device=device, dtype=dtype)
        self.gate_proj = BitLinear(config.d_model, config.d_intermediate, **bl)
        self.up_proj = BitLinear(config.d_model, config.d_intermediate, **bl)
        self.down_proj = BitLinear(config.d_intermediate, config.d_model, **bl)
        self.dropout = nn.Dropout(config.dropout)

    def _run(self, dt, lead, M, dev, x2=None, codes=None):
        for p in (self.gate_proj, self.up_proj, self.down_proj):
            if p.bias is not None:
                raise backend_error(p.kernel_backend, "FeedForward", "BitLinear bias is not supported here")
            if p.weight.dtype != dt:
                raise RuntimeError(f"expected both operands to have the same dtype, got {dt} and {p.weight.dtype}")
        d_model, d_inter = self.gate_proj.in_features, self.gate_proj.out_features
        y = torch.empty((M, d_model), dtype=dt, device=dev)
        desc = _lib.Ffn()
        desc.dt = hip_ops.dt_code(dt)
        desc.M, desc.d_model, desc.d_inter = M, d_model, d_inter
        desc.bit_eps = float(self.gate_proj.bit_eps)
        if codes is not None:
            q, s, rs = codes
            desc.x_codes, desc.ldq_x, desc.x_scale, desc.x_rowsum = q.data_ptr(), q.stride(0), s.data_ptr(), rs.data_ptr()
            hip_ops.require_device(q, s, rs, y)
        else:
            desc.x, desc.ld_x = x2.data_ptr(), x2.stride(0)
            hip_ops.require_device(x2, y)
        desc.gate_proj = self.gate_proj.linear_desc()
        desc.up_proj = self.up_proj.linear_desc()
        desc.down_proj = self.down_proj.linear_desc()
        desc.y, desc.ld_y = y.data_ptr(), d_model
        lib = _lib.load()
        nbytes = int(lib.tesm_hip_ffn_ws_bytes(ctypes.byref(desc)))
        stream = torch.cuda.current_stream(dev)
        with torch.cuda.device(dev):
            ws = workspace(dev, nbytes, stream)
            _lib.check(lib.tesm_hip_ffn_forward(ctypes.byref(desc), ctypes.c_void_p(ws.data_ptr()), ws.numel(),
                                                ctypes.c_void_p(stream.cuda_stream)))
        return y.reshape(*lead, d_model)

    def forward(self, x):
        check_hip_call(self.gate_proj.kernel_backend, "FeedForward", self, x)
        lead = x.shape[:-1]
        x2 = x.reshape(-1, x.shape[-1])
        if x2.stride(-1) != 1:
            x2 = x2.contiguous()
        return self._run(x.dtype, lead, x2.shape[0], x.device, x2=x2)

    def forward_codes(self, codes, shape):
        """The forward on x given as its per-token int8 codes ``(q, s_x, rowsum)`` (product layout,
        quantized with gate_proj.bit_eps), e.g. from ``RMSNorm.fused``; ``shape`` is x's shape."""
        q = codes[0]
        check_hip_call(self.gate_proj.kernel_backend, "FeedForward", self, q)
        return self._run(self.gate_proj.weight.dtype, tuple(shape[:-1]), q.shape[0], q.device, codes=codes)


def _init_weights(module, n_layer, initializer_range=0.02, rescale_prenorm_residual=True, n_residuals_per_layer=1):
    """mixer_seq_simple.py:790-803.  With recurse=False no parameter name contains a '.', so the
    residual rescale never fires, as in the reference."""
    if isinstance(module, nn.Linear):
        if module.bias is not None:
            nn.init.zeros_(module.bias)
        nn.init.normal_(module.weight, std=initializer_range)
    elif isinstance(module, BitLinear):
        nn.init.normal_(module.weight, std=initializer_range)
    elif isinstance(module, nn.Embedding):
        nn.init.normal_(module.weight, std=initializer_range)
    if rescale_prenorm_residual:
        for name, param in module.named_parameters(recurse=False):
            if name in ["out_proj.weight", "down_proj.weight"]:
                with torch.no_grad():
                    param /= (n_residuals_per_layer * n_layer) ** 0.5


def _merge_stats(stats_list: List) -> Optional[Dict[str, float]]:
    """Positive / negative / zero fractions over the layers' ternary maps (mixer_seq_simple.py:761-787)."""
    if not stats_list:
        return None
    pos = neg = zero = count = 0.0
    for item in stats_list:
        if isinstance(item, tuple) and len(item) == 2:
            ternary, total = item
            if ternary is not None:
                eps = 1e-3
                pos += float((ternary > eps).sum().item())
                neg += float((ternary < -eps).sum().item())
                zero += float((ternary.abs() <= eps).sum().item())
                count += float(total)
    if count > 0:
        return {"positive": pos / count, "negative": neg / count, "zero": zero / count}
    return None


class MixerModel(nn.Module):
    def __init__(self, config: TESMConfig, device=None, dtype=None):
        super().__init__()
        factory_kwargs = {"device": device, "dtype": dtype}
        self.config = config
        self.gradient_checkpointing = config.gradient_checkpointing
        self.residual_in_fp32 = config.residual_in_fp32
        self.embedding = nn.Embedding(config.vocab_size, config.d_model, **factory_kwargs)
        self.position_embedding = nn.Embedding(config.max_seq_len, config.d_model, **factory_kwargs)
        if not config.rms_norm:
            raise backend_error(config.kernel_backend, "LayerNorm", "only RMSNorm (config.rms_norm=True) is implemented")
        norm_cls = partial(RMSNorm, eps=config.norm_epsilon)
        if config.use_mimo:  # mixer_seq_simple.py:84-106
            def mixer_cls(layer_idx):
                return lambda dim: TESMMIMO_Optimized(
                    d_model=dim, n_heads=config.n_heads, d_state=config.d_state, expand=config.expand,
                    ent_rank=config.ent_rank, entanglement_window=config.entanglement_window,
                    entanglement_threshold=config.entanglement_threshold,
                    entanglement_scale=config.entanglement_scale, max_seq_len=config.max_seq_len,
                    dropout=config.dropout, bit_eps=config.bit_eps, bit_threshold=config.bit_threshold,
                    kernel_backend=config.kernel_backend, annealing_enabled=config.annealing_enabled,
                    T_start=config.T_start, T_end=config.T_end, annealing_steps=config.annealing_steps,
                    annealing_schedule=config.annealing_schedule, **factory_kwargs)
        else:  # mixer_seq_simple.py:107-141
            def mixer_cls(layer_idx):
                return lambda dim: TESM_SISO(
                    d_model=dim, d_state=config.d_state, expand=config.expand, ent_rank=config.ent_rank,
                    entanglement_scale=config.entanglement_scale,
                    entanglement_threshold=config.entanglement_threshold,
                    entanglement_window=config.entanglement_window,
                    entanglement_block_size=config.entanglement_block_size,
                    entanglement_init=config.entanglement_init, layer_idx=layer_idx, max_seq_len=config.max_seq_len,
                    dropout=config.dropout, bit_eps=config.bit_eps, bit_threshold=config.bit_threshold,
                    kernel_backend=config.kernel_backend, kernel_mode=config.kernel_mode,
                    use_triton_kernels=config.use_triton_kernels, state_scan_chunk_size=config.state_scan_chunk_size,
                    decay_init_bias=config.decay_init_bias, rope_base=getattr(config, "rope_base", 10000.0),
                    annealing_enabled=config.annealing_enabled, T_start=config.T_start, T_end=config.T_end,
                    annealing_steps=config.annealing_steps, annealing_schedule=config.annealing_schedule,
                    quantum_tunneling_enabled=config.quantum_tunneling_enabled,
                    tunneling_strength=config.tunneling_strength, num_tunnel_paths=config.num_tunnel_paths,
                    energy_landscape=config.energy_landscape, tunneling_schedule=config.tunneling_schedule,
                    **factory_kwargs)

        def mlp_cls(dim):
            return FeedForward(config, device=device, dtype=dtype)

        self.layers = nn.ModuleList([
            Block(config.d_model, mixer_cls(layer_idx), mlp_cls, norm_cls=norm_cls,
                  residual_in_fp32=config.residual_in_fp32)
            for layer_idx in range(config.n_layer)])
        for layer_idx, layer in enumerate(self.layers):
            layer.layer_idx = layer_idx
        self.norm_f = RMSNorm(config.d_model, eps=config.norm_epsilon)
        self.apply(partial(_init_weights, n_layer=config.n_layer, initializer_range=config.initializer_range,
                           rescale_prenorm_residual=config.rescale_prenorm_residual, n_residuals_per_layer=1))

    def allocate_inference_cache(self, batch_size, max_seqlen, dtype=None, **kwargs):
        return {i: layer.allocate_inference_cache(batch_size, max_seqlen, dtype=dtype, **kwargs)
                for i, layer in enumerate(self.layers)}

    def forward(self, input_ids, inference_params=None, prev_states=None, **mixer_kwargs):
        """mixer_seq_simple.py:171-239: embeddings + positions (offset by layer 0's cache position in
        a one-token decode step), the blocks with each layer's cache and the previous layer's
        cross-layer state, the final residual add and norm."""
        batch_size, seqlen = input_ids.shape
        if seqlen == 0:
            raise ValueError("Input sequence length is 0")
        if seqlen > self.config.max_seq_len:
            raise ValueError(f"Sequence length {seqlen} exceeds max_seq_len {self.config.max_seq_len}")
        if self.training:
            raise backend_error(self.config.kernel_backend, "MixerModel", "the hip kernels are forward-only (eval)")
        pos_offset = 0
        if inference_params is not None and seqlen == 1 and "state_cache" in inference_params:
            layer0_cache = inference_params["state_cache"].get(0)
            if layer0_cache is not None and "seq_pos" in layer0_cache:
                pos_offset = layer0_cache["seq_pos"]
        positions = torch.arange(pos_offset, pos_offset + seqlen, device=input_ids.device).unsqueeze(0).expand(
            batch_size, -1)
        hidden_states = self.embedding(input_ids) + self.position_embedding(positions)
        residual = None
        entanglement_maps, entanglement_stats, final_states = [], [], []
        cross_layer_state = None
        for i, layer in enumerate(self.layers):
            layer_prev_state = prev_states[i] if prev_states is not None else None
            layer_mixer_kwargs = dict(mixer_kwargs, cross_layer_state=cross_layer_state)
            layer_inference_params = None
            if inference_params is not None and "state_cache" in inference_params:
                layer_cache = inference_params["state_cache"].get(i)
                if layer_cache is not None:
                    layer_inference_params = {"state_cache": layer_cache}
            hidden_states, residual, final_state = layer(hidden_states, residual,
                                                         inference_params=layer_inference_params,
                                                         prev_state=layer_prev_state, **layer_mixer_kwargs)
            if final_state is not None:
                final_states.append(final_state)
            cross_layer_state = getattr(layer.mixer, "_last_cross_layer_state", None)
            if getattr(layer.mixer, "last_entanglement_map", None) is not None:
                entanglement_maps.append(layer.mixer.last_entanglement_map)
            if getattr(layer.mixer, "_stats_ternary_buffer", None) is not None:
                total_buf = layer.mixer._stats_total_buffer
                entanglement_stats.append((layer.mixer._stats_ternary_buffer,
                                           total_buf.item() if total_buf is not None else 1.0))
            elif getattr(layer.mixer, "_ternary_stats_for_logging", None) is not None:
                entanglement_stats.append(layer.mixer._ternary_stats_for_logging)
            elif getattr(layer.mixer, "last_entanglement_stats", None) is not None:
                entanglement_stats.append(layer.mixer.last_entanglement_stats)
        # residual = hidden + residual; norm_f(residual.to(dtype)) (mixer_seq_simple.py:237-238)
        hidden_states, _, _ = self.norm_f.fused(hidden_states, residual)
        return hidden_states, entanglement_maps, _merge_stats(entanglement_stats), final_states


class TESMLMHeadModel(nn.Module):
    """Backbone + tied LM head (mixer_seq_simple.py:242-345), plain-logits branch."""

    def __init__(self, config: Optional[TESMConfig] = None, device=None, dtype=None):
        super().__init__()
        self.tesm_config = config or TESMConfig()
        self.backbone = MixerModel(self.tesm_config, device=device, dtype=dtype)
        self.lm_head = nn.Linear(self.tesm_config.d_model, self.tesm_config.vocab_size, bias=False, device=device,
                                 dtype=dtype)
        if self.tesm_config.tie_embeddings:
            self.lm_head.weight = self.backbone.embedding.weight
        self.vocab_suppression = getattr(self.tesm_config, "vocab_suppression", False)

    def get_input_embeddings(self):
        return self.backbone.embedding

    def set_input_embeddings(self, value):
        self.backbone.embedding = value
        if self.tesm_config.tie_embeddings:
            self.lm_head.weight = value.weight

    def allocate_inference_cache(self, batch_size, max_seqlen, dtype=None, **kwargs):
        return self.backbone.allocate_inference_cache(batch_size, max_seqlen, dtype=dtype, **kwargs)

    def forward(self, input_ids: torch.Tensor, labels: Optional[torch.Tensor] = None,
                inference_params: Optional[dict] = None, prev_states=None, logits_to_keep: int = 0,
                sparse_logits: bool = False, **kwargs):
        for k in ["attention_mask", "past_key_values", "use_cache"]:
            kwargs.pop(k, None)
        if self.vocab_suppression or sparse_logits:
            raise backend_error(self.tesm_config.kernel_backend, "vocabulary suppression",
                                "only the plain-logits LM head is implemented by the hip backend")
        hidden_states, entanglement_maps, entanglement_stats, final_states = self.backbone(
            input_ids=input_ids, inference_params=inference_params, prev_states=prev_states, **kwargs)
        sl = slice(-logits_to_keep, None) if isinstance(logits_to_keep, int) and logits_to_keep > 0 else slice(None)
        logits = self.lm_head(hidden_states[:, sl, :])
        loss = None
        if labels is not None:  # mixer_seq_simple.py:323-330
            shift_logits = logits[..., :-1, :].contiguous()
            shift_labels = labels[..., 1:].contiguous()
            loss = F.cross_entropy(shift_logits.view(-1, shift_logits.size(-1)), shift_labels.view(-1),
                                   ignore_index=self.tesm_config.label_ignore_index)
        return TESMCausalLMOutput(loss=loss, logits=logits, hidden_states=hidden_states,
                                  entanglement_maps=entanglement_maps, entanglement_stats=entanglement_stats), final_states
