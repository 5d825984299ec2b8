"""Torch restatement of the reference's ``kernel_backend='torch'`` forward path.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``): the checker for the HIP
path, and the timed CPU baseline.  It runs on whatever device its tensors live
on, but tests run it on the CPU.

Each method restates one reference method and keeps that method's sequence of
torch operations, because the parity bar is bit-level (quantized codes, ternary
decisions) and float rounding depends on the exact op order.  Module
construction consumes the global RNG in the reference's order, so
``torch.manual_seed(s)`` before construction yields the reference's parameters.

Reference = WANGLILIN360/tesm; paths are relative to its root.

Deviations, each only where the reference itself raises:
* ``amend_bf16`` (default True).  In bf16 the reference's MIMO forward feeds a
  float32 tensor into a bf16 BitLinear (tesm_mimo.py:1016-1045 -> F.linear dtype
  error), its global branch multiplies bf16 weights with the float32 rank states
  (tesm_mimo.py:678 -> matmul dtype error; amended: weights cast to float32), and
  the SISO/MIMO decode step mixes bf16 queries with float32 ring
  buffers in ``einsum`` (tesm.py:1352, tesm_mimo.py:865).  With the amendment the
  oracle casts those tensors to the module dtype (lossless for the ring
  buffers, whose entries are all module-dtype values) so the path runs.  In
  float32 the amendment never triggers.
* Quantum tunnelling (off by default, tesm.py:293-453, config_tesm.py:179) is
  not restated; enabling it raises NotImplementedError.
"""
from __future__ import annotations

import math
from typing import Optional

import torch
import torch.nn as nn
import torch.nn.functional as F


# ---------------------------------------------------------------------------
# BitLinear  (tesm_ssm/modules/tesm.py:124-290)
# ---------------------------------------------------------------------------
class BitLinear(nn.Module):
    """Ternary-weight / int8-activation fake-quant linear layer, torch path."""

    def __init__(self, in_features, out_features, bias=False, bit_eps=1e-5, bit_threshold=0.5,
                 kernel_backend="torch", kernel_mode="fast", device=None, dtype=None):
        super().__init__()
        self.in_features = in_features
        self.out_features = out_features
        self.bit_eps = bit_eps
        self.bit_threshold = bit_threshold
        self.kernel_backend = str(kernel_backend)
        self.kernel_mode = "precise" if str(kernel_mode) == "precise" else "fast"
        self.weight = nn.Parameter(torch.empty(out_features, in_features, device=device, dtype=dtype))
        self.bias = nn.Parameter(torch.zeros(out_features, device=device, dtype=dtype)) if bias else None
        self._cached_qweight = None
        self._cached_weight_version = -1
        self.reset_parameters()

    def reset_parameters(self):  # tesm.py:200-204
        nn.init.kaiming_uniform_(self.weight, a=math.sqrt(5))
        if self.bias is not None:
            lim = 1 / math.sqrt(self.in_features)
            nn.init.uniform_(self.bias, -lim, lim)

    # Test hook (None by default): ``code_hook(x, v, codes, scale) -> (codes, scale)`` sees the
    # pre-rounding values v = x * scale and the codes before they are dequantized; parity tests use
    # it to feed in another implementation's codes where those differ from these only at near-ties.
    code_hook = None
    # Test switch (False by default): evaluate the product exactly -- float64 sums of the unrounded
    # dequantized operands codes / scale, rounded once to the output dtype -- which is the arithmetic of
    # an int32-accumulator implementation, instead of F.linear on dtype-rounded operands.  bf16 parity
    # tests set it so that two implementations' BitLinear outputs differ only at rounding boundaries.
    exact_products = False
    _exact_input = None

    def quantized_input(self, x):
        """Per-token absmax int8 fake quant (tesm.py:206-209).

        ``127 / t`` is evaluated by torch as ``t.reciprocal() * 127``.
        """
        amax = x.detach().abs().max(dim=-1, keepdim=True).values
        scale = 127 / amax.clamp_min(self.bit_eps)
        v = x * scale
        codes = v.round().clamp(-128, 127)
        if self.code_hook is not None:
            codes, scale = self.code_hook(x, v, codes, scale)
        if self.exact_products:
            self._exact_input = codes.double() / scale.double()
        deq = codes / scale
        return x + (deq - x).detach()

    def quantized_weight(self):
        """Per-tensor absmean ternary fake quant (tesm.py:211-215)."""
        scale = 1.0 / self.weight.detach().abs().mean().clamp_min(self.bit_eps)
        normalized = self.weight * scale
        codes = normalized.round().clamp(-1, 1)
        return (normalized + (codes - normalized).detach()) / scale

    def weight_scale(self):
        """The scalar ``s_w`` used by ``quantized_weight`` (tesm.py:212)."""
        return 1.0 / self.weight.detach().abs().mean().clamp_min(self.bit_eps)

    def _current_quantized_weight(self):  # tesm.py:226-236
        if not self.training and not torch.is_grad_enabled():
            version = self.weight._version
            if self._cached_qweight is None or self._cached_weight_version != version:
                self._cached_qweight = self.quantized_weight()
                self._cached_weight_version = version
            return self._cached_qweight
        return self.quantized_weight()

    def _project_quantized(self, qinput, qweight, bias=None):  # tesm.py:273-276
        ex, self._exact_input = self._exact_input, None
        if self.exact_products and ex is not None and ex.shape == qinput.shape:
            b = bias.double() if bias is not None else None
            return F.linear(ex, qweight.double(), b).to(qinput.dtype)
        return F.linear(qinput, qweight, bias)

    def forward(self, x):  # tesm.py:287-290
        qweight = self._current_quantized_weight()
        return self._project_quantized(self.quantized_input(x), qweight, self.bias)


# ---------------------------------------------------------------------------
# TESM_SISO  (tesm_ssm/modules/tesm.py:456-1400)
# ---------------------------------------------------------------------------
class TESM_SISO(nn.Module):
    """Single-head TESM layer, torch path (eval semantics are the parity target)."""

    def __init__(self, d_model, d_state=256, expand=2, ent_rank=64, entanglement_scale=0.2,
                 entanglement_threshold=0.1, max_seq_len=2048, dropout=0.0, bit_eps=1e-5,
                 bit_threshold=0.5, layer_idx=None, device=None, dtype=None,
                 annealing_enabled=True, T_start=10.0, T_end=0.1, annealing_steps=1000,
                 annealing_schedule="cosine", quantum_tunneling_enabled=False,
                 tunneling_strength=0.1, num_tunnel_paths=4, energy_landscape="entropy",
                 tunneling_schedule="adaptive", amend_bf16=True, **kwargs):
        super().__init__()
        for name, v in (("d_state", d_state), ("d_model", d_model), ("ent_rank", ent_rank),
                        ("max_seq_len", max_seq_len)):
            if v <= 0:  # tesm.py:492-499
                raise ValueError(f"{name} must be positive, got {v}")
        if quantum_tunneling_enabled:
            raise NotImplementedError("quantum tunnelling is not restated by the oracle")
        self.d_model, self.d_state, self.expand = d_model, d_state, expand
        self.ent_rank = ent_rank
        self.entanglement_scale = entanglement_scale
        self.entanglement_threshold = entanglement_threshold
        self.entanglement_init = kwargs.get("entanglement_init", 0.3)
        self.entanglement_window = int(kwargs.get("entanglement_window", 0) or 0)
        self.entanglement_block_size = int(kwargs.get("entanglement_block_size", 256) or 256)
        self.state_scan_chunk_size = int(kwargs.get("state_scan_chunk_size", 16) or 16)
        self.kernel_backend = str(kwargs.get("kernel_backend", "torch"))
        self.kernel_mode = "precise" if str(kwargs.get("kernel_mode", "fast")) == "precise" else "fast"
        self.max_seq_len = max_seq_len
        self.layer_idx = layer_idx
        self.annealing_enabled = annealing_enabled
        self.T_start, self.T_end = T_start, T_end
        self.annealing_steps = annealing_steps
        self.annealing_schedule = annealing_schedule
        self.amend_bf16 = amend_bf16
        self.register_buffer("annealing_step", torch.tensor(0))
        self.quantum_tunneling_enabled = False
        self.quantum_tunneler = None

        bl = dict(bias=False, bit_eps=bit_eps, bit_threshold=bit_threshold,
                  kernel_backend=self.kernel_backend, kernel_mode=self.kernel_mode,
                  device=device, dtype=dtype)
        n_proj = 2 * d_model + 3 * d_state + 2 * ent_rank  # tesm.py:533
        self.in_proj = BitLinear(d_model, n_proj, **bl)
        self.state_proj = BitLinear(d_state, d_model, **bl)
        self.ent_proj = BitLinear(d_state, d_model, **bl)
        self.out_proj = BitLinear(d_model, d_model, **bl)
        self.dropout = nn.Dropout(dropout)
        self.decay_bias = nn.Parameter(torch.full((d_state,), float(kwargs.get("decay_init_bias", 3.0)),
                                                  device=device, dtype=torch.float32))
        if self.entanglement_window > 0:  # tesm.py:543-551
            self.register_parameter("entanglement", None)
            self.local_entanglement_bias = nn.Parameter(
                torch.randn(self.entanglement_window, device=device, dtype=torch.float32) * self.entanglement_init)
        else:  # tesm.py:553-570
            self.register_parameter("local_entanglement_bias", None)
            self.global_rel_pos_scale = nn.Parameter(torch.ones(1, device=device, dtype=torch.float32))
            self.global_rel_pos_bias = nn.Parameter(torch.zeros(1, device=device, dtype=torch.float32))
            self.global_rel_pos_dim = int(kwargs.get("global_rel_pos_dim", 64))
            self.global_rel_pos_embed = nn.Parameter(
                torch.randn(self.global_rel_pos_dim, device=device, dtype=torch.float32) * 0.02)
            self.register_parameter("entanglement", None)
        self.rope_base = float(kwargs.get("rope_base", 10000.0))
        self.cross_layer_q_proj = BitLinear(d_state, ent_rank, **bl)
        self.last_entanglement_map = None
        self.last_entanglement_stats = None
        self._last_cross_layer_state = None
        self._last_scan_state_f64 = None
        self.register_buffer("_stats_ternary_buffer", None, persistent=False)  # tesm.py:582-584
        self.register_buffer("_stats_total_buffer", torch.tensor(1.0), persistent=False)

    # -- temperature and ternary decision (tesm.py:587-618, 672-714) -----------
    def get_temperature(self):
        if not self.training or not self.annealing_enabled:
            return self.T_end
        p = min(self.annealing_step.item() / self.annealing_steps, 1.0)
        if self.annealing_schedule == "linear":
            T = self.T_start * (1 - p) + self.T_end * p
        elif self.annealing_schedule == "exponential":
            T = self.T_start * math.exp(-p * math.log(self.T_start / max(self.T_end, 1e-6)))
        elif self.annealing_schedule == "cosine":
            T = self.T_end + 0.5 * (self.T_start - self.T_end) * (1 + math.cos(math.pi * p))
        else:
            T = self.T_start
        return max(T, self.T_end)

    # Test hook (None by default): ``state_hook(states, where) -> states`` sees the layer-dtype states
    # the entanglement reads (``where``: ("prefill",), ("decode",), or ("mimo",) with the list of
    # per-rank states); bf16 parity tests feed in another implementation's states, because a one-ulp
    # difference of a state is amplified by the cancellation in C = E - S.
    state_hook = None

    # Test hook (None by default): ``mix_hook(te, c, ent, states, where) -> (te, c)`` sees the inputs of
    # state_proj (tanh E) and ent_proj (C = E - S) with the E and S they came from; bf16 parity tests feed
    # in another implementation's values after bounding their difference by a rounding of E.
    mix_hook = None

    # Test hook (None by default): ``gate_hook(y, terms, where) -> y`` sees the out_proj input
    # y = local + gate * sp + ep with its three terms; used like mix_hook.
    gate_hook = None

    # Test hook (None by default): ``tern_hook(scores, tern, where) -> tern`` sees every hard
    # ternary decision with its place (``where``: ("local", t0, t1), ("global",), ("decode",),
    # ("mimo", t, w)); parity tests use it like BitLinear.code_hook.
    tern_hook = None

    def _hard_ternary(self, scores, where=None):
        thr = self.entanglement_threshold
        one = torch.ones_like(scores)
        tern = torch.where(scores > thr, one, torch.where(scores < -thr, -one, torch.zeros_like(scores)))
        if self.tern_hook is not None:
            tern = self.tern_hook(scores, tern, where)
        return tern

    def ternary_entanglement(self, scores, where=None):
        T = self.get_temperature()
        if T > 1.0:
            return F.softmax(scores / T, dim=-1)
        hard = self._hard_ternary(scores, where)
        return scores + (hard - scores).detach()

    # -- RoPE (tesm.py:783-793) --------------------------------------------------
    def _apply_rope(self, x, pos_offset=0):
        D = x.shape[-1]
        half = D // 2
        L = x.shape[1]
        pos = torch.arange(pos_offset, pos_offset + L, device=x.device, dtype=torch.float32)
        idx = torch.arange(half, device=x.device, dtype=torch.float32)
        theta = pos.unsqueeze(1) * (1.0 / (self.rope_base ** (2.0 * idx / D)))
        if x.dim() == 4:
            theta = theta.unsqueeze(1)
        cos_t = theta.cos().unsqueeze(0).to(x.dtype)
        sin_t = theta.sin().unsqueeze(0).to(x.dtype)
        x1, x2 = x[..., :half], x[..., half:]
        return torch.cat([x1 * cos_t - x2 * sin_t, x1 * sin_t + x2 * cos_t], dim=-1)

    # -- state scan (tesm.py:1065-1164) ----------------------------------------
    @staticmethod
    def _parallel_prefix_scan(decay, update, h0):
        A = torch.cumprod(decay, dim=1)
        acc = torch.cumsum(update / A.clamp_min(1e-12), dim=1)
        return A * (h0.unsqueeze(1) + acc)

    def _parallel_state_scan(self, decay, update, prev_state=None):
        B, L, _ = decay.shape
        out_dtype = decay.dtype
        chunk = min(max(self.state_scan_chunk_size, 1), L)
        d64 = decay.to(torch.float64).clamp_min(1e-12)
        u64 = update.to(torch.float64)
        if prev_state is None:
            h = torch.zeros(B, self.d_state, device=decay.device, dtype=torch.float64)
        else:
            h = prev_state.to(torch.float64)
        pieces = []
        for c0 in range(0, L, chunk):
            s = self._parallel_prefix_scan(d64[:, c0:c0 + chunk], u64[:, c0:c0 + chunk], h)
            h = s[:, -1, :].detach()
            pieces.append(s)
        self._last_scan_state_f64 = h
        return torch.cat(pieces, dim=1).to(dtype=out_dtype)

    # -- entanglement (tesm.py:716-744, 853-961, 963-1063) ----------------------
    def _record_map(self, ternary):
        self.last_entanglement_map = ternary.detach() if not self.training else None

    def _compute_local_entanglement(self, q, k, values):
        """Causal sliding-window ternary entanglement (torch branch, tesm.py:921-952)."""
        L = q.shape[1]
        W = min(self.entanglement_window, L)
        blk = min(max(self.entanglement_block_size, 1), L)
        out = torch.empty_like(values)
        rel_bias = self.local_entanglement_bias[-W:].to(dtype=q.dtype).view(1, 1, W)
        offs = torch.arange(W, device=q.device)
        maps = []
        for t0 in range(0, L, blk):
            t1 = min(t0 + blk, L)
            wpos = torch.arange(t0, t1, device=q.device).unsqueeze(1) - (W - 1) + offs.unsqueeze(0)
            gpos = wpos.clamp(min=0, max=L - 1)
            valid = (wpos >= 0).unsqueeze(0)
            kb, vb = k[:, gpos, :], values[:, gpos, :]
            scores = torch.einsum("bqr,bqwr->bqw", q[:, t0:t1, :], kb) / math.sqrt(self.ent_rank)
            scores = scores + rel_bias[:, :, -W:].masked_fill(~valid, 0.0)
            tern = self.ternary_entanglement(scores, ("local", t0, t1)).masked_fill(~valid, 0.0)
            norm = tern.abs().sum(dim=-1, keepdim=True).clamp_min(1.0)
            out[:, t0:t1, :] = torch.einsum("bqw,bqwd->bqd", tern / norm, vb)
            maps.append(tern.detach())
        self._record_map(torch.cat(maps, dim=1))
        return out

    def _global_rel_bias(self, L, dtype, device):  # tesm.py:970-982
        pos = torch.arange(L, device=device, dtype=dtype)
        rel = pos.unsqueeze(1) - pos.unsqueeze(0)
        freq = torch.arange(1, self.global_rel_pos_dim + 1, device=device, dtype=dtype) * math.pi / 1000.0
        ang = rel.unsqueeze(-1) * freq.unsqueeze(0).unsqueeze(0)
        emb = self.global_rel_pos_embed.to(dtype)
        b = (torch.sin(ang) * emb).sum(dim=-1) + (torch.cos(ang) * emb).sum(dim=-1)
        return b * self.global_rel_pos_scale.to(dtype) + self.global_rel_pos_bias.to(dtype)

    def _compute_entanglement(self, q, k, values):
        L = q.size(1)
        if self.entanglement_window > 0:
            return self._compute_local_entanglement(q, k, values)
        rel_bias = self._global_rel_bias(L, q.dtype, q.device)  # tesm.py:1032-1043
        scores = torch.matmul(q, k.transpose(-2, -1)) / math.sqrt(self.ent_rank)
        scores = scores + rel_bias.unsqueeze(0)
        causal = torch.tril(torch.ones(L, L, dtype=torch.bool, device=q.device))
        tern = self.ternary_entanglement(scores, ("global",)) * causal.unsqueeze(0).to(scores.dtype)
        norm = tern.abs().sum(dim=-1, keepdim=True).clamp_min(1.0)
        self._record_map(tern)
        return torch.matmul(tern / norm, values)

    # -- split + gates shared by prefill and decode (tesm.py:1195-1205) ---------
    def _split_gate(self, proj):
        local, sv, decay, write, gate, q, k = torch.split(
            proj, [self.d_model, self.d_state, self.d_state, self.d_state, self.d_model,
                   self.ent_rank, self.ent_rank], dim=-1)
        return (local, torch.tanh(sv), torch.sigmoid(decay + self.decay_bias),
                torch.sigmoid(write), torch.sigmoid(gate), q, k)

    def forward(self, u, inference_params=None, cross_layer_state=None, prev_state=None, **kwargs):
        """Prefill forward (tesm.py:1175-1272); returns ``(y, final_state_f64)``."""
        B, L, _ = u.shape
        if L > self.max_seq_len:
            raise ValueError(f"Sequence length {L} exceeds max_seq_len {self.max_seq_len}")
        if L == 0:
            return u, None
        if inference_params is not None and L == 1:
            cache = inference_params.get("state_cache")
            if cache is not None and "state" in cache:
                return self._forward_incremental(u, inference_params, cross_layer_state)
        local, sv, decay, write, gate, q, k = self._split_gate(self.in_proj(u))
        q = self._apply_rope(q)
        k = self._apply_rope(k)
        if cross_layer_state is not None:  # tesm.py:1213-1218
            cq = self.cross_layer_q_proj(cross_layer_state)
            if cq.dim() == 2:
                cq = cq.unsqueeze(1)
            q = q + cq
        states = self._parallel_state_scan(decay, write * sv, prev_state=prev_state)
        if self.state_hook is not None:
            states = self.state_hook(states, ("prefill",))
        avg = self._compute_entanglement(q, k, states)
        ent = states + self.entanglement_scale * (avg - states)
        change = ent - states
        if inference_params is not None:  # tesm.py:1235-1253
            cache = inference_params.get("state_cache")
            if cache is not None and "state" in cache:
                h = self._last_scan_state_f64
                cache["state"] = (h if h is not None else states[:, -1, :].detach().to(torch.float64)).clone()
                cache["seq_pos"] = L
                W = cache["ent_k_cache"].shape[1]
                if L >= W:
                    cache["ent_k_cache"] = k[:, -W:, :].detach().float()
                    cache["ent_v_cache"] = states[:, -W:, :].detach().float()
                else:
                    cache["ent_k_cache"][:, -L:, :] = k.detach().float()
                    cache["ent_v_cache"][:, -L:, :] = states.detach().float()
                cache["cache_idx"] = 0
        te = torch.tanh(ent)
        if self.mix_hook is not None:
            te, change = self.mix_hook(te, change, ent, states, ("prefill",))
        sp, ep = self.state_proj(te), self.ent_proj(change)
        y = local + gate * sp + ep
        if self.gate_hook is not None:
            y = self.gate_hook(y, (local, gate * sp, ep), ("prefill",))
        y = self.out_proj(self.dropout(y))
        self._last_cross_layer_state = states.detach()
        if self.training and self.annealing_enabled:
            self.annealing_step.add_(1)
        return y, self._last_scan_state_f64

    def allocate_inference_cache(self, batch_size, max_seqlen, dtype=None, **kwargs):  # tesm.py:620-670
        dev = self.out_proj.weight.device
        cdt = dtype or torch.float32
        W = max(self.entanglement_window, 1)
        if kwargs.get("use_paged_cache", False) and max_seqlen > 1024:
            raise NotImplementedError("paged state cache is not restated by the oracle")
        return {
            "use_paged": False,
            "state": torch.zeros(batch_size, self.d_state, device=dev, dtype=torch.float64),
            "seq_pos": 0,
            "ent_k_cache": torch.zeros(batch_size, W, self.ent_rank, device=dev, dtype=cdt),
            "ent_v_cache": torch.zeros(batch_size, W, self.d_state, device=dev, dtype=cdt),
            "cache_idx": 0,
            "cache_filled": False,
        }

    def _ring_window(self, cache, slot_written, valid_len):
        """Ring-buffer slots in the order the reference reads them (tesm.py:1338-1349).

        With a full ring the reference starts at the slot it has just written
        (the local ``cache_idx`` is not advanced), so the newest key comes first
        and meets ``bias[0]``; with a partial ring it reads slots ``0..valid-1``.
        """
        W = cache["ent_k_cache"].shape[1]
        if valid_len >= W:
            idx = torch.arange(slot_written, slot_written + W, device=cache["ent_k_cache"].device) % W
            return cache["ent_k_cache"][:, idx], cache["ent_v_cache"][:, idx]
        return cache["ent_k_cache"][:, :valid_len], cache["ent_v_cache"][:, :valid_len]

    def _forward_incremental(self, u, inference_params, cross_layer_state=None):
        """One-token decode step (tesm.py:1274-1400)."""
        B = u.shape[0]
        cache = inference_params["state_cache"]
        local, sv, decay, write, gate, q, k = self._split_gate(self.in_proj(u))
        pos = cache["seq_pos"]
        qv = self._apply_rope(q, pos_offset=pos)[:, 0, :]
        kv = self._apply_rope(k, pos_offset=pos)[:, 0, :]
        vv = sv[:, 0, :]
        if cross_layer_state is not None:
            qv = qv + self.cross_layer_q_proj(cross_layer_state)
        new64 = decay[:, 0, :].double() * cache["state"] + write[:, 0, :].double() * vv.double()
        new = new64.to(decay.dtype)
        if self.state_hook is not None:
            new = self.state_hook(new, ("decode",))
        W = cache["ent_k_cache"].shape[1]
        slot = cache.get("cache_idx", 0)
        cache["ent_k_cache"][:, slot, :] = kv
        cache["ent_v_cache"][:, slot, :] = new
        cache["cache_idx"] = (slot + 1) % W
        valid = min(cache["seq_pos"] + 1, W)
        k_eff, v_eff = self._ring_window(cache, slot, valid)
        zdt = cache["ent_k_cache"].dtype
        if self.amend_bf16 and k_eff.dtype != qv.dtype:
            k_eff, v_eff, zdt = k_eff.to(qv.dtype), v_eff.to(qv.dtype), qv.dtype
        scores = torch.einsum("br,bwr->bw", qv, k_eff) / (self.ent_rank ** 0.5)
        if self.local_entanglement_bias is not None:
            scores = scores + self.local_entanglement_bias[-valid:].to(dtype=scores.dtype, device=scores.device)
        if valid < W:
            full = torch.zeros(B, W, device=scores.device, dtype=zdt)
            full[:, W - valid:] = scores
            scores = full
        tern = self.ternary_entanglement(scores, ("decode",))
        if valid < W:
            tern[:, :W - valid] = 0.0
        norm = tern.abs().sum(dim=-1, keepdim=True).clamp_min(1.0)
        if valid < W:
            fv = torch.zeros(B, W, self.d_state, device=v_eff.device, dtype=v_eff.dtype)
            fv[:, W - valid:] = v_eff
            v_eff = fv
        avg = torch.einsum("bw,bwd->bd", tern / norm, v_eff)
        ent = new + self.entanglement_scale * (avg - new)
        change = ent - new
        cache["state"] = new64.detach()
        cache["seq_pos"] += 1
        te = torch.tanh(ent)
        if self.mix_hook is not None:
            te, change = self.mix_hook(te, change, ent, new, ("decode",))
        sp, ep = self.state_proj(te), self.ent_proj(change)
        y = local[:, 0, :] + gate[:, 0, :] * sp + ep
        if self.gate_hook is not None:
            y = self.gate_hook(y, (local[:, 0, :], gate[:, 0, :] * sp, ep), ("decode",))
        y = self.out_proj(y.unsqueeze(1))
        self._last_cross_layer_state = new.detach()
        return y, new64.detach()


TESM = TESM_SISO


# ---------------------------------------------------------------------------
# TESMMIMO_Optimized  (tesm_ssm/modules/tesm_mimo.py:76-1062)
# ---------------------------------------------------------------------------
class TESMMIMO_Optimized(TESM_SISO):
    """Multi-head TESM layer with MIMO rank expansion, torch path."""

    def __init__(self, d_model, d_state=256, n_heads=4, mimo_rank=4, expand=2, ent_rank=48,
                 entanglement_window=16, max_seq_len=2048, entanglement_threshold=0.5, dropout=0.0,
                 bit_eps=1e-5, bit_threshold=0.5, kernel_backend="torch", annealing_enabled=True,
                 T_start=10.0, T_end=0.1, annealing_steps=1000, annealing_schedule="cosine", **kwargs):
        # The parent is built without kernel_backend (tesm_mimo.py:119-136) and its
        # in/state/ent projections and biases are then replaced; they still consume RNG.
        super().__init__(d_model=d_model, d_state=d_state, expand=expand, ent_rank=ent_rank,
                         entanglement_window=entanglement_window, max_seq_len=max_seq_len,
                         entanglement_threshold=entanglement_threshold, dropout=dropout,
                         bit_eps=bit_eps, bit_threshold=bit_threshold,
                         annealing_enabled=annealing_enabled, T_start=T_start, T_end=T_end,
                         annealing_steps=annealing_steps, annealing_schedule=annealing_schedule,
                         **kwargs)
        dev, dt = kwargs.get("device"), kwargs.get("dtype")
        self.n_heads = n_heads
        self.mimo_rank = mimo_rank
        self.d_inner = int(expand * d_model)
        self.d_head = self.d_inner // n_heads
        self.d_state_total = d_state * n_heads
        self.kernel_backend = kernel_backend
        self.decay_bias = nn.Parameter(torch.full((n_heads, d_state), float(kwargs.get("decay_init_bias", 3.0)),
                                                  device=dev, dtype=torch.float32))
        if entanglement_window > 0:  # tesm_mimo.py:160-165
            self.local_entanglement_bias = nn.Parameter(
                torch.randn(n_heads, entanglement_window, device=dev, dtype=torch.float32) * 0.02)
        else:
            self.register_parameter("local_entanglement_bias", None)
        self.rope_base = float(kwargs.get("rope_base", 10000.0))
        ones = torch.ones(n_heads, mimo_rank, d_state, device=dev, dtype=torch.float32)
        self.mimo_x = nn.Parameter(ones / mimo_rank)
        self.mimo_z = nn.Parameter(ones.clone())
        self.mimo_o = nn.Parameter(ones / mimo_rank)
        bl = dict(bias=False, bit_eps=bit_eps, bit_threshold=bit_threshold,
                  kernel_backend=kernel_backend, device=dev, dtype=dt)
        n_proj = 2 * d_model + 3 * d_state * n_heads + 2 * ent_rank * n_heads  # tesm_mimo.py:194
        self.in_proj = BitLinear(d_model, n_proj, **bl)
        self.state_proj = BitLinear(self.d_state_total, d_model, **bl)
        self.ent_proj = BitLinear(self.d_state_total, d_model, **bl)

    def _scan_mimo(self, decay, update):
        """Sequential recurrence in the inputs' promoted dtype (tesm_mimo.py:375-392)."""
        B, L, H, D = decay.shape
        dflat = decay.permute(0, 2, 1, 3).reshape(B * H, L, D)
        uflat = update.permute(0, 2, 1, 3).reshape(B * H, L, D)
        h = torch.zeros(B * H, D, device=decay.device, dtype=decay.dtype)
        rows = []
        for t in range(L):
            h = dflat[:, t] * h + uflat[:, t]
            rows.append(h.unsqueeze(1))
        return torch.cat(rows, dim=1).reshape(B, H, L, D).permute(0, 2, 1, 3)

    def _local_ent_mimo(self, q, k, v, bias):
        """Per-head window entanglement with the reference's early-window
        truncation (tesm_mimo.py:525-588): for t < W-1 the loop runs w < t+1 and
        keys ``t-W+1+w < 0`` are skipped."""
        B, L, H, R = q.shape
        W = self.entanglement_window
        T = self.get_temperature()
        out = torch.zeros_like(v)
        for t in range(L):
            terms, vals = [], []
            for w in range(min(W, t + 1)):
                j = t - W + 1 + w
                if j < 0:
                    continue
                s = (q[:, t] * k[:, j]).sum(dim=-1) / math.sqrt(R) + bias[:, w]
                terms.append(s if T > 1.0 else self.ternary_entanglement(s, ("mimo", t, w)))
                vals.append(v[:, j])
            if not terms:
                continue
            st = torch.stack(terms, dim=-1)
            if T > 1.0:
                wts = F.softmax(st / T, dim=-1)
            else:
                wts = st / st.abs().sum(dim=-1, keepdim=True).clamp_min(1.0)
            for i, vj in enumerate(vals):
                out[:, t] += wts[:, :, i:i + 1] * vj
        return out

    def _global_ent_mimo(self, q, k, states):  # tesm_mimo.py:590-687 (torch branch)
        B, L, H, R = q.shape
        D = states.shape[-1]
        rel_bias = self._global_rel_bias(L, q.dtype, q.device)
        scores = torch.matmul(q.reshape(B, L, H * R), k.reshape(B, L, H * R).transpose(-2, -1)) / math.sqrt(H * R)
        scores = scores + rel_bias.unsqueeze(0)
        causal = torch.tril(torch.ones(L, L, dtype=torch.bool, device=q.device))
        tern = self.ternary_entanglement(scores, ("global",)) * causal.unsqueeze(0).to(scores.dtype)
        norm = tern.abs().sum(dim=-1, keepdim=True).clamp_min(1.0)
        w = tern / norm
        if self.amend_bf16 and w.dtype != states.dtype:  # bf16 weights against float32 rank states
            w = w.to(states.dtype)
        ent = torch.matmul(w, states.reshape(B, L, H * D)).reshape(B, L, H, D)
        self._record_map(tern)
        return ent, ent - states

    def _update_entanglement_stats_mimo(self, q, k):
        """tesm_mimo.py:458-523: hard-threshold ternary statistics of the first positions (q, k RoPE'd)."""
        with torch.no_grad():
            B, L, H, R = q.shape
            W = min(self.entanglement_window, L) if self.entanglement_window > 0 else L
            thr = self.entanglement_threshold
            if self.entanglement_window == 0:  # :469-482, sampled global scores
                n = min(L, 32)
                scores = torch.einsum("bshr,bthr->bst", q[:, :n], k[:, :n]) / math.sqrt(R)
            else:  # :483-503
                n = min(L, 64)
                qs, ks = q[:, :n], k[:, :n]
                kw = ks.unfold(1, W, 1)  # (B, n-W+1, H, R, W)
                V = kw.size(1)
                qv = qs[:, W - 1:W - 1 + V]
                scores = (qv.unsqueeze(-1) * kw).sum(dim=-2) / math.sqrt(R)
            tern = torch.where(scores > thr, torch.ones_like(scores),
                               torch.where(scores < -thr, -torch.ones_like(scores), torch.zeros_like(scores)))
            total = float(tern.numel())
            if total > 0:  # :506-519
                flat = tern.detach().flatten()
                self._ternary_stats_for_logging = (flat, total)
                self._stats_ternary_buffer = flat
                self._stats_total_buffer = torch.tensor(total, device=tern.device)
                self.last_entanglement_stats = {
                    "positive": float((tern > 0).sum().item()) / total,
                    "negative": float((tern < 0).sum().item()) / total,
                    "zero": float((tern == 0).sum().item()) / total,
                }
            else:
                self._ternary_stats_for_logging = None
                self._stats_ternary_buffer = None
                self.last_entanglement_stats = None

    def _split_heads(self, proj, B, L):
        H, D, R = self.n_heads, self.d_state, self.ent_rank
        local, sv, decay, write, gate, q, k = torch.split(
            proj, [self.d_model, D * H, D * H, D * H, self.d_model, R * H, R * H], dim=-1)
        decay = torch.sigmoid(decay.view(B, L, H, D) + self.decay_bias.unsqueeze(0).unsqueeze(0))
        write = torch.sigmoid(write.view(B, L, H, D))
        sv = torch.tanh(sv.view(B, L, H, D))
        return local, sv, decay, write, torch.sigmoid(gate), q.view(B, L, H, R), k.view(B, L, H, R)

    def _to_proj_dtype(self, x, proj):
        if self.amend_bf16 and x.dtype != proj.weight.dtype:
            return x.to(proj.weight.dtype)
        return x

    def forward(self, u, inference_params=None, cross_layer_state=None, prev_state=None, **kwargs):
        """Prefill forward (tesm_mimo.py:914-1062)."""
        B, L, _ = u.shape
        if inference_params is not None and L == 1:
            cache = inference_params.get("state_cache")
            if cache is not None and "state" in cache:
                return self._forward_incremental(u, inference_params, cross_layer_state)
        local, sv, decay, write, gate, q, k = self._split_heads(self.in_proj(u), B, L)
        Rm = self.mimo_rank
        sv_m = torch.einsum("blhd,hrd->blrhd", sv.float(), self.mimo_x.float())
        wr_m = torch.einsum("blhd,hrd->blrhd", write.float(), self.mimo_x.float())
        upd = wr_m * sv_m
        states_r = [self._scan_mimo(decay, upd[:, :, r].contiguous()) for r in range(Rm)]
        if self.state_hook is not None:
            states_r = self.state_hook(states_r, ("mimo",))
        finals = [s[:, -1] for s in states_r]
        states_m = torch.stack(states_r, dim=2)
        q = self._apply_rope(q)
        k = self._apply_rope(k)
        ents, changes = [], []
        for r in range(Rm):
            s = states_m[:, :, r].contiguous()
            if self.entanglement_window > 0 and self.local_entanglement_bias is not None:
                a = self._local_ent_mimo(q, k, s, self.local_entanglement_bias)
                e = s + self.entanglement_scale * (a - s)
                c = e - s
            else:
                e, c = self._global_ent_mimo(q, k, s)
            ents.append(e.unsqueeze(2))
            changes.append(c.unsqueeze(2))
        ent = torch.einsum("blrhd,hrd->blhd", torch.cat(ents, dim=2).float(), self.mimo_o.float())
        chg = torch.einsum("blrhd,hrd->blhd", torch.cat(changes, dim=2).float(), self.mimo_o.float())
        self._update_entanglement_stats_mimo(q, k)  # tesm_mimo.py:1019-1020
        if inference_params is not None:  # tesm_mimo.py:1022-1037
            cache = inference_params.get("state_cache")
            if cache is not None and "state" in cache:
                cache["state"] = finals[0].detach().to(torch.float64).clone()
                cache["seq_pos"] = L
                W = cache["ent_k_cache"].shape[1]
                if L >= W:
                    cache["ent_k_cache"] = k[:, -W:].detach().float()
                    cache["ent_v_cache"] = states_m[:, -W:, 0].detach().float()
                else:
                    cache["ent_k_cache"][:, -L:] = k.detach().float()
                    cache["ent_v_cache"][:, -L:] = states_m[:, -L:, 0].detach().float()
                cache["cache_idx"] = 0
        HD = self.n_heads * self.d_state
        ent_flat = ent.reshape(B, L, HD).contiguous()
        chg_flat = chg.reshape(B, L, HD).contiguous()
        te = self._to_proj_dtype(torch.tanh(ent_flat), self.state_proj)
        ce = self._to_proj_dtype(chg_flat, self.ent_proj)
        if self.mix_hook is not None:
            te, ce = self.mix_hook(te, ce, ent_flat, None, ("mimo",))
        sp = self.state_proj(te)
        ep = self.ent_proj(ce)
        yg = local + gate * sp + ep
        if self.gate_hook is not None:
            yg = self.gate_hook(yg, (local, gate * sp, ep), ("mimo",))
        y = self.out_proj(self.dropout(yg))
        self._last_cross_layer_state = states_m[:, -1, 0].detach()
        if self.training and self.annealing_enabled:
            self.annealing_step.add_(1)
        return y, (finals[0].detach().to(torch.float64) if finals else None)

    def allocate_inference_cache(self, batch_size, max_seqlen, dtype=None, **kwargs):  # tesm_mimo.py:689-731
        dev = self.out_proj.weight.device
        cdt = dtype or torch.float32
        W = max(self.entanglement_window, 1)
        H = self.n_heads
        return {
            "use_paged": False,
            "state": torch.zeros(batch_size, H, self.d_state, device=dev, dtype=torch.float64),
            "seq_pos": 0,
            "ent_k_cache": torch.zeros(batch_size, W, H, self.ent_rank, device=dev, dtype=cdt),
            "ent_v_cache": torch.zeros(batch_size, W, H, self.d_state, device=dev, dtype=cdt),
            "cache_idx": 0,
            "cache_filled": False,
        }

    def _forward_incremental(self, u, inference_params, cross_layer_state=None):
        """One-token MIMO decode step (tesm_mimo.py:753-912)."""
        B = u.shape[0]
        H, D, R = self.n_heads, self.d_state, self.ent_rank
        cache = inference_params["state_cache"]
        local, sv, decay, write, gate, q, k = self._split_heads(self.in_proj(u), B, 1)
        pos = cache["seq_pos"]
        qr = self._apply_rope(q, pos_offset=pos)
        kr = self._apply_rope(k, pos_offset=pos)
        if cross_layer_state is not None:
            if cross_layer_state.dim() == 3:
                cq = self.cross_layer_q_proj(cross_layer_state.reshape(B * H, D)).view(B, H, R)
            else:
                B2, L2, H2, _ = cross_layer_state.shape
                cq = self.cross_layer_q_proj(cross_layer_state.reshape(B2 * L2 * H2, D)).view(B2, L2, H2, R)
            qr = qr + cq.unsqueeze(1)
        new64 = decay[:, 0].double() * cache["state"] + write[:, 0].double() * sv[:, 0].double()
        new = new64.to(decay.dtype)
        if self.state_hook is not None:
            new = self.state_hook(new, ("decode",))
        W = cache["ent_k_cache"].shape[1]
        slot = cache.get("cache_idx", 0)
        cache["ent_k_cache"][:, slot] = kr[:, 0]
        cache["ent_v_cache"][:, slot] = new
        cache["cache_idx"] = (slot + 1) % W
        valid = min(cache["seq_pos"] + 1, W)
        k_eff, v_eff = self._ring_window(cache, slot, valid)
        qv = qr[:, 0]
        if self.amend_bf16 and k_eff.dtype != qv.dtype:
            k_eff, v_eff = k_eff.to(qv.dtype), v_eff.to(qv.dtype)
        scores = torch.einsum("bhr,bwhr->bhw", qv, k_eff) / (R ** 0.5)
        if self.local_entanglement_bias is not None:
            scores = scores + self.local_entanglement_bias[:, -valid:].to(dtype=scores.dtype).unsqueeze(0)
        if valid < W:
            full = scores.new_zeros(B, H, W)
            full[:, :, W - valid:] = scores
            scores = full
        tern = self.ternary_entanglement(scores, ("decode",))
        if valid < W:
            tern[:, :, :W - valid] = 0.0
        norm = tern.abs().sum(dim=-1, keepdim=True).clamp_min(1.0)
        if valid < W:
            fv = v_eff.new_zeros(B, W, H, D)
            fv[:, W - valid:] = v_eff
            v_eff = fv
        avg = torch.einsum("bhw,bwhd->bhd", tern / norm, v_eff)
        ent = new + self.entanglement_scale * (avg - new)
        change = ent - new
        cache["state"] = new64.detach()
        cache["seq_pos"] += 1
        te = torch.tanh(ent.reshape(B, H * D))
        ce = change.reshape(B, H * D)
        if self.mix_hook is not None:
            te, ce = self.mix_hook(te, ce, ent.reshape(B, H * D), new.reshape(B, H * D), ("decode",))
        sp = self.state_proj(te)
        ep = self.ent_proj(ce)
        yg = local[:, 0] + gate[:, 0] * sp + ep
        if self.gate_hook is not None:
            yg = self.gate_hook(yg, (local[:, 0], gate[:, 0] * sp, ep), ("decode",))
        y = self.out_proj(yg.unsqueeze(1))
        self._last_cross_layer_state = new.detach()
        return y, new64.detach()


# ---------------------------------------------------------------------------
# LM harness around the layers (block.py:7-50, mixer_seq_simple.py:25-345, 790-803)
# ---------------------------------------------------------------------------
class RMSNorm(nn.Module):
    def __init__(self, dim, eps=1e-5):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim))

    def forward(self, x):
        return x * torch.rsqrt(x.pow(2).mean(dim=-1, keepdim=True) + self.eps) * self.weight


class Block(nn.Module):
    def __init__(self, dim, mixer, mlp, eps, residual_in_fp32=True):
        super().__init__()
        self.residual_in_fp32 = residual_in_fp32
        self.norm = RMSNorm(dim, eps=eps)
        self.mixer = mixer(dim)
        self.norm2 = RMSNorm(dim, eps=eps)
        self.mlp = mlp(dim)

    def forward(self, hidden, residual=None, inference_params=None, prev_state=None, **mixer_kwargs):
        residual = hidden + residual if residual is not None else hidden
        hidden = self.norm(residual.to(dtype=self.norm.weight.dtype))
        if self.residual_in_fp32:
            residual = residual.to(torch.float32)
        out = self.mixer(hidden, inference_params=inference_params, prev_state=prev_state, **mixer_kwargs)
        hidden, final = out if isinstance(out, tuple) else (out, None)
        residual = hidden + residual
        hidden = self.norm2(residual.to(dtype=self.norm2.weight.dtype))
        if self.residual_in_fp32:
            residual = residual.to(torch.float32)
        return self.mlp(hidden), residual, final


class FeedForward(nn.Module):
    """Gate/up/down BitLinears; gate and up share one projection (mixer_seq_simple.py:25-67)."""

    def __init__(self, cfg, device=None, dtype=None):
        super().__init__()
        bl = dict(bias=False, bit_eps=cfg.bit_eps, bit_threshold=cfg.bit_threshold,
                  kernel_backend=cfg.kernel_backend, kernel_mode=cfg.kernel_mode, device=device, dtype=dtype)
        self.gate_proj = BitLinear(cfg.d_model, cfg.d_intermediate, **bl)
        self.up_proj = BitLinear(cfg.d_model, cfg.d_intermediate, **bl)
        self.down_proj = BitLinear(cfg.d_intermediate, cfg.d_model, **bl)
        self.dropout = nn.Dropout(cfg.dropout)

    def forward(self, x):
        qx = self.gate_proj.quantized_input(x)
        w = torch.cat([self.gate_proj._current_quantized_weight(), self.up_proj._current_quantized_weight()], dim=0)
        g, u = torch.split(self.gate_proj._project_quantized(qx, w, None),
                           [self.gate_proj.out_features, self.up_proj.out_features], dim=-1)
        return self.dropout(self.down_proj(F.silu(g) * u))


def _init_weights(module, std):
    """mixer_seq_simple.py:790-803; the residual rescale never fires (Q17)."""
    if isinstance(module, nn.Linear):
        if module.bias is not None:
            nn.init.zeros_(module.bias)
        nn.init.normal_(module.weight, std=std)
    elif isinstance(module, (BitLinear, nn.Embedding)):
        nn.init.normal_(module.weight, std=std)


class MixerModel(nn.Module):
    def __init__(self, cfg, device=None, dtype=None, mixer_factory=None, mlp_factory=None):
        super().__init__()
        self.config = cfg
        self.embedding = nn.Embedding(cfg.vocab_size, cfg.d_model, device=device, dtype=dtype)
        self.position_embedding = nn.Embedding(cfg.max_seq_len, cfg.d_model, device=device, dtype=dtype)
        mixer_factory = mixer_factory or _default_mixer(cfg, device, dtype)
        mlp_factory = mlp_factory or (lambda dim: FeedForward(cfg, device=device, dtype=dtype))
        self.layers = nn.ModuleList([
            Block(cfg.d_model, mixer_factory(i), mlp_factory, eps=cfg.norm_epsilon,
                  residual_in_fp32=cfg.residual_in_fp32) for i in range(cfg.n_layer)])
        self.norm_f = RMSNorm(cfg.d_model, eps=cfg.norm_epsilon)
        self.apply(lambda m: _init_weights(m, cfg.initializer_range))

    def forward(self, input_ids, inference_params=None, prev_states=None, record_mixer_outputs=None):
        B, L = input_ids.shape
        if L == 0:
            raise ValueError("Input sequence length is 0")
        if L > self.config.max_seq_len:
            raise ValueError(f"Sequence length {L} exceeds max_seq_len {self.config.max_seq_len}")
        off = 0
        if inference_params is not None and L == 1 and "state_cache" in inference_params:
            c0 = inference_params["state_cache"].get(0)
            if c0 is not None and "seq_pos" in c0:
                off = c0["seq_pos"]
        pos = torch.arange(off, off + L, device=input_ids.device).unsqueeze(0).expand(B, -1)
        hidden = self.embedding(input_ids) + self.position_embedding(pos)
        residual, cross, finals = None, None, []
        for i, layer in enumerate(self.layers):
            lip = None
            if inference_params is not None and "state_cache" in inference_params:
                lc = inference_params["state_cache"].get(i)
                if lc is not None:
                    lip = {"state_cache": lc}
            if record_mixer_outputs is not None:
                _hook = layer.mixer.register_forward_hook(
                    lambda m, a, out: record_mixer_outputs.append(out[0].detach().clone()))
            hidden, residual, final = layer(hidden, residual, inference_params=lip,
                                            prev_state=prev_states[i] if prev_states is not None else None,
                                            cross_layer_state=cross)
            if record_mixer_outputs is not None:
                _hook.remove()
            if final is not None:
                finals.append(final)
            cross = getattr(layer.mixer, "_last_cross_layer_state", None)
        residual = hidden + residual if residual is not None else hidden
        return self.norm_f(residual.to(dtype=self.norm_f.weight.dtype)), finals


def _default_mixer(cfg, device, dtype):
    def make(i):
        def build(dim):
            if cfg.use_mimo:
                return TESMMIMO_Optimized(
                    d_model=dim, n_heads=cfg.n_heads, d_state=cfg.d_state, expand=cfg.expand,
                    ent_rank=cfg.ent_rank, entanglement_window=cfg.entanglement_window,
                    entanglement_threshold=cfg.entanglement_threshold,
                    entanglement_scale=cfg.entanglement_scale, max_seq_len=cfg.max_seq_len,
                    dropout=cfg.dropout, bit_eps=cfg.bit_eps, bit_threshold=cfg.bit_threshold,
                    kernel_backend=cfg.kernel_backend, annealing_enabled=cfg.annealing_enabled,
                    T_start=cfg.T_start, T_end=cfg.T_end, annealing_steps=cfg.annealing_steps,
                    annealing_schedule=cfg.annealing_schedule, device=device, dtype=dtype)
            return TESM_SISO(
                d_model=dim, d_state=cfg.d_state, expand=cfg.expand, ent_rank=cfg.ent_rank,
                entanglement_scale=cfg.entanglement_scale,
                entanglement_threshold=cfg.entanglement_threshold,
                entanglement_window=cfg.entanglement_window,
                entanglement_block_size=cfg.entanglement_block_size,
                entanglement_init=cfg.entanglement_init, layer_idx=i, max_seq_len=cfg.max_seq_len,
                dropout=cfg.dropout, bit_eps=cfg.bit_eps, bit_threshold=cfg.bit_threshold,
                kernel_backend=cfg.kernel_backend, kernel_mode=cfg.kernel_mode,
                state_scan_chunk_size=cfg.state_scan_chunk_size, decay_init_bias=cfg.decay_init_bias,
                rope_base=getattr(cfg, "rope_base", 10000.0), annealing_enabled=cfg.annealing_enabled,
                T_start=cfg.T_start, T_end=cfg.T_end, annealing_steps=cfg.annealing_steps,
                annealing_schedule=cfg.annealing_schedule, device=device, dtype=dtype)
        return build
    return make


class TESMLMHeadModel(nn.Module):
    """Embeddings -> layers -> norm -> tied LM head (mixer_seq_simple.py:245-345).

    Only the plain-logits branch is restated (vocabulary suppression is off by
    default); the co-occurrence buffers consume no RNG and are not allocated.
    """

    def __init__(self, cfg, device=None, dtype=None, **factories):
        super().__init__()
        self.tesm_config = cfg
        self.backbone = MixerModel(cfg, device=device, dtype=dtype, **factories)
        self.lm_head = nn.Linear(cfg.d_model, cfg.vocab_size, bias=False, device=device, dtype=dtype)
        if cfg.tie_embeddings:
            self.lm_head.weight = self.backbone.embedding.weight

    def forward(self, input_ids, inference_params=None, prev_states=None, record_mixer_outputs=None):
        hidden, finals = self.backbone(input_ids, inference_params=inference_params,
                                       prev_states=prev_states, record_mixer_outputs=record_mixer_outputs)
        return self.lm_head(hidden), finals
