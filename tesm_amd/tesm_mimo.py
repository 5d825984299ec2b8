"""TESMMIMO_Optimized with ``kernel_backend='hip'``.

Constructor, parameter names, creation order and forward signature follow the reference's
TESMMIMO_Optimized (tesm_ssm/modules/tesm_mimo.py:76-208, 914-1062): the TESM_SISO parent is
built first (its in/state/ent projections and biases still consume the RNG), then the per-head
decay bias, the (n_heads, window) local bias, mimo_x / mimo_z / mimo_o and the MIMO-shaped
in_proj / state_proj / ent_proj replace them.  A module built under the same seed holds the same
parameters.

The prefill forward is one call into ``tesm_hip_mimo_prefill``, which runs the ranks collapsed:
the reference scans and entangles mimo_rank scaled copies of each head's update and merges them
with mimo_o; both steps are linear in the update and the window weights do not depend on the
rank, so one float32 scan, one window mix and a per-channel merge factor
c = sum_r mimo_x_r^2 * mimo_o_r give the same tensors (the rank-0 states, which the reference
returns and caches, are x0^2 times the rank-free ones).
"""
from __future__ import annotations

import ctypes

import torch
import torch.nn as nn

from . import _lib, hip_ops
from .bitlinear import BitLinear, check_hip_call
from .tesm import TESM_SISO, workspace


class TESMMIMO_Optimized(TESM_SISO):
    def __init__(self, d_model, d_state=256, n_heads=4, mimo_rank=4, expand=2, ent_rank=48, entanglement_window=16,
                 max_seq_len=2048, entanglement_threshold=0.5, dropout=0.0, bit_eps=1e-5, bit_threshold=0.5,
                 kernel_backend="hip", annealing_enabled=True, T_start=10.0, T_end=0.1, annealing_steps=1000,
                 annealing_schedule="cosine", **kwargs):
        # the parent is built without kernel_backend (tesm_mimo.py:119-136)
        super().__init__(d_model=d_model, d_state=d_state, expand=expand, ent_rank=ent_rank,
                         entanglement_window=entanglement_window, max_seq_len=max_seq_len,
                         entanglement_threshold=entanglement_threshold, dropout=dropout, bit_eps=bit_eps,
                         bit_threshold=bit_threshold, annealing_enabled=annealing_enabled, T_start=T_start,
                         T_end=T_end, annealing_steps=annealing_steps, annealing_schedule=annealing_schedule,
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
        bl = dict(bias=False, bit_eps=bit_eps, bit_threshold=bit_threshold, kernel_backend=kernel_backend,
                  device=dev, dtype=dt)
        n_proj = 2 * d_model + 3 * d_state * n_heads + 2 * ent_rank * n_heads  # tesm_mimo.py:194
        self.in_proj = BitLinear(d_model, n_proj, **bl)
        self.state_proj = BitLinear(self.d_state_total, d_model, **bl)
        self.ent_proj = BitLinear(self.d_state_total, d_model, **bl)
        self._coef_cache = None
        self._stats_totals = {}

    # -- entanglement statistics (tesm_mimo.py:458-523) --------------------------------
    # The forward leaves the per-row counts on the device; the dict the reference fills with three
    # .item() calls is formed when the attribute is first read, so a forward never waits on the host.
    @property
    def last_entanglement_stats(self):
        pending = self.__dict__.get("_stats_pending")
        if pending is not None:
            counts, total = pending
            pos, neg, zero = (int(v) for v in counts.cpu().sum(dim=0).tolist())
            self.__dict__["_stats_value"] = {"positive": pos / total, "negative": neg / total, "zero": zero / total}
            self.__dict__["_stats_pending"] = None
        return self.__dict__.get("_stats_value")

    @last_entanglement_stats.setter
    def last_entanglement_stats(self, value):
        self.__dict__["_stats_value"] = value
        self.__dict__["_stats_pending"] = None

    def _stats_buffers(self, B, L, dt, dev):
        """Ternary and per-row counts for the statistics: window branch (B, V, n_heads, W) over the first
        min(L, 64) positions, V = min(L, 64) - min(window, L) + 1 complete windows (tesm_mimo.py:465,
        485-490); global branch (B, S, S) over the first S = min(L, 32) positions (:469-482)."""
        counts = torch.empty((B, 3), dtype=torch.int32, device=dev)
        if self.entanglement_window <= 0:
            S = min(L, 32)
            return torch.empty((B, S, S), dtype=dt, device=dev), counts
        W = min(self.entanglement_window, L)
        S = min(L, 64)
        if W > S:  # the reference's unfold (tesm_mimo.py:487) raises here
            raise RuntimeError(f"maximum size for tensor at dimension 1 is {S} but size is {W}")
        tern = torch.empty((B, S - W + 1, self.n_heads, W), dtype=dt, device=dev)
        return tern, counts

    # -- cached device constants ---------------------------------------------------
    def _mimo_coef(self, dtype):
        """(coef, x0sq), each (n_heads, d_state) float32, recomputed when mimo_x / mimo_o change."""
        x, o = self.mimo_x, self.mimo_o
        if x.dtype != dtype or o.dtype != dtype:
            raise RuntimeError(f"mimo_x / mimo_o are {x.dtype} but activations are {dtype}: convert the whole module "
                               f"with module.to({dtype})")
        key = (x._version, x.data_ptr(), o._version, o.data_ptr(), dtype)
        if self._coef_cache is None or self._coef_cache[0] != key:
            H, Rm, D = x.shape
            coef = torch.empty(H, D, dtype=torch.float32, device=x.device)
            x0sq = torch.empty(H, D, dtype=torch.float32, device=x.device)
            xc, oc = x.detach().contiguous(), o.detach().contiguous()
            hip_ops.require_device(xc, oc, coef, x0sq)
            lib = _lib.load()
            _lib.check(lib.tesm_hip_mimo_coef(xc.data_ptr(), oc.data_ptr(), hip_ops.dt_code(dtype), H, Rm, D,
                                              coef.data_ptr(), x0sq.data_ptr(),
                                              ctypes.c_void_p(torch.cuda.current_stream(x.device).cuda_stream)))
            self._coef_cache = (key, coef, x0sq)
        return self._coef_cache[1], self._coef_cache[2]

    # -- forward ---------------------------------------------------------------------
    def forward(self, u, inference_params=None, cross_layer_state=None, prev_state=None, **kwargs):
        """Prefill forward (tesm_mimo.py:914-1062); returns ``(y, rank-0 final state float64)``.
        ``cross_layer_state`` and ``prev_state`` are accepted and unused, as in the reference."""
        B, L, dm = u.shape
        if L == 0:
            return u, None
        check_hip_call(self.kernel_backend, "TESMMIMO", self, u)
        if inference_params is not None and L == 1:
            cache = inference_params.get("state_cache")
            if cache is not None and "state" in cache:
                return self._forward_incremental(u, inference_params, cross_layer_state)
        cache = None
        if inference_params is not None:
            cache = inference_params.get("state_cache")
            if cache is None or "state" not in cache:
                cache = None
        dt = u.dtype
        H, D, R = self.n_heads, self.d_state, self.ent_rank
        dev = u.device
        for p in (self.in_proj, self.state_proj, self.ent_proj, self.out_proj):
            if p.weight.dtype != dt:
                raise RuntimeError(f"expected both operands to have the same dtype, got {dt} and {p.weight.dtype}")
        u = u.contiguous()
        y = torch.empty((B, L, dm), dtype=dt, device=dev)
        h_final = torch.empty((B, H, D), dtype=torch.float64, device=dev)
        last = torch.empty((B, H, D), dtype=torch.float32, device=dev)
        decay_bias = self._decay_bias_dt(dt).contiguous()
        glob = self.entanglement_window <= 0
        local_bias = None if glob else self._local_bias_f32(dt)
        gparams = self._global_params_f32(dt) if glob else None
        rope = self.rope_table(L, dt, dev)
        coef, x0sq = self._mimo_coef(dt)
        hip_ops.require_device(u, decay_bias, local_bias, rope, coef, x0sq, y, h_final, last,
                               *(gparams if gparams is not None else ()))
        lib = _lib.load()
        desc = _lib.MimoLayer()
        desc.dt = hip_ops.dt_code(dt)
        desc.B, desc.L, desc.d_model, desc.d_state, desc.n_heads = B, L, dm, D, H
        desc.ent_rank, desc.window = R, max(self.entanglement_window, 0)
        desc.bit_eps = self.in_proj.bit_eps
        desc.thr = hip_ops.round_dtype(self.entanglement_threshold, dt)
        desc.ent_scale = float(self.entanglement_scale)
        desc.u = u.data_ptr()
        desc.in_proj = self.in_proj.linear_desc()
        desc.state_proj = self.state_proj.linear_desc()
        desc.ent_proj = self.ent_proj.linear_desc()
        desc.out_proj = self.out_proj.linear_desc()
        desc.decay_bias = decay_bias.data_ptr()
        desc.local_bias = local_bias.data_ptr() if local_bias is not None else None
        if gparams is not None:
            emb, scale, bias = gparams
            desc.global_embed, desc.global_dim = emb.data_ptr(), emb.numel()
            desc.global_scale, desc.global_bias = scale.data_ptr(), bias.data_ptr()
        desc.rope = rope.data_ptr()
        desc.mimo_coef, desc.mimo_x0sq = coef.data_ptr(), x0sq.data_ptr()
        desc.y = y.data_ptr()
        desc.h_final = h_final.data_ptr()
        desc.last_state = last.data_ptr()
        stern, scount = self._stats_buffers(B, L, dt, dev)
        desc.stats_ternary, desc.stats_counts = stern.data_ptr(), scount.data_ptr()
        k_cache = v_cache = None
        if cache is not None:
            k_cache, v_cache = self._mimo_cache_buffers(cache, B, L, dev)
            desc.k_cache, desc.v_cache = k_cache.data_ptr(), v_cache.data_ptr()
            desc.cache_dt = hip_ops.dt_code(k_cache.dtype)
            desc.cache_window = k_cache.shape[1]
        nbytes = int(lib.tesm_hip_mimo_prefill_ws_bytes(ctypes.byref(desc)))
        with torch.cuda.device(dev):
            ws = workspace(dev, nbytes)
            _lib.check(lib.tesm_hip_mimo_prefill(ctypes.byref(desc), ctypes.c_void_p(ws.data_ptr()), ws.numel(),
                                                 ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)))
        if cache is not None:  # tesm_mimo.py:1022-1037
            cache["state"] = h_final.clone()
            cache["seq_pos"] = L
            cache["ent_k_cache"], cache["ent_v_cache"] = k_cache, v_cache
            cache["cache_idx"] = 0
        self._last_cross_layer_state = last
        self._last_scan_state_f64 = h_final
        self.last_entanglement_map = None
        flat = stern.reshape(-1)  # tesm_mimo.py:506-519
        total = float(flat.numel())
        key = (total, dev)
        if key not in self._stats_totals:
            self._stats_totals[key] = torch.tensor(total, device=dev)
        self._stats_ternary_buffer = flat
        self._stats_total_buffer = self._stats_totals[key]
        self._ternary_stats_for_logging = (flat, total)
        self.__dict__["_stats_pending"] = (scount, total)
        return y, h_final

    # -- inference cache (tesm_mimo.py:689-731) ----------------------------------------
    def allocate_inference_cache(self, batch_size, max_seqlen, dtype=None, **kwargs):
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

    def _check_mimo_cache(self, kc, vc, B, dev):
        H = self.n_heads
        W = kc.shape[1] if kc.dim() == 4 else -1
        ok = (kc.dim() == 4 and vc.dim() == 4 and tuple(kc.shape) == (B, W, H, self.ent_rank)
              and tuple(vc.shape) == (B, W, H, self.d_state) and kc.dtype == vc.dtype
              and kc.dtype in (torch.float32, torch.bfloat16) and kc.is_contiguous() and vc.is_contiguous()
              and kc.device == dev and vc.device == dev and 1 <= W <= 64)
        if not ok:
            raise RuntimeError("TESMMIMO hip decode: the inference cache must hold contiguous (B, W, n_heads, ent_rank) "
                               "and (B, W, n_heads, d_state) float32 or bfloat16 ring buffers on the layer's device, "
                               "W <= 64")

    def _mimo_step_plan(self, B, dt, dev, cdt, W, cross):
        """The decode descriptor's fields that stay fixed from step to step, rebuilt when a shape, a
        dtype, a weight or a bias changes."""
        lins = (self.in_proj, self.state_proj, self.ent_proj, self.out_proj, self.cross_layer_q_proj)
        db, lb = self.decay_bias, self.local_entanglement_bias
        lb_key = (lb._version, lb.data_ptr()) if lb is not None else None
        key = (B, dt, dev, cdt, W, cross, self.entanglement_threshold, float(self.entanglement_scale), db._version,
               db.data_ptr(), db.dtype, lb_key, tuple(p.cache_key() for p in lins))
        plan = self.__dict__.get("_mimo_decode_plan")
        if plan is not None and plan[0] == key:
            return plan[1]
        for p in lins[:4 + int(cross)]:
            if p.weight.dtype != dt:
                raise RuntimeError(f"expected both operands to have the same dtype, got {dt} and {p.weight.dtype}")
        decay_bias = self._decay_bias_dt(dt).contiguous()
        if lb is not None:
            local_bias = self._local_bias_f32(dt)
        else:
            # global layers decode over their one-slot rings with no bias (tesm_mimo.py:698, 862-866)
            local_bias = torch.zeros(self.n_heads, W, dtype=torch.float32, device=dev)
        hip_ops.require_device(decay_bias, local_bias)
        if decay_bias.device != dev or local_bias.shape[-1] != W:
            raise RuntimeError("TESMMIMO hip decode: the ring size must equal entanglement_window and the biases "
                               "must live on the input's device")
        desc = _lib.MimoStep()
        desc.dt = hip_ops.dt_code(dt)
        desc.cache_dt = hip_ops.dt_code(cdt)
        desc.B, desc.d_model, desc.d_state, desc.n_heads = B, self.d_model, self.d_state, self.n_heads
        desc.ent_rank, desc.window = self.ent_rank, W
        desc.bit_eps = self.in_proj.bit_eps
        desc.thr = hip_ops.round_dtype(self.entanglement_threshold, dt)
        desc.ent_scale = float(self.entanglement_scale)
        desc.in_proj = self.in_proj.linear_desc()
        desc.state_proj = self.state_proj.linear_desc()
        desc.ent_proj = self.ent_proj.linear_desc()
        desc.out_proj = self.out_proj.linear_desc()
        if cross:
            desc.cross_q_proj = self.cross_layer_q_proj.linear_desc()
        desc.decay_bias = decay_bias.data_ptr()
        desc.local_bias = local_bias.data_ptr()
        keep = (decay_bias, local_bias) + tuple(p.packed_weight() for p in lins[:4 + int(cross)])
        nbytes = int(_lib.load().tesm_hip_mimo_decode_ws_bytes(ctypes.byref(desc)))
        self.__dict__["_mimo_decode_plan"] = (key, (desc, nbytes, keep))
        return desc, nbytes, keep

    def _forward_incremental(self, u, inference_params, cross_layer_state=None):
        """One decode step per sequence (tesm_mimo.py:753-912); returns ``(y (B, 1, d_model), state f64
        (B, n_heads, d_state))``.  Like the reference's step it runs each head as a single-rank layer (no
        mimo_x / mimo_o expansion)."""
        lib = _lib.load()
        cache = inference_params["state_cache"]
        dt = u.dtype
        B, _, dm = u.shape
        H, D = self.n_heads, self.d_state
        dev = u.device
        kc, vc = cache["ent_k_cache"], cache["ent_v_cache"]
        self._check_mimo_cache(kc, vc, B, dev)
        W = kc.shape[1]
        if self.entanglement_window > 0 and W != self.entanglement_window:
            raise RuntimeError(f"TESMMIMO hip decode: ring of {W} slots for entanglement_window "
                               f"{self.entanglement_window}")
        state = cache["state"]
        if state.dtype != torch.float64 or tuple(state.shape) != (B, H, D) or state.device != dev:
            raise RuntimeError("TESMMIMO hip decode: cache['state'] must be a (B, n_heads, d_state) float64 tensor on "
                               "the layer's device")
        state = state.contiguous()
        pos = int(cache["seq_pos"])
        slot = int(cache.get("cache_idx", 0))
        u2 = u.reshape(B, dm)
        if u2.stride(1) != 1:
            u2 = u2.contiguous()
        cs = None
        if cross_layer_state is not None:
            if cross_layer_state.dim() != 3:
                # the reference's step broadcasts a 4-D state into a 5-D query and its einsum raises
                raise RuntimeError("TESMMIMO decode: cross_layer_state must be (B, n_heads, d_state)")
            cs = cross_layer_state.reshape(B, H, D).to(dt).contiguous()
            if cs.device != dev:
                raise RuntimeError(f"hip backend ops need all tensors on one device, got {cs.device} and {dev}")
        desc, nbytes, _ = self._mimo_step_plan(B, dt, dev, kc.dtype, W, cs is not None)
        y = torch.empty((B, 1, dm), dtype=dt, device=dev)
        state_out = torch.empty_like(state)
        new = torch.empty((B, H, D), dtype=dt, device=dev)
        rope = self.rope_table(pos + 1, dt, dev)
        desc.seq_pos, desc.cache_idx = pos, slot
        desc.u, desc.ld_u = u2.data_ptr(), u2.stride(0)
        desc.cross_state = cs.data_ptr() if cs is not None else None
        desc.rope = rope.data_ptr()
        desc.state, desc.state_out = state.data_ptr(), state_out.data_ptr()
        desc.k_cache, desc.v_cache = kc.data_ptr(), vc.data_ptr()
        desc.y = y.data_ptr()
        desc.new_state = new.data_ptr()
        stream = torch.cuda.current_stream(dev)
        with torch.cuda.device(dev):
            ws = workspace(dev, nbytes, stream)
            rc = lib.tesm_hip_mimo_decode(ctypes.byref(desc), ctypes.c_void_p(ws.data_ptr()), ws.numel(),
                                          ctypes.c_void_p(stream.cuda_stream))
        _lib.check(rc)
        cache["cache_idx"] = (slot + 1) % W
        cache["state"] = state_out
        cache["seq_pos"] = pos + 1
        self._last_cross_layer_state = new
        self._last_scan_state_f64 = state_out
        self.last_entanglement_map = None
        return y, state_out

    def _mimo_cache_buffers(self, cache, B, L, dev):
        """With L >= W the reference replaces the rings by new float32 tensors, otherwise it writes the
        last L slots of the existing ones (tesm_mimo.py:1028-1035)."""
        kc, vc = cache["ent_k_cache"], cache["ent_v_cache"]
        W, H = kc.shape[1], self.n_heads
        if L >= W:
            return (torch.empty(B, W, H, self.ent_rank, dtype=torch.float32, device=dev),
                    torch.empty(B, W, H, self.d_state, dtype=torch.float32, device=dev))
        ok = (kc.dim() == 4 and vc.dim() == 4 and tuple(kc.shape) == (B, W, H, self.ent_rank)
              and tuple(vc.shape) == (B, W, H, self.d_state) and kc.dtype == vc.dtype
              and kc.dtype in (torch.float32, torch.bfloat16) and kc.is_contiguous() and vc.is_contiguous()
              and kc.device == dev and vc.device == dev)
        if not ok:
            raise RuntimeError("TESMMIMO hip: the inference cache must hold contiguous (B, W, n_heads, ent_rank) and "
                               "(B, W, n_heads, d_state) float32 or bfloat16 ring buffers on the layer's device")
        return kc, vc
