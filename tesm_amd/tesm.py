"""TESM_SISO with ``kernel_backend='hip'``.

Constructor, parameter names, initialisation order and forward signature follow
the reference's TESM_SISO (tesm_ssm/modules/tesm.py:456-1272), so a module built
under the same seed holds the same parameters and ``MixerModel``-style callers
run it unchanged.  The prefill forward is one call into the C-ABI driver
``tesm_hip_siso_prefill``, which queues the layer's kernels on the current
stream: in_proj, gates + state scan, RoPE'd local-window ternary entanglement,
mix, state_proj/ent_proj with the fused output gate, out_proj.

Like the reference's CUDA fast path, eval runs leave ``last_entanglement_map``
and ``last_entanglement_stats`` at ``None`` (tesm.py:902-904).
"""
from __future__ import annotations

import ctypes
import math

import torch
import torch.nn as nn

from . import _lib, hip_ops
from .bitlinear import BitLinear, backend_error, check_hip_call

_WORKSPACES = {}


def raw_stream(index: int) -> int:
    """The raw handle of device ``index``'s current stream (``torch.cuda.current_stream(..).cuda_stream``
    without building a Stream object, which costs over a microsecond on the per-token decode path)."""
    return torch._C._cuda_getCurrentRawStream(index)


def workspace(device: torch.device, nbytes: int, stream=None, raw=None) -> torch.Tensor:
    """A per-(device, stream) scratch buffer, grown on demand; reused across calls on that stream.
    ``raw``: the stream's raw handle, in place of ``stream``."""
    if raw is None:
        if stream is None:
            stream = torch.cuda.current_stream(device)
        raw = stream.cuda_stream
    key = (device.index, raw)
    buf = _WORKSPACES.get(key)
    if buf is None or buf.numel() < nbytes:
        buf = torch.empty((max(nbytes, 256),), dtype=torch.uint8, device=device)
        _WORKSPACES[key] = buf
    return buf


class TESM_SISO(nn.Module):
    def __init__(self, d_model, d_state=256, expand=2, ent_rank=64, entanglement_scale=0.2,
                 entanglement_threshold=0.1, max_seq_len=2048, dropout=0.0, bit_eps=1e-5, bit_threshold=0.5,
                 layer_idx=None, device=None, dtype=None, annealing_enabled=True, T_start=10.0, T_end=0.1,
                 annealing_steps=1000, annealing_schedule="cosine", quantum_tunneling_enabled=False,
                 tunneling_strength=0.1, num_tunnel_paths=4, energy_landscape="entropy",
                 tunneling_schedule="adaptive", **kwargs):
        super().__init__()
        self.d_model = d_model
        self.d_state = d_state
        self.expand = expand
        for name, v in (("d_state", d_state), ("d_model", d_model), ("ent_rank", ent_rank),
                        ("max_seq_len", max_seq_len)):
            if v <= 0:  # tesm.py:492-499
                raise ValueError(f"{name} must be positive, got {v}")
        if quantum_tunneling_enabled:
            raise NotImplementedError("quantum tunnelling is a training-time option; the hip backend is eval-only")
        self.ent_rank = ent_rank
        self.entanglement_scale = entanglement_scale
        self.entanglement_threshold = entanglement_threshold
        self.entanglement_init = kwargs.get("entanglement_init", 0.3)
        self.entanglement_window = int(kwargs.get("entanglement_window", 0) or 0)
        self.entanglement_block_size = int(kwargs.get("entanglement_block_size", 256) or 256)
        self.state_scan_chunk_size = int(kwargs.get("state_scan_chunk_size", 16) or 16)
        self.use_triton_kernels = False
        self.kernel_backend = str(kwargs.get("kernel_backend", "hip"))
        self.kernel_mode = "precise" if str(kwargs.get("kernel_mode", "fast")) == "precise" else "fast"
        self.max_seq_len = max_seq_len
        self.layer_idx = layer_idx
        self.annealing_enabled = annealing_enabled
        self.T_start, self.T_end = T_start, T_end
        self.annealing_steps = annealing_steps
        self.annealing_schedule = annealing_schedule
        self.register_buffer("annealing_step", torch.tensor(0))
        self.quantum_tunneling_enabled = False
        self.quantum_tunneler = None

        bl = dict(bias=False, bit_eps=bit_eps, bit_threshold=bit_threshold, kernel_backend=self.kernel_backend,
                  kernel_mode=self.kernel_mode, device=device, dtype=dtype)
        total_proj = 2 * d_model + 3 * d_state + 2 * ent_rank  # tesm.py:533
        self.in_proj = BitLinear(d_model, total_proj, **bl)
        self.state_proj = BitLinear(d_state, d_model, **bl)
        self.ent_proj = BitLinear(d_state, d_model, **bl)
        self.out_proj = BitLinear(d_model, d_model, **bl)
        self.dropout = nn.Dropout(dropout)
        decay_init = float(kwargs.get("decay_init_bias", 3.0))
        self.decay_bias = nn.Parameter(torch.full((d_state,), decay_init, device=device, dtype=torch.float32))
        if self.entanglement_window > 0:  # tesm.py:543-551
            self.register_parameter("entanglement", None)
            self.local_entanglement_bias = nn.Parameter(
                torch.randn(self.entanglement_window, device=device, dtype=torch.float32) * self.entanglement_init)
        else:  # tesm.py:553-570: global entanglement parameters (same RNG use)
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
        self._rope = {}
        self._bias_cache = None

    # -- cached device constants ---------------------------------------------------
    def rope_table(self, L: int, dtype: torch.dtype, device: torch.device, pos_offset: int = 0) -> torch.Tensor:
        key = (dtype, device, pos_offset)
        tab = self._rope.get(key)
        if tab is None or tab.shape[0] < L:
            n = max(L, min(self.max_seq_len, 2 * L))
            tab = hip_ops.rope_table(n, self.ent_rank, dtype, device, self.rope_base, pos_offset)
            self._rope[key] = tab
        return tab

    def _local_bias_f32(self, dtype: torch.dtype) -> torch.Tensor:
        """``local_entanglement_bias`` rounded to the layer dtype (tesm.py:925), as float32.

        The kernels use its last ``min(W, L)`` entries, as the reference does."""
        p = self.local_entanglement_bias
        key = (p._version, p.data_ptr(), dtype)
        if self._bias_cache is None or self._bias_cache[0] != key:
            with torch.no_grad():
                v = p.detach().to(dtype).to(torch.float32).contiguous()
            self._bias_cache = (key, v)
        return self._bias_cache[1]

    def _global_params_f32(self, dtype):
        """global_rel_pos_embed / _scale / _bias rounded to the layer dtype (tesm.py:980-982), as float32."""
        ps = (self.global_rel_pos_embed, self.global_rel_pos_scale, self.global_rel_pos_bias)
        key = tuple((p._version, p.data_ptr()) for p in ps) + (dtype,)
        cached = self.__dict__.get("_global_cache")
        if cached is None or cached[0] != key:
            with torch.no_grad():
                vals = tuple(p.detach().to(dtype).to(torch.float32).contiguous() for p in ps)
            self.__dict__["_global_cache"] = (key, vals)
        return self.__dict__["_global_cache"][1]

    def _decay_bias_dt(self, dtype):
        if self.decay_bias.dtype != dtype:
            raise RuntimeError(
                f"decay_bias is {self.decay_bias.dtype} but activations are {dtype}: convert the whole module with "
                f"module.to({dtype}) (building with dtype= leaves decay_bias float32)")
        return self.decay_bias.detach()

    # -- forward ---------------------------------------------------------------------
    def forward(self, u, inference_params=None, cross_layer_state=None, prev_state=None, **kwargs):
        batch, seqlen, _ = u.shape
        if seqlen > self.max_seq_len:  # tesm.py:1180-1181
            raise ValueError(f"Sequence length {seqlen} exceeds max_seq_len {self.max_seq_len}")
        if seqlen == 0:  # tesm.py:1184-1185
            return u, None
        check_hip_call(self.kernel_backend, "TESM", self, u)
        if inference_params is not None and seqlen == 1:
            cache = inference_params.get("state_cache")
            if cache is not None and "state" in cache:
                return self._forward_incremental(u, inference_params, cross_layer_state)
        cache = None
        if inference_params is not None:  # tesm.py:1235-1253
            cache = inference_params.get("state_cache")
            if cache is None or "state" not in cache:
                cache = None
        y, states, h_final = self._prefill(u, cross_layer_state, prev_state, cache)
        self._last_cross_layer_state = states
        self._last_scan_state_f64 = h_final
        self.last_entanglement_map = None
        self.last_entanglement_stats = None
        return y, h_final

    def _prefill(self, u, cross_layer_state, prev_state, cache=None):
        lib = _lib.load()
        dt = u.dtype
        B, L, dm = u.shape
        D, R = self.d_state, self.ent_rank
        u = u.contiguous()
        dev = u.device
        y = torch.empty((B, L, dm), dtype=dt, device=dev)
        states = torch.empty((B, L, D), dtype=dt, device=dev)
        h_final = torch.empty((B, D), dtype=torch.float64, device=dev)
        for p in (self.in_proj, self.state_proj, self.ent_proj, self.out_proj, self.cross_layer_q_proj):
            if p.weight.dtype != dt:
                raise RuntimeError(f"expected both operands to have the same dtype, got {dt} and {p.weight.dtype}")
        cs = None
        if cross_layer_state is not None:
            cs = cross_layer_state
            if cs.dim() == 2:
                cs = cs.unsqueeze(1).expand(B, L, D)
            cs = cs.to(dt).contiguous()
        h0 = prev_state.to(device=dev, dtype=torch.float64).contiguous() if prev_state is not None else None
        decay_bias = self._decay_bias_dt(dt)
        glob = self.entanglement_window <= 0
        local_bias = None if glob else self._local_bias_f32(dt)
        gparams = self._global_params_f32(dt) if glob else None
        rope = self.rope_table(L, dt, dev)
        hip_ops.require_device(u, cs, h0, decay_bias, local_bias, rope, y, states, h_final,
                               *(gparams if gparams is not None else ()))
        desc = _lib.SisoLayer()
        desc.dt = hip_ops.dt_code(dt)
        desc.B, desc.L, desc.d_model, desc.d_state, desc.ent_rank = B, L, dm, D, R
        desc.window, desc.chunk_size = max(self.entanglement_window, 0), self.state_scan_chunk_size
        desc.bit_eps = self.in_proj.bit_eps
        desc.thr = hip_ops.round_dtype(self.entanglement_threshold, dt)
        desc.ent_scale = float(self.entanglement_scale)
        desc.u = u.data_ptr()
        desc.in_proj = self.in_proj.linear_desc()
        desc.state_proj = self.state_proj.linear_desc()
        desc.ent_proj = self.ent_proj.linear_desc()
        desc.out_proj = self.out_proj.linear_desc()
        if cs is not None:
            desc.cross_q_proj = self.cross_layer_q_proj.linear_desc()
            desc.cross_state = cs.data_ptr()
        desc.decay_bias = decay_bias.data_ptr()
        desc.local_bias = local_bias.data_ptr() if local_bias is not None else None
        if gparams is not None:
            emb, scale, bias = gparams
            desc.global_embed, desc.global_dim = emb.data_ptr(), emb.numel()
            desc.global_scale, desc.global_bias = scale.data_ptr(), bias.data_ptr()
        desc.rope = rope.data_ptr()
        desc.h0 = h0.data_ptr() if h0 is not None else None
        desc.y = y.data_ptr()
        desc.states = states.data_ptr()
        desc.h_final = h_final.data_ptr()
        k_cache = v_cache = None
        if cache is not None:
            k_cache, v_cache = self._prefill_cache_buffers(cache, B, L, dev)
            desc.k_cache, desc.v_cache = k_cache.data_ptr(), v_cache.data_ptr()
            desc.cache_dt = hip_ops.dt_code(k_cache.dtype)
            desc.cache_window = k_cache.shape[1]
        nbytes = int(lib.tesm_hip_siso_prefill_ws_bytes(ctypes.byref(desc)))
        with torch.cuda.device(dev):
            ws = workspace(dev, nbytes)
            _lib.check(lib.tesm_hip_siso_prefill(ctypes.byref(desc), ctypes.c_void_p(ws.data_ptr()), ws.numel(),
                                                 ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)))
        if cache is not None:  # tesm.py:1240-1252
            cache["state"] = h_final.clone()
            cache["seq_pos"] = L
            cache["ent_k_cache"], cache["ent_v_cache"] = k_cache, v_cache
            cache["cache_idx"] = 0
        return y, states, h_final

    def _prefill_cache_buffers(self, cache, B, L, dev):
        """Ring buffers the prefill writes: with L >= W the reference replaces them by new float32
        tensors (tesm.py:1244-1247), otherwise it writes the last L slots of the existing ones."""
        kc, vc = cache["ent_k_cache"], cache["ent_v_cache"]
        W = kc.shape[1]
        if L >= W:
            return (torch.empty(B, W, self.ent_rank, dtype=torch.float32, device=dev),
                    torch.empty(B, W, self.d_state, dtype=torch.float32, device=dev))
        self._check_cache(kc, vc, B, dev)
        return kc, vc

    def _check_cache(self, kc, vc, B, dev):
        # sizes compared as torch.Size against tuples and devices by index: this runs once per decoded token
        di = -1 if dev.index is None else dev.index
        ks, vs = kc.size(), vc.size()
        W = ks[1] if len(ks) == 3 else -1
        ok = (len(ks) == 3 and ks == (B, W, self.ent_rank) and vs == (B, W, self.d_state) and kc.dtype == vc.dtype
              and kc.dtype in (torch.float32, torch.bfloat16) and kc.is_contiguous() and vc.is_contiguous()
              and kc.get_device() == di and vc.get_device() == di and 1 <= W <= 64)
        if not ok:
            raise RuntimeError("TESM hip decode: the inference cache must hold contiguous (B, W, ent_rank) and "
                               "(B, W, d_state) float32 or bfloat16 ring buffers on the layer's device, W <= 64")

    # -- inference cache (tesm.py:620-670, 1235-1253) -----------------------------------
    def allocate_inference_cache(self, batch_size, max_seqlen, dtype=None, **kwargs):
        dev = self.out_proj.weight.device
        cdt = dtype or torch.float32
        W = max(self.entanglement_window, 1)
        if kwargs.get("use_paged_cache", False) and max_seqlen > 1024:
            raise NotImplementedError("paged state cache is not supported by the hip backend")
        return {
            "use_paged": False,
            "state": torch.zeros(batch_size, self.d_state, device=dev, dtype=torch.float64),
            "seq_pos": 0,
            "ent_k_cache": torch.zeros(batch_size, W, self.ent_rank, device=dev, dtype=cdt),
            "ent_v_cache": torch.zeros(batch_size, W, self.d_state, device=dev, dtype=cdt),
            "cache_idx": 0,
            "cache_filled": False,
        }

    def _step_key(self, B, dt, dev, cdt, W, cross):
        """What the decode descriptor depends on: shapes, dtypes, thresholds, and the version and storage
        of every weight and bias (the packed weights follow tesm.py:226-236's cache rule)."""
        # modules and parameters read from their dicts: this runs once per decoded token, and
        # nn.Module.__getattr__ costs a fraction of a microsecond per lookup
        mods, params = self._modules, self._parameters
        lins = (mods["in_proj"], mods["state_proj"], mods["ent_proj"], mods["out_proj"], mods["cross_layer_q_proj"])
        db, lb = params["decay_bias"], params["local_entanglement_bias"]
        lb_key = (lb._version, lb.data_ptr()) if lb is not None else None
        return (B, dt, dev, cdt, W, cross, self.entanglement_threshold, float(self.entanglement_scale), db._version,
                db.data_ptr(), db.dtype, lb_key, tuple(p.cache_key() for p in lins))

    def _step_plan(self, B, dt, dev, cdt, W, cross):
        """The decode descriptor's fields that stay fixed from step to step, rebuilt when a shape, a
        dtype, a weight or a bias changes (``_step_key``)."""
        mods, params = self._modules, self._parameters
        lins = (mods["in_proj"], mods["state_proj"], mods["ent_proj"], mods["out_proj"], mods["cross_layer_q_proj"])
        lb = params["local_entanglement_bias"]
        key = self._step_key(B, dt, dev, cdt, W, cross)
        plan = self.__dict__.get("_decode_plan")
        if plan is not None and plan[0] == key:
            return plan[1]
        for p in lins:
            if p.weight.dtype != dt:
                raise RuntimeError(f"expected both operands to have the same dtype, got {dt} and {p.weight.dtype}")
        decay_bias = self._decay_bias_dt(dt)
        if lb is not None:
            local_bias = self._local_bias_f32(dt)
        else:
            # global layers decode over their one-slot ring with no bias (tesm.py:633, 1355-1357);
            # adding 0 to a score leaves it unchanged
            local_bias = torch.zeros(W, dtype=torch.float32, device=dev)
        D, R, dm = self.d_state, self.ent_rank, self.d_model
        desc = _lib.SisoStep()
        desc.dt = hip_ops.dt_code(dt)
        desc.cache_dt = hip_ops.dt_code(cdt)
        desc.B, desc.d_model, desc.d_state, desc.ent_rank, desc.window = B, dm, D, R, W
        desc.bit_eps = self.in_proj.bit_eps
        desc.thr = hip_ops.round_dtype(self.entanglement_threshold, dt)
        desc.ent_scale = float(self.entanglement_scale)
        desc.in_proj = self.in_proj.linear_desc()
        desc.state_proj = self.state_proj.linear_desc()
        desc.ent_proj = self.ent_proj.linear_desc()
        desc.out_proj = self.out_proj.linear_desc()
        if cross:
            desc.cross_q_proj = self.cross_layer_q_proj.linear_desc()
        hip_ops.require_device(decay_bias, local_bias)
        if decay_bias.device != dev:
            raise RuntimeError(f"hip backend ops need all tensors on one device, got {decay_bias.device} and {dev}")
        desc.decay_bias = decay_bias.data_ptr()
        desc.local_bias = local_bias.data_ptr()
        keep = (decay_bias, local_bias) + tuple(p.packed_weight() for p in lins[:4 + int(cross)])
        nbytes = int(_lib.load().tesm_hip_siso_decode_ws_bytes(ctypes.byref(desc)))
        self.__dict__["_decode_plan"] = (key, (desc, nbytes, keep))
        return desc, nbytes, keep

    def _forward_incremental(self, u, inference_params, cross_layer_state=None):
        """One decode step per sequence (tesm.py:1274-1400); returns ``(y (B, 1, d_model), state f64)``."""
        lib = _lib.load()
        cache = inference_params["state_cache"]
        dt = u.dtype
        B, _, dm = u.shape
        D = self.d_state
        dev = u.device
        kc, vc = cache["ent_k_cache"], cache["ent_v_cache"]
        self._check_cache(kc, vc, B, dev)
        W = kc.shape[1]
        state = cache["state"]
        if state.dtype != torch.float64 or state.size() != (B, D) or state.get_device() != (-1 if dev.index is None else dev.index):
            raise RuntimeError("TESM hip decode: cache['state'] must be a (B, d_state) float64 tensor on the layer's "
                               "device")
        state = state.contiguous()
        pos = int(cache["seq_pos"])
        slot = int(cache.get("cache_idx", 0))
        if u.stride(2) != 1:
            u = u.contiguous()
        ld_u = u.stride(0) if B > 1 else dm  # rows of a one-token slice of a longer sequence, no view needed
        cs = None
        if cross_layer_state is not None:
            cs = cross_layer_state.reshape(B, D).to(dt).contiguous()
            if cs.device != dev:
                raise RuntimeError(f"hip backend ops need all tensors on one device, got {cs.device} and {dev}")
        desc, nbytes, _ = self._step_plan(B, dt, dev, kc.dtype, W, cs is not None)
        y = torch.empty((B, 1, dm), dtype=dt, device=dev)
        state_out = torch.empty_like(state)
        new = torch.empty((B, D), dtype=dt, device=dev)
        rope = self.rope_table(pos + 1, dt, dev)
        desc.seq_pos, desc.cache_idx = pos, slot
        desc.u, desc.ld_u = u.data_ptr(), ld_u
        desc.cross_state = cs.data_ptr() if cs is not None else None
        desc.rope = rope.data_ptr()
        desc.state, desc.state_out = state.data_ptr(), state_out.data_ptr()
        desc.k_cache, desc.v_cache = kc.data_ptr(), vc.data_ptr()
        desc.y = y.data_ptr()
        desc.new_state = new.data_ptr()
        raw = raw_stream(dev.index)
        if torch.cuda.current_device() == dev.index:
            ws = workspace(dev, nbytes, raw=raw)
            rc = lib.tesm_hip_siso_decode(ctypes.byref(desc), ctypes.c_void_p(ws.data_ptr()), ws.numel(),
                                          ctypes.c_void_p(raw))
        else:
            with torch.cuda.device(dev):
                ws = workspace(dev, nbytes, raw=raw)
                rc = lib.tesm_hip_siso_decode(ctypes.byref(desc), ctypes.c_void_p(ws.data_ptr()), ws.numel(),
                                              ctypes.c_void_p(raw))
        _lib.check(rc)
        cache["cache_idx"] = (slot + 1) % W
        cache["state"] = state_out
        cache["seq_pos"] = pos + 1
        # plain attributes (never parameters, buffers or modules): set without nn.Module.__setattr__,
        # which costs microseconds per call on this per-token path
        self.__dict__.update(_last_cross_layer_state=new, _last_scan_state_f64=state_out, last_entanglement_map=None)
        return y, state_out


TESM = TESM_SISO
