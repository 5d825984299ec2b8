"""Tensor-level wrappers over the C-ABI (device memory and streams come from torch).

Every function queues HIP kernels on the current torch stream of the tensors'
device and returns torch tensors allocated here.  Nothing computes on the host
and nothing falls back to torch ops: a missing library raises.

Row-major 2-D operands may have a row stride (``x.stride(0)``) larger than their
width as long as the last dimension is contiguous, so slices of a wider
projection output are passed without copies.
"""
from __future__ import annotations

import ctypes
import functools
from typing import Optional

import torch

from . import _lib

_DT = {torch.float32: 0, torch.bfloat16: 1}


def dt_code(dtype: torch.dtype) -> int:
    try:
        return _DT[dtype]
    except KeyError:
        raise TypeError(f"hip backend supports float32 and bfloat16, got {dtype}") from None


def _p(t: Optional[torch.Tensor]):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(t: torch.Tensor):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _rows(x: torch.Tensor) -> torch.Tensor:
    """2-D view with a contiguous last dimension (copies only if needed)."""
    if x.dim() != 2:
        raise ValueError("expected a 2-D tensor")
    if x.stride(1) != 1 or x.stride(0) < x.shape[1]:
        x = x.contiguous()
    return x


def require_device(*ts):
    """Every tensor handed to a kernel must live on one ROCm device: a host pointer would be
    dereferenced by the GPU."""
    dev = None
    for t in ts:
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError(f"hip backend ops need tensors on a ROCm device, got one on {t.device}")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"hip backend ops need all tensors on one device, got {dev} and {t.device}")


def kpad(K: int) -> int:
    return int(_lib.load().tesm_hip_kpad(K))


@functools.lru_cache(maxsize=1024)
def round_dtype(v: float, dtype: torch.dtype) -> float:
    """The float value that torch uses for a Python scalar compared against a ``dtype`` tensor."""
    return float(torch.tensor(v, dtype=torch.float32).to(dtype).float())


# ---------------------------------------------------------------------------
# BitLinear pieces
# ---------------------------------------------------------------------------
def quant_act(x: torch.Tensor, eps: float = 1e-5, layout: int = 1, ldq: Optional[int] = None):
    """Per-token int8 codes of ``x`` (M, K): returns (codes (M, ldq), s_x (M), rowsum (M))."""
    lib = _lib.load()
    x = _rows(x)
    require_device(x)
    M, K = x.shape
    ldq = kpad(K) if ldq is None else ldq
    q = torch.empty((M, ldq), dtype=torch.int8, device=x.device)
    s = torch.empty((M,), dtype=torch.float32, device=x.device)
    rs = torch.empty((M,), dtype=torch.int32, device=x.device)
    with torch.cuda.device(x.device):
        _lib.check(lib.tesm_hip_quant_act_i8(_p(x), dt_code(x.dtype), M, K, x.stride(0), eps, layout, _p(q), ldq,
                                             _p(s), _p(rs), _stream(x)))
    return q, s, rs


def absmean_scale(w: torch.Tensor, eps: float = 1e-5):
    """(s_w, c_w) device scalars: s_w = 1/max(mean|w|, eps), c_w = 1/s_w, rounded to w's dtype."""
    lib = _lib.load()
    w = w.contiguous()
    require_device(w)
    ws = torch.empty((int(lib.tesm_hip_absmean_ws_bytes()),), dtype=torch.uint8, device=w.device)
    s_w = torch.empty((1,), dtype=torch.float32, device=w.device)
    c_w = torch.empty((1,), dtype=torch.float32, device=w.device)
    with torch.cuda.device(w.device):
        _lib.check(lib.tesm_hip_absmean_scale(_p(w), dt_code(w.dtype), w.numel(), eps, _p(ws), _p(s_w), _p(c_w),
                                              _stream(w)))
    return s_w, c_w


def pack_weight(w: torch.Tensor, s_w: torch.Tensor, per_row: bool = False, ldp: Optional[int] = None):
    """Ternary codes of ``w`` (N, K) at scale ``s_w`` packed 4 per byte: (N, ldp) uint8.

    ``ldp`` defaults to kpad(K)/4 (the layout the products read); pass
    ``ldp=ceil(K/4)`` for the canonical export layout.
    """
    lib = _lib.load()
    w = _rows(w)
    require_device(w, s_w)
    N, K = w.shape
    ldp = kpad(K) // 4 if ldp is None else ldp
    packed = torch.empty((N, ldp), dtype=torch.uint8, device=w.device)
    s_w = s_w.to(torch.float32).contiguous()
    with torch.cuda.device(w.device):
        _lib.check(lib.tesm_hip_pack_w_i2(_p(w), dt_code(w.dtype), N, K, w.stride(0), _p(s_w), int(per_row),
                                          _p(packed), ldp, _stream(w)))
    return packed


def unpack_weight(packed: torch.Tensor, K: int):
    lib = _lib.load()
    packed = _rows(packed)
    require_device(packed)
    N = packed.shape[0]
    codes = torch.empty((N, K), dtype=torch.int8, device=packed.device)
    with torch.cuda.device(packed.device):
        _lib.check(lib.tesm_hip_unpack_w_i2(_p(packed), N, K, packed.stride(0), _p(codes), K, _stream(packed)))
    return codes


def bitlinear(q, s_x, rowsum, packed, c_w, N: int, K: int, out_dtype: torch.dtype, bias=None,
              c_w_per_row: bool = False, acc_dump: bool = False, out: Optional[torch.Tensor] = None):
    """out (M, N) = (q . codes) / s_x * c_w (+ bias); optionally also the int32 accumulators."""
    lib = _lib.load()
    M = q.shape[0]
    if out is None:
        out = torch.empty((M, N), dtype=out_dtype, device=q.device)
    acc = torch.empty((M, N), dtype=torch.int32, device=q.device) if acc_dump else None
    require_device(q, s_x, rowsum, packed, c_w, bias, out, acc)
    with torch.cuda.device(q.device):
        _lib.check(lib.tesm_hip_bitlinear_i2(_p(q), q.stride(0), _p(s_x), _p(rowsum), _p(packed), packed.stride(0),
                                             _p(c_w), int(c_w_per_row), _p(bias), M, N, K, _p(out),
                                             dt_code(out.dtype), out.stride(0), _p(acc), _stream(q)))
    return (out, acc) if acc_dump else out


def bitlinear_fwd(x, packed, c_w, N: int, eps: float = 1e-5, bias=None, c_w_per_row: bool = False,
                  fuse: bool = True, out: Optional[torch.Tensor] = None):
    """BitLinear forward from raw activations x (M, K): codes + product in one C-ABI call (fused
    for decode-size M when ``fuse``); out (M, N) in x's dtype."""
    lib = _lib.load()
    x = _rows(x)
    M, K = x.shape
    if out is None:
        out = torch.empty((M, N), dtype=x.dtype, device=x.device)
    require_device(x, packed, c_w, bias, out)
    nbytes = int(lib.tesm_hip_bitlinear_fwd_ws_bytes(M, K))
    from .tesm import workspace
    ws = workspace(x.device, nbytes)
    with torch.cuda.device(x.device):
        _lib.check(lib.tesm_hip_bitlinear_fwd(_p(x), dt_code(x.dtype), x.stride(0), eps, _p(packed), packed.stride(0),
                                              _p(c_w), int(c_w_per_row), _p(bias), M, N, K, _p(out),
                                              dt_code(out.dtype), out.stride(0), int(fuse), _p(ws), nbytes,
                                              _stream(x)))
    return out


# ---------------------------------------------------------------------------
# diagnostics: launch log, device status, decision taps
# ---------------------------------------------------------------------------
class launch_log:
    """Context manager recording the kernel instantiations launched inside it::

        with hip_ops.launch_log() as log:
            layer(u)
        assert "scan_lb_kernel<1,1,1,16,8>" in log.kernels
    """

    def __enter__(self):
        self.kernels = []
        _lib.check(_lib.load().tesm_hip_launch_log(1))
        return self

    def __exit__(self, *exc):
        lib = _lib.load()
        n = int(lib.tesm_hip_launch_log_read(None, 0, 0))
        buf = ctypes.create_string_buffer(n + 1)
        lib.tesm_hip_launch_log_read(buf, n + 1, 1)
        lib.tesm_hip_launch_log(0)
        self.kernels = [k for k in buf.value.decode().split("\n") if k]
        return False


def stream_copy(dst: torch.Tensor, src: torch.Tensor) -> None:
    """Copy src's bytes into dst with the library's streaming copy kernel (a bandwidth reference)."""
    require_device(dst, src)
    if not (dst.is_contiguous() and src.is_contiguous()):
        raise ValueError("stream_copy: tensors must be contiguous")
    n = src.numel() * src.element_size()
    if dst.numel() * dst.element_size() < n:
        raise ValueError("stream_copy: destination too small")
    with torch.cuda.device(src.device):
        _lib.check(_lib.load().tesm_hip_stream_copy(_p(dst), _p(src), n, _stream(src)))


def device_status(clear: bool = True) -> int:
    """The device status word of the current device (bit 0: a scan look-back gave up); synchronises."""
    v = ctypes.c_uint32(0)
    lib = _lib.load()
    _lib.check(lib.tesm_hip_device_status(ctypes.byref(v), int(clear)))
    return int(v.value)


def debug_scan_spin_limit(limit: int) -> None:
    _lib.check(_lib.load().tesm_hip_debug_scan_spin_limit(int(limit)))


def set_taps(**bufs) -> None:
    """Point the decision taps at device tensors (q_te, s_te, q_c, s_c, q_y, s_y, tern, wts); no
    arguments stops tapping."""
    lib = _lib.load()
    if not bufs:
        _lib.check(lib.tesm_hip_debug_taps(None))
        return
    require_device(*bufs.values())
    t = _lib.Taps(**{k: (v.data_ptr() if v is not None else None) for k, v in bufs.items()})
    _lib.check(lib.tesm_hip_debug_taps(ctypes.byref(t)))


# ---------------------------------------------------------------------------
# scan / RoPE / entanglement
# ---------------------------------------------------------------------------
def scan(decay: torch.Tensor, update: torch.Tensor, chunk_size: int = 16, h0: Optional[torch.Tensor] = None,
         out_dtype: Optional[torch.dtype] = None):
    """States of h_t = d_t h_{t-1} + u_t for (B, L, C) inputs; returns (states, h_final fp64)."""
    lib = _lib.load()
    if decay.shape != update.shape or decay.dim() != 3:
        raise ValueError("decay and update must both be (B, L, C)")
    if decay.dtype != update.dtype:
        raise TypeError("decay and update must share a dtype")
    decay, update = decay.contiguous(), update.contiguous()
    require_device(decay, update, h0)
    B, L, C = decay.shape
    out_dtype = out_dtype or decay.dtype
    states = torch.empty((B, L, C), dtype=out_dtype, device=decay.device)
    h_final = torch.empty((B, C), dtype=torch.float64, device=decay.device)
    if h0 is not None:
        h0 = h0.to(dtype=torch.float64).contiguous()
    nbytes = int(lib.tesm_hip_scan_ws_bytes(B, L, C, chunk_size))
    ws = torch.empty((max(nbytes, 1),), dtype=torch.uint8, device=decay.device)
    with torch.cuda.device(decay.device):
        _lib.check(lib.tesm_hip_scan(_p(decay), C, _p(update), C, dt_code(decay.dtype), B, L, C, chunk_size, _p(h0),
                                     _p(states), C, dt_code(out_dtype), _p(h_final), _p(ws), nbytes, _stream(decay)))
    return states, h_final


def rope_table(L: int, R: int, dtype: torch.dtype, device, base: float = 10000.0, pos_offset: int = 0):
    """(L, R/2, 2) float32 (cos, sin) of positions pos_offset..pos_offset+L-1, rounded to ``dtype``."""
    lib = _lib.load()
    tab = torch.empty((max(L, 1), R // 2, 2), dtype=torch.float32, device=device)
    with torch.cuda.device(tab.device):
        _lib.check(lib.tesm_hip_rope_table(_p(tab), L, R, pos_offset, float(base), dt_code(dtype), _stream(tab)))
    return tab


def window_bias(bias, H: int, W: int, dt, device):
    """The window bias as the entanglement kernels take it: float32 (H, W) on ``device``, each value rounded
    to the layer dtype ``dt`` first (the reference adds the bias in that dtype)."""
    return bias.reshape(H, W).to(device=device, dtype=dt).to(torch.float32).contiguous()


def _ready_bias(bias, H: int, W: int, dt, device, bias_rounded: bool):
    if not bias_rounded:
        return window_bias(bias, H, W, dt, device)
    if bias.dtype != torch.float32 or bias.numel() != H * W or not bias.is_contiguous() or bias.device != device:
        raise ValueError("bias_rounded=True needs the float32 (H, W) contiguous tensor window_bias() returns, "
                         "on the states' device")
    return bias


def local_ent(q, k, rope, S, bias, W: int, thr: float, ent_scale: float, q_add=None, mimo: bool = False, H: int = 1,
              outputs=("avg",), want_tern: bool = False, bias_rounded: bool = False):
    """Window entanglement over (B, L, H*R) queries/keys and (B, L, H*D) states.

    ``bias`` is (H, W) (or (W,)) in any float dtype; it is rounded to the states' dtype (with
    ``bias_rounded`` it is already ``window_bias()``'s result and is passed as it is, so the call
    launches no conversion).  ``thr`` is rounded to that dtype too.  Returns a dict of the requested
    outputs among ``avg``, ``e``, ``c``, ``e_tanh`` (and ``tern`` if ``want_tern``).
    """
    lib = _lib.load()
    B, L, HR = q.shape
    D = S.shape[-1] // H
    R = HR // H
    dt = S.dtype
    q = q.reshape(B * L, HR)
    k = k.reshape(B * L, HR)
    q, k = _rows(q), _rows(k)
    S2 = _rows(S.reshape(B * L, H * D))
    qa = _rows(q_add.reshape(B * L, HR)) if q_add is not None else None
    # small parameter: accepted from any device, copied next to the states
    bias_f = _ready_bias(bias, H, W, dt, S.device, bias_rounded)
    weff = W if mimo else min(W, L)
    outs = {name: torch.empty((B, L, H * D), dtype=dt, device=S.device) for name in outputs}
    tern = torch.empty((B, L, H, weff), dtype=torch.int8, device=S.device) if want_tern else None
    nbytes = int(lib.tesm_hip_local_ent_ws_bytes(B, L, H, weff))
    ws = torch.empty((nbytes,), dtype=torch.uint8, device=S.device)
    require_device(q, k, rope, qa, bias_f, S2, tern, ws, *outs.values())
    with torch.cuda.device(S.device):
        _lib.check(lib.tesm_hip_local_ent(
            _p(q), q.stride(0), _p(k), k.stride(0), _p(rope), _p(qa), qa.stride(0) if qa is not None else 0,
            _p(bias_f), _p(S2), S2.stride(0), dt_code(dt), int(mimo), B, L, H, R, D, W, round_dtype(thr, dt),
            float(ent_scale), _p(outs.get("avg")), _p(outs.get("e")), _p(outs.get("c")), _p(outs.get("e_tanh")),
            H * D, _p(tern), _p(ws), nbytes, _stream(S)))
    if want_tern:
        outs["tern"] = tern
    return outs



def local_ent_quant(q, k, rope, S, bias, W: int, thr: float, ent_scale: float, eps: float = 1e-5, q_add=None,
                    want_floats: bool = False, want_tern: bool = False, bias_rounded: bool = False):
    """Fused SISO entanglement + int8 codes of tanh(E) and C (the state_proj / ent_proj inputs).
    ``bias`` as in ``local_ent`` (one head).

    Returns a dict with ``te`` and ``c`` = (codes (M, kpad(D)) layout 1, scales (M), rowsums (M)),
    plus ``e_tanh`` / ``c_float`` / ``tern`` when asked for.
    """
    lib = _lib.load()
    B, L, R = q.shape
    D = S.shape[-1]
    dt = S.dtype
    q2, k2 = _rows(q.reshape(B * L, R)), _rows(k.reshape(B * L, R))
    S2 = _rows(S.reshape(B * L, D))
    qa = _rows(q_add.reshape(B * L, R)) if q_add is not None else None
    bias_f = _ready_bias(bias, 1, W, dt, S.device, bias_rounded)
    M, ldq = B * L, kpad(D)
    dev = S.device
    te = (torch.empty((M, ldq), dtype=torch.int8, device=dev), torch.empty(M, device=dev),
          torch.empty(M, dtype=torch.int32, device=dev))
    cc = (torch.empty((M, ldq), dtype=torch.int8, device=dev), torch.empty(M, device=dev),
          torch.empty(M, dtype=torch.int32, device=dev))
    et = torch.empty((B, L, D), dtype=dt, device=dev) if want_floats else None
    cf = torch.empty((B, L, D), dtype=dt, device=dev) if want_floats else None
    tern = torch.empty((B, L, min(W, L)), dtype=torch.int8, device=dev) if want_tern else None
    require_device(q2, k2, rope, qa, bias_f, S2, *te, *cc, et, cf, tern)
    d = _lib.EntQuant()
    d.dt = dt_code(dt)
    d.B, d.L, d.R, d.D, d.W = B, L, R, D, W
    d.thr, d.ent_scale, d.eps = round_dtype(thr, dt), float(ent_scale), float(eps)
    d.q, d.ld_q, d.k, d.ld_k = q2.data_ptr(), q2.stride(0), k2.data_ptr(), k2.stride(0)
    d.rope = rope.data_ptr()
    d.q_add, d.ld_qadd = (qa.data_ptr(), qa.stride(0)) if qa is not None else (None, 0)
    d.bias, d.S, d.ld_s = bias_f.data_ptr(), S2.data_ptr(), S2.stride(0)
    d.q_te, d.s_te, d.rs_te = (t.data_ptr() for t in te)
    d.q_c, d.s_c, d.rs_c = (t.data_ptr() for t in cc)
    d.ldq = ldq
    d.e_tanh = et.data_ptr() if et is not None else None
    d.c_out = cf.data_ptr() if cf is not None else None
    d.ld_out = D
    d.tern = tern.data_ptr() if tern is not None else None
    with torch.cuda.device(dev):
        _lib.check(lib.tesm_hip_local_ent_quant(ctypes.byref(d), _stream(S)))
    out = {"te": te, "c": cc}
    if want_floats:
        out["e_tanh"], out["c_float"] = et, cf
    if want_tern:
        out["tern"] = tern
    return out


def output_gate(te, cc, sp_packed, sp_cw, ep_packed, ep_cw, local, gate, d_state: int, eps: float = 1e-5,
                quantize: bool = True, want_y: bool = True):
    """y = local + sigmoid(gate) * state_proj(tanh E) + ent_proj(C) from code triples ``te``/``cc``.

    ``local``/``gate`` are (M, d_model) views (row stride allowed).  With ``quantize`` the kernel
    also returns y's out_proj codes (codes, scales, rowsums).
    """
    lib = _lib.load()
    local, gate = _rows(local), _rows(gate)
    M, dm = local.shape
    dt = local.dtype
    dev = local.device
    y = torch.empty((M, dm), dtype=dt, device=dev) if (want_y or not quantize) else None
    qy = None
    if quantize:
        ldq = kpad(dm)
        qy = (torch.empty((M, ldq), dtype=torch.int8, device=dev), torch.empty(M, device=dev),
              torch.empty(M, dtype=torch.int32, device=dev))
    require_device(*te, *cc, sp_packed, sp_cw, ep_packed, ep_cw, local, gate, y, *(qy or ()))
    d = _lib.OutputGate()
    d.dt = dt_code(dt)
    d.M, d.d_model, d.d_state, d.eps = M, dm, d_state, float(eps)
    d.q_te, d.ldq_te, d.s_te, d.rs_te = te[0].data_ptr(), te[0].stride(0), te[1].data_ptr(), te[2].data_ptr()
    d.q_c, d.ldq_c, d.s_c, d.rs_c = cc[0].data_ptr(), cc[0].stride(0), cc[1].data_ptr(), cc[2].data_ptr()
    d.state_proj = _lib.Linear(sp_packed.data_ptr(), sp_packed.stride(0), sp_cw.data_ptr(), 0)
    d.ent_proj = _lib.Linear(ep_packed.data_ptr(), ep_packed.stride(0), ep_cw.data_ptr(), 0)
    d.local, d.ld_local, d.gate, d.ld_gate = local.data_ptr(), local.stride(0), gate.data_ptr(), gate.stride(0)
    d.y, d.ld_y = (y.data_ptr(), dm) if y is not None else (None, 0)
    if qy is not None:
        d.q_y, d.ldq_y, d.s_y, d.rs_y = qy[0].data_ptr(), qy[0].stride(0), qy[1].data_ptr(), qy[2].data_ptr()
    with torch.cuda.device(dev):
        _lib.check(lib.tesm_hip_output_gate_i2(ctypes.byref(d), _stream(local)))
    return y, qy
