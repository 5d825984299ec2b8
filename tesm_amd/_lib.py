"""ctypes binding of ``libtesm_hip.so`` (C-ABI declared in ``include/tesm_hip.h``).

The library is built in-tree by ``tesm_amd.build`` into ``tesm_amd/_build/``;
``TESM_HIP_LIB`` overrides the path.  Loading never falls back to anything: a
missing or mismatched library raises ``HipBackendUnavailable`` (a
``RuntimeError``), mirroring the reference's strict-backend errors
(tesm_ssm/modules/tesm.py:278-285, tesm_ssm/ops/cuda/__init__.py:41-48).
"""
from __future__ import annotations

import ctypes
import os
import threading

ABI_VERSION = 9
_DEFAULT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_build", "libtesm_hip.so")

P = ctypes.c_void_p
I64 = ctypes.c_int64
I32 = ctypes.c_int
F32 = ctypes.c_float
F64 = ctypes.c_double


NOALLOC_SCRATCH_BYTES = 8 << 20  # TESM_HIP_NOALLOC_SCRATCH_BYTES


class HipBackendUnavailable(RuntimeError):
    pass


class Linear(ctypes.Structure):
    """``tesm_hip_linear``."""
    _fields_ = [("packed", P), ("ldw", I64), ("c_w", P), ("c_w_per_row", I32)]


class EntQuant(ctypes.Structure):
    """``tesm_hip_ent_quant``."""
    _fields_ = [
        ("dt", I32),
        ("B", I64), ("L", I64), ("R", I64), ("D", I64), ("W", I64),
        ("thr", F32), ("ent_scale", F32), ("eps", F32),
        ("q", P), ("ld_q", I64), ("k", P), ("ld_k", I64), ("rope", P), ("q_add", P), ("ld_qadd", I64),
        ("bias", P), ("S", P), ("ld_s", I64),
        ("q_te", P), ("s_te", P), ("rs_te", P), ("q_c", P), ("s_c", P), ("rs_c", P), ("ldq", I64),
        ("e_tanh", P), ("c_out", P), ("ld_out", I64), ("tern", P),
    ]


class OutputGate(ctypes.Structure):
    """``tesm_hip_output_gate``."""
    _fields_ = [
        ("dt", I32),
        ("M", I64), ("d_model", I64), ("d_state", I64),
        ("eps", F32),
        ("q_te", P), ("ldq_te", I64), ("s_te", P), ("rs_te", P),
        ("q_c", P), ("ldq_c", I64), ("s_c", P), ("rs_c", P),
        ("state_proj", Linear), ("ent_proj", Linear),
        ("local", P), ("ld_local", I64), ("gate", P), ("ld_gate", I64),
        ("y", P), ("ld_y", I64),
        ("q_y", P), ("ldq_y", I64), ("s_y", P), ("rs_y", P),
    ]


class SisoLayer(ctypes.Structure):
    """``tesm_hip_siso_layer``."""
    _fields_ = [
        ("dt", I32),
        ("B", I64), ("L", I64), ("d_model", I64), ("d_state", I64), ("ent_rank", I64), ("window", I64),
        ("chunk_size", I64),
        ("bit_eps", F32), ("thr", F32), ("ent_scale", F32),
        ("u", P),
        ("in_proj", Linear), ("state_proj", Linear), ("ent_proj", Linear), ("out_proj", Linear),
        ("cross_q_proj", Linear),
        ("decay_bias", P), ("local_bias", P), ("rope", P), ("cross_state", P), ("h0", P),
        ("y", P), ("states", P), ("h_final", P), ("proj_out", P),
        ("k_cache", P), ("v_cache", P), ("cache_dt", I32),
        ("global_embed", P), ("global_dim", I64), ("global_scale", P), ("global_bias", P), ("cache_window", I64),
    ]


class SisoStep(ctypes.Structure):
    """``tesm_hip_siso_step``."""
    _fields_ = [
        ("dt", I32), ("cache_dt", I32),
        ("B", I64), ("d_model", I64), ("d_state", I64), ("ent_rank", I64), ("window", I64),
        ("seq_pos", I64), ("cache_idx", I64),
        ("bit_eps", F32), ("thr", F32), ("ent_scale", F32),
        ("u", P),
        ("in_proj", Linear), ("state_proj", Linear), ("ent_proj", Linear), ("out_proj", Linear),
        ("cross_q_proj", Linear),
        ("decay_bias", P), ("local_bias", P), ("rope", P), ("cross_state", P),
        ("state", P), ("state_out", P), ("k_cache", P), ("v_cache", P), ("y", P), ("new_state", P),
        ("ld_u", I64), ("step_pos", P), ("rope_rows", I64),
    ]


class MimoLayer(ctypes.Structure):
    """``tesm_hip_mimo_layer``."""
    _fields_ = [
        ("dt", I32),
        ("B", I64), ("L", I64), ("d_model", I64), ("d_state", I64), ("n_heads", I64), ("ent_rank", I64),
        ("window", I64),
        ("bit_eps", F32), ("thr", F32), ("ent_scale", F32),
        ("u", P),
        ("in_proj", Linear), ("state_proj", Linear), ("ent_proj", Linear), ("out_proj", Linear),
        ("decay_bias", P), ("local_bias", P), ("rope", P), ("mimo_coef", P), ("mimo_x0sq", P),
        ("y", P), ("h_final", P), ("last_state", P), ("k_cache", P), ("v_cache", P), ("cache_dt", I32),
        ("stats_ternary", P), ("stats_counts", P),
        ("global_embed", P), ("global_dim", I64), ("global_scale", P), ("global_bias", P), ("cache_window", I64),
    ]


class MimoStep(ctypes.Structure):
    """``tesm_hip_mimo_step``."""
    _fields_ = [
        ("dt", I32), ("cache_dt", I32),
        ("B", I64), ("d_model", I64), ("d_state", I64), ("n_heads", I64), ("ent_rank", I64), ("window", I64),
        ("seq_pos", I64), ("cache_idx", I64),
        ("bit_eps", F32), ("thr", F32), ("ent_scale", F32),
        ("u", P), ("ld_u", I64),
        ("in_proj", Linear), ("state_proj", Linear), ("ent_proj", Linear), ("out_proj", Linear),
        ("cross_q_proj", Linear),
        ("decay_bias", P), ("local_bias", P), ("rope", P), ("cross_state", P),
        ("state", P), ("state_out", P), ("k_cache", P), ("v_cache", P), ("y", P), ("new_state", P),
    ]


class RmsNorm(ctypes.Structure):
    """``tesm_hip_rmsnorm``."""
    _fields_ = [
        ("dt", I32),
        ("M", I64), ("D", I64),
        ("eps", F32),
        ("x", P), ("ld_x", I64),
        ("residual", P), ("residual_dt", I32), ("ld_res", I64),
        ("residual_out", P), ("residual_out_dt", I32), ("ld_res_out", I64),
        ("weight", P),
        ("y", P), ("ld_y", I64),
        ("q", P), ("ldq", I64), ("s_x", P), ("rowsum", P),
        ("bit_eps", F32),
    ]


class Ffn(ctypes.Structure):
    """``tesm_hip_ffn``."""
    _fields_ = [
        ("dt", I32),
        ("M", I64), ("d_model", I64), ("d_inter", I64),
        ("bit_eps", F32),
        ("x", P), ("ld_x", I64),
        ("x_codes", P), ("ldq_x", I64), ("x_scale", P), ("x_rowsum", P),
        ("gate_proj", Linear), ("up_proj", Linear), ("down_proj", Linear),
        ("y", P), ("ld_y", I64),
    ]


class Taps(ctypes.Structure):
    """``tesm_hip_taps``."""
    _fields_ = [("q_u", P), ("s_u", P), ("q_cs", P), ("s_cs", P), ("q_te", P), ("s_te", P), ("q_c", P), ("s_c", P),
                ("q_y", P), ("s_y", P), ("q_h", P), ("s_h", P), ("tern", P), ("wts", P), ("S", P),
                ("te", P), ("c", P), ("yv", P)]


_SIGNATURES = {
    "tesm_hip_abi_version": ([], I32),
    "tesm_hip_last_error": ([], ctypes.c_char_p),
    "tesm_hip_kpad": ([I64], I64),
    "tesm_hip_launch_log": ([I32], I32),
    "tesm_hip_launch_log_read": ([ctypes.c_char_p, I64, I32], I64),
    "tesm_hip_device_status": ([ctypes.POINTER(ctypes.c_uint32), I32], I32),
    "tesm_hip_stream_copy": ([P, P, I64, P], I32),
    "tesm_hip_debug_scan_spin_limit": ([I32], I32),
    "tesm_hip_debug_taps": ([ctypes.POINTER(Taps)], I32),
    "tesm_hip_bitlinear_fwd_ws_bytes": ([I64, I64], I64),
    "tesm_hip_bitlinear_fwd": ([P, I32, I64, F32, P, I64, P, I32, P, I64, I64, I64, P, I32, I64, I32, P, I64, P], I32),
    "tesm_hip_quant_act_i8": ([P, I32, I64, I64, I64, F32, I32, P, I64, P, P, P], I32),
    "tesm_hip_absmean_ws_bytes": ([], I64),
    "tesm_hip_absmean_scale": ([P, I32, I64, F32, P, P, P, P], I32),
    "tesm_hip_pack_w_i2": ([P, I32, I64, I64, I64, P, I32, P, I64, P], I32),
    "tesm_hip_unpack_w_i2": ([P, I64, I64, I64, P, I64, P], I32),
    "tesm_hip_bitlinear_i2": ([P, I64, P, P, P, I64, P, I32, P, I64, I64, I64, P, I32, I64, P, P], I32),
    "tesm_hip_scan_ws_bytes": ([I64, I64, I64, I64], I64),
    "tesm_hip_scan": ([P, I64, P, I64, I32, I64, I64, I64, I64, P, P, I64, I32, P, P, I64, P], I32),
    "tesm_hip_rope_table": ([P, I64, I64, I64, F64, I32, P], I32),
    "tesm_hip_local_ent_ws_bytes": ([I64, I64, I64, I64], I64),
    "tesm_hip_local_ent": ([P, I64, P, I64, P, P, I64, P, P, I64, I32, I32, I64, I64, I64, I64, I64, I64, F32, F32,
                            P, P, P, P, I64, P, P, I64, P], I32),
    "tesm_hip_local_ent_quant": ([ctypes.POINTER(EntQuant), P], I32),
    "tesm_hip_output_gate_i2": ([ctypes.POINTER(OutputGate), P], I32),
    "tesm_hip_siso_prefill_ws_bytes": ([ctypes.POINTER(SisoLayer)], I64),
    "tesm_hip_siso_prefill": ([ctypes.POINTER(SisoLayer), P, I64, P], I32),
    "tesm_hip_siso_decode_ws_bytes": ([ctypes.POINTER(SisoStep)], I64),
    "tesm_hip_siso_decode": ([ctypes.POINTER(SisoStep), P, I64, P], I32),
    "tesm_hip_siso_decode_noalloc": ([ctypes.POINTER(SisoStep), P], I32),
    "tesm_hip_mimo_decode_ws_bytes": ([ctypes.POINTER(MimoStep)], I64),
    "tesm_hip_mimo_decode": ([ctypes.POINTER(MimoStep), P, I64, P], I32),
    "tesm_hip_add_rmsnorm": ([ctypes.POINTER(RmsNorm), P], I32),
    "tesm_hip_ffn_ws_bytes": ([ctypes.POINTER(Ffn)], I64),
    "tesm_hip_ffn_forward": ([ctypes.POINTER(Ffn), P, I64, P], I32),
    "tesm_hip_mimo_coef": ([P, P, I32, I64, I64, I64, P, P, P], I32),
    "tesm_hip_mimo_prefill_ws_bytes": ([ctypes.POINTER(MimoLayer)], I64),
    "tesm_hip_mimo_prefill": ([ctypes.POINTER(MimoLayer), P, I64, P], I32),
}

_lock = threading.Lock()
_lib = None


def lib_path() -> str:
    return os.environ.get("TESM_HIP_LIB", _DEFAULT)


def exported_symbols():
    """Names the binding expects the library to export."""
    return sorted(_SIGNATURES)


def load():
    """Load and type the library once; raise HipBackendUnavailable if it cannot be used."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        path = lib_path()
        if not os.path.exists(path):
            raise HipBackendUnavailable(
                f"libtesm_hip.so not found at {path}; build it with `python -m tesm_amd.build`")
        try:
            lib = ctypes.CDLL(path)
        except OSError as e:
            raise HipBackendUnavailable(f"cannot load {path}: {e}") from e
        for name, (args, res) in _SIGNATURES.items():
            try:
                fn = getattr(lib, name)
            except AttributeError as e:
                raise HipBackendUnavailable(f"{path} does not export {name}") from e
            fn.argtypes, fn.restype = args, res
        ver = lib.tesm_hip_abi_version()
        if ver != ABI_VERSION:
            raise HipBackendUnavailable(f"{path} has ABI version {ver}, expected {ABI_VERSION}")
        _lib = lib
        return lib


def check(rc: int) -> None:
    if rc != 0:
        msg = _lib.tesm_hip_last_error().decode(errors="replace") if _lib is not None else "unknown error"
        raise RuntimeError(f"tesm_hip error {rc}: {msg}")
