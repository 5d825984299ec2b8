"""ctypes loader for ``oracle/int_ref.c`` (test infrastructure only).

Builds ``oracle/_build/liboracle_int.so`` with ``make`` on first use if it is
missing.  All functions take and return numpy arrays.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "liboracle_int.so")
_lib = None


def build():
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        lib = ctypes.CDLL(_LIB_PATH)
        P, I64, F = ctypes.c_void_p, ctypes.c_int64, ctypes.c_float
        for name, args, res in [
            ("oracle_round_bf16", [F], F),
            ("oracle_quant_act_f32", [P, I64, I64, F, P, P], None),
            ("oracle_quant_act_bf16", [P, I64, I64, F, P, P], None),
            ("oracle_weight_codes_f32", [P, I64, F, P], None),
            ("oracle_weight_codes_bf16", [P, I64, F, P], None),
            ("oracle_pack_i2", [P, I64, I64, P], None),
            ("oracle_unpack_i2", [P, I64, I64, P], None),
            ("oracle_bitlinear_acc", [P, P, I64, I64, I64, P], ctypes.c_int),
        ]:
            fn = getattr(lib, name)
            fn.argtypes, fn.restype = args, res
        _lib = lib
    return _lib


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def quant_act(x: np.ndarray, eps: float = 1e-5, bf16_bits: bool = False):
    """Per-row int8 codes + scales.  ``x`` is (M, K) float32, or uint16 bf16 bits."""
    lib = _load()
    x = np.ascontiguousarray(x)
    M, K = x.shape
    q = np.empty((M, K), np.int8)
    s = np.empty((M,), np.float32)
    fn = lib.oracle_quant_act_bf16 if bf16_bits else lib.oracle_quant_act_f32
    fn(_ptr(x), M, K, eps, _ptr(q), _ptr(s))
    return q, s


def weight_codes(w: np.ndarray, s_w: float, bf16_bits: bool = False):
    lib = _load()
    w = np.ascontiguousarray(w)
    out = np.empty(w.shape, np.int8)
    fn = lib.oracle_weight_codes_bf16 if bf16_bits else lib.oracle_weight_codes_f32
    fn(_ptr(w), w.size, float(s_w), _ptr(out))
    return out


def pack_i2(codes: np.ndarray):
    lib = _load()
    codes = np.ascontiguousarray(codes, dtype=np.int8)
    N, K = codes.shape
    out = np.empty((N, (K + 3) // 4), np.uint8)
    lib.oracle_pack_i2(_ptr(codes), N, K, _ptr(out))
    return out


def unpack_i2(packed: np.ndarray, K: int):
    lib = _load()
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    N = packed.shape[0]
    out = np.empty((N, K), np.int8)
    lib.oracle_unpack_i2(_ptr(packed), N, K, _ptr(out))
    return out


def bitlinear_acc(q: np.ndarray, wcodes: np.ndarray):
    lib = _load()
    q = np.ascontiguousarray(q, dtype=np.int8)
    wcodes = np.ascontiguousarray(wcodes, dtype=np.int8)
    M, K = q.shape
    N = wcodes.shape[0]
    out = np.empty((M, N), np.int32)
    if lib.oracle_bitlinear_acc(_ptr(q), _ptr(wcodes), M, N, K, _ptr(out)) != 0:
        raise OverflowError("int32 accumulator overflow")
    return out


def round_bf16(v: float) -> float:
    return float(_load().oracle_round_bf16(v))
