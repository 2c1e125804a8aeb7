"""ctypes binding of the C restatement (``gdn_ref.c``): test infrastructure
only, same import rule as the rest of ``oracle/``."""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libgdn_ref.so")
_lib = None


def build() -> str:
    """Compile ``libgdn_ref.so`` with the committed Makefile."""

    subprocess.run(["make", "-s", "-B", "-C", _HERE, "libgdn_ref.so"], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        fp = ctypes.POINTER(ctypes.c_float)
        i = ctypes.c_int
        _lib.gdn_ref_scan_f32.argtypes = [fp] * 8 + [i] * 6
        _lib.gdn_ref_scan_f32.restype = None
        _lib.gdn_ref_decode_f32.argtypes = [fp] * 12 + [ctypes.c_float, fp] + [i] * 7
        _lib.gdn_ref_decode_f32.restype = None
        _lib.gdn_ref_bf16_of_double.argtypes = [ctypes.c_double]
        _lib.gdn_ref_bf16_of_double.restype = ctypes.c_float
    return _lib


def bf16_of_double(x) -> np.ndarray:
    """The C oracle's one rounding of each float64 to bfloat16."""

    f = lib().gdn_ref_bf16_of_double
    return np.array([f(float(v)) for v in np.asarray(x, np.float64).reshape(-1)], np.float32)


def _p(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float)) if a is not None else None


def _f32(a):
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32))


def scan(q, k, v, g, beta, state):
    """Batched sequential scan: q/k ``(B, L, Hk, Dk)``, v ``(B, L, Hv, Dv)``,
    g/beta ``(B, L, Hv)``, state ``(B, Hv, Dv, Dk)``. Returns ``(y, state)``."""

    q, k, v, g, beta, state = map(_f32, (q, k, v, g, beta, state))
    B, L, Hk, Dk = q.shape
    Hv, Dv = v.shape[-2:]
    out = np.empty_like(state)
    y = np.empty(v.shape, np.float32)
    lib().gdn_ref_scan_f32(_p(q), _p(k), _p(v), _p(g), _p(beta), _p(state), _p(out), _p(y),
                           B, L, Hk, Hv, Dk, Dv)
    return y, out


def decode_step(qkv, conv_state, conv_w, a, b, A_log, dt_bias, state, z, norm_w, eps, dims,
                act_bf16, state_out=None):
    """One fused decode step (see ``gdn_ref.c``). Returns
    ``(out, new_conv_state, new_state)``; ``state_out`` may be ``state`` for
    an in-place update."""

    Hk, Hv, Dk, Dv = dims
    qkv, conv_state, conv_w, a, b, A_log, dt_bias = map(
        _f32, (qkv, conv_state, conv_w, a, b, A_log, dt_bias))
    state = _f32(state)
    B = qkv.shape[0]
    K = conv_w.shape[1]
    z = None if z is None else _f32(z)
    norm_w = None if norm_w is None else _f32(norm_w)
    conv_out = np.empty_like(conv_state)
    if state_out is None:
        state_out = np.empty_like(state)
    out = np.empty((B, Hv, Dv), np.float32)
    lib().gdn_ref_decode_f32(_p(qkv), _p(conv_state), _p(conv_out), _p(conv_w), _p(a), _p(b),
                             _p(A_log), _p(dt_bias), _p(state), _p(state_out), _p(z),
                             _p(norm_w), float(eps), _p(out), B, Hk, Hv, Dk, Dv, K,
                             int(bool(act_bf16)))
    return out, conv_out, state_out
