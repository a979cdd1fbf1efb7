"""ctypes binding to the reference's own C forward pieces, compiled from source by ``oracle/Makefile`` into
``oracle/_ref/libgdn_ref.so``.  TEST INFRASTRUCTURE ONLY (a checker for the NumPy oracle).

Entry points mirror ``engine/include/gdn.h:7-38`` and ``engine/include/ops.h:7-11``.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

_LIB_PATH = Path(__file__).resolve().parent / "_ref" / "libgdn_ref.so"
_lib = None
_F = ctypes.POINTER(ctypes.c_float)


def available() -> bool:
    return _LIB_PATH.exists()


def _load():
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            raise FileNotFoundError(f"{_LIB_PATH} is not built (run: make -C oracle)")
        lib = ctypes.CDLL(os.fspath(_LIB_PATH))
        lib.gdn_recurrent_step.argtypes = [_F] * 7 + [ctypes.c_int] * 4
        lib.gdn_conv_step.argtypes = [_F, _F, _F, _F, ctypes.c_int, ctypes.c_int]
        lib.gdn_l2norm.argtypes = [_F, ctypes.c_int, ctypes.c_float, ctypes.c_float]
        lib.gdn_gates.argtypes = [_F] * 6 + [ctypes.c_int]
        lib.op_rmsnorm.argtypes = [_F, _F, _F, ctypes.c_int, ctypes.c_float]
        lib.op_silu_mul.argtypes = [_F, _F, _F, ctypes.c_int]
        _lib = lib
    return _lib


def _p(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(_F)


def recurrence(q, k, v, g, beta, state0=None):
    """Whole-sequence forward by repeated ``gdn_recurrent_step`` (engine/include/gdn.h:27-38, engine/src/gdn.c:63-108).

    q, k [T,Hk,Dk]; v [T,Hv,Dv]; g, beta [T,Hv] (multiplicative decay); state [Hv,Dv,Dk].
    Returns (y [T,Hv,Dv], final state).  No mask, scalar gates (the C spec's scope).
    """
    lib = _load()
    T, Hk, Dk = q.shape
    Hv, Dv = v.shape[1:]
    state = (np.zeros((Hv, Dv, Dk), np.float32) if state0 is None
             else np.ascontiguousarray(state0, np.float32).copy())
    ys = np.zeros((T, Hv, Dv), np.float32)
    for t in range(T):
        y = np.zeros(Hv * Dv, np.float32)
        args = [np.ascontiguousarray(x[t], np.float32) for x in (q, k, v, g, beta)]
        lib.gdn_recurrent_step(_p(y), _p(state), *[_p(a) for a in args], Hk, Hv, Dk, Dv)
        ys[t] = y.reshape(Hv, Dv)
    return ys, state


def gates(a, b, A_log, dt_bias):
    lib = _load()
    Hv = a.size
    g = np.zeros(Hv, np.float32)
    beta = np.zeros(Hv, np.float32)
    lib.gdn_gates(_p(g), _p(beta), *[_p(np.ascontiguousarray(x, np.float32)) for x in
                                      (a, b, A_log, dt_bias)], Hv)
    return g, beta


def l2norm(x, eps, scale):
    lib = _load()
    out = np.ascontiguousarray(x, np.float32).copy()
    n = out.shape[-1]
    flat = out.reshape(-1, n)
    for row in flat:
        lib.gdn_l2norm(row.ctypes.data_as(_F), n, eps, scale)
    return flat.reshape(out.shape)


def conv_silu(x, w):
    """x [T,C], w [C,K] -> out [T,C] via gdn_conv_step with a zero initial state."""
    lib = _load()
    T, C = x.shape
    K = w.shape[1]
    state = np.zeros((K - 1) * C, np.float32)
    wf = np.ascontiguousarray(w, np.float32).ravel()
    out = np.zeros((T, C), np.float32)
    for t in range(T):
        o = np.zeros(C, np.float32)
        xt = np.ascontiguousarray(x[t], np.float32)
        lib.gdn_conv_step(_p(o), _p(state), _p(xt), _p(wf), C, K)
        out[t] = o
    return out


def rmsnorm(x, w, eps):
    lib = _load()
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros_like(x)
    lib.op_rmsnorm(_p(out), _p(x), _p(np.ascontiguousarray(w, np.float32)), x.size, eps)
    return out


def silu_mul(gate, up):
    lib = _load()
    gate = np.ascontiguousarray(gate, np.float32)
    out = np.zeros_like(gate)
    lib.op_silu_mul(_p(out), _p(gate), _p(np.ascontiguousarray(up, np.float32)), gate.size)
    return out
