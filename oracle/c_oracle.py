"""ctypes binding of oracle/ring_oracle.c (test infrastructure only)."""
from __future__ import annotations

import ctypes

import numpy as np

from .build import LIBRARY, build

_lib = None


def _load():
    global _lib
    if _lib is None:
        if not LIBRARY.exists():
            build()
        lib = ctypes.CDLL(str(LIBRARY))
        dp = ctypes.POINTER(ctypes.c_double)
        ip = ctypes.POINTER(ctypes.c_int)
        lib.oracle_tr_forward_f64.argtypes = [dp, ctypes.c_int, dp, dp, dp, ip, ip, ctypes.c_int, dp]
        lib.oracle_tr_forward_f64.restype = ctypes.c_int
        lib.oracle_dense_weight_f64.argtypes = [dp, dp, dp, ip, ip, ctypes.c_int, dp]
        lib.oracle_dense_weight_f64.restype = ctypes.c_int
        _lib = lib
    return _lib


def _dp(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_double))


def _modes(cores):
    g1, g2, g3 = cores
    ins = (ctypes.c_int * 3)(g1.shape[2], g2.shape[2], g3.shape[2])
    outs = (ctypes.c_int * 3)(g1.shape[1], g2.shape[1], g3.shape[1])
    return ins, outs


def tr_forward(x, cores):
    lib = _load()
    x = np.ascontiguousarray(x, dtype=np.float64)
    cs = [np.ascontiguousarray(c, dtype=np.float64) for c in cores]
    ins, outs = _modes(cs)
    out = cs[0].shape[1] * cs[1].shape[1] * cs[2].shape[1]
    y = np.empty((x.shape[0], out), dtype=np.float64)
    status = lib.oracle_tr_forward_f64(_dp(x), x.shape[0], _dp(cs[0]), _dp(cs[1]), _dp(cs[2]),
                                       ins, outs, cs[0].shape[0], _dp(y))
    if status:
        raise RuntimeError(f"oracle_tr_forward_f64 failed with status {status}")
    return y


def dense_weight(cores):
    lib = _load()
    cs = [np.ascontiguousarray(c, dtype=np.float64) for c in cores]
    ins, outs = _modes(cs)
    w = np.empty((outs[0] * outs[1] * outs[2], ins[0] * ins[1] * ins[2]), dtype=np.float64)
    status = lib.oracle_dense_weight_f64(_dp(cs[0]), _dp(cs[1]), _dp(cs[2]), ins, outs,
                                         cs[0].shape[0], _dp(w))
    if status:
        raise RuntimeError(f"oracle_dense_weight_f64 failed with status {status}")
    return w
