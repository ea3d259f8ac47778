"""ctypes binding of oracle/canon.c (test infrastructure only)."""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None


def build() -> str:
    """Compiles liboracle.so with the committed Makefile."""
    res = subprocess.run(["make", "-s", "-C", _HERE, "liboracle.so"], capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{res.stdout}\n{res.stderr}")
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        fp = ctypes.POINTER(ctypes.c_float)
        dp = ctypes.POINTER(ctypes.c_double)
        L.vnx_ref_exp_canon.restype = ctypes.c_float
        L.vnx_ref_exp_canon.argtypes = [ctypes.c_float]
        L.vnx_ref_exp_canon_arr.restype = None
        L.vnx_ref_exp_canon_arr.argtypes = [fp, fp, ctypes.c_int64]
        L.vnx_ref_div_markstein.restype = ctypes.c_float
        L.vnx_ref_div_markstein.argtypes = [ctypes.c_float, ctypes.c_float]
        L.vnx_ref_markstein_mismatches.restype = ctypes.c_int64
        L.vnx_ref_markstein_mismatches.argtypes = [ctypes.c_float]
        L.vnx_ref_resid_weights.restype = None
        L.vnx_ref_resid_weights.argtypes = [fp, fp, ctypes.c_int64, ctypes.c_float, ctypes.c_float,
                                            ctypes.c_float, ctypes.c_float, ctypes.c_float, fp, fp]
        L.vnx_ref_icdf.restype = ctypes.c_int64
        L.vnx_ref_icdf.argtypes = [fp, ctypes.c_int64, ctypes.c_double, dp, dp, dp]
        _lib = L
    return _lib


def _fptr(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


def exp_canon(t) -> np.ndarray:
    t = np.asarray(t, dtype=np.float32)
    shape = t.shape
    flat = np.ascontiguousarray(t.reshape(-1))
    out = np.empty_like(flat)
    lib().vnx_ref_exp_canon_arr(_fptr(flat), _fptr(out), flat.size)
    return out.reshape(shape)


def markstein_mismatches(T: float) -> int:
    return int(lib().vnx_ref_markstein_mismatches(np.float32(T)))


def div_markstein(l: float, T: float) -> np.float32:
    return np.float32(lib().vnx_ref_div_markstein(np.float32(l), np.float32(T)))


def resid_weights(P: np.ndarray, Q, T: float, thr_p: float, thr_q: float, Lp: float, Lq: float):
    """Returns (w_r, w_p) for one row pair (Q None = bonus draw from P)."""
    P = np.ascontiguousarray(P, dtype=np.float32)
    V = P.shape[0]
    w_r = np.empty(V, np.float32)
    w_p = np.empty(V, np.float32)
    qptr = None
    if Q is not None:
        Q = np.ascontiguousarray(Q, dtype=np.float32)
        qptr = _fptr(Q)
    lib().vnx_ref_resid_weights(_fptr(P), qptr, V, np.float32(T), np.float32(thr_p), np.float32(thr_q),
                                np.float32(Lp), np.float32(Lq), _fptr(w_r), _fptr(w_p))
    return w_r, w_p


def icdf(w: np.ndarray, u: float):
    """Returns (index, C_{j-1}, C_j, total) of the inverse-CDF draw: the
    first j with C_j > u * total, u taken as given (a float32 uniform
    converts to double exactly; a float64 one is not rounded)."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    before = ctypes.c_double(0.0)
    after = ctypes.c_double(0.0)
    total = ctypes.c_double(0.0)
    j = lib().vnx_ref_icdf(_fptr(w), w.shape[0], float(u), ctypes.byref(before),
                           ctypes.byref(after), ctypes.byref(total))
    return int(j), before.value, after.value, total.value
