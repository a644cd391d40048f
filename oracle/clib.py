"""ctypes bindings of the oracle's C restatement (`nca_oracle.c`), built by `oracle/Makefile`.

Test infrastructure only. `build()` compiles it when the shared object is missing or stale.
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_DIR = os.path.dirname(os.path.abspath(__file__))
_SO = os.path.join(_DIR, "_build", "libnca_oracle.so")
_lib = None


def build(force: bool = False) -> str:
    src = os.path.join(_DIR, "nca_oracle.c")
    if force or not os.path.exists(_SO) or os.path.getmtime(_SO) < os.path.getmtime(src):
        subprocess.run(["make", "-C", _DIR, "-B" if force else "all"], check=True,
                       stdout=subprocess.DEVNULL)
    return _SO


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_SO):
            build()
        L = ctypes.CDLL(_SO)
        f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
        u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
        i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
        u32p = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")
        L.oracle_philox4x32_10.argtypes = [u32p, u32p, u32p]
        L.oracle_cell_uniform.argtypes = [ctypes.c_uint64, ctypes.c_uint32, ctypes.c_uint32,
                                          ctypes.c_uint32]
        L.oracle_cell_uniform.restype = ctypes.c_float
        L.oracle_fire_mask.argtypes = [
            ctypes.c_uint64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int, ctypes.c_int,
            ctypes.c_float, ctypes.c_float, ctypes.c_float, ctypes.c_void_p, ctypes.c_void_p, u8p,
        ]
        L.oracle_expf.argtypes = [ctypes.c_float]
        L.oracle_expf.restype = ctypes.c_float
        L.oracle_readout.argtypes = [
            f32p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
            ctypes.c_int, ctypes.c_int, ctypes.c_int, f32p, f32p, ctypes.c_void_p,
            ctypes.c_void_p, ctypes.c_void_p,
        ]
        L.oracle_conf_select.argtypes = [f32p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                         ctypes.c_int, i32p]
        _lib = L
    return _lib


def philox(ctr, key) -> np.ndarray:
    out = np.zeros(4, np.uint32)
    lib().oracle_philox4x32_10(np.asarray(ctr, np.uint32), np.asarray(key, np.uint32), out)
    return out


def expf(x: float) -> float:
    return lib().oracle_expf(ctypes.c_float(x))


def fire_mask(seed, row0, rows, step, hw, p, p_low=None, tau=None, conf=None, given=None):
    """(rows, hw) uint8; adaptive when p_low, tau and conf are given."""
    out = np.zeros(rows * hw, np.uint8)
    conf_p = given_p = None
    keep = []
    if p_low is not None and tau is not None and conf is not None:
        c = np.ascontiguousarray(conf, np.float32).reshape(-1)
        keep.append(c)
        conf_p = c.ctypes.data
        if given is not None:
            g = np.ascontiguousarray(given, np.uint8).reshape(-1)
            keep.append(g)
            given_p = g.ctypes.data
    lib().oracle_fire_mask(int(seed) & 0xFFFFFFFFFFFFFFFF, row0, step, rows, hw, p,
                           0.0 if p_low is None else p_low, 0.0 if tau is None else tau,
                           conf_p, given_p, out)
    return out.reshape(rows, hw)


def readout(x: np.ndarray, out_offset: int, c_out: int, head_kind: int, head_w: np.ndarray,
            head_b: np.ndarray | None):
    """x: (rows, C, H, W) fp32. Returns (conf_cell (rows,H,W), conf_board (rows,), argmax)."""
    x = np.ascontiguousarray(x, np.float32)
    R, C, H, W = x.shape
    hw_ = np.ascontiguousarray(head_w, np.float32).reshape(-1, c_out)
    n_out = hw_.shape[0]
    hb = np.ascontiguousarray(np.zeros(n_out) if head_b is None else head_b, np.float32)
    cc = np.zeros((R, H, W), np.float32)
    cb = np.zeros(R, np.float32)
    am = np.zeros((R, H, W), np.int32)
    lib().oracle_readout(x, R, C, H, W, out_offset, c_out, n_out, head_kind, hw_.reshape(-1),
                         hb, cc.ctypes.data, cb.ctypes.data, am.ctypes.data)
    return cc, cb, am


def conf_select(conf: np.ndarray, alive: np.ndarray | None, k: int) -> np.ndarray:
    conf = np.ascontiguousarray(conf, np.float32)
    N, K = conf.shape
    best = np.zeros(N, np.int32)
    a = None if alive is None else np.ascontiguousarray(alive, np.uint8)
    lib().oracle_conf_select(conf, None if a is None else a.ctypes.data, N, K, k, best)
    return best
