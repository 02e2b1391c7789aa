"""ctypes binding of the oracle (libgdn_ref.so), the CPU restatement of quotebound's gated delta rule.

Test infrastructure only: tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg compare the kernels'
results with it.
Arrays are numpy, float32 or float64, in the layouts of gdn_ref.h; g is the log-decay unless g_is_log=False.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libgdn_ref.so")
_lib = None


class _Shape(ctypes.Structure):
    _fields_ = [
        ("B", ctypes.c_int),
        ("T", ctypes.c_int),
        ("Hk", ctypes.c_int),
        ("Hv", ctypes.c_int),
        ("Dk", ctypes.c_int),
        ("Dv", ctypes.c_int),
        ("chunk", ctypes.c_int),
        ("g_is_log", ctypes.c_int),
        ("cu_seqlens", ctypes.POINTER(ctypes.c_int)),
        ("n_seqs", ctypes.c_int),
    ]


def build() -> str:
    """Compiles libgdn_ref.so with the Makefile beside this file."""
    subprocess.run(["make", "-C", _HERE, "-s"], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            raise RuntimeError(f"{_LIB_PATH} is not built (make -C oracle)")
        L = ctypes.CDLL(_LIB_PATH)
        P = ctypes.c_void_p
        for suf in ("f32", "f64"):
            f = getattr(L, f"gdn_ref_fwd_{suf}")
            f.argtypes = [ctypes.POINTER(_Shape)] + [P] * 9
            f.restype = ctypes.c_int
            b = getattr(L, f"gdn_ref_bwd_{suf}")
            b.argtypes = [ctypes.POINTER(_Shape)] + [P] * 14
            b.restype = ctypes.c_int
        L.gdn_ref_num_chunks.argtypes = [ctypes.POINTER(_Shape)]
        L.gdn_ref_num_chunks.restype = ctypes.c_long
        L.gdn_ref_threads.restype = ctypes.c_int
        L.gdn_ref_set_threads.argtypes = [ctypes.c_int]
        _lib = L
    return _lib


def threads() -> int:
    return lib().gdn_ref_threads()


def set_threads(n: int) -> None:
    lib().gdn_ref_set_threads(int(n))


def _shape(q, v, chunk, g_is_log, cu_seqlens):
    B, T, Hk, Dk = q.shape
    Hv, Dv = v.shape[2], v.shape[3]
    sh = _Shape(B, T, Hk, Hv, Dk, Dv, chunk, 1 if g_is_log else 0, None, 0)
    keep = None
    if cu_seqlens is not None:
        keep = np.ascontiguousarray(cu_seqlens, dtype=np.int32)
        sh.cu_seqlens = keep.ctypes.data_as(ctypes.POINTER(ctypes.c_int))
        sh.n_seqs = len(keep) - 1
    return sh, keep


def _ptr(x):
    return None if x is None else x.ctypes.data


def _as(x, dt):
    return None if x is None else np.ascontiguousarray(x, dtype=dt)


def num_chunks(T, chunk=64, B=1, cu_seqlens=None):
    if cu_seqlens is None:
        return B * ((T + chunk - 1) // chunk)
    lens = np.diff(np.asarray(cu_seqlens))
    return int(sum((int(l) + chunk - 1) // chunk for l in lens))


def fwd(q, k, v, g, beta, s0=None, *, chunk=64, g_is_log=True, cu_seqlens=None, dtype=np.float64):
    """Returns (y, s_out, ckpt)."""
    dt = np.dtype(dtype)
    q, k, v, g, beta, s0 = (_as(x, dt) for x in (q, k, v, g, beta, s0))
    sh, keep = _shape(q, v, chunk, g_is_log, cu_seqlens)
    N = sh.n_seqs if cu_seqlens is not None else sh.B
    y = np.empty(v.shape, dt)
    s_out = np.empty((N, sh.Hv, sh.Dv, sh.Dk), dt)
    nc = num_chunks(sh.T, chunk, sh.B, cu_seqlens)
    ckpt = np.empty((nc, sh.Hv, sh.Dv, sh.Dk), dt)
    f = lib().gdn_ref_fwd_f64 if dt == np.float64 else lib().gdn_ref_fwd_f32
    rc = f(ctypes.byref(sh), *map(_ptr, (q, k, v, g, beta, s0, y, s_out, ckpt)))
    if rc:
        raise ValueError("oracle forward rejected the shape")
    del keep
    return y, s_out, ckpt


def bwd(q, k, v, g, beta, ckpt, dy, ds_out=None, *, chunk=64, g_is_log=True, cu_seqlens=None, dtype=np.float64):
    """Returns (dq, dk, dv, dg, dbeta, ds0)."""
    dt = np.dtype(dtype)
    q, k, v, g, beta, ckpt, dy, ds_out = (_as(x, dt) for x in (q, k, v, g, beta, ckpt, dy, ds_out))
    sh, keep = _shape(q, v, chunk, g_is_log, cu_seqlens)
    N = sh.n_seqs if cu_seqlens is not None else sh.B
    dq, dk = np.empty(q.shape, dt), np.empty(k.shape, dt)
    dv = np.empty(v.shape, dt)
    dg, dbeta = np.empty(g.shape, dt), np.empty(beta.shape, dt)
    ds0 = np.empty((N, sh.Hv, sh.Dv, sh.Dk), dt)
    f = lib().gdn_ref_bwd_f64 if dt == np.float64 else lib().gdn_ref_bwd_f32
    rc = f(ctypes.byref(sh), *map(_ptr, (q, k, v, g, beta, ckpt, dy, ds_out, dq, dk, dv, dg, dbeta, ds0)))
    if rc:
        raise ValueError("oracle backward rejected the shape")
    del keep
    return dq, dk, dv, dg, dbeta, ds0


def fwd_bwd(inputs: dict, *, chunk=64, cu_seqlens=None, dtype=np.float64):
    """Forward then backward on a dict of host arrays (keys q, k, v, g, beta, s0, dy, ds_out); g is log-decay."""
    y, s_out, ckpt = fwd(inputs["q"], inputs["k"], inputs["v"], inputs["g"], inputs["beta"], inputs.get("s0"),
                         chunk=chunk, cu_seqlens=cu_seqlens, dtype=dtype)
    grads = bwd(inputs["q"], inputs["k"], inputs["v"], inputs["g"], inputs["beta"], ckpt, inputs["dy"],
                inputs.get("ds_out"), chunk=chunk, cu_seqlens=cu_seqlens, dtype=dtype)
    names = ("dq", "dk", "dv", "dg", "dbeta", "ds0")
    out = {"y": y, "s_out": s_out, "ckpt": ckpt}
    out.update(dict(zip(names, grads)))
    return out
