"""ctypes binding of libqb_gdn.so, the C ABI declared in include/qb_gdn.h.

There is no fallback: if the library is missing or fails to load, every call raises.
"""
from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libqb_gdn.so")
HEADER_PATH = os.path.join(os.path.dirname(_HERE), "include", "qb_gdn.h")

F32, BF16 = 0, 1
RECURRENT, CHUNKED = 1, 2
MAX_SEQS = 255


class Desc(ctypes.Structure):
    """qb_gdn_desc."""

    _fields_ = [
        ("B", ctypes.c_int32),
        ("T", ctypes.c_int32),
        ("Hk", ctypes.c_int32),
        ("Hv", ctypes.c_int32),
        ("Dk", ctypes.c_int32),
        ("Dv", ctypes.c_int32),
        ("chunk", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
        ("g_is_log", ctypes.c_int32),
        ("design", ctypes.c_int32),
        ("out_f32", ctypes.c_int32),
        ("cu_seqlens", ctypes.POINTER(ctypes.c_int32)),
        ("n_seqs", ctypes.c_int32),
        ("trace_events", ctypes.POINTER(ctypes.c_void_p)),
        ("n_trace_events", ctypes.c_int32),
    ]


_lib = None


def load():
    """Loads libqb_gdn.so (built by __graft_entry__.build() or `make -C quotebound_amd`)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is missing: build it with `make -C quotebound_amd` (no fallback exists)")
    L = ctypes.CDLL(LIB_PATH)
    P, D = ctypes.c_void_p, ctypes.POINTER(Desc)
    L.qb_gdn_version.restype = ctypes.c_char_p
    L.qb_gdn_validate.argtypes = [D, ctypes.c_char_p, ctypes.c_int]
    L.qb_gdn_validate.restype = ctypes.c_int
    L.qb_gdn_num_chunks.argtypes = [D]
    L.qb_gdn_num_chunks.restype = ctypes.c_int64
    L.qb_gdn_ckpt_bytes.argtypes = [D]
    L.qb_gdn_ckpt_bytes.restype = ctypes.c_size_t
    L.qb_gdn_workspace_bytes.argtypes = [D]
    L.qb_gdn_workspace_bytes.restype = ctypes.c_size_t
    L.qb_gdn_launches.argtypes = [D, ctypes.c_int, ctypes.c_char_p, ctypes.c_int]
    L.qb_gdn_launches.restype = ctypes.c_int
    L.qb_gdn_fwd.argtypes = [D] + [P] * 11 + [ctypes.c_char_p, ctypes.c_int]
    L.qb_gdn_fwd.restype = ctypes.c_int
    L.qb_gdn_fwd_rows.argtypes = [D] + [P] * 9 + [ctypes.c_char_p, ctypes.c_int]
    L.qb_gdn_fwd_rows.restype = ctypes.c_int
    L.qb_gdn_bwd.argtypes = [D] + [P] * 16 + [ctypes.c_char_p, ctypes.c_int]
    L.qb_gdn_bwd.restype = ctypes.c_int
    L.qb_gdn_bwd_static.argtypes = [D] + [P] * 15 + [ctypes.c_char_p, ctypes.c_int]
    L.qb_gdn_bwd_static.restype = ctypes.c_int
    L.qb_gdn_neighbours_workspace_bytes.argtypes = [D]
    L.qb_gdn_neighbours_workspace_bytes.restype = ctypes.c_size_t
    L.qb_gdn_prologue_fwd.argtypes = [D] + [P] * 11 + [ctypes.c_char_p, ctypes.c_int]
    L.qb_gdn_prologue_fwd.restype = ctypes.c_int
    L.qb_gdn_prologue_bwd.argtypes = [D] + [P] * 18 + [ctypes.c_char_p, ctypes.c_int]
    L.qb_gdn_prologue_bwd.restype = ctypes.c_int
    L.qb_gdn_fwd_prologue.argtypes = [D] + [P] * 17 + [ctypes.c_char_p, ctypes.c_int]
    L.qb_gdn_fwd_prologue.restype = ctypes.c_int
    L.qb_gdn_bwd_prologue.argtypes = [D] + [P] * 24 + [ctypes.c_char_p, ctypes.c_int]
    L.qb_gdn_bwd_prologue.restype = ctypes.c_int
    F = ctypes.c_float
    L.qb_gdn_epilogue_fwd.argtypes = [D, P, P, P, F, P, P, ctypes.c_char_p, ctypes.c_int]
    L.qb_gdn_epilogue_fwd.restype = ctypes.c_int
    L.qb_gdn_epilogue_bwd.argtypes = [D, P, P, P, F, P, P, P, P, P, P, ctypes.c_char_p, ctypes.c_int]
    L.qb_gdn_epilogue_bwd.restype = ctypes.c_int
    _lib = L
    return L


def make_desc(B, T, Hk, Hv, Dk, Dv, *, dtype=BF16, g_is_log=True, design=CHUNKED, cu_seqlens=None, chunk=64,
              out_f32=False):
    """Returns (desc, keepalive): keepalive holds the host cu_seqlens array the desc points at."""
    d = Desc(B, T, Hk, Hv, Dk, Dv, chunk, dtype, 1 if g_is_log else 0, design, 1 if out_f32 else 0, None, 0, None, 0)
    keep = None
    if cu_seqlens is not None:
        vals = [int(x) for x in cu_seqlens]
        keep = (ctypes.c_int32 * len(vals))(*vals)
        d.cu_seqlens = ctypes.cast(keep, ctypes.POINTER(ctypes.c_int32))
        d.n_seqs = len(vals) - 1
    return d, keep


def validate(desc) -> str | None:
    """None when the library accepts desc, else its reason."""
    err = ctypes.create_string_buffer(512)
    rc = load().qb_gdn_validate(ctypes.byref(desc), err, len(err))
    return None if rc == 0 else err.value.decode()


def launches(desc, which: int) -> list[str]:
    """Names of the kernels qb_gdn_fwd (which=0) or qb_gdn_bwd (which=1) launches, in order."""
    buf = ctypes.create_string_buffer(1024)
    n = load().qb_gdn_launches(ctypes.byref(desc), which, buf, len(buf))
    if n < 0:
        raise RuntimeError(validate(desc) or "invalid descriptor")
    names = buf.value.decode().split(",") if n else []
    assert len(names) == n
    return names


def set_trace(desc, events) -> object:
    """Points desc at a list of hipEvent_t handles (ints); returns the array to keep alive."""
    arr = (ctypes.c_void_p * len(events))(*events)
    desc.trace_events = ctypes.cast(arr, ctypes.POINTER(ctypes.c_void_p))
    desc.n_trace_events = len(events)
    return arr


def num_chunks(desc) -> int:
    return int(load().qb_gdn_num_chunks(ctypes.byref(desc)))


def ckpt_bytes(desc) -> int:
    return int(load().qb_gdn_ckpt_bytes(ctypes.byref(desc)))


def workspace_bytes(desc) -> int:
    return int(load().qb_gdn_workspace_bytes(ctypes.byref(desc)))


def fwd_rows(desc, q, k, v, g, beta, s0, y, row_states, stream) -> None:
    """The forward keeping the state after every token (always the recurrent design)."""
    _call(load().qb_gdn_fwd_rows, desc, q, k, v, g, beta, s0, y, row_states, stream)


def fwd(desc, q, k, v, g, beta, s0, y, s_out, ckpt, workspace, stream) -> None:
    """Pointers are ints (device addresses) or None; raises RuntimeError with the library's reason on failure."""
    err = ctypes.create_string_buffer(512)
    rc = load().qb_gdn_fwd(ctypes.byref(desc), q, k, v, g, beta, s0, y, s_out, ckpt, workspace, stream, err,
                           len(err))
    if rc != 0:
        raise RuntimeError(err.value.decode())


def bwd(desc, q, k, v, g, beta, ckpt, dy, ds_out, dq, dk, dv, dg, dbeta, ds0, workspace, stream) -> None:
    err = ctypes.create_string_buffer(512)
    rc = load().qb_gdn_bwd(ctypes.byref(desc), q, k, v, g, beta, ckpt, dy, ds_out, dq, dk, dv, dg, dbeta, ds0,
                           workspace, stream, err, len(err))
    if rc != 0:
        raise RuntimeError(err.value.decode())


def bwd_static(desc, q, k, v, g, beta, ckpt, dy, ds_out, dq, dk, dv, dg, dbeta, ds0, stream) -> None:
    """qb_gdn_bwd with the library's static per-GPU scratch in place of a workspace (no allocation)."""
    _call(load().qb_gdn_bwd_static, desc, q, k, v, g, beta, ckpt, dy, ds_out, dq, dk, dv, dg, dbeta, ds0, stream)


STATIC_SCRATCH_BYTES = 257 << 20  # QB_GDN_STATIC_SCRATCH_BYTES


def neighbours_workspace_bytes(desc) -> int:
    return int(load().qb_gdn_neighbours_workspace_bytes(ctypes.byref(desc)))


def _call(fn, desc, *args) -> None:
    err = ctypes.create_string_buffer(512)
    if fn(ctypes.byref(desc), *args, err, len(err)) != 0:
        raise RuntimeError(err.value.decode())


def fwd_prologue(desc, q_raw, k_raw, v, a, b, a_log, dt_bias, s0, q, k, beta, log_decay, y, s_out, ckpt, workspace,
                 stream) -> None:
    _call(load().qb_gdn_fwd_prologue, desc, q_raw, k_raw, v, a, b, a_log, dt_bias, s0, q, k, beta, log_decay, y, s_out,
          ckpt, workspace, stream)


def bwd_prologue(desc, q_raw, k_raw, a, b, a_log, dt_bias, q, k, v, beta, log_decay, ckpt, dy, ds_out, dq_raw,
                 dk_raw, dv, da, db, da_log, ddt_bias, ds0, workspace, stream) -> None:
    _call(load().qb_gdn_bwd_prologue, desc, q_raw, k_raw, a, b, a_log, dt_bias, q, k, v, beta, log_decay, ckpt, dy,
          ds_out, dq_raw, dk_raw, dv, da, db, da_log, ddt_bias, ds0, workspace, stream)


def prologue_fwd(desc, q_raw, k_raw, a, b, a_log, dt_bias, q, k, beta, log_decay, stream) -> None:
    _call(load().qb_gdn_prologue_fwd, desc, q_raw, k_raw, a, b, a_log, dt_bias, q, k, beta, log_decay, stream)


def prologue_bwd(desc, q_raw, k_raw, a, b, a_log, dt_bias, dq, dk, dbeta, dlog_decay, dq_raw, dk_raw, da, db, da_log,
                 ddt_bias, workspace, stream) -> None:
    _call(load().qb_gdn_prologue_bwd, desc, q_raw, k_raw, a, b, a_log, dt_bias, dq, dk, dbeta, dlog_decay, dq_raw,
          dk_raw, da, db, da_log, ddt_bias, workspace, stream)


def epilogue_fwd(desc, y, z, norm_w, eps, o, stream) -> None:
    _call(load().qb_gdn_epilogue_fwd, desc, y, z, norm_w, eps, o, stream)


def epilogue_bwd(desc, y, z, norm_w, eps, dout, dy, dz, dnorm_w, workspace, stream) -> None:
    _call(load().qb_gdn_epilogue_bwd, desc, y, z, norm_w, eps, dout, dy, dz, dnorm_w, workspace, stream)
