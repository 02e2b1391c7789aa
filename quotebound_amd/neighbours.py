"""The layer's pointwise neighbours of the recurrence on torch device tensors, through the C ABI's
qb_gdn_prologue_* and qb_gdn_epilogue_* (reference src/deltanet.cpp):

  prologue(q_raw, k_raw, a, b, a_log, dt_bias) -> (q, k, beta, log_decay)     :22-33, :94-100
      q = (1/Dk) rms_norm(q_raw), k = Dk^-1/2 rms_norm(k_raw), beta = sigmoid(b),
      log_decay = -exp(a_log) softplus(a + dt_bias)  (feed it to gated_delta with log_decay=True)
  epilogue(y, z, norm_w, eps) -> o                                              :35-45, :122
      o = silu(z) rms_norm(y, norm_w, eps)

q_raw, k_raw [B, T, Hk, Dk]; a, b [B, T, Hv]; y, z [B, T, Hv, Dv]; the activations in bf16 or float32, the parameters
(a_log, dt_bias [Hv]; norm_w [Dv]) in float32. Both are differentiable (torch autograd calls the library's
backward entry points); all arithmetic runs in the library's HIP kernels.
"""
from __future__ import annotations

import torch

from . import _lib


def _ptr(t):
    return None if t is None else t.data_ptr()


def _stream(device):
    return torch.cuda.current_stream(device).cuda_stream


def _act_dtype(*ts):
    return torch.bfloat16 if all(t.dtype == torch.bfloat16 for t in ts) else torch.float32


def _desc(B, T, Hk, Hv, Dk, Dv, dtype):
    d, keep = _lib.make_desc(B, T, Hk, Hv, Dk, Dv, dtype=_lib.BF16 if dtype == torch.bfloat16 else _lib.F32)
    return d, keep


def _ws(desc, device):
    return torch.empty(max(_lib.neighbours_workspace_bytes(desc), 1), dtype=torch.uint8, device=device)


def _check(*ts):
    if not all(t.is_cuda for t in ts):
        raise RuntimeError("gated delta neighbours: tensors must be on a HIP device (there is no CPU path)")


def prologue_forward(q_raw, k_raw, a, b, a_log, dt_bias):
    _check(q_raw, k_raw, a, b, a_log, dt_bias)
    dt = _act_dtype(q_raw, k_raw, a, b)
    c = lambda t: t.to(dt).contiguous()  # noqa: E731
    q_raw, k_raw, a, b = c(q_raw), c(k_raw), c(a), c(b)
    a_log, dt_bias = a_log.float().contiguous(), dt_bias.float().contiguous()
    B, T, Hk, Dk = q_raw.shape
    Hv = a.shape[2]
    desc, keep = _desc(B, T, Hk, Hv, Dk, Dk, dt)
    q, k = torch.empty_like(q_raw), torch.empty_like(k_raw)
    beta = torch.empty_like(b)
    log_decay = torch.empty(a.shape, dtype=torch.float32, device=a.device)
    _lib.prologue_fwd(desc, _ptr(q_raw), _ptr(k_raw), _ptr(a), _ptr(b), _ptr(a_log), _ptr(dt_bias), _ptr(q), _ptr(k),
                      _ptr(beta), _ptr(log_decay), _stream(a.device))
    del keep
    return q, k, beta, log_decay


def prologue_backward(q_raw, k_raw, a, b, a_log, dt_bias, dq, dk, dbeta, dlog_decay):
    """Returns (dq_raw, dk_raw, da, db, da_log, ddt_bias)."""
    dt = _act_dtype(q_raw, k_raw, a, b)
    c = lambda t: t.to(dt).contiguous()  # noqa: E731
    q_raw, k_raw, a, b, dq, dk, dbeta = map(c, (q_raw, k_raw, a, b, dq, dk, dbeta))
    a_log, dt_bias = a_log.float().contiguous(), dt_bias.float().contiguous()
    dlog_decay = dlog_decay.float().contiguous()
    B, T, Hk, Dk = q_raw.shape
    Hv = a.shape[2]
    desc, keep = _desc(B, T, Hk, Hv, Dk, Dk, dt)
    dq_raw, dk_raw, da, db = (torch.empty_like(t) for t in (q_raw, k_raw, a, b))
    da_log, ddt = torch.empty_like(a_log), torch.empty_like(dt_bias)
    _lib.prologue_bwd(desc, _ptr(q_raw), _ptr(k_raw), _ptr(a), _ptr(b), _ptr(a_log), _ptr(dt_bias), _ptr(dq),
                      _ptr(dk), _ptr(dbeta), _ptr(dlog_decay), _ptr(dq_raw), _ptr(dk_raw), _ptr(da), _ptr(db),
                      _ptr(da_log), _ptr(ddt), _ptr(_ws(desc, a.device)), _stream(a.device))
    del keep
    return dq_raw, dk_raw, da, db, da_log, ddt


def epilogue_forward(y, z, norm_w, eps):
    _check(y, z, norm_w)
    dt = _act_dtype(y, z)
    y, z = y.to(dt).contiguous(), z.to(dt).contiguous()
    B, T, Hv, Dv = y.shape
    desc, keep = _desc(B, T, Hv, Hv, Dv, Dv, dt)
    o = torch.empty_like(y)
    _lib.epilogue_fwd(desc, _ptr(y), _ptr(z), _ptr(norm_w.float().contiguous()), float(eps), _ptr(o),
                      _stream(y.device))
    del keep
    return o


def epilogue_backward(y, z, norm_w, eps, dout):
    """Returns (dy, dz, dnorm_w)."""
    dt = _act_dtype(y, z)
    y, z, dout = y.to(dt).contiguous(), z.to(dt).contiguous(), dout.to(dt).contiguous()
    B, T, Hv, Dv = y.shape
    desc, keep = _desc(B, T, Hv, Hv, Dv, Dv, dt)
    w = norm_w.float().contiguous()
    dy, dz, dw = torch.empty_like(y), torch.empty_like(z), torch.empty_like(w)
    _lib.epilogue_bwd(desc, _ptr(y), _ptr(z), _ptr(w), float(eps), _ptr(dout), _ptr(dy), _ptr(dz), _ptr(dw),
                      _ptr(_ws(desc, y.device)), _stream(y.device))
    del keep
    return dy, dz, dw


class _Prologue(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q_raw, k_raw, a, b, a_log, dt_bias):
        out = prologue_forward(q_raw, k_raw, a, b, a_log, dt_bias)
        ctx.save_for_backward(q_raw, k_raw, a, b, a_log, dt_bias)
        return out

    @staticmethod
    def backward(ctx, dq, dk, dbeta, dlog_decay):
        q_raw, k_raw, a, b, a_log, dt_bias = ctx.saved_tensors
        z = lambda g, like, dt=None: torch.zeros_like(like, dtype=dt) if g is None else g  # noqa: E731
        grads = prologue_backward(q_raw, k_raw, a, b, a_log, dt_bias, z(dq, q_raw), z(dk, k_raw), z(dbeta, b),
                                  z(dlog_decay, a, torch.float32))
        like = (q_raw, k_raw, a, b, a_log, dt_bias)
        return tuple(g.to(t.dtype) for g, t in zip(grads, like))


class _Epilogue(torch.autograd.Function):
    @staticmethod
    def forward(ctx, y, z, norm_w, eps):
        ctx.save_for_backward(y, z, norm_w)
        ctx.eps = eps
        return epilogue_forward(y, z, norm_w, eps)

    @staticmethod
    def backward(ctx, dout):
        y, z, norm_w = ctx.saved_tensors
        dy, dz, dw = epilogue_backward(y, z, norm_w, ctx.eps, dout)
        return dy.to(y.dtype), dz.to(z.dtype), dw.to(norm_w.dtype), None


def prologue(q_raw, k_raw, a, b, a_log, dt_bias):
    """(q, k, beta, log_decay); differentiable."""
    return _Prologue.apply(q_raw, k_raw, a, b, a_log, dt_bias)


def epilogue(y, z, norm_w, eps):
    """o = silu(z) rms_norm(y, norm_w, eps); differentiable."""
    return _Epilogue.apply(y, z, norm_w, eps)
