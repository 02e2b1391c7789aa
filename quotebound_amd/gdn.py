"""The reference's recurrence interface on torch device tensors, running the HIP kernels through the C ABI.

  gated_delta(q, k, v, g, beta, state, train=False)      reference src/deltanet.h:17-19, src/deltanet.cpp:49-61
  gated_delta_trainable(q, k, v, g, beta, state)         reference src/delta_grad.h:14-16, src/delta_grad.cpp:201-212
  gated_delta_vjp(primals, dy, dstate)                   reference src/delta_grad.h:19-20, src/delta_grad.cpp:155-199

Shapes and meaning follow the reference: q, k [B, T, Hk, Dk]; v [B, T, Hv, Dv]; g, beta [B, T, Hv]; state
[B, Hv, Dv, Dk] float32; y comes back in q's dtype and the state in float32. g is the decay factor unless
log_decay=True, in which case it is the log-decay and its cotangent is d/d(log-decay). Errors are raised as
RuntimeError carrying the library's message (the reference throws std::runtime_error, src/delta_grad.cpp:164-170).
torch provides device memory and the stream only; all arithmetic runs in the library's HIP kernels, and there is
no CPU or eager fallback.
"""
from __future__ import annotations

import torch

from . import _lib

DEFAULT_DESIGN = None  # the chunked design where the library supports the shape and T > SHORT_T, else recurrent
# At most this many steps per sequence, the recurrent design is the faster one (4B layer shape, launches included):
# forward + backward 43.7 against 47.0 us at T = 32, 53.0 against 47.4 us at T = 48 (crossing near T = 38); a
# one-token decode call takes about 6 us with it and 15 us with the chunked design's two launches.
SHORT_T = 40


def _dev_ptr(t):
    return None if t is None else t.data_ptr()


def _stream(device):
    return torch.cuda.current_stream(device).cuda_stream


def _io_dtype(*ts):
    """bf16 when every activation is bf16, else float32 (the reference computes in float32 either way)."""
    return torch.bfloat16 if all(t.dtype == torch.bfloat16 for t in ts) else torch.float32


def _prep(q, k, v, g, beta, dtype):
    if not q.is_cuda:
        raise RuntimeError("gated delta: tensors must be on a HIP device (there is no CPU path)")
    c = lambda t: t.to(dtype).contiguous()  # noqa: E731
    return c(q), c(k), c(v), g.to(torch.float32).contiguous(), c(beta)


def _desc(q, v, dtype, g_is_log, design, cu_seqlens, out_f32):
    B, T, Hk, Dk = q.shape
    Hv, Dv = v.shape[2], v.shape[3]
    make = lambda d: _lib.make_desc(B, T, Hk, Hv, Dk, Dv,  # noqa: E731
                                    dtype=_lib.BF16 if dtype == torch.bfloat16 else _lib.F32, g_is_log=g_is_log,
                                    design=d, cu_seqlens=cu_seqlens, out_f32=out_f32)
    if design is None:
        longest = T if cu_seqlens is None else max(int(b) - int(a) for a, b in zip(cu_seqlens[:-1], cu_seqlens[1:]))
        if longest > SHORT_T:
            desc, keep = make(_lib.CHUNKED)
            if not _lib.validate(desc):
                return desc, keep
        design = _lib.RECURRENT
    return make(design)


def _workspace(desc, device):
    n = _lib.workspace_bytes(desc)
    return torch.empty(max(n, 1), dtype=torch.uint8, device=device)


def forward(q, k, v, g, beta, state=None, *, log_decay=False, design=DEFAULT_DESIGN, cu_seqlens=None,
            save_ckpt=True, out_f32=False):
    """Returns (y, s_out, ckpt); ckpt is the residual buffer the backward reads (None unless save_ckpt).
    y is in the inputs' dtype, or float32 with out_f32."""
    dtype = _io_dtype(q, k, v, beta)
    q, k, v, g, beta = _prep(q, k, v, g, beta, dtype)
    desc, keep = _desc(q, v, dtype, log_decay, design, cu_seqlens, out_f32)
    odt = torch.float32 if out_f32 else dtype
    why = _lib.validate(desc)
    if why:
        raise RuntimeError(why)
    N = q.shape[0] if cu_seqlens is None else len(cu_seqlens) - 1
    dev = q.device
    Hv, Dv, Dk = v.shape[2], v.shape[3], q.shape[3]
    s0 = None if state is None else state.to(torch.float32).contiguous()
    y = torch.empty(v.shape, dtype=odt, device=dev)
    s_out = torch.empty(N, Hv, Dv, Dk, dtype=torch.float32, device=dev)
    ckpt = None
    if save_ckpt:
        ckpt = torch.empty(max(_lib.ckpt_bytes(desc) // 4, 1), dtype=torch.float32, device=dev)
    ws = _workspace(desc, dev)
    _lib.fwd(desc, _dev_ptr(q), _dev_ptr(k), _dev_ptr(v), _dev_ptr(g), _dev_ptr(beta), _dev_ptr(s0), _dev_ptr(y),
             _dev_ptr(s_out), _dev_ptr(ckpt), _dev_ptr(ws), _stream(dev))
    del keep
    return y, s_out, ckpt


def backward(q, k, v, g, beta, ckpt, dy, ds_out=None, *, log_decay=False, design=DEFAULT_DESIGN, cu_seqlens=None,
             want_ds0=True, out_f32=False):
    """Returns (dq, dk, dv, dg, dbeta, ds0): dg and ds0 float32, the others in the inputs' dtype (float32 with
    out_f32, in which case dy is taken as float32 too)."""
    dtype = _io_dtype(q, k, v, beta)
    q, k, v, g, beta = _prep(q, k, v, g, beta, dtype)
    odt = torch.float32 if out_f32 else dtype
    dy = dy.to(odt).contiguous()
    desc, keep = _desc(q, v, dtype, log_decay, design, cu_seqlens, out_f32)
    why = _lib.validate(desc)
    if why:
        raise RuntimeError(why)
    N = q.shape[0] if cu_seqlens is None else len(cu_seqlens) - 1
    dev = q.device
    Hv, Dv, Dk = v.shape[2], v.shape[3], q.shape[3]
    dso = None if ds_out is None else ds_out.to(torch.float32).contiguous()
    dq, dk = torch.empty(q.shape, dtype=odt, device=dev), torch.empty(k.shape, dtype=odt, device=dev)
    dv, dbeta = torch.empty(v.shape, dtype=odt, device=dev), torch.empty(beta.shape, dtype=odt, device=dev)
    dg = torch.empty_like(g)
    ds0 = torch.empty(N, Hv, Dv, Dk, dtype=torch.float32, device=dev) if want_ds0 else None
    ws = _workspace(desc, dev)
    _lib.bwd(desc, _dev_ptr(q), _dev_ptr(k), _dev_ptr(v), _dev_ptr(g), _dev_ptr(beta), _dev_ptr(ckpt), _dev_ptr(dy),
             _dev_ptr(dso), _dev_ptr(dq), _dev_ptr(dk), _dev_ptr(dv), _dev_ptr(dg), _dev_ptr(dbeta), _dev_ptr(ds0),
             _dev_ptr(ws), _stream(dev))
    del keep
    return dq, dk, dv, dg, dbeta, ds0


def forward_prologue(q_raw, k_raw, v, a, b, a_log, dt_bias, state=None, *, cu_seqlens=None, out_f32=False):
    """The layer's prologue fused into the chunked forward (qb_gdn_fwd_prologue): from the raw q/k rows and gate
    inputs, (y, s_out, ckpt, q, k, beta, log_decay), the last four exactly what neighbours.prologue_forward returns,
    y, s_out and ckpt what forward(q, k, v, log_decay, beta, state, log_decay=True, design=CHUNKED) returns on them.
    bf16 activations; a_log and dt_bias float32."""
    for t in (q_raw, k_raw, v, a, b):
        if t.dtype != torch.bfloat16 or not t.is_cuda:
            raise RuntimeError("gated delta: the fused prologue takes bf16 device tensors")
    q_raw, k_raw, v, a, b = (t.contiguous() for t in (q_raw, k_raw, v, a, b))
    a_log, dt_bias = a_log.float().contiguous(), dt_bias.float().contiguous()
    desc, keep = _desc(q_raw, v, torch.bfloat16, True, _lib.CHUNKED, cu_seqlens, out_f32)
    why = _lib.validate(desc)
    if why:
        raise RuntimeError(why)
    N = q_raw.shape[0] if cu_seqlens is None else len(cu_seqlens) - 1
    dev = q_raw.device
    Hv, Dv, Dk = v.shape[2], v.shape[3], q_raw.shape[3]
    s0 = None if state is None else state.to(torch.float32).contiguous()
    q, k = torch.empty_like(q_raw), torch.empty_like(k_raw)
    beta = torch.empty_like(b)
    log_decay = torch.empty(a.shape, dtype=torch.float32, device=dev)
    y = torch.empty(v.shape, dtype=torch.float32 if out_f32 else torch.bfloat16, device=dev)
    s_out = torch.empty(N, Hv, Dv, Dk, dtype=torch.float32, device=dev)
    ckpt = torch.empty(max(_lib.ckpt_bytes(desc) // 4, 1), dtype=torch.float32, device=dev)
    ws = _workspace(desc, dev)
    _lib.fwd_prologue(desc, _dev_ptr(q_raw), _dev_ptr(k_raw), _dev_ptr(v), _dev_ptr(a), _dev_ptr(b), _dev_ptr(a_log),
                      _dev_ptr(dt_bias), _dev_ptr(s0), _dev_ptr(q), _dev_ptr(k), _dev_ptr(beta), _dev_ptr(log_decay),
                      _dev_ptr(y), _dev_ptr(s_out), _dev_ptr(ckpt), _dev_ptr(ws), _stream(dev))
    del keep
    return y, s_out, ckpt, q, k, beta, log_decay


def backward_prologue(q_raw, k_raw, a, b, a_log, dt_bias, q, k, v, beta, log_decay, ckpt, dy, ds_out=None, *,
                      cu_seqlens=None, want_ds0=True):
    """The chunked backward with the prologue's backward at the end of its last kernel (qb_gdn_bwd_prologue), after
    forward_prologue (q, k, beta, log_decay, ckpt are what it returned): (dq_raw, dk_raw, dv, da, db, da_log,
    ddt_bias, ds0). The first five are exactly what backward(q, k, v, log_decay, beta, ckpt, dy, ds_out,
    log_decay=True, design=CHUNKED) followed by neighbours.prologue_backward on its cotangents returns; da_log and
    ddt_bias are the same sums taken per chunk and then over chunks. bf16 activations and dy."""
    for t in (q_raw, k_raw, a, b, q, k, v, beta, dy):
        if t.dtype != torch.bfloat16 or not t.is_cuda:
            raise RuntimeError("gated delta: the fused prologue backward takes bf16 device tensors")
    q_raw, k_raw, a, b, q, k, v, beta, dy = (t.contiguous() for t in (q_raw, k_raw, a, b, q, k, v, beta, dy))
    a_log, dt_bias = a_log.float().contiguous(), dt_bias.float().contiguous()
    log_decay = log_decay.float().contiguous()
    desc, keep = _desc(q_raw, v, torch.bfloat16, True, _lib.CHUNKED, cu_seqlens, False)
    why = _lib.validate(desc)
    if why:
        raise RuntimeError(why)
    N = q_raw.shape[0] if cu_seqlens is None else len(cu_seqlens) - 1
    dev = q_raw.device
    Hv, Dv, Dk = v.shape[2], v.shape[3], q_raw.shape[3]
    dso = None if ds_out is None else ds_out.to(torch.float32).contiguous()
    dq_raw, dk_raw, dv = torch.empty_like(q_raw), torch.empty_like(k_raw), torch.empty_like(v)
    da, db = torch.empty_like(a), torch.empty_like(b)
    da_log, ddt_bias = torch.empty_like(a_log), torch.empty_like(dt_bias)
    ds0 = torch.empty(N, Hv, Dv, Dk, dtype=torch.float32, device=dev) if want_ds0 else None
    ws = _workspace(desc, dev)
    _lib.bwd_prologue(desc, _dev_ptr(q_raw), _dev_ptr(k_raw), _dev_ptr(a), _dev_ptr(b), _dev_ptr(a_log),
                      _dev_ptr(dt_bias), _dev_ptr(q), _dev_ptr(k), _dev_ptr(v), _dev_ptr(beta), _dev_ptr(log_decay),
                      _dev_ptr(ckpt), _dev_ptr(dy), _dev_ptr(dso), _dev_ptr(dq_raw), _dev_ptr(dk_raw), _dev_ptr(dv),
                      _dev_ptr(da), _dev_ptr(db), _dev_ptr(da_log), _dev_ptr(ddt_bias), _dev_ptr(ds0), _dev_ptr(ws),
                      _stream(dev))
    del keep
    return dq_raw, dk_raw, dv, da, db, da_log, ddt_bias, ds0


def forward_rows(q, k, v, g, beta, state=None, *, log_decay=False, cu_seqlens=None):
    """(y, row_states): the forward keeping the state after every token, row_states [B, T, Hv, Dv, Dk] float32 (or
    [total, Hv, Dv, Dk] packed) — the reference's rows pass for exact drafts (src/deltanet.cpp:101-117), whose
    decoder rolls back to any row's state (src/exact.cpp:152-162). Runs the recurrent design."""
    dtype = _io_dtype(q, k, v, beta)
    q, k, v, g, beta = _prep(q, k, v, g, beta, dtype)
    desc, keep = _desc(q, v, dtype, log_decay, _lib.RECURRENT, cu_seqlens, False)
    B, T, Hv, Dv = v.shape
    y = torch.empty(v.shape, dtype=dtype, device=v.device)
    rows = torch.empty((B, T, Hv, Dv, q.shape[-1]), dtype=torch.float32, device=v.device)
    s0 = None if state is None else state.to(torch.float32).contiguous()
    _lib.fwd_rows(desc, _dev_ptr(q), _dev_ptr(k), _dev_ptr(v), _dev_ptr(g), _dev_ptr(beta), _dev_ptr(s0),
                  _dev_ptr(y), _dev_ptr(rows), _stream(q.device))
    del keep
    if cu_seqlens is not None:
        rows = rows.view(B * T, Hv, Dv, q.shape[-1])
    return y, rows


class _GatedDelta(torch.autograd.Function):
    """custom_vjp of the recurrence: the forward keeps the chunk-start states, the backward is gated_delta_vjp
    (reference src/delta_grad.cpp:204-211, which saves only the primals and rebuilds the states instead)."""

    @staticmethod
    def forward(ctx, q, k, v, g, beta, state, log_decay, design):
        y, s_out, ckpt = forward(q, k, v, g, beta, state, log_decay=log_decay, design=design)
        ctx.save_for_backward(q, k, v, g, beta, ckpt)
        ctx.state_meta = (state is not None, None if state is None else state.dtype)
        ctx.opts = (log_decay, design)
        return y.to(q.dtype), s_out

    @staticmethod
    def backward(ctx, dy, dstate):
        q, k, v, g, beta, ckpt = ctx.saved_tensors
        log_decay, design = ctx.opts
        if dy is None:
            dy = torch.zeros(v.shape, dtype=q.dtype, device=q.device)
        dq, dk, dv, dg, dbeta, ds0 = backward(q, k, v, g, beta, ckpt, dy, dstate, log_decay=log_decay, design=design)
        has_state, sdt = ctx.state_meta
        return (dq.to(q.dtype), dk.to(k.dtype), dv.to(v.dtype), dg.to(g.dtype), dbeta.to(beta.dtype),
                ds0.to(sdt) if has_state else None, None, None)


class _GatedDeltaPrologue(torch.autograd.Function):
    """The layer's prologue and the trainable recurrence as one autograd node on the fused entry points
    (qb_gdn_fwd_prologue, qb_gdn_bwd_prologue): neighbours.prologue followed by gated_delta_trainable(...,
    log_decay=True), with the same results bit for bit (the gate parameters' cotangents up to float32 reassociation
    of their sums over tokens), without the prologue's separate passes over q_raw and k_raw (reference
    src/deltanet.cpp:94-100 feeding gated_delta at :111). The forward keeps its chunk-start states and the
    recurrence's inputs q, k, beta, log_decay for the backward."""

    @staticmethod
    def forward(ctx, q_raw, k_raw, v, a, b, a_log, dt_bias, state):
        y, s_out, ckpt, q, k, beta, log_decay = forward_prologue(q_raw, k_raw, v, a, b, a_log, dt_bias, state)
        ctx.save_for_backward(q_raw, k_raw, a, b, a_log, dt_bias, q, k, v, beta, log_decay, ckpt)
        ctx.meta = (state is not None, None if state is None else state.dtype, a_log.dtype, dt_bias.dtype)
        return y, s_out

    @staticmethod
    def backward(ctx, dy, dstate):
        q_raw, k_raw, a, b, a_log, dt_bias, q, k, v, beta, log_decay, ckpt = ctx.saved_tensors
        has_state, sdt, adt, ddt = ctx.meta
        if dy is None:
            dy = torch.zeros(v.shape, dtype=torch.bfloat16, device=v.device)
        dq_raw, dk_raw, dv, da, db, da_log, ddt_bias, ds0 = backward_prologue(
            q_raw, k_raw, a, b, a_log, dt_bias, q, k, v, beta, log_decay, ckpt, dy.to(torch.bfloat16), dstate,
            want_ds0=has_state)
        return (dq_raw, dk_raw, dv, da, db, da_log.to(adt), ddt_bias.to(ddt), ds0.to(sdt) if has_state else None)


def gated_delta_prologue(q_raw, k_raw, v, a, b, a_log, dt_bias, state=None):
    """(y in bf16, new float32 state) of the layer's prologue then the trainable recurrence in one fused call:
    q = rms_norm(q_raw) / Dk, k = rms_norm(k_raw) / sqrt(Dk), beta = sigmoid(b), log-decay = -exp(a_log) *
    softplus(a + dt_bias), then gated_delta_trainable(q, k, v, log-decay, beta, state, log_decay=True). Autograd
    runs the fused backward. The chunked design's shapes only: bf16 activations, Dk = 128, Dv a multiple of 32."""
    return _GatedDeltaPrologue.apply(q_raw, k_raw, v, a, b, a_log, dt_bias, state)


def gated_delta_trainable(q, k, v, g, beta, state, *, log_decay=False, design=DEFAULT_DESIGN):
    """(y, new_state) with gated_delta_vjp as the backward."""
    return _GatedDelta.apply(q, k, v, g, beta, state, log_decay, design)


def gated_delta(q, k, v, g, beta, state, train=False, *, log_decay=False, design=DEFAULT_DESIGN):
    """(y in q's dtype, new float32 state). With train, the trainable form (reference src/deltanet.cpp:55-58)."""
    if train:
        return gated_delta_trainable(q, k, v, g, beta, state, log_decay=log_decay, design=design)
    y, s_out, _ = forward(q, k, v, g, beta, state, log_decay=log_decay, design=design, save_ckpt=False)
    return y.to(q.dtype), s_out


def gated_delta_vjp(primals, dy, dstate, *, log_decay=False, design=DEFAULT_DESIGN):
    """Cotangents [dq, dk, dv, dg, dbeta, dstate0] of primals (q, k, v, g, beta, state) given those of y and the
    final state (reference src/delta_grad.cpp:155-199). Runs the forward once to get the chunk-start states."""
    q, k, v, g, beta, state = primals
    _, _, ckpt = forward(q, k, v, g, beta, state, log_decay=log_decay, design=design)
    dq, dk, dv, dg, dbeta, ds0 = backward(q, k, v, g, beta, ckpt, dy, dstate, log_decay=log_decay, design=design)
    return [dq.to(q.dtype), dk.to(k.dtype), dv.to(v.dtype), dg.to(g.dtype), dbeta.to(beta.dtype), ds0]
