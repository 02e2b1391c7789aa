"""The oracle of the layer's pointwise neighbours of the recurrence (reference src/deltanet.cpp), in numpy.

Test infrastructure only: tests/ and __graft_entry__.smoke() compare the kernels' results with it.

Forward, following the reference's ops in order (arithmetic in float64; with bf16 activations every op's output
is rounded to bf16 where the reference's op rounds it, each op returning its input's dtype):
  q = s_q * rms_norm(q_raw), k = s_k * rms_norm(k_raw)     src/deltanet.cpp:94-97 (rms_norm without weight, eps
                                                           1e-6; s_q = float(1/Dk), s_k = float(Dk^-1/2), each in the
                                                           activation dtype)
  beta = sigmoid(b)                                         :99
  log_decay = -exp(A_log) * softplus(a + dt_bias)           :22-33, :100 (compute_g; softplus = logaddexp(x, 0) in
                                                           the activation dtype; the reference then takes exp)
  o = silu(z) * rms_norm(y, w, eps)                         :35-45, :122 (precise_swiglu: silu in float32 times the
                                                           normed y, rounded once to the activation dtype; the
                                                           weight is float32, as the checkpoints store it (reference
                                                           src/model.h:95; tests/tiny.h:53-55), so MLX 0.32.3's
                                                           fast::rms_norm returns float32 and nothing rounds before
                                                           the product)
Backward: the exact adjoint in float64 of the same ops without the roundings (the GPU kernels compute it in
float32 and round each output once).
"""
from __future__ import annotations

import numpy as np

NORM_EPS = 1e-6  # src/deltanet.cpp:96-97


def round_bf16(x):
    """Round to nearest even bf16, returned as float64 (NaN stays NaN)."""
    a = np.asarray(x, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
    out = r.view(np.float32).astype(np.float64)
    return np.where(np.isnan(a), np.nan, out)


def _rnd(x, bf16):
    return round_bf16(x) if bf16 else np.asarray(x, np.float32).astype(np.float64)


def scales(Dk, bf16):
    inv = float(Dk) ** -0.5
    sq, sk = np.float32(inv * inv), np.float32(inv)
    return float(_rnd(sq, bf16)), float(_rnd(sk, bf16))


def _sigmoid(x):
    return 1.0 / (1.0 + np.exp(-x))


def _softplus(x):
    return np.maximum(x, 0.0) + np.log1p(np.exp(-np.abs(x)))


def _rho(x, eps):
    return 1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)


def prologue_fwd(q_raw, k_raw, a, b, a_log, dt_bias, *, bf16):
    """Returns (q, k, beta, log_decay) as float64 arrays holding the activation dtype's values."""
    q_raw, k_raw, a, b = (np.asarray(x, np.float64) for x in (q_raw, k_raw, a, b))
    a_log, dt_bias = np.asarray(a_log, np.float64), np.asarray(dt_bias, np.float64)
    sq, sk = scales(q_raw.shape[-1], bf16)
    q = _rnd(sq * _rnd(q_raw * _rho(q_raw, NORM_EPS), bf16), bf16)
    k = _rnd(sk * _rnd(k_raw * _rho(k_raw, NORM_EPS), bf16), bf16)
    beta = _rnd(_sigmoid(b), bf16)
    x = _rnd(a + dt_bias, bf16)
    log_decay = -np.exp(a_log) * _rnd(_softplus(x), bf16)
    return q, k, beta, log_decay


def _norm_bwd(x, g, eps):
    """d/dx of sum(g * x rho(x))."""
    rho = _rho(x, eps)
    n = x.shape[-1]
    return rho * g - rho ** 3 * x * np.sum(g * x, axis=-1, keepdims=True) / n


def prologue_bwd(q_raw, k_raw, a, b, a_log, dt_bias, dq, dk, dbeta, dlog_decay, *, bf16):
    """Returns (dq_raw, dk_raw, da, db, da_log, ddt_bias) in float64. The forward's roundings are not
    differentiated (a + dt_bias and softplus enter at their rounded values, as in the kernels)."""
    f = lambda x: np.asarray(x, np.float64)  # noqa: E731
    q_raw, k_raw, a, b, dq, dk, dbeta, dlog_decay = map(f, (q_raw, k_raw, a, b, dq, dk, dbeta, dlog_decay))
    a_log, dt_bias = f(a_log), f(dt_bias)
    sq, sk = scales(q_raw.shape[-1], bf16)
    dq_raw = _norm_bwd(q_raw, sq * dq, NORM_EPS)
    dk_raw = _norm_bwd(k_raw, sk * dk, NORM_EPS)
    sb = _sigmoid(b)
    db = dbeta * sb * (1 - sb)
    x = _rnd(a + dt_bias, bf16)
    ea = np.exp(a_log)
    da = -dlog_decay * ea * _sigmoid(x)
    log_decay = -ea * _rnd(_softplus(x), bf16)
    sum_tok = lambda t: t.reshape(-1, t.shape[-1]).sum(axis=0)  # noqa: E731
    return dq_raw, dk_raw, da, db, sum_tok(dlog_decay * log_decay), sum_tok(da)


def epilogue_fwd(y, z, w, eps, *, bf16):
    """o = silu(z) * rms_norm(y, w, eps), as float64 holding the activation dtype's values."""
    y, z, w = (np.asarray(x, np.float64) for x in (y, z, w))
    n = w * (y * _rho(y, eps))
    return _rnd(z * _sigmoid(z) * n, bf16)


def epilogue_bwd(y, z, w, eps, dout):
    """Returns (dy, dz, dw) in float64, the adjoint of o = silu(z) * (y rho(y) w)."""
    y, z, w, dout = (np.asarray(x, np.float64) for x in (y, z, w, dout))
    rho = _rho(y, eps)
    sg = _sigmoid(z)
    silu = z * sg
    nh = y * rho
    dz = dout * nh * w * sg * (1 + z * (1 - sg))
    dn = dout * silu
    dw = (dn * nh).reshape(-1, y.shape[-1]).sum(axis=0)
    dy = _norm_bwd(y, dn * w, eps)
    return dy, dz, dw
