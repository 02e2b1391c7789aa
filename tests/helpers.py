"""Shared test helpers: the reference's normwise error metric and seeded input builders."""
from __future__ import annotations

import numpy as np

GRAD_NAMES = ("dq", "dk", "dv", "dg", "dbeta", "ds0")


def normwise(x, ref) -> float:
    """max|x - ref| / max|ref|, the reference's per-tensor criterion (reference tests/test_deltanet.cpp:93-94,
    127-128). Zero when both are zero."""
    x = np.asarray(x, np.float64)
    ref = np.asarray(ref, np.float64)
    scale = np.max(np.abs(ref)) if ref.size else 0.0
    diff = np.max(np.abs(x - ref)) if ref.size else 0.0
    if scale == 0.0:
        return float(diff)
    return float(diff / scale)


def bf16_half_ulp(x):
    """Half the bf16 spacing at |x| (x in [2^(e-1), 2^e) has spacing 2^(e-8)): the most that rounding to nearest
    can move it."""
    return np.ldexp(1.0, np.frexp(np.asarray(x, np.float64))[1] - 9)


def unit_rows(rng, shape, scale):
    """Unit-RMS rows times scale: the reference's test inputs (reference tests/test_deltanet.cpp:29-32, 106-107)."""
    x = rng.standard_normal(shape)
    x = x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + 1e-6)
    return x * scale


def reference_case(B, T, Hk, Hv, Dk, Dv, g_lo, seed):
    """Inputs as the reference's trainable-gradient test draws them (reference tests/test_deltanet.cpp:106-112):
    q, k unit RMS scaled by 1/Dk and 1/sqrt(Dk); g uniform in [g_lo, 1) as the decay factor; beta uniform in [0, 1);
    state ~N(0, 0.1); cotangents on y and on the final state."""
    rng = np.random.default_rng(seed)
    return {
        "q": unit_rows(rng, (B, T, Hk, Dk), 1.0 / Dk),
        "k": unit_rows(rng, (B, T, Hk, Dk), 1.0 / np.sqrt(Dk)),
        "v": rng.standard_normal((B, T, Hv, Dv)),
        "g": rng.uniform(g_lo, 1.0, (B, T, Hv)),
        "beta": rng.uniform(0.0, 1.0, (B, T, Hv)),
        "s0": rng.normal(0.0, 0.1, (B, Hv, Dv, Dk)),
        "dy": rng.standard_normal((B, T, Hv, Dv)),
        "ds_out": rng.standard_normal((B, Hv, Dv, Dk)),
    }


def small_case(B, T, Hk, Hv, Dk, Dv, seed, s0=True, ds_out=True, log_decay=True):
    """Unit-norm keys and queries, log-decay -softplus(N(0,1)), beta sigmoid(N(0,1))."""
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((B, T, Hk, Dk))
    k = rng.standard_normal((B, T, Hk, Dk))
    q /= np.linalg.norm(q, axis=-1, keepdims=True)
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    a = -np.logaddexp(rng.standard_normal((B, T, Hv)), 0.0)
    return {
        "q": q,
        "k": k,
        "v": rng.standard_normal((B, T, Hv, Dv)),
        "g": a if log_decay else np.exp(a),
        "beta": 1.0 / (1.0 + np.exp(-rng.standard_normal((B, T, Hv)))),
        "s0": rng.normal(0.0, 0.1, (B, Hv, Dv, Dk)) if s0 else None,
        "dy": rng.standard_normal((B, T, Hv, Dv)),
        "ds_out": rng.standard_normal((B, Hv, Dv, Dk)) if ds_out else None,
    }
