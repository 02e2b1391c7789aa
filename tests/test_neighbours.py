"""The layer's pointwise neighbours of the recurrence (reference src/deltanet.cpp:22-45, :94-100, :122): the oracle
(oracle/neighbours_ref.py) pinned on the CPU, then the HIP kernels against it on the GPU through the C ABI.

Pins of the oracle (each chosen so that a slip in it fails one):
  * bf16 rounding against torch's float32 -> bfloat16 conversion, ties included;
  * closed forms at bf16: sigmoid(0) = 1/2, a + dt_bias rounding to 1 and softplus(1) rounding to 1.3125, a constant
    row normalising to 1 (so q = 1/Dk and k = the bf16 value of Dk^-1/2), silu(0) = 0, and the float32 norm weight
    entering the gated product unrounded;
  * the float32 forward against torch's own rms_norm, sigmoid, logaddexp and silu in float64;
  * every backward output against torch autograd through those library ops in float64.
GPU criteria:
  * bf16 forward: the kernels compute each op in float32 and round where the oracle rounds, so a value can land on
    the other side of a rounding boundary, and a flip can carry through a later rounding. Elementwise within 2 bf16
    units in the last place (ulp), with at most 1 value in 10^4 differing at all;
  * float32 forward: within 1e-5 relative, elementwise;
  * backward, normwise (max|x - ref| / max|ref|): 4e-3 for bf16 outputs, whose one rounding moves an element by at
    most half its ulp, that is by at most 2^-8 of the largest element; 1e-5 for float32; 5e-5 for the parameter
    gradients summed over tokens in float32.
"""
import numpy as np
import pytest

from helpers import normwise
from oracle import neighbours_ref as nb

EPS = 1e-6


def _torch():
    import torch

    return torch


def _prologue_inputs(rng, B, T, Hk, Hv, Dk, *, bf16):
    r = nb.round_bf16 if bf16 else (lambda x: np.asarray(x, np.float32).astype(np.float64))
    return {
        "q_raw": r(rng.standard_normal((B, T, Hk, Dk))),
        "k_raw": r(rng.standard_normal((B, T, Hk, Dk))),
        "a": r(rng.standard_normal((B, T, Hv))),
        "b": r(rng.standard_normal((B, T, Hv))),
        "a_log": np.log(rng.uniform(1.0, 16.0, Hv)).astype(np.float32).astype(np.float64),
        "dt_bias": rng.normal(0.0, 0.5, Hv).astype(np.float32).astype(np.float64),
    }


def _prologue_cotangents(rng, B, T, Hk, Hv, Dk, *, bf16):
    r = nb.round_bf16 if bf16 else (lambda x: np.asarray(x, np.float32).astype(np.float64))
    return {
        "dq": r(rng.standard_normal((B, T, Hk, Dk))),
        "dk": r(rng.standard_normal((B, T, Hk, Dk))),
        "dbeta": r(rng.standard_normal((B, T, Hv))),
        "dlog_decay": rng.standard_normal((B, T, Hv)).astype(np.float32).astype(np.float64),
    }


def _epilogue_inputs(rng, B, T, Hv, Dv, *, bf16):
    r = nb.round_bf16 if bf16 else (lambda x: np.asarray(x, np.float32).astype(np.float64))
    return {
        "y": r(0.05 * rng.standard_normal((B, T, Hv, Dv))),
        "z": r(2.0 * rng.standard_normal((B, T, Hv, Dv))),
        "w": r(1.0 + 0.2 * rng.standard_normal(Dv)),
        "dout": r(rng.standard_normal((B, T, Hv, Dv))),
    }


# ---------------------------------------------------------------------------------------------------------------
# The oracle, on the CPU


def test_round_bf16_matches_torch():
    torch = _torch()
    rng = np.random.default_rng(1)
    x = (rng.standard_normal(200_000) * np.exp(rng.uniform(-30, 30, 200_000))).astype(np.float32)
    u = x.view(np.uint32)
    ties = ((u & 0xFFFF0000) | 0x8000).astype(np.uint32).view(np.float32)  # exactly halfway
    for v in (x, ties, np.array([0.0, -0.0, 1.0, -1.0, 3.0e38, 1e-40], np.float32)):
        exp = torch.from_numpy(v).to(torch.bfloat16).float().numpy()
        got = nb.round_bf16(v)
        assert np.array_equal(got.astype(np.float32).view(np.uint32), exp.view(np.uint32))


@pytest.mark.parametrize("Dk", [64, 128, 256])
def test_prologue_closed_forms_bf16(Dk):
    Hv = 3
    q_raw = np.full((1, 2, 1, Dk), 0.75)
    k_raw = np.full((1, 2, 1, Dk), -3.0)
    a = np.ones((1, 2, Hv))
    b = np.stack([np.zeros(Hv), np.ones(Hv)])[None]
    a_log = np.zeros(Hv)
    dt_bias = np.full(Hv, 2.0 ** -10)  # 1 + 2^-10 rounds to 1 in bf16
    q, k, beta, ld = nb.prologue_fwd(q_raw, k_raw, a, b, a_log, dt_bias, bf16=True)
    assert np.all(q == 1.0 / Dk)
    sk = float(np.float32(Dk ** -0.5))
    assert np.all(k == -nb.round_bf16(sk))
    assert np.all(beta[0, 0] == 0.5)
    assert np.all(beta[0, 1] == nb.round_bf16(1.0 / (1.0 + np.exp(-1.0))))
    assert np.all(ld == -1.3125)  # softplus(1) = 1.31326... rounds to 1.3125
    # In float32 neither rounding happens.
    _, _, _, ld32 = nb.prologue_fwd(q_raw, k_raw, a, b, a_log, dt_bias, bf16=False)
    np.testing.assert_allclose(ld32, -np.logaddexp(1.0 + 2.0 ** -10, 0.0), rtol=1e-7)


def test_epilogue_closed_forms():
    Dv = 64
    y = np.full((1, 1, 2, Dv), 0.5)
    z = np.zeros((1, 1, 2, Dv))
    z[0, 0, 1] = 2.0
    w = np.full(Dv, 0.3)  # not a bf16 value: the float32 weight enters the product unrounded
    o = nb.epilogue_fwd(y, z, w, EPS, bf16=True)
    assert np.all(o[0, 0, 0] == 0.0)
    silu2 = 2.0 / (1.0 + np.exp(-2.0))
    rho = 1.0 / np.sqrt(0.25 + EPS)
    assert np.all(o[0, 0, 1] == nb.round_bf16(silu2 * 0.3 * 0.5 * rho))


@pytest.mark.parametrize("Dk", [64, 128])
def test_prologue_forward_matches_torch_ops(Dk):
    torch = _torch()
    F = torch.nn.functional
    rng = np.random.default_rng(2)
    x = _prologue_inputs(rng, 2, 9, 2, 4, Dk, bf16=False)
    q, k, beta, ld = nb.prologue_fwd(**x, bf16=False)
    t = {n: torch.from_numpy(v) for n, v in x.items()}
    sq, sk = float(np.float32(1.0 / Dk)), float(np.float32(Dk ** -0.5))
    tq = sq * F.rms_norm(t["q_raw"], (Dk,), eps=EPS)
    tk = sk * F.rms_norm(t["k_raw"], (Dk,), eps=EPS)
    tld = -torch.exp(t["a_log"]) * torch.logaddexp(t["a"] + t["dt_bias"], torch.zeros(()))
    for got, exp in ((q, tq), (k, tk), (beta, torch.sigmoid(t["b"])), (ld, tld)):
        np.testing.assert_allclose(got, exp.numpy(), rtol=1e-6, atol=0)


def test_epilogue_forward_matches_torch_ops():
    torch = _torch()
    F = torch.nn.functional
    rng = np.random.default_rng(3)
    x = _epilogue_inputs(rng, 2, 5, 3, 128, bf16=False)
    o = nb.epilogue_fwd(x["y"], x["z"], x["w"], 1e-5, bf16=False)
    y, z, w = (torch.from_numpy(x[n]) for n in ("y", "z", "w"))
    exp = F.silu(z) * F.rms_norm(y, (128,), weight=w, eps=1e-5)
    np.testing.assert_allclose(o, exp.numpy(), rtol=1e-6, atol=1e-30)


def test_prologue_backward_matches_autograd():
    torch = _torch()
    F = torch.nn.functional
    rng = np.random.default_rng(4)
    B, T, Hk, Hv, Dk = 2, 7, 2, 4, 64
    x = _prologue_inputs(rng, B, T, Hk, Hv, Dk, bf16=False)
    c = _prologue_cotangents(rng, B, T, Hk, Hv, Dk, bf16=False)
    got = nb.prologue_bwd(**x, **c, bf16=False)
    t = {n: torch.from_numpy(v).requires_grad_(True) for n, v in x.items()}
    sq, sk = float(np.float32(1.0 / Dk)), float(np.float32(Dk ** -0.5))
    outs = (sq * F.rms_norm(t["q_raw"], (Dk,), eps=EPS), sk * F.rms_norm(t["k_raw"], (Dk,), eps=EPS),
            torch.sigmoid(t["b"]),
            -torch.exp(t["a_log"]) * torch.logaddexp(t["a"] + t["dt_bias"], torch.zeros((), dtype=torch.float64)))
    cots = [torch.from_numpy(c[n]) for n in ("dq", "dk", "dbeta", "dlog_decay")]
    exp = torch.autograd.grad(outs, [t[n] for n in ("q_raw", "k_raw", "a", "b", "a_log", "dt_bias")], cots)
    for name, g, e in zip(("dq_raw", "dk_raw", "da", "db", "da_log", "ddt_bias"), got, exp):
        assert normwise(g, e.numpy()) <= 1e-6, name


def test_epilogue_backward_matches_autograd():
    torch = _torch()
    F = torch.nn.functional
    rng = np.random.default_rng(5)
    x = _epilogue_inputs(rng, 2, 6, 3, 64, bf16=False)
    got = nb.epilogue_bwd(x["y"], x["z"], x["w"], 1e-5, x["dout"])
    y, z, w = (torch.from_numpy(x[n]).requires_grad_(True) for n in ("y", "z", "w"))
    o = F.silu(z) * F.rms_norm(y, (64,), weight=w, eps=1e-5)
    exp = torch.autograd.grad(o, [y, z, w], torch.from_numpy(x["dout"]))
    for name, g, e in zip(("dy", "dz", "dw"), got, exp):
        assert normwise(g, e.numpy()) <= 1e-12, name


# ---------------------------------------------------------------------------------------------------------------
# The HIP kernels, on the GPU

PROLOGUE_ULPS, EPILOGUE_ULPS = 2, 2  # bf16 units in the last place, elementwise
MAX_INEXACT = 1e-4  # the fraction of bf16 forward values that may differ from the oracle's
BF16_GRAD_TOL = 4e-3
F32_TOL = 1e-5
PARAM_TOL = 5e-5


@pytest.fixture(scope="module")
def dev():
    torch = _torch()
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    from quotebound_amd import _lib

    _lib.load()  # raises when the library is missing: there is no fallback
    return torch


def _to_dev(torch, x, bf16, names=None):
    out = {}
    for n, v in x.items():
        t = torch.tensor(np.asarray(v, np.float32)).cuda()
        if bf16 and (names is None or n in names):
            t = t.to(torch.bfloat16)
        out[n] = t
    return out


def _host(t):
    return t.float().cpu().numpy().astype(np.float64)


def _assert_ulps(got, ref, ulps, label):
    half = np.ldexp(1.0, np.frexp(np.abs(ref))[1] - 9)  # half the bf16 spacing at |ref|
    bad = np.abs(got - ref) > 2 * ulps * half + 1e-38
    assert not bad.any(), f"{label}: {bad.sum()} values beyond {ulps} bf16 ulp, first at {np.argwhere(bad)[0]}"
    inexact = np.mean(got != ref)
    print(label, "inexact fraction %.2e" % inexact)
    assert inexact <= MAX_INEXACT, f"{label}: {inexact:.3g} of the values differ from the oracle's"


def _assert_rel(got, ref, tol, label):
    rel = np.abs(got - ref) / np.maximum(np.abs(ref), 1e-30)
    assert rel.max() <= tol, f"{label}: max relative error {rel.max():.3g} > {tol}"


PROLOGUE_CASES = [  # (B, T, Hk, Hv, Dk, bf16)
    (2, 100, 4, 8, 128, True),
    (1, 70, 2, 4, 64, False),
    (3, 37, 2, 6, 256, True),
    (1, 1, 16, 32, 128, True),
    (1, 600, 16, 48, 128, True),  # several 256-token tiles of the gates' sums; 48 heads do not divide 256 threads
]


@pytest.mark.gpu
@pytest.mark.parametrize("case", PROLOGUE_CASES,
                         ids=lambda c: "B%dT%dHk%dHv%dDk%d_%s" % (*c[:5], "bf16" if c[5] else "f32"))
def test_prologue_parity(dev, case):
    torch = dev
    from quotebound_amd import neighbours

    B, T, Hk, Hv, Dk, bf16 = case
    rng = np.random.default_rng(40 + T)
    x = _prologue_inputs(rng, B, T, Hk, Hv, Dk, bf16=bf16)
    c = _prologue_cotangents(rng, B, T, Hk, Hv, Dk, bf16=bf16)
    act = ("q_raw", "k_raw", "a", "b", "dq", "dk", "dbeta")
    d = _to_dev(torch, {**x, **c}, bf16, act)
    q, k, beta, ld = neighbours.prologue_forward(d["q_raw"], d["k_raw"], d["a"], d["b"], d["a_log"], d["dt_bias"])
    grads = neighbours.prologue_backward(d["q_raw"], d["k_raw"], d["a"], d["b"], d["a_log"], d["dt_bias"], d["dq"],
                                         d["dk"], d["dbeta"], d["dlog_decay"])
    grads2 = neighbours.prologue_backward(d["q_raw"], d["k_raw"], d["a"], d["b"], d["a_log"], d["dt_bias"], d["dq"],
                                          d["dk"], d["dbeta"], d["dlog_decay"])
    torch.cuda.synchronize()
    assert ld.dtype == torch.float32 and q.dtype == (torch.bfloat16 if bf16 else torch.float32)
    rq, rk, rbeta, rld = nb.prologue_fwd(**x, bf16=bf16)
    if bf16:
        for name, got, ref in (("q", q, rq), ("k", k, rk), ("beta", beta, rbeta)):
            _assert_ulps(_host(got), ref, PROLOGUE_ULPS, name)
        rel = np.abs(_host(ld) - rld) / np.abs(rld)
        assert rel.max() <= 2.0 ** -7  # softplus may round to the neighbouring bf16 value
        assert np.mean(rel > 1e-5) <= 0.01
    else:
        for name, got, ref in (("q", q, rq), ("k", k, rk), ("beta", beta, rbeta), ("log_decay", ld, rld)):
            _assert_rel(_host(got), ref, F32_TOL, name)
    ref = nb.prologue_bwd(**x, **c, bf16=bf16)
    names = ("dq_raw", "dk_raw", "da", "db", "da_log", "ddt_bias")
    for i, (name, g, r) in enumerate(zip(names, grads, ref)):
        tol = PARAM_TOL if i >= 4 else (BF16_GRAD_TOL if bf16 else F32_TOL)
        err = normwise(_host(g), r)
        print(name, "%.2e" % err)
        assert err <= tol, f"{name}: normwise {err:.3g} > {tol}"
        assert torch.equal(g, grads2[i]), f"{name}: not deterministic"


EPILOGUE_CASES = [  # (B, T, Hv, Dv, bf16)
    (2, 100, 8, 128, True),
    (1, 70, 4, 64, False),
    (3, 37, 6, 256, True),
    (1, 4500, 32, 128, True),  # more than 1024 groups of 64 rows: blocks take several groups
]


@pytest.mark.gpu
@pytest.mark.parametrize("case", EPILOGUE_CASES,
                         ids=lambda c: "B%dT%dHv%dDv%d_%s" % (*c[:4], "bf16" if c[4] else "f32"))
def test_epilogue_parity(dev, case):
    torch = dev
    from quotebound_amd import neighbours

    B, T, Hv, Dv, bf16 = case
    eps = 1e-6
    rng = np.random.default_rng(60 + T)
    x = _epilogue_inputs(rng, B, T, Hv, Dv, bf16=bf16)
    d = _to_dev(torch, x, bf16, ("y", "z", "dout"))
    w32 = d["w"].float()
    o = neighbours.epilogue_forward(d["y"], d["z"], w32, eps)
    dy, dz, dw = neighbours.epilogue_backward(d["y"], d["z"], w32, eps, d["dout"])
    dy2, dz2, dw2 = neighbours.epilogue_backward(d["y"], d["z"], w32, eps, d["dout"])
    torch.cuda.synchronize()
    ro = nb.epilogue_fwd(x["y"], x["z"], x["w"], eps, bf16=bf16)
    if bf16:
        _assert_ulps(_host(o), ro, EPILOGUE_ULPS, "o")
    else:
        _assert_rel(_host(o), ro, F32_TOL, "o")
    ref = nb.epilogue_bwd(x["y"], x["z"], x["w"], eps, x["dout"])
    for i, (name, g, r) in enumerate(zip(("dy", "dz", "dw"), (dy, dz, dw), ref)):
        tol = PARAM_TOL if i == 2 else (BF16_GRAD_TOL if bf16 else F32_TOL)
        err = normwise(_host(g), r)
        print(name, "%.2e" % err)
        assert err <= tol, f"{name}: normwise {err:.3g} > {tol}"
    assert torch.equal(dy, dy2) and torch.equal(dz, dz2) and torch.equal(dw, dw2)


@pytest.mark.gpu
def test_neighbours_autograd_and_empty(dev):
    """The autograd wrappers give the oracle's gradients, with unused outputs' cotangents taken as zero; an empty
    batch gives empty outputs and zero parameter gradients."""
    torch = dev
    from quotebound_amd import neighbours

    rng = np.random.default_rng(77)
    B, T, Hk, Hv, Dk = 1, 50, 2, 4, 128
    x = _prologue_inputs(rng, B, T, Hk, Hv, Dk, bf16=False)
    c = _prologue_cotangents(rng, B, T, Hk, Hv, Dk, bf16=False)
    d = {n: torch.tensor(v, dtype=torch.float32, device="cuda", requires_grad=True) for n, v in x.items()}
    q, k, beta, ld = neighbours.prologue(*(d[n] for n in ("q_raw", "k_raw", "a", "b", "a_log", "dt_bias")))
    loss = (q * torch.tensor(c["dq"], dtype=torch.float32, device="cuda")).sum() + (
        ld * torch.tensor(c["dlog_decay"], dtype=torch.float32, device="cuda")).sum()
    loss.backward()
    c0 = dict(c, dk=np.zeros_like(c["dk"]), dbeta=np.zeros_like(c["dbeta"]))
    ref = nb.prologue_bwd(**x, **c0, bf16=False)
    for n, r in zip(("q_raw", "k_raw", "a", "b", "a_log", "dt_bias"), ref):
        assert normwise(_host(d[n].grad), r) <= PARAM_TOL, n

    e = _epilogue_inputs(rng, 1, 20, 4, 64, bf16=False)
    t = {n: torch.tensor(e[n], dtype=torch.float32, device="cuda", requires_grad=True) for n in ("y", "z", "w")}
    o = neighbours.epilogue(t["y"], t["z"], t["w"], 1e-6)
    o.backward(torch.tensor(e["dout"], dtype=torch.float32, device="cuda"))
    for n, r in zip(("y", "z", "w"), nb.epilogue_bwd(e["y"], e["z"], e["w"], 1e-6, e["dout"])):
        assert normwise(_host(t[n].grad), r) <= PARAM_TOL, n

    empty = torch.empty((1, 0, 2, 64), dtype=torch.bfloat16, device="cuda")
    ab = torch.empty((1, 0, 4), dtype=torch.bfloat16, device="cuda")
    p = torch.ones(4, device="cuda")
    q, k, beta, ld = neighbours.prologue_forward(empty, empty, ab, ab, p, p)
    assert q.shape == empty.shape and ld.shape == ab.shape
    g = neighbours.prologue_backward(empty, empty, ab, ab, p, p, empty, empty, ab, ab.float())
    assert torch.count_nonzero(g[4]) == 0 and torch.count_nonzero(g[5]) == 0
    yv = torch.empty((1, 0, 4, 64), dtype=torch.bfloat16, device="cuda")
    dy, dz, dw = neighbours.epilogue_backward(yv, yv, torch.ones(64, device="cuda"), 1e-6, yv)
    torch.cuda.synchronize()
    assert dy.numel() == 0 and torch.count_nonzero(dw) == 0


FUSED_CASES = [  # (B, T, Hk, Hv, Dv, packed lengths or None, initial state)
    (2, 150, 2, 4, 64, None, True),
    (1, 333, 4, 12, 32, [70, 0, 130, 133], False),  # packed, an empty sequence, GQA ratio 3
    (1, 4096, 16, 32, 128, None, False),             # the 4B layer shape
]


@pytest.mark.gpu
@pytest.mark.parametrize("case", FUSED_CASES, ids=lambda c: "B%dT%dHk%dHv%dDv%d%s%s" % (
    *c[:5], "_packed" if c[5] else "", "_s0" if c[6] else ""))
def test_fused_prologue_forward_is_the_two_passes(dev, case):
    """qb_gdn_fwd_prologue (the prologue inside the chunked forward's first kernel) against the separate prologue
    pass followed by the chunked forward on its outputs: q, k, beta, the log-decay, y, the final state and the whole
    residual buffer (states and chunk tiles) equal bit for bit."""
    torch = dev
    from quotebound_amd import gdn, neighbours

    B, T, Hk, Hv, Dv, lens, with_s0 = case
    Dk = 128
    rng = np.random.default_rng(70 + T)
    x = _prologue_inputs(rng, B, T, Hk, Hv, Dk, bf16=True)
    x["v"] = nb.round_bf16(rng.standard_normal((B, T, Hv, Dv)))
    d = _to_dev(torch, x, True, ("q_raw", "k_raw", "a", "b", "v"))
    cu = None if lens is None else np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    N = B if cu is None else len(lens)
    s0 = torch.tensor(rng.normal(0.0, 0.1, (N, Hv, Dv, Dk)).astype(np.float32)).cuda() if with_s0 else None
    fused = gdn.forward_prologue(d["q_raw"], d["k_raw"], d["v"], d["a"], d["b"], d["a_log"], d["dt_bias"], s0,
                                 cu_seqlens=cu)
    q, k, beta, ld = neighbours.prologue_forward(d["q_raw"], d["k_raw"], d["a"], d["b"], d["a_log"], d["dt_bias"])
    y, s_out, ckpt = gdn.forward(q, k, d["v"], ld, beta, s0, log_decay=True, design=2, cu_seqlens=cu)
    torch.cuda.synchronize()
    names = ("y", "s_out", "ckpt", "q", "k", "beta", "log_decay")
    for name, got, ref in zip(names, fused, (y, s_out, ckpt, q, k, beta, ld)):
        assert got.dtype == ref.dtype and got.shape == ref.shape, name
        assert torch.equal(got.view(torch.int16) if got.dtype == torch.bfloat16 else got.view(torch.int32),
                           ref.view(torch.int16) if ref.dtype == torch.bfloat16 else ref.view(torch.int32)), name


@pytest.mark.gpu
@pytest.mark.parametrize("case", FUSED_CASES, ids=lambda c: "B%dT%dHk%dHv%dDv%d%s%s" % (
    *c[:5], "_packed" if c[5] else "", "_s0" if c[6] else ""))
def test_fused_prologue_backward_is_the_two_passes(dev, case):
    """qb_gdn_bwd_prologue (the prologue's backward at the end of the chunked backward's gradient kernel) against the
    chunked backward followed by the separate prologue backward on its cotangents: dq_raw, dk_raw, dv, da, db and ds0
    equal bit for bit; da_log and ddt_bias, summed per chunk and then over chunks instead of per token tile, within
    1e-5 of the separate pass's sums relative to the sum of the terms' magnitudes."""
    torch = dev
    from quotebound_amd import gdn, neighbours

    B, T, Hk, Hv, Dv, lens, with_s0 = case
    Dk = 128
    rng = np.random.default_rng(170 + T)
    x = _prologue_inputs(rng, B, T, Hk, Hv, Dk, bf16=True)
    x["v"] = nb.round_bf16(rng.standard_normal((B, T, Hv, Dv)))
    x["dy"] = nb.round_bf16(rng.standard_normal((B, T, Hv, Dv)))
    d = _to_dev(torch, x, True, ("q_raw", "k_raw", "a", "b", "v", "dy"))
    cu = None if lens is None else np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    N = B if cu is None else len(lens)
    s0 = torch.tensor(rng.normal(0.0, 0.1, (N, Hv, Dv, Dk)).astype(np.float32)).cuda() if with_s0 else None
    dso = torch.tensor(rng.normal(0.0, 0.1, (N, Hv, Dv, Dk)).astype(np.float32)).cuda() if with_s0 else None
    _, _, ckpt, q, k, beta, ld = gdn.forward_prologue(d["q_raw"], d["k_raw"], d["v"], d["a"], d["b"], d["a_log"],
                                                      d["dt_bias"], s0, cu_seqlens=cu)
    fused = gdn.backward_prologue(d["q_raw"], d["k_raw"], d["a"], d["b"], d["a_log"], d["dt_bias"], q, k, d["v"],
                                  beta, ld, ckpt, d["dy"], dso, cu_seqlens=cu)
    dq, dk, dv, dld, dbeta, ds0 = gdn.backward(q, k, d["v"], ld, beta, ckpt, d["dy"], dso, log_decay=True, design=2,
                                               cu_seqlens=cu)
    dq_raw, dk_raw, da, db, da_log, ddt = neighbours.prologue_backward(d["q_raw"], d["k_raw"], d["a"], d["b"],
                                                                       d["a_log"], d["dt_bias"], dq, dk, dbeta, dld)
    torch.cuda.synchronize()
    names = ("dq_raw", "dk_raw", "dv", "da", "db", "ds0")
    for name, got, ref in zip(names, fused[:5] + fused[7:], (dq_raw, dk_raw, dv, da, db, ds0)):
        assert got.dtype == ref.dtype and got.shape == ref.shape, name
        assert torch.equal(got.view(torch.int16) if got.dtype == torch.bfloat16 else got.view(torch.int32),
                           ref.view(torch.int16) if ref.dtype == torch.bfloat16 else ref.view(torch.int32)), name
    # The per-head sums' terms: dlog_decay * log_decay for dA_log, da for ddt_bias.
    mag_a = (dld.double() * ld.double()).abs().reshape(-1, Hv).sum(0)
    mag_d = da.double().abs().reshape(-1, Hv).sum(0)
    for name, got, ref, mag in (("da_log", fused[5], da_log, mag_a), ("ddt_bias", fused[6], ddt, mag_d)):
        err = ((got.double() - ref.double()).abs() / mag.clamp_min(1e-30)).max().item()
        assert err <= 1e-5, (name, err)


@pytest.mark.gpu
def test_fused_prologue_autograd_is_the_separate_ops(dev):
    """gdn.gated_delta_prologue, the autograd op on the fused entry points, against neighbours.prologue followed by
    gdn.gated_delta_trainable(log_decay=True) under torch autograd, with a nonzero initial state and cotangents on
    y and the final state: y, the final state and the gradients of q_raw, k_raw, v, a, b and the state equal bit for
    bit; those of a_log and dt_bias (sums over tokens in another fixed order) within 1e-5 relative to the sum of
    their terms' magnitudes."""
    torch = dev
    from quotebound_amd import gdn, neighbours

    B, T, Hk, Hv, Dk, Dv = 2, 150, 2, 4, 128, 64
    rng = np.random.default_rng(91)
    x = _prologue_inputs(rng, B, T, Hk, Hv, Dk, bf16=True)
    x["v"] = nb.round_bf16(rng.standard_normal((B, T, Hv, Dv)))
    d = _to_dev(torch, x, True, ("q_raw", "k_raw", "a", "b", "v"))
    s0 = torch.tensor(rng.normal(0.0, 0.1, (B, Hv, Dv, Dk)).astype(np.float32)).cuda()
    dy = torch.tensor(nb.round_bf16(rng.standard_normal((B, T, Hv, Dv)))).cuda().to(torch.bfloat16)
    dso = torch.tensor(rng.normal(0.0, 0.1, (B, Hv, Dv, Dk)).astype(np.float32)).cuda()
    names = ("q_raw", "k_raw", "v", "a", "b", "a_log", "dt_bias", "state")

    def run(fused):
        leaves = [d[n].detach().clone().requires_grad_() for n in names[:7]] + [s0.clone().requires_grad_()]
        qr, kr, v, a, b, al, dt, st = leaves
        if fused:
            y, s = gdn.gated_delta_prologue(qr, kr, v, a, b, al, dt, st)
        else:
            q, k, beta, ld = neighbours.prologue(qr, kr, a, b, al, dt)
            y, s = gdn.gated_delta_trainable(q, k, v, ld, beta, st, log_decay=True, design=2)
        torch.autograd.backward([y, s], [dy, dso])
        torch.cuda.synchronize()
        return y.detach(), s.detach(), [t.grad for t in leaves]

    yf, sf, gf = run(True)
    ys, ss, gs = run(False)
    bits = lambda t: t.view(torch.int16) if t.dtype == torch.bfloat16 else t.view(torch.int32)  # noqa: E731
    assert torch.equal(bits(yf), bits(ys)) and torch.equal(bits(sf), bits(ss))
    for name, a_, b_ in zip(names, gf, gs):
        assert a_.dtype == b_.dtype and a_.shape == b_.shape, name
        if name in ("a_log", "dt_bias"):
            err = ((a_.double() - b_.double()).abs().max() / b_.double().abs().max().clamp_min(1e-30)).item()
            assert err <= 1e-5, (name, err)
        else:
            assert torch.equal(bits(a_), bits(b_)), name
