"""Pins the oracle (oracle/gdn_ref.c) before anything is checked against it.

Each check is chosen so that a plausible slip in the restatement (a dropped decay, a wrong sign in du, a transposed
state, a wrong key-head index, an off-by-one in the chunk recompute) fails at least one of them:
  * golden vectors written by autodiff through the plain-ops loop (tests/golden/make_golden.py);
  * the reference's own gradient cases (reference tests/test_deltanet.cpp:145-154) against autodiff through the
    plain ops, with the reference's criterion (worst max|d grad| / max|grad| <= 1e-5 in float32);
  * closed forms: one step; beta = 0; associative-memory recall with orthonormal keys;
  * invariances: GQA by duplicated key heads, split of the sequence, checkpoint stride, packed sequences;
  * central finite differences in float64 on every input;
  * gradient cut by a zero decay; the log-decay chain rule.
"""
import numpy as np
import pytest

from helpers import GRAD_NAMES, normwise, reference_case, small_case
import plain_ops

GOLDEN_KEYS = ("y", "s_out") + GRAD_NAMES


def _golden(name):
    import os

    path = os.path.join(os.path.dirname(__file__), "golden", name + ".npz")
    z = np.load(path)
    inp = {k[3:]: z[k] for k in z.files if k.startswith("in_")}
    out = {k[4:]: z[k] for k in z.files if k.startswith("out_")}
    return inp, out


@pytest.mark.parametrize("name", ["tiny_fp32", "tiny_fp32_s0"])
def test_golden_vectors(oracle, name):
    inp, exp = _golden(name)
    got64 = oracle.fwd_bwd(inp, dtype=np.float64)
    got32 = oracle.fwd_bwd(inp, dtype=np.float32)
    for key in GOLDEN_KEYS:
        assert normwise(got64[key], exp[key]) <= 1e-12, key
        assert normwise(got32[key], exp[key]) <= 2e-6, key


REFERENCE_CASES = [  # (B, T, Hk, Hv, Dk, Dv, g_lo): reference tests/test_deltanet.cpp:145-154
    (1, 19, 16, 32, 128, 128, 0.5),
    (1, 64, 16, 32, 128, 128, 0.9),
    (2, 150, 16, 32, 128, 128, 0.99),
    (1, 129, 16, 32, 128, 128, 0.9),
    (1, 70, 2, 8, 32, 32, 0.9),
    (2, 33, 4, 4, 64, 64, 0.99),
    (1, 70, 2, 4, 128, 4, 0.9),
    (1, 40, 2, 4, 256, 64, 0.9),
]


@pytest.mark.parametrize("case", REFERENCE_CASES, ids=lambda c: "B%dT%dHk%dHv%dDk%dDv%d" % c[:6])
def test_reference_gradient_cases(oracle, case):
    B, T, Hk, Hv, Dk, Dv, g_lo = case
    inp = reference_case(B, T, Hk, Hv, Dk, Dv, g_lo, seed=100 + T)
    exp = plain_ops.fwd_bwd(inp, g_is_log=False)
    for dt, tol in ((np.float64, 1e-11), (np.float32, 1e-5)):
        y, s, ck = oracle.fwd(inp["q"], inp["k"], inp["v"], inp["g"], inp["beta"], inp["s0"], g_is_log=False,
                              dtype=dt)
        grads = oracle.bwd(inp["q"], inp["k"], inp["v"], inp["g"], inp["beta"], ck, inp["dy"], inp["ds_out"],
                           g_is_log=False, dtype=dt)
        assert normwise(y, exp["y"]) <= tol
        assert normwise(s, exp["s_out"]) <= tol
        for name, got in zip(GRAD_NAMES, grads):
            assert normwise(got, exp[name]) <= tol, (name, dt)


def test_one_step_closed_form(oracle):
    inp = small_case(1, 1, 1, 1, 8, 5, seed=1, log_decay=False)
    S0 = inp["s0"][0, 0]
    g, b = inp["g"][0, 0, 0], inp["beta"][0, 0, 0]
    k, q, v = inp["k"][0, 0, 0], inp["q"][0, 0, 0], inp["v"][0, 0, 0]
    S1 = g * S0 + b * np.outer(v - g * S0 @ k, k)
    y, s, _ = oracle.fwd(inp["q"], inp["k"], inp["v"], inp["g"], inp["beta"], inp["s0"], g_is_log=False)
    assert np.allclose(s[0, 0], S1, rtol=0, atol=1e-14)
    assert np.allclose(y[0, 0, 0], S1 @ q, rtol=0, atol=1e-14)


def test_zero_beta_is_pure_decay(oracle):
    inp = small_case(1, 37, 2, 4, 16, 8, seed=2)
    inp["beta"][:] = 0.0
    y, s, _ = oracle.fwd(inp["q"], inp["k"], inp["v"], inp["g"], inp["beta"], inp["s0"])
    cum = np.exp(np.cumsum(inp["g"][0], axis=0))  # [T, Hv]
    hk = np.arange(4) // 2
    for t in range(37):
        for hv in range(4):
            exp = cum[t, hv] * inp["s0"][0, hv] @ inp["q"][0, t, hk[hv]]
            assert np.allclose(y[0, t, hv], exp, rtol=1e-12, atol=1e-14)
    assert np.allclose(s[0], cum[-1][:, None, None] * inp["s0"][0], rtol=1e-12, atol=1e-15)


def test_orthonormal_recall(oracle):
    """g = 1, beta = 1, zero state, orthonormal keys: S_T = sum v_s k_s^T and querying k_j returns v_j."""
    rng = np.random.default_rng(3)
    T, D = 12, 16
    Qm, _ = np.linalg.qr(rng.standard_normal((D, D)))
    keys = Qm.T[:T]  # orthonormal rows
    v = rng.standard_normal((1, T, 1, 6))
    k = keys.reshape(1, T, 1, D)
    j = rng.integers(0, np.arange(T) + 1)  # query an already written key at every step
    q = keys[j].reshape(1, T, 1, D)
    y, s, _ = oracle.fwd(q, k, v, np.ones((1, T, 1)), np.ones((1, T, 1)), None, g_is_log=False)
    assert np.allclose(y[0, :, 0], v[0, j, 0], atol=1e-12)
    assert np.allclose(s[0, 0], v[0, :, 0].T @ keys, atol=1e-12)


def test_gqa_equals_duplicated_key_heads(oracle):
    inp = small_case(1, 50, 2, 6, 16, 8, seed=4)
    rep = {n: (np.repeat(inp[n], 3, axis=2) if n in ("q", "k") else inp[n]) for n in inp}
    a = oracle.fwd_bwd(inp, chunk=16)
    b = oracle.fwd_bwd(rep, chunk=16)
    assert normwise(a["y"], b["y"]) <= 1e-14
    for name in ("dv", "dg", "dbeta", "ds0"):
        assert normwise(a[name], b[name]) <= 1e-13
    for name in ("dq", "dk"):  # the group's value heads sum into their key head
        summed = b[name].reshape(1, 50, 2, 3, 16).sum(3)
        assert normwise(a[name], summed) <= 1e-13


def test_split_invariance(oracle):
    """Carrying the state across calls equals one call (reference tests/test_deltanet.cpp:47-52)."""
    inp = small_case(2, 70, 2, 4, 16, 8, seed=5)
    y, s, _ = oracle.fwd(inp["q"], inp["k"], inp["v"], inp["g"], inp["beta"], inp["s0"])
    cut = lambda x, a, b: x[:, a:b]  # noqa: E731
    y1, s1, _ = oracle.fwd(*(cut(inp[n], 0, 20) for n in ("q", "k", "v", "g", "beta")), inp["s0"])
    y2, s2, _ = oracle.fwd(*(cut(inp[n], 20, 70) for n in ("q", "k", "v", "g", "beta")), s1)
    assert normwise(np.concatenate([y1, y2], 1), y) <= 1e-14
    assert normwise(s2, s) <= 1e-14


@pytest.mark.parametrize("chunk", [1, 7, 16, 64, 200])
def test_checkpoint_stride_invariance(oracle, chunk):
    inp = small_case(1, 90, 1, 2, 16, 8, seed=6)
    base = oracle.fwd_bwd(inp, chunk=64)
    other = oracle.fwd_bwd(inp, chunk=chunk)
    for key in GOLDEN_KEYS:
        assert normwise(other[key], base[key]) <= 1e-13, key


def test_checkpoints_are_chunk_start_states(oracle):
    inp = small_case(1, 150, 1, 2, 16, 8, seed=7)
    _, _, ck = oracle.fwd(inp["q"], inp["k"], inp["v"], inp["g"], inp["beta"], inp["s0"], chunk=64)
    assert ck.shape[0] == 3
    assert np.array_equal(ck[0], inp["s0"][0])
    for c in (1, 2):
        _, s, _ = oracle.fwd(*(inp[n][:, :64 * c] for n in ("q", "k", "v", "g", "beta")), inp["s0"], chunk=64)
        assert np.array_equal(ck[c], s[0])


def test_packed_sequences_equal_separate_calls(oracle):
    lens = [5, 64, 0, 130, 1]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    T = int(cu[-1])
    inp = small_case(1, T, 2, 4, 16, 8, seed=8, s0=False, ds_out=False)
    rng = np.random.default_rng(9)
    inp["s0"] = rng.normal(0, 0.1, (len(lens), 4, 8, 16))
    inp["ds_out"] = rng.standard_normal((len(lens), 4, 8, 16))
    packed = oracle.fwd_bwd(inp, cu_seqlens=cu)
    for n, (a, b) in enumerate(zip(cu[:-1], cu[1:])):
        part = {x: inp[x][:, a:b] for x in ("q", "k", "v", "g", "beta", "dy")}
        part["s0"], part["ds_out"] = inp["s0"][n:n + 1], inp["ds_out"][n:n + 1]
        if b == a:
            assert np.array_equal(packed["s_out"][n], inp["s0"][n])
            assert np.array_equal(packed["ds0"][n], inp["ds_out"][n])
            continue
        one = oracle.fwd_bwd(part)
        for key in ("y", "dq", "dk", "dv", "dg", "dbeta"):
            assert normwise(packed[key][:, a:b], one[key]) <= 1e-14, (n, key)
        assert normwise(packed["s_out"][n], one["s_out"][0]) <= 1e-14
        assert normwise(packed["ds0"][n], one["ds0"][0]) <= 1e-14
    ref = plain_ops.fwd_bwd(inp, cu_seqlens=cu)
    for key in GOLDEN_KEYS:
        assert normwise(packed[key], ref[key]) <= 1e-11, key


def _loss(oracle, inp, chunk=4):
    y, s, _ = oracle.fwd(inp["q"], inp["k"], inp["v"], inp["g"], inp["beta"], inp["s0"], chunk=chunk)
    return float(np.sum(y * inp["dy"]) + np.sum(s * inp["ds_out"]))


@pytest.mark.parametrize("name", ["q", "k", "v", "g", "beta", "s0"])
def test_finite_differences(oracle, name):
    """Central differences in float64 along random directions, one input at a time (the method of reference
    tests/test_train.cpp:105-181, applied to the recurrence). With the loss <dy, y> + <dS_out, S_T> this is the
    dot-product (adjoint) test: <dy, J d> by differences against <J^T dy, d> from the backward."""
    inp = small_case(1, 11, 1, 2, 6, 5, seed=10)
    grads = oracle.fwd_bwd(inp, chunk=4)
    gname = {"s0": "ds0"}.get(name, "d" + name)
    rng = np.random.default_rng(11)
    for _ in range(3):
        d = rng.standard_normal(inp[name].shape)
        eps = 1e-6
        plus = dict(inp)
        minus = dict(inp)
        plus[name] = inp[name] + eps * d
        minus[name] = inp[name] - eps * d
        fd = (_loss(oracle, plus) - _loss(oracle, minus)) / (2 * eps)
        an = float(np.sum(grads[gname] * d))
        assert abs(fd - an) <= 1e-7 * max(1.0, abs(an)), (name, fd, an)


def test_zero_decay_cuts_the_gradient(oracle):
    """With g_t = 0 the state is wiped at t: inputs before t get no gradient from cotangents at or after t."""
    inp = small_case(1, 40, 1, 2, 8, 4, seed=12, s0=True, ds_out=True, log_decay=False)
    inp["g"][0, 25, :] = 0.0
    y, s, ck = oracle.fwd(inp["q"], inp["k"], inp["v"], inp["g"], inp["beta"], inp["s0"], chunk=16, g_is_log=False)
    base = oracle.bwd(inp["q"], inp["k"], inp["v"], inp["g"], inp["beta"], ck, inp["dy"], inp["ds_out"], chunk=16,
                      g_is_log=False)
    dy2 = inp["dy"].copy()
    dy2[:, 25:] = np.random.default_rng(13).standard_normal(dy2[:, 25:].shape)
    other = oracle.bwd(inp["q"], inp["k"], inp["v"], inp["g"], inp["beta"], ck, dy2, inp["ds_out"] * 3, chunk=16,
                       g_is_log=False)
    for name, x, z in zip(GRAD_NAMES, base, other):
        if name == "ds0":
            assert np.array_equal(x, z)
        elif name == "dg":  # g_25 itself still sees the cotangents after it; earlier steps do not
            assert np.array_equal(x[:, :25], z[:, :25])
        else:
            assert np.array_equal(x[:, :25], z[:, :25]), name


def test_decay_factor_gradient_is_an_exact_difference(oracle):
    """The loss <dy, y> + <ds_out, s_out> is affine in each decay factor g_t (the decayed state g_t S_{t-1} enters
    every later quantity linearly), so dL/dg_t = L(g_t = 1) - L(g_t = 0) exactly, at g_t = 0 as anywhere else. Zeros
    at a chunk start, mid-chunk, twice in a row and at the last step."""
    inp = small_case(1, 40, 1, 2, 8, 4, seed=15, s0=True, ds_out=True, log_decay=False)
    zeros = (0, 16, 21, 22, 39)
    for t in zeros:
        inp["g"][0, t, 0] = 0.0
    inp["g"][0, 9, 1] = 0.0

    def loss(g):
        y, s, _ = oracle.fwd(inp["q"], inp["k"], inp["v"], g, inp["beta"], inp["s0"], chunk=16, g_is_log=False)
        return float(np.sum(inp["dy"] * y) + np.sum(inp["ds_out"] * s))

    y, s, ck = oracle.fwd(inp["q"], inp["k"], inp["v"], inp["g"], inp["beta"], inp["s0"], chunk=16, g_is_log=False)
    dg = oracle.bwd(inp["q"], inp["k"], inp["v"], inp["g"], inp["beta"], ck, inp["dy"], inp["ds_out"], chunk=16,
                    g_is_log=False)[3]
    assert np.all(np.isfinite(dg))
    for t, h in [(t, 0) for t in zeros] + [(9, 1), (5, 0), (30, 1)]:
        g1, g0 = inp["g"].copy(), inp["g"].copy()
        g1[0, t, h], g0[0, t, h] = 1.0, 0.0
        diff = loss(g1) - loss(g0)
        assert abs(dg[0, t, h] - diff) <= 1e-11 * max(1.0, abs(diff)), (t, h, dg[0, t, h], diff)


def test_log_decay_chain_rule(oracle):
    inp = small_case(1, 30, 1, 2, 8, 4, seed=14)
    log = oracle.fwd_bwd(inp, chunk=8)
    fac = dict(inp)
    fac["g"] = np.exp(inp["g"])
    y, s, ck = oracle.fwd(fac["q"], fac["k"], fac["v"], fac["g"], fac["beta"], fac["s0"], chunk=8, g_is_log=False)
    grads = oracle.bwd(fac["q"], fac["k"], fac["v"], fac["g"], fac["beta"], ck, fac["dy"], fac["ds_out"], chunk=8,
                       g_is_log=False)
    assert normwise(y, log["y"]) <= 1e-14
    assert normwise(grads[3] * fac["g"], log["dg"]) <= 1e-13
    for name, got in zip(GRAD_NAMES, grads):
        if name != "dg":
            assert normwise(got, log[name]) <= 1e-13, name


def test_beta_gradient_vanishes_when_value_is_predicted(oracle):
    """dbeta_t = dd (v_t - u_t): zero at a step whose value equals the decayed state's prediction."""
    inp = small_case(1, 1, 1, 1, 8, 4, seed=15, log_decay=False)
    S0, g, k = inp["s0"][0, 0], inp["g"][0, 0, 0], inp["k"][0, 0, 0]
    inp["v"][0, 0, 0] = g * S0 @ k
    out = oracle.fwd_bwd({**inp, "g": np.log(inp["g"])}, chunk=4)
    assert np.all(np.abs(out["dbeta"]) <= 1e-14)
