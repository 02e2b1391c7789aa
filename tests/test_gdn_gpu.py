"""Parity of the HIP kernels with the oracle, on the GPU, through the C ABI.

Criterion (the reference's normwise metric, reference tests/test_deltanet.cpp:93-94, 127-128):
max|x - ref| / max|ref| per output tensor, against the oracle run on the same inputs (bf16 inputs rounded once,
the oracle in float32 on their exact values):
  * bf16 I/O, fp32 state (the layer shapes and the packed batch):     <= 2e-3 for y, s_out and every gradient;
  * float32 I/O (the tiny workload, the golden vectors and the reference's gradient cases): <= 1e-5, the reference's
    own criterion for its float32 backward.
"""
import os

import numpy as np
import pytest

from helpers import GRAD_NAMES, bf16_half_ulp, normwise, reference_case, small_case
from quotebound_amd import _lib

pytestmark = pytest.mark.gpu

OUT_NAMES = ("y", "s_out") + GRAD_NAMES
DESIGNS = [_lib.RECURRENT, _lib.CHUNKED]
DESIGN_IDS = {_lib.RECURRENT: "recurrent", _lib.CHUNKED: "chunked"}
BF16_TOL = 2e-3
F32_TOL = 1e-5


@pytest.fixture(scope="module")
def torch_dev():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    _lib.load()  # raises when the library is missing: there is no fallback
    return torch


def run(torch, d, design, *, log_decay=True, cu=None, need_s0_grad=True, out_f32=False):
    from quotebound_amd import gdn

    y, s_out, ckpt = gdn.forward(d["q"], d["k"], d["v"], d["g"], d["beta"], d.get("s0"), log_decay=log_decay,
                                 design=design, cu_seqlens=cu, out_f32=out_f32)
    grads = gdn.backward(d["q"], d["k"], d["v"], d["g"], d["beta"], ckpt, d["dy"], d.get("ds_out"),
                         log_decay=log_decay, design=design, cu_seqlens=cu, want_ds0=need_s0_grad,
                         out_f32=out_f32)
    torch.cuda.synchronize()
    out = {"y": y, "s_out": s_out, "ckpt": ckpt}
    out.update(zip(GRAD_NAMES, grads))
    return {k: (None if v is None else v.float().cpu().numpy()) for k, v in out.items()}


def host_to_dev(torch, arrays, dtype):
    out = {}
    for k, x in arrays.items():
        if x is None:
            continue
        t = torch.tensor(np.asarray(x, dtype=np.float32))
        if k in ("q", "k", "v", "beta", "dy"):
            t = t.to(dtype)
        out[k] = t.cuda()
    return out


def assert_close(got, ref, tol, names=OUT_NAMES, label=""):
    errs = {n: normwise(got[n], ref[n]) for n in names}
    report = "; ".join(f"{n} {errs[n]:.2e} (max-abs {np.max(np.abs(got[n] - ref[n])):.2e})" for n in names)
    print(label, report)
    for n in names:
        assert errs[n] <= tol, f"{label}: {n} normwise error {errs[n]:.3g} > {tol}; {report}"


def _golden(name):
    z = np.load(os.path.join(os.path.dirname(__file__), "golden", name + ".npz"))
    inp = {k[3:]: z[k] for k in z.files if k.startswith("in_")}
    out = {k[4:]: z[k] for k in z.files if k.startswith("out_")}
    return inp, out


@pytest.mark.parametrize("design", [_lib.RECURRENT], ids=DESIGN_IDS.get)
@pytest.mark.parametrize("name", ["tiny_fp32", "tiny_fp32_s0"])
def test_golden_vectors(torch_dev, design, name):
    torch = torch_dev
    inp, exp = _golden(name)
    got = run(torch, host_to_dev(torch, inp, torch.float32), design)
    assert_close(got, exp, F32_TOL, label=f"{name} design {design}")


@pytest.mark.parametrize("design", DESIGNS, ids=DESIGN_IDS.get)
@pytest.mark.parametrize("case", [  # reference tests/test_deltanet.cpp:145-154
    (1, 19, 16, 32, 128, 128, 0.5), (1, 64, 16, 32, 128, 128, 0.9), (2, 150, 16, 32, 128, 128, 0.99),
    (1, 129, 16, 32, 128, 128, 0.9), (1, 70, 2, 8, 32, 32, 0.9), (2, 33, 4, 4, 64, 64, 0.99),
    (1, 70, 2, 4, 128, 4, 0.9), (1, 40, 2, 4, 256, 64, 0.9)], ids=lambda c: "B%dT%dHk%dHv%dDk%dDv%d" % c[:6])
def test_reference_gradient_cases(torch_dev, oracle, design, case):
    torch = torch_dev
    B, T, Hk, Hv, Dk, Dv, g_lo = case
    inp = reference_case(B, T, Hk, Hv, Dk, Dv, g_lo, seed=100 + T)
    d, _ = _lib.make_desc(B, T, Hk, Hv, Dk, Dv, dtype=_lib.F32, g_is_log=False, design=design)
    why = _lib.validate(d)
    if why is not None:  # no parity evidence for a shape the design refuses (the refusal is tested in test_capi)
        pytest.skip(f"design {design} refuses this shape: {why}")
    y, s, ck = oracle.fwd(inp["q"], inp["k"], inp["v"], inp["g"], inp["beta"], inp["s0"], g_is_log=False)
    grads = oracle.bwd(inp["q"], inp["k"], inp["v"], inp["g"], inp["beta"], ck, inp["dy"], inp["ds_out"],
                       g_is_log=False)
    exp = {"y": y, "s_out": s, **dict(zip(GRAD_NAMES, grads))}
    got = run(torch, host_to_dev(torch, inp, torch.float32), design, log_decay=False)
    assert_close(got, exp, F32_TOL, label=f"case {case} design {design}")


REF_SHAPES_BF16 = [c for c in [  # the reference's gradient cases, bf16 inputs (reference tests/test_deltanet.cpp:145-154)
    (1, 19, 16, 32, 128, 128, 0.5), (1, 64, 16, 32, 128, 128, 0.9), (2, 150, 16, 32, 128, 128, 0.99),
    (1, 129, 16, 32, 128, 128, 0.9)]]


@pytest.mark.parametrize("design", DESIGNS, ids=DESIGN_IDS.get)
@pytest.mark.parametrize("case", REF_SHAPES_BF16, ids=lambda c: "B%dT%dHk%dHv%dDk%dDv%d" % c[:6])
def test_reference_cases_bf16_inputs(torch_dev, oracle, design, case):
    """The reference's gradient cases with the inputs rounded to bf16: the kernels' float32 outputs against the oracle
    on the same rounded inputs (decay factor input, cotangents on y and the final state, nonzero initial state)."""
    torch = torch_dev
    from quotebound_amd.synthetic import round_bf16

    B, T, Hk, Hv, Dk, Dv, g_lo = case
    inp = reference_case(B, T, Hk, Hv, Dk, Dv, g_lo, seed=100 + T)
    for n in ("q", "k", "v", "beta", "dy"):
        inp[n] = round_bf16(np.asarray(inp[n], np.float32)).astype(np.float64)
    y, s, ck = oracle.fwd(inp["q"], inp["k"], inp["v"], inp["g"], inp["beta"], inp["s0"], g_is_log=False)
    grads = oracle.bwd(inp["q"], inp["k"], inp["v"], inp["g"], inp["beta"], ck, inp["dy"], inp["ds_out"],
                       g_is_log=False)
    exp = {"y": y, "s_out": s, **dict(zip(GRAD_NAMES, grads))}
    d = host_to_dev(torch, inp, torch.bfloat16)
    d["dy"] = d["dy"].float()
    got = run(torch, d, design, log_decay=False, out_f32=True)
    assert_close(got, exp, BF16_TOL, label=f"bf16 case {case} design {design}")


@pytest.mark.parametrize("design", DESIGNS, ids=DESIGN_IDS.get)
def test_forward_only(torch_dev, oracle, design):
    """The forward alone at the 4B layer shape: y, the final state and the chunk-start states."""
    torch = torch_dev
    from quotebound_amd import gdn
    from quotebound_amd.synthetic import make_inputs, to_device, workload

    w = workload("qwen35_4b")
    inp = make_inputs(w)
    y, s, ck = oracle.fwd(inp.f32["q"], inp.f32["k"], inp.f32["v"], inp.f32["g"], inp.f32["beta"], None,
                          dtype=np.float32)
    d = to_device(inp)
    gy, gs, gck = gdn.forward(d["q"], d["k"], d["v"], d["g"], d["beta"], None, log_decay=True, design=design,
                              out_f32=True)
    torch.cuda.synchronize()
    got = {"y": gy.cpu().numpy(), "s_out": gs.cpu().numpy(),
           "ckpt": gck[:ck.size].cpu().numpy().reshape(ck.shape)}
    assert_close(got, {"y": y, "s_out": s, "ckpt": ck}, BF16_TOL, names=("y", "s_out", "ckpt"),
                 label=f"forward design {design}")


@pytest.mark.parametrize("design", DESIGNS, ids=DESIGN_IDS.get)
@pytest.mark.parametrize("wname", ["qwen35_4b", "qwen35_9b", "qwen35_4b_varlen"])
def test_layer_shapes_bf16(torch_dev, oracle, design, wname):
    """The benchmark workloads at full size: B=1, T=4096, Dk=Dv=128, Hk=16, Hv=32 (4B) or 48 (9B, nonzero initial
    state, dS0 returned), and 8 packed sequences at the 4B shape."""
    torch = torch_dev
    from quotebound_amd.synthetic import make_inputs, to_device, workload

    from quotebound_amd.synthetic import round_bf16

    w = workload(wname)
    inp = make_inputs(w)
    cu = w.cu_seqlens
    exp = oracle.fwd_bwd(inp.f32, cu_seqlens=cu, dtype=np.float32)
    d = to_device(inp)
    # The kernels' float32 results (bf16 inputs, float32 outputs): the 2e-3 criterion on every output.
    d32 = dict(d, dy=d["dy"].float())
    got32 = run(torch, d32, design, cu=cu, out_f32=True)
    assert_close(got32, exp, BF16_TOL, label=f"{wname} design {design} (f32 out)")
    nc = exp["ckpt"].size
    assert normwise(got32["ckpt"][:nc].reshape(exp["ckpt"].shape), exp["ckpt"]) <= BF16_TOL
    # bf16 outputs are those float32 results rounded once to nearest even, and nothing else changes.
    got16 = run(torch, d, design, cu=cu)
    for n in ("y", "dq", "dk", "dv", "dbeta"):
        assert np.array_equal(got16[n], round_bf16(got32[n].astype(np.float32))), n
    for n in ("s_out", "dg", "ds0"):
        assert np.array_equal(got16[n], got32[n]), n
    # Against the oracle, the bf16 outputs miss by at most the criterion plus their own half-ulp rounding.
    for n in ("y", "dq", "dk", "dv", "dbeta"):
        slack = np.abs(got16[n] - exp[n]) - bf16_half_ulp(np.maximum(np.abs(exp[n]), np.abs(got32[n])))
        assert slack.max() <= BF16_TOL * np.max(np.abs(exp[n])), n


@pytest.mark.parametrize("design", DESIGNS, ids=DESIGN_IDS.get)
def test_long_sequence(torch_dev, oracle, design):
    """A sequence four times the layer shapes' length (T = 16384, 256 chunks, at the 4B head widths with 4 value
    heads): the error against the oracle stays at the layer shapes' level, in the last 1024 tokens of y as over all
    outputs, so nothing accumulates along the chain of chunk states."""
    torch = torch_dev
    from quotebound_amd.synthetic import Workload, make_inputs, to_device

    w = Workload("long", 1, 16384, 2, 4, 128, 128, seed=43, s0_std=0.02, ds_out=True)
    print(f"long sequence: T={w.T} Hk={w.Hk} Hv={w.Hv} design {design}", flush=True)
    inp = make_inputs(w)
    exp = oracle.fwd_bwd(inp.f32, dtype=np.float32)
    d = to_device(inp)
    got = run(torch, dict(d, dy=d["dy"].float()), design, out_f32=True)
    assert_close(got, exp, BF16_TOL, label=f"long design {design}")
    tail = normwise(got["y"][:, -1024:], exp["y"][:, -1024:])
    head = normwise(got["y"][:, :1024], exp["y"][:, :1024])
    print(f"y error, first 1024 tokens {head:.2e}, last 1024 tokens {tail:.2e}")
    assert tail <= 1e-4  # measured 4e-7 (recurrent) and 1e-5 (chunked), as in the first 1024 tokens


@pytest.mark.parametrize("design", DESIGNS, ids=DESIGN_IDS.get)
def test_decode_steps_carry_the_state(torch_dev, oracle, design):
    """The inference path: a prefill of 66 tokens, then one-token calls that carry the state (the reference's decode
    and exact-draft rows, src/deltanet.cpp:101-120), give the y and final state of one call over the whole sequence,
    and both match the oracle."""
    torch = torch_dev
    from quotebound_amd import gdn
    from quotebound_amd.synthetic import Workload, make_inputs, to_device

    w = Workload("decode", 1, 72, 4, 8, 128, 128, seed=23, s0_std=0.02)
    inp = make_inputs(w)
    y_ref, s_ref, _ = oracle.fwd(inp.f32["q"], inp.f32["k"], inp.f32["v"], inp.f32["g"], inp.f32["beta"],
                                 inp.f32["s0"], dtype=np.float32)
    d = to_device(inp)
    fwd = lambda sl, state: gdn.forward(d["q"][:, sl], d["k"][:, sl], d["v"][:, sl], d["g"][:, sl], d["beta"][:, sl],
                                        state, log_decay=True, design=design, save_ckpt=False, out_f32=True)[:2]
    y_one, s_one = fwd(slice(0, w.T), d["s0"])
    ys, state = [], d["s0"]
    y_pre, state = fwd(slice(0, 66), state)
    ys.append(y_pre)
    for t in range(66, w.T):
        y_t, state = fwd(slice(t, t + 1), state)
        ys.append(y_t)
    torch.cuda.synchronize()
    y_steps = torch.cat(ys, dim=1)
    got_one = {"y": y_one.cpu().numpy(), "s_out": s_one.cpu().numpy()}
    got_steps = {"y": y_steps.cpu().numpy(), "s_out": state.cpu().numpy()}
    assert_close(got_steps, got_one, F32_TOL, names=("y", "s_out"), label=f"decode vs one call, design {design}")
    assert_close(got_steps, {"y": y_ref, "s_out": s_ref}, BF16_TOL, names=("y", "s_out"),
                 label=f"decode vs oracle, design {design}")


@pytest.mark.parametrize("packed", [False, True], ids=["batch", "packed"])
def test_row_states(torch_dev, oracle, packed):
    """qb_gdn_fwd_rows keeps the state after every token (the reference's rows pass for exact drafts,
    src/deltanet.cpp:101-117; keep_rows rolls back to one, src/exact.cpp:152-162): each row equals the oracle's state
    after that token (its checkpoints at stride 1, shifted by one, then its final state), y and the last row equal
    the plain forward's bit for bit, and one-token calls chained from a row's state reach the next rows' states."""
    torch = torch_dev
    from quotebound_amd import gdn
    from quotebound_amd.synthetic import Workload, make_inputs, to_device

    w = Workload("rows", 2, 37, 2, 4, 64, 64, seed=29, s0_std=0.02)
    inp = make_inputs(w)
    f = inp.f32
    cu = [0, 37, 74] if packed else None
    shape = lambda x: x.reshape(1, 74, *x.shape[2:]) if packed else x  # noqa: E731
    q, k, v, g, beta = (shape(f[n]) for n in ("q", "k", "v", "g", "beta"))
    y_ref, s_ref, ck = oracle.fwd(q, k, v, g, beta, f["s0"], chunk=1, cu_seqlens=cu, dtype=np.float32)
    d = {n: (t.reshape(1, 74, *t.shape[2:]) if packed and n != "s0" else t) for n, t in to_device(inp).items()
         if t is not None}
    y, rows = gdn.forward_rows(d["q"], d["k"], d["v"], d["g"], d["beta"], d["s0"], log_decay=True, cu_seqlens=cu)
    y1, s1, _ = gdn.forward(d["q"], d["k"], d["v"], d["g"], d["beta"], d["s0"], log_decay=True,
                            design=_lib.RECURRENT, cu_seqlens=cu, save_ckpt=False)
    torch.cuda.synchronize()
    rows = rows.reshape(2, 37, *rows.shape[-3:]).cpu().numpy()
    ck = np.asarray(ck).reshape(2, 37, *ck.shape[-3:])  # state before each token, per sequence
    s_ref = np.asarray(s_ref)
    for b in range(2):
        want = np.concatenate([ck[b, 1:], s_ref[b][None]], 0)
        assert normwise(rows[b], want) <= F32_TOL, b
        assert np.array_equal(rows[b, -1], s1[b].cpu().numpy())
    assert torch.equal(y, y1)
    # Roll back to row 20 of the first sequence and step one token at a time from there.
    state = torch.tensor(rows[0, 20][None]).cuda()
    for t in range(21, 25):
        sl = slice(t, t + 1)
        _, state, _ = gdn.forward(d["q"][:1, sl], d["k"][:1, sl], d["v"][:1, sl], d["g"][:1, sl],
                                  d["beta"][:1, sl], state, log_decay=True, design=_lib.RECURRENT, save_ckpt=False)
        assert np.array_equal(state[0].cpu().numpy(), rows[0, t]), t


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
@pytest.mark.parametrize("Dk,Dv", [(128, 128), (64, 48), (256, 40), (96, 32)])
def test_one_token_steps_match_rows(torch_dev, dtype, Dk, Dv):
    """One-token calls without checkpoints run a kernel of their own (rec_step_kernel), which must give the bits of
    the multi-token forward: from the state the rows pass kept after token t - 1 (S0 for t = 0), one call on token t
    gives that pass's state after token t and its y at t, bit for bit, in batch mode and as packed one-token
    sequences beside an empty one (whose state passes through unchanged). Every lane layout (16 or 32 lanes per row,
    4 to 8 columns per lane, contiguous or in runs of four) and a last row block that Dv only partly fills."""
    torch = torch_dev
    from quotebound_amd import gdn
    from quotebound_amd.synthetic import Workload, make_inputs, to_device

    w = Workload("one_token", 2, 9, 2, 4, Dk, Dv, dtype=dtype, seed=67, s0_std=0.02)
    print(f"one-token steps: {dtype} Dk={w.Dk} Dv={w.Dv} B={w.B} T={w.T}", flush=True)
    d = to_device(make_inputs(w))
    y, rows = gdn.forward_rows(d["q"], d["k"], d["v"], d["g"], d["beta"], d["s0"], log_decay=True)
    rows = rows.reshape(w.B, w.T, *rows.shape[-3:])
    step = lambda sl, state, cu=None, src=d: gdn.forward(  # noqa: E731
        src["q"][:, sl], src["k"][:, sl], src["v"][:, sl], src["g"][:, sl], src["beta"][:, sl], state,
        log_decay=True, design=_lib.RECURRENT, cu_seqlens=cu, save_ckpt=False)[:2]
    for t in range(w.T):
        before = d["s0"] if t == 0 else rows[:, t - 1].contiguous()
        y_t, s_t = step(slice(t, t + 1), before)
        assert torch.equal(s_t, rows[:, t]), t
        assert torch.equal(y_t[:, 0], y[:, t]), t
        # The same tokens as packed sequences of lengths 1, 0, 1.
        packed = {n: d[n][:, t].unsqueeze(0) for n in ("q", "k", "v", "g", "beta")}
        keep = rows[0, 0].unsqueeze(0)
        y_p, s_p = step(slice(0, 2), torch.cat([before[:1], keep, before[1:]]), cu=[0, 1, 1, 2], src=packed)
        assert torch.equal(s_p[0], rows[0, t]) and torch.equal(s_p[2], rows[1, t]), t
        assert torch.equal(s_p[1], keep[0]), t
        assert torch.equal(y_p[0], y[:, t]), t


@pytest.mark.parametrize("design", DESIGNS, ids=DESIGN_IDS.get)
@pytest.mark.parametrize("case", ["empty_sequences", "max_sequences"])
def test_packed_edge_cases(torch_dev, oracle, design, case):
    """Packed batches at the edges: empty sequences among others (their final state is S0 and their dS0 is the
    final state's cotangent), and the maximum of 255 sequences of 0 to 40 tokens, every output against the oracle."""
    torch = torch_dev
    from quotebound_amd.synthetic import Workload, make_inputs, to_device

    if case == "empty_sequences":
        lens = [5, 64, 0, 130, 1, 0, 63]
    else:
        lens = np.random.default_rng(7).integers(0, 41, _lib.MAX_SEQS).tolist()
    w = Workload(case, 1, int(sum(lens)), 2, 4, 128, 128, seed=31, s0_std=0.02, ds_out=True, seq_lens=lens)
    inp = make_inputs(w)
    exp = oracle.fwd_bwd(inp.f32, cu_seqlens=w.cu_seqlens, dtype=np.float32)
    d = to_device(inp)
    got = run(torch, dict(d, dy=d["dy"].float()), design, cu=w.cu_seqlens, out_f32=True)
    assert_close(got, exp, BF16_TOL, label=f"{case} design {design}")
    for i, n in enumerate(lens):
        if n == 0:
            assert np.array_equal(got["s_out"][i], inp.f32["s0"][i])
            assert np.array_equal(got["ds0"][i], inp.f32["ds_out"][i])


@pytest.mark.parametrize("design", DESIGNS, ids=DESIGN_IDS.get)
def test_empty_batch(torch_dev, design):
    """T = 0: nothing to compute; the final state is S0 and dS0 is the final state's cotangent."""
    torch = torch_dev
    from quotebound_amd import gdn

    B, Hk, Hv, D = 2, 2, 4, 128
    e = lambda *s: torch.empty(*s, dtype=torch.bfloat16, device="cuda")  # noqa: E731
    q, k, v, beta, dy = e(B, 0, Hk, D), e(B, 0, Hk, D), e(B, 0, Hv, D), e(B, 0, Hv), e(B, 0, Hv, D)
    g = torch.empty(B, 0, Hv, device="cuda")
    s0 = torch.randn(B, Hv, D, D, device="cuda")
    ds_out = torch.randn(B, Hv, D, D, device="cuda")
    y, s_out, ckpt = gdn.forward(q, k, v, g, beta, s0, log_decay=True, design=design)
    grads = gdn.backward(q, k, v, g, beta, ckpt, dy, ds_out, log_decay=True, design=design)
    torch.cuda.synchronize()
    assert y.shape == v.shape and torch.equal(s_out, s0)
    assert torch.equal(grads[5], ds_out) and all(t.numel() == 0 for t in grads[:5])


def _random_shape(seed):
    """A seeded draw of an odd shape: B 1-3 (or 2-6 packed sequences of 0-150 tokens), T 1-300, 1-4 value heads per
    key head, Dk 32/64/128, Dv 32/64/96/128, bf16 or float32, with or without S0 and dS_out."""
    r = np.random.default_rng(1000 + seed)
    Hk = int(r.choice([1, 2, 4]))
    Hv = Hk * int(r.integers(1, 5))
    Dk = int(r.choice([32, 64, 128, 128]))
    Dv = int(r.choice([32, 64, 96, 128]))
    bf16 = bool(r.integers(0, 4) > 0)
    if r.integers(0, 3) == 0:
        lens = r.integers(0, 151, int(r.integers(2, 7))).tolist()
        return dict(B=1, T=int(sum(lens)), Hk=Hk, Hv=Hv, Dk=Dk, Dv=Dv, bf16=bf16, lens=lens,
                    s0=bool(r.integers(0, 2)), ds_out=bool(r.integers(0, 2)))
    return dict(B=int(r.integers(1, 4)), T=int(r.integers(1, 301)), Hk=Hk, Hv=Hv, Dk=Dk, Dv=Dv, bf16=bf16, lens=None,
                s0=bool(r.integers(0, 2)), ds_out=bool(r.integers(0, 2)))


@pytest.mark.parametrize("seed", range(16))
def test_random_shapes(torch_dev, oracle, seed):
    """Both designs, wherever they take the shape, against the oracle on seeded odd shapes: forward and every
    cotangent normwise within 2e-3 (bf16 inputs, float32 outputs) or 1e-5 (float32)."""
    torch = torch_dev
    from quotebound_amd.synthetic import round_bf16

    c = _random_shape(seed)
    B, T, Hk, Hv, Dk, Dv = c["B"], c["T"], c["Hk"], c["Hv"], c["Dk"], c["Dv"]
    inp = small_case(B, T, Hk, Hv, Dk, Dv, seed=seed, s0=c["s0"], ds_out=c["ds_out"])
    cu = None
    if c["lens"] is not None:
        cu = np.concatenate([[0], np.cumsum(c["lens"])]).astype(np.int32)
        N = len(c["lens"])
        r = np.random.default_rng(seed)
        inp["s0"] = r.normal(0.0, 0.1, (N, Hv, Dv, Dk)) if c["s0"] else None
        inp["ds_out"] = r.standard_normal((N, Hv, Dv, Dk)) if c["ds_out"] else None
    for n in ("q", "k", "v", "beta", "dy"):
        x = np.asarray(inp[n], np.float32)
        inp[n] = round_bf16(x) if c["bf16"] else x
    for n in ("g", "s0", "ds_out"):
        if inp[n] is not None:
            inp[n] = np.asarray(inp[n], np.float32)
    exp = oracle.fwd_bwd(inp, cu_seqlens=cu, dtype=np.float32)
    d = host_to_dev(torch, inp, torch.bfloat16 if c["bf16"] else torch.float32)
    if c["bf16"]:
        d["dy"] = d["dy"].float()
    ran = 0
    for design in DESIGNS:
        desc, _ = _lib.make_desc(B, T, Hk, Hv, Dk, Dv, dtype=_lib.BF16 if c["bf16"] else _lib.F32, design=design,
                                 cu_seqlens=cu)
        if _lib.validate(desc):
            continue
        ran += 1
        got = run(torch, d, design, cu=cu, need_s0_grad=True, out_f32=c["bf16"])
        names = [n for n in OUT_NAMES if not (n == "ds0" and inp["s0"] is None and inp["ds_out"] is None)]
        assert_close(got, exp, BF16_TOL if c["bf16"] else F32_TOL, names=names,
                     label=f"seed {seed} {c} design {design}")
    assert ran >= 1, c


@pytest.mark.parametrize("design", DESIGNS, ids=DESIGN_IDS.get)
@pytest.mark.parametrize("mode", ["factor", "log"])
@pytest.mark.parametrize("crowded", [False, True], ids=["spread", "crowded"])
def test_zero_and_tiny_decays(torch_dev, oracle, design, mode, crowded):
    """Decay factors of 0 (a log-decay of -inf) and tiny ones: at a chunk's first and last step, twice in a row,
    mid-chunk and at the sequence's last step, beside ordinary ones. Every output finite and within the bf16
    tolerance of the oracle. (The chunked design floors the log-decay at -150 and, with g given as the factor, takes
    dL/dg at factors below 2^-10 from its exact replay of the chunk, four flagged steps per replay.) crowded: seven
    such factors in one (chunk, value head), its first and last steps among them, so that the replay runs twice."""
    torch = torch_dev
    from quotebound_amd.synthetic import round_bf16

    B, T, Hk, Hv, Dk, Dv = 1, 200, 2, 4, 128, 64
    inp = small_case(B, T, Hk, Hv, Dk, Dv, seed=21, s0=True, ds_out=True, log_decay=False)
    g = inp["g"]
    g[0, [0, 63, 64, 100, 101, 150], 0] = 0.0
    g[0, 70, 1], g[0, 71, 1], g[0, 72, 1] = 1e-30, 2.0 ** -12, 2.0 ** -9
    g[0, 199, 2] = 0.0
    g[0, 128, 3] = 1e-42  # subnormal in float32
    if crowded:  # chunk 1 (steps 64-127) of value head 2: zeros and tiny factors, first and last steps included
        g[0, [64, 65, 80, 96, 111, 126, 127], 2] = [0.0, 1e-30, 2.0 ** -12, 0.0, 2.0 ** -11, 1e-38, 0.0]
    for n in ("q", "k", "v", "beta", "dy"):
        inp[n] = round_bf16(np.asarray(inp[n], np.float32))
    for n in ("s0", "ds_out"):
        inp[n] = np.asarray(inp[n], np.float32)
    log = mode == "log"
    with np.errstate(divide="ignore"):
        inp["g"] = np.log(np.asarray(g, np.float32)) if log else np.asarray(g, np.float32)
    y, s, ck = oracle.fwd(inp["q"], inp["k"], inp["v"], inp["g"], inp["beta"], inp["s0"], g_is_log=log,
                          dtype=np.float32)
    grads = oracle.bwd(inp["q"], inp["k"], inp["v"], inp["g"], inp["beta"], ck, inp["dy"], inp["ds_out"],
                       g_is_log=log, dtype=np.float32)
    exp = {"y": y, "s_out": s}
    exp.update(zip(GRAD_NAMES, grads))
    for n, x in exp.items():
        assert np.all(np.isfinite(x)), n
    desc, _ = _lib.make_desc(B, T, Hk, Hv, Dk, Dv, dtype=_lib.BF16, g_is_log=log, design=design)
    assert not _lib.validate(desc)
    d = host_to_dev(torch, inp, torch.bfloat16)
    d["dy"] = d["dy"].float()
    got = run(torch, d, design, log_decay=log, out_f32=True)
    for n in OUT_NAMES:
        assert np.all(np.isfinite(got[n])), n
    assert_close(got, exp, BF16_TOL, label=f"{mode} design {design}")


@pytest.mark.parametrize("Dk", [96, 160, 192, 224, 256])
@pytest.mark.parametrize("bf16", [False, True], ids=["f32", "bf16"])
def test_recurrent_key_widths(torch_dev, oracle, Dk, bf16):
    """The recurrent design at the key widths beyond 32/64/128 (the wide variant, 32 lanes per state row, from 160):
    a packed batch with a nonzero initial state and a final-state cotangent, every output against the oracle."""
    torch = torch_dev
    from quotebound_amd.synthetic import round_bf16

    lens = [70, 0, 131, 1]
    Hk, Hv, Dv = 2, 4, 64
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    inp = small_case(1, int(cu[-1]), Hk, Hv, Dk, Dv, seed=Dk)
    r = np.random.default_rng(Dk)
    inp["s0"] = r.normal(0.0, 0.1, (len(lens), Hv, Dv, Dk))
    inp["ds_out"] = r.standard_normal((len(lens), Hv, Dv, Dk))
    for n in ("q", "k", "v", "beta", "dy"):
        x = np.asarray(inp[n], np.float32)
        inp[n] = round_bf16(x) if bf16 else x
    for n in ("g", "s0", "ds_out"):
        inp[n] = np.asarray(inp[n], np.float32)
    exp = oracle.fwd_bwd(inp, cu_seqlens=cu, dtype=np.float32)
    d = host_to_dev(torch, inp, torch.bfloat16 if bf16 else torch.float32)
    if bf16:
        d["dy"] = d["dy"].float()
    got = run(torch, d, _lib.RECURRENT, cu=cu, out_f32=bf16)
    assert_close(got, exp, BF16_TOL if bf16 else F32_TOL, label=f"Dk {Dk} {'bf16' if bf16 else 'f32'}")


@pytest.mark.parametrize("Dk,Dv,lens", [
    (288, 64, [70, 0, 131, 1]), (512, 64, [70, 0, 131, 1]), (1024, 32, [70, 0, 131, 1]),
    (2080, 16, [70, 0, 40, 1]), (4096, 16, [70, 0, 40, 1])], ids=lambda x: str(x) if isinstance(x, int) else None)
@pytest.mark.parametrize("bf16", [False, True], ids=["f32", "bf16"])
def test_recurrent_wide_key_widths(torch_dev, oracle, Dk, Dv, lens, bf16):
    """The recurrent design past Dk = 256, up to the 4096 the reference's vjp accepts (src/delta_grad.cpp:159-170):
    one wave per state row (four, two or one rows per block by width). A packed batch with an empty sequence, a
    nonzero initial state and a final-state cotangent, every output against the oracle, float32 at the reference's
    1e-5."""
    torch = torch_dev
    from quotebound_amd.synthetic import round_bf16

    Hk, Hv = 2, 4
    print(f"recurrent design, Dk {Dk}, Dv {Dv}, packed {lens}, {'bf16' if bf16 else 'f32'}", flush=True)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    inp = small_case(1, int(cu[-1]), Hk, Hv, Dk, Dv, seed=Dk)
    r = np.random.default_rng(Dk)
    inp["s0"] = r.normal(0.0, 0.1, (len(lens), Hv, Dv, Dk))
    inp["ds_out"] = r.standard_normal((len(lens), Hv, Dv, Dk))
    for n in ("q", "k", "v", "beta", "dy"):
        x = np.asarray(inp[n], np.float32)
        inp[n] = round_bf16(x) if bf16 else x
    for n in ("g", "s0", "ds_out"):
        inp[n] = np.asarray(inp[n], np.float32)
    exp = oracle.fwd_bwd(inp, cu_seqlens=cu, dtype=np.float32)
    d = host_to_dev(torch, inp, torch.bfloat16 if bf16 else torch.float32)
    if bf16:
        d["dy"] = d["dy"].float()
    got = run(torch, d, _lib.RECURRENT, cu=cu, out_f32=bf16)
    assert_close(got, exp, BF16_TOL if bf16 else F32_TOL, label=f"Dk {Dk} {'bf16' if bf16 else 'f32'}")


@pytest.mark.parametrize("lens,Dv", [(None, 128), ([70, 0, 100, 1], 128), ([40, 64, 10, 1], 64),
                                     ([40, 64, 10, 1], 32)], ids=["batch", "packed", "packed_Dv64", "packed_Dv32"])
def test_state_rows_per_block_change_no_bits(torch_dev, oracle, lens, Dv):
    """The chunked state passes take 32 state rows per block when their 16-row blocks would not all be resident at
    once (more than one per CU), else 16. Heads are independent, so the first two key heads of a problem that takes
    32-row blocks (Hv = 48: 384 to 1,536 blocks of 16 rows; with Dv = 32 a head is one 32-row block) give the bits of
    the same heads run alone (Hv = 6: 48 to 192 blocks, 16 rows each), and the whole problem matches the oracle.
    Both sizes keep NC * Hv <= 256, so the gradient kernel takes one work item per value head in both and sums dq, dk
    the same way."""
    torch = torch_dev
    from quotebound_amd.synthetic import Workload, make_inputs, to_device

    packed = lens is not None
    w = Workload("rows", 1, sum(lens) if packed else 200, 16, 48, 128, Dv, seed=41, s0_std=0.02, ds_out=True,
                 seq_lens=lens)
    assert w.n_states * w.Hv * Dv // 16 > 256 >= w.n_states * 6 * Dv // 16  # 32-row blocks in full, 16 in the slice
    inp = make_inputs(w)
    cu = w.cu_seqlens
    d = to_device(inp)
    d = dict(d, dy=d["dy"].float())
    full = run(torch, d, _lib.CHUNKED, cu=cu, out_f32=True)
    exp = oracle.fwd_bwd(inp.f32, cu_seqlens=cu, dtype=np.float32)
    assert_close(full, exp, BF16_TOL, label=f"rows packed={packed} Dv={Dv}")
    sub = {n: d[n][:, :, :2].contiguous() for n in ("q", "k")}
    sub.update({n: d[n][:, :, :6].contiguous() for n in ("v", "g", "beta", "dy")})
    sub.update({n: d[n][:, :6].contiguous() for n in ("s0", "ds_out")})
    part = run(torch, sub, _lib.CHUNKED, cu=cu, out_f32=True)
    for n in ("y", "dv", "dg", "dbeta"):
        assert np.array_equal(part[n], full[n][:, :, :6]), n
    for n in ("dq", "dk"):
        assert np.array_equal(part[n], full[n][:, :, :2]), n
    for n in ("s_out", "ds0"):
        assert np.array_equal(part[n], full[n][:, :6]), n


@pytest.mark.parametrize("design", DESIGNS, ids=DESIGN_IDS.get)
def test_deterministic(torch_dev, design):
    """Same inputs, same bits: every sum runs in a fixed order (the reference's resume bit-identity relies on it,
    reference src/delta_grad.cpp:19-22)."""
    torch = torch_dev
    from quotebound_amd.synthetic import Workload, make_inputs, to_device

    w = Workload("det", 1, 700, 4, 8, 128, 128, seed=21, s0_std=0.02, ds_out=True)
    d = to_device(make_inputs(w))
    a = run(torch, d, design)
    b = run(torch, d, design)
    for n in OUT_NAMES:
        assert np.array_equal(a[n], b[n]), n


@pytest.mark.parametrize("design", DESIGNS, ids=DESIGN_IDS.get)
def test_forward_backward_in_a_graph(torch_dev, design):
    """qb_gdn_fwd then qb_gdn_bwd captured into one HIP graph on a side stream (buffers allocated outside the
    capture; the calls issue no allocation and no memset), replayed three times with eager calls of the same pair
    between the replays and every output poisoned before each replay: every replay equals the eager pair, bit for
    bit, for a packed batch with an empty sequence, an initial state and a final-state cotangent."""
    torch = torch_dev
    from quotebound_amd.synthetic import Workload, make_inputs, to_device

    w = Workload("graph", 1, 700, 4, 8, 128, 128, seed=71, s0_std=0.02, ds_out=True, seq_lens=[300, 0, 400])
    print(f"fwd+bwd in a graph: T={w.T} Hk={w.Hk} Hv={w.Hv} packed {w.seq_lens} design {design}", flush=True)
    d = to_device(make_inputs(w))
    desc_f, keep_f = _lib.make_desc(w.B, w.T, w.Hk, w.Hv, w.Dk, w.Dv, design=design, cu_seqlens=w.cu_seqlens)
    desc_b, keep_b = _lib.make_desc(w.B, w.T, w.Hk, w.Hv, w.Dk, w.Dv, design=design, cu_seqlens=w.cu_seqlens)
    N = w.n_states
    ckpt = torch.empty(_lib.ckpt_bytes(desc_f) // 4, device="cuda")
    ws = torch.empty(max(_lib.workspace_bytes(desc_f), 1), dtype=torch.uint8, device="cuda")

    def outs():
        return [torch.empty_like(d["v"]), torch.empty(N, w.Hv, w.Dv, w.Dk, device="cuda"), torch.empty_like(d["q"]),
                torch.empty_like(d["k"]), torch.empty_like(d["v"]), torch.empty_like(d["g"]),
                torch.empty_like(d["beta"]), torch.empty(N, w.Hv, w.Dv, w.Dk, device="cuda")]

    p = lambda t: t.data_ptr()  # noqa: E731

    def pair(o, stream):
        y, s_out, dq, dk, dv, dg, dbeta, ds0 = o
        _lib.fwd(desc_f, p(d["q"]), p(d["k"]), p(d["v"]), p(d["g"]), p(d["beta"]), p(d["s0"]), p(y), p(s_out),
                 p(ckpt), p(ws), stream)
        _lib.bwd(desc_b, p(d["q"]), p(d["k"]), p(d["v"]), p(d["g"]), p(d["beta"]), p(ckpt), p(d["dy"]),
                 p(d["ds_out"]), p(dq), p(dk), p(dv), p(dg), p(dbeta), p(ds0), p(ws), stream)

    names = ("y", "s_out", "dq", "dk", "dv", "dg", "dbeta", "ds0")
    want, got, again = outs(), outs(), outs()
    pair(want, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    for name, t in zip(names, want):
        assert not torch.isnan(t.float()).any(), name
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.graph(graph, stream=side):
        pair(got, side.cuda_stream)
    torch.cuda.synchronize()
    for r in range(3):
        for t in got + [ckpt]:
            t.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for name, a, b in zip(names, want, got):
            assert torch.equal(a, b), f"replay {r} {name}: max |diff| {(a.float() - b.float()).abs().max().item()}"
        pair(again, torch.cuda.current_stream().cuda_stream)  # eager work between the replays
        torch.cuda.synchronize()
        for name, a, b in zip(names, want, again):
            assert torch.equal(a, b), f"eager after replay {r} {name}"
    del graph, keep_f, keep_b


@pytest.mark.parametrize("design", DESIGNS, ids=DESIGN_IDS.get)
def test_trainable_autograd_matches_vjp(torch_dev, design):
    """gated_delta_trainable under torch autograd gives gated_delta_vjp's cotangents (reference
    src/delta_grad.cpp:201-212), with the decay factor as input as the reference's gated_delta takes it."""
    torch = torch_dev
    from quotebound_amd import gdn

    B, T, Hk, Hv, D = 1, 130, 2, 4, 128
    inp = reference_case(B, T, Hk, Hv, D, D, 0.9, seed=31)
    d = host_to_dev(torch, inp, torch.bfloat16)
    leaves = {k: d[k].clone().requires_grad_(True) for k in ("q", "k", "v", "g", "beta", "s0")}
    y, s = gdn.gated_delta(leaves["q"], leaves["k"], leaves["v"], leaves["g"], leaves["beta"], leaves["s0"],
                           train=True, design=design)
    assert y.dtype == torch.bfloat16 and s.dtype == torch.float32
    ((y.float() * d["dy"].float()).sum() + (s * d["ds_out"]).sum()).backward()
    vjp = gdn.gated_delta_vjp([d[k] for k in ("q", "k", "v", "g", "beta", "s0")], d["dy"], d["ds_out"],
                              design=design)
    for name, got in zip(("q", "k", "v", "g", "beta", "s0"), vjp):
        assert torch.equal(leaves[name].grad, got), name
    y2, s2 = gdn.gated_delta(d["q"], d["k"], d["v"], d["g"], d["beta"], d["s0"], design=design)
    assert torch.equal(y2, y.detach()) and torch.equal(s2, s.detach())
