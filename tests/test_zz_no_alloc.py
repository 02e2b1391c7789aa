"""qb_gdn_bwd_static, the backward without a workspace argument (its scratch is a static per-GPU array), against
qb_gdn_bwd with a caller-allocated workspace: the same outputs bit for bit, on two calls in a row, the second with a
smaller input, for each design, all through the C ABI."""
import pytest

from quotebound_amd import _lib

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_dev():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    _lib.load()
    return torch


def _case(torch, w, design):
    """Inputs on the device, the forward's ckpt and two sets of gradient outputs (for the two entry points). The
    tensors behind the pointers come back too (in `hold`), so that they stay allocated while the pointers are used."""
    from quotebound_amd.synthetic import make_inputs, to_device

    d = to_device(make_inputs(w))
    desc, keep = _lib.make_desc(w.B, w.T, w.Hk, w.Hv, w.Dk, w.Dv, dtype=_lib.BF16, design=design,
                                cu_seqlens=w.cu_seqlens)
    assert _lib.validate(desc) is None
    N = w.n_states
    p = lambda t: None if t is None else t.data_ptr()  # noqa: E731
    stream = torch.cuda.current_stream().cuda_stream
    y = torch.empty_like(d["v"])
    s_out = torch.empty(N, w.Hv, w.Dv, w.Dk, dtype=torch.float32, device="cuda")
    ckpt = torch.empty(_lib.ckpt_bytes(desc) // 4, dtype=torch.float32, device="cuda")
    ws = torch.empty(max(_lib.workspace_bytes(desc), 1), dtype=torch.uint8, device="cuda")
    _lib.fwd(desc, p(d["q"]), p(d["k"]), p(d["v"]), p(d["g"]), p(d["beta"]), p(d["s0"]), p(y), p(s_out), p(ckpt),
             p(ws), stream)

    def outs():
        return [torch.full_like(d["q"], float("nan")), torch.full_like(d["k"], float("nan")),
                torch.full_like(d["v"], float("nan")), torch.full_like(d["g"], float("nan")),
                torch.full_like(d["beta"], float("nan")),
                torch.full((N, w.Hv, w.Dv, w.Dk), float("nan"), dtype=torch.float32, device="cuda")]

    args = [p(d["q"]), p(d["k"]), p(d["v"]), p(d["g"]), p(d["beta"]), p(ckpt), p(d["dy"]), p(d["ds_out"])]
    hold = (d, y, s_out, ckpt, keep)
    return desc, hold, args, ws, outs, stream


@pytest.mark.parametrize("design", [_lib.CHUNKED, _lib.RECURRENT], ids=["chunked", "recurrent"])
def test_static_scratch_backward_matches(torch_dev, design):
    torch = torch_dev
    from quotebound_amd.synthetic import Workload

    if design == _lib.CHUNKED:  # the 4B layer shape (128 MiB of workspace), then a smaller packed batch
        shapes = [Workload("big", 1, 4096, 16, 32, 128, 128, seed=61, s0_std=0.02, ds_out=True),
                  Workload("small", 1, 700, 4, 8, 128, 128, seed=62, s0_std=0.02, ds_out=True,
                           seq_lens=[300, 0, 400])]
    else:  # the recurrent design's partial sums are larger per token
        shapes = [Workload("big", 1, 1024, 4, 8, 128, 128, seed=63, s0_std=0.02, ds_out=True),
                  Workload("small", 2, 150, 2, 4, 64, 64, seed=64, ds_out=True)]
    for w in shapes:
        print(f"static-scratch backward, design {design}, {w.name}: B={w.B} T={w.T} Hk={w.Hk} Hv={w.Hv} "
              f"Dk={w.Dk} Dv={w.Dv}", flush=True)
        desc, hold, args, ws, outs, stream = _case(torch, w, design)
        assert 0 < _lib.workspace_bytes(desc) <= _lib.STATIC_SCRATCH_BYTES
        want, got = outs(), outs()
        p = lambda t: t.data_ptr()  # noqa: E731
        _lib.bwd(desc, *args, *[p(t) for t in want], ws.data_ptr(), stream)
        _lib.bwd_static(desc, *args, *[p(t) for t in got], stream)
        torch.cuda.synchronize()
        for name, a, b in zip(("dq", "dk", "dv", "dg", "dbeta", "ds0"), want, got):
            assert not torch.isnan(a).any(), name
            assert torch.equal(a, b), f"{w.name} {name}: max |diff| {(a.float() - b.float()).abs().max().item()}"
        del hold


def test_static_scratch_refuses_oversize(torch_dev):
    """A shape whose workspace exceeds the static array is refused before any GPU work."""
    d, _ = _lib.make_desc(1, 4096, 16, 32, 128, 128, design=_lib.RECURRENT)
    assert _lib.workspace_bytes(d) > _lib.STATIC_SCRATCH_BYTES
    with pytest.raises(RuntimeError, match="without allocation needs"):
        _lib.bwd_static(d, *([16] * 14), None)


def test_static_scratch_backward_in_a_graph(torch_dev):
    """qb_gdn_bwd_static captured into a HIP graph on a side stream (after its first call on the device, outside the
    capture, as the header asks), replayed three times with eager work between the replays: every replay equals
    qb_gdn_bwd with a caller-allocated workspace, bit for bit."""
    torch = torch_dev
    from quotebound_amd.synthetic import Workload

    w = Workload("graph", 1, 700, 4, 8, 128, 128, seed=65, s0_std=0.02, ds_out=True, seq_lens=[300, 0, 400])
    print(f"static-scratch backward in a graph: T={w.T} Hk={w.Hk} Hv={w.Hv} packed {w.seq_lens}", flush=True)
    desc, hold, args, ws, outs, stream = _case(torch, w, _lib.CHUNKED)
    p = lambda t: t.data_ptr()  # noqa: E731
    names = ("dq", "dk", "dv", "dg", "dbeta", "ds0")
    want, got = outs(), outs()
    _lib.bwd(desc, *args, *[p(t) for t in want], ws.data_ptr(), stream)
    _lib.bwd_static(desc, *args, *[p(t) for t in got], stream)  # the first call on the device, outside any capture
    torch.cuda.synchronize()
    for name, a, b in zip(names, want, got):
        assert not torch.isnan(a).any(), name
        assert torch.equal(a, b), name
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.graph(graph, stream=side):
        _lib.bwd_static(desc, *args, *[p(t) for t in got], side.cuda_stream)
    torch.cuda.synchronize()
    again = outs()
    for r in range(3):
        for t in got:
            t.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for name, a, b in zip(names, want, got):
            assert torch.equal(a, b), f"replay {r} {name}: max |diff| {(a.float() - b.float()).abs().max().item()}"
        # eager work between the replays: the allocating backward again, into other buffers
        _lib.bwd(desc, *args, *[p(t) for t in again], ws.data_ptr(), stream)
        torch.cuda.synchronize()
        for name, a, b in zip(names, want, again):
            assert torch.equal(a, b), f"eager after replay {r} {name}"
    del graph, hold
