"""bench.py's arithmetic without a GPU: the per-kernel algorithmic and design bytes and the step roofline that the
bench line reports, against the figures they are derived from (the path's tensor sizes at the 4B layer shape), and
the refusal of a run on more than one GPU."""
import os
import subprocess
import sys

import pytest

from quotebound_amd import _lib
from quotebound_amd.synthetic import workload

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
import bench  # noqa: E402

MB = 1 << 20


def test_tensor_sizes_at_the_4b_shape():
    w = workload("qwen35_4b")  # B=1, T=4096, Hk=16, Hv=32, Dk=Dv=128, bf16 activations
    s = bench._sizes(w, 64)
    assert s["q"] == s["k"] == s["dq"] == 4096 * 16 * 128 * 2 == 16 * MB
    assert s["v"] == s["y"] == s["dy"] == s["dv"] == 32 * MB
    assert s["g"] == 4096 * 32 * 4 and s["beta"] == 4096 * 32 * 2
    assert s["ckpt_read"] == 64 * 32 * 128 * 128 * 4 == 128 * MB
    assert s["ckpt_write"] == 63 * 32 * 128 * 128 * 4  # the first chunk's start state is the initial state
    f = bench._sizes(workload("qwen35_4b_f32"), 64)
    assert f["q"] == 2 * s["q"] and f["v"] == 2 * s["v"] and f["g"] == s["g"]


def test_gradient_kernel_bytes():
    """chunk_bwd_grads reads q, k, v, dy, g, beta and the checkpoints and writes dq, dk, dg, dbeta: 270,008,320
    bytes a launch at 4B; the design's intermediates it reads (the chunk tiles and the chunk-end cotangents) are
    reported apart."""
    w = workload("qwen35_4b")
    desc, _ = _lib.make_desc(w.B, w.T, w.Hk, w.Hv, w.Dk, w.Dv, dtype=_lib.BF16, design=_lib.CHUNKED)
    nc = _lib.num_chunks(desc)
    tiles = _lib.ckpt_bytes(desc) - nc * w.Hv * w.Dv * w.Dk * 4
    kind, amount, design = bench.algorithmic_work(w, "chunk_bwd_grads", nc, tiles)
    assert (kind, nc) == ("bytes", 64)
    s = bench._sizes(w, nc)
    assert amount == sum(s[n] for n in ("q", "k", "v", "dy", "g", "beta", "ckpt_read", "dq", "dk", "dg", "dbeta"))
    assert amount == 270_008_320
    # one tile record per (chunk, value head): T and P as packed bf16 hi/lo blocks (4 x 2560 elements) and four
    # 64-float vectors, 21,504 bytes
    assert tiles == 64 * 32 * (4 * 2560 * 2 + 4 * 64 * 4) == 44_040_192
    assert design == tiles + s["ckpt_read"] == 178_257_920


def test_step_roofline_4b():
    """The step's compulsory bytes (forward and backward I/O, each tensor once per pass, plus the checkpoints
    written and read once) over 8 TB/s: 67.4 us at 4B, well above the MFMA time of its 22 Dk Dv flops per token and
    value head at 2.5 PFLOP/s."""
    t, nbytes, flops = bench.step_roof_us(workload("qwen35_4b"), 64)
    assert nbytes == 539_230_208
    assert t == pytest.approx(nbytes / 8e12 * 1e6) == pytest.approx(67.4037, abs=1e-3)
    assert flops / 2.5e15 * 1e6 < t


def test_roofline_fraction():
    r = bench.roofline_of("bytes", 270_008_320, 0.1650)
    assert r["unit"] == "GB/s" and r["peak"] == 8000.0
    assert r["achieved"] == pytest.approx(270_008_320 / 0.165e-3 / 1e9)
    assert r["frac"] == pytest.approx(r["achieved"] / 8000.0)
    v = bench.roofline_of("flops", 1e12, 10.0)  # 1 TFLOP in 10 ms: 100 TFLOP/s
    assert v["bound"] == "valu" and v["achieved"] == pytest.approx(100.0) and v["frac"] == pytest.approx(100.0 / 157.3)


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=60)
    assert r.returncode == 2 and "measures one GPU" in r.stderr
