"""Writes tests/golden/tiny_fp32.npz: the tiny float32 workload (B=1, T=64, Hk=Hv=2, Dk=Dv=32, seed 0; log-decay
-softplus(N(0,1)), beta sigmoid(N(0,1)), zero initial state, dy ~ N(0,1)) with its outputs and gradients.

The expected values come from autodiff in float64 through the plain-ops recurrence (tests/plain_ops.py, the form of
reference tests/gated_delta_ref.h:100-120), not from the oracle, so the fixture checks the oracle independently.
A second case (tiny_fp32_s0) adds a nonzero initial state ~N(0, 0.1), a final-state cotangent and GQA (Hk=1, Hv=2),
as the reference's gradient tests do (reference tests/test_deltanet.cpp:106-112).

Run from the repository root: python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
sys.path.insert(0, os.path.dirname(HERE))

from plain_ops import fwd_bwd  # noqa: E402
from quotebound_amd.synthetic import Workload, make_inputs, workload  # noqa: E402

KEYS_IN = ("q", "k", "v", "g", "beta", "dy", "s0", "ds_out")
KEYS_OUT = ("y", "s_out", "dq", "dk", "dv", "dg", "dbeta", "ds0")


def write(name, w):
    inp = make_inputs(w)
    ref = fwd_bwd(inp.f32)
    arrays = {}
    for k in KEYS_IN:
        if inp.f32.get(k) is not None:
            arrays["in_" + k] = inp.f32[k].astype(np.float32)
    for k in KEYS_OUT:
        arrays["out_" + k] = ref[k].astype(np.float64)
    path = os.path.join(HERE, name + ".npz")
    np.savez_compressed(path, **arrays)
    print("wrote", path, sum(a.nbytes for a in arrays.values()), "bytes")


if __name__ == "__main__":
    write("tiny_fp32", workload("tiny"))
    w = Workload("tiny_s0", 1, 64, 1, 2, 32, 32, dtype="f32", seed=7, clip_log_decay=None, s0_std=0.1, ds_out=True)
    write("tiny_fp32_s0", w)
