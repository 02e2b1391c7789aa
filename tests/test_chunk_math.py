"""The chunkwise equations the chunked HIP design implements (tests/chunk_math.py) agree with the oracle in
float64, including partial last chunks, GQA groups of 2 and 3, and a nonzero initial state."""
import pytest

from chunk_math import gated_delta_chunked
from helpers import normwise, small_case

NAMES = ("y", "s_out", "dq", "dk", "dv", "dg", "dbeta", "ds0")


@pytest.mark.parametrize("shape", [(1, 20, 1, 2, 8, 6, 8), (2, 37, 2, 4, 16, 8, 16), (1, 130, 1, 3, 16, 8, 64)])
def test_chunk_form_equals_recurrence(oracle, shape):
    B, T, Hk, Hv, Dk, Dv, C = shape
    inp = small_case(B, T, Hk, Hv, Dk, Dv, seed=3)
    ref = oracle.fwd_bwd(inp, chunk=C)
    got = gated_delta_chunked(inp["q"], inp["k"], inp["v"], inp["g"], inp["beta"], inp["s0"], inp["dy"],
                              inp["ds_out"], C=C)
    for name, x in zip(NAMES, got):
        assert normwise(x, ref[name]) <= 1e-12, name
