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


def test_split_bf16_products_on_float32_inputs(oracle):
    """Why float32 callers get the recurrent design: the chunk equations on float32 inputs with every matrix product
    taken as the chunked kernels take theirs (each operand split into bf16 hi + lo, the products hi.hi + hi.lo +
    lo.hi accumulated in float32) land at the reference's 1e-5 float32 criterion, not under it, while the same
    equations in plain float32 stay two orders below. Measured on one of the reference's gradient cases (three chunks,
    the last partial; reference tests/test_deltanet.cpp:145-154) against the oracle in float64."""
    import numpy as np

    import chunk_math
    from helpers import reference_case
    from quotebound_amd.synthetic import round_bf16

    def split_mm(x, y):
        xh, yh = round_bf16(x), round_bf16(y)
        xl, yl = round_bf16(x - xh), round_bf16(y - yh)
        return xh @ yh + (xh @ yl + xl @ yh)

    inp = reference_case(1, 129, 2, 4, 128, 128, 0.9, seed=229)
    inp["g"] = np.log(inp["g"])
    ref = oracle.fwd_bwd(inp)
    keys = ("q", "k", "v", "g", "beta", "s0", "dy", "ds_out")
    errs = {}
    for mode, mm in (("f32", None), ("split", split_mm)):
        chunk_math.MM = mm
        try:
            got = gated_delta_chunked(*(np.asarray(inp[n], np.float32) for n in keys))
        finally:
            chunk_math.MM = None
        errs[mode] = {n: normwise(np.asarray(x, np.float64), ref[n]) for n, x in zip(NAMES, got)}
    print(errs)
    assert max(errs["f32"].values()) <= 1e-6
    assert 5e-6 <= max(errs["split"].values()) <= 5e-5
