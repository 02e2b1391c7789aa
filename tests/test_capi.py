"""The C ABI without a GPU: the library loads, exports everything include/qb_gdn.h declares, and rejects bad
descriptors and pointers with a reason (reference convention: src/constrain_capi.h:8-9; the reference's own shape
checks: src/delta_grad.cpp:159-170). No call here reaches a kernel launch."""
import ctypes
import re
import subprocess

import pytest

from quotebound_amd import _lib


@pytest.fixture(scope="module")
def lib():
    import os

    if not os.path.exists(_lib.LIB_PATH):
        from quotebound_amd import build

        build.build(force=False)
    return _lib.load()


def declared_functions():
    text = open(_lib.HEADER_PATH).read()
    return sorted(set(re.findall(r"\b(qb_gdn_\w+)\s*\(", text)))


def test_exports_every_declared_function(lib):
    names = declared_functions()
    assert {"qb_gdn_fwd", "qb_gdn_bwd", "qb_gdn_workspace_bytes", "qb_gdn_ckpt_bytes"} <= set(names)
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    exported = set(re.findall(r" T (qb_gdn_\w+)", out))
    for n in names:
        assert n in exported, n
        assert getattr(lib, n) is not None
    assert lib.qb_gdn_version().decode().startswith("qb_gdn")


def test_desc_layout_matches_header():
    # 11 int32 fields, then a pointer (8-byte aligned), then n_seqs.
    assert _lib.Desc.out_f32.offset == 40
    assert _lib.Desc.cu_seqlens.offset == 48
    assert _lib.Desc.n_seqs.offset == 56
    assert _lib.Desc.trace_events.offset == 64
    assert _lib.Desc.n_trace_events.offset == 72
    assert ctypes.sizeof(_lib.Desc) == 80


def desc(**kw):
    base = dict(B=1, T=4096, Hk=16, Hv=32, Dk=128, Dv=128, design=_lib.RECURRENT)
    base.update(kw)
    cu = base.pop("cu_seqlens", None)
    return _lib.make_desc(base.pop("B"), base.pop("T"), base.pop("Hk"), base.pop("Hv"), base.pop("Dk"),
                          base.pop("Dv"), cu_seqlens=cu, **base)


def test_accepts_the_layer_shapes(lib):
    for Hv in (32, 48):
        d, _ = desc(Hv=Hv)
        assert _lib.validate(d) is None


@pytest.mark.parametrize("Dk", [32, 64, 96, 128, 160, 192, 224, 256, 288, 512, 1024, 2080, 4096])
def test_recurrent_design_takes_every_key_width_to_4096(lib, Dk):
    """Multiples of 32 up to 4096: the reference's own cases go to 256 (reference tests/test_deltanet.cpp:154) and its
    vjp takes any multiple of 32 whose row reduction fits 32 KB of threadgroup memory (src/delta_grad.cpp:159-170)."""
    for dt in (_lib.F32, _lib.BF16):
        d, _ = desc(Dk=Dk, Dv=64, dtype=dt, design=_lib.RECURRENT)
        assert _lib.validate(d) is None


@pytest.mark.parametrize("kw,needle", [
    (dict(Hv=30), "multiple of key heads"),
    (dict(Dk=100), "Dk a multiple of 32"),
    (dict(chunk=32), "stride must be 64"),
    (dict(dtype=7), "dtype"),
    (dict(design=3), "design"),
    (dict(B=0), "positive"),
    (dict(Dk=4128, design=_lib.RECURRENT), "recurrent design needs Dk a multiple of 32 of at most 4096"),
    (dict(B=2, T=10, cu_seqlens=[0, 4, 10]), "B == 1"),
    (dict(T=10, cu_seqlens=[0, 4, 9]), "from 0 to T"),
    (dict(T=10, cu_seqlens=[0, 6, 4, 10]), "must not decrease"),
    (dict(T=256, cu_seqlens=list(range(257))), "n_seqs"),
])
def test_rejects_with_reason(lib, kw, needle):
    d, _ = desc(**kw)
    why = _lib.validate(d)
    assert why is not None and needle in why, why
    assert _lib.workspace_bytes(d) == 0 and _lib.ckpt_bytes(d) == 0 and _lib.num_chunks(d) == -1


def test_chunk_slots_and_sizes(lib):
    d, _ = desc(T=4096)
    assert _lib.num_chunks(d) == 64
    # The chunk-start states, then the recurrent design's e = v - u per token and state row.
    assert _lib.ckpt_bytes(d) == (64 * 32 * 128 * 128 + 4096 * 32 * 128) * 4
    d, _ = desc(B=3, T=65, Hv=16)
    assert _lib.num_chunks(d) == 6
    lens = [5, 64, 0, 130, 1]
    cu = [0]
    for n in lens:
        cu.append(cu[-1] + n)
    d, keep = desc(T=cu[-1], cu_seqlens=cu)
    assert _lib.num_chunks(d) == 1 + 1 + 0 + 3 + 1


def test_launch_names(lib):
    d, _ = desc()
    assert _lib.launches(d, 0) == ["rec_fwd"]
    assert _lib.launches(d, 1) == ["rec_bwd", "rec_reduce"]
    bad, _ = desc(Hv=30)
    with pytest.raises(RuntimeError):
        _lib.launches(bad, 0)


def test_launch_errors_before_any_gpu_work(lib):
    d, _ = desc(Hv=30)
    with pytest.raises(RuntimeError, match="multiple of key heads"):
        _lib.fwd(d, 16, 16, 16, 16, 16, None, 16, None, None, None, None)
    d, _ = desc()
    with pytest.raises(RuntimeError, match="q is null"):
        _lib.fwd(d, None, 16, 16, 16, 16, None, 16, None, None, 16, None)
    with pytest.raises(RuntimeError, match="k must be 16-byte aligned"):
        _lib.fwd(d, 16, 18, 16, 16, 16, None, 16, None, None, 16, None)
    with pytest.raises(RuntimeError, match="ckpt is null"):
        _lib.bwd(d, 16, 16, 16, 16, 16, None, 16, None, 16, 16, 16, 16, 16, None, 16, None)
    with pytest.raises(RuntimeError, match="workspace is null"):
        _lib.bwd(d, 16, 16, 16, 16, 16, 16, 16, None, 16, 16, 16, 16, 16, None, None, None)


def test_neighbours_errors_before_any_gpu_work(lib):
    d, _ = desc(Dk=32, Dv=32)
    with pytest.raises(RuntimeError, match="Dk of 64, 128 or 256"):
        _lib.prologue_fwd(d, 16, 16, 16, 16, 16, 16, 16, 16, 16, 16, None)
    assert _lib.neighbours_workspace_bytes(d) == 0
    d, _ = desc(Dk=128, Dv=32)  # the prologue runs on Dk alone, the epilogue on Dv alone
    with pytest.raises(RuntimeError, match="a_log is null"):
        _lib.prologue_fwd(d, 16, 16, 16, 16, None, 16, 16, 16, 16, 16, None)
    with pytest.raises(RuntimeError, match="Dv of 64, 128 or 256"):
        _lib.epilogue_fwd(d, 16, 16, 16, 1e-6, 16, None)
    d, _ = desc()
    assert _lib.neighbours_workspace_bytes(d) > 0
    with pytest.raises(RuntimeError, match="a_log is null"):
        _lib.prologue_fwd(d, 16, 16, 16, 16, None, 16, 16, 16, 16, 16, None)
    with pytest.raises(RuntimeError, match="workspace is null"):
        _lib.prologue_bwd(d, *([16] * 16), None, None)
    with pytest.raises(RuntimeError, match="eps must be positive"):
        _lib.epilogue_fwd(d, 16, 16, 16, 0.0, 16, None)
    with pytest.raises(RuntimeError, match="y must be 16-byte aligned"):
        _lib.epilogue_bwd(d, 17, 16, 16, 1e-6, 16, 16, 16, 16, 16, None)


def test_fwd_rows_errors_before_any_gpu_work(lib):
    d, _ = desc(Dk=4128, Dv=64, design=_lib.CHUNKED)
    with pytest.raises(RuntimeError, match="Dk"):
        _lib.fwd_rows(d, 16, 16, 16, 16, 16, None, 16, 16, None)
    d, _ = desc()
    with pytest.raises(RuntimeError, match="row_states is null"):
        _lib.fwd_rows(d, 16, 16, 16, 16, 16, None, 16, None, None)



def test_bwd_static_refuses_before_any_gpu_work(lib):
    """The backward without allocation refuses a shape whose workspace exceeds its static array, and checks its
    pointers, before it touches the GPU."""
    d, _ = desc(T=4096, design=_lib.RECURRENT)
    assert _lib.workspace_bytes(d) > _lib.STATIC_SCRATCH_BYTES
    with pytest.raises(RuntimeError, match="without allocation needs"):
        _lib.bwd_static(d, *([16] * 14), None)
    d, _ = desc(T=4096, design=_lib.CHUNKED)
    assert _lib.workspace_bytes(d) <= _lib.STATIC_SCRATCH_BYTES
    with pytest.raises(RuntimeError, match="ckpt is null"):
        _lib.bwd_static(d, 16, 16, 16, 16, 16, None, 16, None, 16, 16, 16, 16, 16, None, None)
