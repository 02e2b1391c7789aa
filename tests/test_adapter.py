"""The C++ adapters (include/qb: qb::array, gated_delta, gated_delta_trainable, gated_delta_vjp), which keep the
reference's entry points (src/deltanet.h:17-19, src/delta_grad.h:14-20). The GPU check runs tests/cxx/adapter_check,
a C++ program that compares them with the oracle; build() compiles it."""
import ctypes
import os
import subprocess

import pytest

from quotebound_amd import _lib

HERE = os.path.dirname(os.path.abspath(__file__))
CHECK = os.path.join(HERE, "cxx", "adapter_check")

# The C++ entry points, mangled (Itanium ABI), that include/qb declares.
CXX_SYMBOLS = [
    "_ZN2qb11gated_deltaERKNS_5arrayES2_S2_S2_S2_S2_b",
    "_ZN2qb21gated_delta_trainableERKNS_5arrayES2_S2_S2_S2_S2_",
    "_ZN2qb15gated_delta_vjpERKSt6vectorINS_5arrayESaIS1_EERKS1_S7_",
    "_ZN2qb16gated_delta_rowsERKNS_5arrayES2_S2_S2_S2_S2_",
    "_ZN2qb17deltanet_prologueERKNS_5arrayES2_S2_S2_S2_S2_",
    "_ZN2qb21deltanet_prologue_vjpERKNS_5arrayES2_S2_S2_S2_S2_S2_S2_S2_S2_",
    "_ZN2qb17deltanet_epilogueERKNS_5arrayES2_S2_f",
    "_ZN2qb21deltanet_epilogue_vjpERKNS_5arrayES2_S2_fS2_",
    "_ZN2qb5arrayC1ESt6vectorIiSaIiEENS_5DtypeE",
    "_ZN2qb5array9from_hostEPKvSt6vectorIiSaIiEENS_5DtypeE",
    "_ZN2qb5array5zerosESt6vectorIiSaIiEENS_5DtypeE",
    "_ZNK2qb5array7to_hostEPv",
    "_ZN2qb6astypeERKNS_5arrayENS_5DtypeE",
    "_ZN2qb10set_streamEPv",
    "_ZN2qb6streamEv",
]


def test_library_exports_cxx_adapters():
    lib = ctypes.CDLL(_lib.LIB_PATH)
    missing = [s for s in CXX_SYMBOLS if not hasattr(lib, s)]
    assert not missing, missing


def test_adapter_check_is_built():
    assert os.access(CHECK, os.X_OK), "run __graft_entry__.build() first"


@pytest.mark.gpu
def test_adapters_match_oracle():
    r = subprocess.run([CHECK], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0 and r.stdout.rstrip().endswith("PASS"), r.stdout + r.stderr
