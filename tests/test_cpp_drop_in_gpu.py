"""The reference's decode-attention call sequence from C++ through the C ABI.

tests/cpp/drop_in.cpp makes the calls the reference's main() makes (decode_attention with the
three split settings of 01_decode_attention.cu:763 on the correctness cases of 01:750-755;
shared_prefix_pages / plan_cascade / cascade_decode on the cascade cases of 01:782-815), plus
plan / run, from C++ against include/pdattn.h, and checks every result against the fp64 oracle
with the parity bar. It is built as a shared library (tests/cpp/Makefile, run by build()) and
called here in this process.
"""
import ctypes
import os

import pytest

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "cpp", "libdrop_in.so")


def test_cpp_caller_matches_oracle(capfd):
    import _gpu
    _gpu.device()
    if not os.path.exists(LIB):
        raise RuntimeError(f"{LIB} is missing: build it with __graft_entry__.build() or make -C tests/cpp")
    print("[cpp] drop_in checks", flush=True)
    failures = ctypes.CDLL(LIB).pdattn_drop_in_checks()
    out = capfd.readouterr().out
    print(out)
    assert failures == 0, out
    assert "ALL PASS" in out
