"""The timeline build of the library (make -C cuda-kernel-lab_amd timeline: the kernels compiled
with per-workgroup timestamps, read by bench.py --timeline) computes exactly what the library
proper computes, and its stamps come in phase order.

The timeline build is loaded in a child process, so this process keeps the library proper.
"""
import os
import subprocess
import sys
import textwrap

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
TL_LIB = os.path.join(ROOT, "cuda-kernel-lab_amd", "lib", "timeline", "libpdattn.so")

CHILD = textwrap.dedent(r"""
    import ctypes, os, sys
    import numpy as np
    import torch
    sys.path.insert(0, os.path.join(sys.argv[1], "cuda-kernel-lab_amd"))
    sys.path.insert(0, os.path.join(sys.argv[1], "tests"))
    import pdattn
    from pdattn import inputs
    import _gpu

    def run(lib_path, bt):
        pdattn._lib = None
        pdattn.LIB_PATH = lib_path
        L = pdattn.lib()
        db = _gpu.DeviceBatch(bt)
        o, l, info = _gpu.run_plan(db)
        return L, o, l, info

    print("[case] timeline build vs library, lens=[3000, 17, 700]", flush=True)
    bt = inputs.make_batch([3000, 17, 700], 32, 8, seed=51)
    _, o0, l0, _ = run(os.path.join(sys.argv[1], "cuda-kernel-lab_amd", "lib", "libpdattn.so"), bt)
    L, o1, l1, info = run(sys.argv[2], bt)
    assert np.array_equal(o0, o1) and np.array_equal(l0, l1), "timeline build changed the results"
    L.pdattn_timeline_read_decode.argtypes = [ctypes.c_void_p, ctypes.c_size_t]
    buf = np.zeros(8192 * 32, np.uint64)
    assert L.pdattn_timeline_read_decode(buf.ctypes.data, buf.nbytes) == 0
    t = buf.reshape(8192, 32)[:info.workgroups].astype(np.int64)
    ran = t[:, 0] > 0
    assert ran.sum() > 0
    for row in t[ran]:
        seq = [row[0], row[1], row[2]] + [row[s] for s in range(4, 28) if row[s] > 0] + [row[31]]
        assert all(b >= a for a, b in zip(seq, seq[1:])), f"stamps out of order: {seq}"
    print("ok", int(ran.sum()), "workgroups stamped", flush=True)
""")


@pytest.mark.skipif(not os.path.exists(TL_LIB), reason="timeline build absent (make -C cuda-kernel-lab_amd timeline)")
def test_timeline_build_matches_library_and_stamps_in_order():
    r = subprocess.run([sys.executable, "-c", CHILD, ROOT, TL_LIB], capture_output=True, text=True,
                       timeout=110)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    assert "ok" in r.stdout
