"""The timeline build of the library (make -C cuda-kernel-lab_amd timeline: the kernels compiled
with per-workgroup timestamps, read by bench.py --timeline) computes exactly what the library
proper computes, and its stamps come in phase order: the plan path's decode (one kv head per
workgroup, and the paired kernel), the fused cascade step (decode and prefix roles, then the
merge) and the prefix kernel alone with a partial last chunk (its 4-wave and key-split bodies),
each compared bit for bit.

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
    lib0 = os.path.join(sys.argv[1], "cuda-kernel-lab_amd", "lib", "libpdattn.so")
    _, o0, l0, _ = run(lib0, bt)
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

    # the paired kernel (a plan that splits no sequence: 64 x 1024 tokens on 256 CUs)
    print("[case] paired kernel, timeline build vs library, 64 x 1024", flush=True)
    bq = inputs.make_batch([1024] * 64, 32, 8, seed=52)
    _, o0, l0, i0 = run(lib0, bq)
    pdattn._lib = None
    pdattn.LIB_PATH = sys.argv[2]
    assert pdattn.lib().pdattn_timeline_reset_decode() == 0   # (no stamps left from the case above)
    L, o1, l1, i1 = run(sys.argv[2], bq)
    assert np.array_equal(o0, o1) and np.array_equal(l0, l1), "timeline build changed the paired results"
    assert i0.paired == i1.paired
    if i1.paired:
        # (a new handle: its functions need their argument types again, or the pointer is cut to an int)
        L.pdattn_timeline_read_decode.argtypes = [ctypes.c_void_p, ctypes.c_size_t]
        assert L.pdattn_timeline_read_decode(buf.ctypes.data, buf.nbytes) == 0
        t = buf.reshape(8192, 32)[:i1.workgroups // 2].astype(np.int64)
        ran = t[:, 0] > 0
        assert ran.sum() > 0
        for row in t[ran]:
            seq = [row[0], row[1], row[2]] + [row[s] for s in range(4, 28) if row[s] > 0] + [row[31]]
            assert all(b >= a for a, b in zip(seq, seq[1:])), f"paired stamps out of order: {seq}"
        print("ok", int(ran.sum()), "paired workgroups stamped", flush=True)

    # the fused cascade step (decode role and prefix role in one launch, both stamped) and the
    # merge after it
    print("[case] fused cascade step, timeline build vs library, prefix 1024 + 40 x 77", flush=True)
    bc = inputs.make_shared_prefix_batch(1024, [77] * 40, 32, 8, seed=13)
    res = []
    for path in (lib0, sys.argv[2]):
        pdattn._lib = None
        pdattn.LIB_PATH = path
        pdattn.lib()
        o, l, ci = _gpu.run_cascade(_gpu.DeviceBatch(bc), min_prefix=16)
        assert ci.use == 1 and ci.mode == pdattn.CASCADE_FUSED, (ci.use, ci.mode)
        res.append((o, l))
    assert np.array_equal(res[0][0], res[1][0]) and np.array_equal(res[0][1], res[1][1]), \
        "timeline build changed the fused cascade step's results"

    # the prefix kernel alone, with a partial last chunk: 12 rows per kv head (the 4-wave body;
    # 640 keys in chunks of 96: 6 full + 64), and 192 rows (the key-split body, two query groups;
    # 992 keys in chunks of 160: 6 full + 32, three blocks split 2 + 1 between the wave groups)
    for Lpre, seqs, ct, nch, qg, tag in ((640, [3, 20, 50], 96, 7, 1, "4-wave"),
                                        (992, [16] * 48, 160, 7, 2, "key-split")):
        print(f"[case] prefix kernel ({tag}), timeline build vs library, {Lpre} keys in chunks of {ct}",
              flush=True)
        bp = inputs.make_shared_prefix_batch(Lpre, seqs, 32, 8, seed=8)
        rows = bp.B * bp.Hq
        res = []
        for path in (lib0, sys.argv[2]):
            pdattn._lib = None
            pdattn.LIB_PATH = path
            Lp = pdattn.lib()
            if path != lib0:
                assert Lp.pdattn_timeline_reset_prefix() == 0
            db = _gpu.DeviceBatch(bp)
            po = torch.full((rows, nch, 128), float("nan"), dtype=torch.float32, device="cuda:0")
            pl = torch.full((rows, nch), float("nan"), dtype=torch.float32, device="cuda:0")
            pp = pdattn.PrefixParams()
            pp.q, pp.k_cache, pp.v_cache = db.q.data_ptr(), db.k.data_ptr(), db.v.data_ptr()
            pp.prefix_pages = db.indices.data_ptr()
            pp.part_o, pp.part_lse = po.data_ptr(), pl.data_ptr()
            pp.B, pp.Hq, pp.Hkv = bp.B, bp.Hq, bp.Hkv
            pp.prefix_len, pp.chunk_tokens, pp.part_stride = Lpre, ct, nch
            pp.sm_scale = 1.0 / np.sqrt(128)
            pdattn.cascade_prefix(pp)
            torch.cuda.synchronize()
            res.append((po.cpu().numpy(), pl.cpu().numpy()))
        assert np.array_equal(res[0][0].view(np.int32), res[1][0].view(np.int32)) and \
            np.array_equal(res[0][1].view(np.int32), res[1][1].view(np.int32)), \
            f"timeline build changed the prefix kernel's partials ({tag})"
        Lp.pdattn_timeline_read_prefix.argtypes = [ctypes.c_void_p, ctypes.c_size_t]
        buf = np.zeros(8192 * 32, np.uint64)
        assert Lp.pdattn_timeline_read_prefix(buf.ctypes.data, buf.nbytes) == 0
        nwg = nch * qg * bp.Hkv          # grid (chunks, query groups, kv heads)
        t = buf.reshape(8192, 32)[:nwg].astype(np.int64)
        assert (t[:, 0] > 0).all(), f"a prefix workgroup left no stamps ({tag})"
        for row in t:
            seq = [row[0], row[1], row[2]] + [row[s] for s in range(3, 27) if row[s] > 0] + [row[29], row[30]]
            assert all(b >= a for a, b in zip(seq, seq[1:])), f"prefix stamps out of order ({tag}): {seq}"
        print("ok prefix", tag, nwg, "workgroups stamped", flush=True)
""")


@pytest.mark.skipif(not os.path.exists(TL_LIB), reason="timeline build absent (make -C cuda-kernel-lab_amd timeline)")
def test_timeline_build_matches_library_and_stamps_in_order():
    r = subprocess.run([sys.executable, "-c", CHILD, ROOT, TL_LIB], capture_output=True, text=True,
                       timeout=110)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    assert "ok prefix 4-wave" in r.stdout and "ok prefix key-split" in r.stdout
