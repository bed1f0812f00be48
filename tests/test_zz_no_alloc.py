"""pdattn_decode_attention_noalloc (partial states in the library's own device array, no
allocation) against pdattn_decode_attention (partial states in a workspace), through the C ABI.

Two calls in a row, the second with a smaller batch than the first, so the second finds the
first one's partial states in the array: each call's out / lse must equal what
pdattn_decode_attention gives for the same input (bitwise: the same kernels on the same chunking)
and match the fp64 oracle within the parity bar.
"""
import numpy as np
import pytest

import oracle
from _checks import check_lse, check_out
from pdattn import inputs

pytestmark = pytest.mark.gpu

CALLS = [
    ([5, 300, 2049, 4096, 17, 1000], 32, 8, 7, "6 sequences, 7 chunks"),
    ([100, 33], 32, 8, 3, "2 sequences, 3 chunks"),
]


def _with_workspace(db, G, nc, ct):
    import pdattn
    ws = pdattn.Workspace()
    try:
        pdattn.decode_attention(db.params(nc, ct), G, db.out, db.lse, ws)
        return db.results()
    finally:
        pdattn.workspace_release(ws)


def test_noalloc_matches_decode_attention_twice():
    import torch
    import _gpu
    import pdattn
    prepared = []
    for lens, Hq, Hkv, force, tag in CALLS:
        bt = inputs.make_batch(lens, Hq, Hkv, seed=51)
        db = _gpu.DeviceBatch(bt)
        nc, ct = pdattn.plan_chunks(bt.G, bt.B, bt.Hkv, bt.max_len, force)
        assert nc > 1
        print(f"[case] workspace entry point: {tag} (chunks {nc})", flush=True)
        prepared.append((bt, db, nc, ct, tag, _with_workspace(db, bt.G, nc, ct)))
    for bt, db, nc, ct, tag, (wo, wl) in prepared:
        print(f"[case] no-allocation entry point: {tag} (chunks {nc})", flush=True)
        db.out.fill_(float("nan"))
        db.lse.fill_(float("nan"))
        torch.cuda.synchronize()
        pdattn.decode_attention_noalloc(db.params(nc, ct), bt.G, db.out, db.lse)
        o, l = db.results()
        assert np.array_equal(o, wo), f"{tag}: out differs from pdattn_decode_attention"
        assert np.array_equal(l, wl), f"{tag}: lse differs from pdattn_decode_attention"
        ro, rl = oracle.decode(bt.q, bt.k, bt.v, bt.indptr, bt.indices, bt.last, bt.Hq, bt.Hkv, threads=8)
        check_out(o, ro, tag=f"no-allocation {tag}")
        check_lse(l, rl, tag=f"no-allocation {tag}")


def test_noalloc_single_chunk_and_empty():
    """One chunk per sequence (no partial states), and an empty sequence in a split batch."""
    import _gpu
    import pdattn
    for lens, force in (([1024] * 8, 1), ([0, 700, 0, 33], 4)):
        bt = inputs.make_batch(lens, 32, 8, seed=52)
        db = _gpu.DeviceBatch(bt)
        nc, ct = pdattn.plan_chunks(bt.G, bt.B, bt.Hkv, bt.max_len, force)
        print(f"[case] no-allocation entry point: lens {lens} chunks {nc}", flush=True)
        wo, wl = _with_workspace(db, bt.G, nc, ct)
        pdattn.decode_attention_noalloc(db.params(nc, ct), bt.G, db.out, db.lse)
        o, l = db.results()
        assert np.array_equal(o, wo) and np.array_equal(l, wl)
