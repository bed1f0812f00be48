"""GPU parity at kv-head counts past the benchmark's 8: Hkv = 16 and 32 (token rows of 4 KB and
8 KB, pages of 64 KB and 128 KB), for every decode path and the cascade, against the fp64 oracle.

The kernels index a page as Hkv 256-byte rows per token and the planners cut the grid into
Hkv-wide groups of workgroups (01_decode_attention.cu:112 is the layout); these cases check both at
head counts the BASELINE configurations do not reach: MHA with 32 kv heads (G = 1), and G = 4 and 8
over 16 kv heads. Lengths include an empty sequence, a one-page sequence and partial last pages.
"""
import pytest

import oracle
from _checks import check_lse, check_out
from pdattn import inputs

pytestmark = pytest.mark.gpu

HEADS = [(32, 32), (16, 16), (64, 16), (128, 16)]
IDS = [f"Hq{hq}-Hkv{hkv}" for hq, hkv in HEADS]
LENS = [1000, 77, 2049, 0, 16]


def _ref(bt, kv_start=0):
    return oracle.decode(bt.q, bt.k, bt.v, bt.indptr, bt.indices, bt.last, bt.Hq, bt.Hkv,
                         kv_start=kv_start, threads=8)


@pytest.mark.parametrize("Hq,Hkv", HEADS, ids=IDS)
def test_decode_paths_wide_heads(Hq, Hkv):
    """Plan/run (page ranges, and a forced grid that is not a multiple of Hkv: the chunk
    partition), the uniform split and the device-range drop-in, each against the oracle."""
    import _gpu
    print(f"[case] wide heads Hq={Hq} Hkv={Hkv} lens={LENS} seed=31", flush=True)
    bt = inputs.make_batch(LENS, Hq, Hkv, seed=31)
    db = _gpu.DeviceBatch(bt)
    ro, rl = _ref(bt)
    for wg in (0, 37):
        o, l, info = _gpu.run_plan(db, wg)
        check_out(o, ro, tag=f"plan Hq={Hq} Hkv={Hkv} W={info.workgroups}")
        check_lse(l, rl, tag=f"plan Hq={Hq} Hkv={Hkv} W={info.workgroups}")
    for force in (0, 3):
        o, l, nc = _gpu.run_uniform(db, force)
        check_out(o, ro, tag=f"uniform Hq={Hq} Hkv={Hkv} chunks={nc}")
        check_lse(l, rl, tag=f"uniform Hq={Hq} Hkv={Hkv} chunks={nc}")
    o, l = _gpu.run_balanced(db)
    check_out(o, ro, tag=f"device ranges Hq={Hq} Hkv={Hkv}")
    check_lse(l, rl, tag=f"device ranges Hq={Hq} Hkv={Hkv}")


@pytest.mark.parametrize("Hq,Hkv", HEADS, ids=IDS)
def test_cascade_wide_heads(Hq, Hkv):
    """The cascade (detected 512-token shared prefix on fp16 MFMA, suffix decode, merge)."""
    import _gpu
    print(f"[case] wide-head cascade Hq={Hq} Hkv={Hkv} prefix 512 + [5, 40, 17] seed=33", flush=True)
    bt = inputs.make_shared_prefix_batch(512, [5, 40, 17], Hq, Hkv, seed=33)
    assert oracle.shared_prefix_pages(bt.indptr, bt.indices) * 16 == 512
    ro, rl = _ref(bt)
    o, l, info = _gpu.run_cascade(_gpu.DeviceBatch(bt), min_prefix=16)
    assert info.use == 1
    check_out(o, ro, tag=f"cascade Hq={Hq} Hkv={Hkv}")
    check_lse(l, rl, tag=f"cascade Hq={Hq} Hkv={Hkv}")
