"""GPU parity at the plan path's limits, through the C ABI, against the fp64 oracle.

* A workgroup's page list at its maximum (2048 page ids staged in LDS), and a range that would
  exceed it (the planner doubles the number of ranges).
* Thousands of tiny sequences: ranges hold up to 24 segments (the descriptor block's limit) and
  the planner grows the grid past one workgroup per CU.
* The same batches through the reference-shaped uniform split.
"""
import numpy as np
import pytest

import oracle
import pdattn
from _checks import check_lse, check_out
from pdattn import inputs

pytestmark = pytest.mark.gpu


def _ref(bt):
    return oracle.decode(bt.q, bt.k, bt.v, bt.indptr, bt.indices, bt.last, bt.Hq, bt.Hkv, threads=8)


@pytest.mark.parametrize("lens,wg,pages_per_range", [
    ([4096 * 16], 16, 2048),          # 2 ranges of exactly 2048 pages
    ([40000, 40000], 8, 1250),        # 5000 pages: 1 range -> 2 (2500) -> 4 (1250)
], ids=["range_at_2048_pages", "range_past_2048_doubles"])
def test_full_page_lists(lens, wg, pages_per_range):
    import _gpu
    print(f"[case] full page lists lens={lens} W={wg}", flush=True)
    bt = inputs.make_batch(lens, 32, 8, seed=61)
    ro, rl = _ref(bt)
    db = _gpu.DeviceBatch(bt)
    o, l, info = _gpu.run_plan(db, wg)
    assert info.chunk_pages == pages_per_range
    segs, _ = pdattn.Plan(bt.indptr, bt.last, bt.B, 32, 8, force_workgroups=wg).schedule()
    assert max(sum(s[3] for s in ss) for ss in segs) == pages_per_range
    check_out(o, ro, tag=f"full page lists W={info.workgroups}")
    check_lse(l, rl, tag=f"full page lists W={info.workgroups}")


def test_many_tiny_sequences():
    import _gpu
    rng = np.random.default_rng(62)
    lens = [int(x) for x in rng.integers(1, 49, size=2500)]
    lens[7] = 0
    print(f"[case] {len(lens)} tiny sequences", flush=True)
    bt = inputs.make_batch(lens, 32, 8, seed=63)
    ro, rl = _ref(bt)
    db = _gpu.DeviceBatch(bt)
    o, l, info = _gpu.run_plan(db)
    segs, _ = pdattn.Plan(bt.indptr, bt.last, bt.B, 32, 8).schedule()
    most = max(len(ss) for ss in segs)
    assert info.workgroups > pdattn.device_info().compute_units   # the grid grew
    assert 12 < most <= pdattn.SCHEDULE_SEGMENTS
    check_out(o, ro, tag=f"tiny sequences plan W={info.workgroups} segs<={most}")
    check_lse(l, rl, tag="tiny sequences plan")
    o, l, nc = _gpu.run_uniform(db)
    check_out(o, ro, tag=f"tiny sequences uniform chunks={nc}")
    check_lse(l, rl, tag="tiny sequences uniform")
