"""The balanced planner -- CPU only.

Plans are built with a forced grid size (no device query). The schedule each plan exports is
checked against a brute-force restatement of the partition contract in pdattn.h:
  * chunks of up to P pages of one (sequence, kv head) pair, ordered sequence-major, then by chunk
    position, with the kv head varying fastest; one unit per page of a chunk;
  * workgroup w owns the units [U w / W, U (w+1) / W); its segments are the pieces of chunks in
    its range, in order;
  * a pair with more than one segment gets consecutive partial slots, its k-th segment (in unit
    order) writing slot slot0 + k, and one merge-list entry; a pair with one segment writes the
    final output (slot -1); an empty sequence gets a merge entry with no slots;
  * the slots are then laid out by merge entry (entry e's k-th slot is e * cmax + k, cmax = the
    most slots of an entry) unless that takes more than twice the packed slots plus 64, and the
    merge list's header says which {tag, entries, cmax or 0, 0}.
"""
import numpy as np
import pytest

import pdattn
from pdattn import inputs


def brute_schedule(indptr, last, Hkv, W, P):
    B = len(indptr) - 1
    jbase = int(indptr[0])
    units = []                          # (b, kvh, page index within the sequence)
    for b in range(B):
        np_ = int(indptr[b + 1] - indptr[b])
        for pa in range(0, np_, P):
            for kvh in range(Hkv):
                for i in range(pa, min(np_, pa + P)):
                    units.append((b, kvh, i, pa))
    U = len(units)
    segs = []
    for w in range(W):
        u0, u1 = U * w // W, U * (w + 1) // W
        out = []
        for u in range(u0, u1):
            b, kvh, i, pa = units[u]
            if out and out[-1][0] == b and out[-1][1] == kvh and out[-1][-1] == pa:
                out[-1][3] += 1
            else:
                out.append([b, kvh, u - u0, 1, pa])
        full = []
        for b, kvh, qa, npg, pa in out:
            first = units[u0 + qa][2]
            np_ = int(indptr[b + 1] - indptr[b])
            seq_len = (np_ - 1) * 16 + int(last[b])
            t1 = seq_len if first + npg == np_ else (first + npg) * 16
            full.append([b, kvh, qa, npg, first * 16, t1, int(indptr[b]) - jbase + first, -1])
        segs.append(full)
    # contributors per pair, in unit (= workgroup, segment) order
    contrib = {}
    for w, ss in enumerate(segs):
        for k, sg in enumerate(ss):
            contrib.setdefault((sg[0], sg[1]), []).append((w, k))
    merge, slot = [], 0
    for b in range(B):
        for kvh in range(Hkv):
            cs = contrib.get((b, kvh), [])
            if len(cs) > 1:
                for k, (w, i) in enumerate(cs):
                    segs[w][i][7] = slot + k
                merge.append([b, kvh, slot, len(cs)])
                slot += len(cs)
            elif not cs:
                merge.append([b, kvh, 0, 0])
    split = sum(1 for cs in contrib.values() if len(cs) > 1)
    mx = max([len(cs) for cs in contrib.values()] + [1])
    return U, segs, merge, split, mx


def entry_layout(segs, merge):
    """The slots of a packed schedule moved to the layout by merge entry, where that costs at most
    twice the packed slots plus 64: entry e's k-th slot becomes e * cmax + k. Returns cmax (0: the
    packed layout is kept)."""
    packed = sum(m[3] for m in merge)
    cmax = max([m[3] for m in merge] + [0])
    if cmax == 0 or len(merge) * cmax > 2 * packed + 64:
        return 0
    remap = {}
    for e, m in enumerate(merge):
        for k in range(m[3]):
            remap[m[2] + k] = e * cmax + k
        m[2] = e * cmax
    for ss in segs:
        for sg in ss:
            if sg[7] >= 0:
                sg[7] = remap[sg[7]]
    return cmax


def check_header(plan, merge, cmax):
    _, _, hd = plan.schedule(with_header=True)
    assert hd[0] != 0 and hd[0] < 0          # the plan's tag (high bit set)
    assert hd[1:] == [len(merge), cmax, 0]


CASES = [
    ([32768], 8),
    ([1024] * 64, 8),
    ([8192] * 8, 8),
    ([5, 300, 2049, 4096], 8),
    ([1, 17, 1000], 8),
    ([16, 32, 48, 4097], 2),
    ([0, 5, 0, 100], 2),
]


@pytest.mark.parametrize("lens,Hkv", CASES, ids=[f"{len(c[0])}seq-{c[1]}kv" for c in CASES])
@pytest.mark.parametrize("W,P", [(1, 16), (3, 16), (7, 5), (64, 16), (256, 16), (256, 8), (1000, 16)])
def test_schedule_matches_contract(lens, Hkv, W, P):
    bt = inputs.make_batch(lens, Hkv * 4, Hkv, seed=1, fill=False)
    if bt.indptr[-1] == 0:
        pytest.skip("no pages")
    plan = pdattn.Plan(bt.indptr, bt.last, bt.B, Hkv * 4, Hkv, force_workgroups=W, chunk_pages=P)
    info = plan.info()
    assert info.chunk_pages == P
    Wp = info.workgroups
    assert Wp >= min(W, info.units)              # grows only to respect per-workgroup limits
    U, segs, merge, split, mx = brute_schedule(bt.indptr, bt.last, Hkv, Wp, P)
    slots = sum(m[3] for m in merge)
    cmax = entry_layout(segs, merge)
    got_segs, got_merge = plan.schedule()
    assert info.units == U
    assert got_segs == segs
    assert got_merge.tolist() == merge
    check_header(plan, merge, cmax)
    assert info.split_pairs == split and info.max_contributors == mx
    assert info.pairs == bt.B * Hkv
    assert info.segments == sum(len(s) for s in segs)
    assert info.merge_entries == len(merge)
    assert info.workspace_bytes >= max(slots, len(merge) * cmax) * 4 * 129 * 4
    # every (page, kv head) unit exactly once
    seen = set()
    for ss in got_segs:
        assert len(ss) <= pdattn.SCHEDULE_SEGMENTS
        for b, kvh, qa, npg, t0, t1, jpos, slot in ss:
            for i in range(npg):
                key = (kvh, jpos + i)
                assert key not in seen
                seen.add(key)
    assert len(seen) == U


def brute_grouped(indptr, last, Hkv, W):
    """The page-range partition (chunk_pages = 0): the nnz pages, in page-table order, are cut into
    NG = W / Hkv ranges [nnz g / NG, nnz (g+1) / NG); workgroup g Hkv + h takes range g for kv
    head h, one segment per sequence piece in the range."""
    B = len(indptr) - 1
    jbase = int(indptr[0])
    nnz = int(indptr[-1]) - jbase
    NG = W // Hkv
    segs = [[] for _ in range(W)]
    for g in range(NG):
        lo, hi = nnz * g // NG, nnz * (g + 1) // NG
        for b in range(B):
            start, end = int(indptr[b]) - jbase, int(indptr[b + 1]) - jbase
            s0, s1 = max(lo, start), min(hi, end)
            if s1 <= s0:
                continue
            p0, p1, np_ = s0 - start, s1 - start, end - start
            t1 = (np_ - 1) * 16 + int(last[b]) if p1 == np_ else p1 * 16
            for kvh in range(Hkv):
                segs[g * Hkv + kvh].append([b, kvh, s0 - lo, p1 - p0, p0 * 16, t1, s0, -1])
    contrib = {}
    for w, ss in enumerate(segs):
        for k, sg in enumerate(ss):
            contrib.setdefault((sg[0], sg[1]), []).append((w, k))
    merge, slot = [], 0
    for b in range(B):
        for kvh in range(Hkv):
            cs = contrib.get((b, kvh), [])
            if len(cs) > 1:
                for k, (w, i) in enumerate(cs):
                    segs[w][i][7] = slot + k
                merge.append([b, kvh, slot, len(cs)])
                slot += len(cs)
            elif not cs:
                merge.append([b, kvh, 0, 0])
    return segs, merge


@pytest.mark.parametrize("lens,Hkv", CASES, ids=[f"{len(c[0])}seq-{c[1]}kv" for c in CASES])
@pytest.mark.parametrize("W", [8, 64, 256, 512, 1000])
def test_grouped_schedule_matches_contract(lens, Hkv, W):
    """The default partition: every page of every kv head exactly once, and the Hkv workgroups of a
    group hold the same page ranges (they stream whole token rows together)."""
    bt = inputs.make_batch(lens, Hkv * 4, Hkv, seed=1, fill=False)
    if bt.indptr[-1] == 0:
        pytest.skip("no pages")
    if W % Hkv:
        pytest.skip("grid not a multiple of Hkv")
    plan = pdattn.Plan(bt.indptr, bt.last, bt.B, Hkv * 4, Hkv, force_workgroups=W)
    info = plan.info()
    Wp = info.workgroups
    assert Wp % Hkv == 0
    segs, merge = brute_grouped(bt.indptr, bt.last, Hkv, Wp)
    cmax = entry_layout(segs, merge)
    got_segs, got_merge = plan.schedule()
    assert got_segs == segs
    assert got_merge.tolist() == merge
    check_header(plan, merge, cmax)
    for g in range(Wp // Hkv):
        ranges = [[(s[0], s[2], s[3], s[6]) for s in got_segs[g * Hkv + h]] for h in range(Hkv)]
        assert all(r == ranges[0] for r in ranges)
        assert all(s[1] == h for h in range(Hkv) for s in got_segs[g * Hkv + h])
        assert len(got_segs[g * Hkv]) <= pdattn.SCHEDULE_SEGMENTS
    seen = set()
    for ss in got_segs:
        for b, kvh, qa, npg, t0, t1, jpos, slot in ss:
            for i in range(npg):
                assert (kvh, jpos + i) not in seen
                seen.add((kvh, jpos + i))
    assert len(seen) == info.units


def test_every_workgroup_mixes_kv_heads():
    """One long sequence: every workgroup's range covers several kv heads (the order's purpose)."""
    bt = inputs.make_batch([32768], 32, 8, seed=1, fill=False)
    plan = pdattn.Plan(bt.indptr, bt.last, bt.B, 32, 8, force_workgroups=256, chunk_pages=16)
    segs, _ = plan.schedule()
    assert all(len({s[1] for s in ss}) >= 4 for ss in segs)


def test_many_tiny_sequences_grow_the_grid():
    """More segments per workgroup than descriptor slots: the planner doubles the grid."""
    lens = [16] * 4096
    bt = inputs.make_batch(lens, 32, 8, seed=2, fill=False)
    plan = pdattn.Plan(bt.indptr, bt.last, bt.B, 32, 8, force_workgroups=256)
    assert plan.info().workgroups > 256


def test_all_empty_batch():
    plan = pdattn.Plan([0, 0, 0], [0, 0], 2, 8, 2, force_workgroups=5)
    info = plan.info()
    assert info.units == 0 and info.split_pairs == 0
    _, merge = plan.schedule()
    assert merge.tolist() == [[0, 0, 0, 0], [0, 1, 0, 0], [1, 0, 0, 0], [1, 1, 0, 0]]


def test_rejects_bad_chunk_pages():
    bt = inputs.make_batch([100], 8, 2, seed=1, fill=False)
    with pytest.raises(pdattn.PdattnError):
        pdattn.Plan(bt.indptr, bt.last, bt.B, 8, 2, force_workgroups=4, chunk_pages=-1)
