"""The balanced (stream-K) planner -- CPU only.

Plans are built with a forced grid size (no device query). Their reported structure is checked
against a brute-force restatement of the partition contract in pdattn.h: workgroup w owns the
kv-head-major page units [U w / W, U (w+1) / W), and a (sequence, kv head) pair is split when
its units fall into more than one workgroup.
"""
import numpy as np
import pytest

import pdattn
from pdattn import inputs


def brute_contributors(indptr, Hkv, W):
    nnz = int(indptr[-1] - indptr[0])
    U = Hkv * nnz
    owner = [0] * U
    for w in range(W):
        for u in range(U * w // W, U * (w + 1) // W):
            owner[u] = w
    split, mx = 0, 1
    for kvh in range(Hkv):
        for b in range(len(indptr) - 1):
            pb, pe = indptr[b] - indptr[0], indptr[b + 1] - indptr[0]
            if pe == pb:
                continue
            ws = {owner[kvh * nnz + j] for j in range(pb, pe)}
            if len(ws) > 1:
                split += 1
            mx = max(mx, len(ws))
    return U, split, mx


CASES = [
    ([32768], 8),
    ([1024] * 64, 8),
    ([8192] * 8, 8),
    ([5, 300, 2049, 4096], 8),
    ([1, 17, 1000], 8),
    ([16, 32, 48, 4097], 2),
    ([0, 5, 0, 100], 2),
]


@pytest.mark.parametrize("lens,Hkv", CASES, ids=[f"{len(c[0])}seq" for c in CASES])
@pytest.mark.parametrize("W", [1, 3, 7, 64, 256, 1000])
def test_partition_matches_contract(lens, Hkv, W):
    bt = inputs.make_batch(lens, Hkv * 4, Hkv, seed=1, fill=False)
    if bt.indptr[-1] == 0:
        pytest.skip("no pages")
    plan = pdattn.Plan(bt.indptr, bt.last, bt.B, Hkv * 4, Hkv, force_workgroups=W)
    info = plan.info()
    U, split, mx = brute_contributors(bt.indptr, Hkv, info.workgroups)
    assert info.units == U
    assert 1 <= info.workgroups <= U
    assert info.workgroups >= min(W, U)          # grows only to respect per-workgroup limits
    assert info.split_pairs == split and info.max_contributors == mx
    assert info.pairs == bt.B * Hkv
    slots = bt.B * Hkv + info.workgroups
    assert info.workspace_bytes >= slots * 4 * 129 * 4


def test_many_tiny_sequences_grow_the_grid():
    """More sequences per workgroup than descriptor slots: the planner doubles the grid."""
    lens = [16] * 4096
    bt = inputs.make_batch(lens, 32, 8, seed=2, fill=False)
    plan = pdattn.Plan(bt.indptr, bt.last, bt.B, 32, 8, force_workgroups=256)
    assert plan.info().workgroups > 256


def test_all_empty_batch():
    plan = pdattn.Plan([0, 0, 0], [0, 0], 2, 8, 2, force_workgroups=5)
    info = plan.info()
    assert info.units == 0 and info.split_pairs == 0
