"""Seeded random shared-prefix forests through the cascade path, single-level and tree planners,
against the fp64 oracle.

Each seed draws a forest (depth up to 3, up to 3 children per node, node lengths whole pages from
16 to 512 tokens) and hangs 0-4 sequences on every node with 0-200 private tokens (so a sequence
may end exactly where its node does, and the planners then keep its last page private). Even
seeds: one root shared by the whole batch. Odd seeds: one or two roots and a few sequences that
share nothing (one of them possibly empty). The head counts and min_prefix are drawn too. Whatever the planners detect, the output must be the oracle's attention
over each sequence's full page list (the reference's cascade semantics, 01_decode_attention.cu:656-712,
generalised to a tree where the reference lists it as not done, README.md:73).
"""
import numpy as np
import pytest

import oracle
from _checks import check_lse, check_out
from pdattn import inputs

pytestmark = pytest.mark.gpu

HEADS = [(32, 8), (16, 2), (8, 8), (64, 8), (32, 4)]


def _forest(rng, one_root):
    """one_root: a single tree and no unshared sequence, so that the whole batch shares the root
    (the single-level planner's case)."""
    nodes, leaves = [], []

    def grow(path, depth):
        nodes.append((path, 16 * int(rng.integers(1, 33))))
        leaves.append(path)
        if depth < 3:
            for c in range(int(rng.integers(0, 4))):
                grow(path + (len(nodes) + c,), depth + 1)

    for r in range(1 if one_root else int(rng.integers(1, 3))):
        grow((100 * r,), 1)
    seqs = []
    for path in leaves:
        for _ in range(int(rng.integers(0 if len(leaves) > 1 else 2, 5))):
            seqs.append((path, int(rng.integers(0, 201))))
    if one_root:
        while len(seqs) < 2:
            seqs.append((leaves[0], int(rng.integers(1, 201))))
    else:
        for _ in range(int(rng.integers(1, 4))):
            seqs.append(((), int(rng.integers(0, 300))))
    order = rng.permutation(len(seqs))
    return nodes, [seqs[i] for i in order]


@pytest.mark.parametrize("seed", range(10))
def test_random_forest_cascade_matches_oracle(seed):
    import _gpu
    rng = np.random.default_rng(7000 + seed)
    nodes, seqs = _forest(rng, one_root=seed % 2 == 0)
    Hq, Hkv = HEADS[int(rng.integers(0, len(HEADS)))]
    min_prefix = int(rng.choice([16, 48, 256]))
    print(f"[case] random forest seed={seed}: {len(nodes)} nodes, {len(seqs)} sequences, Hq={Hq} "
          f"Hkv={Hkv} min_prefix={min_prefix}", flush=True)
    bt = inputs.make_prefix_tree_batch(nodes, seqs, Hq, Hkv, seed=seed)
    ro, rl = oracle.decode(bt.q, bt.k, bt.v, bt.indptr, bt.indices, bt.last, Hq, Hkv, threads=8)
    db = _gpu.DeviceBatch(bt)
    for tree in (False, True):
        o, l, info = _gpu.run_cascade(db, min_prefix=min_prefix, tree=tree)
        tag = f"seed={seed} tree={tree} use={info.use} nodes={info.nodes} levels={info.levels}"
        print(f"[case] {tag}", flush=True)
        check_out(o, ro, tag=tag)
        check_lse(l, rl, tag=tag)
