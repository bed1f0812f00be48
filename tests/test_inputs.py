"""Synthetic batch builders (restating Batch / make_shared_prefix_batch,
01_decode_attention.cu:333-368, 714-742) -- CPU only."""
import numpy as np

from pdattn import inputs


def test_batch_page_table():
    bt = inputs.make_batch([1, 16, 17, 0, 4097], 8, 2, seed=5)
    assert list(bt.indptr) == [0, 1, 2, 4, 4, 261]
    assert list(bt.last) == [1, 16, 1, 0, 1]
    assert sorted(bt.indices) == list(range(bt.num_pages))       # a permutation of the pages
    assert bt.k.shape == (261, 16, 2, 128) and bt.q.shape == (5, 8, 128)
    again = inputs.make_batch([1, 16, 17, 0, 4097], 8, 2, seed=5)
    assert np.array_equal(bt.indices, again.indices) and np.array_equal(bt.k, again.k)


def test_shared_prefix_batch():
    bt = inputs.make_shared_prefix_batch(64, [1, 17, 40], 8, 8, seed=13)
    pp = 4
    first = bt.indices[:pp]
    for b in range(bt.B):
        assert np.array_equal(bt.indices[bt.indptr[b]:bt.indptr[b] + pp], first)
    private = np.concatenate([bt.indices[bt.indptr[b] + pp:bt.indptr[b + 1]] for b in range(bt.B)])
    assert len(set(private)) == len(private) and not set(private) & set(first)
    assert bt.num_pages == pp + len(private)
    assert bt.lens == [65, 81, 104]


def test_algorithmic_bytes_formula():
    bt = inputs.make_batch([32768], 32, 8, seed=11, fill=False)
    assert bt.algorithmic_bytes() == 134_242_444           # the figure quoted for 1 x 32K
    bt = inputs.make_batch([1024] * 64, 32, 8, seed=11, fill=False)
    assert bt.algorithmic_bytes() == 269_509_124


def test_ragged_lengths_are_seeded():
    a = inputs.ragged_lens(64, 256, 4096, 11)
    assert a == inputs.ragged_lens(64, 256, 4096, 11)
    assert min(a) >= 256 and max(a) <= 4096


def test_prefix_tree_batch():
    """Node pages are shared exactly along each sequence's path; private pages are its own."""
    groups = [((0,), 32), ((0, 1), 48), ((0, 2), 16)]
    seqs = [((0, 1), 5), ((0, 1), 16), ((0, 2), 1), ((0,), 20)]
    bt = inputs.make_prefix_tree_batch(groups, seqs, 8, 2, seed=7, fill=False)
    assert bt.lens == [85, 96, 49, 52]
    rows = [bt.indices[bt.indptr[b]:bt.indptr[b + 1]].tolist() for b in range(bt.B)]
    root = rows[0][:2]
    assert all(r[:2] == root for r in rows)
    assert rows[0][2:5] == rows[1][2:5]                     # node (0, 1)
    assert rows[2][2] not in rows[0] and rows[3][2] not in rows[0] + rows[2]
    flat = sorted(bt.indices.tolist())
    assert sorted(set(flat)) == list(range(bt.num_pages))   # every page used, ids in range
    # each page is used by one sequence, or by the members of the one node that owns it
    assert bt.num_pages == 2 + 3 + 1 + (1 + 1 + 1 + 2)


def test_unique_bytes():
    """Shared pages count once; without sharing it equals the per-sequence algorithmic bytes."""
    bt = inputs.make_shared_prefix_batch(64, [1, 17, 40], 8, 8, seed=13, fill=False)
    tokens = 64 + 1 + 17 + 40
    table = 4 * (2 * bt.B + 1 + int(bt.indptr[-1]))
    assert inputs.unique_bytes(bt) == tokens * 8 * 512 + 2 * bt.B * 8 * 256 + bt.B * 8 * 4 + table
    assert bt.algorithmic_bytes() - inputs.unique_bytes(bt) == 2 * 64 * 8 * 512   # two extra reads
    plain = inputs.make_batch([5, 300, 17], 8, 2, seed=3, fill=False)
    assert inputs.unique_bytes(plain) == plain.algorithmic_bytes()
