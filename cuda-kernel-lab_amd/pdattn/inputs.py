"""Seeded synthetic decode batches: CSR page tables with shuffled physical pages, fp16 q/K/V.

Restates the reference's test-input builders (qilem/cuda-kernel-lab, 01_decode_attention.cu):
  * ``Batch``                     01:333-368  -- ``make_batch`` here
  * ``make_shared_prefix_batch``  01:714-742  -- ``make_shared_prefix_batch`` here
with numpy's PCG64 generator in place of ``std::mt19937``/``std::uniform_real_distribution``
(the reference's exact bytes come from MSVC's implementation-defined distributions and cannot be
regenerated). Values are N(0,1) by default, as the benchmark configurations ask; ``dist="uniform"``
gives the reference's U(-1, 1).

Layouts: q [B, Hq, 128]; K and V [num_pages, 16, Hkv, 128]; indptr [B+1], indices [nnz],
last_page_len [B] (int32). A sequence of length 0 has no pages and last_page_len 0.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

HEAD_DIM = 128
PAGE = 16


@dataclass
class Batch:
    lens: list
    Hq: int
    Hkv: int
    indptr: np.ndarray
    indices: np.ndarray
    last: np.ndarray
    num_pages: int
    seed: int
    q: np.ndarray | None = None   # float16 [B, Hq, 128]
    k: np.ndarray | None = None   # float16 [num_pages, 16, Hkv, 128]
    v: np.ndarray | None = None
    shared_prefix_tokens: int = 0
    meta: dict = field(default_factory=dict)

    @property
    def B(self) -> int:
        return len(self.lens)

    @property
    def G(self) -> int:
        return self.Hq // self.Hkv

    @property
    def max_len(self) -> int:
        return max(self.lens) if self.lens else 0

    def kv_elems(self) -> int:
        return self.num_pages * PAGE * self.Hkv * HEAD_DIM

    def algorithmic_bytes(self, kv_start: int = 0) -> int:
        """HBM bytes a decode step must move: K+V of the valid tokens, q, o, lse and the page
        table (int32 indptr, last_page_len, indices)."""
        tokens = sum(max(0, L - kv_start) for L in self.lens)
        kv = tokens * self.Hkv * HEAD_DIM * 2 * 2
        qo = 2 * self.B * self.Hq * HEAD_DIM * 2
        lse = self.B * self.Hq * 4
        table = 4 * (2 * self.B + 1 + int(self.indptr[-1]))
        return kv + qo + lse + table


def unique_bytes(bt) -> int:
    """HBM bytes a step must move when every physical page is read once, however many sequences
    share it (what a cascade can reach): the valid tokens of each distinct page, plus q, o, lse
    and the page table."""
    valid = {}
    for b in range(bt.B):
        pb, pe = int(bt.indptr[b]), int(bt.indptr[b + 1])
        for j in range(pb, pe):
            n = PAGE if j < pe - 1 else int(bt.last[b])
            pid = int(bt.indices[j])
            valid[pid] = max(valid.get(pid, 0), n)
    kv = sum(valid.values()) * bt.Hkv * HEAD_DIM * 2 * 2
    return kv + 2 * bt.B * bt.Hq * HEAD_DIM * 2 + bt.B * bt.Hq * 4 + 4 * (2 * bt.B + 1 + int(bt.indptr[-1]))


def page_table(lens, rng: np.random.Generator):
    """CSR page table for the given lengths with a random permutation of physical pages
    (01_decode_attention.cu:343-354)."""
    indptr = [0]
    last = []
    for L in lens:
        np_ = (L + PAGE - 1) // PAGE
        indptr.append(indptr[-1] + np_)
        last.append(L - (np_ - 1) * PAGE if np_ > 0 else 0)
    num_pages = indptr[-1]
    indices = rng.permutation(num_pages).astype(np.int32)
    return np.asarray(indptr, np.int32), indices, np.asarray(last, np.int32), num_pages


def _values(rng: np.random.Generator, n: int, dist: str) -> np.ndarray:
    if dist == "normal":
        x = rng.standard_normal(n, dtype=np.float32)
    elif dist == "uniform":
        x = rng.uniform(-1.0, 1.0, n).astype(np.float32)
    elif dist == "zeros":
        x = np.zeros(n, np.float32)
    else:
        raise ValueError(f"unknown dist {dist!r}")
    return x.astype(np.float16)


def _fill(bt: Batch, rng: np.random.Generator, dist: str):
    bt.q = _values(rng, bt.B * bt.Hq * HEAD_DIM, dist).reshape(bt.B, bt.Hq, HEAD_DIM)
    shape = (bt.num_pages, PAGE, bt.Hkv, HEAD_DIM)
    bt.k = _values(rng, bt.kv_elems(), dist).reshape(shape)
    bt.v = _values(rng, bt.kv_elems(), dist).reshape(shape)


def make_batch(lens, Hq: int, Hkv: int, seed: int, fill: bool = True, dist: str = "normal") -> Batch:
    """Batch of variable-length sequences whose pages are scattered randomly in the cache
    (01_decode_attention.cu:341-366)."""
    lens = [int(L) for L in lens]
    if any(L < 0 for L in lens):
        raise ValueError("negative sequence length")
    rng = np.random.Generator(np.random.PCG64(seed))
    indptr, indices, last, num_pages = page_table(lens, rng)
    bt = Batch(lens, Hq, Hkv, indptr, indices, last, num_pages, seed)
    if fill:
        _fill(bt, rng, dist)
    return bt


def make_shared_prefix_batch(Lp: int, suffix, Hq: int, Hkv: int, seed: int, fill: bool = True,
                             dist: str = "normal") -> Batch:
    """B sequences sharing the first Lp tokens (the same physical pages, as prefix caching
    produces) followed by private suffixes; all pages scattered randomly
    (01_decode_attention.cu:714-742). Lp must be a multiple of the page size."""
    if Lp % PAGE:
        raise ValueError("shared prefix must be whole pages")
    lens = [Lp + int(s) for s in suffix]
    rng = np.random.Generator(np.random.PCG64(seed))
    indptr = [0]
    last = []
    for L in lens:
        np_ = (L + PAGE - 1) // PAGE
        indptr.append(indptr[-1] + np_)
        last.append(L - (np_ - 1) * PAGE if np_ > 0 else 0)
    pp = Lp // PAGE
    total = pp + sum((indptr[b + 1] - indptr[b]) - pp for b in range(len(lens)))
    perm = rng.permutation(total).astype(np.int32)
    indices = np.empty(indptr[-1], np.int32)
    nxt = pp
    for b in range(len(lens)):
        for i in range(indptr[b + 1] - indptr[b]):
            if i < pp:
                indices[indptr[b] + i] = perm[i]
            else:
                indices[indptr[b] + i] = perm[nxt]
                nxt += 1
    bt = Batch(lens, Hq, Hkv, np.asarray(indptr, np.int32), indices, np.asarray(last, np.int32),
               total, seed, shared_prefix_tokens=Lp)
    if fill:
        _fill(bt, rng, dist)
    return bt


def make_prefix_tree_batch(groups, suffix, Hq: int, Hkv: int, seed: int, fill: bool = True,
                           dist: str = "normal") -> Batch:
    """Sequences that share prefixes in a tree, with the same physical pages where shared.

    groups: list of (path, tokens) for each tree node, path being the tuple of node ids from the
    root (e.g. [((0,), 2048), ((0, 1), 4096), ((0, 2), 4096)]: node 0 shared by all, then two
    sub-prefixes). suffix: list of (leaf path, private tokens) per sequence; a sequence's
    context is the concatenation of the nodes on its leaf path, then its private tokens. Node
    lengths must be whole pages; all pages are scattered randomly."""
    node_tokens = {tuple(path): int(t) for path, t in groups}
    if any(t % PAGE for t in node_tokens.values()):
        raise ValueError("shared nodes must be whole pages")
    rng = np.random.Generator(np.random.PCG64(seed))
    node_pages = {path: t // PAGE for path, t in node_tokens.items()}
    seqs = []
    for leaf, priv in suffix:
        leaf = tuple(leaf)
        chain = [leaf[:i + 1] for i in range(len(leaf))]
        seqs.append((chain, int(priv)))
    lens = [sum(node_tokens[c] for c in chain) + priv for chain, priv in seqs]
    total = sum(node_pages.values()) + sum((L + PAGE - 1) // PAGE - sum(node_pages[c] for c in chain)
                                         for (chain, _), L in zip(seqs, lens))
    perm = rng.permutation(total).astype(np.int32)
    nxt = 0
    node_ids = {}
    for path in sorted(node_pages):
        node_ids[path] = perm[nxt:nxt + node_pages[path]]
        nxt += node_pages[path]
    indptr, indices, last = [0], [], []
    for (chain, priv), L in zip(seqs, lens):
        np_ = (L + PAGE - 1) // PAGE
        ids = [int(x) for c in chain for x in node_ids[c]]
        while len(ids) < np_:
            ids.append(int(perm[nxt]))
            nxt += 1
        indices += ids
        indptr.append(indptr[-1] + np_)
        last.append(L - (np_ - 1) * PAGE if np_ > 0 else 0)
    bt = Batch(lens, Hq, Hkv, np.asarray(indptr, np.int32), np.asarray(indices, np.int32),
               np.asarray(last, np.int32), total, seed)
    if fill:
        _fill(bt, rng, dist)
    return bt


def ragged_lens(B: int, lo: int, hi: int, seed: int):
    """Lengths uniform in [lo, hi] (inclusive) from a seeded PCG64 stream."""
    rng = np.random.Generator(np.random.PCG64(seed))
    return [int(x) for x in rng.integers(lo, hi + 1, size=B)]
