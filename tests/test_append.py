"""Paged KV append (pdattn_append_kv) and its host restatement (oracle.append_kv).

CPU: the restatement is pinned against a decode-side check it does not share code with: after
appending each sequence's newest token, the fp64 decode oracle over the paged caches must equal
a dense softmax over keys gathered by numpy from the original pages plus the new rows placed
directly at their positions. Every planted addressing mistake must fail that check. Read-back,
untouched bytes and the invalid-token count are checked as well.

GPU: the library's caches after an append must equal the restatement's byte for byte, for
decode-style (one token per sequence) and prefill-style (several positions per sequence)
appends, with out-of-range tokens counted and skipped; decode after the append matches the
oracle.
"""
import numpy as np
import pytest
from scipy.special import logsumexp, softmax

import oracle
from pdattn import inputs

SCALE = 1.0 / np.sqrt(128.0)


def _new_rows(n, Hkv, seed):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal((n, Hkv, 128)).astype(np.float16),
            rng.standard_normal((n, Hkv, 128)).astype(np.float16))


def _dense_after_append(bt, k_new, v_new):
    """Decode over dense keys: positions < L-1 from the original pages, position L-1 = new row."""
    G = bt.Hq // bt.Hkv
    out = np.zeros((bt.B, bt.Hq, 128))
    lse = np.full((bt.B, bt.Hq), -np.inf)
    for b in range(bt.B):
        L = bt.lens[b]
        if L == 0:
            continue
        pages = bt.indices[bt.indptr[b]:bt.indptr[b + 1]]
        K = bt.k[pages].astype(np.float64).reshape(-1, bt.Hkv, 128)[:L].copy()
        V = bt.v[pages].astype(np.float64).reshape(-1, bt.Hkv, 128)[:L].copy()
        K[L - 1] = k_new[b]
        V[L - 1] = v_new[b]
        for h in range(bt.Hq):
            s = K[:, h // G] @ bt.q[b, h].astype(np.float64) * SCALE
            out[b, h] = softmax(s) @ V[:, h // G]
            lse[b, h] = logsumexp(s)
    return out, lse


def _decode_after_append(lens, Hq, Hkv, seed, fault="none"):
    bt = inputs.make_batch(lens, Hq, Hkv, seed)
    k_new, v_new = _new_rows(bt.B, Hkv, seed + 1)
    pos = np.array(bt.lens) - 1
    kc, vc, bad = oracle.append_kv(bt.k, bt.v, k_new, v_new, np.arange(bt.B), pos, bt.indptr,
                                   bt.indices, fault=fault)
    out, lse = oracle.decode(bt.q, kc, vc, bt.indptr, bt.indices, bt.last, Hq, Hkv)
    ref_o, ref_l = _dense_after_append(bt, k_new, v_new)
    return bad == 0 and np.allclose(out, ref_o, atol=1e-9) and np.allclose(lse, ref_l, atol=1e-9)


CASES = [([37, 16, 1, 300], 32, 8), ([17, 33], 8, 8), ([5, 64, 100], 16, 2)]


@pytest.mark.parametrize("lens,Hq,Hkv", CASES)
def test_oracle_append_then_decode_matches_dense(lens, Hq, Hkv, oracle_lib):
    assert _decode_after_append(lens, Hq, Hkv, seed=3)


@pytest.mark.parametrize("fault", [f for f in oracle.APPEND_FAULTS if f != "none"])
def test_planted_append_fault_is_caught(fault, oracle_lib):
    assert not all(_decode_after_append(lens, Hq, Hkv, seed=3, fault=fault) for lens, Hq, Hkv in CASES)


def test_oracle_append_read_back_and_untouched():
    bt = inputs.make_batch([40, 70], 16, 2, seed=5)
    k_new, v_new = _new_rows(4, 2, 6)
    bidx, pos = np.array([0, 1, 1, 0]), np.array([39, 69, 10, 0])
    kc, vc, bad = oracle.append_kv(bt.k, bt.v, k_new, v_new, bidx, pos, bt.indptr, bt.indices)
    assert bad == 0
    touched = np.zeros(bt.k.shape[:2], bool)
    for t in range(4):
        page = bt.indices[bt.indptr[bidx[t]] + pos[t] // 16]
        assert np.array_equal(kc[page, pos[t] % 16], k_new[t])
        assert np.array_equal(vc[page, pos[t] % 16], v_new[t])
        touched[page, pos[t] % 16] = True
    assert np.array_equal(kc[~touched], bt.k[~touched]) and np.array_equal(vc[~touched], bt.v[~touched])


def test_oracle_append_counts_invalid():
    bt = inputs.make_batch([20, 0], 8, 2, seed=7)
    k_new, v_new = _new_rows(4, 2, 8)
    # position 32 is past sequence 0's two pages; sequence 1 has no pages; b = 5 does not exist
    kc, vc, bad = oracle.append_kv(bt.k, bt.v, k_new, v_new, np.array([0, 0, 1, 5]),
                                   np.array([31, 32, 0, 0]), bt.indptr, bt.indices)
    assert bad == 3


# ---- GPU: the library against the restatement ---------------------------------------------------

def _gpu_append_case(lens, Hq, Hkv, bidx, pos, seed):
    import torch
    import pdattn
    from _gpu import DeviceBatch, device
    bt = inputs.make_batch(lens, Hq, Hkv, seed)
    db = DeviceBatch(bt)
    n = len(bidx)
    k_new, v_new = _new_rows(n, Hkv, seed + 1)
    d = device()
    kn, vn = torch.from_numpy(k_new).to(d), torch.from_numpy(v_new).to(d)
    bi = torch.from_numpy(np.asarray(bidx, np.int32)).to(d)
    po = torch.from_numpy(np.asarray(pos, np.int32)).to(d)
    bad = torch.zeros(1, dtype=torch.int32, device=d)
    print(f"append case lens={lens} Hkv={Hkv} n={n}", flush=True)
    pdattn.append_kv(kn, vn, db.k, db.v, db.indptr, db.indices, bi, po, bt.B, Hkv, bad)
    torch.cuda.synchronize()
    kc, vc, nbad = oracle.append_kv(bt.k, bt.v, k_new, v_new, bidx, pos, bt.indptr, bt.indices)
    assert int(bad.item()) == nbad
    assert np.array_equal(db.k.cpu().numpy().view(np.uint16), kc.view(np.uint16))
    assert np.array_equal(db.v.cpu().numpy().view(np.uint16), vc.view(np.uint16))
    return bt, db, kc, vc


@pytest.mark.gpu
@pytest.mark.parametrize("lens,Hq,Hkv", CASES + [([32768], 32, 8), ([1024] * 64, 32, 8)])
def test_append_decode_style_bitexact(lens, Hq, Hkv):
    B = len(lens)
    _gpu_append_case(lens, Hq, Hkv, np.arange(B), np.array(lens) - 1, seed=11)


@pytest.mark.gpu
def test_append_prefill_style_and_invalid():
    lens = [200, 45, 1, 64]
    rng = np.random.default_rng(2)
    bidx, pos = [], []
    for b, L in enumerate(lens):
        ps = rng.choice(L, size=min(L, 17), replace=False)
        bidx += [b] * len(ps)
        pos += ps.tolist()
    bidx += [0, 3, 7, 2]           # out of range: position 200 of 200, 64 of 64, no sequence 7, -1
    pos += [208, 64, 0, -1]
    _gpu_append_case(lens, 32, 8, np.array(bidx), np.array(pos), seed=4)


@pytest.mark.gpu
@pytest.mark.parametrize("Hkv,lens", [(8, [2000, 1500, 37, 700]), (1, [20000, 15000, 3])])
def test_append_prefill_many_tokens_per_workgroup(Hkv, lens):
    """A prefill-sized append (thousands of tokens, so a workgroup takes 16 tokens at Hkv = 8 and
    up to 128 at Hkv = 1): every position of every sequence, shuffled so that one workgroup's
    tokens land in different pages and sequences, with invalid tokens at random places and a
    token count that leaves a ragged last workgroup."""
    rng = np.random.default_rng(5 + Hkv)
    bidx = np.concatenate([np.full(L, b) for b, L in enumerate(lens)])
    pos = np.concatenate([np.arange(L) for L in lens])
    bad_b = rng.choice([-1, len(lens), 0], size=41)   # no such sequence, or sequence 0 ...
    bad_p = np.where(bad_b == 0, -(-lens[0] // 16) * 16, 0)   # ... at the first position past its pages
    bidx, pos = np.concatenate([bidx, bad_b]), np.concatenate([pos, bad_p])
    perm = rng.permutation(len(bidx))
    _gpu_append_case(lens, 4 * Hkv, Hkv, bidx[perm], pos[perm], seed=21)


@pytest.mark.gpu
def test_decode_after_append_matches_oracle():
    from _checks import check_lse, check_out
    from _gpu import run_plan
    lens = [129, 1000, 16, 2049]
    bt, db, kc, vc = _gpu_append_case(lens, 32, 8, np.arange(4), np.array(lens) - 1, seed=9)
    o, l, _ = run_plan(db)
    ro, rl = oracle.decode(bt.q, kc, vc, bt.indptr, bt.indices, bt.last, 32, 8)
    check_out(o, ro, tag="decode after append")
    check_lse(l, rl, tag="decode after append")
