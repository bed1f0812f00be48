"""Pins of the fp64 CPU oracle (oracle/pdattn_oracle.c) -- CPU only.

The oracle is only trusted because each of its functions is checked here against something it
does not restate:
  * the binary16 codec against numpy's float16 (all 65536 patterns; ties, subnormals, overflow);
  * decode against closed forms: one key (o = v, lse = s), identical keys (o = mean v,
    lse = s + ln L), one dominant key (o -> its v), two keys with known scores;
  * decode against a dense gather + scipy.special softmax / logsumexp (library routines);
  * invariances: relocating physical pages, permuting the batch, split + merge == whole;
  * the merge against the associativity and identity laws and against logsumexp of the pieces;
  * shared-prefix detection against brute force on small random tables and the reference's
    known cases (01_decode_attention.cu:636-646, 810-815).
Then every plausible mistake that the oracle can be switched into (oracle.FAULTS) is planted in
turn, and at least one pin must catch it; that is what makes the pins meaningful.
"""
import numpy as np
import pytest
from scipy.special import logsumexp, softmax

import oracle
from pdattn import inputs

SCALE = 1.0 / np.sqrt(128.0)


# ---- helpers -------------------------------------------------------------------------------

def dense_reference(bt, kv_start=0):
    """Gather each sequence's keys/values densely with numpy fancy indexing and apply scipy."""
    G = bt.Hq // bt.Hkv
    out = np.zeros((bt.B, bt.Hq, 128))
    lse = np.full((bt.B, bt.Hq), -np.inf)
    for b in range(bt.B):
        L = bt.lens[b]
        pages = bt.indices[bt.indptr[b]:bt.indptr[b + 1]]
        if L <= kv_start:
            continue
        K = bt.k[pages].astype(np.float64).reshape(-1, bt.Hkv, 128)[kv_start:L]
        V = bt.v[pages].astype(np.float64).reshape(-1, bt.Hkv, 128)[kv_start:L]
        for h in range(bt.Hq):
            s = K[:, h // G] @ bt.q[b, h].astype(np.float64) * SCALE
            out[b, h] = softmax(s) @ V[:, h // G]
            lse[b, h] = logsumexp(s)
    return out, lse


def run_oracle(bt, kv_start=0):
    return oracle.decode(bt.q, bt.k, bt.v, bt.indptr, bt.indices, bt.last, bt.Hq, bt.Hkv, kv_start)


def close(a, b, tol=1e-9):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    if not np.array_equal(np.isneginf(a), np.isneginf(b)):
        return False
    fin = ~np.isneginf(b)
    return np.allclose(a[fin], b[fin], atol=tol, rtol=tol)


# ---- individual pins (each returns True when the oracle passes it) ---------------------------

def pin_codec():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = bits.view(np.float16).astype(np.float64)
    got = np.array([oracle.half_to_double(int(x)) for x in bits[::97]])
    if not np.array_equal(np.isnan(got), np.isnan(ref[::97])):
        return False
    ok = np.isnan(ref[::97]) | (got == ref[::97])
    if not ok.all():
        return False
    rng = np.random.default_rng(0)
    xs = np.concatenate([
        rng.standard_normal(3000) * 10.0 ** rng.integers(-8, 5, 3000),
        [1 + 2 ** -11, 1 + 3 * 2 ** -11, 65504.0, 65519.0, 65520.0, 2 ** -24, 2 ** -25,
         3 * 2 ** -25, 2 ** -14, 2 ** -14 - 2 ** -25, -0.0, 1e-30],
    ])
    with np.errstate(over="ignore"):
        want = xs.astype(np.float16).view(np.uint16)
    got = np.array([oracle.double_to_half(float(x)) for x in xs], dtype=np.uint16)
    return np.array_equal(got, want)


def pin_single_key():
    """L = 1: o = v_0 exactly, lse = scale * q . k_0."""
    bt = inputs.make_batch([1, 1], 4, 2, seed=21)
    o, l = run_oracle(bt)
    for b in range(bt.B):
        pg = bt.indices[bt.indptr[b]]
        for h in range(4):
            k0 = bt.k[pg, 0, h // 2].astype(np.float64)
            v0 = bt.v[pg, 0, h // 2].astype(np.float64)
            if not np.array_equal(o[b, h], v0):
                return False
            if abs(l[b, h] - SCALE * float(np.dot(bt.q[b, h].astype(np.float64), k0))) > 1e-12:
                return False
    return True


def pin_identical_keys():
    """All keys equal: uniform weights, o = mean of v, lse = s + ln L."""
    L = 37
    bt = inputs.make_batch([L], 2, 1, seed=22)
    row = bt.k[bt.indices[0], 0, 0].copy()
    bt.k[:] = row
    o, l = run_oracle(bt)
    V = bt.v[bt.indices].astype(np.float64).reshape(-1, 1, 128)[:L, 0]
    for h in range(2):
        s = SCALE * float(np.dot(bt.q[0, h].astype(np.float64), row.astype(np.float64)))
        if not (np.allclose(o[0, h], V.mean(axis=0), atol=1e-12) and abs(l[0, h] - (s + np.log(L))) < 1e-12):
            return False
    return True


def pin_two_keys():
    """Two keys with scores s1, s2: o = (e1 v1 + e2 v2) / (e1 + e2), lse = ln(e1 + e2)."""
    bt = inputs.make_batch([2], 1, 1, seed=23)
    K = bt.k[bt.indices[0], :2, 0].astype(np.float64)
    V = bt.v[bt.indices[0], :2, 0].astype(np.float64)
    q = bt.q[0, 0].astype(np.float64)
    s1, s2 = SCALE * K[0] @ q, SCALE * K[1] @ q
    e1, e2 = np.exp(s1), np.exp(s2)
    o, l = run_oracle(bt)
    return np.allclose(o[0, 0], (e1 * V[0] + e2 * V[1]) / (e1 + e2), atol=1e-12) and \
        abs(l[0, 0] - np.log(e1 + e2)) < 1e-12


def pin_dominant_key():
    """One key far above the rest: o is its value row."""
    bt = inputs.make_batch([50], 1, 1, seed=24)
    q = bt.q[0, 0].astype(np.float64)
    j = 29
    pg, slot = bt.indices[j // 16], j % 16
    bt.k[pg, slot, 0] = (np.sign(q) * 8.0).astype(np.float16)   # q . k_j >> q . k_i
    o, _ = run_oracle(bt)
    return np.allclose(o[0, 0], bt.v[pg, slot, 0].astype(np.float64), atol=1e-6)


def pin_dense_scipy():
    for lens, Hq, Hkv, seed in [([1, 17, 100, 0], 8, 2, 3), ([16, 33, 250], 8, 8, 4), ([40, 7], 8, 1, 5)]:
        bt = inputs.make_batch(lens, Hq, Hkv, seed=seed)
        o, l = run_oracle(bt)
        ro, rl = dense_reference(bt)
        if not (close(o, ro) and close(l, rl)):
            return False
    bt = inputs.make_batch([100, 20], 4, 2, seed=6)
    o, l = run_oracle(bt, kv_start=37)
    ro, rl = dense_reference(bt, kv_start=37)
    return close(o, ro) and close(l, rl)


def pin_page_relocation():
    """Moving pages to other physical slots (table updated) leaves results bit-identical."""
    bt = inputs.make_batch([70, 33], 4, 2, seed=7)
    o1, l1 = run_oracle(bt)
    perm = np.random.default_rng(8).permutation(bt.num_pages)
    k2, v2 = np.empty_like(bt.k), np.empty_like(bt.v)
    k2[perm], v2[perm] = bt.k, bt.v
    o2, l2 = oracle.decode(bt.q, k2, v2, bt.indptr, perm[bt.indices], bt.last, 4, 2)
    return np.array_equal(o1, o2) and np.array_equal(l1, l2)


def pin_split_merge():
    """Per-chunk partials merged with the oracle merge equal the unsplit decode."""
    bt = inputs.make_batch([300, 65, 1], 4, 2, seed=9)
    o, l = run_oracle(bt)
    for nc, ct in [(1, 512), (7, 48), (19, 16)]:
        po, pl = oracle.partials(bt.q, bt.k, bt.v, bt.indptr, bt.indices, bt.last, 4, 2, nc, ct)
        mo, ml = oracle.merge(po, pl)
        if not (close(mo.reshape(o.shape), o, 1e-12) and close(ml.reshape(l.shape), l, 1e-12)):
            return False
    return True


def pin_merge_laws():
    rng = np.random.default_rng(10)
    rows = 6
    po = rng.standard_normal((rows, 5, 128))
    pl = rng.standard_normal((rows, 5)) * 3
    pl[0, 2] = -np.inf
    po[0, 2] = 0.0
    whole_o, whole_l = oracle.merge(po, pl)
    # associativity: merge(merge(0..1), merge(2..4)) == merge(0..4)
    ao, al = oracle.merge(po[:, :2], pl[:, :2])
    bo, bl = oracle.merge(po[:, 2:], pl[:, 2:])
    co, cl = oracle.merge(np.stack([ao, bo], 1), np.stack([al, bl], 1))
    if not (close(co, whole_o, 1e-12) and close(cl, whole_l, 1e-12)):
        return False
    # lse of the merge = logsumexp of the pieces
    if not np.allclose(whole_l, logsumexp(pl, axis=1), atol=1e-12):
        return False
    # (0, -inf) is an identity; an all-empty row gives 0 / -inf
    eo, el = oracle.merge(np.concatenate([po, np.zeros((rows, 1, 128))], 1),
                          np.concatenate([pl, np.full((rows, 1), -np.inf)], 1))
    zo, zl = oracle.merge(np.zeros((1, 3, 128)), np.full((1, 3), -np.inf))
    return close(eo, whole_o, 1e-12) and close(el, whole_l, 1e-12) and not zo.any() and np.isneginf(zl[0])


def _prefix_brute(indptr, indices):
    B = len(indptr) - 1
    if B < 2:
        return 0
    best = 0
    for P in range(0, min(indptr[b + 1] - indptr[b] for b in range(B))):
        if all(indices[indptr[b] + i] == indices[indptr[0] + i] for b in range(B) for i in range(P + 1)):
            best = P + 1
        else:
            break
    return min(best, min(indptr[b + 1] - indptr[b] for b in range(B)) - 1)


def pin_shared_prefix():
    rng = np.random.default_rng(11)
    for _ in range(300):
        B = int(rng.integers(1, 5))
        shared = list(rng.integers(0, 6, size=int(rng.integers(0, 5))))
        indptr, indices = [0], []
        for b in range(B):
            tail = list(rng.integers(0, 6, size=int(rng.integers(0, 4))))
            seq = shared + tail
            indices += seq
            indptr.append(len(indices))
        if oracle.shared_prefix_pages(indptr, indices) != max(0, _prefix_brute(indptr, indices)):
            return False
    # known cases: unshared batch -> 0 (01:810-815); B < 2 -> 0; a fully shared table keeps one
    # private page per sequence (01:641)
    bt = inputs.make_batch([1000] * 4, 32, 8, seed=3, fill=False)
    if oracle.shared_prefix_pages(bt.indptr, bt.indices) != 0:
        return False
    if oracle.shared_prefix_pages([0, 5], [1, 2, 3, 4, 5]) != 0:
        return False
    if oracle.shared_prefix_pages([0, 3, 6], [7, 8, 9, 7, 8, 9]) != 2:
        return False
    sp = inputs.make_shared_prefix_batch(64, [1, 17, 40], 8, 8, seed=13, fill=False)
    return oracle.shared_prefix_pages(sp.indptr, sp.indices) == 4


PINS = {
    "codec": pin_codec,
    "single_key": pin_single_key,
    "identical_keys": pin_identical_keys,
    "two_keys": pin_two_keys,
    "dominant_key": pin_dominant_key,
    "dense_scipy": pin_dense_scipy,
    "page_relocation": pin_page_relocation,
    "split_merge": pin_split_merge,
    "merge_laws": pin_merge_laws,
    "shared_prefix": pin_shared_prefix,
}


@pytest.mark.parametrize("name", list(PINS))
def test_oracle_pin(name, oracle_lib):
    assert PINS[name](), f"oracle fails pin {name}"


@pytest.mark.parametrize("fault", [f for f in oracle.FAULTS if f != "none"])
def test_planted_fault_is_caught(fault, oracle_lib):
    """Each plausible mistake planted in the oracle fails at least one pin."""
    caught = []
    with oracle.fault(fault):
        for name, fn in PINS.items():
            try:
                ok = fn()
            except Exception:
                ok = False
            if not ok:
                caught.append(name)
    assert caught, f"planted fault {fault!r} passes every pin"


def test_plan_chunks_reference_rule(oracle_lib):
    """The restated reference split rule (01:289-312) reproduces the reference's logged chunk
    counts on its 26-SM GPU: 1x32K -> 13 chunks with v2 occupancy 4, 6 with v3 occupancy 2
    (results/01_decode_attention.txt:101-103 report 104 and 48 blocks over 8 pairs)."""
    assert oracle.plan_chunks_ref(26 * 4, 1, 8, 32768)[0] == 13
    assert oracle.plan_chunks_ref(26 * 2, 1, 8, 32768)[0] == 6
    # force_chunks and the <=1 wave / >=256-token caps
    assert oracle.plan_chunks_ref(104, 1, 8, 4097, 7) == (7, 608)
    assert oracle.plan_chunks_ref(104, 64, 8, 1024)[0] == 1
