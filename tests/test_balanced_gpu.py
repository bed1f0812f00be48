"""GPU parity of pdattn_decode_attention_balanced (decode_attention's arguments, with the attended
pages cut into equal ranges on the device) against the fp64 oracle, through the C ABI.

The attended keys of sequence b are [kv_start, min(len_b, kv_start + num_chunks * chunk_tokens)),
the keys the reference's uniform chunks cover (01_decode_attention.cu:88-97), so the oracle runs on
the page table cut to those lengths. Cases: the benchmark configurations, seeded random batches
(kv_start offsets, clipping spans, group sizes, empty sequences), more sequence pieces in a range
than a workgroup stages at once, fewer pages than ranges, the 1023-sequence limit and the uniform
split past it, empty batches, and bitwise determinism for every group size.
"""
import numpy as np
import pytest

import oracle
from _checks import check_lse, check_out
from pdattn import inputs

pytestmark = pytest.mark.gpu


def _clipped(bt, kv_start, span):
    """The batch with every sequence cut to its last attended key (kv_start + span)."""
    lens, ind, ip, last = [], [], [0], []
    for b, L in enumerate(bt.lens):
        Lc = min(L, kv_start + span) if span is not None else L
        npg = (Lc + 15) // 16
        lens.append(Lc)
        ind.extend(bt.indices[bt.indptr[b]:bt.indptr[b] + npg].tolist())
        ip.append(ip[-1] + npg)
        last.append(Lc - (npg - 1) * 16 if npg else 0)
    return (np.array(ip, np.int32), np.array(ind if ind else [0], np.int32), np.array(last, np.int32))


def _ref(bt, kv_start=0, span=None):
    ip, ind, last = _clipped(bt, kv_start, span)
    return oracle.decode(bt.q, bt.k, bt.v, ip, ind, last, bt.Hq, bt.Hkv, kv_start=kv_start, threads=8)


BASELINE_CONFIGS = [
    ("C1 B=1 L=2048", [2048], 7),
    ("C2 B=1 L=32768", [32768], 11),
    ("C3 B=8 L=8192", [8192] * 8, 11),
    ("64x1K", [1024] * 64, 11),
    ("C4 B=64 ragged U[256,4096]", None, 17),
]


@pytest.mark.parametrize("cfg", BASELINE_CONFIGS, ids=[c[0] for c in BASELINE_CONFIGS])
def test_baseline_configs_match_oracle(cfg):
    import _gpu
    tag, lens, seed = cfg
    if lens is None:
        lens = inputs.ragged_lens(64, 256, 4096, seed)
    print(f"[case] balanced {tag} seed={seed}", flush=True)
    bt = inputs.make_batch(lens, 32, 8, seed=seed)
    ro, rl = _ref(bt)
    o, l = _gpu.run_balanced(_gpu.DeviceBatch(bt))
    check_out(o, ro, tag=f"{tag} balanced")
    check_lse(l, rl, tag=f"{tag} balanced")


@pytest.mark.parametrize("seed", range(12))
def test_random_batches_match_oracle(seed):
    """Seeded random shapes: batch size, lengths (empty sequences, partial last pages), group
    size, kv_start (aligned or not) and a span that may clip the longest sequences."""
    import _gpu
    rng = np.random.default_rng(2000 + seed)
    Hkv = int(rng.choice([1, 2, 4, 8]))
    G = int(rng.choice([1, 2, 4, 8]))
    B = int(rng.integers(1, 40))
    lens = [int(x) for x in rng.integers(0, 3000, B)]
    if rng.random() < 0.3:
        lens[int(rng.integers(0, B))] = 0
    kv_start = int(rng.choice([0, 0, 16, 37, 512]))
    nc = int(rng.integers(1, 9))
    ct = int(rng.choice([16, 48, 100, 256, 1024]))
    print(f"[case] balanced random seed={seed}: B={B} Hq={G * Hkv} Hkv={Hkv} kv_start={kv_start} "
          f"chunks={nc}x{ct} lens={lens}", flush=True)
    bt = inputs.make_batch(lens, G * Hkv, Hkv, seed=seed)
    ro, rl = _ref(bt, kv_start, nc * ct)
    o, l = _gpu.run_balanced(_gpu.DeviceBatch(bt), kv_start=kv_start, chunks=(nc, ct))
    check_out(o, ro, tag=f"balanced random seed={seed}")
    check_lse(l, rl, tag=f"balanced random seed={seed}")


@pytest.mark.parametrize("lens_case", ["1000 short", "1023 max", "1024 uniform", "long+short"])
def test_many_sequences(lens_case):
    """More sequence pieces in one range than a workgroup stages at once (batches of segments),
    the largest batch the kernel takes (1023 sequences), one more (run as the uniform split), and
    one long sequence beside many short ones."""
    import _gpu
    rng = np.random.default_rng(7)
    if lens_case == "1000 short":
        lens = [int(x) for x in rng.integers(1, 60, 1000)]
    elif lens_case == "1023 max":
        lens = [int(x) for x in rng.integers(0, 200, 1023)]
    elif lens_case == "1024 uniform":
        lens = [int(x) for x in rng.integers(0, 200, 1024)]
    else:
        lens = [20000] + [int(x) for x in rng.integers(1, 40, 300)]
    print(f"[case] balanced many sequences: {lens_case} B={len(lens)}", flush=True)
    bt = inputs.make_batch(lens, 32, 8, seed=8)
    ro, rl = _ref(bt)
    o, l = _gpu.run_balanced(_gpu.DeviceBatch(bt))
    check_out(o, ro, tag=lens_case)
    check_lse(l, rl, tag=lens_case)


@pytest.mark.parametrize("lens", [[1], [17], [100], [300, 0, 5], [0, 40, 0], [16] * 3],
                         ids=["1", "17", "100", "300-0-5", "0-40-0", "3x16"])
def test_fewer_pages_than_ranges(lens):
    """Fewer attended pages than ranges: empty ranges between the pieces of a sequence weigh
    nothing in its merge."""
    import _gpu
    print(f"[case] balanced few pages lens={lens}", flush=True)
    bt = inputs.make_batch(lens, 32, 8, seed=9)
    ro, rl = _ref(bt)
    o, l = _gpu.run_balanced(_gpu.DeviceBatch(bt))
    check_out(o, ro, tag=f"few pages {lens}")
    check_lse(l, rl, tag=f"few pages {lens}")


@pytest.mark.parametrize("lens", [[0], [0, 0, 0]])
def test_empty_batches(lens):
    import _gpu
    bt = inputs.make_batch(lens, 8, 2, seed=9)
    db = _gpu.DeviceBatch(bt)
    db.out.fill_(7.0)
    db.lse.fill_(7.0)
    o, l = _gpu.run_balanced(db)
    assert np.all(o == 0) and np.all(np.isneginf(l))


def test_kv_start_past_every_sequence():
    """kv_start beyond the end of every sequence: no key is attended, every row 0 / -inf."""
    import _gpu
    bt = inputs.make_batch([100, 33], 32, 8, seed=3)
    o, l = _gpu.run_balanced(_gpu.DeviceBatch(bt), kv_start=200, chunks=(2, 64))
    assert np.all(o == 0) and np.all(np.isneginf(l))


@pytest.mark.parametrize("Hq,Hkv", [(8, 8), (16, 8), (32, 8), (32, 4)], ids=["G1", "G2", "G4", "G8"])
def test_bitwise_deterministic(Hq, Hkv):
    import _gpu
    print(f"[case] balanced determinism Hq={Hq} Hkv={Hkv}", flush=True)
    bt = inputs.make_batch([3000, 777, 16, 1, 9000], Hq, Hkv, seed=12)
    db = _gpu.DeviceBatch(bt)
    ro, rl = _ref(bt)
    first = None
    for _ in range(4):
        o, l = _gpu.run_balanced(db)
        if first is None:
            first = (o.copy(), l.copy())
            check_out(o, ro, tag=f"G={Hq // Hkv}")
            check_lse(l, rl, tag=f"G={Hq // Hkv}")
        else:
            assert np.array_equal(o, first[0]) and np.array_equal(l, first[1])
