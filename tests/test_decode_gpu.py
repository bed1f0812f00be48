"""GPU parity of the split-KV decode paths against the fp64 oracle.

Case matrix: the reference's correctness cases (01_decode_attention.cu:750-755, seed 7 at 01:758)
with its three split settings {no split, heuristic, 7 chunks} (01:763), on both its U(-1,1) data
and the N(0,1) data of the benchmark configurations; then the benchmark configurations themselves,
edge cases (empty sequences, partial last pages, kv_start), determinism and invariances.
"""
import numpy as np
import pytest

import oracle
from _checks import check_lse, check_out
from pdattn import inputs

pytestmark = pytest.mark.gpu

REF_CASES = [
    ([1, 17, 1000], 8, 8, "MHA"),
    ([5, 300, 2049, 4096], 32, 8, "GQA G=4 mixed"),
    ([33, 777], 16, 2, "GQA G=8"),
    ([16, 32, 48, 4097], 4, 2, "page boundaries G=2"),
]
DISTS = ["uniform", "normal"]


def _ref(bt, kv_start=0, threads=8):
    return oracle.decode(bt.q, bt.k, bt.v, bt.indptr, bt.indices, bt.last, bt.Hq, bt.Hkv,
                         kv_start=kv_start, threads=threads)


@pytest.fixture(scope="module", params=[(c, d) for c in REF_CASES for d in DISTS],
                ids=lambda p: f"{p[0][3]}-{p[1]}")
def ref_case(request):
    import _gpu
    (lens, Hq, Hkv, tag), dist = request.param
    print(f"[case] {tag} lens={lens} Hq={Hq} Hkv={Hkv} dist={dist} seed=7", flush=True)
    bt = inputs.make_batch(lens, Hq, Hkv, seed=7, dist=dist)
    o, l = _ref(bt)
    return bt, _gpu.DeviceBatch(bt), o, l


@pytest.mark.parametrize("force", [1, 0, 7])
def test_uniform_split_matches_oracle(ref_case, force):
    import _gpu
    bt, db, ro, rl = ref_case
    o, l, nc = _gpu.run_uniform(db, force)
    if force:
        assert nc <= force
    check_out(o, ro, tag=f"chunks={nc}")
    check_lse(l, rl, tag=f"chunks={nc}")


@pytest.mark.parametrize("wg", [0, 1, 3, 7, 64, 1000])
def test_plan_matches_oracle(ref_case, wg):
    import _gpu
    bt, db, ro, rl = ref_case
    o, l, info = _gpu.run_plan(db, wg)
    check_out(o, ro, tag=f"W={info.workgroups}")
    check_lse(l, rl, tag=f"W={info.workgroups}")


@pytest.mark.parametrize("kv_start", [0, 37, 512])
def test_partials_match_oracle(ref_case, kv_start):
    """Per-chunk normalized partials and lse (decode_partial, 01:88-97, 228-235)."""
    import _gpu
    bt, db, _, _ = ref_case
    nc, ct = 7, 96
    po, pl = _gpu.run_partials(db, nc, ct, kv_start)
    ro, rl = oracle.partials(bt.q, bt.k, bt.v, bt.indptr, bt.indices, bt.last, bt.Hq, bt.Hkv,
                             nc, ct, kv_start)
    check_lse(pl, rl, tag="part_lse")
    # partial o is fp32 here: hold it to the same 2e-3 bar
    check_out(po, ro, tag="part_o")


def test_uniform_kv_start_matches_oracle():
    import _gpu, pdattn
    bt = inputs.make_batch([100, 700, 33], 16, 4, seed=5)
    db = _gpu.DeviceBatch(bt)
    for kv_start in (0, 16, 50, 99):
        nc, ct = pdattn.plan_chunks(bt.G, bt.B, bt.Hkv, bt.max_len, 3)
        p = db.params(nc, ct, kv_start=kv_start)
        ws = pdattn.Workspace()
        pdattn.decode_attention(p, bt.G, db.out, db.lse, ws)
        o, l = db.results()
        pdattn.workspace_release(ws)
        ro, rl = _ref(bt, kv_start)
        check_out(o, ro, tag=f"kv_start={kv_start}")
        check_lse(l, rl, tag=f"kv_start={kv_start}")


UNIFORM_SHAPES = [
    # tag, lens, Hq, Hkv, num_chunks, chunk_tokens, kv_start
    ("chunk past the LDS page list", [40000, 123], 32, 8, 1, 40000, 0),   # 2501 pages: one-chunk kernel
    ("long chunks", [40000, 123], 32, 8, 2, 20000, 0),
    ("many items per workgroup", "ragged300", 8, 8, 1, 304, 0),         # 2400 items, 10 per workgroup
    ("segment cap per workgroup", "ragged300", 8, 8, 3, 100, 0),        # 7200 items, 24 per workgroup
    ("unaligned start and chunk", [1000, 77, 0, 513], 32, 8, 5, 200, 23),
    ("G=8, segment cap of the compact layout", "ragged300", 64, 8, 2, 160, 0),   # 4800 items, 8 per workgroup
]


@pytest.mark.parametrize("case", UNIFORM_SHAPES, ids=[c[0] for c in UNIFORM_SHAPES])
def test_uniform_items_per_workgroup(case):
    """The reference-shaped split runs several (pair, chunk) items per workgroup on the balanced
    body, with descriptors built in the kernel: items per workgroup up to the segment cap, empty
    sequences among them, chunks that do not start or end on a page, and a chunk too long for the
    LDS page list (the one-chunk-per-workgroup kernel). Final out / lse and the partials."""
    import _gpu
    import pdattn
    tag, lens, Hq, Hkv, nc, ct, kv_start = case
    if lens == "ragged300":
        lens = [int(x) for x in np.random.default_rng(3).integers(0, 301, 300)]
    print(f"[case] {tag} B={len(lens)} max_len={max(lens)} nc={nc} ct={ct} kv_start={kv_start}", flush=True)
    bt = inputs.make_batch(lens, Hq, Hkv, seed=29)
    db = _gpu.DeviceBatch(bt)
    p = db.params(nc, ct, kv_start=kv_start)
    ws = pdattn.Workspace()
    pdattn.decode_attention(p, bt.G, db.out, db.lse, ws)
    o, l = db.results()
    pdattn.workspace_release(ws)
    ro, rl = _ref(bt, kv_start)
    check_out(o, ro, tag=tag)
    check_lse(l, rl, tag=tag)
    if bt.B * bt.Hq * nc <= 20000:
        po, pl = _gpu.run_partials(db, nc, ct, kv_start)
        pro, prl = oracle.partials(bt.q, bt.k, bt.v, bt.indptr, bt.indices, bt.last, bt.Hq, bt.Hkv,
                                   nc, ct, kv_start)
        check_lse(pl, prl, tag=tag + " part_lse")
        check_out(po, pro, tag=tag + " part_o")


@pytest.mark.parametrize("kv_start", [0, 40])
def test_single_chunk_skips_the_merge_bitwise(kv_start):
    """decode_attention with one chunk per sequence writes out / lse from the partial kernel:
    bitwise what decode_partial + merge_states give (a merge of one state returns it), and the
    oracle's result; an empty sequence still gets 0 / -inf."""
    import torch
    import _gpu
    import pdattn
    bt = inputs.make_batch([0, 1, 300, 1000], 32, 8, seed=19)
    db = _gpu.DeviceBatch(bt)
    ct = 1024 - kv_start
    p = db.params(1, ct, kv_start=kv_start)
    ws = pdattn.Workspace()
    pdattn.decode_attention(p, bt.G, db.out, db.lse, ws)
    o1, l1 = db.results()
    pdattn.workspace_release(ws)
    rows = bt.B * bt.Hq
    po, pl = _gpu.run_partials(db, 1, ct, kv_start)
    out = torch.empty(rows, 128, dtype=torch.float16, device=_gpu.device())
    lse = torch.empty(rows, dtype=torch.float32, device=_gpu.device())
    pdattn.merge_states(torch.from_numpy(po.astype(np.float32)).to(out.device),
                        torch.from_numpy(pl.astype(np.float32)).to(out.device), out, lse, rows, 1)
    torch.cuda.synchronize()
    o2 = out.float().cpu().numpy().astype(np.float64).reshape(o1.shape)
    l2 = lse.cpu().numpy().astype(np.float64).reshape(l1.shape)
    assert np.array_equal(o1, o2) and np.array_equal(l1, l2)
    assert np.all(o1[0] == 0) and np.all(np.isneginf(l1[0]))
    ro, rl = _ref(bt, kv_start)
    check_out(o1, ro, tag=f"one chunk, kv_start={kv_start}")
    check_lse(l1, rl, tag=f"one chunk, kv_start={kv_start}")


def test_merge_states_matches_oracle():
    import torch
    import pdattn
    rng = np.random.default_rng(3)
    rows, C = 40, 9
    po = rng.standard_normal((rows, C, 128)).astype(np.float32)
    pl = (rng.standard_normal((rows, C)) * 5).astype(np.float32)
    pl[rng.random((rows, C)) < 0.2] = -np.inf      # empty chunks
    pl[3, :] = -np.inf                              # an all-empty row
    po[pl == -np.inf] = 0.0
    d = torch.device("cuda:0")
    tpo, tpl = torch.from_numpy(po).to(d), torch.from_numpy(pl).to(d)
    out = torch.empty(rows, 128, dtype=torch.float16, device=d)
    lse = torch.empty(rows, dtype=torch.float32, device=d)
    pdattn.merge_states(tpo, tpl, out, lse, rows, C)
    torch.cuda.synchronize()
    ro, rl = oracle.merge(po.astype(np.float64), pl.astype(np.float64))
    check_out(out.float().cpu().numpy(), ro, tag="merge out")
    check_lse(lse.cpu().numpy(), rl, tag="merge lse")
    assert np.all(out[3].float().cpu().numpy() == 0) and np.isneginf(lse[3].item())


BASELINE_CONFIGS = [
    ("C1 B=1 L=2048", [2048], 7),
    ("C2 B=1 L=32768", [32768], 11),
    ("C3 B=8 L=8192", [8192] * 8, 11),
    ("64x1K", [1024] * 64, 11),
    ("C4 B=64 ragged U[256,4096]", None, 11),
]


@pytest.mark.parametrize("cfg", BASELINE_CONFIGS, ids=[c[0] for c in BASELINE_CONFIGS])
def test_baseline_configs_match_oracle(cfg):
    import _gpu
    tag, lens, seed = cfg
    if lens is None:
        lens = inputs.ragged_lens(64, 256, 4096, seed)
    print(f"[case] {tag} seed={seed}", flush=True)
    bt = inputs.make_batch(lens, 32, 8, seed=seed)
    ro, rl = _ref(bt)
    db = _gpu.DeviceBatch(bt)
    o, l, info = _gpu.run_plan(db)
    check_out(o, ro, tag=f"{tag} plan W={info.workgroups}")
    check_lse(l, rl, tag=f"{tag} plan")
    o, l, nc = _gpu.run_uniform(db)
    check_out(o, ro, tag=f"{tag} uniform chunks={nc}")
    check_lse(l, rl, tag=f"{tag} uniform")


@pytest.mark.parametrize("lens", [[0, 5, 0, 100], [0], [0, 0, 0], [16, 0], [1]])
def test_empty_sequences(lens):
    import _gpu
    bt = inputs.make_batch(lens, 8, 2, seed=9)
    ro, rl = _ref(bt)
    db = _gpu.DeviceBatch(bt)
    for wg in (0, 1, 5):
        o, l, _ = _gpu.run_plan(db, wg)
        check_out(o, ro, tag=f"plan W={wg}")
        check_lse(l, rl, tag=f"plan W={wg}")
    o, l, _ = _gpu.run_uniform(db)
    check_out(o, ro, tag="uniform")
    check_lse(l, rl, tag="uniform")


def test_plan_bitwise_deterministic():
    """Split pairs are merged in fixed order, whoever arrives last."""
    import _gpu
    bt = inputs.make_batch([5000, 3001, 17], 32, 8, seed=2)
    db = _gpu.DeviceBatch(bt)
    first = None
    for _ in range(5):
        o, l, info = _gpu.run_plan(db, 97)
        assert info.split_pairs > 0
        if first is None:
            first = (o.copy(), l.copy())
        else:
            assert np.array_equal(o, first[0]) and np.array_equal(l, first[1])


@pytest.mark.parametrize("Hq,Hkv", [(8, 8), (16, 8), (32, 8), (32, 4)], ids=["G1", "G2", "G4", "G8"])
@pytest.mark.parametrize("path", ["plan", "uniform"])
def test_bitwise_deterministic_every_group_size(Hq, Hkv, path):
    """Each kernel instantiation (G = 1, 2, 4, 8; balanced and uniform-split paths) gives the
    same bits on repeated launches, with split pairs merged."""
    import _gpu
    print(f"determinism: {path} Hq={Hq} Hkv={Hkv}", flush=True)
    bt = inputs.make_batch([3000, 777, 16, 1], Hq, Hkv, seed=12)
    db = _gpu.DeviceBatch(bt)
    first = None
    for _ in range(4):
        if path == "plan":
            o, l, info = _gpu.run_plan(db, 61)
            assert info.split_pairs > 0
        else:
            o, l, nc = _gpu.run_uniform(db, 5)
            assert nc > 1
        if first is None:
            first = (o.copy(), l.copy())
        else:
            assert np.array_equal(o, first[0]) and np.array_equal(l, first[1])


@pytest.mark.parametrize("seed", range(12))
def test_random_batches_match_oracle(seed):
    """Seeded random shapes: batch size, lengths (empty sequences and partial last pages
    included), group size, forced grid and chunk size of the balanced planner, and forced chunk
    counts of the uniform split."""
    import _gpu
    rng = np.random.default_rng(1000 + seed)
    Hkv = int(rng.choice([1, 2, 4, 8]))
    G = int(rng.choice([1, 2, 4, 8]))
    B = int(rng.integers(1, 24))
    lens = [int(x) for x in rng.integers(0, 2500, B)]
    if rng.random() < 0.3:
        lens[int(rng.integers(0, B))] = 0
    wg = int(rng.choice([0, 1, 5, 33, 256, 700]))
    print(f"random batch seed={seed}: B={B} Hq={G * Hkv} Hkv={Hkv} W={wg} lens={lens}", flush=True)
    bt = inputs.make_batch(lens, G * Hkv, Hkv, seed=seed)
    db = _gpu.DeviceBatch(bt)
    ro, rl = _ref(bt)
    o, l, info = _gpu.run_plan(db, wg)
    check_out(o, ro, tag=f"random plan seed={seed} W={info.workgroups}")
    check_lse(l, rl, tag=f"random plan seed={seed}")
    force = int(rng.integers(0, 9))
    o, l, nc = _gpu.run_uniform(db, force)
    check_out(o, ro, tag=f"random uniform seed={seed} chunks={nc}")
    check_lse(l, rl, tag=f"random uniform seed={seed}")


def test_page_permutation_invariance():
    """Moving the pages to other physical slots (and the page table with them) changes nothing."""
    import _gpu
    bt = inputs.make_batch([700, 1500], 16, 4, seed=4)
    db = _gpu.DeviceBatch(bt)
    o1, l1, _ = _gpu.run_plan(db, 13)
    rng = np.random.default_rng(1)
    perm = rng.permutation(bt.num_pages)          # new slot of physical page i
    k2 = np.empty_like(bt.k)
    v2 = np.empty_like(bt.v)
    k2[perm] = bt.k
    v2[perm] = bt.v
    bt2 = inputs.Batch(bt.lens, bt.Hq, bt.Hkv, bt.indptr, perm[bt.indices].astype(np.int32),
                       bt.last, bt.num_pages, bt.seed, bt.q, k2, v2)
    o2, l2, _ = _gpu.run_plan(_gpu.DeviceBatch(bt2), 13)
    assert np.array_equal(o1, o2) and np.array_equal(l1, l2)


def test_split_invariance_across_workgroup_counts():
    """Different plan cuts agree within fp32 rounding of the merge."""
    import _gpu
    bt = inputs.make_batch([4096, 2500, 100], 32, 8, seed=6)
    db = _gpu.DeviceBatch(bt)
    outs = [_gpu.run_plan(db, wg)[:2] for wg in (1, 24, 256, 2000)]
    for o, l in outs[1:]:
        assert np.max(np.abs(o - outs[0][0])) <= 2e-3
        assert np.max(np.abs(l - outs[0][1])) <= 1e-4
