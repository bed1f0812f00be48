"""GPU parity of the shared-prefix (cascade) path against the fp64 oracle.

Cases: the reference's cascade correctness cases (01_decode_attention.cu:782-787, seed 13,
min_prefix 16, with the check that the detected prefix equals Lp at 01:796), the benchmark's
cascade configuration (64 requests x 8192 shared + 512 private tokens), the prefix kernel on its
own against per-chunk oracle partials, and the no-sharing fallback.
"""
import numpy as np
import pytest

import oracle
from _checks import check_lse, check_out
from pdattn import inputs

pytestmark = pytest.mark.gpu

SCASES = [
    (64, [1, 17, 40], 8, 8, "MHA prefix 64"),
    (48, [5, 300, 33, 16, 2], 32, 8, "G=4 prefix 48 (partial tile)"),
    (1024, [77] * 40, 32, 8, "G=4 40 seqs = 160 queries"),
    (256, [100, 3], 16, 2, "G=8 prefix 256"),
    (2048, [1] * 70, 32, 8, "G=4 280 queries (two query groups)"),
]


def _ref(bt, threads=8):
    return oracle.decode(bt.q, bt.k, bt.v, bt.indptr, bt.indices, bt.last, bt.Hq, bt.Hkv,
                         threads=threads)


@pytest.mark.parametrize("dist", ["uniform", "normal"])
@pytest.mark.parametrize("case", SCASES, ids=[c[4] for c in SCASES])
def test_cascade_matches_oracle(case, dist):
    import _gpu
    Lp, suffix, Hq, Hkv, tag = case
    print(f"[case] cascade {tag} dist={dist} seed=13", flush=True)
    bt = inputs.make_shared_prefix_batch(Lp, suffix, Hq, Hkv, seed=13, dist=dist)
    assert oracle.shared_prefix_pages(bt.indptr, bt.indices) * 16 == Lp
    ro, rl = _ref(bt)
    o, l, info = _gpu.run_cascade(_gpu.DeviceBatch(bt), min_prefix=16)
    assert info.use == 1 and info.prefix_tokens == Lp
    check_out(o, ro, tag=tag)
    check_lse(l, rl, tag=tag)


def test_cascade_benchmark_config():
    """64 requests sharing an 8192-token prefix plus 512 private tokens each (config 5)."""
    import _gpu
    bt = inputs.make_shared_prefix_batch(8192, [512] * 64, 32, 8, seed=21)
    print("[case] cascade 64 x (8192 + 512) seed=21", flush=True)
    ro, rl = _ref(bt)
    db = _gpu.DeviceBatch(bt)
    o, l, info = _gpu.run_cascade(db)
    assert info.use == 1 and info.prefix_tokens == 8192
    check_out(o, ro, tag="cascade")
    check_lse(l, rl, tag="cascade")
    o2, l2, _ = _gpu.run_plan(db)
    check_out(o2, ro, tag="non-shared plan")
    check_lse(l2, rl, tag="non-shared plan")


@pytest.mark.parametrize("chunk_tokens,Lp", [(16, 640), (64, 640), (96, 640), (1024, 640), (8192, 8240)],
                         ids=["16", "64", "96", "1024", "8192-max"])
def test_prefix_kernel_partials(chunk_tokens, Lp):
    """The MFMA prefix kernel alone: per-chunk partials over the shared keys (8192 tokens: the
    largest chunk, 512 staged page ids, followed by a 48-token partial chunk)."""
    import torch
    import _gpu
    import pdattn
    print(f"[case] prefix kernel chunk_tokens={chunk_tokens} Lp={Lp}", flush=True)
    bt = inputs.make_shared_prefix_batch(Lp, [3, 20, 50], 32, 8, seed=8)
    db = _gpu.DeviceBatch(bt)
    nchunks = (Lp + chunk_tokens - 1) // chunk_tokens
    rows = bt.B * bt.Hq
    d = torch.device("cuda:0")
    po = torch.full((rows, nchunks, 128), float("nan"), dtype=torch.float32, device=d)
    pl = torch.full((rows, nchunks), float("nan"), dtype=torch.float32, device=d)
    pp = pdattn.PrefixParams()
    pp.q, pp.k_cache, pp.v_cache = db.q.data_ptr(), db.k.data_ptr(), db.v.data_ptr()
    pp.prefix_pages = db.indices.data_ptr()          # sequence 0 starts at indptr[0] = 0
    pp.part_o, pp.part_lse = po.data_ptr(), pl.data_ptr()
    pp.B, pp.Hq, pp.Hkv = bt.B, bt.Hq, bt.Hkv
    pp.prefix_len, pp.chunk_tokens, pp.part_stride = Lp, chunk_tokens, nchunks
    pp.sm_scale = 1.0 / np.sqrt(128)
    pdattn.cascade_prefix(pp)
    torch.cuda.synchronize()
    # oracle: per-chunk partials of a batch whose sequences are cut to the shared prefix
    lens = [Lp] * bt.B
    indptr = np.arange(bt.B + 1, dtype=np.int32) * (Lp // 16)
    indices = np.concatenate([bt.indices[bt.indptr[b]:bt.indptr[b] + Lp // 16] for b in range(bt.B)])
    last = np.full(bt.B, 16, np.int32)
    ro, rl = oracle.partials(bt.q, bt.k, bt.v, indptr, indices, last, bt.Hq, bt.Hkv, nchunks, chunk_tokens)
    check_lse(pl.cpu().numpy(), rl, tag="prefix part_lse")
    check_out(po.cpu().numpy(), ro, tag="prefix part_o")
    assert lens


@pytest.mark.parametrize("B,Lp,chunk_tokens,scale",
                         [(64, 1024, 256, 1.0), (70, 640, 96, 1.0), (33, 512, 64, -2.0), (64, 8240, 8192, 1.0),
                          (48, 992, 160, 0.5), (32, 704, 128, 1.0), (40, 64, 64, 1.0)],
                         ids=["64 seqs, two full 128-row groups", "70 seqs, 128 + 128 + 24 rows, partial last chunk",
                              "33 seqs, 128 + 4 rows, negative scale", "64 seqs, 8192-token chunk + 48-token chunk",
                              "48 seqs, 128 + 64 rows, 3-block chunks with a partial block",
                              "32 seqs, 128 rows (the 4-wave body)", "40 seqs, one block per chunk"])
def test_prefix_kernel_full_query_groups(B, Lp, chunk_tokens, scale):
    """The prefix kernel with more than 128 query rows per kv head, which runs the 8-wave key-split
    body (128 rows per workgroup, the chunk's blocks split between two wave groups and combined in
    LDS): full groups (both tiles of every wave), ragged groups (24 and 4 rows: one tile of some
    waves; 64 rows: one tile of every wave), chunks of one block (the second wave group idle), two,
    three (the last partial, on the second group) and 128 blocks, and the 4-wave body at exactly
    128 rows; against the oracle's per-chunk partials."""
    _prefix_partials_vs_oracle(B, Lp, chunk_tokens, scale, 32, 8)


@pytest.mark.parametrize("Hq,Hkv,B,Lp,chunk_tokens",
                         [(64, 8, 20, 640, 128), (8, 2, 40, 512, 64), (64, 16, 40, 256, 16), (128, 16, 36, 320, 96)],
                         ids=["G8 160 rows", "Hkv2 G4 160 rows", "Hkv16 16-token chunks", "Hkv16 G8 288 rows"])
def test_prefix_key_split_head_layouts(Hq, Hkv, B, Lp, chunk_tokens):
    """The key-split body at other head layouts: G = 8; Hkv = 2, whose grid width (query groups x
    kv heads = 4) is not a multiple of the 8 XCDs; Hkv = 16 with 16-token chunks (one partial block,
    the second wave group idle); three query groups at G = 8; partial rows two columns wider than
    the chunks (part_stride = chunks + 2, the untouched columns must stay as they were); against the
    oracle's partials."""
    _prefix_partials_vs_oracle(B, Lp, chunk_tokens, 1.0, Hq, Hkv, pad=2)


def _prefix_partials_vs_oracle(B, Lp, chunk_tokens, scale, Hq, Hkv, pad=0):
    import torch
    import _gpu
    import pdattn
    print(f"[case] prefix kernel B={B} Lp={Lp} chunk_tokens={chunk_tokens} scale={scale} Hq={Hq} Hkv={Hkv}",
          flush=True)
    bt = inputs.make_shared_prefix_batch(Lp, [16] * B, Hq, Hkv, seed=30 + B)
    db = _gpu.DeviceBatch(bt)
    nchunks = (Lp + chunk_tokens - 1) // chunk_tokens
    rows = bt.B * bt.Hq
    d = torch.device("cuda:0")
    po = torch.full((rows, nchunks + pad, 128), float("nan"), dtype=torch.float32, device=d)
    pl = torch.full((rows, nchunks + pad), float("nan"), dtype=torch.float32, device=d)
    pp = pdattn.PrefixParams()
    pp.q, pp.k_cache, pp.v_cache = db.q.data_ptr(), db.k.data_ptr(), db.v.data_ptr()
    pp.prefix_pages = db.indices.data_ptr()
    pp.part_o, pp.part_lse = po.data_ptr(), pl.data_ptr()
    pp.B, pp.Hq, pp.Hkv = bt.B, bt.Hq, bt.Hkv
    pp.prefix_len, pp.chunk_tokens, pp.part_stride = Lp, chunk_tokens, nchunks + pad
    pp.sm_scale = scale / np.sqrt(128)
    pdattn.cascade_prefix(pp)
    torch.cuda.synchronize()
    if pad:
        assert torch.isnan(po[:, nchunks:]).all() and torch.isnan(pl[:, nchunks:]).all(), \
            "columns past the chunks were written"
        po, pl = po[:, :nchunks], pl[:, :nchunks]
    indptr = np.arange(bt.B + 1, dtype=np.int32) * (Lp // 16)
    indices = np.concatenate([bt.indices[bt.indptr[b]:bt.indptr[b] + Lp // 16] for b in range(bt.B)])
    last = np.full(bt.B, 16, np.int32)
    ro, rl = oracle.partials(bt.q, bt.k, bt.v, indptr, indices, last, bt.Hq, bt.Hkv, nchunks, chunk_tokens,
                             sm_scale=scale / np.sqrt(128))
    check_lse(pl.cpu().numpy(), rl, tag="prefix part_lse")
    check_out(po.cpu().numpy(), ro, tag="prefix part_o")


@pytest.mark.parametrize("B,chunk_tokens", [(1, 64), (2, 96), (4, 128), (5, 96), (8, 256)])
def test_small_groups_are_deterministic(B, chunk_tokens):
    """Query groups of 4 to 32 rows (B x 4 heads here), which leave query tiles of the
    workgroup empty: repeated launches give the same bits, and the partials match the oracle."""
    import torch
    import _gpu
    import pdattn
    Lp = 640
    print(f"small prefix group: B={B} chunk_tokens={chunk_tokens}", flush=True)
    bt = inputs.make_shared_prefix_batch(Lp, [16] * B, 32, 8, seed=8)
    db = _gpu.DeviceBatch(bt)
    nchunks = (Lp + chunk_tokens - 1) // chunk_tokens
    rows = bt.B * bt.Hq
    d = torch.device("cuda:0")
    po = torch.full((rows, nchunks, 128), float("nan"), dtype=torch.float32, device=d)
    pl = torch.full((rows, nchunks), float("nan"), dtype=torch.float32, device=d)
    pp = pdattn.PrefixParams()
    pp.q, pp.k_cache, pp.v_cache = db.q.data_ptr(), db.k.data_ptr(), db.v.data_ptr()
    pp.prefix_pages = db.indices.data_ptr()
    pp.part_o, pp.part_lse = po.data_ptr(), pl.data_ptr()
    pp.B, pp.Hq, pp.Hkv = bt.B, bt.Hq, bt.Hkv
    pp.prefix_len, pp.chunk_tokens, pp.part_stride = Lp, chunk_tokens, nchunks
    pp.sm_scale = 1.0 / np.sqrt(128)
    runs = []
    for _ in range(6):
        pdattn.cascade_prefix(pp)
        torch.cuda.synchronize()
        runs.append((po.clone(), pl.clone()))
    for o, l in runs[1:]:
        assert torch.equal(o.view(torch.int32), runs[0][0].view(torch.int32))
        assert torch.equal(l.view(torch.int32), runs[0][1].view(torch.int32))
    indptr = np.arange(bt.B + 1, dtype=np.int32) * (Lp // 16)
    indices = np.concatenate([bt.indices[bt.indptr[b]:bt.indptr[b] + Lp // 16] for b in range(bt.B)])
    last = np.full(bt.B, 16, np.int32)
    ro, rl = oracle.partials(bt.q, bt.k, bt.v, indptr, indices, last, bt.Hq, bt.Hkv, nchunks, chunk_tokens)
    check_lse(runs[0][1].cpu().numpy(), rl, tag="small group part_lse")
    check_out(runs[0][0].cpu().numpy(), ro, tag="small group part_o")


def test_unshared_batch_falls_back():
    """No shared pages: the plan reports use = 0 and the result equals plain decode
    (01_decode_attention.cu:810-815)."""
    import _gpu
    bt = inputs.make_batch([1000] * 4, 32, 8, seed=3)
    assert oracle.shared_prefix_pages(bt.indptr, bt.indices) == 0
    ro, rl = _ref(bt)
    o, l, info = _gpu.run_cascade(_gpu.DeviceBatch(bt), min_prefix=16)
    assert info.use == 0
    check_out(o, ro, tag="fallback")
    check_lse(l, rl, tag="fallback")


def test_short_prefix_below_min_prefix_falls_back():
    import _gpu
    bt = inputs.make_shared_prefix_batch(32, [10, 20], 8, 2, seed=3)
    ro, rl = _ref(bt)
    o, l, info = _gpu.run_cascade(_gpu.DeviceBatch(bt), min_prefix=256)
    assert info.use == 0
    check_out(o, ro)
    check_lse(l, rl)


# ---- multi-level cascade (shared-prefix tree) ----------------------------------------------------
# (label, nodes [(path, tokens)], sequences [(leaf path, private tokens)], Hq, Hkv, nodes, levels)
TREE_CASES = [
    ("two levels, two groups", [((0,), 64), ((0, 1), 128), ((0, 2), 32)],
     [((0, 1), 5), ((0, 1), 40), ((0, 2), 1), ((0,), 17), ((0, 2), 16)], 8, 2, 3, 2),
    ("three levels, G=4", [((0,), 256), ((0, 1), 512), ((0, 1, 2), 256), ((0, 3), 64)],
     [((0, 1, 2), 100), ((0, 1, 2), 3), ((0, 1), 50), ((0, 3), 7), ((0, 3), 300), ((0,), 1)],
     32, 8, 4, 3),
    ("forest of two roots", [((0,), 256), ((1,), 512)],
     [((0,), 10), ((0,), 20), ((1,), 5), ((1,), 300), ((), 77)], 32, 8, 2, 1),
    ("system prompt + 4 documents", [((0,), 1024)] + [((0, g), 512) for g in range(1, 5)],
     [((0, g), 64 + 17 * i) for g in range(1, 5) for i in range(4)], 32, 8, 5, 2),
    ("G=8 two levels", [((0,), 128), ((0, 1), 256), ((0, 2), 64)],
     [((0, 1), 9), ((0, 1), 100), ((0, 2), 33), ((0, 2), 1)], 32, 4, 3, 2),
    ("G=2 three levels", [((0,), 64), ((0, 1), 64), ((0, 1, 2), 128)],
     [((0, 1, 2), 5), ((0, 1, 2), 70), ((0, 1), 16), ((0,), 40)], 16, 8, 3, 3),
    ("MHA (G=1) forest", [((0,), 160), ((1,), 96), ((1, 2), 48)],
     [((0,), 3), ((0,), 200), ((1, 2), 7), ((1, 2), 31), ((1,), 12)], 8, 8, 3, 2),
    ("root of 70 requests: two query groups", [((0,), 512), ((0, 1), 256)],
     [((0, 1), 1 + i) for i in range(35)] + [((0,), 3 + i) for i in range(35)], 32, 8, 2, 2),
]


@pytest.mark.parametrize("case", TREE_CASES, ids=[c[0] for c in TREE_CASES])
def test_tree_cascade_matches_oracle(case):
    import _gpu
    label, nodes, seqs, Hq, Hkv, n_nodes, levels = case
    bt = inputs.make_prefix_tree_batch(nodes, seqs, Hq, Hkv, seed=51)
    print(f"tree cascade: {label}", flush=True)
    o, l, info = _gpu.run_cascade(_gpu.DeviceBatch(bt), min_prefix=16, tree=True)
    assert info.use == 1 and info.nodes == n_nodes and info.levels == levels
    ro, rl = _ref(bt)
    check_out(o, ro, tag=label)
    check_lse(l, rl, tag=label)


def test_tree_cascade_without_sharing_falls_back():
    import _gpu
    bt = inputs.make_batch([100, 37, 300], 32, 8, seed=52)
    o, l, info = _gpu.run_cascade(_gpu.DeviceBatch(bt), min_prefix=16, tree=True)
    assert info.use == 0 and info.nodes == 0
    ro, rl = _ref(bt)
    check_out(o, ro)
    check_lse(l, rl)


@pytest.mark.parametrize("Hkv", [8, 4], ids=["G4", "G8"])
@pytest.mark.parametrize("tree", [False, True], ids=["single-level", "tree"])
def test_cascade_modes_bitwise_equal(tree, Hkv):
    """The fused step (the default), separate launches on one stream, and the prefix forked onto a
    second stream: the same arithmetic, so the same bits; against the oracle. At G=8 the fused
    step's decode role uses its compact layout (the flush in two passes of 4 heads), which
    computes the same sums in the same order as the plain decode kernel's."""
    import torch

    import _gpu
    import pdattn
    if tree:
        nodes = [((0,), 256), ((0, 1), 512), ((0, 2), 128)]
        seqs = [((0, 1), 40), ((0, 1), 3), ((0, 2), 100), ((0, 2), 16), ((0,), 77)]
        bt = inputs.make_prefix_tree_batch(nodes, seqs, 32, Hkv, seed=61)
    else:
        bt = inputs.make_shared_prefix_batch(1024, [1] * 70, 32, Hkv, seed=62)
    db = _gpu.DeviceBatch(bt)
    print(f"cascade modes: tree={tree} G={bt.G}", flush=True)
    cp = pdattn.CascadePlan(db.params(), bt.indptr, bt.indices, bt.lens, db.indices, 16, tree)
    ws = pdattn.Workspace()
    got = []
    try:
        assert cp.info().use == 1 and cp.info().mode == pdattn.CASCADE_FUSED
        s = torch.cuda.current_stream()
        for mode in (pdattn.CASCADE_FUSED, pdattn.CASCADE_SERIAL, pdattn.CASCADE_TWO_STREAMS,
                     pdattn.CASCADE_FUSED):
            cp.set_mode(mode)
            db.out.fill_(float("nan"))
            db.lse.fill_(float("nan"))
            cp.decode(db.out, db.lse, ws, s)
            torch.cuda.synchronize()
            got.append((db.out.clone(), db.lse.clone()))
    finally:
        cp.close()
        pdattn.workspace_release(ws)
    for o, l in got[1:]:
        assert torch.equal(o.view(torch.int16), got[0][0].view(torch.int16))
        assert torch.equal(l.view(torch.int32), got[0][1].view(torch.int32))
    o = got[0][0].float().cpu().numpy().astype(np.float64)
    l = got[0][1].cpu().numpy().astype(np.float64)
    ro, rl = _ref(bt)
    check_out(o, ro)
    check_lse(l, rl)


def test_fused_mode_at_g8_and_unknown_mode():
    """At G=8 the fused step still fits two workgroups per CU (its decode role's compact layout):
    the plan defaults to it; every mode can be set; an unknown mode is refused."""
    import _gpu
    import pdattn
    bt = inputs.make_shared_prefix_batch(256, [5, 40, 17], 32, 4, seed=63)
    db = _gpu.DeviceBatch(bt)
    cp = pdattn.CascadePlan(db.params(), bt.indptr, bt.indices, bt.lens, db.indices, 16)
    try:
        assert cp.info().mode == pdattn.CASCADE_FUSED
        with pytest.raises(pdattn.PdattnError):
            cp.set_mode(7)
        cp.set_mode(pdattn.CASCADE_TWO_STREAMS)
        assert cp.info().mode == pdattn.CASCADE_TWO_STREAMS
        cp.set_mode(pdattn.CASCADE_SERIAL)
        assert cp.info().mode == pdattn.CASCADE_SERIAL
    finally:
        cp.close()
    o, l, info = _gpu.run_cascade(db, min_prefix=16)
    assert info.use == 1
    ro, rl = _ref(bt)
    check_out(o, ro)
    check_lse(l, rl)


@pytest.mark.parametrize("n,Hq,Hkv", [(3500, 8, 2), (1200, 32, 4)], ids=["G4", "G8"])
def test_many_short_sequences_grow_the_suffix_grid(n, Hq, Hkv):
    """n sequences of 1..16 private tokens behind a 64-token prefix: the (sequence, kv head) pairs
    need more than one suffix workgroup per CU (at most 24 segments each, 8 at G=8, where the
    fused step's decode role stages q rows for 8), so the fused step's prefix blocks start after a
    grid larger than the CU count."""
    import _gpu
    import pdattn
    rng = np.random.default_rng(64)
    suffix = [int(x) for x in rng.integers(1, 17, size=n)]
    bt = inputs.make_shared_prefix_batch(64, suffix, Hq, Hkv, seed=64)
    db = _gpu.DeviceBatch(bt)
    print(f"cascade: {n} short sequences G={bt.G}", flush=True)
    cp = pdattn.CascadePlan(db.params(), bt.indptr, bt.indices, bt.lens, db.indices, 16)
    info = cp.info()
    cp.close()
    assert info.use == 1 and info.mode == pdattn.CASCADE_FUSED
    assert info.suffix_workgroups > pdattn.device_info().compute_units
    o, l, info = _gpu.run_cascade(db, min_prefix=16)
    ro, rl = _ref(bt)
    check_out(o, ro)
    check_lse(l, rl)
