"""GPU tests of inputs outside the reference's happy path, through the C ABI, against the fp64 oracle.

* Cache slots that no key of the decode covers hold NaN / Inf bit patterns (the unused slots of
  every last page, which a cache allocated with torch.empty and filled by appends leaves as they
  were, and with kv_start the slots before it): the result must not see them, on every decode
  path (balanced plan, uniform split, its long-chunk kernel, the cascade's suffix).
* A negative, zero or large sm_scale (scores in the hundreds, a softmax close to an argmax):
  every path computes softmax(scale * q.k) as the oracle does.
* Plans and workspaces: a plan whose uploaded schedule another upload or launch has written over
  is refused (PDATTN_ERR_NOT_READY) or, for the cascade (which uploads by itself), re-uploaded;
  never run on someone else's schedule. A workspace the caller writes over itself (random bytes,
  or another plan's schedule copied in from torch), which the library cannot see, fails the tag
  check of the decode and merge kernels: the run writes nothing, and the plan is correct again
  after its next upload.
* An all-empty batch whose kv_indices points at the end of a buffer (no element): nothing reads
  it, and every row is 0 / -inf.
"""
import numpy as np
import pytest

import oracle
from _checks import check_lse, check_out
from pdattn import inputs

pytestmark = pytest.mark.gpu

SCALE = 1.0 / np.sqrt(128)


def _ref(bt, kv_start=0, sm_scale=None):
    return oracle.decode(bt.q, bt.k, bt.v, bt.indptr, bt.indices, bt.last, bt.Hq, bt.Hkv,
                         kv_start=kv_start, sm_scale=sm_scale, threads=8)


def _poison(bt, kv_start=0):
    """NaN and +Inf (alternating by slot) in K and V of every slot that holds no key of the
    decode: the tail of each sequence's last page and, with kv_start, every slot before it."""
    n = 0
    for b in range(bt.B):
        pb, pe = int(bt.indptr[b]), int(bt.indptr[b + 1])
        L = bt.lens[b]
        for j in range(pb, pe):
            pid = int(bt.indices[j])
            for slot in range(16):
                tok = (j - pb) * 16 + slot
                if tok >= L or tok < kv_start:
                    bad = np.float16(np.nan) if slot % 2 == 0 else np.float16(np.inf)
                    bt.k[pid, slot] = bad
                    bt.v[pid, slot] = bad
                    n += 1
    assert n > 0
    return n


POISON_LENS = [5, 300, 2049, 17, 1000]


@pytest.mark.parametrize("wg", [0, 7])
def test_poisoned_tails_balanced(wg):
    import _gpu
    print(f"[case] poisoned tails, balanced plan W={wg} lens={POISON_LENS}", flush=True)
    bt = inputs.make_batch(POISON_LENS, 32, 8, seed=31)
    ro, rl = _ref(bt)
    _poison(bt)
    o, l, info = _gpu.run_plan(_gpu.DeviceBatch(bt), wg)
    check_out(o, ro, tag=f"poisoned balanced W={info.workgroups}")
    check_lse(l, rl, tag=f"poisoned balanced W={info.workgroups}")


@pytest.mark.parametrize("force", [1, 7])
def test_poisoned_tails_uniform(force):
    import _gpu
    print(f"[case] poisoned tails, uniform split force={force}", flush=True)
    bt = inputs.make_batch(POISON_LENS, 32, 8, seed=32)
    ro, rl = _ref(bt)
    _poison(bt)
    o, l, nc = _gpu.run_uniform(_gpu.DeviceBatch(bt), force)
    check_out(o, ro, tag=f"poisoned uniform chunks={nc}")
    check_lse(l, rl, tag=f"poisoned uniform chunks={nc}")


@pytest.mark.parametrize("kv_start", [0, 5, 21])
def test_poisoned_tails_balanced_on_device(kv_start):
    """decode_attention_balanced (page ranges found on the device) with NaN / Inf in every slot
    it must not read: the last pages' tails and the slots before kv_start."""
    import _gpu
    print(f"[case] poisoned tails, device ranges kv_start={kv_start}", flush=True)
    bt = inputs.make_batch(POISON_LENS, 32, 8, seed=34)
    ro, rl = _ref(bt, kv_start=kv_start)
    _poison(bt, kv_start)
    o, l = _gpu.run_balanced(_gpu.DeviceBatch(bt), kv_start=kv_start)
    check_out(o, ro, tag=f"poisoned device ranges kv_start={kv_start}")
    check_lse(l, rl, tag=f"poisoned device ranges kv_start={kv_start}")


@pytest.mark.parametrize("kv_start,chunk_tokens", [(5, 40), (21, 64), (16, 48)])
def test_poisoned_before_kv_start(kv_start, chunk_tokens):
    """Partials with kv_start inside a page: the slots before it hold NaN / Inf."""
    import _gpu
    print(f"[case] poisoned before kv_start={kv_start} chunk_tokens={chunk_tokens}", flush=True)
    bt = inputs.make_batch([300, 129, 1000], 32, 8, seed=33)
    nc = (max(bt.lens) - kv_start + chunk_tokens - 1) // chunk_tokens
    rpo, rpl = oracle.partials(bt.q, bt.k, bt.v, bt.indptr, bt.indices, bt.last, bt.Hq, bt.Hkv,
                               nc, chunk_tokens, kv_start)
    _poison(bt, kv_start)
    po, pl = _gpu.run_partials(_gpu.DeviceBatch(bt), nc, chunk_tokens, kv_start)
    check_lse(pl, rpl, tag="poisoned partial lse")
    fin = ~np.isneginf(rpl)
    check_out(po[fin], rpo[fin], tag="poisoned partial o")


def test_poisoned_tail_long_chunk_kernel():
    """One chunk of more than 2047 pages runs on the one-chunk-per-workgroup kernel."""
    import _gpu
    print("[case] poisoned tail, 1 x 40007 tokens in one chunk", flush=True)
    bt = inputs.make_batch([40007], 32, 8, seed=34)
    ro, rl = _ref(bt)
    _poison(bt)
    o, l, nc = _gpu.run_uniform(_gpu.DeviceBatch(bt), 1)
    assert nc == 1
    check_out(o, ro, tag="poisoned long chunk")
    check_lse(l, rl, tag="poisoned long chunk")


def test_poisoned_tails_cascade():
    import _gpu
    print("[case] poisoned tails, cascade 256 + [5, 40, 17, 300]", flush=True)
    bt = inputs.make_shared_prefix_batch(256, [5, 40, 17, 300], 32, 8, seed=35)
    ro, rl = _ref(bt)
    _poison(bt)
    o, l, info = _gpu.run_cascade(_gpu.DeviceBatch(bt), min_prefix=16)
    assert info.use == 1
    check_out(o, ro, tag="poisoned cascade")
    check_lse(l, rl, tag="poisoned cascade")


# ---- sm_scale of any sign ----------------------------------------------------------------

def _cascade_with_scale(bt, db, scale, mode=None):
    import pdattn
    base = db.params()
    base.sm_scale = scale
    cp = pdattn.CascadePlan(base, bt.indptr, bt.indices, bt.lens, db.indices, 16)
    ws = pdattn.Workspace()
    try:
        if mode is not None:
            cp.set_mode(mode)
        cp.decode(db.out, db.lse, ws)
        o, l = db.results()
        info = cp.info()
    finally:
        cp.close()
        pdattn.workspace_release(ws)
    return o, l, info


@pytest.mark.parametrize("scale", [-SCALE, 0.0, -1.0, 1.0, 8.0])
def test_scale_sign_cascade_and_plan(scale):
    import torch
    import _gpu
    import pdattn
    print(f"[case] sm_scale={scale}: cascade (both modes), plan, uniform", flush=True)
    bt = inputs.make_shared_prefix_batch(320, [5, 40, 17, 300], 32, 8, seed=36)
    ro, rl = _ref(bt, sm_scale=scale)
    db = _gpu.DeviceBatch(bt)
    for mode in (pdattn.CASCADE_FUSED, pdattn.CASCADE_SERIAL):
        o, l, info = _cascade_with_scale(bt, db, scale, mode)
        assert info.use == 1
        check_out(o, ro, tag=f"cascade mode {mode} scale {scale}")
        check_lse(l, rl, tag=f"cascade mode {mode} scale {scale}")
    plan = pdattn.Plan(bt.indptr, bt.last, bt.B, bt.Hq, bt.Hkv, 7)
    ws = torch.empty(max(plan.workspace_bytes, 256), dtype=torch.uint8, device="cuda:0")
    plan.upload(ws, ws.numel())
    plan.run(db.q, db.k, db.v, db.indptr, db.indices, db.last, db.out, db.lse, ws, ws.numel(),
             sm_scale=scale)
    o, l = db.results()
    plan.close()
    check_out(o, ro, tag=f"plan scale {scale}")
    check_lse(l, rl, tag=f"plan scale {scale}")
    nc, ct = pdattn.plan_chunks(bt.G, bt.B, bt.Hkv, bt.max_len, 5)
    p = db.params(nc, ct)
    p.sm_scale = scale
    w = pdattn.Workspace()
    pdattn.decode_attention(p, bt.G, db.out, db.lse, w)
    o, l = db.results()
    pdattn.workspace_release(w)
    check_out(o, ro, tag=f"uniform scale {scale}")
    check_lse(l, rl, tag=f"uniform scale {scale}")


def test_scale_sign_prefix_kernel():
    """The MFMA prefix kernel alone with a negative scale and a chunk end inside a key block."""
    import torch
    import _gpu
    import pdattn
    print("[case] prefix kernel, negative scale, chunk_tokens 48", flush=True)
    Lp, ct = 208, 48
    bt = inputs.make_shared_prefix_batch(Lp, [3, 20, 50], 32, 8, seed=37)
    db = _gpu.DeviceBatch(bt)
    nchunks = (Lp + ct - 1) // ct
    rows = bt.B * bt.Hq
    d = torch.device("cuda:0")
    po = torch.full((rows, nchunks, 128), float("nan"), dtype=torch.float32, device=d)
    pl = torch.full((rows, nchunks), float("nan"), dtype=torch.float32, device=d)
    pp = pdattn.PrefixParams()
    pp.q, pp.k_cache, pp.v_cache = db.q.data_ptr(), db.k.data_ptr(), db.v.data_ptr()
    pp.prefix_pages = db.indices.data_ptr()
    pp.part_o, pp.part_lse = po.data_ptr(), pl.data_ptr()
    pp.B, pp.Hq, pp.Hkv = bt.B, bt.Hq, bt.Hkv
    pp.prefix_len, pp.chunk_tokens, pp.part_stride = Lp, ct, nchunks
    pp.sm_scale = -SCALE
    pdattn.cascade_prefix(pp)
    torch.cuda.synchronize()
    # the prefix keys of every sequence are its first Lp tokens: oracle partials over the page
    # table truncated to the prefix
    ind = np.concatenate([bt.indices[bt.indptr[b]:bt.indptr[b] + Lp // 16] for b in range(bt.B)])
    iptr = np.arange(bt.B + 1, dtype=np.int32) * (Lp // 16)
    last = np.full(bt.B, 16, np.int32)
    rpo, rpl = oracle.partials(bt.q, bt.k, bt.v, iptr, ind, last, bt.Hq, bt.Hkv, nchunks, ct,
                               sm_scale=-SCALE)
    gpo, gpl = po.cpu().numpy(), pl.cpu().numpy()
    check_lse(gpl, rpl, tag="prefix lse, negative scale")
    check_out(gpo, rpo, tag="prefix o, negative scale")


# ---- plans, uploads and shared workspaces --------------------------------------------------

def _plan_batch(lens, seed, wg):
    import _gpu
    import pdattn
    bt = inputs.make_batch(lens, 32, 8, seed=seed)
    db = _gpu.DeviceBatch(bt)
    plan = pdattn.Plan(bt.indptr, bt.last, bt.B, bt.Hq, bt.Hkv, wg)
    return bt, db, plan, _ref(bt)


def _run(plan, db, ws):
    plan.run(db.q, db.k, db.v, db.indptr, db.indices, db.last, db.out, db.lse, ws, ws.numel())
    return db.results()


def test_plan_overwritten_by_another_upload_is_refused():
    import torch
    import pdattn
    print("[case] plans A and B uploaded into one workspace", flush=True)
    btA, dbA, A, (roA, rlA) = _plan_batch([300, 5000, 17], 41, 64)
    btB, dbB, B, (roB, rlB) = _plan_batch([2048] * 3, 42, 64)
    n = max(A.workspace_bytes, B.workspace_bytes) + 4096
    ws = torch.zeros(n, dtype=torch.uint8, device="cuda:0")
    A.upload(ws, n)
    B.upload(ws, n)
    with pytest.raises(pdattn.PdattnError) as e:
        _run(A, dbA, ws)
    assert e.value.status == 6
    o, l = _run(B, dbB, ws)
    check_out(o, roB, tag="B after B's upload")
    check_lse(l, rlB, tag="B after B's upload")
    A.upload(ws, n)
    o, l = _run(A, dbA, ws)
    check_out(o, roA, tag="A after its re-upload")
    check_lse(l, rlA, tag="A after its re-upload")
    with pytest.raises(pdattn.PdattnError) as e:
        _run(B, dbB, ws)
    assert e.value.status == 6
    # B uploaded 256 bytes further on: its schedule overlaps A's, so A is refused
    wsB = ws[256:]
    B.upload(wsB, n - 256)
    with pytest.raises(pdattn.PdattnError) as e:
        _run(A, dbA, ws)
    assert e.value.status == 6
    o, l = _run(B, dbB, wsB)
    check_out(o, roB, tag="B at an offset")
    A.close()
    B.close()


def test_plan_overwritten_by_decode_attention_is_refused():
    import torch
    import pdattn
    print("[case] plan A uploaded, then decode_attention partials in the same memory", flush=True)
    btA, dbA, A, (roA, rlA) = _plan_batch([300, 5000, 17], 43, 64)
    btC = inputs.make_batch([4096, 4096], 32, 8, seed=44)
    import _gpu
    dbC = _gpu.DeviceBatch(btC)
    n = max(A.workspace_bytes, pdattn.decode_workspace_size(2, 32, 16)) + 4096
    ws = torch.zeros(n, dtype=torch.uint8, device="cuda:0")
    A.upload(ws, n)
    o, l = _run(A, dbA, ws)
    check_out(o, roA, tag="A")
    nc, ct = pdattn.plan_chunks(btC.G, btC.B, btC.Hkv, btC.max_len, 16)
    p = dbC.params(nc, ct)
    w = pdattn.Workspace(ws.data_ptr(), n, 0)   # the same memory, caller-provided
    pdattn.decode_attention(p, btC.G, dbC.out, dbC.lse, w)
    roC, rlC = _ref(btC)
    oc, lc = dbC.results()
    check_out(oc, roC, tag="decode_attention")
    with pytest.raises(pdattn.PdattnError) as e:
        _run(A, dbA, ws)
    assert e.value.status == 6
    A.close()


def test_cascade_plans_share_one_workspace():
    """Two cascade plans and a many-chunk decode_attention alternate on one pdattn_workspace;
    every call matches the oracle (the cascade re-uploads what the others overwrote)."""
    import _gpu
    import pdattn
    print("[case] cascade plans X, Y and decode_attention Z on one workspace", flush=True)
    btX = inputs.make_shared_prefix_batch(512, [5, 40, 17, 300], 32, 8, seed=45)
    btY = inputs.make_shared_prefix_batch(2048, [77] * 40, 32, 8, seed=46)
    btZ = inputs.make_batch([3000, 1000, 5000], 32, 8, seed=47)
    refs = {k: _ref(bt) for k, bt in (("X", btX), ("Y", btY), ("Z", btZ))}
    dbs = {"X": _gpu.DeviceBatch(btX), "Y": _gpu.DeviceBatch(btY), "Z": _gpu.DeviceBatch(btZ)}
    plans = {}
    for k, bt in (("X", btX), ("Y", btY)):
        plans[k] = pdattn.CascadePlan(dbs[k].params(), bt.indptr, bt.indices, bt.lens, dbs[k].indices, 16)
        assert plans[k].info().use == 1
    # reserved once at the largest size: every call below writes into the same memory
    nc, ct = pdattn.plan_chunks(btZ.G, btZ.B, btZ.Hkv, btZ.max_len, 40)
    need = max(plans["X"].info().workspace_bytes, plans["Y"].info().workspace_bytes,
               pdattn.decode_workspace_size(btZ.B, btZ.Hq, nc))
    ws = pdattn.Workspace()
    pdattn.workspace_reserve(ws, need)
    try:
        for k in ("X", "Y", "X", "Z", "Y", "X", "Z", "X"):
            db = dbs[k]
            if k == "Z":
                pdattn.decode_attention(db.params(nc, ct), btZ.G, db.out, db.lse, ws)
            else:
                plans[k].decode(db.out, db.lse, ws)
            o, l = db.results()
            check_out(o, refs[k][0], tag=f"{k} on a shared workspace")
            check_lse(l, refs[k][1], tag=f"{k} on a shared workspace")
    finally:
        for p in plans.values():
            p.close()
        pdattn.workspace_release(ws)


@pytest.mark.parametrize("what", ["random bytes", "another plan's schedule"])
def test_plan_workspace_written_by_the_caller(what):
    """The caller overwrites an uploaded plan's workspace with torch (unseen by the library's
    records): the run's kernels find a descriptor block and merge list without the plan's tag and
    leave out / lse as they were; after a new upload the plan is correct again."""
    import torch
    import pdattn
    print(f"[case] plan workspace overwritten from torch with {what}", flush=True)
    btA, dbA, A, (roA, rlA) = _plan_batch([300, 5000, 17], 48, 64)
    btB, dbB, B, _ = _plan_batch([2048] * 3, 49, 64)
    n = max(A.workspace_bytes, B.workspace_bytes) + 4096
    ws = torch.zeros(n, dtype=torch.uint8, device="cuda:0")
    A.upload(ws, n)
    o, l = _run(A, dbA, ws)
    check_out(o, roA, tag="A before")
    assert A.info().merge_entries > 0          # both kernels of the run are exercised
    if what == "random bytes":
        g = torch.Generator(device="cuda:0")
        g.manual_seed(50)
        ws.copy_(torch.randint(0, 256, (n,), dtype=torch.uint8, device="cuda:0", generator=g))
    else:
        ws2 = torch.zeros_like(ws)
        B.upload(ws2, n)
        torch.cuda.synchronize()
        ws.copy_(ws2)                            # B's schedule, where A's was
    dbA.out.fill_(7.0)
    dbA.lse.fill_(7.0)
    _run(A, dbA, ws)                             # the library's records still hold A's upload
    torch.cuda.synchronize()
    assert bool((dbA.out == 7.0).all()) and bool((dbA.lse == 7.0).all()), \
        "a run over someone else's bytes wrote results"
    A.upload(ws, n)
    o, l = _run(A, dbA, ws)
    check_out(o, roA, tag="A after its re-upload")
    check_lse(l, rlA, tag="A after its re-upload")
    A.close()
    B.close()


def test_all_empty_batch_with_an_empty_page_list():
    """Every sequence empty and kv_indices pointing just past the end of a buffer (no element):
    the uniform split (one chunk and several), the device-range drop-in, the plan path and
    decode_partial run without reading it, and every row is 0 / -inf."""
    import torch
    import pdattn
    print("[case] all-empty batch, kv_indices at the end of its buffer", flush=True)
    d = torch.device("cuda:0")
    B, Hq, Hkv = 5, 32, 8
    q = torch.randn(B, Hq, 128, device=d).half()
    k = torch.zeros(1, 16, Hkv, 128, dtype=torch.float16, device=d)
    v = torch.zeros_like(k)
    indptr = torch.zeros(B + 1, dtype=torch.int32, device=d)
    last = torch.zeros(B, dtype=torch.int32, device=d)
    holder = torch.zeros(64, dtype=torch.int32, device=d)
    indices = holder.data_ptr() + holder.numel() * 4   # no element: the address just past `holder`
    out = torch.empty(B, Hq, 128, dtype=torch.float16, device=d)
    lse = torch.empty(B, Hq, dtype=torch.float32, device=d)

    def check(tag):
        torch.cuda.synchronize()
        assert bool((out == 0).all()), tag
        assert bool(torch.isinf(lse).all()) and bool((lse < 0).all()), tag

    for nc in (1, 3):
        out.fill_(7.0)
        lse.fill_(7.0)
        p = pdattn.make_params(q, k, v, indptr, indices, last, B, Hq, Hkv, nc, 16)
        ws = pdattn.Workspace()
        try:
            pdattn.decode_attention(p, 4, out, lse, ws)
            check(f"decode_attention, {nc} chunks")
            out.fill_(7.0)
            lse.fill_(7.0)
            pdattn.decode_attention_balanced(p, 4, out, lse, ws)
            check(f"decode_attention_balanced, {nc} chunks")
        finally:
            pdattn.workspace_release(ws)
    plan = pdattn.Plan([0] * (B + 1), [0] * B, B, Hq, Hkv)
    wsp = torch.zeros(max(256, plan.workspace_bytes), dtype=torch.uint8, device=d)
    plan.upload(wsp, wsp.numel())
    out.fill_(7.0)
    lse.fill_(7.0)
    plan.run(q, k, v, indptr, indices, last, out, lse, wsp, wsp.numel())
    check("plan path")
    plan.close()
    po = torch.full((B * Hq, 2, 128), float("nan"), dtype=torch.float32, device=d)
    pl = torch.full((B * Hq, 2), float("nan"), dtype=torch.float32, device=d)
    p = pdattn.make_params(q, k, v, indptr, indices, last, B, Hq, Hkv, 2, 16, 0, 0, 2, None, po, pl)
    pdattn.decode_partial(p, 4)
    torch.cuda.synchronize()
    assert bool(torch.isinf(pl).all()) and bool((pl < 0).all())
    assert bool((po == 0).all())
