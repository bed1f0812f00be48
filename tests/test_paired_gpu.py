"""GPU parity of the paired decode kernel against the fp64 oracle, through the C ABI.

A default page-range plan at G <= 4 with an even Hkv is first built with two plan workgroups per
CU; when it splits no sequence, the decode launch runs plan workgroups w and w + 1 (kv heads 2k and
2k + 1 of the same page range) as one 4-wave workgroup whose pages go through LDS (info.paired).
Cases: the metric's 64x1K shape at G = 4, 2 and 1; many sequences per range (several segments per
workgroup); partial last pages with NaN / Inf in every slot past a sequence's end; Hkv = 2;
bitwise determinism; a workspace the caller wrote over (the kernel leaves out / lse alone); and
the shapes that must not be paired (a split sequence, G = 8, an odd Hkv).
"""
import numpy as np
import pytest

import oracle
from _checks import check_lse, check_out
from pdattn import inputs

pytestmark = pytest.mark.gpu


def _ref(bt):
    return oracle.decode(bt.q, bt.k, bt.v, bt.indptr, bt.indices, bt.last, bt.Hq, bt.Hkv, threads=8)


def _cus():
    import torch
    return torch.cuda.get_device_properties(0).multi_processor_count


def _need_256_cus():
    # which batches split depends on the grid (two plan workgroups per CU); the cases are sized
    # for MI355X's 256 CUs
    if _cus() != 256:
        pytest.skip(f"cases sized for 256 CUs, device has {_cus()}")


def _lens_partial(B, pages, seed):
    """B sequences of `pages` pages each, the last page holding 1..16 tokens."""
    rng = np.random.default_rng(seed)
    return [(pages - 1) * 16 + int(r) for r in rng.integers(1, 17, size=B)]


PAIRED = [
    ("64x1K G=4", [1024] * 64, 32, 8, 3),
    ("64x1K G=2", [1024] * 64, 16, 8, 4),
    ("64x1K G=1", [1024] * 64, 8, 8, 5),
    ("256x256, four segments per workgroup", [256] * 256, 32, 8, 6),
    ("128 x 32 pages, partial last pages", _lens_partial(128, 32, 7), 32, 8, 7),
    ("256x256 Hkv=2", [256] * 256, 8, 2, 8),
]


@pytest.mark.parametrize("name,lens,Hq,Hkv,seed", PAIRED, ids=[c[0] for c in PAIRED])
def test_paired_plan_parity(name, lens, Hq, Hkv, seed):
    import _gpu
    _need_256_cus()
    print(f"[case] paired plan: {name}", flush=True)
    bt = inputs.make_batch(lens, Hq, Hkv, seed=seed)
    ro, rl = _ref(bt)
    o, l, info = _gpu.run_plan(_gpu.DeviceBatch(bt))
    assert info.paired == 1 and info.merge_entries == 0, (info.paired, info.merge_entries)
    assert info.workgroups == 2 * _cus()
    check_out(o, ro, tag=name)
    check_lse(l, rl, tag=name)


def test_paired_poisoned_tails():
    """NaN / +Inf in K and V of every slot past a sequence's end (the unused tail of its last
    page): masked keys must not reach the output through 0 * v."""
    import _gpu
    _need_256_cus()
    print("[case] paired plan, poisoned tails", flush=True)
    bt = inputs.make_batch(_lens_partial(128, 32, 9), 32, 8, seed=9)
    ro, rl = _ref(bt)
    n = 0
    for b in range(bt.B):
        pb, pe, L = int(bt.indptr[b]), int(bt.indptr[b + 1]), bt.lens[b]
        for j in range(pb, pe):
            for slot in range(16):
                if (j - pb) * 16 + slot >= L:
                    bad = np.float16(np.nan) if slot % 2 == 0 else np.float16(np.inf)
                    bt.k[int(bt.indices[j]), slot] = bad
                    bt.v[int(bt.indices[j]), slot] = bad
                    n += 1
    assert n > 0
    o, l, info = _gpu.run_plan(_gpu.DeviceBatch(bt))
    assert info.paired == 1
    check_out(o, ro, tag="paired, poisoned tails")
    check_lse(l, rl, tag="paired, poisoned tails")


def test_paired_deterministic():
    import _gpu
    _need_256_cus()
    print("[case] paired plan, two runs bitwise equal", flush=True)
    bt = inputs.make_batch([1024] * 64, 32, 8, seed=10)
    db = _gpu.DeviceBatch(bt)
    o1, l1, info = _gpu.run_plan(db)
    o2, l2, _ = _gpu.run_plan(db)
    assert info.paired == 1
    assert np.array_equal(o1, o2) and np.array_equal(l1, l2)


@pytest.mark.parametrize("what", ["random bytes", "another plan's schedule"])
def test_paired_workspace_written_by_the_caller(what):
    """The caller overwrites a paired plan's uploaded workspace (unseen by the library's records):
    both heads' descriptor blocks lack the plan's tag, so the kernel writes nothing; after a new
    upload the plan is correct again."""
    import torch
    import _gpu
    import pdattn
    _need_256_cus()
    print(f"[case] paired plan workspace overwritten with {what}", flush=True)
    btA = inputs.make_batch([1024] * 64, 32, 8, seed=11)
    btB = inputs.make_batch([256] * 256, 32, 8, seed=12)
    dbA = _gpu.DeviceBatch(btA)
    roA, rlA = _ref(btA)
    A = pdattn.Plan(btA.indptr, btA.last, btA.B, btA.Hq, btA.Hkv)
    B = pdattn.Plan(btB.indptr, btB.last, btB.B, btB.Hq, btB.Hkv)
    assert A.info().paired == 1 and B.info().paired == 1
    n = max(A.workspace_bytes, B.workspace_bytes) + 4096
    ws = torch.zeros(n, dtype=torch.uint8, device="cuda:0")

    def run():
        A.run(dbA.q, dbA.k, dbA.v, dbA.indptr, dbA.indices, dbA.last, dbA.out, dbA.lse, ws, n)
        return dbA.results()

    A.upload(ws, n)
    o, l = run()
    check_out(o, roA, tag="A before")
    if what == "random bytes":
        g = torch.Generator(device="cuda:0")
        g.manual_seed(13)
        ws.copy_(torch.randint(0, 256, (n,), dtype=torch.uint8, device="cuda:0", generator=g))
    else:
        ws2 = torch.zeros_like(ws)
        B.upload(ws2, n)
        torch.cuda.synchronize()
        ws.copy_(ws2)
    dbA.out.fill_(7.0)
    dbA.lse.fill_(7.0)
    run()
    torch.cuda.synchronize()
    assert bool((dbA.out == 7.0).all()) and bool((dbA.lse == 7.0).all()), \
        "a paired run over someone else's bytes wrote results"
    A.upload(ws, n)
    o, l = run()
    check_out(o, roA, tag="A after its re-upload")
    check_lse(l, rlA, tag="A after its re-upload")
    A.close()
    B.close()


NOT_PAIRED = [
    ("1x32K (the paired plan would split it)", [32768], 32, 8, 14),
    ("G=8", [1024] * 64, 64, 8, 15),
    ("odd Hkv", [1024] * 64, 12, 3, 16),
]


@pytest.mark.parametrize("name,lens,Hq,Hkv,seed", NOT_PAIRED, ids=[c[0] for c in NOT_PAIRED])
def test_not_paired(name, lens, Hq, Hkv, seed):
    import _gpu
    print(f"[case] unpaired plan: {name}", flush=True)
    bt = inputs.make_batch(lens, Hq, Hkv, seed=seed)
    ro, rl = _ref(bt)
    o, l, info = _gpu.run_plan(_gpu.DeviceBatch(bt))
    assert info.paired == 0
    check_out(o, ro, tag=name)
    check_lse(l, rl, tag=name)
