"""GPU tests on a KV cache larger than 4 GiB per tensor, through the C ABI, against the fp64 oracle.

A device holds caches of tens of GB, so page ids reach far past 2^17 (32 KB pages, byte offsets
past 4 GiB) and past 2^31 bytes of any 32-bit offset. Each case builds an ordinary small batch,
moves its pages to ids spread over a 200,000-page cache (6.5 GB each for K and V: most ids above
131,072, and the last page of the cache among them), and checks every path against the oracle
run on the small batch with the original ids:

* the plan path (page-range plan) and the reference-shaped uniform split;
* the shared-prefix cascade (its prefix pages at large ids);
* the paged append into large-id pages, compared byte for byte, then a decode that reads them.

Pages of the big cache that the batch does not use are never written: a wrong offset would read
other bytes, not the batch's.
"""
import numpy as np
import pytest
import torch

import oracle
import pdattn
from _checks import check_lse, check_out
from pdattn import inputs

pytestmark = pytest.mark.gpu

BIG_PAGES = 200_000          # x 32 KB = 6.55 GB per cache at Hkv = 8
HKV = 8


def _big_ids(n, seed):
    """n distinct page ids of the big cache: random, and the last page of the cache."""
    rng = np.random.default_rng(seed)
    ids = rng.choice(BIG_PAGES - 1, size=n, replace=False).astype(np.int64)
    ids[rng.integers(n)] = BIG_PAGES - 1
    assert (ids >= 131_072).sum() > n // 4
    return ids


class BigCache:
    """Device caches of BIG_PAGES pages holding the small batch's pages at ids `ids`."""

    def __init__(self, bt, seed):
        assert bt.Hkv == HKV
        d = torch.device("cuda:0")
        self.ids = _big_ids(bt.num_pages, seed)
        self.k = torch.empty(BIG_PAGES, 16, HKV, 128, dtype=torch.float16, device=d)
        self.v = torch.empty_like(self.k)
        idx = torch.from_numpy(self.ids).to(d)
        self.k[idx] = torch.from_numpy(np.ascontiguousarray(bt.k)).to(d)
        self.v[idx] = torch.from_numpy(np.ascontiguousarray(bt.v)).to(d)
        self.indices_host = self.ids[bt.indices].astype(np.int32)
        self.q = torch.from_numpy(np.ascontiguousarray(bt.q)).to(d)
        self.indptr = torch.from_numpy(bt.indptr.astype(np.int32)).to(d)
        self.indices = torch.from_numpy(self.indices_host).to(d)
        self.last = torch.from_numpy(bt.last.astype(np.int32)).to(d)
        self.out = torch.empty(bt.B, bt.Hq, 128, dtype=torch.float16, device=d)
        self.lse = torch.empty(bt.B, bt.Hq, dtype=torch.float32, device=d)
        pdattn.check_page_table(bt.indptr, self.indices_host, bt.last, BIG_PAGES)   # raises if not

    def results(self):
        torch.cuda.synchronize()
        return (self.out.float().cpu().numpy().astype(np.float64),
                self.lse.cpu().numpy().astype(np.float64))

    def close(self):
        del self.k, self.v
        torch.cuda.empty_cache()


def _ref(bt):
    return oracle.decode(bt.q, bt.k, bt.v, bt.indptr, bt.indices, bt.last, bt.Hq, bt.Hkv, threads=8)


@pytest.fixture(scope="module")
def decode_case():
    lens = [7000, 33, 1, 2048, 517, 0, 3000]
    bt = inputs.make_batch(lens, 32, HKV, seed=41)
    print(f"[case] large cache decode lens={lens} pages={bt.num_pages}", flush=True)
    big = BigCache(bt, seed=42)
    yield bt, big, _ref(bt)
    big.close()


def test_plan_path_on_large_cache(decode_case):
    bt, big, (ro, rl) = decode_case
    plan = pdattn.Plan(bt.indptr, bt.last, bt.B, bt.Hq, bt.Hkv)
    ws = torch.empty(max(plan.workspace_bytes, 256), dtype=torch.uint8, device="cuda:0")
    plan.upload(ws, ws.numel())
    plan.run(big.q, big.k, big.v, big.indptr, big.indices, big.last, big.out, big.lse, ws, ws.numel())
    o, l = big.results()
    plan.close()
    check_out(o, ro, tag="large cache plan")
    check_lse(l, rl, tag="large cache plan")


@pytest.mark.parametrize("force_chunks", [0, 1])
def test_uniform_split_on_large_cache(decode_case, force_chunks):
    """decode_attention: the uniform split, with the planned chunk count and with one chunk per
    sequence (every pair whole, out / lse written by the partial launch itself)."""
    bt, big, (ro, rl) = decode_case
    nc, ct = pdattn.plan_chunks(bt.G, bt.B, bt.Hkv, bt.max_len, force_chunks)
    p = pdattn.make_params(big.q, big.k, big.v, big.indptr, big.indices, big.last, bt.B, bt.Hq,
                           bt.Hkv, nc, ct)
    ws = pdattn.Workspace()
    try:
        pdattn.decode_attention(p, bt.G, big.out, big.lse, ws)
        o, l = big.results()
    finally:
        pdattn.workspace_release(ws)
    check_out(o, ro, tag=f"large cache uniform nc={nc}")
    check_lse(l, rl, tag=f"large cache uniform nc={nc}")


def test_cascade_on_large_cache():
    bt = inputs.make_shared_prefix_batch(4096, [300, 17, 900, 64] * 4, 32, HKV, seed=43)
    print(f"[case] large cache cascade B={bt.B} pages={bt.num_pages}", flush=True)
    ro, rl = _ref(bt)
    big = BigCache(bt, seed=44)
    try:
        base = pdattn.make_params(big.q, big.k, big.v, big.indptr, big.indices, big.last, bt.B,
                                  bt.Hq, bt.Hkv)
        cp = pdattn.CascadePlan(base, bt.indptr, big.indices_host, bt.lens, big.indices)
        assert cp.info().use == 1
        ws = pdattn.Workspace()
        for mode in (pdattn.CASCADE_FUSED, pdattn.CASCADE_SERIAL):
            cp.set_mode(mode)
            cp.decode(big.out, big.lse, ws)
            o, l = big.results()
            check_out(o, ro, tag=f"large cache cascade mode {mode}")
            check_lse(l, rl, tag=f"large cache cascade mode {mode}")
        cp.close()
        pdattn.workspace_release(ws)
    finally:
        big.close()


def test_append_then_decode_on_large_cache():
    """Append one token to each sequence (into pages at large ids), compare the written pages
    byte for byte with the restatement, then decode over them."""
    lens_after = [129, 16, 1000, 1]
    bt = inputs.make_batch(lens_after, 32, HKV, seed=45)
    print(f"[case] large cache append lens={lens_after}", flush=True)
    rng = np.random.default_rng(46)
    k_new = rng.standard_normal((bt.B, HKV, 128)).astype(np.float16)
    v_new = rng.standard_normal((bt.B, HKV, 128)).astype(np.float16)
    pos = np.array([L - 1 for L in lens_after], np.int32)
    kc, vc, bad = oracle.append_kv(bt.k, bt.v, k_new, v_new, np.arange(bt.B), pos, bt.indptr,
                                   bt.indices)
    assert bad == 0
    big = BigCache(bt, seed=47)
    try:
        d = torch.device("cuda:0")
        nbad = torch.zeros(1, dtype=torch.int32, device=d)
        pdattn.append_kv(torch.from_numpy(k_new).to(d), torch.from_numpy(v_new).to(d), big.k, big.v,
                         big.indptr, big.indices,
                         torch.arange(bt.B, dtype=torch.int32, device=d),
                         torch.from_numpy(pos).to(d), bt.B, HKV, nbad)
        torch.cuda.synchronize()
        assert int(nbad.item()) == 0
        idx = torch.from_numpy(big.ids).to(d)
        got_k = big.k[idx].cpu().numpy()
        got_v = big.v[idx].cpu().numpy()
        assert np.array_equal(got_k.view(np.uint16), kc.view(np.uint16))
        assert np.array_equal(got_v.view(np.uint16), vc.view(np.uint16))
        ro, rl = oracle.decode(bt.q, kc, vc, bt.indptr, bt.indices, bt.last, bt.Hq, bt.Hkv, threads=8)
        plan = pdattn.Plan(bt.indptr, bt.last, bt.B, bt.Hq, bt.Hkv)
        ws = torch.empty(max(plan.workspace_bytes, 256), dtype=torch.uint8, device=d)
        plan.upload(ws, ws.numel())
        plan.run(big.q, big.k, big.v, big.indptr, big.indices, big.last, big.out, big.lse, ws,
                 ws.numel())
        o, l = big.results()
        plan.close()
        check_out(o, ro, tag="large cache append+decode")
        check_lse(l, rl, tag="large cache append+decode")
    finally:
        big.close()
