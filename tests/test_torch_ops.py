"""PyTorch operators over the C ABI (pdattn.torch_ops).

CPU: the operators are registered and their fake implementations give the right shapes (what
torch.compile traces with). GPU: torch.ops.pdattn.paged_decode equals the direct balanced path
bit for bit and the fp64 oracle within the parity bar; torch.ops.pdattn.append_kv writes the
caches like the host restatement; both trace into a full graph under torch.compile.
"""
import numpy as np
import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode

import oracle
import pdattn
import pdattn.torch_ops  # noqa: F401  (registers torch.ops.pdattn.*)
from pdattn import inputs

SCALE = float(1.0 / np.sqrt(128.0))   # a Python float: traced as a constant under torch.compile


def _inputs_on(dev, bt):
    t = lambda a, dt=None: torch.from_numpy(np.ascontiguousarray(a if dt is None else a.astype(dt))).to(dev)  # noqa: E731
    return (t(bt.q), t(bt.k), t(bt.v), t(bt.indptr, np.int32), t(bt.indices, np.int32),
            t(bt.last, np.int32), torch.from_numpy(bt.indptr.astype(np.int32)),
            torch.from_numpy(bt.last.astype(np.int32)))


def test_ops_registered():
    assert hasattr(torch.ops.pdattn, "paged_decode") and hasattr(torch.ops.pdattn, "append_kv")


def test_fake_shapes():
    bt = inputs.make_batch([40, 7], 32, 8, seed=1)
    with FakeTensorMode() as mode:
        args = [mode.from_tensor(x) for x in _inputs_on("cpu", bt)]
        out, lse = torch.ops.pdattn.paged_decode(*args, 0.088)
        assert out.shape == (2, 32, 128) and out.dtype == torch.float16
        assert lse.shape == (2, 32) and lse.dtype == torch.float32


@pytest.mark.gpu
def test_paged_decode_op_matches_plan_and_oracle():
    from _checks import check_lse, check_out
    from _gpu import DeviceBatch, run_plan
    bt = inputs.make_batch([3000, 1, 515, 0, 64], 32, 8, seed=41)
    q, k, v, ip, ix, la, iph, lah = _inputs_on("cuda:0", bt)
    print("op: paged_decode", flush=True)
    out, lse = torch.ops.pdattn.paged_decode(q, k, v, ip, ix, la, iph, lah, SCALE)
    torch.cuda.synchronize()
    db = DeviceBatch(bt)
    o_ref, l_ref, _ = run_plan(db)
    assert np.array_equal(out.float().cpu().numpy(), o_ref)
    assert np.array_equal(lse.cpu().numpy().astype(np.float64), l_ref)
    ro, rl = oracle.decode(bt.q, bt.k, bt.v, bt.indptr, bt.indices, bt.last, 32, 8, threads=8)
    check_out(out.float().cpu().numpy(), ro)
    check_lse(lse.cpu().numpy(), rl)


@pytest.mark.gpu
def test_append_op_and_compiled_step():
    from _checks import check_lse, check_out
    lens = [100, 1024, 17]
    bt = inputs.make_batch(lens, 32, 8, seed=42)
    q, k, v, ip, ix, la, iph, lah = _inputs_on("cuda:0", bt)
    rng = np.random.default_rng(43)
    k_new = rng.standard_normal((3, 8, 128)).astype(np.float16)
    v_new = rng.standard_normal((3, 8, 128)).astype(np.float16)
    kn, vn = torch.from_numpy(k_new).cuda(), torch.from_numpy(v_new).cuda()
    bidx = torch.arange(3, dtype=torch.int32, device="cuda")
    pos = torch.tensor([L - 1 for L in lens], dtype=torch.int32, device="cuda")

    def step(q, k, v, kn, vn):
        torch.ops.pdattn.append_kv(kn, vn, k, v, ip, ix, bidx, pos)
        return torch.ops.pdattn.paged_decode(q, k, v, ip, ix, la, iph, lah, SCALE)

    print("op: compiled append + decode", flush=True)
    compiled = torch.compile(step, backend="aot_eager", fullgraph=True)
    out, lse = compiled(q, k, v, kn, vn)
    torch.cuda.synchronize()
    kc, vc, _ = oracle.append_kv(bt.k, bt.v, k_new, v_new, np.arange(3), np.array(lens) - 1,
                                 bt.indptr, bt.indices)
    assert np.array_equal(k.cpu().numpy().view(np.uint16), kc.view(np.uint16))
    assert np.array_equal(v.cpu().numpy().view(np.uint16), vc.view(np.uint16))
    ro, rl = oracle.decode(bt.q, kc, vc, bt.indptr, bt.indices, bt.last, 32, 8, threads=8)
    check_out(out.float().cpu().numpy(), ro)
    check_lse(lse.cpu().numpy(), rl)
