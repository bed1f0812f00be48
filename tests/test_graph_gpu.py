"""Graph capture of whole decode steps (HIP graphs through torch.cuda.graph).

Each run path, once its plan is uploaded and its workspace reserved, launches kernels only: no
allocation, no host synchronization, no memset. So a step can be captured into a graph and
replayed. Every test here replays the graph several times, with eager work (clearing the outputs)
and synchronizations in between, and checks every replay bit for bit against the eager result of
the same call, which is itself checked against the fp64 oracle.
"""
import numpy as np
import pytest
import torch

import oracle
import pdattn
from _checks import check_lse, check_out
from _gpu import DeviceBatch, device
from pdattn import inputs

pytestmark = pytest.mark.gpu

REPLAYS = 4


def _replay_and_compare(g, db, ref_o, ref_l, tag):
    for i in range(REPLAYS):
        db.out.fill_(float("nan"))
        db.lse.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(db.out.view(torch.int16), ref_o.view(torch.int16)), f"{tag}: replay {i} out differs"
        assert torch.equal(db.lse.view(torch.int32), ref_l.view(torch.int32)), f"{tag}: replay {i} lse differs"


def _check_oracle(db, bt):
    o, l = db.results()
    ro, rl = oracle.decode(bt.q, bt.k, bt.v, bt.indptr, bt.indices, bt.last, bt.Hq, bt.Hkv, threads=8)
    check_out(o, ro)
    check_lse(l, rl)


def test_plan_run_graph():
    bt = inputs.make_batch([3000, 17, 1000, 64, 0, 515], 32, 8, seed=31)
    db = DeviceBatch(bt)
    print("graph: plan_run", flush=True)
    plan = pdattn.Plan(bt.indptr, bt.last, bt.B, bt.Hq, bt.Hkv, force_workgroups=16, chunk_pages=16)
    ws = torch.empty(max(256, plan.workspace_bytes), dtype=torch.uint8, device=device())
    s = torch.cuda.current_stream()
    plan.upload(ws, ws.numel(), s)
    run = lambda st: plan.run(db.q, db.k, db.v, db.indptr, db.indices, db.last, db.out, db.lse,  # noqa: E731
                              ws, ws.numel(), stream=st)
    run(s)
    torch.cuda.synchronize()
    _check_oracle(db, bt)
    ref_o, ref_l = db.out.clone(), db.lse.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        run(torch.cuda.current_stream())
    _replay_and_compare(g, db, ref_o, ref_l, "plan_run")
    plan.close()


def test_cascade_graph():
    bt = inputs.make_shared_prefix_batch(1024, [77, 300, 5, 16], 32, 8, seed=32)
    db = DeviceBatch(bt)
    print("graph: cascade", flush=True)
    cp = pdattn.CascadePlan(db.params(), bt.indptr, bt.indices, bt.lens, db.indices, 256)
    assert cp.info().use == 1
    ws = pdattn.Workspace()
    s = torch.cuda.current_stream()
    cp.decode(db.out, db.lse, ws, s)       # eager call: reserves the workspace, uploads the schedule
    torch.cuda.synchronize()
    _check_oracle(db, bt)
    ref_o, ref_l = db.out.clone(), db.lse.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        cp.decode(db.out, db.lse, ws, torch.cuda.current_stream())
    _replay_and_compare(g, db, ref_o, ref_l, "cascade")
    cp.close()
    pdattn.workspace_release(ws)


def test_cascade_two_streams_graph():
    """The cascade with its prefix launch forked onto the plan's second stream: the fork / join
    events are captured into the graph along with the launches. (test_cascade_graph covers the
    default fused step.)"""
    bt = inputs.make_shared_prefix_batch(512, [40, 1, 300, 17, 64], 32, 8, seed=36)
    db = DeviceBatch(bt)
    print("graph: cascade, two streams", flush=True)
    cp = pdattn.CascadePlan(db.params(), bt.indptr, bt.indices, bt.lens, db.indices, 256)
    assert cp.info().use == 1
    cp.set_mode(pdattn.CASCADE_TWO_STREAMS)
    ws = pdattn.Workspace()
    s = torch.cuda.current_stream()
    cp.decode(db.out, db.lse, ws, s)
    torch.cuda.synchronize()
    _check_oracle(db, bt)
    ref_o, ref_l = db.out.clone(), db.lse.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        cp.decode(db.out, db.lse, ws, torch.cuda.current_stream())
    _replay_and_compare(g, db, ref_o, ref_l, "cascade two streams")
    cp.close()
    pdattn.workspace_release(ws)


def test_uniform_decode_attention_graph():
    bt = inputs.make_batch([2048, 100, 1], 16, 4, seed=33)
    db = DeviceBatch(bt)
    print("graph: decode_attention", flush=True)
    nc, ct = pdattn.plan_chunks(bt.G, bt.B, bt.Hkv, bt.max_len, force_chunks=7)
    p = db.params(nc, ct)
    ws = pdattn.Workspace()
    pdattn.workspace_reserve(ws, pdattn.decode_workspace_size(bt.B, bt.Hq, nc))
    s = torch.cuda.current_stream()
    pdattn.decode_attention(p, bt.G, db.out, db.lse, ws, s)
    torch.cuda.synchronize()
    _check_oracle(db, bt)
    ref_o, ref_l = db.out.clone(), db.lse.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        pdattn.decode_attention(p, bt.G, db.out, db.lse, ws, torch.cuda.current_stream())
    _replay_and_compare(g, db, ref_o, ref_l, "decode_attention")
    pdattn.workspace_release(ws)


def test_balanced_decode_attention_graph():
    bt = inputs.make_batch([300, 5000, 17, 2048], 32, 8, seed=35)
    db = DeviceBatch(bt)
    print("graph: decode_attention_balanced", flush=True)
    nc, ct = pdattn.plan_chunks(bt.G, bt.B, bt.Hkv, bt.max_len, 0)
    p = db.params(nc, ct)
    ws = pdattn.Workspace()
    pdattn.workspace_reserve(ws, pdattn.decode_balanced_workspace_size(p, bt.G))
    s = torch.cuda.current_stream()
    pdattn.decode_attention_balanced(p, bt.G, db.out, db.lse, ws, s)
    torch.cuda.synchronize()
    _check_oracle(db, bt)
    ref_o, ref_l = db.out.clone(), db.lse.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        pdattn.decode_attention_balanced(p, bt.G, db.out, db.lse, ws, torch.cuda.current_stream())
    _replay_and_compare(g, db, ref_o, ref_l, "decode_attention_balanced")
    pdattn.workspace_release(ws)


def test_append_then_decode_graph():
    """A serving step as one graph: append each sequence's newest token, then decode."""
    lens = [700, 33, 1024]
    bt = inputs.make_batch(lens, 32, 8, seed=34)
    db = DeviceBatch(bt)
    print("graph: append + decode", flush=True)
    d = device()
    rng = np.random.default_rng(35)
    k_new = rng.standard_normal((3, 8, 128)).astype(np.float16)
    v_new = rng.standard_normal((3, 8, 128)).astype(np.float16)
    kn, vn = torch.from_numpy(k_new).to(d), torch.from_numpy(v_new).to(d)
    bidx = torch.arange(3, dtype=torch.int32, device=d)
    pos = torch.tensor([L - 1 for L in lens], dtype=torch.int32, device=d)
    plan = pdattn.Plan(bt.indptr, bt.last, bt.B, bt.Hq, bt.Hkv)
    ws = torch.empty(max(256, plan.workspace_bytes), dtype=torch.uint8, device=d)
    s = torch.cuda.current_stream()
    plan.upload(ws, ws.numel(), s)

    def step(st):
        pdattn.append_kv(kn, vn, db.k, db.v, db.indptr, db.indices, bidx, pos, bt.B, 8, stream=st)
        plan.run(db.q, db.k, db.v, db.indptr, db.indices, db.last, db.out, db.lse, ws, ws.numel(),
                 stream=st)
    step(s)
    torch.cuda.synchronize()
    kc, vc, _ = oracle.append_kv(bt.k, bt.v, k_new, v_new, np.arange(3), np.array(lens) - 1,
                                 bt.indptr, bt.indices)
    o, l = db.results()
    ro, rl = oracle.decode(bt.q, kc, vc, bt.indptr, bt.indices, bt.last, 32, 8)
    check_out(o, ro)
    check_lse(l, rl)
    ref_o, ref_l = db.out.clone(), db.lse.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step(torch.cuda.current_stream())
    _replay_and_compare(g, db, ref_o, ref_l, "append+decode")
    plan.close()
