"""GPU-side helpers for the parity tests: upload a batch, run each path through the C ABI.

Device memory and streams come from torch; every computation is a libpdattn call.
"""
import numpy as np
import torch

import pdattn


def device():
    if not torch.cuda.is_available():
        raise RuntimeError("this test needs a GPU (run with -m 'not gpu' on a CPU-only machine)")
    return torch.device("cuda:0")


class DeviceBatch:
    """Device copies of a Batch (the role of DeviceBatch, 01_decode_attention.cu:402-444)."""

    def __init__(self, bt):
        d = device()
        self.bt = bt
        self.q = torch.from_numpy(np.ascontiguousarray(bt.q)).to(d)
        if bt.num_pages > 0:
            self.k = torch.from_numpy(np.ascontiguousarray(bt.k)).to(d)
            self.v = torch.from_numpy(np.ascontiguousarray(bt.v)).to(d)
        else:  # keep valid pointers for an all-empty batch
            self.k = torch.zeros(1, 16, bt.Hkv, 128, dtype=torch.float16, device=d)
            self.v = torch.zeros_like(self.k)
        self.indptr = torch.from_numpy(bt.indptr.astype(np.int32)).to(d)
        idx = bt.indices.astype(np.int32) if bt.indices.size else np.zeros(1, np.int32)
        self.indices = torch.from_numpy(idx).to(d)
        lst = bt.last.astype(np.int32) if bt.last.size else np.zeros(1, np.int32)
        self.last = torch.from_numpy(lst).to(d)
        self.out = torch.empty(bt.B, bt.Hq, 128, dtype=torch.float16, device=d)
        self.lse = torch.empty(bt.B, bt.Hq, dtype=torch.float32, device=d)

    def params(self, num_chunks=1, chunk_tokens=16, kv_start=0, chunk_base=0, part_stride=None,
               part_o=None, part_lse=None):
        bt = self.bt
        return pdattn.make_params(self.q, self.k, self.v, self.indptr, self.indices, self.last,
                                  bt.B, bt.Hq, bt.Hkv, num_chunks, chunk_tokens, kv_start,
                                  chunk_base, part_stride, None, part_o, part_lse)

    def results(self):
        torch.cuda.synchronize()
        return (self.out.float().cpu().numpy().astype(np.float64),
                self.lse.cpu().numpy().astype(np.float64))


def run_uniform(db: DeviceBatch, force_chunks: int = 0):
    """decode_attention with the uniform chunk plan (01_decode_attention.cu:316-331)."""
    bt = db.bt
    nc, ct = pdattn.plan_chunks(bt.G, bt.B, bt.Hkv, bt.max_len, force_chunks)
    p = db.params(nc, ct)
    ws = pdattn.Workspace()
    try:
        pdattn.decode_attention(p, bt.G, db.out, db.lse, ws)
        o, l = db.results()
    finally:
        pdattn.workspace_release(ws)
    return o, l, nc


def run_balanced(db: DeviceBatch, force_chunks: int = 0, kv_start: int = 0, chunks=None):
    """decode_attention_balanced (the reference-shaped arguments, page ranges found on the
    device) with plan_chunks' chunking, or an explicit (num_chunks, chunk_tokens)."""
    bt = db.bt
    nc, ct = chunks if chunks else pdattn.plan_chunks(bt.G, bt.B, bt.Hkv, max(bt.max_len - kv_start, 0),
                                                      force_chunks)
    p = db.params(nc, ct, kv_start)
    ws = pdattn.Workspace()
    try:
        pdattn.decode_attention_balanced(p, bt.G, db.out, db.lse, ws)
        o, l = db.results()
    finally:
        pdattn.workspace_release(ws)
    return o, l


def run_plan(db: DeviceBatch, force_workgroups: int = 0):
    bt = db.bt
    plan = pdattn.Plan(bt.indptr, bt.last, bt.B, bt.Hq, bt.Hkv, force_workgroups)
    ws = torch.empty(max(plan.workspace_bytes, 256), dtype=torch.uint8, device=device())
    plan.upload(ws, ws.numel())
    plan.run(db.q, db.k, db.v, db.indptr, db.indices, db.last, db.out, db.lse, ws, ws.numel())
    o, l = db.results()
    info = plan.info()
    plan.close()
    return o, l, info


def run_partials(db: DeviceBatch, num_chunks: int, chunk_tokens: int, kv_start: int = 0):
    bt = db.bt
    rows = bt.B * bt.Hq
    po = torch.full((rows, num_chunks, 128), float("nan"), dtype=torch.float32, device=device())
    pl = torch.full((rows, num_chunks), float("nan"), dtype=torch.float32, device=device())
    p = db.params(num_chunks, chunk_tokens, kv_start, 0, num_chunks, po, pl)
    pdattn.decode_partial(p, bt.G)
    torch.cuda.synchronize()
    return po.cpu().numpy().astype(np.float64), pl.cpu().numpy().astype(np.float64)


def run_cascade(db: DeviceBatch, min_prefix: int = 256, tree: bool = False):
    bt = db.bt
    base = db.params()
    cp = pdattn.CascadePlan(base, bt.indptr, bt.indices, bt.lens, db.indices, min_prefix, tree)
    ws = pdattn.Workspace()
    try:
        cp.decode(db.out, db.lse, ws)
        o, l = db.results()
        info = cp.info()
    finally:
        cp.close()
        pdattn.workspace_release(ws)
    return o, l, info
