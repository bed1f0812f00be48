"""Benchmark of the paged split-KV GQA decode attention on one MI355X.

A "step" is one decode-attention launch over one batch already resident in HBM: the balanced
single-launch path (pdattn_plan_run), H_q=32, H_kv=8, d=128, page 16, fp16 q/K/V ~ N(0,1) with
shuffled pages (seeded).

Two timings, both cold-cache:
  * value / ms_per_step -- the reference's method (common/bench.cuh:144-175): before every step a
    1 GiB buffer (4x the 256 MB Infinity Cache) is read by a flush kernel, each step is bracketed
    by HIP events on the stream the kernel runs on, methods are interleaved, and the median is
    reported. The event pair includes the dispatch of the kernel after the first event.
  * roofline.achieved -- the kernel's average launch duration: K launches back to back between one
    event pair, each over its own copy of K/V (copies totalling >= 1 GiB, so every launch reads
    lines that have left the caches). This is what a trace of the kernel reports as its duration.

Headline workload: B=1, L=32768; `value` is its achieved HBM GB/s
(algorithmic bytes / median step time). The same line carries the 64 x 1K workload the metric also
names, the streaming-read ceiling, the cascade comparison and the CPU oracle baseline.
"""
import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "cuda-kernel-lab_amd"))

PEAK_GBS = 8000.0
FLUSH_BYTES = 1 << 30
METRIC = "decode-attn µs/step + achieved HBM GB/s (% of 8 TB/s) at 1×32K and 64×1K"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-secondary", action="store_true")
    ap.add_argument("--only", default="", choices=["", "32k", "64x1k", "cascade", "cascade8", "prefix", "append",
                                                   "graph", "tree", "legs"],
                    help="run one workload only (for profiling)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run only torch copies of COPY_BYTES (known-size traffic for counter runs)")
    ap.add_argument("--timeline", default="", choices=["", "32k", "64x1k", "prefix", "cascade"],
                    help="per-workgroup phase timestamps from the timeline build of the library "
                         "(make -C cuda-kernel-lab_amd timeline) instead of the bench")
    return ap.parse_args()


def make_device_batch(lens, Hq, Hkv, seed, shared_prefix=0, suffix=None):
    """Page table on the host (seeded permutation), q/K/V ~ N(0,1) generated on the device."""
    import torch
    from pdattn import inputs
    if shared_prefix:
        bt = inputs.make_shared_prefix_batch(shared_prefix, suffix, Hq, Hkv, seed, fill=False)
    else:
        bt = inputs.make_batch(lens, Hq, Hkv, seed, fill=False)
    d = torch.device("cuda:0")
    g = torch.Generator(device=d)
    g.manual_seed(seed)
    q = torch.randn(bt.B, Hq, 128, generator=g, device=d, dtype=torch.float32).half()
    k = torch.randn(bt.num_pages, 16, Hkv, 128, generator=g, device=d, dtype=torch.float32).half()
    v = torch.randn(bt.num_pages, 16, Hkv, 128, generator=g, device=d, dtype=torch.float32).half()
    t = dict(
        q=q, k=k, v=v,
        indptr=torch.from_numpy(bt.indptr).to(d), indices=torch.from_numpy(bt.indices).to(d),
        last=torch.from_numpy(bt.last).to(d),
        out=torch.empty(bt.B, Hq, 128, dtype=torch.float16, device=d),
        lse=torch.empty(bt.B, Hq, dtype=torch.float32, device=d),
    )
    return bt, t


class Timer:
    """Cold-cache timing: flush, event, launch, event; medians over interleaved methods."""

    def __init__(self):
        import torch
        import pdattn
        self.torch = torch
        self.pdattn = pdattn
        self.stream = torch.cuda.current_stream()
        self.flush_buf = torch.empty(FLUSH_BYTES, dtype=torch.uint8, device="cuda:0")

    def flush(self):
        self.pdattn.flush_cache(self.flush_buf, FLUSH_BYTES, self.stream)

    def run(self, fns, steps, warmup, rounds=1):
        """fns: list of callables launching on self.stream. Returns per-method lists of ms."""
        torch = self.torch
        for fn in fns:
            for _ in range(warmup):
                self.flush()
                fn()
        torch.cuda.synchronize()
        times = [[] for _ in fns]
        # exactly `steps` timed steps per method, spread over the rounds
        counts = [steps // rounds + (1 if r < steps % rounds else 0) for r in range(rounds)]
        for r in range(rounds):
            for m, fn in enumerate(fns):
                evs = []
                for _ in range(counts[r]):
                    self.flush()
                    e0 = torch.cuda.Event(enable_timing=True)
                    e1 = torch.cuda.Event(enable_timing=True)
                    e0.record(self.stream)
                    fn()
                    e1.record(self.stream)
                    evs.append((e0, e1))
                torch.cuda.synchronize()
                times[m].extend(e0.elapsed_time(e1) for e0, e1 in evs)
        return times


def plan_runner(bt, t, stream):
    import torch
    import pdattn
    plan = pdattn.Plan(bt.indptr, bt.last, bt.B, bt.Hq, bt.Hkv)
    ws = torch.empty(max(256, plan.workspace_bytes), dtype=torch.uint8, device="cuda:0")
    plan.upload(ws, ws.numel(), stream)

    def fn():
        plan.run(t["q"], t["k"], t["v"], t["indptr"], t["indices"], t["last"], t["out"], t["lse"],
                 ws, ws.numel(), stream=stream)
    return fn, plan, ws


def uniform_runner(bt, t, stream, force_chunks=0):
    """decode_attention (the reference-shaped uniform split); force_chunks=1 is the reference's
    "no split" row (one chunk, i.e. one workgroup item, per sequence and kv head)."""
    import pdattn
    nc, ct = pdattn.plan_chunks(bt.G, bt.B, bt.Hkv, bt.max_len, force_chunks)
    p = pdattn.make_params(t["q"], t["k"], t["v"], t["indptr"], t["indices"], t["last"],
                           bt.B, bt.Hq, bt.Hkv, nc, ct)
    ws = pdattn.Workspace()
    pdattn.workspace_reserve(ws, pdattn.decode_workspace_size(bt.B, bt.Hq, nc))

    def fn():
        pdattn.decode_attention(p, bt.G, t["out"], t["lse"], ws, stream)
    return fn, (p, ws), nc


def balanced_runner(bt, t, stream):
    """decode_attention_balanced: decode_attention's arguments (plan_chunks' chunking), the pages
    cut into equal ranges on the device, with no host plan."""
    import pdattn
    nc, ct = pdattn.plan_chunks(bt.G, bt.B, bt.Hkv, bt.max_len)
    p = pdattn.make_params(t["q"], t["k"], t["v"], t["indptr"], t["indices"], t["last"],
                           bt.B, bt.Hq, bt.Hkv, nc, ct)
    ws = pdattn.Workspace()
    pdattn.workspace_reserve(ws, pdattn.decode_balanced_workspace_size(p, bt.G))

    def fn():
        pdattn.decode_attention_balanced(p, bt.G, t["out"], t["lse"], ws, stream)
    return fn, (p, ws)


ROT_BYTES = 1 << 30
COPY_BYTES = 256 << 20
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "decode_balanced_1x32k_traffic.md")


def ceiling_gbs(timer, steps):
    """Achievable streaming-read bandwidth: 2 GiB of 16-byte loads (stream_read)."""
    import torch
    import pdattn
    nbytes = 2 << 30
    buf = torch.ones(nbytes // 4, dtype=torch.int32, device="cuda:0")
    sink = torch.zeros(1, dtype=torch.int32, device="cuda:0")
    fn = lambda: pdattn.stream_read(buf, nbytes, sink, timer.stream)  # noqa: E731
    ms = timer.run([fn], max(5, steps // 3), 2)[0]
    del buf
    return nbytes / (statistics.median(ms) * 1e-3) / 1e9


def size_matched_read_us(nbytes, stream, steps):
    """Average duration of one stream_read launch over exactly `nbytes` (the workload's algorithmic
    bytes, contiguous), timed like rotated_kernel_us: K launches back to back between one event
    pair, launch i over buffer i mod n, the n buffers totalling >= ROT_BYTES. A single launch that
    moves this many bytes pays the same launch, ramp-up and drain as the decode does, so this is the
    achievable rate for a read of this size, beside the asymptotic 2 GiB ceiling."""
    import torch
    import pdattn
    nbytes = (nbytes + 15) // 16 * 16
    n = max(2, -(-ROT_BYTES // nbytes))
    bufs = [torch.ones(nbytes // 4, dtype=torch.int32, device="cuda:0") for _ in range(n)]
    sink = torch.zeros(1, dtype=torch.int32, device="cuda:0")
    for i in range(n):
        pdattn.stream_read(bufs[i], nbytes, sink, stream)
    k = max(steps, 4 * n)
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for i in range(k):
        pdattn.stream_read(bufs[i % n], nbytes, sink, stream)
    e1.record(stream)
    torch.cuda.synchronize()
    del bufs
    return e0.elapsed_time(e1) * 1e3 / k


def rotated_kernel_us(plan, ws, t, stream, steps, parts=None):
    """Average duration of one balanced step, K steps back to back between one event pair; with
    `parts` (pdattn.RUN_DECODE or RUN_MERGE) only that launch of each step (pdattn_plan_run_part),
    so that each kernel of the step is timed on its own. Returns (us, K, n).

    Step i reads K/V copy i mod n; the n copies total >= ROT_BYTES (4x the Infinity Cache), so
    each decode launch reads lines no cache still holds, with no flush kernel between launches."""
    import torch
    kv_bytes = 2 * t["k"].numel() * t["k"].element_size()
    n = max(2, -(-ROT_BYTES // kv_bytes))
    ks, vs = [t["k"]], [t["v"]]
    for _ in range(n - 1):
        ks.append(torch.empty_like(t["k"]).normal_())
        vs.append(torch.empty_like(t["v"]).normal_())

    def launch(i):
        if parts is None:
            plan.run(t["q"], ks[i % n], vs[i % n], t["indptr"], t["indices"], t["last"], t["out"],
                     t["lse"], ws, ws.numel(), stream=stream)
        else:
            plan.run_part(parts, t["q"], ks[i % n], vs[i % n], t["indptr"], t["indices"], t["last"],
                          t["out"], t["lse"], ws, ws.numel(), stream=stream)
    for i in range(n):
        launch(i)
    k = max(steps, 4 * n)
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for i in range(k):
        launch(i)
    e1.record(stream)
    torch.cuda.synchronize()
    del ks, vs
    return e0.elapsed_time(e1) * 1e3 / k, k, n


def kernel_sources_sha():
    """sha256 (first 16 hex digits) of the library's sources: every file of
    cuda-kernel-lab_amd/csrc and include/pdattn.h, in name order. The profile summaries record the
    same digest, so a figure read from them can be matched to the kernels this run measures."""
    import hashlib
    h = hashlib.sha256()
    csrc = os.path.join(ROOT, "cuda-kernel-lab_amd", "csrc")
    files = [os.path.join(csrc, n) for n in sorted(os.listdir(csrc))] + [os.path.join(ROOT, "include", "pdattn.h")]
    for path in files:
        with open(path, "rb") as f:
            h.update(os.path.basename(path).encode() + b"\0" + f.read())
    return h.hexdigest()[:16]


def measured_traffic():
    """(HBM bytes per launch of the headline kernel, commit and kernel-source digest the counters
    were collected on) from the committed counter summary (FETCH_SIZE + WRITE_SIZE per dispatch,
    each scaled by its copy-kernel calibration), or Nones."""
    nbytes, commit, sha = None, None, None
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    nbytes = int(float(line.split(":", 1)[1]))
                elif line.startswith("commit:"):
                    commit = line.split(":", 1)[1].strip()
                elif line.startswith("kernel_sources_sha256:"):
                    sha = line.split(":", 1)[1].strip()
    except OSError:
        pass
    return nbytes, commit, sha


def copy_calibration(steps):
    """Known-size traffic for counter calibration: dst.copy_(src) of COPY_BYTES, steps times."""
    import torch
    src = torch.ones(COPY_BYTES // 4, dtype=torch.int32, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(steps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes": COPY_BYTES, "launches": steps}))


def cpu_baseline(bt_lens, Hq, Hkv, seed, budget_s=10.0):
    """fp64 oracle on the host cores over the same workload shape (regenerated on the host)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle
    from pdattn import inputs
    bt = inputs.make_batch(bt_lens, Hq, Hkv, seed)
    host_cores = os.cpu_count() or 1
    # the box's CPU share for one GPU is 16 cores, whatever os.cpu_count() reports there
    threads = min(16, host_cores)
    runs, t0 = 0, time.perf_counter()
    while True:
        oracle.decode(bt.q, bt.k, bt.v, bt.indptr, bt.indices, bt.last, Hq, Hkv, threads=threads)
        runs += 1
        el = time.perf_counter() - t0
        if el >= budget_s or runs >= 200:
            break
    per = el / runs
    # the reference's own oracle is single-threaded: one thread as well, on a bounded sample
    runs1, t1 = 0, time.perf_counter()
    while True:
        oracle.decode(bt.q, bt.k, bt.v, bt.indptr, bt.indices, bt.last, Hq, Hkv, threads=1)
        runs1 += 1
        el1 = time.perf_counter() - t1
        if el1 >= budget_s / 2 or runs1 >= 50:
            break
    per1 = el1 / runs1
    return {"value": round(bt.algorithmic_bytes() / per / 1e9, 3), "unit": "GB/s",
            "cores": threads, "kind": "port", "host_cpu_count": host_cores,
            "sample": f"full B={bt.B} L={bt_lens[0]} workload, fp64 oracle (oracle/pdattn_oracle.c) "
                      f"x{runs} runs, {per * 1e3:.1f} ms/run on {threads} threads ({threads} of the "
                      f"{host_cores} CPUs os.cpu_count() reports: the box's share for one GPU)",
            "value_1_thread": round(bt.algorithmic_bytes() / per1 / 1e9, 3),
            "sample_1_thread": f"same workload x{runs1} runs, {per1 * 1e3:.1f} ms/run on 1 thread"}


def decode_workload(timer, lens, args, with_uniform, seed=11, nosplit=False):
    """Median cold step (flush before each) of the plan/run path, and of decode_attention (the
    uniform split) and its one-chunk "no split" form beside it; the plan path's kernel duration
    (rotated back to back); plan info."""
    import torch
    s = timer.stream
    bt, t = make_device_batch(lens, 32, 8, seed=seed)
    fn_sk, plan, ws = plan_runner(bt, t, s)
    fns, keep = [fn_sk], []
    if with_uniform:
        fn_un, k_un, nc = uniform_runner(bt, t, s)
        fns.append(fn_un)
        keep.append(k_un)
    if nosplit:
        fn_ns, k_ns, nc1 = uniform_runner(bt, t, s, force_chunks=1)
        fns.append(fn_ns)
        keep.append(k_ns)
    if with_uniform:
        fn_bd, k_bd = balanced_runner(bt, t, s)
        fns.append(fn_bd)
        keep.append(k_bd)
    times = timer.run(fns, args.steps, args.warmup, rounds=3)
    nbytes = bt.algorithmic_bytes()
    ms = statistics.median(times[0])
    kern_us, k, ncopy = rotated_kernel_us(plan, ws, t, s, args.steps)
    import pdattn
    dec_us, _, _ = rotated_kernel_us(plan, ws, t, s, args.steps, parts=pdattn.RUN_DECODE)
    info = plan.info()
    mrg_us = (rotated_kernel_us(plan, ws, t, s, args.steps, parts=pdattn.RUN_MERGE)[0]
              if info.merge_entries else 0.0)
    r = {"bytes": nbytes, "ms": ms, "steps": len(times[0]), "kernel_us": kern_us,
         "decode_kernel_us": dec_us, "merge_kernel_us": mrg_us,
         "kernel_launches": k, "kv_copies": ncopy, "workgroups": info.workgroups,
         "split_pairs": info.split_pairs, "paired": info.paired,
         "decode_kernel": "decode_pair_kernel" if info.paired else "decode_balanced_kernel"}
    if with_uniform:
        mu = statistics.median(times[1])
        r["uniform"] = {"us_per_step": round(mu * 1e3, 2), "chunks": nc,
                        "GB/s": round(nbytes / (mu * 1e-3) / 1e9, 1)}
    if with_uniform:
        mb = statistics.median(times[-1])
        r["balanced"] = {"us_per_step": round(mb * 1e3, 2), "GB/s": round(nbytes / (mb * 1e-3) / 1e9, 1),
                         "vs_plan_run": round(mb / ms, 4),
                         "path": "decode_attention_balanced: decode_attention's arguments, page ranges "
                                 "found on the device (no host plan)"}
    if nosplit:
        mn = statistics.median(times[2 if with_uniform else 1])
        r["no_split"] = {"us_per_step": round(mn * 1e3, 2), "chunks": nc1,
                         "items": nc1 * bt.B * bt.Hkv, "GB/s": round(nbytes / (mn * 1e-3) / 1e9, 1),
                         "path": "decode_attention, force_chunks = 1"}
    del keep, t, ws
    torch.cuda.empty_cache()
    return r


def decode_leg(timer, lens, args, ceil, seed=11, reference=None):
    """One decode configuration as a bench line: cold step, kernel time, both decode paths and the
    no-split row, as % of 8 TB/s and of the measured streaming ceiling."""
    h = decode_workload(timer, lens, args, with_uniform=True, seed=seed, nosplit=True)
    v, a = gbs(h["bytes"], h["ms"] * 1e-3), gbs(h["bytes"], h["kernel_us"] * 1e-6)
    out = {"B": len(lens), "L_mean": round(sum(lens) / len(lens), 1), "L_max": max(lens),
           "algorithmic_bytes": h["bytes"], "workgroups": h["workgroups"], "split_pairs": h["split_pairs"],
           "decode_kernel": h["decode_kernel"],
           "us_per_step": round(h["ms"] * 1e3, 2), "GB/s": round(v, 1),
           "pct_of_peak": round(100 * v / PEAK_GBS, 1), "pct_of_ceiling": round(100 * v / ceil, 1),
           "kernel_us": round(h["kernel_us"], 2), "kernel_GB/s": round(a, 1),
           "kernel_pct_of_peak": round(100 * a / PEAK_GBS, 1),
           "kernel_pct_of_ceiling": round(100 * a / ceil, 1),
           "decode_kernel_us": round(h["decode_kernel_us"], 2),
           "merge_kernel_us": round(h["merge_kernel_us"], 2),
           "decode_kernel_pct_of_peak": round(100 * gbs(h["bytes"], h["decode_kernel_us"] * 1e-6) / PEAK_GBS, 1),
           "uniform_path": h["uniform"], "no_split": h["no_split"], "balanced_path": h["balanced"]}
    for leg in (out["uniform_path"], out["no_split"], out["balanced_path"]):
        leg["pct_of_peak"] = round(100 * leg["GB/s"] / PEAK_GBS, 1)
        leg["pct_of_ceiling"] = round(100 * leg["GB/s"] / ceil, 1)
    if reference:
        out["reference_published"] = reference
    return out


# The reference's published perf runs (results/01_decode_attention.txt:99-121, RTX 5060 Laptop,
# 384 GB/s theoretical, 336 GB/s measured ceiling): its best split-KV variant and its no-split row.
REF_DECODE = {
    "1x32K": {"best_ms": 0.4134, "best_pct_of_peak": 84.6, "no_split_ms": 2.7655},
    "8x8K": {"best_ms": 0.9032, "best_pct_of_peak": 77.4, "no_split_ms": 0.9032},
    "64x1K": {"best_ms": 0.7925, "best_pct_of_peak": 88.5, "no_split_ms": 0.8250},
}
REF_CASCADE = {(64, 4096, 256): 2.34, (32, 16384, 512): 4.72, (8, 16384, 512): 2.20}


def cascade_shape_leg(timer, args, B, Lp, Ls):
    """One of the reference's shared-prefix perf shapes (01_decode_attention.cu:871-875): B requests
    sharing an Lp-token prefix plus Ls private tokens each. The cascade against both non-shared
    paths, same cold-cache method; the reference compares its cascade with its own non-shared
    decode_attention."""
    import pdattn
    from pdattn import inputs
    s = timer.stream
    bt, t = make_device_batch(None, 32, 8, seed=21, shared_prefix=Lp, suffix=[Ls] * B)
    f_plan, plan, ws = plan_runner(bt, t, s)
    f_uni, keep, nc = uniform_runner(bt, t, s)
    base = pdattn.make_params(t["q"], t["k"], t["v"], t["indptr"], t["indices"], t["last"], bt.B, 32, 8)
    cp = pdattn.CascadePlan(base, bt.indptr, bt.indices, bt.lens, t["indices"])
    cws = pdattn.Workspace()
    cp.decode(t["out"], t["lse"], cws, s)
    f_cas = lambda: cp.decode(t["out"], t["lse"], cws, s)  # noqa: E731
    wu, wp, wc = timer.run([f_uni, f_plan, f_cas], args.steps, args.warmup, rounds=3)
    mu, mp, mc = (statistics.median(w) * 1e3 for w in (wu, wp, wc))
    ci = cp.info()
    ub = inputs.unique_bytes(bt)
    out = {"cascade_us": round(mc, 2), "non_shared_uniform_us": round(mu, 2),
           "non_shared_plan_us": round(mp, 2), "speedup_vs_uniform": round(mu / mc, 2),
           "speedup_vs_plan": round(mp / mc, 2), "reference_speedup": REF_CASCADE.get((B, Lp, Ls)),
           "unique_bytes": ub, "cascade_GB/s_unique": round(gbs(ub, mc * 1e-6), 1),
           "mode": {0: "fused", 1: "serial", 2: "two_streams"}[ci.mode],
           "prefix_chunks": ci.prefix_chunks, "prefix_workgroups": ci.prefix_workgroups}
    cp.close()
    pdattn.workspace_release(cws)
    del t, ws, keep
    return out


def gbs(nbytes, seconds):
    return nbytes / seconds / 1e9


def cascade_workload(timer, args, Hq=32, Hkv=8):
    """64 requests x (8192 shared + 512 private): cascade vs the non-shared kernel, same method.
    Hq=32, Hkv=8 is BASELINE configs[4]; Hq=64, Hkv=8 (G=8) is the same batch with twice the query
    heads per kv head."""
    import pdattn
    s = timer.stream
    bt3, t3 = make_device_batch(None, Hq, Hkv, seed=21, shared_prefix=8192, suffix=[512] * 64)
    f3n, plan3, ws3 = plan_runner(bt3, t3, s)
    base = pdattn.make_params(t3["q"], t3["k"], t3["v"], t3["indptr"], t3["indices"], t3["last"],
                              bt3.B, Hq, Hkv)
    cp = pdattn.CascadePlan(base, bt3.indptr, bt3.indices, bt3.lens, t3["indices"])
    cws = pdattn.Workspace()
    cp.decode(t3["out"], t3["lse"], cws, s)  # uploads the schedule

    default = cp.info().mode

    def mode_fn(mode):
        def f():
            cp.set_mode(mode)
            cp.decode(t3["out"], t3["lse"], cws, s)
        return f
    f3c, f3s, f3o = (mode_fn(m) for m in (default, pdattn.CASCADE_SERIAL, pdattn.CASCADE_TWO_STREAMS))
    w3n, w3c, w3s, w3o = timer.run([f3n, f3c, f3s, f3o], args.steps, args.warmup, rounds=3)
    mn, mc, ms, mo = (statistics.median(w) for w in (w3n, w3c, w3s, w3o))
    cp.set_mode(default)
    ci = cp.info()
    from pdattn import inputs
    ub, nb = inputs.unique_bytes(bt3), bt3.algorithmic_bytes()
    out = {"non_shared_us": round(mn * 1e3, 2), "cascade_us": round(mc * 1e3, 2),
           "speedup": round(mn / mc, 2),
           "mode": {0: "fused", 1: "serial", 2: "two_streams"}[default],
           "cascade_serial_us": round(ms * 1e3, 2), "cascade_two_streams_us": round(mo * 1e3, 2),
           "unique_bytes": ub, "cascade_GB/s": round(gbs(ub, mc * 1e-3), 1),
           "non_shared_bytes": nb, "non_shared_GB/s": round(gbs(nb, mn * 1e-3), 1),
           "prefix_chunks": ci.prefix_chunks,
           "prefix_workgroups": ci.prefix_workgroups, "suffix_workgroups": ci.suffix_workgroups}
    cp.close()
    pdattn.workspace_release(cws)
    del t3, ws3
    return out


def prefix_workload(timer, args):
    """The cascade's MFMA prefix pass alone (pdattn_cascade_prefix) on the benchmark's shared
    prefix: 64 requests x 8192 shared tokens, chunks of 512 tokens. With 256 query rows per kv head
    the pass runs the key-split kernel: 16 chunks x 2 query groups of 128 rows x 8 kv heads = 256
    workgroups, one per CU, each splitting its chunk's keys between two wave groups. Flops per
    launch: 4 x (B Hq rows) x 128 x 8192 (QK^T and PV, 2 each)."""
    import numpy as np
    import torch
    import pdattn
    s = timer.stream
    d = torch.device("cuda:0")
    Lp, ct = 8192, 512
    bt, t = make_device_batch(None, 32, 8, seed=21, shared_prefix=Lp, suffix=[512] * 64)
    nch = Lp // ct
    rows = bt.B * 32
    po = torch.empty(rows, nch, 128, dtype=torch.float32, device=d)
    pl = torch.empty(rows, nch, dtype=torch.float32, device=d)
    pp = pdattn.PrefixParams()
    pp.q, pp.k_cache, pp.v_cache = t["q"].data_ptr(), t["k"].data_ptr(), t["v"].data_ptr()
    pp.prefix_pages = t["indices"].data_ptr()   # every sequence starts with the shared pages
    pp.part_o, pp.part_lse = po.data_ptr(), pl.data_ptr()
    pp.B, pp.Hq, pp.Hkv = bt.B, 32, 8
    pp.prefix_len, pp.chunk_tokens, pp.part_stride = Lp, ct, nch
    pp.sm_scale = float(1.0 / np.sqrt(128))
    fn = lambda: pdattn.cascade_prefix(pp, s)  # noqa: E731
    cold = statistics.median(timer.run([fn], args.steps, args.warmup)[0]) * 1e-3
    # back to back: the 33.5 MB of prefix K/V stay in the 256 MB Infinity Cache between launches
    n = 32
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(s)
    for _ in range(n):
        fn()
    e1.record(s)
    torch.cuda.synchronize()
    hot = e0.elapsed_time(e1) * 1e-3 / n
    flops = 4.0 * rows * 128 * Lp
    del t, po, pl
    qgroups = -(-(bt.B * 32 // 8) // 128)   # 128 stacked query rows per workgroup, per kv head
    return {"flops": flops, "chunk_tokens": ct, "workgroups": nch * qgroups * 8,
            "partial_bytes": rows * nch * (128 + 1) * 4, "cold_us": round(cold * 1e6, 2),
            "cold_TFLOP/s": round(flops / cold / 1e12, 1),
            "back_to_back_us": round(hot * 1e6, 2), "TFLOP/s": round(flops / hot / 1e12, 1),
            "frac_of_fp16_mfma_peak": round(flops / hot / 2.5e15, 4), "peak_TFLOP/s": 2500.0}


def append_workload(timer, args):
    """Paged KV append: all 32768 tokens of one sequence (the 1x32K caches: 2 x 134 MB read and
    written), and one decode step (one token for each of 64 sequences of 1K)."""
    import torch
    import pdattn
    s = timer.stream
    d = torch.device("cuda:0")
    out = {}
    for tag, lens, full in [("prefill_1x32K", [32768], True), ("decode_step_64x1K", [1024] * 64, False)]:
        bt, t = make_device_batch(lens, 32, 8, seed=13)
        if full:
            bidx = torch.zeros(lens[0], dtype=torch.int32, device=d)
            pos = torch.arange(lens[0], dtype=torch.int32, device=d)
        else:
            bidx = torch.arange(bt.B, dtype=torch.int32, device=d)
            pos = torch.tensor([L - 1 for L in lens], dtype=torch.int32, device=d)
        n = bidx.numel()
        kn = torch.randn(n, 8, 128, device=d, dtype=torch.float32).half()
        vn = torch.randn(n, 8, 128, device=d, dtype=torch.float32).half()
        fn = lambda: pdattn.append_kv(kn, vn, t["k"], t["v"], t["indptr"], t["indices"], bidx, pos,  # noqa: E731
                                      bt.B, 8, stream=s)
        ms = statistics.median(timer.run([fn], args.steps, args.warmup)[0])
        nbytes = 2 * 2 * n * 8 * 128 * 2           # K and V rows, read and written
        out[tag] = {"tokens": n, "us_per_step": round(ms * 1e3, 2),
                    "GB/s": round(nbytes / (ms * 1e-3) / 1e9, 1), "bytes": nbytes}
        del t, kn, vn
    return out


def graph_workload(timer, args):
    """A whole step captured as one HIP graph vs the same launches made eagerly (same cold-cache
    method): the 1x32K balanced step (decode + merge) and the cascade step (prefix + suffix +
    merge)."""
    import torch
    import pdattn
    s = timer.stream
    out = {}
    bt, t = make_device_batch([32768], 32, 8, seed=11)
    fn, plan, ws = plan_runner(bt, t, s)
    fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        plan.run(t["q"], t["k"], t["v"], t["indptr"], t["indices"], t["last"], t["out"], t["lse"],
                 ws, ws.numel(), stream=torch.cuda.current_stream())
    we, wg = timer.run([fn, g.replay], args.steps, args.warmup, rounds=3)
    out["1x32K"] = {"eager_us": round(statistics.median(we) * 1e3, 2),
                    "graph_us": round(statistics.median(wg) * 1e3, 2)}
    del t, ws, g
    bt3, t3 = make_device_batch(None, 32, 8, seed=21, shared_prefix=8192, suffix=[512] * 64)
    base = pdattn.make_params(t3["q"], t3["k"], t3["v"], t3["indptr"], t3["indices"], t3["last"],
                              bt3.B, 32, 8)
    cp = pdattn.CascadePlan(base, bt3.indptr, bt3.indices, bt3.lens, t3["indices"])
    cws = pdattn.Workspace()
    fc = lambda: cp.decode(t3["out"], t3["lse"], cws, s)  # noqa: E731
    fc()
    torch.cuda.synchronize()
    g3 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g3):
        cp.decode(t3["out"], t3["lse"], cws, torch.cuda.current_stream())
    we, wg = timer.run([fc, g3.replay], args.steps, args.warmup, rounds=3)
    out["cascade_64x(8192+512)"] = {"eager_us": round(statistics.median(we) * 1e3, 2),
                                    "graph_us": round(statistics.median(wg) * 1e3, 2)}
    cp.close()
    pdattn.workspace_release(cws)
    del t3, g3
    return out


def op_workload(timer, args):
    """torch.ops.pdattn.paged_decode (plan cached by table contents) vs the direct plan call, 1x32K."""
    import torch
    import pdattn
    import pdattn.torch_ops  # noqa: F401
    s = timer.stream
    bt, t = make_device_batch([32768], 32, 8, seed=11)
    fn, plan, ws = plan_runner(bt, t, s)
    iph = torch.from_numpy(bt.indptr.astype("int32"))
    lah = torch.from_numpy(bt.last.astype("int32"))
    sc = float(1.0 / 128 ** 0.5)
    op = lambda: torch.ops.pdattn.paged_decode(t["q"], t["k"], t["v"], t["indptr"], t["indices"],  # noqa: E731
                                               t["last"], iph, lah, sc)
    wd, wo = timer.run([fn, op], args.steps, args.warmup, rounds=3)
    del t, ws
    return {"1x32K": {"direct_us": round(statistics.median(wd) * 1e3, 2),
                      "op_us": round(statistics.median(wo) * 1e3, 2)}}


def tree_workload(timer, args):
    """Multi-level cascade: 64 requests = a 2048-token system prompt shared by all, then 8
    documents of 4096 tokens each shared by 8 requests, then 256 private tokens each. Non-shared
    decode vs the single-level cascade (system prompt only) vs the tree cascade."""
    import torch
    import pdattn
    from pdattn import inputs
    s = timer.stream
    nodes = [((0,), 2048)] + [((0, g), 4096) for g in range(1, 9)]
    seqs = [((0, g), 256) for g in range(1, 9) for _ in range(8)]
    bt = inputs.make_prefix_tree_batch(nodes, seqs, 32, 8, seed=23, fill=False)
    d = torch.device("cuda:0")
    g = torch.Generator(device=d)
    g.manual_seed(23)
    t = dict(q=torch.randn(bt.B, 32, 128, generator=g, device=d, dtype=torch.float32).half(),
             k=torch.randn(bt.num_pages, 16, 8, 128, generator=g, device=d, dtype=torch.float32).half(),
             v=torch.randn(bt.num_pages, 16, 8, 128, generator=g, device=d, dtype=torch.float32).half(),
             indptr=torch.from_numpy(bt.indptr).to(d), indices=torch.from_numpy(bt.indices).to(d),
             last=torch.from_numpy(bt.last).to(d),
             out=torch.empty(bt.B, 32, 128, dtype=torch.float16, device=d),
             lse=torch.empty(bt.B, 32, dtype=torch.float32, device=d))
    fn, plan, ws = plan_runner(bt, t, s)
    base = pdattn.make_params(t["q"], t["k"], t["v"], t["indptr"], t["indices"], t["last"], bt.B, 32, 8)
    plans, fns = [], [fn]
    for tree in (False, True):
        cp = pdattn.CascadePlan(base, bt.indptr, bt.indices, bt.lens, t["indices"], 256, tree)
        cws = pdattn.Workspace()
        cp.decode(t["out"], t["lse"], cws, s)
        plans.append((cp, cws))
        fns.append(lambda cp=cp, cws=cws: cp.decode(t["out"], t["lse"], cws, s))
    wn, w1, wt = timer.run(fns, args.steps, args.warmup, rounds=3)
    mn, m1, mt = (statistics.median(w) * 1e3 for w in (wn, w1, wt))
    info = plans[1][0].info()
    for cp, cws in plans:
        cp.close()
        pdattn.workspace_release(cws)
    del t, ws
    ub = inputs.unique_bytes(bt)
    return {"requests": 64, "unique_bytes": ub, "tree_GB/s": round(gbs(ub, mt * 1e-6), 1),
            "non_shared_us": round(mn, 2), "single_level_us": round(m1, 2),
            "tree_us": round(mt, 2), "tree_speedup_vs_non_shared": round(mn / mt, 2),
            "tree_speedup_vs_single_level": round(m1 / mt, 2), "tree_nodes": info.nodes,
            "tree_levels": info.levels}


TIMELINE_LIB = os.path.join(ROOT, "cuda-kernel-lab_amd", "lib", "timeline", "libpdattn.so")
TL_ROWS, TL_SLOTS = 8192, 32          # the stamp table of csrc/timeline.h
DECODE_STAMPS = ([(0, "start"), (1, "descriptors staged"), (2, "q rows staged"), (3, "first ring step")]
                 + [(4 + 2 * s, f"segment {s} streamed") for s in range(12)]
                 + [(5 + 2 * s, f"segment {s} flushed") for s in range(12)] + [(31, "done")])
# the paired kernel's stamp 2: its first page read back from LDS (q pieces go to registers)
PAIR_STAMPS = ([(0, "start"), (1, "descriptors staged"), (2, "first page in registers"), (3, "first ring step")]
                 + [(4 + 2 * s, f"segment {s} streamed") for s in range(12)]
                 + [(5 + 2 * s, f"segment {s} flushed") for s in range(12)] + [(31, "done")])
PREFIX_STAMPS = ([(0, "start"), (1, "ids staged"), (2, "block 0 in LDS")]
                 + [(3 + k, f"block {k} done") for k in range(24)]
                 + [(29, "blocks done"), (30, "partials written")])


def timeline(args):
    """Phase timestamps of every workgroup (thread 0's s_memrealtime at the stamps of
    csrc/timeline.h), in µs from the launch's first workgroup start: for each stamp the median
    over workgroups and the last workgroup, medians over `reps` launches. "cold": a 1 GiB flush
    before the launch; "b2b": the last of a run of launches back to back (the decode cases over
    rotated K/V copies of >= 1 GiB, so every launch reads from HBM)."""
    import ctypes
    import numpy as np
    import torch
    import pdattn
    if not os.path.exists(TIMELINE_LIB):
        sys.exit("no timeline build: run make -C cuda-kernel-lab_amd timeline")
    pdattn._lib = None
    pdattn.LIB_PATH = TIMELINE_LIB
    L = pdattn.lib()
    for t in ("decode", "prefix"):
        getattr(L, "pdattn_timeline_read_" + t).argtypes = [ctypes.c_void_p, ctypes.c_size_t]
    timer = Timer()
    s = timer.stream
    reps = max(3, min(args.steps, 9))

    def grab(table):
        torch.cuda.synchronize()
        buf = np.zeros(TL_ROWS * TL_SLOTS, np.uint64)
        assert getattr(L, "pdattn_timeline_read_" + table)(buf.ctypes.data, buf.nbytes) == 0
        return buf.reshape(TL_ROWS, TL_SLOTS).astype(np.int64)

    def reset(table):
        assert getattr(L, "pdattn_timeline_reset_" + table)() == 0

    def summary(runs, lo, hi, stamps):
        """runs: tables of the launches; rows [lo, hi) are the workgroups of one role."""
        rel = []
        for a in runs:
            a = a[lo:hi]
            t0 = a[:, 0][a[:, 0] > 0].min()
            rel.append(np.where(a > 0, (a - t0) * 0.01, np.nan))   # 100 MHz counter
        out = {}
        for slot, name in stamps:
            col = np.stack([r[:, slot] for r in rel])
            if np.isnan(col).all():
                continue
            med = np.nanmedian([np.nanmedian(c) for c in col])
            last = np.nanmedian([np.nanmax(c) for c in col])
            out[name] = [round(float(med), 2), round(float(last), 2)]
        return out

    def report(case, mode, workgroups, stamps):
        print(json.dumps({"timeline": case, "mode": mode, "workgroups": workgroups,
                          "stamps_us_median_last": stamps}), flush=True)

    if args.timeline in ("32k", "64x1k"):
        lens = [32768] if args.timeline == "32k" else [1024] * 64
        bt, t = make_device_batch(lens, 32, 8, seed=11)
        fn, plan, ws = plan_runner(bt, t, s)
        info = plan.info()
        W = info.workgroups // 2 if info.paired else info.workgroups   # workgroups of the launch
        stamps = PAIR_STAMPS if info.paired else DECODE_STAMPS
        print(json.dumps({"timeline": args.timeline, "kernel": "decode_pair_kernel" if info.paired
                          else "decode_balanced_kernel", "launch_workgroups": W}), flush=True)
        reset("decode")
        runs = []
        for _ in range(reps):
            fn()
            reset("decode")
            timer.flush()
            fn()
            runs.append(grab("decode"))
        report(args.timeline, "cold", W, summary(runs, 0, W, stamps))
        kv_bytes = 2 * t["k"].numel() * t["k"].element_size()
        n = max(2, -(-ROT_BYTES // kv_bytes))
        ks = [t["k"]] + [torch.empty_like(t["k"]).normal_() for _ in range(n - 1)]
        vs = [t["v"]] + [torch.empty_like(t["v"]).normal_() for _ in range(n - 1)]
        runs = []
        for _ in range(reps):
            for i in range(2 * n):
                plan.run(t["q"], ks[i % n], vs[i % n], t["indptr"], t["indices"], t["last"], t["out"],
                         t["lse"], ws, ws.numel(), stream=s)
            runs.append(grab("decode"))
        report(args.timeline, "b2b", W, summary(runs, 0, W, stamps))
        return
    if args.timeline == "prefix":
        bt, t = make_device_batch(None, 32, 8, seed=21, shared_prefix=8192, suffix=[512] * 64)
        for ct in (512, 256):
            nch = 8192 // ct
            po = torch.empty(bt.B * 32, nch, 128, dtype=torch.float32, device="cuda:0")
            pl = torch.empty(bt.B * 32, nch, dtype=torch.float32, device="cuda:0")
            pp = pdattn.PrefixParams()
            pp.q, pp.k_cache, pp.v_cache = t["q"].data_ptr(), t["k"].data_ptr(), t["v"].data_ptr()
            pp.prefix_pages = t["indices"].data_ptr()
            pp.part_o, pp.part_lse = po.data_ptr(), pl.data_ptr()
            pp.B, pp.Hq, pp.Hkv = bt.B, 32, 8
            pp.prefix_len, pp.chunk_tokens, pp.part_stride = 8192, ct, nch
            pp.sm_scale = float(1.0 / np.sqrt(128))
            W = nch * 2 * 8
            reset("prefix")   # (the other chunk size stamps other slots)
            runs = []
            for _ in range(reps):
                for _ in range(4):
                    pdattn.cascade_prefix(pp, s)
                runs.append(grab("prefix"))
            report(f"prefix 64x8192, {ct}-token chunks", "b2b", W, summary(runs, 0, W, PREFIX_STAMPS))
        return
    # the fused cascade step at config 5: decode-role and prefix-role workgroups
    bt, t = make_device_batch(None, 32, 8, seed=21, shared_prefix=8192, suffix=[512] * 64)
    base = pdattn.make_params(t["q"], t["k"], t["v"], t["indptr"], t["indices"], t["last"], bt.B, 32, 8)
    cp = pdattn.CascadePlan(base, bt.indptr, bt.indices, bt.lens, t["indices"])
    cws = pdattn.Workspace()
    info = cp.info()
    nd, npre = info.suffix_workgroups, info.prefix_workgroups
    for mode in ("cold", "b2b"):
        reset("decode")
        runs = []
        for _ in range(reps):
            cp.decode(t["out"], t["lse"], cws, s)
            if mode == "cold":
                reset("decode")
                timer.flush()
                cp.decode(t["out"], t["lse"], cws, s)
            else:
                for _ in range(4):
                    cp.decode(t["out"], t["lse"], cws, s)
            runs.append(grab("decode"))
        report("cascade 64x(8192+512) step, decode role", mode, nd, summary(runs, 0, nd, DECODE_STAMPS))
        report("cascade 64x(8192+512) step, prefix role", mode, npre,
               summary(runs, nd, nd + npre, PREFIX_STAMPS))
    cp.close()
    pdattn.workspace_release(cws)


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported in this build "
              f"(one GPU per box; the path would shard by sequence / kv head with no exchange)",
              file=sys.stderr)
        sys.exit(2)
    if args.timeline:
        timeline(args)
        return
    import torch
    import pdattn
    pdattn.lib()
    if args.copy_calibration:
        copy_calibration(args.steps)
        return
    dinfo = pdattn.device_info()
    timer = Timer()
    if args.only == "cascade":
        print(json.dumps({"cascade_64x(8192+512)": cascade_workload(timer, args)}))
        return
    if args.only == "cascade8":
        print(json.dumps({"cascade_64x(8192+512)_G8": cascade_workload(timer, args, 64, 8)}))
        return
    if args.only == "prefix":
        print(json.dumps({"cascade_prefix_mfma": prefix_workload(timer, args)}))
        return
    if args.only == "append":
        print(json.dumps({"append_kv": append_workload(timer, args)}))
        return
    if args.only == "graph":
        print(json.dumps({"hip_graph": graph_workload(timer, args)}))
        return
    if args.only == "tree":
        print(json.dumps({"cascade_tree": tree_workload(timer, args)}))
        return
    if args.only == "legs":
        from pdattn import inputs
        ceil = ceiling_gbs(timer, args.steps)
        out = {"stream_read_ceiling_GBs": round(ceil, 1)}
        for tag, lens_i, seed in [("C1 1x2K", [2048], 11), ("C3 8x8K", [8192] * 8, 11),
                                  ("C4 ragged B=64 L~U[256,4096]", inputs.ragged_lens(64, 256, 4096, seed=17), 17)]:
            out[tag] = decode_leg(timer, lens_i, args, ceil, seed=seed)
        out["cascade_reference_shapes"] = {
            f"{B}x({Lp}+{Ls})": cascade_shape_leg(timer, args, B, Lp, Ls) for (B, Lp, Ls) in REF_CASCADE}
        print(json.dumps(out))
        return
    lens = [1024] * 64 if args.only == "64x1k" else [32768]
    name = ("paged GQA decode B=64 L=1024 (metric's 64x1K)" if args.only == "64x1k"
            else "paged GQA decode B=1 L=32768 (configs[1])")
    full = not args.only and not args.no_secondary
    ceil = ceiling_gbs(timer, args.steps) if full else None
    h = decode_workload(timer, lens, args, with_uniform=args.only in ("", "32k", "64x1k"),
                        nosplit=args.only in ("", "32k", "64x1k"))
    value = gbs(h["bytes"], h["ms"] * 1e-3)
    achieved = gbs(h["bytes"], h["kernel_us"] * 1e-6)
    traffic, traffic_commit, traffic_sha = (measured_traffic() if not args.only or args.only == "32k"
                                            else (None, None, None))
    sources_sha = kernel_sources_sha()
    dec_achieved = gbs(h["bytes"], h["decode_kernel_us"] * 1e-6)
    result = dict(
        metric=METRIC, value=round(value, 1), unit="GB/s", n_gpus=1, steps=h["steps"],
        warmup=args.warmup, ms_per_step=round(h["ms"], 5), us_per_step=round(h["ms"] * 1e3, 2),
        pct_of_peak=round(100 * value / PEAK_GBS, 1), higher_is_better=True, scaling="weak",
        vs_baseline=None, dtype="f16", data="synthetic N(0,1) q/K/V, seeded, shuffled pages",
        config={"workload": name, "B": len(lens), "L": lens[0], "Hq": 32, "Hkv": 8,
                "head_dim": 128, "page": 16, "seed": 11, "accumulate": "f32",
                "path": f"pdattn_plan_run ({h['decode_kernel']} launch + merge launch for split pairs)",
                "workgroups": h["workgroups"],
                "algorithmic_bytes": h["bytes"], "cache_flush_bytes": FLUSH_BYTES,
                "timing": "median of per-step HIP events, 1 GiB read flush before each step"},
        roofline={"bound": "hbm", "achieved": round(dec_achieved, 1), "peak": PEAK_GBS, "unit": "GB/s",
                  "frac": round(dec_achieved / PEAK_GBS, 4), "traffic": traffic,
                  "traffic_source": (f"{os.path.relpath(TRAFFIC_FILE, ROOT)}: rocprofv3 --pmc FETCH_SIZE / "
                                     f"WRITE_SIZE of the decode launch, copy-calibrated, collected at "
                                     f"commit {traffic_commit}" if traffic else None),
                  "traffic_sources_match": (traffic_sha == sources_sha) if traffic else None,
                  "kernel": f"{h['decode_kernel']}, the dominant kernel: achieved = the algorithmic bytes "
                            "of one launch / its average duration, decode launches alone "
                            "(pdattn_plan_run_part) back to back over rotated K/V copies between one "
                            "HIP event pair on their stream; step_* = the whole step, the decode launch "
                            "plus the merge launch (merge_split_kernel, when pairs are split)",
                  "kernel_us": round(h["decode_kernel_us"], 2),
                  "kernel_frac": round(dec_achieved / PEAK_GBS, 4),
                  "decode_kernel_us": round(h["decode_kernel_us"], 2),
                  "decode_kernel_GB/s": round(dec_achieved, 1),
                  "merge_kernel_us": round(h["merge_kernel_us"], 2),
                  "step_us": round(h["kernel_us"], 2),
                  "step_achieved": round(achieved, 1),
                  "step_frac": round(achieved / PEAK_GBS, 4),
                  "timing": f"{h['kernel_launches']} back-to-back launches over {h['kv_copies']} "
                            f"K/V copies (>= 1 GiB) between one event pair"},
        device={"arch": dinfo.arch.decode(), "cus": dinfo.compute_units},
        kernel_sources_sha256=sources_sha,
    )
    if "uniform" in h:
        result["uniform_path"] = h["uniform"]
    if "balanced" in h:
        result["balanced_path"] = h["balanced"]
    if "no_split" in h:
        result["no_split"] = h["no_split"]
    if full:
        sec = {}
        result["stream_read_ceiling_GBs"] = round(ceil, 1)
        result["pct_of_ceiling"] = round(100 * value / ceil, 1)
        result["roofline"]["frac_of_ceiling"] = round(dec_achieved / ceil, 4)
        result["roofline"]["kernel_frac_of_ceiling"] = round(dec_achieved / ceil, 4)
        result["roofline"]["step_frac_of_ceiling"] = round(achieved / ceil, 4)
        sm_us = size_matched_read_us(h["bytes"], timer.stream, args.steps)
        result["roofline"]["size_matched_read"] = {
            "bytes": h["bytes"], "us": round(sm_us, 2), "GB/s": round(gbs(h["bytes"], sm_us * 1e-6), 1),
            "kernel_frac": round(sm_us / h["decode_kernel_us"], 4),
            "step_frac": round(sm_us / h["kernel_us"], 4),
            "what": "stream_read over the workload's algorithmic bytes in one launch, back to back "
                    "over rotated buffers (>= 1 GiB); kernel_frac = its time / the decode launch's, "
                    "step_frac = its time / the decode step's"}
        result["reference_published"] = REF_DECODE["1x32K"]
        for sub in (result.get("no_split"), result.get("uniform_path"), result.get("balanced_path")):
            if sub:
                sub["pct_of_peak"] = round(100 * sub["GB/s"] / PEAK_GBS, 1)
                sub["pct_of_ceiling"] = round(100 * sub["GB/s"] / ceil, 1)
        from pdattn import inputs
        legs = [("64x1K", [1024] * 64, 11), ("C1 1x2K", [2048], 11), ("C3 8x8K", [8192] * 8, 11),
                ("C4 ragged B=64 L~U[256,4096]", inputs.ragged_lens(64, 256, 4096, seed=17), 17)]
        for tag, lens_i, seed in legs:
            leg = decode_leg(timer, lens_i, args, ceil, seed=seed,
                             reference=REF_DECODE.get(tag.split()[-1] if tag != "64x1K" else "64x1K"))
            if tag == "64x1K":
                sm2_us = size_matched_read_us(leg["algorithmic_bytes"], timer.stream, args.steps)
                leg["size_matched_read_us"] = round(sm2_us, 2)
                leg["kernel_frac_of_size_matched_read"] = round(sm2_us / leg["kernel_us"], 4)
            sec[tag] = leg
        sec["cascade_64x(8192+512)"] = cascade_workload(timer, args)
        sec["cascade_64x(8192+512)_G8"] = cascade_workload(timer, args, 64, 8)
        sec["cascade_reference_shapes"] = {
            f"{B}x({Lp}+{Ls})": cascade_shape_leg(timer, args, B, Lp, Ls) for (B, Lp, Ls) in REF_CASCADE}
        sec["cascade_prefix_mfma"] = prefix_workload(timer, args)
        sec["append_kv"] = append_workload(timer, args)
        sec["hip_graph"] = graph_workload(timer, args)
        sec["torch_op"] = op_workload(timer, args)
        sec["cascade_tree"] = tree_workload(timer, args)
        result["secondary"] = sec
    if not args.no_cpu_baseline and not args.only:
        result["cpu_baseline"] = cpu_baseline([32768], 32, 8, seed=11)
    else:
        result["cpu_baseline"] = None
    print(json.dumps(result))


if __name__ == "__main__":
    main()
