"""Benchmark of the hot path: one layer's clustered sparse decode-attention step on one MI355X.

Workload: batch 1, 16 query heads / 8 KV heads, head_dim 128, bf16
KV cache, context 32768, keys from the synthetic mixture-of-directions distribution
(ssa_amd.synth), 256 k-means clusters per KV head (10 iterations), window 64, budgets 5 / 10 /
20 / 40 %, each against the same GPU's dense split-K decode over the full cache.

A step is what the reference's graph decoder runs per layer and token
(src/ssa/kernels/graph_kernels.py:220-244): insertion of the key leaving the recent window,
cluster scoring, selection, label scan, split-K attention over the selected rows and the
log-sum-exp merge. Here that is one kernel, ssa_sparse_step, captured in a hipGraph: it selects
and attends on the state binned for the current length, and its last workgroup per head then
bins the key that leaves the window at the next length (the reference bins it at the start of
the next step; the state each selection sees is the same). Timing follows the reference's harness (src/ssa/harness/kernel_bench.py:34-49,
165-214) with two changes for MI355X: one graph holds ROT steps, one per independent cache
(ROT x 134 MB, well above the 256 MB Infinity Cache, so every step reads its K/V rows from HBM),
and events bracket each replay of that graph with replays queued back to back, so the host's
launch gaps never enter a measurement; per-step time is the replay time divided by ROT.

Bytes per step follow the reference's accounting (src/ssa/attn/accounting.py:19-32) per
(sequence, KV head): selected K+V rows 2*rows*d*2, label scan 2n, 6 B per row read, summaries
C*(d+12) and centroids C*d (8-bit), inserted key 2d and its cluster's fp32 sum 8d. The step is
one kernel, so the roofline entry is that kernel: these bytes over its graph-timed duration per
launch (the mean over replays of the timed region). Each budget's detail also times the parts
the reference reports apart (maint_select and attention in its harness): the fused kernel
without the insertion (select_attention_us), the selection alone (ssa_select: score and pick
into w; select_us) and the attention alone given labels and w (ssa_label_attention: label
scan, split-K attention, merge; labelled_attention_us).

The CPU baseline times the oracle's numpy restatement of the reference's CPU path
(SphereIndexRef: observe one key, labels_and_weights, label_weighted_attention) at the same
shape in fp32, on a bounded number of steps.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]; prints one JSON line.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (ROOT, ROOT / "sparse-kv-reads_amd"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

H, H_KV, D, N, C, WINDOW = 16, 8, 128, 32768, 256, 64
BUDGETS = (0.05, 0.10, 0.20, 0.40)
HEADLINE = 0.20
PEAK_GBS = 8000.0


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def step_bytes(rows_per_head, n, *, d=D, C=C, summary_bits=8):
    """Reference accounting (src/ssa/attn/accounting.py:19-32) summed over KV heads."""
    vec = d * summary_bits / 8
    tot = 0.0
    for r in rows_per_head:
        tot += 2 * r * d * 2 + C * (vec + 12) + C * vec + 2 * n + 6 * r + 2 * d + 8 * d
    return tot


def attn_bytes(rows_per_head, n, *, d=D, C=C):
    """What the fused selection + attention kernel must read per launch: the selected K and V
    rows, the label scan and, once per head, the cluster summaries it scores (int8 direction,
    two fp32 lengths, an int32 count)."""
    return float(sum(2 * r * d * 2 + 2 * n + C * (d + 12) for r in rows_per_head))


class Set:
    """One independent (cache, index) pair; its length lives in ``n_dev`` (a slice of one
    tensor shared by all sets, so one launch advances every set)."""

    def __init__(self, seed, n, extra, splits, device, n_dev, dense_splits=None):
        import torch
        from ssa_amd.graph_kernels import DenseAttentionGraph, SphereIndexGraph
        from ssa_amd.synth import make_cache
        cap = n + extra
        K, V, q, _ = make_cache(1, H_KV, cap, D, H=H, centers=C, capacity=cap, seed=seed, dtype=torch.bfloat16,
                                device=device, gen_device=str(device))
        self.K, self.V, self.q = K[0], V[0], q[0].contiguous()
        self.n_dev = n_dev
        t = time.time()
        self.idx = SphereIndexGraph(budget=HEADLINE, C=C, window=WINDOW, delta=0.03, capacity=cap,
                                    check_every=10 ** 9, partition="kmeans", num_splits=splits)
        self.idx.prepare(self.K, n, H)
        torch.cuda.synchronize()
        self.prefill_s = time.time() - t
        self.dense = DenseAttentionGraph(H=H, H_kv=H_KV, d=D, dtype=torch.bfloat16, device=device,
                                         num_splits=dense_splits)


def capture(fns):
    """One graph running ``fns`` in order (each one layer-step on its own cache)."""
    import torch
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for f in fns:
            f()
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for f in fns:
            f()
    return g


def time_graph(g, reps, per, *, advance=None):
    """Median microseconds per step over ``reps`` replays of graph ``g`` holding ``per`` steps.
    Replays are queued back to back (the GPU never waits on the host inside a measurement);
    ``advance`` (one small kernel, between replays) moves every cache to its next position."""
    import torch
    ev = []
    for _ in range(reps):
        if advance is not None:
            advance()
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record()
        g.replay()
        b.record()
        ev.append((a, b))
    torch.cuda.synchronize()
    us = sorted(a.elapsed_time(b) * 1e3 / per for a, b in ev[1:])
    return us[len(us) // 2], sum(us) / len(us)


def cpu_baseline(seconds: float):
    """The reference's CPU path, restated in PyTorch (oracle/torch_ref.py), on this host's cores at
    the configs[1] shape in fp32 (the reference computes in fp32, src/ssa/attn/geometry.py:20-24):
    per step one key observed, labels_and_weights (sum_share) and label_weighted_attention over
    every cached key, as src/ssa/attn/labeled.py:24-44 computes it. Beside it, the oracle's numpy
    port that reads only the selected rows (the same selection, the attention restricted to the
    rows the GPU reads), and the configs[0] case (n = 4096) of the reference-shaped path."""
    import numpy as np
    import torch
    from oracle.reference import SphereIndexRef
    from oracle.torch_ref import SphereIndexTorch
    from ssa_amd.sphere_fused import kmeans_init_indices
    from ssa_amd.synth import make_cache
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    K, V, q, _ = make_cache(1, H_KV, N + 64, D, H=H, centers=C, seed=0, dtype=torch.float32)
    K, V, q = K[0].contiguous(), V[0].contiguous(), q[0].contiguous()
    init = lambda m, c: kmeans_init_indices(m, c, 0)                      # noqa: E731
    ref = SphereIndexTorch(C=C, window=WINDOW, init_indices=init)
    t0 = time.time()
    ref.observe(K, N)
    prefill = time.time() - t0
    times, rows = [], []
    n = N
    t_end = time.time() + seconds * 0.6
    with torch.inference_mode():
        while time.time() < t_end and n < N + 64:
            n += 1
            t = time.time()
            _, labels, w = ref.attend(q, K, V, n=n, budget=HEADLINE)
            times.append(time.time() - t)
            rows = [int((w[h][labels[h].long()] > 0).sum()) for h in range(H_KV)]
    times.sort()
    med = times[len(times) // 2]
    # the numpy port reading only the selected rows, same shape and steps
    port = SphereIndexRef(C=C, window=WINDOW, init_indices=lambda m, c, s: kmeans_init_indices(m, c, s).numpy())
    Kn, Vn, qn = K.numpy(), V.numpy(), q.numpy()
    port.observe(Kn, N)
    pt, m = [], N
    t_end = time.time() + seconds * 0.25
    while time.time() < t_end and m < N + 64:
        m += 1
        t = time.time()
        port.attend(qn, Kn, Vn, n=m, budget=HEADLINE, fast=True)
        pt.append(time.time() - t)
    pt.sort()
    # configs[0] exactly: n = 4096, the reference-shaped path, 20 steps
    n0 = 4096
    K0, V0, q0, _ = make_cache(1, H_KV, n0 + 32, D, H=H, centers=C, seed=0, dtype=torch.float32)
    K0, V0, q0 = K0[0].contiguous(), V0[0].contiguous(), q0[0].contiguous()
    ref0 = SphereIndexTorch(C=C, window=WINDOW, init_indices=init)
    ref0.observe(K0, n0)
    t0s = []
    with torch.inference_mode():
        for k in range(1, 21):
            t = time.time()
            ref0.attend(q0, K0, V0, n=n0 + k, budget=HEADLINE)
            t0s.append(time.time() - t)
    t0s.sort()
    return {"value": round(step_bytes(rows, n) / med / 1e9, 3), "unit": "GB/s", "cores": cores, "kind": "port",
            "us_per_step": round(med * 1e6, 1), "prefill_s": round(prefill, 2),
            "sparse_port_us_per_step": round(pt[len(pt) // 2] * 1e6, 1) if pt else None,
            "config0_us_per_step": round(t0s[len(t0s) // 2] * 1e6, 1),
            "sample": f"{len(times)} decode steps at n={N}..{n}, fp32, B=1, 16/8 heads, d=128, C=256, budget "
                      f"{HEADLINE}, after one k-means prefill ({prefill:.1f} s); median step of the reference-shaped "
                      f"PyTorch path (all {N} keys scored, then masked); sparse_port_us_per_step: the numpy port "
                      f"that reads only the selected rows ({len(pt)} steps); config0_us_per_step: the "
                      f"reference-shaped path at configs[0], n=4096, median of 20 steps",
            "threads": torch.get_num_threads(), "cpu_count": os.cpu_count(), "affinity": cores,
            "cpu": _cpu_model()}


def _cpu_model() -> str:
    """The host CPU as /proc/cpuinfo names it (model name, family / model / stepping)."""
    info = {}
    try:
        for line in open("/proc/cpuinfo"):
            if ":" in line:
                k, v = line.split(":", 1)
                info.setdefault(k.strip(), v.strip())
    except OSError:
        return "unknown"
    name = info.get("model name", "unknown")
    return f"{name} (family {info.get('cpu family', '?')}, model {info.get('model', '?')}, " \
           f"stepping {info.get('stepping', '?')})"


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--rot", type=int, default=16, help="independent caches; one graph steps through all of them")
    ap.add_argument("--splits", type=int, default=0, help="split-K factor of the sparse step (0: the default)")
    ap.add_argument("--dense-splits", type=int, default=0, help="split-K factor of the dense baseline (0: default)")
    ap.add_argument("--cpu-seconds", type=float, default=20.0)
    ap.add_argument("--budgets", type=str, default="", help="comma list of budgets to time (default: all)")
    ap.add_argument("--modes", type=str, default="dense,20,5",
                    help="configs[3]: comma list of decode modes (dense, 20, 5 = cluster budget in percent)")
    ap.add_argument("--calib-copy", action="store_true",
                    help="only copy 256 MiB device-to-device 5 times (calibrates rocprofv3 FETCH/WRITE_SIZE)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-batched", action="store_true",
                    help="config 1: skip the 16 x 32k and 64 x 32k batched steps reported under detail.batched")
    ap.add_argument("--config", type=int, default=1, choices=(1, 2, 3, 4),
                    help="1: the headline workload; 2: the batched sweep of configs[2]; 3: whole-model Qwen3-0.6B "
                         "decode of configs[3]; 4: Qwen3-4B long generation and batch-16 decode of configs[4] "
                         "(one JSON line each)")
    ap.add_argument("--shapes", type=str, default="", help="config 2: comma list of BxN shapes (default: all)")
    ap.add_argument("--long-prompt", type=int, default=8192, help="config 4: prompt of the long generation")
    ap.add_argument("--long-total", type=int, default=32768, help="config 4: length the generation reaches")
    ap.add_argument("--tokens", type=int, default=1024, help="config 3: tokens generated per mode")
    ap.add_argument("--prompt", type=int, default=32768, help="config 3: prompt length per sequence")
    ap.add_argument("--batch", type=int, default=2, help="config 3: sequences")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print(json.dumps({"error": "this benchmark runs on one GPU: the clustered sparse decode step of one "
                                   "GPU's share is the measured unit; multi-GPU sharding is described in DESIGN.md "
                                   "and not run"}))
        return 2
    import torch
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.calib_copy:
        x = torch.ones(256 * 1024 * 1024 // 4, device=dev)
        y = torch.empty_like(x)
        for _ in range(5):
            y.copy_(x)
        torch.cuda.synchronize()
        print(json.dumps({"calib_copy_bytes": x.numel() * 4, "copies": 5}))
        return 0
    if args.config == 2:
        res = batched_sweep(args, dev)
        print(json.dumps(_stamped({"metric": "configs[2] batched sparse decode-attention sweep (us, GB/s)",
                                   "unit": "us", "n_gpus": 1, "dtype": "bf16", "data": "synthetic (ssa_amd.synth)",
                                   "peak_GBs": PEAK_GBS,
                                   "config": {"workload": "configs[2]: B x ctx in " + str(list(BATCHED)) + ", 16 q / "
                                              "8 kv heads per sequence, d=128, bf16, 256 k-means clusters, window 64",
                                              "budgets": list(BATCHED_BUDGETS)},
                                   "results": res})), flush=True)
        return 0
    if args.config == 3:
        print(json.dumps(_stamped(model_decode(args, dev))), flush=True)
        return 0
    if args.config == 4:
        print(json.dumps(_stamped(model_long(args, dev))), flush=True)
        return 0
    global BUDGETS
    if args.budgets:
        BUDGETS = tuple(float(b) for b in args.budgets.split(","))
        if HEADLINE not in BUDGETS:
            BUDGETS = BUDGETS + (HEADLINE,)
    splits = args.splits or None
    reps = max(args.steps // args.rot, 4)
    extra = (args.warmup + 3) * len(BUDGETS) + reps * (len(BUDGETS) + 1) + 3 * (args.steps // args.rot + 2) + 64
    n_all = torch.full((args.rot,), N, dtype=torch.int32, device=dev)
    log(f"building {args.rot} caches of {N} tokens ...")
    sets = [Set(s, N, extra, splits, dev, n_all[s:s + 1], args.dense_splits or None) for s in range(args.rot)]
    log(f"prefill (k-means fit, binning, summaries) per cache: {sets[0].prefill_s:.3f} s (first), "
        f"{sets[-1].prefill_s:.3f} s (last)")
    advance = lambda: n_all.add_(1)                                   # noqa: E731

    graphs = {"dense": capture([lambda st=st: st.dense(st.q, st.K, st.V, st.n_dev) for st in sets])}
    for b in BUDGETS:
        for st in sets:
            st.idx.budget = b
        graphs[("step", b)] = capture([lambda st=st: st.idx.step(st.q, st.K, st.V, st.n_dev) for st in sets])
        graphs[("attn", b)] = capture([lambda st=st: _fused_only(st) for st in sets])
        # the unfused parts, as the reference's maint_select and attention report them
        graphs[("select", b)] = capture([lambda st=st: _select_only(st) for st in sets])
        graphs[("lattn", b)] = capture([lambda st=st: _label_attention_only(st) for st in sets])
    for st in sets:
        st.idx.budget = HEADLINE

    res = {}
    R = args.rot
    for b in BUDGETS:
        time_graph(graphs[("step", b)], args.warmup, R, advance=advance)
        res[("step", b)] = time_graph(graphs[("step", b)], reps, R, advance=advance)
        res[("attn", b)] = time_graph(graphs[("attn", b)], reps, R)
        res[("select", b)] = time_graph(graphs[("select", b)], reps, R)
        res[("lattn", b)] = time_graph(graphs[("lattn", b)], reps, R)
        res[("rows", b)] = sets[-1].idx.work.cnt.tolist()      # rows read per head, counted by the kernel
    time_graph(graphs["dense"], 3, R)
    res["dense"] = time_graph(graphs["dense"], reps, R)

    # The timed region: exactly K steps at the headline budget, as one graph that walks the
    # caches in turn and advances every length after each full round of them, bracketed by
    # synchronisations.
    for st in sets:
        st.idx.budget = HEADLINE
    K_steps = max(1, args.steps)
    seq = []
    for k in range(K_steps):
        st = sets[k % R]
        seq.append(lambda st=st: st.idx.step(st.q, st.K, st.V, st.n_dev))
        if k % R == R - 1 and k + 1 < K_steps:
            seq.append(advance)
    advance()
    g = capture(seq)
    g.replay()                                                        # untimed: graph upload
    advance()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    g.replay()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    steps_timed = K_steps
    n_now = int(n_all[0])

    dense_us = res["dense"][0]
    detail = {}
    for b in BUDGETS:
        rows = res[("rows", b)]
        step_us, attn_us = res[("step", b)][0], res[("attn", b)][0]
        detail[f"{int(b * 100)}%"] = {
            "step_us": round(step_us, 2), "select_attention_us": round(attn_us, 2),
            "select_us": round(res[("select", b)][0], 2), "labelled_attention_us": round(res[("lattn", b)][0], 2),
            "rows_per_head": int(sum(rows) / len(rows)),
            "step_effective_GBs": round(step_bytes(rows, N) / step_us / 1e3, 1),
            "attention_GBs": round(attn_bytes(rows, N) / attn_us / 1e3, 1),
            "speedup_vs_dense": round(dense_us / step_us, 2)}
    rows20 = res[("rows", HEADLINE)]
    head = detail[f"{int(HEADLINE * 100)}%"]
    step_mean = res[("step", HEADLINE)][1]
    achieved = step_bytes(rows20, N) / step_mean / 1e3
    out = {
        "metric": "sparse decode-attn effective HBM GB/s @32k ctx 20% budget (reference byte accounting, "
                  "per-layer graph step: insert+score+pick+attention)",
        "value": head["step_effective_GBs"], "unit": "GB/s", "n_gpus": 1, "steps": steps_timed,
        "warmup": args.warmup, "ms_per_step": round(wall / steps_timed * 1e3, 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (mixture-of-directions keys, N(0,1) values; ssa_amd.synth)",
        "config": {"workload": "configs[1]: one layer, B=1, 16 q / 8 kv heads, d=128, bf16 cache, ctx 32768, "
                               "256 k-means clusters, window 64", "batch": 1, "context": N, "heads": [H, H_KV],
                   "head_dim": D, "clusters": C, "budgets": list(BUDGETS), "rotation_caches": args.rot,
                   "splits": sets[0].idx.work.S, "dense_splits": sets[0].dense.work.S, "context_at_end": n_now},
        "detail": {**detail, "insert_ahead_us": round(res[("step", HEADLINE)][0] - res[("attn", HEADLINE)][0], 2),
                   "dense_us": round(dense_us, 2),
                   "dense_GBs": round(2 * H_KV * N * D * 2 / dense_us / 1e3, 1),
                   "dense_frac": round(2 * H_KV * N * D * 2 / dense_us / 1e3 / PEAK_GBS, 4),
                   "prefill_s": round(sets[-1].prefill_s, 4)},
        "roofline": {"bound": "hbm", "kernel": "ssa_sparse_step with insert-ahead (decode_kernel<bf16,128,2,"
                               "false,true,true,256>: selection, attention, merge, next step's insertion)",
                     "achieved": round(achieved, 1),
                     "peak": PEAK_GBS, "unit": "GB/s", "frac": round(achieved / PEAK_GBS, 4),
                     "traffic": _profiled_traffic(),
                     "bytes_per_launch": step_bytes(rows20, N), "avg_launch_us": round(step_mean, 3)},
    }
    if not args.no_batched:
        # configs[2]'s large batches, where the step amortises its fixed latency: reported beside
        # the headline (the value stays configs[1]'s B = 1 step)
        del graphs, g, sets
        torch.cuda.empty_cache()
        log("batched steps (configs[2]: 16 x 32768, 64 x 32768) ...")
        out["detail"]["batched"] = batched_sweep(args, dev, shapes=((16, N), (64, N)))
    if not args.no_cpu:
        log("timing the CPU baseline ...")
        out["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(_stamped(out)), flush=True)
    return 0


def _stamped(line: dict) -> dict:
    """The JSON line with the provenance header appended (src/ssa/harness/stamp.py:35-45): the
    driver's fields stay first, the header goes under "provenance"."""
    from ssa_amd.stamp import stamp
    return {**line, "provenance": stamp({})}


BATCHED = ((8, 8192), (2, 32768), (16, 32768), (64, 32768))
BATCHED_BUDGETS = (0.20, 0.05)


def batched_sweep(args, dev, shapes=None) -> dict:
    """batch x context in BATCHED, budgets 20% / 5%, every sequence with its own
    seeded clusters (batch folded into the KV heads). Per shape: the whole step (insert + fused
    selection and attention), the fused kernel alone and the dense baseline, each as a graph of
    ``rot`` steps over independent caches (at least 1 GB of K/V per graph, so rows come from HBM)."""
    import torch
    from ssa_amd.graph_kernels import DenseAttentionGraph, SphereIndexGraph
    from ssa_amd.synth import make_cache
    out = {}
    shapes = shapes or BATCHED
    if args.shapes and args.config == 2:
        shapes = tuple(tuple(int(v) for v in sh.split("x")) for sh in args.shapes.split(","))
    for B, n in shapes:
        hk = B * H_KV
        kv_bytes = 2 * hk * n * D * 2
        rot = max(1, -(-(1 << 30) // kv_bytes))
        reps = max(args.steps // rot, 4) if rot > 1 else max(args.steps // 8, 4)
        extra = (args.warmup + 3) * len(BATCHED_BUDGETS) + reps * (len(BATCHED_BUDGETS) + 1) + 64
        cap = n + extra
        n_all = torch.full((rot,), n, dtype=torch.int32, device=dev)
        sets = []
        t0 = time.time()
        for r in range(rot):
            K, V, q, _ = make_cache(B, H_KV, cap, D, H=H, centers=C, capacity=cap, seed=100 + r,
                                    dtype=torch.bfloat16, device=dev, gen_device=str(dev))
            K, V, q = K.view(hk, cap, D), V.view(hk, cap, D), q.view(B * H, D)
            idx = SphereIndexGraph(budget=BATCHED_BUDGETS[0], C=C, window=WINDOW, delta=0.03, capacity=cap,
                                   check_every=10 ** 9, partition="kmeans")
            idx.prepare(K, n, B * H)
            dense = DenseAttentionGraph(H=B * H, H_kv=hk, d=D, dtype=torch.bfloat16, device=dev)
            sets.append((K, V, q, idx, dense, n_all[r:r + 1]))
        torch.cuda.synchronize()
        log(f"B={B} n={n}: {rot} caches built in {time.time() - t0:.1f} s")
        advance = lambda: n_all.add_(1)                               # noqa: E731
        gd = capture([lambda s=s: s[4](s[2], s[0], s[1], s[5]) for s in sets])
        time_graph(gd, 3, rot)
        dense_first = time_graph(gd, reps, rot)[0]
        row = {"rotation_caches": rot, "kv_heads": hk, "splits": sets[0][3].work.S}
        for b in BATCHED_BUDGETS:
            for s in sets:
                s[3].budget = b
            # the step with the next key binned inside the fused launch (insert-ahead), and with
            # a separate insertion launch before it; both leave the same state
            ahead = {}
            for mode in (True, False):
                for s in sets:
                    s[3].insert_ahead = mode
                gs = capture([lambda s=s: s[3].step(s[2], s[0], s[1], s[5]) for s in sets])
                time_graph(gs, args.warmup, rot, advance=advance)
                ahead[mode] = time_graph(gs, reps, rot, advance=advance)[0]
                del gs
            for s in sets:
                s[3].insert_ahead = s[3].auto_insert_ahead()
            step_us = ahead[sets[0][3].insert_ahead]
            ga = capture([lambda s=s: _fused_only(_Shim(*s)) for s in sets])
            attn_us = time_graph(ga, reps, rot)[0]
            rows = sets[-1][3].work.cnt.tolist()
            by = attn_bytes(rows, n)
            row[f"{int(b * 100)}%"] = {
                "step_us": round(step_us, 2), "select_attention_us": round(attn_us, 2),
                "insert_ahead": sets[0][3].insert_ahead,
                "step_us_insert_ahead": round(ahead[True], 2), "step_us_insert_launch": round(ahead[False], 2),
                "rows_per_head": int(sum(rows) / len(rows)),
                "attention_GBs": round(by / attn_us / 1e3, 1), "attention_frac": round(by / attn_us / 1e3 / PEAK_GBS, 4),
                "step_effective_GBs": round(step_bytes(rows, n) / step_us / 1e3, 1)}
            del ga
        # dense is timed again after the sparse runs, at the same length, and the faster of the two
        # timings is the baseline
        n_all.fill_(n)
        time_graph(gd, 3, rot)
        dense_us = min(dense_first, time_graph(gd, reps, rot)[0])
        row.update({"dense_us": round(dense_us, 2), "dense_us_first": round(dense_first, 2),
                    "dense_GBs": round(kv_bytes / dense_us / 1e3, 1),
                    "dense_frac": round(kv_bytes / dense_us / 1e3 / PEAK_GBS, 4)})
        for b in BATCHED_BUDGETS:
            row[f"{int(b * 100)}%"]["speedup_vs_dense"] = round(dense_us / row[f"{int(b * 100)}%"]["step_us"], 2)
        out[f"{B}x{n}"] = row
        log(json.dumps({f"{B}x{n}": row}))
        del sets, gd
        torch.cuda.empty_cache()
    return out


MODEL_BUDGETS = (0.20, 0.05)


def model_decode(args, dev) -> dict:
    """Qwen3-0.6B (28 layers, hidden 1024, 16 q / 8 kv heads, d=128, vocab 151936) with
    random bf16 weights; ``batch`` prompts of ``prompt`` random token ids run through the model
    (exact causal attention), then ``tokens`` tokens generated greedily per mode, the whole step
    (embedding, 28 layers, LM head) replayed as one captured graph per token. Modes: dense
    split-K attention, and the clustered index at 20% and 5% (1,024 slots, 256 fitted at the
    prompt, size-cap splits on, per-step insertion). Each mode starts from the same prefilled
    cache. tokens/s = batch x tokens / wall time of the generation loop."""
    import torch
    from ssa_amd.graph_decode import GraphDecoder
    from ssa_amd.qwen3 import QWEN3_0_6B, random_model
    B, P, Tn = args.batch, args.prompt, args.tokens
    t0 = time.time()
    model = random_model(QWEN3_0_6B, dtype=torch.bfloat16, device=dev, seed=0)
    g = torch.Generator(device=dev).manual_seed(0)
    ids = torch.randint(0, QWEN3_0_6B.vocab_size, (B, P), device=dev, generator=g)
    base = model.alloc_cache(P + Tn + 1, batch=B)
    with torch.inference_mode():
        logits = model(ids, base, start_pos=0, last_only=True)
    first = logits[:, -1].argmax(-1, keepdim=True)
    torch.cuda.synchronize()
    log(f"config 3: model + prefill of {B} x {P} tokens in {time.time() - t0:.1f} s")
    res = {}
    modes = {"dense": ("dense", None), "20": ("cluster", 0.20), "5": ("cluster", 0.05)}
    for name in args.modes.split(","):
        mode, budget = modes[name]
        cache = model.alloc_cache(P + Tn + 1, batch=B)
        for i in range(len(cache.k)):
            cache.k[i].copy_(base.k[i])
            cache.v[i].copy_(base.v[i])
        cache.cur_len = P
        t1 = time.time()
        with torch.inference_mode():
            dec = GraphDecoder(model, cache, mode=mode, budget=budget or 0.2, greedy=True)
            dec.prepare(P)
            dec.capture()
        torch.cuda.synchronize()
        prep = time.time() - t1
        tok = first.clone()
        with torch.inference_mode():
            for pos in range(P, P + 8):                                    # warm-up steps, not timed
                dec.step(tok, pos)
                tok = dec.next_tok                                          # the greedy token, in the graph
            torch.cuda.synchronize()
            t2 = time.perf_counter()
            for pos in range(P + 8, P + Tn):
                dec.step(tok, pos)
                tok = dec.next_tok
            torch.cuda.synchronize()
            wall = time.perf_counter() - t2
        steps = Tn - 8
        key = "dense" if mode == "dense" else f"cluster_{int(budget * 100)}%"
        row = {"tokens_per_s": round(B * steps / wall, 1), "ms_per_step": round(wall / steps * 1e3, 4),
               "steps": steps, "prepare_s": round(prep, 2)}
        if mode == "cluster":
            idx = dec.attn[0]
            row.update({"splits_layer0": int(idx.splits), "active_clusters_layer0": round(float(idx.active_clusters), 1),
                        "insert_ahead": bool(idx.insert_ahead)})
        res[key] = row
        log(f"config 3 {key}: {json.dumps(row)}")
        del dec, cache
        torch.cuda.empty_cache()
    for k in list(res):
        if k != "dense" and "dense" in res:
            res[k]["speedup_vs_dense"] = round(res[k]["tokens_per_s"] / res["dense"]["tokens_per_s"], 3)
    return {"metric": "configs[3] Qwen3-0.6B whole-model decode tokens/s (hipGraph step)", "unit": "tokens/s",
            "higher_is_better": True, "n_gpus": 1, "dtype": "bf16",
            "data": "synthetic (random-init bf16 weights, random prompt token ids)",
            "config": {"workload": f"configs[3]: Qwen3-0.6B shape, batch {B}, prompt {P}, {Tn} tokens greedy",
                       "batch": B, "prompt": P, "tokens": Tn, "budgets": list(MODEL_BUDGETS)},
            "results": res}


def _generate(dec, first, start, steps, *, probes=()):
    """Greedy generation from ``first`` at positions start .. start+steps-1; returns the wall time of
    the non-probe steps and {step: mean relative attention error over layers} at the probe steps."""
    import torch
    tok = first.clone()
    errs, probe_s = {}, 0.0
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for k in range(steps):
        if k in probes:
            torch.cuda.synchronize()
            tp = time.perf_counter()
            got = []
            dec.step(tok, start + k, probe=got)
            tok = dec.next_tok
            errs[k] = round(float(torch.cat(got).mean()), 5)
            torch.cuda.synchronize()
            probe_s += time.perf_counter() - tp
        else:
            dec.step(tok, start + k)
            tok = dec.next_tok
        if k and k % 4096 == 0:
            log(f"  step {k} of {steps}")
    torch.cuda.synchronize()
    return time.perf_counter() - t0 - probe_s, errs


def model_long(args, dev) -> dict:
    """configs[4], Qwen3-4B shape (36 layers, hidden 2560, 32 q / 8 kv heads, d=128), random bf16
    weights. (a) One sequence: a random ``long_prompt``-token prompt run through the model, then
    greedy generation to ``long_total`` tokens with the clustered index (1,024 slots, 256 fitted at
    the prompt, clusters split past 2x the prompt's mean cluster size, so the cluster count grows
    with the context), and the same generation with dense attention; the relative error of every
    layer's attention output against exact attention on the same query is probed at steps 1k, 8k
    and 24k. (b) Batch 16 x 32k: synthetic caches (mixture-of-directions keys per layer, as
    configs[1]; a 16 x 32k prefill through a 4B model is not part of the decode measurement), 64
    decode steps per mode. Every step is one hipGraph replay."""
    import torch
    from ssa_amd.graph_decode import GraphDecoder
    from ssa_amd.qwen3 import QWEN3_4B, random_model
    from ssa_amd.synth import make_cache
    cfg = QWEN3_4B
    P, total = args.long_prompt, args.long_total
    T = total - P
    t0 = time.time()
    model = random_model(cfg, dtype=torch.bfloat16, device=dev, seed=0)
    ids = torch.randint(0, cfg.vocab_size, (1, P), device=dev, generator=torch.Generator(device=dev).manual_seed(0))
    base = model.alloc_cache(total + 1, batch=1)
    with torch.inference_mode():
        first = model(ids, base, start_pos=0, last_only=True)[:, -1].argmax(-1, keepdim=True)
    torch.cuda.synchronize()
    log(f"config 4: model + prefill of {P} tokens in {time.time() - t0:.1f} s")
    probes = tuple(k for k in (1000, 8000, 24000) if k < T)
    long_res = {}
    for mode in ("cluster", "dense"):
        cache = model.alloc_cache(total + 1, batch=1)
        for i in range(len(cache.k)):
            cache.k[i].copy_(base.k[i])
            cache.v[i].copy_(base.v[i])
        cache.cur_len = P
        with torch.inference_mode():
            dec = GraphDecoder(model, cache, mode=mode, budget=0.2, greedy=True)
            dec.prepare(P)
            dec.capture()
            wall, errs = _generate(dec, first, P, T, probes=probes if mode == "cluster" else ())
        row = {"tokens_per_s": round((T - len(errs)) / wall, 1), "steps": T}
        if mode == "cluster":
            idx = dec.attn[0]
            row.update({"attention_rel_error_at_step": errs, "clusters_layer0_end": round(float(idx.active_clusters), 1),
                        "splits_layer0": int(idx.splits), "cap_layer0": round(float(idx.cap.float().mean()), 1)})
        long_res[mode] = row
        log(f"config 4 long {mode}: {json.dumps(row)}")
        del dec, cache
        torch.cuda.empty_cache()
    long_res["cluster"]["speedup_vs_dense"] = round(long_res["cluster"]["tokens_per_s"] / long_res["dense"]["tokens_per_s"], 3)
    del base
    torch.cuda.empty_cache()
    # (b) batch 16 x 32k
    B, n, Tb = 16, 32768, 64
    cache = model.alloc_cache(n + Tb + 9, batch=B)
    for i in range(len(cache.k)):
        K, V, _, _ = make_cache(B, cfg.num_key_value_heads, n + Tb + 9, cfg.head_dim, H=cfg.num_attention_heads,
                                centers=C, capacity=n + Tb + 9, seed=500 + i, dtype=torch.bfloat16, device=dev,
                                gen_device=str(dev))
        cache.k[i].copy_(K)
        cache.v[i].copy_(V)
        del K, V
    first = torch.randint(0, cfg.vocab_size, (B, 1), device=dev, generator=torch.Generator(device=dev).manual_seed(1))
    log(f"config 4: batch {B} x {n} synthetic caches ready ({time.time() - t0:.0f} s)")
    b16 = {}
    for mode, budget in (("dense", None), ("cluster", 0.20), ("cluster", 0.05)):
        cache.cur_len = n
        with torch.inference_mode():
            dec = GraphDecoder(model, cache, mode=mode, budget=budget or 0.2, greedy=True)
            dec.prepare(n)
            dec.capture()
            _generate(dec, first, n, 8)
            wall, _ = _generate(dec, first, n + 8, Tb)
        key = "dense" if mode == "dense" else f"cluster_{int(budget * 100)}%"
        b16[key] = {"tokens_per_s": round(B * Tb / wall, 1), "ms_per_step": round(wall / Tb * 1e3, 3)}
        log(f"config 4 batch16 {key}: {json.dumps(b16[key])}")
        del dec
        torch.cuda.empty_cache()
    for k in b16:
        if k != "dense":
            b16[k]["speedup_vs_dense"] = round(b16[k]["tokens_per_s"] / b16["dense"]["tokens_per_s"], 3)
    return {"metric": "configs[4] Qwen3-4B long generation and batch-16 decode tokens/s (hipGraph step)",
            "unit": "tokens/s", "higher_is_better": True, "n_gpus": 1, "dtype": "bf16",
            "data": "random-init bf16 weights; random prompt ids (long run); synthetic KV caches (batch 16)",
            "config": {"workload": f"configs[4]: Qwen3-4B shape, prompt {P} -> {total} greedy (budget 0.2), "
                                   f"batch {B} x {n} decode", "budgets": [0.2, 0.05]},
            "long_generation": long_res, "batch16_32k": b16}


class _Shim:
    """Adapter giving ``_fused_only`` the attributes of a ``Set``."""

    def __init__(self, K, V, q, idx, dense, n_dev):
        self.K, self.V, self.q, self.idx, self.n_dev = K, V, q, idx, n_dev


def _profiled_traffic():
    """HBM bytes per launch of the fused kernel at the headline workload, as measured by
    rocprofv3 FETCH_SIZE + WRITE_SIZE (copy-calibrated) and recorded in profiles/."""
    p = ROOT / "profiles" / "sparse_step_32k_b1_traffic.md"
    try:
        for line in p.read_text().splitlines():
            if line.startswith("traffic_bytes_per_launch:"):
                return float(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def _select_only(st):
    """The selection alone (score + pick into w, ssa_select without insertion): the reference's
    maint_select part."""
    from ssa_amd._lib import check, lib, stream_ptr
    idx = st.idx
    sel = idx._select_args(st.q, idx.wbuf, idx.budget, "sum_share")
    check(lib().ssa_select(idx._state(), None, sel, stream_ptr(st.q.device)), "ssa_select")


def _label_attention_only(st):
    """The attention alone, given labels and w (compaction, split-K attention over the selected
    rows, merge; ssa_label_attention): the reference's attention part."""
    from ssa_amd._lib import check, lib, stream_ptr
    from ssa_amd.labeled_attn import attn_args
    idx = st.idx
    a = attn_args(st.q, st.K, st.V, idx.out, idx.work, labels=idx.labels, w=idx.wbuf, n_dev=st.n_dev)
    check(lib().ssa_label_attention(a, stream_ptr(st.q.device)), "ssa_label_attention")


def _fused_only(st):
    """The fused selection + attention launch of one step (no insertion)."""
    from ssa_amd._lib import check, lib, stream_ptr
    from ssa_amd.labeled_attn import attn_args
    idx = st.idx
    sel = idx._select_args(st.q, idx.wbuf, idx.budget, "sum_share")
    a = attn_args(st.q, st.K, st.V, idx.out, idx.work, labels=idx.labels, w=idx.wbuf, n_dev=st.n_dev)
    check(lib().ssa_sparse_step(idx._state(), sel, a, None, stream_ptr(st.q.device)), "ssa_sparse_step")


if __name__ == "__main__":
    sys.exit(main())
