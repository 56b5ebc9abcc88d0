"""The graph decode step (SphereIndexGraph, src/ssa/kernels/graph_kernels.py:192-279) on the GPU.

With ``insert_ahead`` the fused step bins, after its own attention, the key that leaves the
window at the next length; without it a separate insertion launch bins that key at the start
of the next step, as the reference does. Both orders must give the same outputs at every step
and the same index state, splits included, bit for bit. The captured graph is replayed with the
host's own work (advancing ``n``) between replays and every replay is checked against the
eager result.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

STATE = ("n_c", "sum_dir", "dir8", "cent", "cent8", "mmax", "mmin", "count", "ksum", "labels", "end_dev", "nsplit",
         "flags")


def _cache(H_kv, n, *, H, seed, centers=16):
    from ssa_amd.synth import make_cache
    K, V, q, _ = make_cache(1, H_kv, n, 128, H=H, centers=centers, seed=seed, dtype=torch.bfloat16, device="cuda")
    return K[0], V[0], q[0].contiguous()


def _graph_index(ahead, K, n0, H, cap, budget, splits=None):
    from ssa_amd.graph_kernels import SphereIndexGraph
    idx = SphereIndexGraph(budget=budget, insert_ahead=ahead, C=128, C_init=16, window=16, delta=math.inf,
                           capacity=K.shape[1], check_every=10 ** 9, partition="kmeans", num_splits=splits)
    idx.observe(K, n0)
    idx.cap.fill_(cap)                        # split under the cap from the first inserted key on
    idx.prepare(K, n0, H)
    return idx


def _same_state(a, b):
    torch.cuda.synchronize()
    for f in STATE:
        x, y = getattr(a, f), getattr(b, f)
        if x is None:
            assert y is None
            continue
        assert torch.equal(x, y), f


# (KV heads, splits): 3 heads stage in an extra workgroup per head; 128 x 4, 67 x 8 and 520 x 1
# give more than two workgroups per compute unit with one, so split S - 1 of each head stages
# instead (at S = 1 the head's only workgroup attends, stages, merges and commits)
@pytest.mark.parametrize("H_kv,splits,steps", [(3, None, 120), (128, 4, 40), (67, 8, 40), (520, 1, 12)])
@pytest.mark.parametrize("budget", [0.05, 0.2])
def test_insert_ahead_matches_insertion_at_step_start(budget, H_kv, splits, steps):
    from ssa_amd._lib import check, lib, stream_ptr
    from ssa_amd.labeled_attn import cu_count
    H, n0 = 2 * H_kv, 1000
    if splits is not None:
        assert H_kv * (splits + 1) > 2 * cu_count("cuda"), "the case should fold the staging"
    K, V, q = _cache(H_kv, n0 + steps + 8, H=H, seed=11)
    cap = float(1.5 * (n0 - 17) / 16)
    a = _graph_index(True, K, n0, H, cap, budget, splits)
    b = _graph_index(False, K, n0, H, cap, budget, splits)
    n_a = torch.full((1,), n0, dtype=torch.int32, device="cuda")
    n_b = torch.full((1,), n0, dtype=torch.int32, device="cuda")
    for n in range(n0 + 1, n0 + steps + 1):
        n_a.fill_(n)
        n_b.fill_(n)
        out_a = a.step(q, K, V, n_a).clone()
        out_b = b.step(q, K, V, n_b).clone()
        torch.cuda.synchronize()
        assert torch.equal(out_a, out_b), n
        assert torch.equal(a.wbuf, b.wbuf), n
        assert torch.equal(a.work.cnt, b.work.cnt), n
    assert a.splits > 0, "the cap should have split clusters inside the step"
    # b bins the keys of the next length at the start of its next step: do that now, then compare
    check(lib().ssa_insert(b._state(), b._insert_args(K, n_host=n0 + steps + 1), stream_ptr(b.device)), "ssa_insert")
    _same_state(a, b)
    assert a.splits == b.splits


def test_captured_step_replays_match_eager_steps():
    H_kv, H, n0, steps = 3, 6, 1000, 40
    K, V, q = _cache(H_kv, n0 + steps + 8, H=H, seed=12)
    cap = float(1.5 * (n0 - 17) / 16)
    g_idx = _graph_index(True, K, n0, H, cap, 0.2)
    e_idx = _graph_index(True, K, n0, H, cap, 0.2)
    n_g = torch.full((1,), n0, dtype=torch.int32, device="cuda")
    n_e = torch.full((1,), n0, dtype=torch.int32, device="cuda")
    # capture on a side stream, as torch.cuda.graph requires; the capture itself runs nothing
    graph = torch.cuda.CUDAGraph()
    n_g.fill_(n0 + 1)
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        g_idx.step(q, K, V, n_g)
    for n in range(n0 + 1, n0 + steps + 1):
        n_g.fill_(n)
        graph.replay()
        n_e.fill_(n)
        want = e_idx.step(q, K, V, n_e)
        torch.cuda.synchronize()
        assert torch.equal(g_idx.out, want), n
    _same_state(g_idx, e_idx)
    assert int(g_idx.end_dev[0]) == n0 + steps + 1 - 16
    # the binned keys' labels agree with the cluster counts
    lab = g_idx.labels.cpu().numpy()
    cnt = g_idx.count.cpu().numpy()
    end = int(g_idx.end_dev[0])
    for h in range(H_kv):
        assert np.array_equal(np.bincount(lab[h, 1:end], minlength=128), cnt[h])
