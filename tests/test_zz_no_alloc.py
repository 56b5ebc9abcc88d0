"""ssa_sparse_step_noalloc (the step with its split workspace in the library's own device array)
against ssa_sparse_step with caller-supplied buffers, through the C ABI.

Two twin indexes are stepped side by side, one through each entry point, with the insertion of
the next step's key inside the launch (insert-ahead, in-kernel splits included): outputs, the
selection, the rows read and the whole index state must agree bit for bit. A second, smaller
problem (fewer heads, shorter context, another GQA group) then runs through the no-alloc entry
point after the first, so its results must not depend on what the first left in the array.
Sizes beyond the array are refused before anything is launched.
"""

from __future__ import annotations

import math

import pytest
import torch

pytestmark = pytest.mark.gpu

STATE = ("n_c", "sum_dir", "dir8", "cent", "cent8", "mmax", "mmin", "count", "ksum", "labels", "end_dev", "nsplit",
         "flags")


def _index(K, n0, H, *, C, C_init, window):
    from ssa_amd.graph_kernels import SphereIndexGraph
    idx = SphereIndexGraph(budget=0.2, insert_ahead=True, C=C, C_init=C_init, window=window, delta=math.inf,
                           capacity=K.shape[1], check_every=10 ** 9, partition="kmeans")
    idx.observe(K, n0)
    idx.cap.fill_(float(1.5 * (n0 - window - 1) / C_init))      # splits from the first inserted keys on
    idx.prepare(K, n0, H)
    return idx


def _step(idx, q, K, V, n_dev, noalloc: bool):
    """SphereIndexGraph.step through one of the two entry points."""
    from ssa_amd._lib import check, lib, stream_ptr
    from ssa_amd.labeled_attn import attn_args
    st = idx._state()
    sel = idx._select_args(q, idx.wbuf, idx.budget, "sum_share")
    a = attn_args(q, K, V, idx.out, idx.work, labels=idx.labels, w=idx.wbuf, n_dev=n_dev)
    s = stream_ptr(q.device)
    if noalloc:
        a.part_m = a.part_l = a.part_a = a.part_cnt = a.counter = None     # ignored by the entry point
        check(lib().ssa_sparse_step_noalloc(st, sel, a, idx._insert_args(K), s), "ssa_sparse_step_noalloc")
    else:
        check(lib().ssa_sparse_step(st, sel, a, idx._insert_args(K), s), "ssa_sparse_step")
    return idx.out


def _run_pair(H_kv, H, n0, steps, *, C, C_init, window, seed):
    from ssa_amd.synth import make_cache
    K, V, q, _ = make_cache(1, H_kv, n0 + steps + 8, 128, H=H, centers=C_init, seed=seed, dtype=torch.bfloat16,
                            device="cuda")
    K, V, q = K[0], V[0], q[0].contiguous()
    ref = _index(K, n0, H, C=C, C_init=C_init, window=window)
    new = _index(K, n0, H, C=C, C_init=C_init, window=window)
    n_r = torch.full((1,), n0, dtype=torch.int32, device="cuda")
    n_n = torch.full((1,), n0, dtype=torch.int32, device="cuda")
    for n in range(n0 + 1, n0 + steps + 1):
        print(f"no-alloc step: H_kv={H_kv} H={H} n={n}", flush=True)
        n_r.fill_(n)
        n_n.fill_(n)
        want = _step(ref, q, K, V, n_r, noalloc=False).clone()
        got = _step(new, q, K, V, n_n, noalloc=True).clone()
        torch.cuda.synchronize()
        assert torch.equal(got, want), n
        assert torch.equal(new.wbuf, ref.wbuf), n
        assert torch.equal(new.work.cnt, ref.work.cnt), n
    for f in STATE:
        assert torch.equal(getattr(new, f), getattr(ref, f)), f
    return ref


def test_noalloc_step_equals_the_step_with_caller_buffers():
    big = _run_pair(8, 16, 4000, 12, C=128, C_init=32, window=64, seed=3)
    assert big.splits > 0, "the cap should split clusters inside the step"
    # a second, smaller problem right after the first: fewer heads and splits, a shorter context,
    # four query heads per KV head
    _run_pair(3, 12, 1500, 8, C=64, C_init=16, window=32, seed=4)


def test_noalloc_step_refuses_a_workspace_beyond_the_array():
    from ssa_amd._lib import AttnArgs, IndexState, SelectArgs, lib, stream_ptr
    a = AttnArgs()
    a.n_heads, a.G, a.d, a.S = 4096, 8, 256, 64          # 4096 * 64 * 8 * 256 * 4 B of partials: far above 4 MiB
    rc = lib().ssa_sparse_step_noalloc(IndexState(), SelectArgs(), a, None, stream_ptr())
    assert rc == 1                                        # hipErrorInvalidValue, nothing launched
    a.n_heads, a.G, a.d, a.S = 64, 2, 128, 32             # 2 MiB of partials: fits, but no state: refused
    rc = lib().ssa_sparse_step_noalloc(IndexState(), SelectArgs(), a, None, stream_ptr())
    assert rc == 1
