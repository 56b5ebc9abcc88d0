"""Recentring, resets and refits on the device (ssa_maintain) against the oracle, step by step.

The reference acts on the flags between graph replays on the host (SphereIndexFused._check_flags
/ _act_on / _rebuild, src/ssa/kernels/sphere_fused.py:434-464; SphereIndexGPU._reset_heads,
src/ssa/attn/sphere_gpu.py:283-293; SphereIndexGraph._refit, src/ssa/kernels/graph_kernels.py:
270-279). Here ``after_replay`` issues ssa_maintain, which reads the flags on the device; the
oracle replays the reference's synchronous check (async_check=False) at the same steps:

* recentre: heads with the drift bit and not the reset bit are rebuilt around ksum / nb with
  their centroids kept (canon.build with mu, fit=False);
* reset: heads with the reset bit are fitted again from C_init clusters, seeded by
  torch.randperm on a CPU generator, get cap = split_factor * nb / C_init, and every head's
  clusters over the cap are divided as after the prompt fit;
* refit_every: every head, every refit_every steps;
* then every flag is cleared.

Selections and the whole state must agree bit for bit after every step, with the insertion
inside the step launch (insert-ahead) and as a separate launch.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle.canon import CanonIndex

pytestmark = pytest.mark.gpu

STATE = ("n_c", "sum_dir", "dir8", "cent", "cent8", "mmax", "mmin", "count", "ksum", "mu_ref", "rbar", "end",
         "nsplit", "labels", "flags", "cap")


def _cache(H_kv, n, *, H, seed, centers, drift_from=None):
    from ssa_amd.synth import make_cache
    K, V, q, _ = make_cache(1, H_kv, n, 128, H=H, centers=centers, seed=seed, dtype=torch.float32, device="cuda")
    K, V, q = K[0], V[0], q[0].contiguous()
    if drift_from is not None:
        K[:, drift_from:, :8] += 3.0                       # later keys lean one way: the mean drifts
    return K.to(torch.bfloat16), V.to(torch.bfloat16), q.to(torch.bfloat16)


def _same(idx, canon, fields=STATE):
    torch.cuda.synchronize()
    got = CanonIndex.from_gpu(idx)
    for f in fields:
        a, b = getattr(got, f), getattr(canon, f)
        if a is None and b is None:
            continue
        same = np.array_equal(a.view(np.uint8), b.view(np.uint8)) if a.dtype.kind == "f" else np.array_equal(a, b)
        if not same:
            bad = np.argwhere((a.view(np.uint8) != b.view(np.uint8)) if a.dtype.kind == "f" else (a != b))
            raise AssertionError(f"{f} differs at {len(bad)} places, first {bad[:3].tolist()}")


def _pair(K, n0, H, *, ahead, C, C_init, W, delta, split_factor=0.0, reset_at=0, check_every=4, refit_every=0,
          cap=None):
    from ssa_amd.graph_kernels import SphereIndexGraph
    from ssa_amd.sphere_fused import kmeans_init_indices
    idx = SphereIndexGraph(budget=0.2, insert_ahead=ahead, C=C, C_init=C_init, window=W, delta=delta,
                           capacity=K.shape[1], check_every=check_every, refit_every=refit_every,
                           partition="kmeans", split_factor=split_factor, reset_at=reset_at)
    assert idx.device_maintenance
    Kf = K.float().cpu().numpy()
    canon = CanonIndex(K.shape[0], 128, C=C, capacity=K.shape[1], C_init=C_init, partition="kmeans",
                       summary_bits=8, ms=min(8192, K.shape[1]))
    end = n0 - W
    canon.build(Kf, start=1, end=end, fit=True, iters=10, init_idx=kmeans_init_indices(end - 1, C_init, 0).numpy())
    if split_factor > 0:
        canon.cap[:] = np.float32(split_factor * (end - 1) / C_init)
        canon.split_after_fit(Kf, start=1, end=end, split_factor=split_factor)
    idx.observe(K, n0)
    if cap is not None:                                      # a smaller cap from here on: splits grow n_c
        idx.cap.fill_(cap)
        canon.cap[:] = np.float32(cap)
    idx.prepare(K, n0, H)
    if ahead:
        canon.insert(Kf, n0 + 1, window=W, delta=delta, reset_at=reset_at)
    _same(idx, canon)
    return idx, canon, Kf


def _oracle_check(canon, Kf, *, refit_all, refit, C_init, split_factor, seed=0):
    """The reference's synchronous check on the oracle: refit, then recentre, then clear."""
    from ssa_amd.sphere_fused import kmeans_init_indices
    flags = canon.flags.copy()
    end = int(canon.end[0])
    nb = end - 1
    H_kv = canon.H_kv
    reset = [h for h in range(H_kv) if refit and (refit_all or flags[h] & 2)]
    rec = [h for h in range(H_kv) if not refit_all and not (flags[h] & 2) and (flags[h] & 1) and nb > 0]
    if reset:
        canon.build(Kf, start=1, end=end, heads=reset, fit=True, iters=10,
                    init_idx=kmeans_init_indices(nb, C_init, seed).numpy())
        if split_factor > 0:
            for h in reset:
                canon.cap[h] = np.float32(split_factor * nb / C_init)
            canon.split_after_fit(Kf, start=1, end=end, split_factor=split_factor)
    if rec:
        mu = (canon.ksum[rec] / np.float32(nb)).astype(np.float32)
        canon.build(Kf, start=1, end=end, heads=rec, mu=mu, fit=False)
    canon.flags[:] = 0
    return len(rec), len(reset), nb


def _run(idx, canon, Kf, K, V, q, n0, steps, *, ahead, W, delta, reset_at=0, check_every=4, refit_every=0,
         C_init=16, split_factor=0.0):
    n_dev = torch.full((1,), n0, dtype=torch.int32, device="cuda")
    rec_total = reset_total = 0
    refit_nb = None                                        # binned keys at the last refit
    base = idx._steps                                      # steps the index has counted so far
    for i, m in enumerate(range(n0 + 1, n0 + steps + 1), 1):
        step = base + i
        n_dev.fill_(m)
        idx.step(q, K, V, n_dev)
        idx.after_replay(K)
        if not ahead:
            canon.insert(Kf, m, window=W, delta=delta, reset_at=reset_at)
        torch.cuda.synchronize()
        assert np.array_equal(idx.wbuf.cpu().numpy(), canon.select(q, budget=0.2)), m
        if ahead:
            canon.insert(Kf, m + 1, window=W, delta=delta, reset_at=reset_at)
        refit_all = bool(refit_every) and step % refit_every == 0
        if refit_all or step % check_every == 0:
            r, s, nb = _oracle_check(canon, Kf, refit_all=refit_all, refit=refit_all or bool(reset_at),
                                     C_init=C_init, split_factor=split_factor)
            rec_total += r
            reset_total += 0 if refit_all else s
            if s:
                refit_nb = nb
        _same(idx, canon)
    return rec_total, reset_total, refit_nb


@pytest.mark.parametrize("ahead", [True, False])
def test_device_recentring_matches_the_oracle(ahead):
    H_kv, H, n0, steps, W = 4, 8, 1200, 40, 16
    K, V, q = _cache(H_kv, n0 + steps + 8, H=H, seed=71, centers=16, drift_from=n0 - W - 200)
    idx, canon, Kf = _pair(K, n0, H, ahead=ahead, C=64, C_init=16, W=W, delta=0.01)
    rec, _, _ = _run(idx, canon, Kf, K, V, q, n0, steps, ahead=ahead, W=W, delta=0.01)
    assert rec > 0, "some head should have been recentred"
    assert idx.rebuilds == rec


@pytest.mark.parametrize("ahead", [True, False])
def test_device_reset_matches_the_oracle(ahead):
    """A small cap splits clusters in the steps until a head's cluster count reaches reset_at; the
    check then refits that head (k-means from 16 clusters, new cap, post-fit division)."""
    H_kv, H, n0, steps, W = 3, 6, 1500, 48, 16
    K, V, q = _cache(H_kv, n0 + steps + 8, H=H, seed=72, centers=16)
    idx, canon, Kf = _pair(K, n0, H, ahead=ahead, C=128, C_init=16, W=W, delta=math.inf, split_factor=2.0,
                           reset_at=40, cap=12.0)
    _, resets, _ = _run(idx, canon, Kf, K, V, q, n0, steps, ahead=ahead, W=W, delta=math.inf, reset_at=40,
                     split_factor=2.0)
    assert resets > 0, "some head should have been reset"
    assert idx.resets == resets


def test_device_refit_every_matches_the_oracle():
    """refit_every: every head fitted again on all its binned keys; the seed members are
    torch.randperm's (the scratch holds the last refit's)."""
    from ssa_amd.graph_kernels import _MAINT
    from ssa_amd.sphere_fused import kmeans_init_indices
    H_kv, H, n0, steps, W = 2, 4, 900, 14, 16
    K, V, q = _cache(H_kv, n0 + steps + 8, H=H, seed=73, centers=16)
    idx, canon, Kf = _pair(K, n0, H, ahead=True, C=128, C_init=16, W=W, delta=math.inf, split_factor=2.0,
                           check_every=10 ** 9, refit_every=7)
    _, _, nb = _run(idx, canon, Kf, K, V, q, n0, steps, ahead=True, W=W, delta=math.inf, check_every=10 ** 9,
                    refit_every=7, split_factor=2.0)
    assert idx.refits == (idx._steps // 7) and idx.refits >= 2
    sc = next(v for k, v in _MAINT.items() if k[1] == H_kv and k[2] == K.shape[1])
    assert np.array_equal(sc.init_idx.cpu().numpy(), kmeans_init_indices(nb, 16, 0).numpy())


def test_device_refit_seeds_cycle_below_c_init():
    """Fewer binned keys than clusters: the seed list cycles over randperm(nb)
    (src/ssa/attn/clusterkv.py:34-36)."""
    from ssa_amd.graph_kernels import _MAINT
    from ssa_amd.sphere_fused import kmeans_init_indices
    H_kv, H, W = 2, 4, 16
    n0 = 1 + 10 + W
    K, V, q = _cache(H_kv, n0 + 8, H=H, seed=74, centers=4)
    idx, canon, Kf = _pair(K, n0, H, ahead=False, C=16, C_init=16, W=W, delta=math.inf, check_every=10 ** 9,
                           refit_every=1)
    _, _, nb = _run(idx, canon, Kf, K, V, q, n0, 1, ahead=False, W=W, delta=math.inf, check_every=10 ** 9,
                    refit_every=1)
    assert nb < 16
    sc = next(v for k, v in _MAINT.items() if k[1] == H_kv and k[2] == K.shape[1])
    assert np.array_equal(sc.init_idx.cpu().numpy(), kmeans_init_indices(nb, 16, 0).numpy())
