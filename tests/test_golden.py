"""The CPU oracle against golden vectors written by the reference's own functions.

The fixtures under tests/golden/ were produced by tests/golden/make_fixtures.py, which imports
the reference's pure-PyTorch code in float64 on the build machine (never on the GPU machine):
  kmeans_trajectory.npz   spherical_kmeans               src/ssa/attn/clusterkv.py:27-46
  padded_division.npz     _kmeans_padded, _bisect_padded src/ssa/attn/sphere_gpu.py:56-102
  index_steps.npz         SphereIndexGPU with splitting: post-fit division and slot handout
                          (:302-391), one key per step with in-step splits, labels_and_weights in the
                          four group modes (:412-442)
The oracle computes in fp32 in its canonical order, the reference in float64, so results agree
except at near-ties; every comparison below is exact away from a stated margin, and each test
also shows that a plausible mistake in the oracle (one k-means iteration fewer, the highest tied
index, no division after the fit) would fail it.
"""

from __future__ import annotations

import hashlib
import json
import math
from pathlib import Path

import numpy as np
import pytest

from oracle import reference as ref
from oracle.canon import CanonIndex, canon_bisect, canon_kmeans_parts

GOLD = Path(__file__).resolve().parent / "golden"


def _load(name: str):
    manifest = json.loads((GOLD / "MANIFEST.json").read_text())
    data = (GOLD / name).read_bytes()
    assert hashlib.sha256(data).hexdigest() == manifest["files"][name], f"{name} does not match its manifest"
    return np.load(GOLD / name)


def _unit(x):
    x = np.asarray(x, np.float64)
    return x / np.maximum(np.linalg.norm(x, axis=-1, keepdims=True), 1e-12)


# -- spherical_kmeans ------------------------------------------------------------------------------

def _fit(d, iters):
    X = d["X"]
    H, m, D = X.shape
    c = CanonIndex(H, D, C=int(d["C"]), capacity=m, summary_bits=32)
    c.build(X, start=0, end=m, mu=np.zeros((H, D), np.float32), fit=True, iters=iters, init_idx=d["init"])
    return c


def _kmeans_agrees(d, c, tol=1e-5) -> bool:
    X, C = d["X"], int(d["C"])
    m = X.shape[1]
    sc = np.einsum("hmd,hcd->hmc", _unit(X), d["cent"])
    top = np.sort(sc, -1)
    clear = (top[..., -1] - top[..., -2]) > tol                      # keys away from a near-tie
    same = c.labels[:, :m].astype(np.int64) == d["assign"]
    return bool(same[clear].all()) and float(np.abs(c.cent[:, :C] - d["cent"]).max()) < 1e-5


def test_kmeans_trajectory_matches_the_reference():
    d = _load("kmeans_trajectory.npz")
    assert list(d["moves_vs_final"][:3]) != [0, 0, 0], "the fixture must not converge in one iteration"
    assert _kmeans_agrees(d, _fit(d, int(d["iters"])))


def test_kmeans_fixture_rejects_one_iteration_fewer():
    """A mistake the trajectory test must catch: an oracle that stops one iteration early."""
    d = _load("kmeans_trajectory.npz")
    assert int(d["moves_vs_final"][-2]) > 0
    assert not _kmeans_agrees(d, _fit(d, int(d["iters"]) - 1))


def test_kmeans_seed_members_are_the_references():
    from ssa_amd.sphere_fused import kmeans_init_indices
    d = _load("kmeans_trajectory.npz")
    assert np.array_equal(kmeans_init_indices(d["X"].shape[1], int(d["C"]), int(d["seed"])).numpy(), d["init"])


# -- _kmeans_padded / _bisect_padded -----------------------------------------------------------------

def test_kmeans_division_matches_the_reference():
    d = _load("padded_division.npz")
    for r in range(d["Kn"].shape[0]):
        m = int(d["valid"][r].sum())
        part = canon_kmeans_parts(d["Kn"][r, :m], int(d["k"][r]), int(d["iters"]))
        assert np.array_equal(part, d["part"][r, :m]), f"row {r}"
        # seeds at evenly spaced members: one iteration fewer gives other parts on these rows
        if r == 0:
            assert not np.array_equal(canon_kmeans_parts(d["Kn"][r, :m], int(d["k"][r]), 1), d["part"][r, :m])


def test_bisection_matches_the_reference():
    d = _load("padded_division.npz")
    for r in range(d["Kn"].shape[0]):
        m = int(d["valid"][r].sum())
        side = canon_bisect(d["Kn"][r, :m])
        assert np.array_equal(side, d["side"][r, :m]), f"row {r}"
        assert not np.array_equal(1 - side, d["side"][r, :m])


# -- SphereIndexGPU with splitting, and labels_and_weights ------------------------------------------

def _index(d, *, divide: bool = True):
    K = d["K"]
    H_kv, n0, win, C, C_init = int(d["H_kv"]), int(d["n0"]), int(d["window"]), int(d["C"]), int(d["C_init"])
    from ssa_amd.sphere_fused import kmeans_init_indices
    c = CanonIndex(H_kv, K.shape[2], C=C, capacity=K.shape[1], C_init=C_init, summary_bits=32)
    end = n0 - win
    nb = end - 1
    init = kmeans_init_indices(nb, C_init, int(d["seed"])).numpy()
    c.build(K, start=1, end=end, fit=True, iters=int(d["kmeans_iters"]), init_idx=init)
    c.cap[:] = np.float32(float(d["split_factor"]) * nb / C_init)
    if divide:
        c.split_after_fit(K, start=1, end=end, split_factor=float(d["split_factor"]), iters=int(d["kmeans_iters"]))
    return c


def test_post_fit_division_matches_the_reference():
    d = _load("index_steps.npz")
    n0 = int(d["n0"])
    c = _index(d)
    assert int(d["fit_splits"]) > 0, "the fixture must exercise the division"
    assert np.array_equal(c.n_c, d["fit_n_c"])
    assert np.array_equal(c.labels[:, :n0], d["fit_labels"])
    assert np.array_equal(c.count, d["fit_count"])
    assert np.abs(c.sum_dir - d["fit_sum_dir"]).max() < 1e-4
    assert np.abs(c.mmax - d["fit_mmax"]).max() < 1e-5
    live = np.isfinite(d["fit_mmin"])
    assert np.array_equal(np.isfinite(c.mmin), live) and np.abs(c.mmin[live] - d["fit_mmin"][live]).max() < 1e-5
    # without the division the clusters are the fit's alone: the test sees the difference
    assert not np.array_equal(_index(d, divide=False).n_c, d["fit_n_c"])


def _near_tie(keys: np.ndarray, c: int, tol: float) -> bool:
    """True if cluster c's float64 key is within tol (relative) of another live cluster's."""
    k = keys[c]
    others = np.delete(keys, c)
    others = others[np.isfinite(others)]
    return bool(np.isfinite(k) and others.size and np.min(np.abs(others - k)) <= tol * max(1.0, abs(k)))


@pytest.mark.parametrize("group", ["sum_share", "per_head", "max", "max_rel"])
def test_decode_steps_match_the_reference(group):
    d = _load("index_steps.npz")
    K, Q = d["K"], d["Q"]
    n0, steps, win, budget = int(d["n0"]), int(d["steps"]), int(d["window"]), float(d["budget"])
    c = _index(d)
    ties = 0
    for s in range(steps):
        n = n0 + 1 + s
        c.insert(K, n, window=win, delta=math.inf)
        assert np.array_equal(c.n_c, d["n_c_steps"][s]), f"step {s}: clusters in use"
        w = c.select(Q[s], budget=budget, group=group)
        want = d[f"w_{group}"][s]
        if np.array_equal(w, want):
            continue
        # a difference is allowed only at a near-tie of the float64 keys (torch's argsort breaks
        # ties arbitrarily; the oracle breaks them by index)
        keys = ref.selection_keys(Q[s], c.sum_dir, c.mmax, c.mmin, c.count, c.n_c, group=group)
        keys = keys.reshape(-1, keys.shape[-1])
        for r, cc in zip(*np.nonzero(w != want)):
            assert cc < c.C and _near_tie(keys[r], cc, 1e-6), f"step {s} row {r} cluster {cc}"
            ties += 1
    assert ties <= 2
    n_end = n0 + steps
    assert int(d["splits_steps"][-1]) > int(d["fit_splits"]), "the fixture must exercise in-step splits"
    assert np.array_equal(c.labels[:, :n_end], d["end_labels"])
    assert np.array_equal(c.count, d["end_count"])
    assert np.abs(c.sum_dir - d["end_sum_dir"]).max() < 1e-4


def test_decode_steps_reject_ties_to_the_highest_index():
    """A planted mistake: ranking equal keys highest index first changes the selection of a
    cluster whose key ties another's (two identical summaries)."""
    d = _load("index_steps.npz")
    c = _index(d)
    q = d["Q"][0]
    h, a, b = 0, 1, 2
    for arr in (c.sum_dir, c.mmax, c.mmin, c.count):
        arr[h, b] = arr[h, a]
    keys = ref.selection_keys(q, c.sum_dir, c.mmax, c.mmin, c.count, c.n_c)[h]
    order = np.argsort(-keys, kind="stable")
    cnt = np.where(np.arange(c.C) < c.n_c[h], c.count[h], 0)
    before = np.cumsum(cnt[order]) - cnt[order]
    pos_a = int(np.nonzero(order == a)[0][0])
    need = int(before[pos_a] + cnt[a])            # budget ends exactly at cluster a: its tie b is not taken
    nb = int(c.end[h]) - 1
    w = c.select(q, budget=need / nb, group="sum_share")
    assert w[h, a] == 1.0 and w[h, b] == 0.0
