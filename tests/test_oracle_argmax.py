"""The oracle's nearest-cluster choices against brute force in float64.

Insertion bins each key into the argmax over the live slots of <centroid_c, unit(k - mu_ref)>,
scored with the int8 centroid copies (8-bit summaries) or the fp32 centroids (32-bit), lowest
index on ties (src/ssa/kernels/sphere_fused.py:171-227; the torch path's argmax,
src/ssa/attn/sphere_gpu.py:166-184); the prefill labels every binned key with its nearest fitted
centroid (src/ssa/attn/sphere_gpu.py:187-219). The oracle computes these dots in fp32 in its
canonical order; here every label is recomputed in float64 and must agree wherever the best two
scores are not within rounding of each other. Each test also shows that a plausible mistake — the
wrong table scored (the summaries' directions instead of the centroids), or ties to the highest
index — would be caught.
"""

from __future__ import annotations

import math

import numpy as np
import pytest

from oracle.canon import CanonIndex

H_KV, D, C = 2, 32, 16


def _keys(seed: int, n: int, centers: int = 12, kappa: float = 3.0) -> np.ndarray:
    rng = np.random.default_rng(seed)
    K = np.empty((H_KV, n, D), np.float32)
    for h in range(H_KV):
        c = rng.standard_normal((centers, D))
        c /= np.linalg.norm(c, axis=1, keepdims=True)
        lab = rng.integers(0, centers, n)
        u = kappa * c[lab] + rng.standard_normal((n, D))
        u /= np.linalg.norm(u, axis=1, keepdims=True)
        K[h] = (0.3 * rng.standard_normal(D) + np.exp(0.3 * rng.standard_normal(n))[:, None] * u).astype(np.float32)
    return K


def _fitted(K, end: int, bits: int, init=None, iters: int = 10) -> CanonIndex:
    c = CanonIndex(H_KV, D, C=C, capacity=K.shape[1], summary_bits=bits)
    init = np.arange(0, 11 * C, 11, dtype=np.int32) if init is None else init
    c.build(K, start=1, end=end, fit=True, iters=iters, init_idx=init)
    return c


def _brute(K, mu, table, n_act, positions):
    """float64 argmax (first index on ties) and the gap to the runner-up, per position."""
    kr = K[positions].astype(np.float64) - mu.astype(np.float64)
    kn = kr / np.maximum(np.linalg.norm(kr, axis=1, keepdims=True), 1e-12)
    sc = kn @ np.asarray(table[:n_act], np.float64).T
    best = sc.argmax(1)
    top = np.sort(sc, 1)
    return best, top[:, -1] - top[:, -2], sc


@pytest.mark.parametrize("bits", [8, 32])
def test_insertion_labels_are_the_float64_argmax(bits):
    n0, n1 = 1200, 1600
    K = _keys(1, n1)
    c = _fitted(K, n0 - 64, bits)
    c.insert(K, n1, window=64, delta=math.inf)
    pos = np.arange(n0 - 64, n1 - 64)
    tol = 1e-3 if bits == 8 else 1e-5                    # int8 rows have norm ~127
    wrong_table = 0
    for h in range(H_KV):
        table = c.cent8[h] if bits == 8 else c.cent[h]
        best, gap, _ = _brute(K[h], c.mu_ref[h], table, int(c.n_c[h]), pos)
        got = c.labels[h, pos].astype(np.int64)
        clear = gap > tol * (127 if bits == 8 else 1)
        assert clear.mean() > 0.95
        assert np.array_equal(got[clear], best[clear]), f"head {h}"
        # the plausible mistake: scoring the summaries' directions instead of the centroids
        alt = c.dir8[h] if bits == 8 else c.sum_dir[h]
        best_alt, gap_alt, _ = _brute(K[h], c.mu_ref[h], alt, int(c.n_c[h]), pos)
        wrong_table += int(((best_alt != best) & clear & (gap_alt > tol)).sum())
    assert wrong_table > 0, "the data must tell the centroid table from the summary table"


@pytest.mark.parametrize("bits", [8, 32])
def test_insertion_ties_go_to_the_lowest_index(bits):
    n0, n1 = 1200, 1500
    K = _keys(2, n1)
    c = _fitted(K, n0 - 64, bits)
    lo, hi = 3, 9
    for h in range(H_KV):                                 # two identical centroid rows: every key
        if bits == 8:                                     # nearest to them ties exactly
            c.cent8[h, hi] = c.cent8[h, lo]
        else:
            c.cent[h, hi] = c.cent[h, lo]
    c.insert(K, n1, window=64, delta=math.inf)
    pos = np.arange(n0 - 64, n1 - 64)
    tied = 0
    for h in range(H_KV):
        table = c.cent8[h] if bits == 8 else c.cent[h]
        best, _, sc = _brute(K[h], c.mu_ref[h], table, int(c.n_c[h]), pos)
        got = c.labels[h, pos]
        tied += int((best == lo).sum())
        assert not (got == hi).any(), "a tie went to the higher index"
        assert ((got == lo) == (best == lo)).mean() > 0.95
    assert tied > 0, "some keys must fall in the tied pair"


def test_prefill_labels_are_the_float64_argmax():
    n = 1500
    K = _keys(3, n)
    end = n - 64
    c = _fitted(K, end, 32)
    pos = np.arange(1, end)
    for h in range(H_KV):
        best, gap, _ = _brute(K[h], c.mu_ref[h], c.cent[h], int(c.n_c[h]), pos)
        clear = gap > 1e-5
        assert clear.mean() > 0.95
        assert np.array_equal(c.labels[h, pos].astype(np.int64)[clear], best[clear])


def test_prefill_duplicate_seeds_keep_the_lower_slot():
    """Two k-means seeds on the same member give identical centroids: with no update between
    (0 iterations), every key nearest to them ties and goes to the lower slot; the higher slot
    stays empty."""
    n = 1500
    K = _keys(4, n)
    init = np.arange(0, 11 * C, 11, dtype=np.int32)
    init[7] = init[2]
    c = _fitted(K, n - 64, 32, init=init, iters=0)
    assert np.array_equal(c.cent[:, 7], c.cent[:, 2])
    assert (c.count[:, 7] == 0).all() and (c.count[:, 2] > 0).all()
    assert not (c.labels[:, 1:n - 64] == 7).any()
    pos = np.arange(1, n - 64)
    for h in range(H_KV):
        best, _, _ = _brute(K[h], c.mu_ref[h], c.cent[h], int(c.n_c[h]), pos)
        assert ((c.labels[h, pos] == 2) == (best == 2)).mean() > 0.99


def test_non_finite_key_joins_cluster_zero():
    """A key with a NaN element has a NaN score against every centroid: it joins cluster 0 (the
    index torch.argmax returns on a row of NaNs), and the other keys are unaffected."""
    n = 1200
    K = _keys(5, n)
    ref = _fitted(K, n - 64, 32)
    K2 = K.copy()
    K2[:, 100, 5] = np.nan
    c = CanonIndex(H_KV, D, C=C, capacity=n, summary_bits=32)
    c.build(K2, start=1, end=n - 64, fit=False, mu=ref.mu_ref)   # the fitted centroids, kept
    assert (c.labels[:, 100] == 0).all()
    c.cent[:] = ref.cent
    c.n_c[:] = ref.n_c
    c.build(K2, start=1, end=n - 64, fit=False, mu=ref.mu_ref)
    assert (c.labels[:, 100] == 0).all()
    others = np.r_[1:100, 101:n - 64]
    assert np.array_equal(c.labels[:, others], ref.labels[:, others])
    assert np.all(np.isfinite(c.mmax))
