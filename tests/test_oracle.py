"""Pins the CPU oracle (CPU only).

The reference repository holds no golden tensors for this path (its tests draw inputs from
seeds), so each oracle function is checked against what fixes it independently:
  canonical arithmetic   cexp vs math.exp (ulp bound), cdot vs float64, q8 closed values
  attention spec         the naive loop formula, dense equivalence, unread rows ignored
                         (ports of tests/test_labeled_attention.py:21-87)
  merge                  partials of a split dense attention merge back to the dense result
  selection              float64 restatement of labels_and_weights agrees up to the threshold
                         cluster; exact ties go to the lowest index; budget invariants
                         (tests/test_sphere_fused.py:59-75, tests/test_split_kernels.py:97-101)
  k-means                recovers well-separated directions (tests/test_clusterkv.py:25-33); the
                         canonical fit agrees with a float64 fit from the same seeds; every label
                         is a nearest centroid in float64
  insertion              counts, sums, lengths recount exactly or within fp32 rounding
                         (tests/test_split.py:25-41, tests/test_split_kernels.py:35-41, 88-96)
  split                  sides agree with a float64 _bisect_padded within max(1, 2%); lopsided
                         clusters are cut at the median (tests/test_split_kernels.py:121-157)
  accounting             closed forms of tests/test_accounting.py
"""

from __future__ import annotations

import math

import numpy as np
import pytest

from oracle import reference as ref
from oracle.canon import CanonIndex, canon_dot, canon_exp, canon_kmeans_parts, canon_q8


# ---- canonical arithmetic ------------------------------------------------------------------

def test_canonical_exp_is_within_two_ulp_of_exp():
    xs = np.concatenate([np.linspace(-87.0, 0.0, 20001), -np.logspace(-8, 1.9, 2000), [0.0, -1e-30, -86.999]])
    for x in xs.astype(np.float32):
        got = canon_exp(float(x))
        want = math.exp(float(x))
        assert abs(got - want) <= 2 * np.spacing(np.float32(want)), (x, got, want)
    assert canon_exp(0.0) == 1.0
    assert canon_exp(-87.5) == 0.0 and canon_exp(-math.inf) == 0.0


def test_canonical_dot_matches_float64_and_is_exact_on_small_integers():
    g = np.random.default_rng(0)
    for d in (16, 64, 128, 256):
        a = g.standard_normal(d).astype(np.float32)
        b = g.standard_normal(d).astype(np.float32)
        err = abs(canon_dot(a, b) - float(np.dot(a.astype(np.float64), b.astype(np.float64))))
        assert err <= 1e-6 * float(np.abs(a.astype(np.float64) * b).sum()) + 1e-30
        ia = g.integers(-127, 128, d).astype(np.float32)
        ib = g.integers(-127, 128, d).astype(np.float32)
        assert canon_dot(ia, ib) == float(np.dot(ia.astype(np.int64), ib.astype(np.int64)))


def test_scoring_dot_matches_float64_and_is_exact_on_small_integers():
    from oracle.canon import canon_dot_chunked
    g = np.random.default_rng(1)
    for d in (16, 64, 128, 256):
        a = g.standard_normal(d).astype(np.float32)
        b = g.standard_normal(d).astype(np.float32)
        err = abs(canon_dot_chunked(a, b) - float(np.dot(a.astype(np.float64), b.astype(np.float64))))
        assert err <= 1e-6 * float(np.abs(a.astype(np.float64) * b).sum()) + 1e-30
        ia = g.integers(-127, 128, d).astype(np.float32)
        ib = g.integers(-127, 128, d).astype(np.float32)
        assert canon_dot_chunked(ia, ib) == float(np.dot(ia.astype(np.int64), ib.astype(np.int64)))
    # the chains are contiguous blocks: a value that cancels within a block vanishes exactly,
    # while the interleaved order keeps the small term's rounding
    d = 128
    a = np.zeros(d, np.float32)
    a[0], a[1], a[8] = 2.0 ** 30, 1.0, -(2.0 ** 30)       # one block; chains 0, 1, 0 when interleaved
    b = np.ones(d, np.float32)
    assert canon_dot_chunked(a, b) == 0.0                    # 2^30 + 1 rounds to 2^30, then - 2^30
    assert canon_dot(a, b) == 1.0                            # chain 0: 2^30 - 2^30 = 0, chain 1: 1


def test_q8_closed_values():
    assert canon_q8(1.0) == 127 and canon_q8(-1.0) == -127 and canon_q8(0.0) == 0
    assert canon_q8(0.5 / 127) == 1 and canon_q8(-0.5 / 127) == 0          # floor(u*127 + 0.5)
    assert canon_q8(0.999) == 127


# ---- attention spec (ports of tests/test_labeled_attention.py) -----------------------------

def _naive(q, K, V, labels, w):
    H, d = q.shape
    H_kv, n, _ = K.shape
    G = H // H_kv
    out = np.zeros((H, d))
    for h in range(H):
        kv = h // G
        wr = w[h] if w.shape[0] == H else w[kv]
        s = K[kv] @ q[h] / math.sqrt(d)
        m = s.max()
        num, den = np.zeros(d), 0.0
        for j in range(n):
            e = wr[int(labels[kv, j])] * math.exp(s[j] - m)
            num += e * V[kv, j]
            den += e
        out[h] = num / den
    return out


@pytest.mark.parametrize("per_head", [False, True])
def test_spec_matches_naive_formula(per_head):
    g = np.random.default_rng(1)
    q, K, V = g.standard_normal((8, 16)), g.standard_normal((2, 40, 16)), g.standard_normal((2, 40, 16))
    labels = g.integers(0, 7, (2, 40))
    w = g.random((8 if per_head else 2, 8)) * 3
    w[:, 2] = 0.0
    w[:, 7] = 1.0
    np.testing.assert_allclose(ref.label_weighted_attention(q, K, V, labels, w), _naive(q, K, V, labels, w),
                               rtol=1e-10, atol=1e-12)


def test_spec_all_ones_is_dense_and_ignores_unread_rows():
    g = np.random.default_rng(2)
    q, K, V = g.standard_normal((8, 16)), g.standard_normal((2, 70, 16)), g.standard_normal((2, 70, 16))
    labels = g.integers(0, 5, (2, 70))
    a = ref.label_weighted_attention(q, K, V, labels, np.ones((2, 6)))
    s = np.einsum("hd,hnd->hn", q, np.repeat(K, 4, 0)) / 4.0
    p = np.exp(s - s.max(1, keepdims=True))
    np.testing.assert_allclose(a, np.einsum("hn,hnd->hd", p / p.sum(1, keepdims=True), np.repeat(V, 4, 0)),
                               rtol=1e-10, atol=1e-12)
    w = np.array([[1.0, 0.0, 1.0, 0.0, 1.0, 1.0]] * 2)
    b1 = ref.label_weighted_attention(q, K, V, labels, w)
    K2, V2 = K.copy(), V.copy()
    skip = np.isin(labels, [1, 3])
    K2[skip] = 1e3
    V2[skip] = np.nan
    np.testing.assert_array_equal(ref.label_weighted_attention(q, K2, V2, labels, w), b1)


def test_f32_path_matches_float64_spec():
    g = np.random.default_rng(3)
    q = g.standard_normal((16, 128)).astype(np.float32)
    K, V = g.standard_normal((8, 3000, 128)).astype(np.float32), g.standard_normal((8, 3000, 128)).astype(np.float32)
    labels = g.integers(0, 257, (8, 3000))
    w = (g.random((8, 257)) < 0.3).astype(np.float32)
    w[:, 256] = 1
    np.testing.assert_allclose(ref.label_weighted_attention_f32(q, K, V, labels, w),
                               ref.label_weighted_attention(q, K, V, labels, w), rtol=0, atol=2e-6)


def test_merge_of_split_partials_is_the_dense_result():
    g = np.random.default_rng(4)
    H_kv, G, n, d, S = 3, 2, 900, 16, 7
    q, K, V = g.standard_normal((H_kv * G, d)) * 2, g.standard_normal((H_kv, n, d)), g.standard_normal((H_kv, n, d))
    m = np.full((H_kv, S, G), -1e30)
    l = np.zeros((H_kv, S, G))
    a = np.zeros((H_kv, S, G, d))
    bounds = np.linspace(0, n, S).astype(int)            # split S-1 covers nothing: an empty split
    for h in range(H_kv):
        for sp in range(S - 1):
            lo, hi = bounds[sp], bounds[sp + 1]
            s = K[h, lo:hi] @ q[h * G:(h + 1) * G].T / math.sqrt(d)
            m[h, sp] = s.max(0)
            e = np.exp(s - m[h, sp])
            l[h, sp] = e.sum(0)
            a[h, sp] = e.T @ V[h, lo:hi]
    np.testing.assert_allclose(ref.merge(m, l, a), ref.dense(q, K, V), rtol=1e-12, atol=1e-12)


# ---- selection ------------------------------------------------------------------------------

def _random_state(H_kv=4, C=64, d=128, seed=0, summary_bits=8):
    g = np.random.default_rng(seed)
    ci = CanonIndex(H_kv, d, C=C, capacity=8, summary_bits=summary_bits)
    n_act = C - 5
    ci.n_c[:] = n_act
    ci.sum_dir[:] = g.standard_normal((H_kv, C, d)).astype(np.float32) * 3
    u = ci.sum_dir / np.linalg.norm(ci.sum_dir, axis=-1, keepdims=True)
    ci.dir8[:] = np.floor(u * 127 + 0.5).astype(np.int8)
    ci.count[:] = g.integers(0, 40, (H_kv, C)).astype(np.int32)
    ci.count[:, n_act:] = 0
    ci.mmax[:] = (g.random((H_kv, C)) * 5 + 5).astype(np.float32)
    ci.mmin[:] = (ci.mmax * g.random((H_kv, C))).astype(np.float32)
    ci.end[:] = int(ci.count.sum(1).max()) + 1
    return ci


@pytest.mark.parametrize("group", ["sum_share", "per_head", "max", "max_rel"])
@pytest.mark.parametrize("budget", [0.05, 0.3, 1.0])
def test_selection_matches_float64_restatement_up_to_the_threshold(group, budget):
    ci = _random_state(seed=5)
    g = np.random.default_rng(6)
    q = (g.standard_normal((8, 128)) * 2).astype(np.float32)
    w = ci.select(q, budget=budget, group=group)
    nb = int(ci.end[0]) - 1
    w64 = ref.labels_and_weights(q, ci.dir8.astype(np.float64), ci.mmax, ci.mmin, ci.count, ci.n_c, nb=nb,
                                 budget=budget, group=group)
    assert np.all(w[:, -1] == 1.0)
    assert int((w != w64).sum(1).max()) <= 1
    G = w.shape[0] // ci.H_kv
    cnt = np.repeat(ci.count, G, 0).astype(np.int64)
    need = math.ceil(budget * nb)
    assert np.all((w[:, :-1] * cnt).sum(1) >= np.minimum(need, cnt.sum(1)))
    assert np.all(w[:, :-1][cnt == 0] == 0)                                  # empty and spare slots
    if budget == 1.0:
        assert np.array_equal(w[:, :-1] > 0, cnt > 0)


def test_exact_ties_go_to_the_lowest_index():
    ci = _random_state(H_kv=1, C=16, seed=7)
    ci.n_c[:] = 16
    ci.sum_dir[0, :] = ci.sum_dir[0, 3]                                      # 16 identical clusters
    ci.dir8[0, :] = ci.dir8[0, 3]
    ci.mmax[0, :] = 7.0
    ci.mmin[0, :] = 3.0
    ci.count[0, :] = 10
    ci.end[:] = 161
    q = np.random.default_rng(8).standard_normal((2, 128)).astype(np.float32)
    for budget, k in ((0.05, 1), (0.2, 4), (0.5, 8)):                        # need = 8, 32, 80 keys
        w = ci.select(q, budget=budget)
        assert np.array_equal(np.nonzero(w[0, :16])[0], np.arange(k)), (budget, w[0])


def test_no_budget_or_nothing_binned_selects_only_the_exact_set():
    ci = _random_state(seed=9)
    q = np.ones((8, 128), np.float32)
    assert np.array_equal(ci.select(q, budget=0.0)[:, :-1], np.zeros((4, 64)))
    ci.end[:] = 1
    w = ci.select(q, budget=0.5)
    assert np.all(w[:, :-1] == 0) and np.all(w[:, -1] == 1)


# ---- prefill k-means -----------------------------------------------------------------------

def test_kmeans_recovers_well_separated_directions():
    g = np.random.default_rng(0)
    centers = g.standard_normal((4, 16))
    centers /= np.linalg.norm(centers, axis=1, keepdims=True)
    truth = np.arange(200) % 4
    X = centers[truth] * 5 + 0.05 * g.standard_normal((200, 16))
    K = np.zeros((1, 202, 16), np.float32)
    K[0, 1:201] = X                                           # binned range [1, 201)
    ci = CanonIndex(1, 16, C=4, capacity=202)
    import torch                                              # the reference's seed members:
    init = torch.randperm(200, generator=torch.Generator().manual_seed(0))[:4].numpy()   # clusterkv.py:34-35
    ci.build(K, start=1, end=201, mu=[np.zeros(16, np.float32)], init_idx=init)
    lab = ci.labels[0, 1:201]
    for c in range(4):
        assert len(np.unique(lab[truth == c])) == 1
    np.testing.assert_allclose(np.linalg.norm(ci.cent[0, :4], axis=1), 1.0, atol=1e-6)


def _clustered(H_kv, n, d=128, centers=32, seed=0):
    g = np.random.default_rng(seed)
    K = np.zeros((H_kv, n, d))
    for h in range(H_kv):
        cen = g.standard_normal((centers, d))
        cen /= np.linalg.norm(cen, axis=1, keepdims=True)
        which = g.integers(0, centers, n)
        u = 20 * cen[which] + g.standard_normal((n, d))
        K[h] = g.standard_normal(d) + 10 * u / np.linalg.norm(u, axis=1, keepdims=True)
    return K.astype(np.float32)


def test_canonical_kmeans_agrees_with_float64_kmeans_and_labels_are_nearest():
    H_kv, n, C = 2, 1200, 32
    K = _clustered(H_kv, n, centers=C)
    init = np.random.default_rng(1).permutation(n - 1)[:C]
    ci = CanonIndex(H_kv, 128, C=C, capacity=n)
    ci.build(K, start=1, end=n, init_idx=init, iters=10)
    Kb = K[:, 1:n].astype(np.float64)
    assign, cent = ref.spherical_kmeans(Kb - Kb.mean(1, keepdims=True), C=C, iters=10, init=init)
    agree = (assign == ci.labels[:, 1:n]).mean()
    assert agree > 0.99, agree
    Xn = ref.normalize(Kb - ci.mu_ref[:, None].astype(np.float64))
    cos = np.einsum("hmd,hcd->hmc", Xn, ci.cent.astype(np.float64))
    lab = ci.labels[:, 1:n].astype(np.int64)
    chosen = np.take_along_axis(cos, lab[..., None], 2)[..., 0]
    assert np.all(chosen >= cos.max(-1) - 1e-5)
    np.testing.assert_allclose(ci.ksum, Kb.sum(1), rtol=1e-4, atol=1e-2)


# ---- insertion and splitting ---------------------------------------------------------------

def test_insertion_recounts():
    H_kv, n0, n1, C = 2, 900, 1500, 32
    K = _clustered(H_kv, n1, centers=C, seed=3)
    ci = CanonIndex(H_kv, 128, C=C, capacity=n1)
    ci.build(K, start=1, end=n0 - 16, init_idx=np.arange(C) * 7)
    for n in range(n0, n1, 3):
        ci.insert(K, n, window=16, delta=math.inf)
    for h in range(H_kv):
        e = int(ci.end[h])
        lab = ci.labels[h, 1:e].astype(np.int64)
        assert np.array_equal(np.bincount(lab, minlength=C), ci.count[h])
        Kr = K[h, 1:e].astype(np.float64) - ci.mu_ref[h]
        mag = np.linalg.norm(Kr, axis=1)
        sd = np.zeros((C, 128))
        np.add.at(sd, lab, Kr / mag[:, None])
        np.testing.assert_allclose(ci.sum_dir[h], sd, rtol=1e-4, atol=1e-4)
        for c in np.unique(lab):
            np.testing.assert_allclose(ci.mmax[h, c], mag[lab == c].max(), rtol=1e-6)
            np.testing.assert_allclose(ci.mmin[h, c], mag[lab == c].min(), rtol=1e-6)
        assert np.all(ci.labels[h, e:] == C) and ci.labels[h, 0] == C


@pytest.mark.parametrize("lumpy", [False, True])
def test_split_sides_agree_with_bisect_padded(lumpy):
    H_kv, d = 1, 32
    g = np.random.default_rng(10)
    n = 700
    K = g.standard_normal((H_kv, n, d)).astype(np.float32) + 0.3
    if lumpy:
        main = g.standard_normal(d)
        K[0, 300:] = 4 * main + 0.2 * g.standard_normal((n - 300, d))
        K[0, 320::37] = -4 * main
    ci = CanonIndex(H_kv, d, C=16, capacity=n, C_init=1)
    ci.build(K, start=1, end=200, init_idx=np.array([0]))
    ci.cap[:] = 250.0
    splits = 0
    for step in range(200, n - 1):
        before = ci.labels[0].copy()
        ns = int(ci.nsplit[0])
        ci.insert(K, step + 1, window=1, delta=math.inf)         # bins position p = step - 1
        if int(ci.nsplit[0]) == ns:
            continue
        splits += 1
        p, nw = step - 1, int(ci.n_c[0]) - 1
        after = ci.labels[0]
        moved = np.nonzero((after == nw) & (np.arange(n) != p))[0]
        c = int(before[moved[0]])
        members = np.nonzero(((before == c) | (np.arange(n) == p)) & (np.arange(n) >= 1) & (np.arange(n) <= p))[0]
        side = (after[members] == nw).astype(int)
        kr = K[0, members].astype(np.float64) - ci.mu_ref[0]
        kn = kr / np.linalg.norm(kr, axis=1, keepdims=True)
        want = ref.bisect_padded(kn[None], np.ones((1, len(members)), bool))[0]
        dis = int((want != side).sum())
        assert dis <= max(1, int(0.02 * len(members))), (dis, len(members))
        share = side.mean()
        assert 0.25 <= share <= 0.75 or abs(int(side.sum()) - len(members) // 2) <= 1
    assert splits > 0 and int(ci.n_c[0]) < 16                 # balanced cuts leave spare slots
    assert np.all(ci.count[0] <= 250)


# ---- accounting (tests/test_accounting.py) -------------------------------------------------

def test_overhead_counts_every_per_step_read():
    d, n, rows, c = 128, 32768, 6000.0, 1000.0
    row = 2 * d
    got = ref.overhead_rows(n=n, rows=rows, clusters=c, d=d, summary_bits=8)
    want = (c * (d + 12) + c * d + 2 * n + 6 * rows + row + 2 * 4 * d) / row
    assert abs(got - want) < 1e-9
    f32 = ref.overhead_rows(n=n, rows=rows, clusters=c, d=d, summary_bits=32)
    assert abs((f32 - got) - 2 * c * 3 * d / row) < 1e-9
    assert ref.overhead_rows(n=1000, rows=100.0, clusters=256.0, d=128, fitted=False, heads=8) < \
        ref.overhead_rows(n=1000, rows=100.0, clusters=256.0, d=128, fitted=True)
    f = ref.kv_read_fraction(n=1000, rows=200.0, clusters=64.0, d=16, summary_bits=8)
    assert abs(f - (400 + ref.overhead_rows(n=1000, rows=200.0, clusters=64.0, d=16, summary_bits=8)) / 2000) < 1e-12


def test_post_fit_division_keeps_the_cap_and_recounts():
    """The oracle's division after a fit (src/ssa/attn/sphere_gpu.py:307-391): every cluster ends
    at or under the cap (spare slots permitting), counts equal the label histogram, summaries
    equal a float64 recount, and labels stay below the clusters in use."""
    g = np.random.default_rng(3)
    d, n, C, C_init = 32, 1500, 64, 8
    centers = g.standard_normal((5, d))
    which = g.choice(5, n, p=[0.5, 0.2, 0.15, 0.1, 0.05])
    K = (centers[which] * 4 + g.standard_normal((n, d))).astype(np.float32)[None]
    c = CanonIndex(1, d, C=C, capacity=n + 8, C_init=C_init, partition="kmeans", summary_bits=8)
    start, end = 1, n
    init = np.arange(C_init, dtype=np.int32) * ((end - start) // C_init)
    c.build(K, start=start, end=end, fit=True, iters=10, init_idx=init)
    cap = np.float32(2.0 * (end - start) / C_init)
    c.cap[:] = cap
    assert c.count[0].max() > cap                                  # something to divide
    rounds = c.split_after_fit(K, start=start, end=end, split_factor=2.0)
    assert rounds >= 2
    n_c = int(c.n_c[0])
    assert n_c > C_init and int(c.nsplit[0]) == n_c - C_init
    lab = c.labels[0, start:end].astype(np.int64)
    assert lab.max() < n_c
    assert np.array_equal(np.bincount(lab, minlength=C), c.count[0])
    assert np.all(c.count[0] <= cap) or n_c == C
    Kr = K[0, start:end].astype(np.float64) - c.mu_ref[0].astype(np.float64)
    mag = np.linalg.norm(Kr, axis=1)
    kn = Kr / np.maximum(mag, 1e-12)[:, None]
    for s in range(n_c):
        m = lab == s
        np.testing.assert_allclose(c.sum_dir[0, s], kn[m].sum(0), rtol=0, atol=1e-4)
        assert np.isclose(c.mmax[0, s], mag[m].max(), rtol=1e-6) and np.isclose(c.mmin[0, s], mag[m].min(), rtol=1e-6)
        np.testing.assert_allclose(np.linalg.norm(c.cent[0, s]), 1.0, atol=1e-6)


def test_post_fit_kmeans_round_finds_obvious_parts():
    """One cluster holding three tight, well separated groups, cap a third of it: the k-means round
    asks for ceil(count * 2 / cap) = 6 parts, started from members 0, 20, ..., 100 (two in each
    group), so every part lies inside one group and every group is covered."""
    d, per = 16, 40
    dirs = np.eye(d, dtype=np.float32)[:3] * 10
    g = np.random.default_rng(4)
    K = np.concatenate([dirs[i] + 0.01 * g.standard_normal((per, d)) for i in range(3)]).astype(np.float32)
    K = np.concatenate([np.zeros((1, d), np.float32), K])[None]           # position 0 is the sink
    n = K.shape[1]
    c = CanonIndex(1, d, C=16, capacity=n, C_init=1, partition="kmeans", summary_bits=8)
    c.build(K, start=1, end=n, fit=True, iters=10, init_idx=np.zeros(1, np.int32))
    assert int(c.count[0, 0]) == 3 * per
    c.cap[:] = np.float32(per)
    c.split_after_fit(K, start=1, end=n, split_factor=2.0)
    lab = c.labels[0, 1:n]
    groups = [set(lab[i * per:(i + 1) * per].tolist()) for i in range(3)]
    assert all(not (groups[i] & groups[j]) for i in range(3) for j in range(i + 1, 3))   # no part mixes groups
    n_c = int(c.n_c[0])
    assert set.union(*groups) == set(range(n_c)) and 3 <= n_c <= 6
    assert np.all(c.count[0, :n_c] <= per)


def test_kmeans_division_into_70_parts_recovers_70_groups():
    """The k-means division has no limit on the parts (src/ssa/attn/sphere_gpu.py:357-358): 70
    tight groups of 10 members around distinct directions, members in group order, k = 70 parts
    seeded at members j * m / k = 10 j (one per group): every part is exactly one group. A
    division capped at 32 parts, or seeded elsewhere, could not give this."""
    d, per, k = 128, 10, 70
    g = np.random.default_rng(7)
    dirs = g.standard_normal((k, d))
    dirs /= np.linalg.norm(dirs, axis=1, keepdims=True)
    K = np.concatenate([5.0 * dirs[i] + 0.01 * g.standard_normal((per, d)) for i in range(k)]).astype(np.float32)
    part = canon_kmeans_parts(K, k, 10, mu=np.zeros(d, np.float32))
    assert np.array_equal(part, np.repeat(np.arange(k), per))
