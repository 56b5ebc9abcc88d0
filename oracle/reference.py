"""numpy restatement of the reference's PyTorch path for clustered sparse decode attention:
TEST INFRASTRUCTURE ONLY (tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg).

Float-level statements of the reference functions, in float64 unless noted:
  label_weighted_attention   src/ssa/attn/labeled.py:24-44
  dense                      src/ssa/attn/dense.py:16-21 (via geometry.attn_weights :39-45)
  merge                      _merge, src/ssa/kernels/labeled_attn.py:154-160
  rank_mask                  SphereIndexGPU._rank_mask, src/ssa/attn/sphere_gpu.py:402-410 (stable order)
  bisect_padded              _bisect_padded, src/ssa/attn/sphere_gpu.py:76-102
  spherical_kmeans           src/ssa/attn/clusterkv.py:27-46
  overhead_rows / kv_read_fraction   src/ssa/attn/accounting.py:19-32
``SphereIndexRef`` restates SphereIndexGPU (src/ssa/attn/sphere_gpu.py:113-442) for the
k-means partition without splitting (the configuration of the benchmarked workload); it is the
CPU baseline that bench.py times.
"""

from __future__ import annotations

import math

import numpy as np


def _softmax(x: np.ndarray, axis: int = -1) -> np.ndarray:
    m = np.max(x, axis=axis, keepdims=True)
    m = np.where(np.isfinite(m), m, 0.0)
    e = np.exp(x - m)
    return e / e.sum(axis=axis, keepdims=True)


def label_weighted_attention(q, K, V, labels, w):
    """``q [H, d]``, ``K, V [H_kv, n, d]``, ``labels [H_kv, n]``, ``w [H_kv or H, L]`` -> ``[H, d]``
    (float64)."""
    q = np.asarray(q, np.float64)
    K = np.asarray(K, np.float64)
    V = np.asarray(V, np.float64)
    w = np.asarray(w, np.float64)
    H, d = q.shape
    H_kv, n, _ = K.shape
    G = H // H_kv
    lab = np.asarray(labels, np.int64)[:, :n]
    if w.shape[0] == H_kv:
        wr = np.repeat(np.take_along_axis(w, lab, 1), G, 0)
    elif w.shape[0] == H:
        wr = np.take_along_axis(w, np.repeat(lab, G, 0), 1)
    else:
        raise ValueError(f"w has {w.shape[0]} rows; expected H_kv={H_kv} or H={H}")
    Kx = np.repeat(K, G, 0)
    s = np.einsum("hd,hnd->hn", q, Kx) / math.sqrt(d)
    with np.errstate(divide="ignore"):
        logw = np.where(wr > 0, np.log(np.maximum(wr, 1e-300)), -np.inf)
    A = _softmax(s + logw, -1)
    Vx = np.where((wr > 0)[..., None], np.repeat(V, G, 0), 0.0)
    return np.einsum("hn,hnd->hd", A, Vx)


def label_weighted_attention_f32(q, K, V, labels, w):
    """The same quantity in float32 with BLAS products per KV head (the reference computes in
    float32 for bf16 / fp32 caches, src/ssa/attn/geometry.py:20-24); shared ``w [H_kv, L]`` only."""
    q = np.asarray(q, np.float32)
    H, d = q.shape
    H_kv, n, _ = K.shape
    G = H // H_kv
    out = np.empty((H, d), np.float32)
    scale = np.float32(1.0 / math.sqrt(d))
    for h in range(H_kv):
        wr = np.asarray(w, np.float32)[h][np.asarray(labels[h, :n], np.int64)]
        sel = np.nonzero(wr > 0)[0]                                          # only these rows are read
        s = (K[h, sel] @ q[h * G:(h + 1) * G].T) * scale + np.log(wr[sel])[:, None]    # [rows, G]
        s = s - s.max(0, keepdims=True)
        p = np.exp(s)
        p /= p.sum(0, keepdims=True)
        out[h * G:(h + 1) * G] = p.T @ V[h, sel]
    return out


def dense(q, K, V):
    """Exact ``softmax(q K^T / sqrt(d)) V`` with ``K, V [H_kv, n, d]`` -> ``[H, d]`` (float64)."""
    H_kv, n, _ = np.shape(K)
    return label_weighted_attention(q, K, V, np.zeros((H_kv, n), np.int64), np.ones((H_kv, 1)))


def merge(m, l, a):
    """Log-sum-exp merge of natural-log split partials ``m, l [H_kv, S, G]``, ``a [H_kv, S, G, d]``."""
    m = np.asarray(m, np.float64)
    M = m.max(1, keepdims=True)
    f = np.exp(m - M)
    den = (f * np.asarray(l, np.float64)).sum(1)
    num = (f[..., None] * np.asarray(a, np.float64)).sum(1)
    H_kv, G, d = num.shape
    return (num / den[..., None]).reshape(H_kv * G, d)


def rank_mask(e: np.ndarray, count: np.ndarray, need: int) -> np.ndarray:
    """Rows of ``e [R, C]``: take clusters in decreasing ``e`` (ties: lowest index first) until
    their counts reach ``need``."""
    R, C = e.shape
    order = np.argsort(-e, axis=1, kind="stable")
    cum = np.cumsum(np.take_along_axis(count, order, 1), 1)
    n_sel = (cum < need).sum(1) + 1
    rank = np.empty_like(order)
    np.put_along_axis(rank, order, np.broadcast_to(np.arange(C), (R, C)), 1)
    return rank < n_sel[:, None]


def selection_keys(q, sum_dir, mmax, mmin, count, n_c, *, group="sum_share", dtype=np.float64):
    """Cluster scores of ``labels_and_weights`` (src/ssa/attn/sphere_gpu.py:426-440): per KV
    head ``e [G, C]`` (per_head) or the shared key ``[C]``; ``-inf`` for empty or spare slots."""
    q = np.asarray(q, dtype)
    sd = np.asarray(sum_dir, dtype)
    H_kv, C, d = sd.shape
    G = q.shape[0] // H_kv
    cdir = sd / np.maximum(np.linalg.norm(sd, axis=-1, keepdims=True), 1e-12)
    p = np.einsum("hgd,hcd->hgc", q.reshape(H_kv, G, d), cdir)
    mx = np.asarray(mmax, dtype)[:, None, :]
    mn = np.asarray(mmin, dtype)[:, None, :]
    with np.errstate(invalid="ignore"):
        e = np.where(p >= 0, mx * p, mn * p)
    live = (np.asarray(count) > 0) & (np.arange(C)[None, :] < np.asarray(n_c)[:, None])
    e = np.where(live[:, None, :], e, -np.inf)
    if group == "per_head":
        return e
    z = e / math.sqrt(d)
    if group == "max":
        shared = z.max(1)
    elif group == "max_rel":
        shared = (z - z.max(2, keepdims=True)).max(1)
    else:
        shared = _softmax(z, 2).sum(1)
    return np.where(live, shared, -np.inf)


def labels_and_weights(q, sum_dir, mmax, mmin, count, n_c, *, nb: int, budget: float, group="sum_share"):
    """``w`` of SphereIndexGPU.labels_and_weights from the summaries (float64 scores)."""
    sd = np.asarray(sum_dir)
    H_kv, C, _ = sd.shape
    H = np.shape(q)[0]
    G = H // H_kv
    rows = H if group == "per_head" else H_kv
    w = np.zeros((rows, C + 1), np.float32)
    w[:, C] = 1.0
    need = math.ceil(budget * nb)
    if nb <= 0 or need <= 0:
        return w
    keys = selection_keys(q, sum_dir, mmax, mmin, count, n_c, group=group)
    cnt = np.where(np.arange(C)[None, :] < np.asarray(n_c)[:, None], np.asarray(count), 0).astype(np.int64)
    if group == "per_head":
        take = rank_mask(keys.reshape(H, C), np.repeat(cnt, G, 0), need)
        live = np.repeat(cnt > 0, G, 0)
    else:
        take = rank_mask(keys, cnt, need)
        live = cnt > 0
    w[:, :C] = (take & live).astype(np.float32)
    return w


def bisect_padded(Kn: np.ndarray, valid: np.ndarray, min_share: float = 0.25, iters: int = 4) -> np.ndarray:
    """Split each row of unit vectors ``Kn [S, M, d]`` in two: 2-means from the first member and
    the member least similar to it; a lopsided result is replaced by a cut at the median
    projection on the line between the two centroids. Returns ``side [S, M]``."""
    Kn = np.asarray(Kn, np.float64)
    S, M, d = Kn.shape
    cnt = valid.sum(1)
    sim0 = np.einsum("smd,sd->sm", Kn, Kn[:, 0])
    far = np.where(valid, sim0, np.inf).argmin(1)
    two = np.stack([Kn[:, 0], Kn[np.arange(S), far]], 1).copy()
    Kv = Kn * valid[..., None]

    def nrm(x):
        return x / np.maximum(np.linalg.norm(x, axis=-1, keepdims=True), 1e-12)

    for it in range(iters + 1):
        sim = np.einsum("smd,sjd->smj", Kn, two)
        side = (sim[..., 1] > sim[..., 0]) & valid
        if it == iters:
            break
        s1 = (Kv * side[..., None]).sum(1)
        s0 = Kv.sum(1) - s1
        n1 = side.sum(1)
        two = np.stack([np.where((cnt - n1 > 0)[:, None], nrm(s0), two[:, 0]),
                        np.where((n1 > 0)[:, None], nrm(s1), two[:, 1])], 1)
    n1 = side.sum(1)
    lopsided = (n1 < min_share * cnt) | (n1 > (1 - min_share) * cnt)
    proj = np.where(valid, np.einsum("smd,sd->sm", Kn, two[:, 1] - two[:, 0]), np.inf)
    order = np.argsort(proj, axis=1, kind="stable")
    rank = np.empty_like(order)
    np.put_along_axis(rank, order, np.broadcast_to(np.arange(M), (S, M)), 1)
    upper = (rank >= (cnt // 2)[:, None]) & valid
    return np.where(lopsided[:, None], upper, side).astype(np.int64)


def normalize(X: np.ndarray) -> np.ndarray:
    return X / np.maximum(np.linalg.norm(X, axis=-1, keepdims=True), 1e-12)


def spherical_kmeans(X: np.ndarray, *, C: int, iters: int = 10, init: np.ndarray):
    """Cosine k-means, batched over heads: ``X [h, m, d]`` -> ``assign [h, m]``, unit
    ``centroids [h, C, d]``, from the members at ``init [C]`` (the same for every head); an empty
    cluster keeps its previous centroid. Ties go to the lowest index (``argmax``)."""
    X = np.asarray(X)
    h, m, d = X.shape
    Xn = normalize(X)
    cent = Xn[:, init].copy()
    assign = None
    for _ in range(iters):
        assign = np.matmul(Xn, cent.transpose(0, 2, 1)).argmax(-1)
        sums = np.zeros((h, C, d), X.dtype)
        cnt = np.zeros((h, C), np.int64)
        for i in range(h):
            np.add.at(sums[i], assign[i], Xn[i])
            np.add.at(cnt[i], assign[i], 1)
        cent = np.where((cnt > 0)[..., None], normalize(sums), cent)
    assign = np.matmul(Xn, cent.transpose(0, 2, 1)).argmax(-1)
    return assign, cent


def overhead_rows(*, n, rows, clusters, d: int, summary_bits: int = 8, fitted: bool = True, heads: int = 1,
                  key_bits: int = 16):
    """Key-row equivalents read per KV head per step besides the ``rows`` K and V rows."""
    row = d * key_bits / 8
    vec = d * summary_bits / 8
    summaries = clusters * (vec + 12)
    centroids = clusters * vec if fitted else clusters * 4 * d / heads
    return (summaries + centroids + 2 * n + 6 * rows + row + 8 * d) / row


def kv_read_fraction(*, n, rows, clusters, d: int, **kw):
    return (2 * rows + overhead_rows(n=n, rows=rows, clusters=clusters, d=d, **kw)) / (2 * n)


class SphereIndexRef:
    """SphereIndexGPU (k-means partition, no splitting) in numpy float32: ``observe`` bins keys
    leaving the window into their nearest fitted centroid, ``labels_and_weights`` scores and
    selects clusters, and ``attend`` runs ``label_weighted_attention`` over the whole cache as
    the reference's CPU path does."""

    def __init__(self, *, C: int = 256, window: int = 64, kmeans_iters: int = 10, seed: int = 0,
                 init_indices=None):
        self.C, self.window, self.iters, self.seed = C, window, kmeans_iters, seed
        self.init_indices = init_indices     # callable (m, C, seed) -> indices
        self.initialized = False
        self.n = 0

    def _init(self, K: np.ndarray, n: int) -> None:
        H_kv, _, d = K.shape
        C = self.C
        self.start, self.end = 1, max(1, n - self.window)
        Kb = K[:, self.start:self.end].astype(np.float32)
        nb = Kb.shape[1]
        self.mu = Kb.mean(1)
        self.ksum = Kb.sum(1)
        Kr = Kb - self.mu[:, None]
        init = np.asarray(self.init_indices(nb, C, self.seed))
        _, cent = spherical_kmeans(Kr, C=C, iters=self.iters, init=init)
        self.cent = cent.astype(np.float32)
        self.labels = np.full((H_kv, K.shape[1]), C, np.int16)
        self.sum_dir = np.zeros((H_kv, C, d), np.float32)
        self.mmax = np.zeros((H_kv, C), np.float32)
        self.mmin = np.full((H_kv, C), np.inf, np.float32)
        self.count = np.zeros((H_kv, C), np.float32)
        self._bin(Kr, self.start)
        self.initialized = True

    def _bin(self, Kr: np.ndarray, p0: int) -> None:
        mag = np.linalg.norm(Kr, axis=-1)
        Kn = Kr / np.maximum(mag, 1e-12)[..., None]
        lab = np.matmul(Kn, self.cent.transpose(0, 2, 1)).argmax(-1)
        for h in range(Kr.shape[0]):
            np.add.at(self.sum_dir[h], lab[h], Kn[h])
            np.maximum.at(self.mmax[h], lab[h], mag[h])
            np.minimum.at(self.mmin[h], lab[h], mag[h])
            np.add.at(self.count[h], lab[h], 1.0)
        self.labels[:, p0:p0 + Kr.shape[1]] = lab

    def observe(self, K: np.ndarray, n: int) -> None:
        if not self.initialized or n < self.n:
            self._init(K, n)
        else:
            new_end = max(1, n - self.window)
            if new_end > self.end:
                Kn = K[:, self.end:new_end].astype(np.float32)
                self.ksum += Kn.sum(1)
                self._bin(Kn - self.mu[:, None], self.end)
                self.end = new_end
        self.n = n

    def labels_and_weights(self, q: np.ndarray, *, n: int, budget: float):
        H_kv, C = self.count.shape
        n_c = np.full(H_kv, C)
        w = labels_and_weights(q.astype(np.float32), self.sum_dir, self.mmax, self.mmin, self.count, n_c,
                               nb=self.end - self.start, budget=budget)
        return self.labels[:, :n], w

    def attend(self, q, K, V, *, n: int, budget: float, fast: bool = False):
        self.observe(K, n)
        labels, w = self.labels_and_weights(q, n=n, budget=budget)
        f = label_weighted_attention_f32 if fast else label_weighted_attention
        return f(q, K[:, :n], V[:, :n], labels, w), labels, w
