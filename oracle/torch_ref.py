"""PyTorch-CPU restatement of the reference's pure-PyTorch decode path, as that path computes it:
TEST INFRASTRUCTURE ONLY (bench.py's cpu_baseline leg times it; nothing in the product imports it).

The reference runs the same index on the CPU ("Pure PyTorch, so it runs on CPU as well",
src/ssa/attn/sphere_gpu.py:11). Per decode step of one layer that is:
  * ``observe``: keys that leave the recent window are centred with ``mu_ref``, normalised and
    binned into their nearest fitted centroid, and the summaries (sum of directions, longest /
    shortest centred key, count) are updated (SphereIndexGPU._bin, src/ssa/attn/sphere_gpu.py:166-184);
  * ``labels_and_weights``: every cluster is scored from its summary, the per-head softmaxes over
    clusters are summed ("sum_share") and clusters are taken in decreasing score until their keys
    reach the budget (src/ssa/attn/sphere_gpu.py:402-442);
  * ``label_weighted_attention``: scores of the query against EVERY cached key, masked by the
    label weights, softmax, and the value sum with unread rows zeroed
    (src/ssa/attn/labeled.py:24-44).
All of it in float32 (``_accum_dtype``, src/ssa/attn/geometry.py:20-24), as the reference
computes a bf16 or fp32 cache. The prefill fit is ``spherical_kmeans``
(src/ssa/attn/clusterkv.py:27-46): 10 iterations of cosine k-means from seeded members. This is
the k-means partition without splitting: the configuration of the benchmarked workload.
"""

from __future__ import annotations

import math

import torch


def spherical_kmeans(X: torch.Tensor, C: int, iters: int, init: torch.Tensor):
    """``X [h, m, d]`` -> (assign [h, m], unit centroids [h, C, d]); an empty cluster keeps its
    centroid; argmax ties to the lowest index."""
    Xn = X / X.norm(dim=-1, keepdim=True).clamp_min(1e-12)
    cent = Xn[:, init].clone()
    h, m, d = X.shape
    for _ in range(iters):
        assign = torch.einsum("hmd,hcd->hmc", Xn, cent).argmax(-1)
        sums = torch.zeros(h, C, d, dtype=X.dtype).scatter_add_(1, assign[..., None].expand(-1, -1, d), Xn)
        cnt = torch.zeros(h, C, dtype=X.dtype).scatter_add_(1, assign, torch.ones_like(assign, dtype=X.dtype))
        cent = torch.where((cnt > 0)[..., None], sums / sums.norm(dim=-1, keepdim=True).clamp_min(1e-12), cent)
    assign = torch.einsum("hmd,hcd->hmc", Xn, cent).argmax(-1)
    return assign, cent


def label_weighted_attention(q, K, V, labels, w):
    """``q [H, d]``, ``K, V [H_kv, n, d]``, ``labels [H_kv, n]``, ``w [H_kv, L]`` -> ``[H, d]``, every
    key scored and masked, as the reference computes it."""
    H, d = q.shape
    H_kv, n, _ = K.shape
    G = H // H_kv
    wr = torch.gather(w, 1, labels.long()).repeat_interleave(G, 0)
    s = torch.einsum("hd,hnd->hn", q, K.repeat_interleave(G, 0)) / math.sqrt(d)
    logw = torch.where(wr > 0, wr.clamp_min(1e-30).log(), torch.full_like(wr, -math.inf))
    A = torch.softmax(s + logw, dim=-1)
    Vx = torch.where((wr > 0).unsqueeze(-1), V.repeat_interleave(G, 0), torch.zeros((), dtype=V.dtype))
    return torch.einsum("hn,hnd->hd", A, Vx)


class SphereIndexTorch:
    """The reference CPU index (k-means partition, no splitting) on torch CPU tensors, float32."""

    def __init__(self, *, C: int = 256, window: int = 64, kmeans_iters: int = 10, init_indices=None):
        self.C, self.window, self.iters = C, window, kmeans_iters
        self.init_indices = init_indices            # callable (m, C) -> LongTensor
        self.initialized = False

    def _init(self, K: torch.Tensor, n: int) -> None:
        H_kv, _, d = K.shape
        C = self.C
        self.start, self.end = 1, max(1, n - self.window)
        Kb = K[:, self.start:self.end].float()
        self.mu = Kb.mean(1)
        self.ksum = Kb.sum(1)
        _, self.cent = spherical_kmeans(Kb - self.mu[:, None], C, self.iters, self.init_indices(Kb.shape[1], C))
        self.labels = torch.full((H_kv, K.shape[1]), C, dtype=torch.int16)
        self.sum_dir = torch.zeros(H_kv, C, d)
        self.mmax = torch.zeros(H_kv, C)
        self.mmin = torch.full((H_kv, C), math.inf)
        self.count = torch.zeros(H_kv, C)
        self._bin(Kb - self.mu[:, None], self.start)
        self.initialized = True

    def _bin(self, Kr: torch.Tensor, p0: int) -> None:
        mag = Kr.norm(dim=-1)
        Kn = Kr / mag.clamp_min(1e-12)[..., None]
        lab = torch.einsum("hmd,hcd->hmc", Kn, self.cent).argmax(-1)
        d = Kr.shape[-1]
        self.sum_dir.scatter_add_(1, lab[..., None].expand(-1, -1, d), Kn)
        self.mmax.scatter_reduce_(1, lab, mag, reduce="amax")
        self.mmin.scatter_reduce_(1, lab, mag, reduce="amin")
        self.count.scatter_add_(1, lab, torch.ones_like(mag))
        self.labels[:, p0:p0 + Kr.shape[1]] = lab.to(torch.int16)

    def observe(self, K: torch.Tensor, n: int) -> None:
        if not self.initialized:
            self._init(K, n)
            return
        new_end = max(1, n - self.window)
        if new_end > self.end:
            Kn = K[:, self.end:new_end].float()
            self.ksum += Kn.sum(1)
            self._bin(Kn - self.mu[:, None], self.end)
            self.end = new_end

    def labels_and_weights(self, q: torch.Tensor, *, n: int, budget: float):
        H_kv, C = self.count.shape
        H, d = q.shape
        G = H // H_kv
        need = math.ceil(budget * (self.end - self.start))
        cdir = self.sum_dir / self.sum_dir.norm(dim=-1, keepdim=True).clamp_min(1e-12)
        p = torch.einsum("hgd,hcd->hgc", q.view(H_kv, G, d), cdir)
        e = torch.where(p >= 0, self.mmax[:, None] * p, self.mmin[:, None] * p)
        live = self.count > 0
        z = torch.where(live[:, None], e / math.sqrt(d), torch.full_like(e, -math.inf))
        shared = torch.where(live, torch.softmax(z, -1).sum(1), torch.full_like(self.count, -math.inf))
        order = shared.argsort(dim=1, descending=True)
        cum = torch.gather(self.count, 1, order).cumsum(1)
        n_sel = (cum < need).sum(1, keepdim=True) + 1
        take = torch.zeros(H_kv, C, dtype=torch.bool).scatter_(1, order, torch.arange(C).expand(H_kv, C) < n_sel)
        w = torch.zeros(H_kv, C + 1)
        w[:, :C] = (take & live).float()
        w[:, C] = 1.0
        return self.labels[:, :n], w

    def attend(self, q, K, V, *, n: int, budget: float):
        self.observe(K, n)
        labels, w = self.labels_and_weights(q, n=n, budget=budget)
        return label_weighted_attention(q, K[:, :n], V[:, :n], labels, w), labels, w
