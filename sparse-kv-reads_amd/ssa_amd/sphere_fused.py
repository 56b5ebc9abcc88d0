"""The incremental cluster index on the HIP kernels (``SphereIndexFused``).

Mirrors the reference's ``SphereIndexFused`` (src/ssa/kernels/sphere_fused.py:316-519), whose
semantics are those of ``SphereIndexGPU`` (src/ssa/attn/sphere_gpu.py:113-442): one instance per
layer holds every KV head's clusters as batched device tensors. Keys are binned once, when they
leave the recent window, centred with ``mu_ref``; a head is recentred and rebinned when its
running mean drifts by more than ``delta * rbar``. With ``partition="kmeans"`` the ``C_init``
centroids of each head are fitted by cosine k-means on the centred prompt keys and kept; later
keys join their nearest centroid, and a cluster that passes its size cap is split in two inside
the insertion kernel.

All arithmetic runs in libssa_hip.so (insertion ``ssa_insert``, selection ``ssa_select``, prefill
``ssa_build``, selection + attention ``ssa_sparse_step``); the host only allocates state, keeps the
counters the reference keeps, and reads the drift flags every ``check_every`` steps (without a
synchronisation when ``async_check``).

Differences from the reference, all deliberate:
  * selection ranks clusters by (score desc, index asc): a stable sort, where the reference's
    torch index breaks ties arbitrarily and its Triton kernel takes every tied cluster;
  * counts are int32 (exact) rather than float32;
  * decisions use the canonical fp32 arithmetic of csrc/ssa_common.h, so a CPU restatement
    reproduces labels, selections and splits bit for bit.
"""

from __future__ import annotations

import math

import numpy as np
import torch

from ._lib import (STAGE_WORDS, BuildArgs, IndexState, InsertArgs, SelectArgs, SplitArgs, check, dtype_tag, lib,
                   ptr, require_cuda, stream_ptr)
from .labeled_attn import _work, attn_args, default_splits

GROUPS = ("per_head", "max", "max_rel", "sum_share")
_GROUP_ID = {"sum_share": 0, "per_head": 1, "max": 2, "max_rel": 3}


def fixed_directions(C: int, d: int, *, seed: int = 0, kind: str = "random", dtype=torch.float32, device="cpu"):
    """``C`` fixed unit vectors in ``R^d`` (``partition="random"``), drawn as the reference draws
    them (src/ssa/attn/sphere_skip.py:46-68): i.i.d. normal from a seeded CPU generator in
    float64, normalised. ``cross`` gives the first ``C`` signed coordinate axes."""
    if kind == "random":
        g = torch.Generator(device="cpu").manual_seed(seed)
        x = torch.randn(C, d, generator=g, dtype=torch.float64)
    elif kind == "cross":
        if C > 2 * d:
            raise ValueError("cross partition has at most 2d directions")
        eye = torch.eye(d, dtype=torch.float64)
        x = torch.cat([eye, -eye])[:C]
    else:
        raise ValueError(f"unknown direction kind {kind!r}")
    return (x / x.norm(dim=1, keepdim=True)).to(device=device, dtype=dtype)


def kmeans_init_indices(m: int, C: int, seed: int) -> torch.Tensor:
    """The k-means seed members, as ``spherical_kmeans`` picks them (src/ssa/attn/clusterkv.py:34-35):
    the first ``C`` entries (cycled) of a seeded CPU ``randperm(m)``, the same for every head."""
    g = torch.Generator(device="cpu").manual_seed(seed)
    return torch.randperm(m, generator=g)[torch.arange(C) % m]


class SphereIndexFused:
    BUILD_HEADS = 64          # heads (re)built per ssa_build call
    KN_ROWS = 512             # members of a splitting cluster whose unit directions are kept (knbuf)

    def __init__(self, *, C: int = 256, window: int = 64, delta: float = 0.03, capacity: int = 65536,
                 check_every: int = 16, seed: int = 0, kind: str = "random", partition: str = "random",
                 kmeans_iters: int = 10, C_init: int | None = None, split_factor: float = 0.0,
                 grow_cap: bool = False, reset_at: int = 0, cap_keys: float = 0.0, var_factor: float = 0.0,
                 var_min: int = 8, async_check: bool = True, max_lag: int = 2, split_scratch: int = 8192,
                 summary_bits: int = 8):
        # argument checks as in SphereIndexGPU.__init__ (src/ssa/attn/sphere_gpu.py:119-128) and
        # SphereIndexFused.__init__ (src/ssa/kernels/sphere_fused.py:339-340)
        if summary_bits not in (8, 32):
            raise ValueError("summary_bits must be 8 or 32")
        if partition not in ("random", "kmeans"):
            raise ValueError(f"unknown partition {partition!r}")
        if not (C >= 16 and C & (C - 1) == 0 and C <= 1024):
            raise AssertionError("C must be a power of two in [16, 1024]")
        self.partition, self.kmeans_iters = partition, kmeans_iters
        self.C_init = C if C_init is None else C_init
        self.cap_keys = float(cap_keys)
        self.split_factor = float(split_factor) if split_factor or not cap_keys else 2.0
        self.var_factor, self.var_min = float(var_factor), int(var_min)
        self.splitting = self.split_factor > 0 or self.var_factor > 0
        if self.C_init > C or (self.splitting and partition != "kmeans"):
            raise ValueError("C_init must be <= C, and splitting needs partition='kmeans'")
        self.summary_bits = summary_bits
        self.capk = self.split_factor / self.C_init if grow_cap else 0.0
        self.reset_at = reset_at
        self.resets = 0
        self.C, self.window, self.delta, self.capacity = C, window, delta, capacity
        self.check_every, self.seed, self.kind = check_every, seed, kind
        self.async_check, self.max_lag, self.split_scratch = async_check, max_lag, split_scratch
        self.initialized = False
        self.n = 0
        self.start = 1
        self.end = 0
        self.rebuilds = 0
        self.head_steps = 0
        self._steps = 0
        self._splits_host = 0
        self._fresh_fit = False
        self._pending = None
        self._waited = 0
        self._w = {}
        self.nsplit = None

    # -- state ---------------------------------------------------------------------------
    def _alloc(self, H_kv: int, d: int, device) -> None:
        C = self.C
        f32 = dict(dtype=torch.float32, device=device)
        self.H_kv, self.d, self.device, self.dtype = H_kv, d, device, torch.float32
        self.MS = min(self.split_scratch, self.capacity)
        kmeans = self.partition == "kmeans"
        self.n_c = torch.full((H_kv,), self.C_init if kmeans else C, dtype=torch.int32, device=device)
        self.fitted = [False] * H_kv
        self.sum_dir = torch.zeros(H_kv, C, d, **f32)
        self.dir8 = torch.zeros(H_kv, C, d, dtype=torch.int8, device=device) if self.summary_bits == 8 else None
        if kmeans:
            self.cent = torch.zeros(H_kv, C, d, **f32)
            self.cent8 = torch.zeros_like(self.dir8) if self.dir8 is not None else None
        else:
            self.cent = fixed_directions(C, d, seed=self.seed, kind=self.kind, device=device)
            self.cent8 = None
        self.mmax = torch.zeros(H_kv, C, **f32)
        self.mmin = torch.full((H_kv, C), math.inf, **f32)
        self.count = torch.zeros(H_kv, C, dtype=torch.int32, device=device)
        self.ksum = torch.zeros(H_kv, d, **f32)
        self.mu_ref = torch.zeros(H_kv, d, **f32)
        self.rbar = torch.zeros(H_kv, **f32)
        self.cap = torch.full((H_kv,), math.inf, **f32)
        self.vthr = torch.full((H_kv,), math.inf, **f32)
        self.flags = torch.zeros(H_kv, dtype=torch.int32, device=device)
        self.end_dev = torch.zeros(H_kv, dtype=torch.int32, device=device)
        self.nsplit = torch.zeros(H_kv, dtype=torch.int32, device=device)
        self.labels = torch.full((H_kv, self.capacity), C, dtype=torch.int16, device=device)
        self._mem = torch.zeros(H_kv, self.MS, dtype=torch.int32, device=device)
        self._proj = torch.zeros(H_kv, self.MS, **f32)
        self._side = torch.zeros(H_kv, self.MS, dtype=torch.int32, device=device)
        self._smag = torch.zeros(H_kv, self.MS, **f32)
        self._stage = torch.zeros(H_kv, STAGE_WORDS, dtype=torch.int32, device=device)
        # unit directions of a splitting cluster's members, computed once per split (the split's
        # passes otherwise divide every element again); clusters past KN_ROWS members recompute
        self.kn_rows = min(self.MS, self.KN_ROWS) if self.splitting else 0
        self._knbuf = torch.empty(H_kv, self.kn_rows, d, **f32) if self.kn_rows else None
        self._flags_host = torch.zeros(H_kv, dtype=torch.int32, pin_memory=True)
        self._pending = None
        self._w = {}

    def _state(self, layers: int = 1) -> IndexState:
        """The C-ABI view of this index's state (all layers' arrays when stacked)."""
        big = getattr(self, "_stacked", None)
        src = big if (big is not None and layers > 1) else None

        def p(name):
            t = src.get(name, getattr(self, name)) if src is not None else getattr(self, name)
            return ptr(t)

        s = IndexState()
        s.n_heads, s.heads_per_layer = self.H_kv * layers, self.H_kv
        s.C, s.d, s.capacity, s.ms = self.C, self.d, self.capacity, self.MS
        s.summary_bits = self.summary_bits
        s.shared_dirs = int(self.partition != "kmeans")
        s.n_c, s.sum_dir, s.dir8, s.cent, s.cent8 = p("n_c"), p("sum_dir"), p("dir8"), p("cent"), p("cent8")
        s.mmax, s.mmin, s.count = p("mmax"), p("mmin"), p("count")
        s.ksum, s.mu_ref, s.rbar, s.cap, s.vthr = p("ksum"), p("mu_ref"), p("rbar"), p("cap"), p("vthr")
        s.flags, s.end, s.nsplit, s.labels = p("flags"), p("end_dev"), p("nsplit"), p("labels")
        s.mem, s.proj, s.side, s.smag = p("_mem"), p("_proj"), p("_side"), p("_smag")
        s.stage = p("_stage")
        s.knbuf, s.kn_rows = p("_knbuf"), self.kn_rows
        return s

    def _insert_args(self, K: torch.Tensor, *, n_host: int = 0, n_dev: torch.Tensor | None = None,
                     koff: torch.Tensor | None = None) -> InsertArgs:
        a = InsertArgs()
        a.k, a.k_dtype, a.s_kh, a.s_kn = K.data_ptr(), dtype_tag(K.dtype), K.stride(0), K.stride(1)
        a.koff = ptr(koff)
        a.n_dev, a.n_host = ptr(n_dev), int(n_host)
        a.window, a.delta, a.capk = self.window, float(self.delta), float(self.capk)
        a.reset_at = self.reset_at or 2 ** 30
        a.var_min = self.var_min
        return a

    # -- prefill ---------------------------------------------------------------------------
    def _build(self, K: torch.Tensor, heads: torch.Tensor, mu: torch.Tensor | None) -> None:
        """(Re)build the clusters of ``heads`` from binned keys ``K[heads, start:end]``; heads not
        yet fitted are fitted first (k-means with ``C_init`` clusters)."""
        hl = [int(h) for h in heads.tolist()]
        if not hl:
            return
        todo = [h for h in hl if self.partition == "kmeans" and not self.fitted[h]]
        keep = [h for h in hl if h not in todo]
        pos = {h: i for i, h in enumerate(hl)}
        for group, fit in ((todo, True), (keep, False)):
            # at most BUILD_HEADS heads per pass: the scratch is ~2 x heads x keys x d fp32
            for i in range(0, len(group), self.BUILD_HEADS):
                part = group[i:i + self.BUILD_HEADS]
                sel_mu = None if mu is None else mu[[pos[h] for h in part]].to(torch.float32).contiguous()
                self._build_heads(K, part, sel_mu, fit)

    def _build_heads(self, K, heads: list[int], mu, fit: bool) -> None:
        dev, d, C = self.device, self.d, self.C
        nb = max(0, self.end - self.start)
        ns = len(heads)
        nblk = -(-nb // 256)
        ncl = max(C, self.C_init)
        hd = torch.tensor(heads, dtype=torch.int32, device=dev)
        xn = torch.empty(ns, max(nb, 1), d, dtype=torch.float32, device=dev)
        mag = torch.empty(ns, max(nb, 1), dtype=torch.float32, device=dev)
        sq = torch.empty_like(mag)
        assign = torch.empty(ns, max(nb, 1), dtype=torch.int32, device=dev)
        part = torch.empty(ns, max(nblk, 1), ncl, d, dtype=torch.float32, device=dev)
        part_cnt = torch.empty(ns, max(nblk, 1), ncl, dtype=torch.int32, device=dev)
        init = None
        if fit and nb:
            init = kmeans_init_indices(nb, self.C_init, self.seed).to(torch.int32).to(dev)
        b = BuildArgs()
        b.k, b.k_dtype, b.s_kh, b.s_kn = K.data_ptr(), dtype_tag(K.dtype), K.stride(0), K.stride(1)
        b.heads, b.n_sel, b.start, b.end = hd.data_ptr(), ns, self.start, self.start + nb
        b.mu = ptr(mu)
        b.xn, b.mag, b.sq, b.assign = xn.data_ptr(), mag.data_ptr(), sq.data_ptr(), assign.data_ptr()
        b.part, b.part_cnt = part.data_ptr(), part_cnt.data_ptr()
        b.init_idx = ptr(init)
        b.fit = int(fit and nb > 0)
        b.C_fit, b.iters = self.C_init, self.kmeans_iters
        check(lib().ssa_build(self._state(), b, stream_ptr(dev)), "ssa_build")
        if fit and nb > 0:
            for h in heads:
                self.fitted[h] = True
            if self.split_factor > 0:
                cap = self.cap_keys or self.split_factor * nb / self.C_init
                self.cap[hd.long()] = cap
                self._fresh_fit = True
            if self.var_factor > 0:
                used = (self.count[hd.long()] > 0).float()
                self.vthr[hd.long()] = self.var_factor * (self._spread()[hd.long()] * used).sum(1) / \
                    used.sum(1).clamp_min(1)
        elif fit:
            self.n_c[hd.long()] = self.C_init

    def _spread(self) -> torch.Tensor:
        """Per cluster, ``1 - |sum of directions|^2 / count^2`` (0 for an empty cluster)."""
        cnt = self.count.float()
        return (1 - self.sum_dir.pow(2).sum(-1) / cnt.clamp_min(1).pow(2)).clamp_min(0) * (cnt > 0)

    def _init(self, K: torch.Tensor, n: int) -> None:
        H_kv, _, d = K.shape
        if n > self.capacity:
            raise ValueError(f"n={n} exceeds capacity {self.capacity}")
        require_cuda(K)
        self._alloc(H_kv, d, K.device)
        self.start = 1
        self.end = max(1, n - self.window)
        self._build(K, torch.arange(H_kv), None)
        self._split_after_fit(K)
        self.initialized = True

    def _split_after_fit(self, K) -> None:
        if self._fresh_fit:
            self._fresh_fit = False
            self._split_overflow(K, None, nmeans=True)

    def _split_overflow(self, K, cand=None, nmeans: bool = False) -> None:
        """Division of the clusters over their cap right after a fit, in rounds of ``ssa_split_fit``
        (src/ssa/attn/sphere_gpu.py:307-338; src/ssa/kernels/sphere_fused.py:411-413): a k-means
        round, then bisection rounds until no cluster is over its cap or a round divides nothing;
        then the int8 copies. One host synchronisation per round, as in the reference."""
        if not self.splitting:
            return
        H_kv, dev = self.H_kv, self.device
        heads = torch.arange(H_kv, dtype=torch.int32, device=dev)
        ms = max(int(self.count.max()), 2)                            # host sync
        i32 = dict(dtype=torch.int32, device=dev)
        mem, side = torch.empty(H_kv, ms, **i32), torch.empty(H_kv, ms, **i32)
        proj = torch.empty(H_kv, ms, dtype=torch.float32, device=dev)
        smag = torch.empty_like(proj)
        over, done = torch.zeros(H_kv, **i32), torch.zeros(H_kv, **i32)
        a = SplitArgs()
        a.k, a.k_dtype, a.s_kh, a.s_kn = K.data_ptr(), dtype_tag(K.dtype), K.stride(0), K.stride(1)
        a.heads, a.n_sel = heads.data_ptr(), H_kv
        a.start, a.end = self.start, self.end
        a.split_factor = self.split_factor
        a.cap_min = float(torch.tensor(self.capk * (self.end - self.start), dtype=torch.float32))
        a.iters = self.kmeans_iters
        a.mem, a.side, a.proj, a.smag, a.ms = mem.data_ptr(), side.data_ptr(), proj.data_ptr(), smag.data_ptr(), ms
        a.over, a.done = over.data_ptr(), done.data_ptr()
        # the k-means round divides a cluster of m keys into max(2, ceil(m * split_factor / cap))
        # parts (no upper limit, as in the reference); up to 32 parts are held on chip, more in
        # this scratch, sized for the largest cluster against the smallest cap (float32, as the
        # kernel computes it)
        cap_now = np.maximum(np.float32(self.cap.min().item()), np.float32(a.cap_min))
        k_max = int(np.ceil(np.float32(ms) * np.float32(self.split_factor) / cap_now)) if cap_now > 0 else 2
        parts = None
        if k_max > 32:
            a.max_parts = min(k_max + 1, 1024)
            parts = torch.empty(H_kv, 2, a.max_parts, self.d, dtype=torch.float32, device=dev)
            a.parts = parts.data_ptr()
        st = self._state()
        nmeans = True
        while True:
            a.nmeans, a.refresh_only = int(nmeans), 0
            check(lib().ssa_split_fit(st, a, stream_ptr(dev)), "ssa_split_fit")
            n_over, n_done = int(over.sum()), done.cpu()                  # host sync
            if bool((n_done < 0).any()):
                raise RuntimeError("a cluster would be divided into more than 1024 parts by the post-fit k-means")
            if n_over == 0 or (int(n_done.sum()) == 0 and not nmeans):
                break
            nmeans = False
        a.refresh_only = 1
        check(lib().ssa_split_fit(st, a, stream_ptr(dev)), "ssa_split_fit")

    # -- decode ------------------------------------------------------------------------------
    def observe(self, K: torch.Tensor, n: int) -> None:
        """Update from the cache ``K [H_kv, >= n, d]`` (engine layout) holding ``n`` valid positions."""
        if not self.initialized or n < self.n or K.shape[0] != getattr(self, "H_kv", -1):
            self._init(K, n)
        else:
            self._advance(K, n)
        self.n = n

    def _advance(self, K: torch.Tensor, n: int) -> None:
        new_end = max(1, n - self.window)
        if self.partition == "kmeans" and new_end > self.end and not all(self.fitted):
            self.end = new_end                                   # nothing was binned at the first build
            self._build(K, torch.arange(self.H_kv), None)
            self._split_after_fit(K)
        if new_end > self.end:
            st = self._state()
            check(lib().ssa_insert(st, self._insert_args(K, n_host=n), stream_ptr(self.device)), "ssa_insert")
            self.end = new_end
        self.head_steps += self.H_kv
        if self.end - 1 <= 0:
            return
        self._steps += 1
        if self._steps % self.check_every != 0:
            return
        self._check_flags(K)

    def _check_flags(self, K) -> None:
        if not self.async_check:
            self._act_on(K, self.flags.cpu())                    # host sync
            self.flags.zero_()
            return
        if self._pending is not None:
            self._waited += 1
            if self._waited > self.max_lag and not self._pending.query():
                self._pending.synchronize()
        if self._pending is not None and self._pending.query():
            self._pending = None
            self._act_on(K, self._flags_host.clone())          # host copy: no device sync unless a flag is set
        if self._pending is None:
            self._flags_host.copy_(self.flags, non_blocking=True)
            self._pending = torch.cuda.Event()
            self._pending.record()
            self._waited = 0
            self.flags.zero_()

    def _act_on(self, K, flags: torch.Tensor) -> None:
        """Refit the heads whose cluster count reached the reset threshold; recentre the others
        that drifted (src/ssa/kernels/sphere_fused.py:453-464)."""
        reset = (flags & 2) != 0
        self._reset_heads(K, reset.nonzero().squeeze(1))
        self._rebuild(K, (((flags & 1) != 0) & ~reset).nonzero().squeeze(1))

    def _host_end(self) -> None:
        """Bring ``self.end`` up to date before host-side work (kept on the GPU by subclasses)."""

    def _rebuild(self, K, heads: torch.Tensor) -> None:
        if heads.numel():
            self._host_end()
            mu_t = self.ksum[heads.to(self.device).long()] / (self.end - 1)
            self._build(K, heads.cpu(), mu_t)
            self.rebuilds += int(heads.numel())

    def _reset_heads(self, K, heads: torch.Tensor) -> None:
        if heads.numel() == 0:
            return
        self._host_end()
        for h in heads.tolist():
            self.fitted[int(h)] = False
        self.n_c[heads.to(self.device).long()] = self.C_init
        self._build(K, heads.cpu(), None)
        self._split_after_fit(K)
        self.resets += int(heads.numel())

    # -- selection -------------------------------------------------------------------------------
    def _wbuf(self, group: str, rows: int) -> torch.Tensor:
        key = (group, rows)
        if key not in self._w:
            w = torch.zeros(rows, self.C + 1, dtype=torch.float32, device=self.device)
            w[:, self.C] = 1.0
            self._w[key] = w
        return self._w[key]

    def _select_args(self, q: torch.Tensor, w: torch.Tensor, budget: float, group: str) -> SelectArgs:
        a = SelectArgs()
        a.q, a.q_dtype, a.s_qh = q.data_ptr(), dtype_tag(q.dtype), q.stride(0)
        a.G = q.shape[0] // self.H_kv
        a.w, a.s_wr = w.data_ptr(), w.stride(0)
        a.budget, a.group = float(budget), _GROUP_ID[group]
        a.scale = 1.0 / math.sqrt(q.shape[1])
        return a

    def labels_and_weights(self, q: torch.Tensor, *, n: int, budget: float, group: str = "sum_share"):
        """Kernel inputs: ``labels [H_kv, n]`` int16 (label ``C`` = exact set) and ``w``
        (``[H_kv, C+1]`` shared, ``[H, C+1]`` per query head; a buffer the next call overwrites)."""
        if group not in GROUPS:
            raise ValueError(f"unknown group mode {group!r}")
        H, d = q.shape
        if H % self.H_kv != 0 or H // self.H_kv > 8 or d != self.d:
            raise ValueError(f"q [{H}, {d}] does not fit {self.H_kv} KV heads of dim {self.d}")
        rows = H if group == "per_head" else self.H_kv
        w = self._wbuf(group, rows)
        q = q.contiguous()
        check(lib().ssa_select(self._state(), None, self._select_args(q, w, budget, group), stream_ptr(self.device)),
              "ssa_select")
        return self.labels[:, :n], w

    def attend(self, q, K, V, *, n, budget, group="sum_share", num_splits: int | None = None):
        """One decode step for this layer: update the clusters (``ssa_insert``), then select and
        attend over the selected rows in one launch (``ssa_sparse_step``). ``K, V [H_kv, >= n, d]``
        (engine cache layout, read in place). Returns ``(out, labels, w)``."""
        if group not in GROUPS:
            raise ValueError(f"unknown group mode {group!r}")
        self.observe(K, n)
        H, d = q.shape
        if H % self.H_kv != 0 or H // self.H_kv > 8 or d != self.d:
            raise ValueError(f"q [{H}, {d}] does not fit {self.H_kv} KV heads of dim {self.d}")
        if V.shape != K.shape or K.dtype != V.dtype:
            raise AssertionError("K and V must share shape and dtype")
        rows = H if group == "per_head" else self.H_kv
        w = self._wbuf(group, rows)
        q = q.contiguous()
        S = max(1, min(num_splits or default_splits(q.device, self.H_kv), 256, -(-max(n, 1) // 64)))
        work = _work(self.H_kv, S, H // self.H_kv, d, q.device)
        out = torch.empty(H, d, device=q.device, dtype=q.dtype)
        a = attn_args(q, K, V, out, work, labels=self.labels, w=w, n_host=n, per_head=group == "per_head")
        check(lib().ssa_sparse_step(self._state(), self._select_args(q, w, budget, group), a, None,
                                    stream_ptr(q.device)), "ssa_sparse_step")
        return out, self.labels[:, :n], w

    # -- counters ------------------------------------------------------------------------------
    @property
    def splits(self) -> int:
        """Clusters created by splitting (reads a GPU counter)."""
        return self._splits_host + (int(self.nsplit.sum()) if self.nsplit is not None else 0)

    @property
    def active_clusters(self) -> float:
        """Mean number of clusters in use per KV head."""
        return float(self.n_c.float().mean()) if self.initialized else float(self.C)
