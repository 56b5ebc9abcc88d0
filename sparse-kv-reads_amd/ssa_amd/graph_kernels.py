"""Per-layer decode-step objects for hipGraph capture.

A captured graph replays fixed kernels with fixed arguments, so nothing that changes from one
decode step to the next may be a host number: the current length ``n`` lives in device memory
(``n_dev``), each head's binned count in ``end_dev``, and the budget in keys is derived from it
inside the selection kernel.

Mirrors src/ssa/kernels/graph_kernels.py:
  * ``DenseAttentionGraph`` (:171-189): exact split-K decode over ``[0, n)``, one launch.
  * ``SphereIndexGraph`` (:192-279): per step one launch, ``ssa_sparse_step``: each workgroup
    scores the clusters and takes the selection in LDS, scans the labels and runs split-K
    attention over the selected rows; the last workgroup of a head merges the splits and then
    bins the key that leaves the window at the next step (in-kernel split included), which the
    reference bins at the start of that step. The reference issues bin, score, pick, zero,
    compact, list and merge. With ``insert_ahead=False`` the binning is a launch of its own
    (``ssa_insert``) before the step's, as in the reference.
  * ``AllLayerInsert`` (:286-325): one insertion launch for every layer.
"""

from __future__ import annotations

import torch

from ._lib import MAINT_PLAN_WORDS, MaintArgs, check, dtype_tag, lib, stream_ptr
from .labeled_attn import SplitWork, attn_args, cu_count, default_splits
from .sphere_fused import SphereIndexFused

MAINT_BUDGET = 1 << 30        # bytes of build scratch one maintenance pass may use (shared by all layers)


class _MaintScratch:
    """Scratch of ``ssa_maintain`` for one shape. The layers of a model run their maintenance one
    after another on one stream, so they share one of these."""

    def __init__(self, n, capacity, C, C_init, d, device):
        nbmax = capacity - 1
        nblk = -(-nbmax // 256)
        per_head = 4 * nbmax * (d + 3) + 4 * nblk * C * (d + 1)
        self.P = max(1, min(n, MAINT_BUDGET // per_head))
        P = self.P
        f32, i32 = dict(dtype=torch.float32, device=device), dict(dtype=torch.int32, device=device)
        self.mu = torch.empty(n, d, **f32)
        self.xn = torch.empty(P, nbmax, d, **f32)
        self.mag, self.sq = torch.empty(P, nbmax, **f32), torch.empty(P, nbmax, **f32)
        self.assign = torch.empty(P, nbmax, **i32)
        self.part = torch.empty(P, nblk, C, d, **f32)
        self.part_cnt = torch.empty(P, nblk, C, **i32)
        self.init_idx = torch.empty(max(C_init, 1), **i32)
        self.mem, self.side = torch.empty(capacity, **i32), torch.empty(capacity, **i32)
        self.proj, self.smag = torch.empty(capacity, **f32), torch.empty(capacity, **f32)
        self.parts = torch.empty(2, 1024, d, **f32)
        self.over = torch.empty(n, **i32)


_MAINT: dict = {}

STACKED = ("n_c", "sum_dir", "dir8", "cent", "cent8", "mmax", "mmin", "count", "ksum", "mu_ref", "rbar", "flags",
           "cap", "vthr", "_mem", "_proj", "_side", "_smag", "_stage", "_knbuf", "nsplit", "labels", "end_dev")


class DenseAttentionGraph:
    """Exact decode attention over ``[0, n)`` with ``n`` in GPU memory (graph-safe)."""

    def __init__(self, *, H: int, H_kv: int, d: int, dtype, device, block_n: int = 32, num_splits: int | None = None):
        self.G = H // H_kv
        self.d = d
        S = num_splits or default_splits(device, H_kv, dense=True)
        self.work = SplitWork(H_kv, S, self.G, d, device)
        self.out = torch.empty(H, d, device=device, dtype=dtype)

    def __call__(self, q, K, V, n_dev):
        a = attn_args(q, K, V, self.out, self.work, n_dev=n_dev)
        check(lib().ssa_dense_attention(a, stream_ptr(q.device)), "ssa_dense_attention")
        return self.out


class SphereIndexGraph(SphereIndexFused):
    """``SphereIndexFused`` for graph capture: ``step`` issues only fixed-argument kernels."""

    def __init__(self, *, budget: float, block_n: int = 32, compact_block: int = 1024, refit_every: int = 0,
                 num_splits: int | None = None, insert_ahead: bool | None = None,
                 device_maintenance: bool = True, **kw):
        self._plan = None
        super().__init__(**kw)
        # recentring, resets and refits on the device (ssa_maintain), with no host read between
        # replays; the host path (the reference's eager rebuilds) serves var_factor > 0, whose
        # threshold the device does not recompute
        self.device_maintenance = device_maintenance and self.var_factor == 0
        self.insert_ahead = insert_ahead          # None: decided at prepare (auto_insert_ahead)
        self.refit_every = refit_every
        self.refits = 0
        self.budget = budget
        self.block_n, self.compact_block = block_n, compact_block
        self.num_splits = num_splits

    def prepare(self, K: torch.Tensor, n: int, H: int) -> None:
        """Build from the prefilled cache ``K [H_kv, capacity, d]`` holding ``n`` positions (eager,
        outside the graph) and allocate the step's fixed buffers. With ``insert_ahead`` the keys
        that leave the window at length ``n + 1`` are binned too: every step's launch leaves the
        state binned for the next length, so ``step`` must be called at ``n + 1``, ``n + 2``, ..."""
        self.observe(K, n)
        H_kv, d, dev = self.H_kv, self.d, self.device
        self.G = H // H_kv
        S = self.num_splits or default_splits(dev, H_kv)
        self.work = SplitWork(H_kv, S, self.G, d, dev)
        if self.insert_ahead is None:
            self.insert_ahead = self.auto_insert_ahead()
        if self.insert_ahead and max(1, n + 1 - self.window) > self.end:
            check(lib().ssa_insert(self._state(), self._insert_args(K, n_host=n + 1), stream_ptr(self.device)),
                  "ssa_insert")
            self.end = max(1, n + 1 - self.window)
        self.end_dev.fill_(self.end)
        self.wbuf = torch.zeros(H_kv, self.C + 1, dtype=torch.float32, device=dev)
        self.wbuf[:, self.C] = 1.0
        self.need_dev = torch.zeros(H_kv, dtype=torch.int32, device=dev)
        self.out = torch.empty(H, d, device=dev, dtype=K.dtype)

    def auto_insert_ahead(self) -> bool:
        """Bin the next step's key inside the fused launch. The library stages it in one extra
        workgroup per head while those fit beside the splits (two workgroups per compute unit),
        else in each head's last split after its attention; either beats a separate insertion
        launch (measured on MI355X: batch 8 x 8k and 2 x 32k gain 5-9 us per step, 16 x 32k
        6-8 us, 64 x 32k -1..+4 us)."""
        return True

    def extra_stagers_fit(self) -> bool:
        """Whether the fused launch's extra stager workgroups (one per head) fit beside the
        splits; past that a model's decode loop bins every layer's keys in one launch."""
        return 4 * self.H_kv <= cu_count(self.device)

    def _init(self, K, n):
        super()._init(K, n)
        self.end_dev.fill_(self.end)

    def step(self, q, K, V, n_dev, insert: bool = True):
        """One decode step; ``K, V [H_kv, capacity, d]`` with position ``n - 1`` already written.
        With ``insert_ahead`` one launch, ``ssa_sparse_step``, which also bins the keys for the
        next step. Otherwise ``ssa_insert`` (unless ``insert=False``: the keys leaving the window
        were already inserted for every layer by one launch, ``AllLayerInsert``) and then
        ``ssa_sparse_step``. ``wbuf`` receives the selection."""
        s = stream_ptr(q.device)
        st = self._state()
        ahead = None
        if self.insert_ahead:
            ahead = self._insert_args(K)
        elif insert:
            check(lib().ssa_insert(st, self._insert_args(K, n_dev=n_dev), s), "ssa_insert")
        sel = self._select_args(q, self.wbuf, self.budget, "sum_share")
        a = attn_args(q, K, V, self.out, self.work, labels=self.labels, w=self.wbuf, n_dev=n_dev)
        check(lib().ssa_sparse_step(st, sel, a, ahead, s), "ssa_sparse_step")
        return self.out

    def _host_end(self) -> None:
        self.end = int(self.end_dev[0])                          # host sync, only when a flag was set

    def after_replay(self, K: torch.Tensor) -> None:
        """Between replays: every ``check_every`` steps act on the drift and reset flags, and every
        ``refit_every`` steps refit every head. With ``device_maintenance`` that is one
        ``ssa_maintain`` call, which reads the flags on the device (no host read); otherwise the
        flags are copied without a sync and, once a copy has landed, the flagged heads are
        rebuilt eagerly, as in the reference."""
        self.head_steps += self.H_kv
        self._steps += 1
        refit = bool(self.refit_every) and self._steps % self.refit_every == 0
        if self.device_maintenance:
            if refit or self._steps % self.check_every == 0:
                self.maintain(K, refit_all=refit)
            return
        if refit:
            self._refit(K)
        elif self._steps % self.check_every == 0:
            self._check_flags(K)

    def maintain(self, K: torch.Tensor, *, refit_all: bool = False) -> None:
        """``ssa_maintain``: recentre the heads whose drift flag is set, refit those whose reset
        flag is set (or every head, with ``refit_all``), clear the flags; all on the device."""
        key = (str(self.device), self.H_kv, self.capacity, self.C, self.C_init, self.d)
        sc = _MAINT.get(key)
        if sc is None:
            sc = _MAINT[key] = _MaintScratch(self.H_kv, self.capacity, self.C, self.C_init, self.d, self.device)
        if self._plan is None:
            self._plan = torch.zeros(MAINT_PLAN_WORDS + 3 * self.H_kv, dtype=torch.int32, device=self.device)
        a = MaintArgs()
        a.k, a.k_dtype, a.s_kh, a.s_kn = K.data_ptr(), dtype_tag(K.dtype), K.stride(0), K.stride(1)
        a.refit_all = int(refit_all)
        a.refit = int(refit_all or bool(self.reset_at))
        a.C_init, a.iters, a.seed = self.C_init, self.kmeans_iters, self.seed
        a.split_factor, a.cap_keys, a.capk = self.split_factor, self.cap_keys, self.capk
        a.max_heads = sc.P
        a.plan, a.mu = self._plan.data_ptr(), sc.mu.data_ptr()
        a.xn, a.mag, a.sq, a.assign = sc.xn.data_ptr(), sc.mag.data_ptr(), sc.sq.data_ptr(), sc.assign.data_ptr()
        a.part, a.part_cnt, a.init_idx = sc.part.data_ptr(), sc.part_cnt.data_ptr(), sc.init_idx.data_ptr()
        a.mem, a.side, a.proj, a.smag = sc.mem.data_ptr(), sc.side.data_ptr(), sc.proj.data_ptr(), sc.smag.data_ptr()
        a.parts, a.over = sc.parts.data_ptr(), sc.over.data_ptr()
        check(lib().ssa_maintain(self._state(), a, stream_ptr(self.device)), "ssa_maintain")
        if refit_all:
            self.refits += 1

    # heads rebuilt and refitted so far: the host path's counts plus the device's (reading those
    # synchronises, as the reference's ``splits`` does)
    @property
    def rebuilds(self) -> int:
        return self._rebuilds_host + (int(self._plan[4]) if self._plan is not None else 0)

    @rebuilds.setter
    def rebuilds(self, v: int) -> None:
        self._rebuilds_host = v - (int(self._plan[4]) if self._plan is not None else 0)

    @property
    def resets(self) -> int:
        return self._resets_host + (int(self._plan[5]) if self._plan is not None else 0)

    @resets.setter
    def resets(self, v: int) -> None:
        self._resets_host = v

    def _refit(self, K: torch.Tensor) -> None:
        """Fit the clusters again on every binned key, with a fresh mean."""
        self._host_end()
        self.fitted = [False] * self.H_kv
        self.n_c.fill_(self.C_init)
        self._build(K, torch.arange(self.H_kv), None)
        self._split_after_fit(K)
        self.flags.zero_()
        self._pending = None
        self.refits += 1

    def _build_heads(self, K, heads, mu, fit):
        super()._build_heads(K, heads, mu, fit)
        self.end_dev[torch.tensor(heads, device=self.device).long()] = self.end


class AllLayerInsert:
    """One insertion launch for every layer. The key that leaves the recent window at a step was
    written ``window`` steps earlier at every layer, so all layers' insertions (and the splits
    they trigger) run together, one workgroup per (layer, KV head).

    Built after every layer's index is prepared: each per-head state array of all layers is
    moved into one array stacked over layers and every layer's index is pointed at its slice,
    so per-layer kernels and host-side maintenance keep working on the same memory."""

    def __init__(self, layers: list, caches: list):
        first = layers[0]
        if first.window < 1:
            raise AssertionError("with no recent window the key to insert is not yet written at later layers")
        if not all(i.H_kv == first.H_kv and i.end == first.end for i in layers):
            raise AssertionError("layers must share the head count and the binned length")
        self.layers, self.L = layers, len(layers)
        big = {}
        for name in STACKED:
            t0 = getattr(first, name, None)
            if t0 is None:
                continue
            if name == "cent" and first.partition != "kmeans":
                continue                                        # one shared table
            big[name] = torch.stack([getattr(i, name) for i in layers])
            for l, i in enumerate(layers):
                setattr(i, name, big[name][l])
        self.big = big
        first._stacked = big
        k0 = caches[0]
        size = k0.element_size()
        off = [k.data_ptr() - k0.data_ptr() for k in caches]
        if not (all(o % size == 0 for o in off) and all(k.stride() == k0.stride() for k in caches)):
            raise AssertionError("layer caches must share strides")
        self.koff = torch.tensor([o // size for o in off], dtype=torch.int64, device=first.device)
        self.k0 = k0

    def __call__(self, n_dev) -> None:
        f = self.layers[0]
        st = f._state(layers=self.L)
        if f.partition != "kmeans":
            st.cent = f.cent.data_ptr()
        check(lib().ssa_insert(st, f._insert_args(self.k0, n_dev=n_dev, koff=self.koff), stream_ptr(f.device)),
              "ssa_insert")
