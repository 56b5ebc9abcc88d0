"""The engine's decode seam: ``install(model, impl, **cfg)`` sets ``decode_attn_op`` on every
attention module (src/ssa/models/patch.py:245-258).

The engine calls ``decode_attn_op(q, full_k, full_v, *, scale, layer_idx)`` for single-query
decode steps with ``q [1, H, 1, d]`` and ``full_k/full_v [1, H_kv, n_k, d]`` (before GQA
expansion, read in place) and expects ``[1, H, 1, d]`` back (src/ssa/models/patch.py:3-7).

Implementations on this path: ``"cluster_fused"`` (one ``SphereIndexFused`` per layer, as
src/ssa/models/patch.py:109-119 builds it, with the same cfg keys and defaults) and
``"dense"`` (the exact split-K kernel). The old names ``sphere_fused`` / ``voronoi_fused`` are
accepted (src/ssa/attn/__init__.py:17-25). The reference's sampling estimators, tail estimates
and Quest comparisons are not part of this build and raise ``ValueError``.

``ReadStats`` keeps the reference's read accounting (src/ssa/models/patch.py:29-92): rows read
per step stay on the GPU and are summed without a host synchronisation until a property is read.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from .accounting import overhead_rows

_RENAMED = {"skip": "cluster_skip", "skip_v1": "cluster_skip_v1", "fused": "cluster_fused",
            "sample": "cluster_tail_sample", "tail": "cluster_tail"}
LEGACY_NAMES = {f"{old}_{k}": v for old in ("sphere", "voronoi") for k, v in _RENAMED.items()}
IMPLS = ("cluster_fused", "dense")


def canonical(name: str) -> str:
    """The current name for an implementation name, old or new (src/ssa/attn/__init__.py:23-25)."""
    return LEGACY_NAMES.get(name, name)


@dataclass
class ReadStats:
    """Value and key rows read across decode steps (per head, averaged), as the reference's."""

    steps: int = 0
    reads_sum: float = 0.0          # sum over steps of the mean over heads of rows read
    n_k_sum: float = 0.0            # sum over steps of n_k
    kv_rows_sum: float = 0.0        # sum over steps of K+V rows read per KV head, overhead included
    kv_steps: int = 0
    rebuilds: int = 0               # recenterings, all layers and KV heads
    head_steps: int = 0             # KV-head decode steps
    gpu_reads: torch.Tensor | None = None
    gpu_kv_rows: torch.Tensor | None = None

    def record_gpu(self, *, n_k: int, reads_mean: torch.Tensor, kv_rows: torch.Tensor) -> None:
        self.steps += 1
        self.kv_steps += 1
        self.n_k_sum += float(n_k)
        self.gpu_reads = reads_mean if self.gpu_reads is None else self.gpu_reads + reads_mean
        self.gpu_kv_rows = kv_rows if self.gpu_kv_rows is None else self.gpu_kv_rows + kv_rows

    def record(self, *, n_k: int, reads_per_head: torch.Tensor, kv_rows: float | None = None) -> None:
        self.steps += 1
        self.reads_sum += float(reads_per_head.float().mean().item())
        self.n_k_sum += float(n_k)
        if kv_rows is not None:
            self.kv_rows_sum += kv_rows
            self.kv_steps += 1

    def _flush_gpu(self) -> None:
        if self.gpu_reads is not None:
            self.reads_sum += float(self.gpu_reads)
            self.kv_rows_sum += float(self.gpu_kv_rows)
            self.gpu_reads = self.gpu_kv_rows = None

    @property
    def rebuild_rate(self) -> float | None:
        """Recenterings per KV head per decode step; None if not tracked."""
        return self.rebuilds / self.head_steps if self.head_steps else None

    @property
    def kv_read_fraction(self) -> float | None:
        """Fraction of all K and V rows read (summary overhead included); None if not tracked."""
        self._flush_gpu()
        if self.kv_steps != self.steps or not self.n_k_sum:
            return None
        return self.kv_rows_sum / (2 * self.n_k_sum)

    @property
    def avg_reads(self) -> float:
        return self.reads_sum / self.steps if self.steps else 0.0

    @property
    def avg_n_k(self) -> float:
        return self.n_k_sum / self.steps if self.steps else 0.0

    @property
    def read_fraction(self) -> float:
        self._flush_gpu()
        return self.reads_sum / self.n_k_sum if self.n_k_sum else 1.0


def _fused_index(cfg: dict):
    """One layer's index with the reference seam's keys and defaults (src/ssa/models/patch.py:109-119):
    with no ``C`` and the k-means partition, 1,024 slots, 256 fitted, splitting at twice the mean."""
    from .sphere_fused import SphereIndexFused
    part = cfg.get("partition", "kmeans")
    default = cfg.get("C") is None and part == "kmeans"
    return SphereIndexFused(C=int(cfg.get("C") or (1024 if part == "kmeans" else 256)),
                            window=int(cfg.get("window", 64)), delta=float(cfg.get("delta", 0.03)),
                            capacity=int(cfg.get("capacity", 65536)), check_every=int(cfg.get("check_every", 16)),
                            seed=int(cfg.get("seed", 0)), partition=part,
                            C_init=cfg.get("C_init", 256 if default else None),
                            split_factor=float(cfg.get("split_factor", 2.0 if default else 0.0)),
                            summary_bits=int(cfg.get("summary_bits", 8)), cap_keys=float(cfg.get("cap_keys", 0.0)))


def make_decode_op(impl: str, *, base_seed: int, stats: ReadStats, cfg: dict):
    """A decode-seam callback for ``impl`` (src/ssa/models/patch.py:99-242); the closure owns its
    step counter and, for ``cluster_fused``, its layer's index. ``base_seed`` is kept for the
    reference's signature: neither implementation here draws random numbers."""
    impl = canonical(impl)
    if impl not in IMPLS:
        raise ValueError(f"impl {impl!r} is not on this path (available: {', '.join(IMPLS)})")
    if impl == "cluster_fused" and "budget" not in cfg:
        raise KeyError("budget")
    counter = {"step": 0}
    fused = _fused_index(cfg) if impl == "cluster_fused" else None
    track = bool(cfg.get("track_reads", True))
    prev = {"rebuilds": 0, "head_steps": 0}

    def op(q, full_k, full_v, *, scale, layer_idx):
        qd = q[0, :, 0, :]                                   # [H, d]
        Kc, Vc = full_k[0], full_v[0]                        # [H_kv, n, d] views of the engine cache
        n_k = Kc.shape[1]
        d = qd.shape[1]
        if fused is None:
            from .labeled_attn import dense_attention
            out = dense_attention(qd.contiguous(), Kc, Vc, n=n_k)
            if track:
                stats.record(n_k=n_k, reads_per_head=torch.full((qd.shape[0],), float(n_k)), kv_rows=2.0 * n_k)
        else:
            out, labels, w = fused.attend(qd.contiguous(), Kc, Vc, n=n_k, budget=float(cfg["budget"]),
                                          group=cfg.get("group", "sum_share"))
            if track:
                wk = w if w.shape[0] == Kc.shape[0] else w.view(Kc.shape[0], -1, w.shape[1]).amax(1)
                rows = (torch.gather(wk, 1, labels[:, :n_k].long()) > 0).sum(1).float()      # [H_kv]
                rmean = rows.mean()
                stats.record_gpu(n_k=n_k, reads_mean=rmean,
                                 kv_rows=2 * rmean + overhead_rows(
                                     n=n_k, rows=rmean, clusters=fused.n_c.float().mean(), d=d,
                                     summary_bits=fused.summary_bits, fitted=fused.partition == "kmeans",
                                     heads=Kc.shape[0]))
                stats.rebuilds += fused.rebuilds - prev["rebuilds"]
                stats.head_steps += fused.head_steps - prev["head_steps"]
                prev["rebuilds"], prev["head_steps"] = fused.rebuilds, fused.head_steps
        counter["step"] += 1
        return out.view(1, -1, 1, d)

    op.index = fused
    return op


def _attention_modules(model):
    """The modules that carry the seam: the engine's ``Attention`` class when the engine is
    importable, else every module with a ``decode_attn_op`` attribute."""
    try:
        from engine.attention import Attention        # the reference's engine, when installed
    except ImportError:
        Attention = None
    for m in model.modules():
        if (Attention is not None and isinstance(m, Attention)) or (Attention is None and hasattr(m, "decode_attn_op")):
            yield m


def install(model, impl: str, *, base_seed: int = 0, **cfg) -> ReadStats:
    """Set the decode op on every attention module; return the shared ``ReadStats``."""
    stats = ReadStats()
    for m in _attention_modules(model):
        m.decode_attn_op = make_decode_op(impl, base_seed=base_seed, stats=stats, cfg=cfg)
    return stats


def uninstall(model) -> None:
    """Restore the engine's default (dense) decode path."""
    for m in _attention_modules(model):
        m.decode_attn_op = None
