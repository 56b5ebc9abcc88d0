"""Label-weighted decode attention on the HIP kernels: the attention half of the hot path.

For query head ``h`` on KV head ``g`` (``G = H / H_kv`` query heads share a KV head)::

    out[h] = sum_j w[label_j] e^{s_j} v_j / sum_j w[label_j] e^{s_j},    s_j = q_h . k_j / sqrt(d)

with K, V read in place in the engine's cache layout ``[H_kv, n, d]`` (any strides with a unit
last stride). Rows whose weight is 0 for every query head of the group are never fetched.

Mirrors the public functions of the reference's ``ssa.kernels.labeled_attn``
(src/ssa/kernels/labeled_attn.py): ``label_weighted_attention_compact`` (:248),
``label_weighted_attention_triton`` (:88), ``compact_positions`` (:186) and ``merge_splits``
(:143), with the same arguments and shape checks. Tiling knobs of the Triton kernels
(``block_n``, ``num_stages``, ``num_warps``, ``block``) are accepted and have no effect;
``num_splits`` sets the split-K factor.
"""

from __future__ import annotations

import torch

from ._lib import AttnArgs, check, dtype_tag, lib, ptr, require_cuda, stream_ptr

_CUS: dict = {}


def cu_count(device) -> int:
    key = str(device)
    if key not in _CUS:
        _CUS[key] = torch.cuda.get_device_properties(device).multi_processor_count
    return _CUS[key]


def default_splits(device, n_heads: int, *, dense: bool = False) -> int:
    """Split-K factor per head. The reference uses ``cdiv(4 * SMs, H_kv)``
    (src/ssa/kernels/labeled_attn.py:266). Here, at most 32 splits per head (the last workgroup
    of a head then issues every load of its merge at once) and one workgroup per compute unit
    over all heads. When the heads alone nearly fill the GPU (two splits or fewer), the sparse
    kernel takes two workgroups per compute unit: each reads a scattered row list, and one
    resident workgroup per compute unit leaves bandwidth unused (measured on MI355X at 32k
    context: batch 16 goes from 157 to 128 us at 20%, while smaller batches lose to the longer
    merge). With few heads (16 splits or more) the sparse kernel takes 1.5 workgroups per compute
    unit, so that the row phase of one overlaps the selection phase of another (batch 2 x 32k at
    20%: 48.6 us at 16 splits, 45.0 us at 24, 57.1 us at 32; one head per 32 splits is the cap)."""
    cus = cu_count(device)
    s = -(-cus // n_heads)
    if not dense and s <= 2:
        s = -(-2 * cus // n_heads)
    elif not dense and s >= 16:
        s = -(-3 * cus // (2 * n_heads))
    return max(1, min(32, s))


class SplitWork:
    """Per-launch split partials and the arrival counters of the fused log-sum-exp merge. The
    counters start at zero and every launch leaves them at zero, so one ``SplitWork`` serves any
    number of launches issued in order on one stream (also inside a captured graph)."""

    def __init__(self, n_heads: int, S: int, G: int, d: int, device):
        self.n_heads, self.S, self.G, self.d = n_heads, S, G, d
        self.m = torch.empty(n_heads, S, G, device=device, dtype=torch.float32)
        self.l = torch.empty_like(self.m)
        self.a = torch.empty(n_heads, S, G, d, device=device, dtype=torch.float32)
        self.cnt_split = torch.empty(n_heads, S, device=device, dtype=torch.int32)
        self.counter = torch.zeros(n_heads, device=device, dtype=torch.int32)
        self.cnt = torch.zeros(n_heads, device=device, dtype=torch.int32)


_WORK: dict = {}


def _work(n_heads, S, G, d, device) -> SplitWork:
    key = (str(device), n_heads, S, G, d)
    if key not in _WORK:
        _WORK[key] = SplitWork(n_heads, S, G, d, device)
    return _WORK[key]


def _check_qkv(q, K, V):
    H, d = q.shape
    H_kv, n, d2 = K.shape
    if not (d == d2 and V.shape == K.shape and K.stride(-1) == 1 and V.stride(-1) == 1):
        raise AssertionError("q [H, d], K and V [H_kv, n, d] with a unit last stride expected")
    if not (d & (d - 1) == 0 and 16 <= d <= 256):
        raise AssertionError("head dim must be a power of two in [16, 256]")
    if H % H_kv != 0 or H // H_kv > 8:
        raise AssertionError("query heads must be a multiple (at most 8) of the KV heads")
    if K.dtype != V.dtype:
        raise AssertionError("K and V must share a dtype")
    require_cuda(q, K, V)
    return H, d, H_kv, n


def attn_args(q, K, V, out, work: SplitWork, *, labels=None, w=None, n_dev=None, n_host=0, per_head=False):
    """Fill the C-ABI argument block of one attention launch. Rows of q, K and V are read with
    16-byte loads, so their base pointers and row strides must be 16-byte aligned."""
    for name, t in (("q", q), ("K", K), ("V", V)):
        if t.data_ptr() % 16 or any((st * t.element_size()) % 16 for st in t.stride()[:-1]):
            raise AssertionError(f"{name} rows must be 16-byte aligned (base and row strides)")
    a = AttnArgs()
    a.q, a.s_qh, a.q_dtype = q.data_ptr(), q.stride(0), dtype_tag(q.dtype)
    a.k, a.s_kh, a.s_kn = K.data_ptr(), K.stride(0), K.stride(1)
    a.v, a.s_vh, a.s_vn = V.data_ptr(), V.stride(0), V.stride(1)
    a.kv_dtype = dtype_tag(K.dtype)
    if labels is not None:
        a.labels, a.s_lh = labels.data_ptr(), labels.stride(0)
        a.w, a.s_wr, a.w_len, a.per_head = w.data_ptr(), w.stride(0), w.shape[1], int(per_head)
    a.n_dev, a.n_host = ptr(n_dev), int(n_host)
    a.part_m, a.part_l, a.part_a = work.m.data_ptr(), work.l.data_ptr(), work.a.data_ptr()
    a.part_cnt, a.counter = work.cnt_split.data_ptr(), work.counter.data_ptr()
    a.out, a.s_oh, a.out_dtype = out.data_ptr(), out.stride(0), dtype_tag(out.dtype)
    a.cnt_out = work.cnt.data_ptr()
    a.n_heads, a.G, a.d, a.S, a.chunk_align = work.n_heads, work.G, work.d, work.S, 64
    return a


def label_weighted_attention_compact(q: torch.Tensor, K: torch.Tensor, V: torch.Tensor,
                                     labels: torch.Tensor, w: torch.Tensor, *,
                                     block_n: int = 32, num_splits: int | None = None,
                                     num_stages: int | None = None, num_warps: int = 4,
                                     compact_block: int = 1024, out: torch.Tensor | None = None) -> torch.Tensor:
    """``q [H, d]``, ``K, V [H_kv, n, d]`` (unit last stride), ``labels [H_kv, n]`` int16,
    ``w [H_kv or H, L]`` -> ``[H, d]`` in ``q``'s dtype. One kernel: selection scan, split-K
    attention over the selected rows, and the log-sum-exp merge."""
    H, d, H_kv, n = _check_qkv(q, K, V)
    G = H // H_kv
    per_head = w.shape[0] == H and H != H_kv
    if not per_head and w.shape[0] != H_kv:
        raise AssertionError(f"w has {w.shape[0]} rows; expected H_kv={H_kv} or H={H}")
    if labels.shape[0] != H_kv or labels.shape[1] < n:
        raise AssertionError("labels must be [H_kv, >= n]")
    if w.shape[1] > 1025:
        raise AssertionError("at most 1024 clusters (+1 exact label)")
    require_cuda(labels, w)
    if labels.dtype != torch.int16:
        labels = labels.to(torch.int16)
    if labels.stride(-1) != 1:
        labels = labels.contiguous()
    w = w.to(torch.float32).contiguous()
    q = q.contiguous()
    S = num_splits or default_splits(q.device, H_kv)
    S = max(1, min(S, 256, -(-max(n, 1) // 64)))
    work = _work(H_kv, S, G, d, q.device)
    if out is None:
        out = torch.empty(H, d, device=q.device, dtype=q.dtype)
    a = attn_args(q, K, V, out, work, labels=labels, w=w, n_host=n, per_head=per_head)
    check(lib().ssa_label_attention(a, stream_ptr(q.device)), "ssa_label_attention")
    return out


def label_weighted_attention_triton(q, K, V, labels, w, *, block_n: int = 64, num_splits: int | None = None,
                                    num_stages: int | None = None, num_warps: int = 4) -> torch.Tensor:
    """The reference's masked-scan variant; here the same fused kernel (it always scans labels
    and reads only the selected rows)."""
    return label_weighted_attention_compact(q, K, V, labels, w, num_splits=num_splits)


def dense_attention(q, K, V, *, n: int | None = None, n_dev: torch.Tensor | None = None,
                    num_splits: int | None = None, out: torch.Tensor | None = None,
                    work: SplitWork | None = None) -> torch.Tensor:
    """Exact ``softmax(q K^T / sqrt(d)) V`` over positions ``[0, n)`` (``n`` on the host or in
    device memory), the dense split-K baseline."""
    H, d, H_kv, nk = _check_qkv(q, K, V)
    G = H // H_kv
    n = nk if n is None else n
    if work is None:
        S = num_splits or default_splits(q.device, H_kv, dense=True)
        work = _work(H_kv, S, G, d, q.device)
    if out is None:
        out = torch.empty(H, d, device=q.device, dtype=q.dtype)
    a = attn_args(q.contiguous(), K, V, out, work, n_dev=n_dev, n_host=n)
    check(lib().ssa_dense_attention(a, stream_ptr(q.device)), "ssa_dense_attention")
    return out


def compact_positions(labels: torch.Tensor, w: torch.Tensor, *, block: int = 1024, n: int | None = None,
                      n_dev: torch.Tensor | None = None):
    """Selected positions per KV head: ``idx [H_kv, n]`` int32 (first ``cnt[kv]`` valid, in
    ascending order) and ``cnt [H_kv]`` int32. A position is selected if its label has positive
    weight for any query head of its group."""
    H_kv, cap = labels.shape
    n = cap if n is None else n
    per_head = w.shape[0] != H_kv
    G = w.shape[0] // H_kv if per_head else 1
    require_cuda(labels, w)
    labels = labels.to(torch.int16)
    if labels.stride(-1) != 1:
        labels = labels.contiguous()
    w = w.to(torch.float32).contiguous()
    rows = max(cap if n_dev is not None else n, 1)
    idx = torch.empty(H_kv, rows, device=labels.device, dtype=torch.int32)
    cnt = torch.zeros(H_kv, device=labels.device, dtype=torch.int32)
    nblk = -(-rows // 1024)
    bc = torch.empty(H_kv, nblk, device=labels.device, dtype=torch.int32)
    rc = lib().ssa_compact_positions(labels.data_ptr(), labels.stride(0), w.data_ptr(), w.stride(0), H_kv, G,
                                     int(per_head), ptr(n_dev), int(n), rows, bc.data_ptr(), idx.data_ptr(),
                                     idx.stride(0), cnt.data_ptr(), stream_ptr(labels.device))
    check(rc, "ssa_compact_positions")
    return idx, cnt


def merge_splits(m: torch.Tensor, l: torch.Tensor, a: torch.Tensor, dtype, out: torch.Tensor | None = None):
    """Combine natural-log split partials ``m, l [H_kv, S, G]``, ``a [H_kv, S, G, d]`` by
    log-sum-exp into ``[H_kv * G, d]`` of ``dtype``."""
    H_kv, S, G = m.shape
    d = a.shape[-1]
    require_cuda(m, l, a)
    if m.dtype != torch.float32 or l.dtype != torch.float32 or a.dtype != torch.float32:
        raise AssertionError("split partials must be float32")
    if m.stride() != l.stride() or a.stride(-1) != 1 or m.stride(-1) != 1:
        raise AssertionError("m and l must share strides; unit last strides expected")
    if out is None:
        out = torch.empty(H_kv * G, d, device=m.device, dtype=dtype)
    rc = lib().ssa_merge_splits(m.data_ptr(), l.data_ptr(), a.data_ptr(), m.stride(0), m.stride(1), a.stride(0),
                                a.stride(1), a.stride(2), H_kv, S, G, d, out.data_ptr(), out.stride(0),
                                dtype_tag(out.dtype), stream_ptr(m.device))
    check(rc, "ssa_merge_splits")
    return out


__all__ = ["label_weighted_attention_compact", "label_weighted_attention_triton", "dense_attention",
           "compact_positions", "merge_splits", "default_splits", "SplitWork"]
