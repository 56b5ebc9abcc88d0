"""HIP label-weighted / dense decode attention vs the float64 spec (GPU only).

Mirrors the reference's tests/test_labeled_triton.py and the merge test of
tests/test_sphere_fused.py:98-108, with the oracle's numpy restatement of
label_weighted_attention (src/ssa/attn/labeled.py:24-44) as the checker.
Tolerances: 2e-2 abs for bf16 inputs, 1e-5 abs for fp32 inputs.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import reference as ref

pytestmark = pytest.mark.gpu

H, H_KV, D, L = 32, 8, 128, 257          # Qwen3-4B geometry; 256 clusters + exact label


def _inputs(n, *, seed=0, dtype=torch.bfloat16, capacity=None, H=H, H_kv=H_KV, d=D, labels_max=L):
    g = torch.Generator(device="cpu").manual_seed(seed)
    cap = capacity or n
    q = (torch.randn(H, d, generator=g) * 2).to(dtype).cuda()
    Kbuf = torch.randn(1, H_kv, cap, d, generator=g).to(dtype).cuda()
    Vbuf = torch.randn(1, H_kv, cap, d, generator=g).to(dtype).cuda()
    labels = torch.randint(0, labels_max, (H_kv, n), generator=g).to(torch.int16).cuda()
    return q, Kbuf[0, :, :n], Vbuf[0, :, :n], labels


def _np(t):
    return t.detach().double().cpu().numpy()


def _check(q, K, V, labels, w, atol=2e-2, **kw):
    from ssa_amd.labeled_attn import label_weighted_attention_compact
    out = label_weighted_attention_compact(q, K, V, labels, w, **kw)
    torch.cuda.synchronize()
    want = ref.label_weighted_attention(_np(q), _np(K), _np(V), labels.cpu().numpy(), _np(w))
    assert out.shape == q.shape and out.dtype == q.dtype
    np.testing.assert_allclose(_np(out), want, rtol=0, atol=atol)
    return out


@pytest.mark.parametrize("n", [1, 63, 64, 65, 1000, 4097])
def test_all_ones_is_dense(n):
    q, K, V, labels = _inputs(n, seed=n)
    w = torch.ones(H_KV, L, device="cuda")
    out = _check(q, K, V, labels, w)
    np.testing.assert_allclose(_np(out), ref.dense(_np(q), _np(K), _np(V)), rtol=0, atol=2e-2)


@pytest.mark.parametrize("per_head", [False, True])
def test_random_selection(per_head):
    q, K, V, labels = _inputs(3000, seed=1)
    g = torch.Generator(device="cpu").manual_seed(2)
    w = (torch.rand(H if per_head else H_KV, L, generator=g) < 0.2).float().cuda()
    w[:, L - 1] = 1.0
    _check(q, K, V, labels, w)


def test_non_unit_weights():
    q, K, V, labels = _inputs(2500, seed=3)
    g = torch.Generator(device="cpu").manual_seed(4)
    w = torch.rand(H_KV, L, generator=g).cuda() * 5
    w[w < 1.0] = 0.0
    w[:, L - 1] = 1.0
    _check(q, K, V, labels, w)


def test_unread_rows_are_never_used():
    from ssa_amd.labeled_attn import label_weighted_attention_compact as f
    q, K, V, labels = _inputs(2000, seed=5)
    w = torch.zeros(H_KV, L, device="cuda")
    w[:, :64] = 1.0
    w[:, L - 1] = 1.0
    a = f(q, K, V, labels, w).clone()
    skip = torch.gather(w, 1, labels.long()) == 0
    K2, V2 = K.clone(), V.clone()
    K2[skip] = float("nan")
    V2[skip] = float("nan")
    b = f(q, K2, V2, labels, w)
    assert torch.isfinite(b).all()
    assert torch.equal(a, b)                 # the selection order is deterministic: identical results


def test_strided_cache_view_with_spare_capacity():
    q, K, V, labels = _inputs(1500, seed=6, capacity=4096)
    assert not K.is_contiguous()
    w = torch.ones(H_KV, L, device="cuda")
    w[:, 5:100] = 0.0
    _check(q, K, V, labels, w)


@pytest.mark.parametrize("num_splits", [1, 7, 40, 300])
def test_split_counts(num_splits):
    q, K, V, labels = _inputs(5000, seed=7)
    g = torch.Generator(device="cpu").manual_seed(8)
    w = (torch.rand(H_KV, L, generator=g) < 0.3).float().cuda()
    w[:, L - 1] = 1.0
    _check(q, K, V, labels, w, num_splits=num_splits)


def test_long_context():
    q, K, V, labels = _inputs(65536, seed=9)
    g = torch.Generator(device="cpu").manual_seed(10)
    w = (torch.rand(H_KV, L, generator=g) < 0.1).float().cuda()
    w[:, L - 1] = 1.0
    _check(q, K, V, labels, w)


@pytest.mark.parametrize("Hq,Hk,d", [(16, 8, 128), (8, 8, 128), (64, 8, 128), (16, 8, 64), (4, 2, 16),
                                     (16, 8, 256), (12, 4, 32)])
def test_shapes(Hq, Hk, d):
    q, K, V, labels = _inputs(1777, seed=11, H=Hq, H_kv=Hk, d=d)
    g = torch.Generator(device="cpu").manual_seed(12)
    w = (torch.rand(Hk, L, generator=g) < 0.4).float().cuda()
    w[:, L - 1] = 1.0
    _check(q, K, V, labels, w)


@pytest.mark.parametrize("per_head", [False, True])
def test_fp32_within_1e5(per_head):
    q, K, V, labels = _inputs(4096, seed=13, dtype=torch.float32)
    g = torch.Generator(device="cpu").manual_seed(14)
    w = (torch.rand(H if per_head else H_KV, L, generator=g) < 0.25).float().cuda()
    w[:, L - 1] = 1.0
    _check(q, K, V, labels, w, atol=1e-5)


def test_fp16_inputs():
    q, K, V, labels = _inputs(3000, seed=15, dtype=torch.float16)
    w = (torch.rand(H_KV, L, generator=torch.Generator().manual_seed(16)) < 0.3).float().cuda()
    w[:, L - 1] = 1.0
    _check(q, K, V, labels, w)


def test_rows_read_count():
    from ssa_amd import labeled_attn as la
    q, K, V, labels = _inputs(3333, seed=17)
    w = (torch.rand(H_KV, L, generator=torch.Generator().manual_seed(18)) < 0.2).float().cuda()
    w[:, L - 1] = 1.0
    la.label_weighted_attention_compact(q, K, V, labels, w, num_splits=9)
    work = la._work(H_KV, 9, H // H_KV, D, q.device)
    want = (torch.gather(w, 1, labels.long()) > 0).sum(1).to(torch.int32)
    assert torch.equal(work.cnt, want)
    assert int(work.counter.abs().sum()) == 0           # arrival counters are left at zero


def test_compaction_list_is_exactly_the_needed_rows_in_order():
    from ssa_amd.labeled_attn import compact_positions
    _, _, _, labels = _inputs(5000, seed=19)
    g = torch.Generator(device="cpu").manual_seed(20)
    for rows in (H_KV, H):
        w = (torch.rand(rows, L, generator=g) < 0.25).float().cuda()
        idx, cnt = compact_positions(labels, w)
        wk = w if rows == H_KV else w.view(H_KV, H // H_KV, L).amax(1)
        need = torch.gather(wk, 1, labels.long()) > 0
        for kv in range(H_KV):
            got = idx[kv, :int(cnt[kv])].long()
            assert torch.equal(got, need[kv].nonzero().squeeze(1))     # ascending, exact


def test_compaction_with_device_length():
    from ssa_amd.labeled_attn import compact_positions
    _, _, _, labels = _inputs(3000, seed=21, capacity=4096)
    w = (torch.rand(H_KV, L, generator=torch.Generator().manual_seed(22)) < 0.3).float().cuda()
    full = torch.full((H_KV, 4096), L - 1, dtype=torch.int16, device="cuda")
    full[:, :3000] = labels
    n_dev = torch.tensor([2500], dtype=torch.int32, device="cuda")
    idx, cnt = compact_positions(full, w, n_dev=n_dev)
    need = torch.gather(w, 1, full[:, :2500].long()) > 0
    for kv in range(H_KV):
        assert torch.equal(idx[kv, :int(cnt[kv])].long(), need[kv].nonzero().squeeze(1))


def test_merge_matches_closed_form():
    from ssa_amd.labeled_attn import merge_splits
    g = torch.Generator(device="cpu").manual_seed(6)
    for S, G in ((1, 4), (18, 4), (72, 2)):
        m = torch.randn(H_KV, S, G, generator=g) * 3
        m[:, 0, 0] = -1.0e30                                          # an empty split
        l = torch.rand(H_KV, S, G, generator=g)
        a = torch.randn(H_KV, S, G, D, generator=g)
        got = merge_splits(m.cuda(), l.cuda(), a.cuda(), torch.float32)
        np.testing.assert_allclose(got.cpu().numpy(), ref.merge(m.numpy(), l.numpy(), a.numpy()), rtol=1e-5,
                                   atol=1e-5)


@pytest.mark.parametrize("dtype,atol", [(torch.bfloat16, 2e-2), (torch.float32, 1e-5)])
def test_dense_attention_host_and_device_length(dtype, atol):
    from ssa_amd.labeled_attn import dense_attention
    from ssa_amd.graph_kernels import DenseAttentionGraph
    q, K, V, _ = _inputs(4096, seed=23, dtype=dtype, H=16, capacity=8192)
    n = 3001
    want = ref.dense(_np(q), _np(K[:, :n]), _np(V[:, :n]))
    got = dense_attention(q, K, V, n=n)
    np.testing.assert_allclose(_np(got), want, rtol=0, atol=atol)
    dag = DenseAttentionGraph(H=16, H_kv=H_KV, d=D, dtype=dtype, device=q.device)
    got2 = dag(q, K, V, torch.tensor([n], dtype=torch.int32, device="cuda"))
    np.testing.assert_allclose(_np(got2), want, rtol=0, atol=atol)


@pytest.mark.parametrize("field,value", [("G", 0), ("G", 9), ("S", 0), ("S", 257), ("n_heads", 0), ("d", 48),
                                         ("w_len", 0), ("w_len", 1026)])
def test_bad_arguments_are_refused_before_any_launch(field, value):
    """The C ABI checks its scalar arguments and returns hipErrorInvalidValue (1) without
    launching: GQA group 1..8, splits 1..256, head size 16/32/64/128/256, weight slots 1..1025."""
    from ssa_amd._lib import lib, stream_ptr
    from ssa_amd.labeled_attn import SplitWork, attn_args
    q, K, V, labels = _inputs(300)
    w = torch.ones(H_KV, L, device="cuda")
    work = SplitWork(H_KV, 4, H // H_KV, D, q.device)
    out = torch.empty_like(q)
    a = attn_args(q, K, V, out, work, labels=labels, w=w, n_host=300)
    setattr(a, field, value)
    rc = lib().ssa_label_attention(a, stream_ptr(q.device))
    torch.cuda.synchronize()
    assert rc == 1
    # the same arguments with the field restored still work
    a = attn_args(q, K, V, out, work, labels=labels, w=w, n_host=300)
    assert lib().ssa_label_attention(a, stream_ptr(q.device)) == 0
    torch.cuda.synchronize()
