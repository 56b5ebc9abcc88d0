"""configs[2] on the GPU against the oracle: batched decode steps with the batch folded into the
KV heads (src/ssa/models/graph_decode.py:14-17), each sequence with its own seeded clusters and
ragged cluster sizes.

* 8 x 8192 at full size (64 folded heads): the graph step (selection in every workgroup,
  split-K attention, merge, insertion of the next key inside the launch).
* 16 x 2048 and 64 x 1024 (128 and 512 folded heads): the launch paths of many heads, i.e. the
  doubled split count (S <= 2 per head), the XCD placement permutation over large grids, and the
  separate insertion launch (``ssa_insert``), over several steps against the full C oracle.
* ``AllLayerInsert`` over three layers, with their caches at layer offsets: one insertion launch
  for all layers, each layer's state against the oracle's per-layer insertion.

Selections and states bit for bit; outputs within 2e-2 of the float64 spec
(src/ssa/attn/labeled.py:24-44). Reference: SphereIndexGraph.step and AllLayerInsert
(src/ssa/kernels/graph_kernels.py:192-325).
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import reference as ref
from oracle.canon import CanonIndex

pytestmark = pytest.mark.gpu

D, H_KV, H = 128, 8, 16
STATE = ("n_c", "sum_dir", "dir8", "cent", "cent8", "mmax", "mmin", "count", "ksum", "mu_ref", "rbar", "end",
         "nsplit", "labels", "flags")


def _folded(B, n, extra, *, seed, centers):
    from ssa_amd.synth import make_cache
    K, V, q, _ = make_cache(B, H_KV, n + extra, D, H=H, centers=centers, seed=seed, dtype=torch.bfloat16,
                            device="cuda", gen_device="cuda")
    hk = B * H_KV
    return K.view(hk, n + extra, D), V.view(hk, n + extra, D), q.view(B * H, D)


def _same(idx, canon, fields=STATE):
    torch.cuda.synchronize()
    got = CanonIndex.from_gpu(idx)
    for f in fields:
        a, b = getattr(got, f), getattr(canon, f)
        if a is None and b is None:
            continue
        same = np.array_equal(a.view(np.uint8), b.view(np.uint8)) if a.dtype.kind == "f" else np.array_equal(a, b)
        if not same:
            bad = np.argwhere((a.view(np.uint8) != b.view(np.uint8)) if a.dtype.kind == "f" else (a != b))
            raise AssertionError(f"{f} differs at {len(bad)} places, first {bad[:3].tolist()}")


def _check_output(out, q, K, V, labels, w, n):
    want = ref.label_weighted_attention(q.double().cpu().numpy(), K[:, :n].double().cpu().numpy(),
                                        V[:, :n].double().cpu().numpy(), labels[:, :n].astype(np.int64), w)
    np.testing.assert_allclose(out.double().cpu().numpy(), want, rtol=0, atol=2e-2)


@pytest.mark.parametrize("budget", [0.2, 0.05])
def test_config2_8x8k_full_size_step(budget):
    """8 sequences x 8192 tokens, 256 k-means clusters each, window 64: one graph step at n + 1.
    The 64-head fit is checked through the state it leaves (counts against a recount of the
    labels); the oracle, given that state, fixes the selection, the rows read per head, the
    output, and the state after the step's own insertion of the key that leaves the window at
    n + 2 (drift flags included, delta = 0.03)."""
    from ssa_amd.graph_kernels import SphereIndexGraph
    B, n, C, W = 8, 8192, 256, 64
    K, V, q = _folded(B, n, 8, seed=31, centers=C)
    hk = B * H_KV
    idx = SphereIndexGraph(budget=budget, C=C, window=W, delta=0.03, capacity=n + 8, check_every=10 ** 9,
                           partition="kmeans")
    idx.prepare(K, n, B * H)
    assert idx.insert_ahead and idx.work.S >= 2
    canon = CanonIndex.from_gpu(idx)
    end = int(canon.end[0])
    assert end == n + 1 - W
    sizes = canon.count[:, :C]
    assert sizes.max() > 3 * sizes[sizes > 0].min()          # ragged cluster sizes
    for h in range(hk):
        assert np.array_equal(np.bincount(canon.labels[h, 1:end], minlength=C)[:C], canon.count[h])
    n_dev = torch.full((1,), n + 1, dtype=torch.int32, device="cuda")
    out = idx.step(q, K, V, n_dev).clone()
    torch.cuda.synchronize()
    want_w = canon.select(q, budget=budget)
    assert np.array_equal(idx.wbuf.cpu().numpy(), want_w)
    rows = [len(p) for p in canon.compact(want_w, n + 1)]
    assert idx.work.cnt.tolist() == rows
    need = math.ceil(budget * (end - 1))
    for h in range(hk):
        assert int(canon.count[h][want_w[h, :C] > 0].sum()) >= need
    _check_output(out, q, K, V, canon.labels, want_w, n + 1)
    canon.insert(K, n + 2, window=W, delta=0.03)
    _same(idx, canon)


@pytest.mark.parametrize("ahead", [False, True])
@pytest.mark.parametrize("B,n", [(16, 2048), (64, 1024)])
@pytest.mark.parametrize("budget", [0.2, 0.05])
def test_many_heads_steps_match_the_oracle(B, n, budget, ahead):
    """128 and 512 folded heads: the doubled split count and the XCD placement over large grids,
    with a separate insertion launch and with insert-ahead (staged by each head's last split: an
    extra workgroup per head would not be resident), for 12 steps, against the full oracle (fit
    included)."""
    from ssa_amd.graph_kernels import SphereIndexGraph
    from ssa_amd.sphere_fused import kmeans_init_indices
    C, W, steps = 64, 64, 12
    K, V, q = _folded(B, n, steps + 8, seed=41 + B, centers=C)
    hk = B * H_KV
    idx = SphereIndexGraph(budget=budget, C=C, window=W, delta=0.03, capacity=n + steps + 8, check_every=10 ** 9,
                           partition="kmeans", insert_ahead=ahead)
    idx.prepare(K, n, B * H)
    from ssa_amd.labeled_attn import cu_count
    cus = cu_count(q.device)
    assert idx.insert_ahead == ahead
    assert -(-cus // hk) <= 2 and idx.work.S == max(1, -(-2 * cus // hk))   # two workgroups per compute unit
    if ahead:
        assert hk * (idx.work.S + 1) > 2 * cus                # the stage folds into split S - 1
    Kf = K.float().cpu().numpy()                              # the oracle's fp32 copy of the cache
    canon = CanonIndex(hk, D, C=C, capacity=idx.capacity, C_init=C, partition="kmeans", summary_bits=8, ms=idx.MS)
    end0 = n - W
    canon.build(Kf, start=1, end=end0, fit=True, iters=idx.kmeans_iters,
                init_idx=kmeans_init_indices(end0 - 1, C, idx.seed).numpy())
    if ahead:                                                 # prepare binned the first step's keys
        canon.insert(Kf, n + 1, window=W, delta=0.03)
    _same(idx, canon)
    n_dev = torch.full((1,), n, dtype=torch.int32, device="cuda")
    for m in range(n + 1, n + steps + 1):
        n_dev.fill_(m)
        out = idx.step(q, K, V, n_dev).clone()
        torch.cuda.synchronize()
        canon.insert(Kf, m, window=W, delta=0.03)
        want_w = canon.select(q, budget=budget)
        assert np.array_equal(idx.wbuf.cpu().numpy(), want_w), m
        assert idx.work.cnt.tolist() == [len(p) for p in canon.compact(want_w, m)], m
        if m == n + steps:
            _check_output(out, q, K, V, canon.labels, want_w, m)
    if ahead:                                                 # the last step binned the next length's keys
        canon.insert(Kf, n + steps + 1, window=W, delta=0.03)
    _same(idx, canon)


def test_all_layer_insert_matches_per_layer_insertion():
    """Three layers with caches at layer offsets of one allocation: AllLayerInsert bins every
    layer's leaving key in one launch (in-kernel splits included) and each layer's step then
    selects from its own state; every layer's state and selection against the oracle."""
    from ssa_amd.graph_kernels import AllLayerInsert, SphereIndexGraph
    from ssa_amd.sphere_fused import kmeans_init_indices
    from ssa_amd.synth import make_cache
    L, B, n, C, C_init, W, steps = 3, 2, 1500, 64, 16, 32, 40
    hk = B * H_KV
    Kall = torch.zeros(L, hk, n + steps + 8, D, dtype=torch.bfloat16, device="cuda")
    Vall = torch.zeros_like(Kall)
    qs = []
    for layer in range(L):
        K, V, q, _ = make_cache(B, H_KV, n + steps + 8, D, H=H, centers=C_init, seed=60 + layer,
                                dtype=torch.bfloat16, device="cuda")
        Kall[layer], Vall[layer] = K.view(hk, -1, D), V.view(hk, -1, D)
        qs.append(q.view(B * H, D))
    layers, canons = [], []
    cap = float(1.5 * (n - W - 1) / C_init)
    for layer in range(L):
        idx = SphereIndexGraph(budget=0.2, insert_ahead=False, C=C, C_init=C_init, window=W, delta=0.03,
                               capacity=n + steps + 8, check_every=10 ** 9, partition="kmeans")
        idx.observe(Kall[layer], n)
        idx.cap.fill_(cap)
        idx.prepare(Kall[layer], n, B * H)
        c = CanonIndex(hk, D, C=C, capacity=idx.capacity, C_init=C_init, partition="kmeans", summary_bits=8,
                       ms=idx.MS)
        c.build(Kall[layer], start=1, end=n - W, fit=True, iters=idx.kmeans_iters,
                init_idx=kmeans_init_indices(n - W - 1, C_init, idx.seed).numpy())
        c.cap[:] = np.float32(cap)
        layers.append(idx)
        canons.append(c)
    ins = AllLayerInsert(layers, [Kall[layer] for layer in range(L)])
    n_dev = torch.full((1,), n, dtype=torch.int32, device="cuda")
    for m in range(n + 1, n + steps + 1):
        n_dev.fill_(m)
        ins(n_dev)
        for layer in range(L):
            layers[layer].step(qs[layer], Kall[layer], Vall[layer], n_dev, insert=False)
        torch.cuda.synchronize()
        for layer in range(L):
            canons[layer].insert(Kall[layer], m, window=W, delta=0.03)
            assert np.array_equal(layers[layer].wbuf.cpu().numpy(), canons[layer].select(qs[layer], budget=0.2)), \
                (m, layer)
    for layer in range(L):
        _same(layers[layer], canons[layer])
    assert sum(int(c.nsplit.sum()) for c in canons) > 0, "the cap should split clusters during the steps"
