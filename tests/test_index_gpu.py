"""HIP cluster index (prefill fit, insertion, in-kernel split, selection) vs the canonical C
oracle, bit for bit (GPU only).

The oracle (oracle/canon.c) restates SphereIndexGPU's algorithm (src/ssa/attn/sphere_gpu.py),
the fused insertion (src/ssa/kernels/sphere_fused.py:171-227) and split (:49-167) in the same
canonical fp32 order of operations, so labels, counts, summaries, int8 copies, selections and
splits must match exactly. Reference tests mirrored: tests/test_sphere_fused.py (binning and
selection agreement), tests/test_split_kernels.py (in-kernel splits, recounts, cap).
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle.canon import CanonIndex
from oracle import reference as ref

pytestmark = pytest.mark.gpu

FIELDS = ("n_c", "sum_dir", "dir8", "cent", "cent8", "mmax", "mmin", "count", "ksum", "mu_ref", "rbar", "end",
          "nsplit", "labels", "flags")


def _keys(H_kv, n, d=128, *, H=None, seed=0, dtype=torch.bfloat16, centers=64):
    from ssa_amd.synth import make_cache
    K, V, q, _ = make_cache(1, H_kv, n, d, H=H, centers=centers, seed=seed, dtype=dtype, device="cuda")
    return K[0], V[0], q[0]


def _same(gpu_idx, canon: CanonIndex, fields=FIELDS):
    torch.cuda.synchronize()
    other = CanonIndex.from_gpu(gpu_idx)
    for f in fields:
        a, b = getattr(other, f), getattr(canon, f)
        if a is None and b is None:
            continue
        if f == "cent" and gpu_idx.partition != "kmeans":
            continue
        assert a.shape == b.shape, f
        same = np.array_equal(a.view(np.uint8), b.view(np.uint8)) if a.dtype.kind == "f" else np.array_equal(a, b)
        if not same:
            bad = np.argwhere(a != b) if a.dtype.kind != "f" else np.argwhere(a.view(np.uint8) != b.view(np.uint8))
            raise AssertionError(f"{f} differs at {len(bad)} places, first {bad[:3].tolist()}")


def _fused(**kw):
    from ssa_amd.sphere_fused import SphereIndexFused
    base = dict(C=64, window=16, delta=math.inf, capacity=4096, check_every=1, partition="kmeans", async_check=False)
    base.update(kw)
    return SphereIndexFused(**base)


def _canon_like(idx, K, n):
    from ssa_amd.sphere_fused import kmeans_init_indices
    c = CanonIndex(idx.H_kv, idx.d, C=idx.C, capacity=idx.capacity, C_init=idx.C_init, partition=idx.partition,
                   summary_bits=idx.summary_bits, ms=idx.MS,
                   dirs=None if idx.partition == "kmeans" else idx.cent.cpu().numpy())
    end = max(1, n - idx.window)
    nb = end - 1
    init = kmeans_init_indices(nb, idx.C_init, idx.seed).numpy() if nb > 0 else None
    c.build(K, start=1, end=end, fit=True, iters=idx.kmeans_iters, init_idx=init)
    return c


@pytest.mark.parametrize("summary_bits", [8, 32])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_prefill_fit_is_bit_exact(summary_bits, dtype):
    K, V, q = _keys(3, 1500, seed=1, dtype=dtype)
    idx = _fused(summary_bits=summary_bits)
    idx.observe(K, 1500)
    _same(idx, _canon_like(idx, K, 1500))


def test_prefill_random_partition_is_bit_exact():
    K, V, q = _keys(2, 1200, seed=2)
    idx = _fused(partition="random", C=128)
    idx.observe(K, 1200)
    _same(idx, _canon_like(idx, K, 1200))


def test_prefill_duplicate_seeds_tie_to_the_lowest_index():
    """Fewer binned keys than seeds: the seed list cycles (src/ssa/attn/clusterkv.py:34-35), so
    centroids c and c + nb start equal and every assignment between them is an exact tie, which
    the matrix-core assignment must settle as the canonical argmax does (lowest index)."""
    K, V, q = _keys(2, 16 + 1 + 40, seed=4)
    idx = _fused()
    idx.observe(K, 57)
    canon = _canon_like(idx, K, 57)
    _same(idx, canon)
    assert int(canon.count[:, 40:].sum()) == 0


def test_prefill_exact_ties_against_axis_directions():
    """Keys on the diagonals of the first coordinate axes, in +/- pairs so that the binned mean is
    exactly zero: each key's best axes score exactly the same, and the label must be the lowest
    of them (bf16 copies of such keys score the tied axes equally too, and the rescoring breaks
    the tie by index)."""
    g = torch.Generator().manual_seed(5)
    H_kv, d, n = 2, 128, 16 + 1 + 2 * 300
    K = torch.zeros(H_kv, n, d)
    for h in range(H_kv):
        for p in range(300):
            k = torch.zeros(d)
            axes = torch.randperm(64, generator=g)[: int(torch.randint(1, 4, (1,), generator=g))]
            k[axes] = float(torch.randint(1, 3, (1,), generator=g))
            K[h, 1 + 2 * p], K[h, 2 + 2 * p] = k, -k
        K[h, 0] = torch.randn(d, generator=g)
        K[h, 1 + 600:] = torch.randn(16, d, generator=g)
    K = K.to(torch.bfloat16).cuda()
    idx = _fused(partition="random", kind="cross", C=64)
    idx.observe(K, n)
    canon = _canon_like(idx, K, n)
    _same(idx, canon)
    lab = canon.labels[:, 1:601]
    keys = K[:, 1:601].float().cpu().numpy()
    for h in range(H_kv):
        pos = keys[h, ::2, :64]
        assert np.array_equal(lab[h, ::2], np.argmax(pos, axis=1))          # first of the tied maxima


@pytest.mark.parametrize("summary_bits", [8, 32])
def test_insertion_is_bit_exact(summary_bits):
    K, V, q = _keys(4, 1600, seed=3)
    idx = _fused(summary_bits=summary_bits)
    idx.observe(K, 1000)
    canon = _canon_like(idx, K, 1000)
    for n in range(1001, 1600, 7):
        idx.observe(K, n)
        canon.insert(K, n, window=16, delta=math.inf)
    _same(idx, canon)
    counts = np.stack([np.bincount(canon.labels[h, 1:canon.end[h]], minlength=64) for h in range(4)])
    assert np.array_equal(counts, canon.count)


@pytest.mark.parametrize("delta", [0.02, 0.2])
def test_insertion_drift_flags_are_bit_exact(delta):
    """The flags the insertion kernel sets (src/ssa/kernels/sphere_fused.py:223-227), step by
    step: bit 0 when |ksum / nb - mu_ref| > delta * rbar, on keys whose mean moves away from the
    fitted one; bit 1 once a head's cluster count, grown by in-kernel splits, reaches reset_at.
    The host never acts on the flags here (check_every is huge), so GPU and oracle see the same
    keys."""
    K, V, q = _keys(4, 1800, seed=13, centers=16)
    drift = torch.zeros_like(K)
    drift[:, 1000:, :8] = 3.0                                  # keys after the fit lean one way
    K = (K.float() + drift.float()).to(K.dtype)
    idx = _fused(C=64, C_init=16, delta=delta, check_every=10 ** 9, reset_at=20)
    idx.observe(K, 1000)
    canon = _canon_like(idx, K, 1000)
    cap = float(1.5 * (1000 - 17) / 16)
    idx.cap.fill_(cap)
    canon.cap[:] = cap
    seen = set()
    for n in range(1001, 1800, 9):
        idx.observe(K, n)
        canon.insert(K, n, window=16, delta=delta, reset_at=20)
        _same(idx, canon, fields=("flags", "end", "ksum", "count", "n_c"))
        seen |= set(np.unique(canon.flags).tolist())
    _same(idx, canon)
    assert seen & {1, 3}, "some head should drift"
    assert seen & {2, 3} and int(canon.n_c.max()) >= 20, "some head should reach reset_at"


@pytest.mark.parametrize("group", ["sum_share", "per_head", "max", "max_rel"])
@pytest.mark.parametrize("budget", [0.05, 0.2, 0.5, 1.0])
def test_selection_is_bit_exact_given_identical_summaries(group, budget):
    K, V, q = _keys(4, 1500, H=16, seed=4)
    idx = _fused()
    idx.observe(K, 1500)
    canon = CanonIndex.from_gpu(idx)
    for t in range(3):
        qq = q if t == 0 else (q * (t + 0.5)).to(q.dtype)
        _, w = idx.labels_and_weights(qq, n=1500, budget=budget, group=group)
        want = canon.select(qq, budget=budget, group=group)
        assert np.array_equal(w.cpu().numpy(), want)
        # a float64 restatement of the reference agrees up to clusters at the threshold
        w64 = ref.labels_and_weights(qq.float().cpu().numpy(), canon.sum_dir if idx.summary_bits == 32 else
                                     canon.dir8.astype(np.float64), canon.mmax, canon.mmin, canon.count, canon.n_c,
                                     nb=int(canon.end[0]) - 1, budget=budget, group=group)
        assert int((w64 != want).sum(1).max()) <= 1


@pytest.mark.parametrize("group", ["sum_share", "per_head", "max", "max_rel"])
@pytest.mark.parametrize("H", [8, 16])
def test_selection_past_256_clusters_is_bit_exact(group, H):
    """Scoring runs in rounds of 256 slots: with 520 clusters fitted (rounds 0, 1 and a partial
    round 2), the standalone selection and the fused step's own selection both equal the
    oracle's, at two and four query heads per KV head."""
    n = 4096
    K, V, q = _keys(4, n, d=64, H=H, seed=31, centers=128)
    idx = _fused(C=1024, C_init=520, window=16, capacity=n + 64, check_every=10 ** 9)
    idx.observe(K, n)
    canon = CanonIndex.from_gpu(idx)
    assert int(canon.n_c.min()) == 520
    for budget in (0.05, 0.2):
        _, w = idx.labels_and_weights(q, n=n, budget=budget, group=group)
        want = canon.select(q, budget=budget, group=group)
        assert np.array_equal(w.cpu().numpy(), want)
    out, labels, w = idx.attend(q, K, V, n=n, budget=0.2, group=group)
    torch.cuda.synchronize()
    assert np.array_equal(w.cpu().numpy(), canon.select(q, budget=0.2, group=group))
    want = ref.label_weighted_attention(q.double().cpu().numpy(), K.double().cpu().numpy(),
                                        V.double().cpu().numpy(), canon.labels[:, :n], w.cpu().numpy())
    np.testing.assert_allclose(out.double().cpu().numpy(), want, rtol=0, atol=2e-2)


@pytest.mark.parametrize("kn_rows", [0, 8, 512])
def test_in_kernel_splits_are_bit_exact_and_keep_the_cap(kn_rows):
    """In-kernel splits with the members' unit directions recomputed in every pass (kn_rows 0),
    computed once into the state's split scratch (512 rows: every cluster fits), or both (8 rows:
    the larger clusters recompute): the same state as the oracle in each case."""
    K, V, q = _keys(3, 2600, seed=5, centers=16)
    idx = _fused(C=128, C_init=16)
    idx.observe(K, 1000)
    if kn_rows:                                   # the scratch a splitting index allocates
        idx.kn_rows = kn_rows
        idx._knbuf = torch.empty(3, kn_rows, 128, device="cuda")
    canon = _canon_like(idx, K, 1000)
    cap = float(1.5 * (1000 - 17) / 16)
    idx.cap.fill_(cap)
    canon.cap[:] = cap
    for n in range(1001, 2600, 5):
        idx.observe(K, n)
        canon.insert(K, n, window=16, delta=math.inf)
    _same(idx, canon)
    assert int(canon.nsplit.sum()) > 0 and idx.splits == int(canon.nsplit.sum())
    assert np.all(canon.count <= cap)
    for h in range(3):
        e = canon.end[h]
        assert np.array_equal(np.bincount(canon.labels[h, 1:e], minlength=128), canon.count[h])
        assert np.all(canon.labels[h, 1:e] < canon.n_c[h])
    assert np.all(canon.count[np.arange(128)[None, :] >= canon.n_c[:, None]] == 0)


@pytest.mark.parametrize("summary_bits", [8, 32])
def test_post_fit_division_is_bit_exact(summary_bits):
    """split_factor > 0 at the fit: the k-means round then the bisection rounds of the post-fit
    division (src/ssa/attn/sphere_gpu.py:307-391) leave the same state on the GPU as in the
    oracle, every cluster under the cap, and the following insertions and selection agree too."""
    K, V, q = _keys(3, 2400, H=6, seed=9, centers=6)
    n = 2000
    idx = _fused(C=128, C_init=16, split_factor=2.0, summary_bits=summary_bits)
    idx.observe(K, n)
    canon = _canon_like(idx, K, n)
    end = n - idx.window
    canon.cap[:] = np.float32(2.0 * (end - 1) / 16)
    rounds = canon.split_after_fit(K, start=1, end=end, split_factor=2.0, iters=idx.kmeans_iters)
    _same(idx, canon)
    assert rounds >= 2 and int(canon.nsplit.sum()) > 0 and idx.splits == int(canon.nsplit.sum())
    for h in range(3):
        nc = int(canon.n_c[h])
        assert np.all(canon.count[h, :nc] <= canon.cap[h]) or nc == 128
        assert np.array_equal(np.bincount(canon.labels[h, 1:end], minlength=128), canon.count[h])
    for m in range(n + 1, n + 40):
        idx.observe(K, m)
        canon.insert(K, m, window=16, delta=math.inf)
    _same(idx, canon)
    w = idx.labels_and_weights(q, n=n + 39, budget=0.2)[1]
    assert np.array_equal(w.cpu().numpy(), canon.select(q, budget=0.2))


def test_post_fit_division_into_more_than_64_parts():
    """A cap far below the fitted clusters' sizes (cap_keys = 10 against ~370 keys per cluster):
    the k-means round divides each cluster into max(2, ceil(m * split_factor / cap)) >= 64 parts,
    beyond the 32 held on chip, so the parts' centroids and sums live in the caller's scratch.
    Same state as the oracle, which has no limit on the parts (src/ssa/attn/sphere_gpu.py:56-73,
    357-358), and the following insertions and selection agree too."""
    K, V, q = _keys(2, 3100, H=4, seed=23, centers=8)
    n = 3000
    idx = _fused(C=1024, C_init=8, cap_keys=10.0, capacity=4096)
    idx.observe(K, n)
    canon = _canon_like(idx, K, n)
    end = n - idx.window
    canon.cap[:] = np.float32(10.0)
    fitted = canon.count.copy()
    assert math.ceil(int(fitted.max()) * 2.0 / 10.0) >= 64
    rounds = canon.split_after_fit(K, start=1, end=end, split_factor=idx.split_factor, iters=idx.kmeans_iters)
    _same(idx, canon)
    assert rounds >= 1 and int(canon.n_c.min()) > 8 * 32
    for h in range(2):
        assert np.array_equal(np.bincount(canon.labels[h, 1:end], minlength=1024), canon.count[h])
    for m in range(n + 1, n + 20):
        idx.observe(K, m)
        canon.insert(K, m, window=16, delta=math.inf)
    _same(idx, canon)
    w = idx.labels_and_weights(q, n=n + 19, budget=0.2)[1]
    assert np.array_equal(w.cpu().numpy(), canon.select(q, budget=0.2))


def test_end_to_end_config0_step():
    """Config 0: fp32, 16 query / 8 KV heads, d=128, n=4096, 256 clusters, 10 k-means iterations,
    20% budget: labels, selection and selected indices bit-exact; output within 1e-5."""
    from ssa_amd.labeled_attn import compact_positions
    K, V, q = _keys(8, 4096, H=16, seed=0, dtype=torch.float32, centers=256)
    idx = _fused(C=256, window=64, delta=0.03, check_every=16)
    out, labels, w = idx.attend(q, K, V, n=4096, budget=0.2)
    torch.cuda.synchronize()
    canon = _canon_like(idx, K, 4096)
    _same(idx, canon)
    want_w = canon.select(q, budget=0.2)
    assert np.array_equal(w.cpu().numpy(), want_w)
    idx_list, cnt = compact_positions(labels, w)
    want_idx = canon.compact(want_w, 4096)
    for h in range(8):
        assert np.array_equal(idx_list[h, :int(cnt[h])].cpu().numpy(), want_idx[h])
    want = ref.label_weighted_attention(q.double().cpu().numpy(), K.double().cpu().numpy(),
                                        V.double().cpu().numpy(), canon.labels[:, :4096], want_w)
    np.testing.assert_allclose(out.double().cpu().numpy(), want, rtol=0, atol=1e-5)


@pytest.mark.parametrize("H,H_kv,d,dtype,group", [
    (8, 8, 64, torch.float16, "sum_share"),      # G = 1
    (32, 8, 128, torch.bfloat16, "sum_share"),   # G = 4 (Qwen3-4B)
    (16, 2, 256, torch.bfloat16, "max"),         # G = 8, d = 256
    (8, 4, 16, torch.float32, "per_head"),       # smallest head
])
def test_fused_step_shapes_match_the_oracle(H, H_kv, d, dtype, group):
    """The fused step (selection in every workgroup, compaction, split-K attention, merge) at
    the GQA groups, head sizes and cache dtypes the kernels are built for: selection bit-exact
    against the oracle, output within the dtype's tolerance of the float64 spec."""
    n = 2500
    K, V, q = _keys(H_kv, n, d=d, H=H, seed=21, dtype=dtype, centers=32)
    idx = _fused(C=64, window=16, delta=math.inf, check_every=10 ** 9)
    out, labels, w = idx.attend(q, K, V, n=n, budget=0.2, group=group)
    torch.cuda.synchronize()
    canon = _canon_like(idx, K, n)
    _same(idx, canon)
    want_w = canon.select(q, budget=0.2, group=group)
    assert np.array_equal(w.cpu().numpy(), want_w)
    want = ref.label_weighted_attention(q.double().cpu().numpy(), K.double().cpu().numpy(),
                                        V.double().cpu().numpy(), canon.labels[:, :n], want_w)
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    np.testing.assert_allclose(out.double().cpu().numpy(), want, rtol=0, atol=tol)


@pytest.mark.parametrize("budget", [0.4, 0.2, 0.1, 0.05])
def test_config1_full_size_selection_and_output(budget):
    """configs[1] at its full size (B=1, 16 q / 8 kv heads, d=128, bf16, n=32768, 256 k-means
    clusters, window 64) through the fused step. The 10-iteration fit at 32k is too slow for the
    C oracle in a test, so the oracle takes the GPU's fitted state (``CanonIndex.from_gpu``) and
    restates what the north_star contract pins given identical summaries: the selection ``w`` and
    the selected positions, bit for bit; the summaries against a recount of the labels; the
    output against the float64 spec (2e-2)."""
    from ssa_amd.labeled_attn import compact_positions
    n, C, W = 32768, 256, 64
    K, V, q = _keys(8, n + 64, H=16, seed=3, dtype=torch.bfloat16, centers=256)
    idx = _fused(C=C, window=W, delta=0.03, capacity=n + 64, check_every=10 ** 9)
    out, labels, w = idx.attend(q, K, V, n=n, budget=budget)
    torch.cuda.synchronize()
    canon = CanonIndex.from_gpu(idx)
    end = n - W
    lab = canon.labels[:, :n].astype(np.int64)
    assert (lab[:, 0] == C).all() and (lab[:, end:] == C).all()          # sink and window: exact set
    assert (lab[:, 1:end] < canon.n_c[:, None]).all()
    for h in range(8):
        assert np.array_equal(np.bincount(lab[h, 1:end], minlength=C)[:C], canon.count[h].astype(np.int64))
    want_w = canon.select(q, budget=budget)
    got_w = w.cpu().numpy()
    assert np.array_equal(got_w, want_w)
    need = math.ceil(budget * (end - 1))
    for h in range(8):
        sel = got_w[h, :C] > 0
        assert got_w[h, C] == 1.0 and int(canon.count[h][sel].sum()) >= need
    idx_list, cnt = compact_positions(labels, w)
    want_idx = canon.compact(want_w, n)
    for h in range(8):
        assert np.array_equal(idx_list[h, :int(cnt[h])].cpu().numpy(), want_idx[h])
    want = ref.label_weighted_attention(q.double().cpu().numpy(), K[:, :n].double().cpu().numpy(),
                                        V[:, :n].double().cpu().numpy(), lab, want_w)
    np.testing.assert_allclose(out.double().cpu().numpy(), want, rtol=0, atol=2e-2)


def test_fused_step_refuses_labels_other_than_the_state_rows():
    """ssa_sparse_step computes its selection from the index state, so it accepts only the
    state's own label buffer with its row stride (hipErrorInvalidValue = 1 otherwise)."""
    from ssa_amd._lib import lib, stream_ptr
    from ssa_amd.labeled_attn import SplitWork, attn_args
    K, V, q = _keys(4, 600, H=8, seed=2, dtype=torch.bfloat16, centers=16)
    idx = _fused(C=16, window=16, capacity=600)
    idx.attend(q, K, V, n=600, budget=0.2)
    w = idx._wbuf("sum_share", 4)
    work = SplitWork(4, 2, 2, 128, q.device)
    out = torch.empty_like(q)
    st, sel = idx._state(), idx._select_args(q, w, 0.2, "sum_share")
    wider = torch.full((4, idx.capacity + 64), 0, device="cuda", dtype=idx.labels.dtype)
    for labels in (idx.labels.clone(), wider):
        a = attn_args(q, K, V, out, work, labels=labels, w=w, n_host=600)
        assert lib().ssa_sparse_step(st, sel, a, None, stream_ptr(q.device)) == 1
    a = attn_args(q, K, V, out, work, labels=idx.labels, w=w, n_host=600)
    assert lib().ssa_sparse_step(st, sel, a, None, stream_ptr(q.device)) == 0
    torch.cuda.synchronize()
