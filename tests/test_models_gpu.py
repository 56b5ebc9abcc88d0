"""The captured decode loop at the real model widths of configs[3] and configs[4] (random bf16
weights; there is no checkpoint): Qwen3-0.6B (28 layers, hidden 1024, 16 / 8 heads, vocab
151936) and Qwen3-4B (36 layers, hidden 2560, 32 / 8 heads, G = 4).

* graph replays equal the eager step bit for bit (0.6B, batch 2, cluster mode with the graph
  decoder's defaults: 1,024 slots, 256 fitted, post-fit division, in-step splits);
* the full budget equals dense (0.6B);
* a few hundred decode steps at the 4B shape with the cluster count growing by in-step splits:
  one layer's whole index state against the oracle replaying the same steps (prompt fit, post-fit
  division, insertion with splits, and the drift checks every 16 steps).

Reference: src/ssa/models/graph_decode.py:29-157 and its tests/test_graph_decode.py (graph equals
eager; full budget equals dense); whole-model logits have no golden values (the reference's
engine is not available), so the model is pinned by these equalities.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.canon import CanonIndex
from ssa_amd.graph_decode import GraphDecoder
from ssa_amd.qwen3 import QWEN3_0_6B, QWEN3_4B, random_model

pytestmark = pytest.mark.gpu

STATE = ("n_c", "sum_dir", "dir8", "cent", "cent8", "mmax", "mmin", "count", "ksum", "mu_ref", "rbar", "end",
         "nsplit", "labels", "flags", "cap")


def _run(model, ids, P, T, *, mode, capture, **kw):
    cache = model.alloc_cache(P + T + 1, batch=ids.shape[0])
    with torch.inference_mode():
        logits = model(ids[:, :P], cache, start_pos=0, last_only=True)
        dec = GraphDecoder(model, cache, mode=mode, **kw)
        dec.prepare(P)
        if capture:
            dec.capture()
        tok = logits[:, -1].argmax(-1, keepdim=True)
        out = []
        for pos in range(P, P + T):
            lg = dec.step(tok, pos)
            out.append(lg[:, -1].float().clone())
            tok = ids[:, pos + 1:pos + 2] if pos + 1 < P + T else tok
    return torch.stack(out), dec


@pytest.fixture(scope="module")
def small():
    model = random_model(QWEN3_0_6B, dtype=torch.bfloat16, device="cuda", seed=1)
    ids = torch.randint(0, QWEN3_0_6B.vocab_size, (2, 400 + 6), device="cuda",
                        generator=torch.Generator(device="cuda").manual_seed(1))
    return model, ids


def test_qwen3_0p6b_graph_replays_equal_the_eager_step(small):
    model, ids = small
    eager, _ = _run(model, ids, 400, 6, mode="cluster", capture=False, budget=0.2)
    graph, dec = _run(model, ids, 400, 6, mode="cluster", capture=True, budget=0.2)
    assert torch.equal(eager, graph)
    assert dec.attn[0].C == 1024 and dec.attn[0].C_init == 256


def test_qwen3_0p6b_full_budget_equals_dense(small):
    model, ids = small
    dense, _ = _run(model, ids, 400, 6, mode="dense", capture=True)
    full, _ = _run(model, ids, 400, 6, mode="cluster", capture=True, budget=1.0)
    err = float((full - dense).norm() / dense.norm())
    assert err < 1e-2, err


def _oracle_layer(K, P, T, *, C, C_init, W, delta, split_factor, check_every, ahead, seed=0):
    """One layer's index as the reference would leave it after the prompt and T decode steps."""
    from ssa_amd.sphere_fused import kmeans_init_indices
    Hk, cap_len, d = K.shape
    canon = CanonIndex(Hk, d, C=C, capacity=cap_len, C_init=C_init, partition="kmeans", summary_bits=8,
                       ms=min(8192, cap_len))
    end = P - W
    nb = end - 1
    canon.build(K, start=1, end=end, fit=True, iters=10, init_idx=kmeans_init_indices(nb, C_init, seed).numpy())
    canon.cap[:] = np.float32(split_factor * nb / C_init)
    canon.split_after_fit(K, start=1, end=end, split_factor=split_factor)
    if ahead:
        canon.insert(K, P + 1, window=W, delta=delta)
    recentred = 0
    for step, n in enumerate(range(P + 1, P + T + 1), 1):
        canon.insert(K, n + 1 if ahead else n, window=W, delta=delta)
        if step % check_every == 0:                       # the synchronous check, as after_replay does
            flags = canon.flags.copy()
            nbn = int(canon.end[0]) - 1
            rec = [h for h in range(Hk) if (flags[h] & 1) and not (flags[h] & 2)]
            if rec:
                mu = (canon.ksum[rec] / np.float32(nbn)).astype(np.float32)
                canon.build(K, start=1, end=int(canon.end[0]), heads=rec, mu=mu, fit=False)
                recentred += len(rec)
            canon.flags[:] = 0
    return canon, recentred


def test_qwen3_4b_long_decode_layer_state_matches_the_oracle():
    """Batch 1, a 1,000-token prompt and 300 greedy steps at the 4B shape (32 query heads per 8
    KV heads): clusters split past twice the fitted mean size as keys arrive, so the cluster
    count grows; layer 5's state (labels, summaries, int8 copies, counts, splits, flags, lengths)
    equals the oracle's."""
    P, T, layer = 1000, 300, 5
    model = random_model(QWEN3_4B, dtype=torch.bfloat16, device="cuda", seed=2)
    ids = torch.randint(0, QWEN3_4B.vocab_size, (1, P), device="cuda",
                        generator=torch.Generator(device="cuda").manual_seed(2))
    cache = model.alloc_cache(P + T + 1, batch=1)
    with torch.inference_mode():
        logits = model(ids, cache, start_pos=0, last_only=True)
        dec = GraphDecoder(model, cache, mode="cluster", budget=0.2, greedy=True)
        dec.prepare(P)
        dec.capture()
        idx = dec.attn[layer]
        assert idx.insert_ahead and dec.B * dec.H // (dec.B * dec.H_kv) == 4
        n_c0 = int(idx.n_c.sum())
        tok = logits[:, -1].argmax(-1, keepdim=True)
        for pos in range(P, P + T):
            dec.step(tok, pos)
            tok = dec.next_tok.clone()
    torch.cuda.synchronize()
    assert int(idx.n_c.sum()) > n_c0 and idx.splits > 0, "the cluster count should grow"
    K = dec._heads(cache.k[layer]).float().cpu().numpy()
    canon, recentred = _oracle_layer(K, P, T, C=idx.C, C_init=idx.C_init, W=idx.window, delta=idx.delta,
                                     split_factor=idx.split_factor, check_every=idx.check_every, ahead=True)
    got = CanonIndex.from_gpu(idx)
    for f in STATE:
        a, b = getattr(got, f), getattr(canon, f)
        same = np.array_equal(a.view(np.uint8), b.view(np.uint8)) if a.dtype.kind == "f" else np.array_equal(a, b)
        assert same, f
    assert idx.rebuilds == recentred
