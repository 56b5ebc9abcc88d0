"""The engine seam and its model surface on the CPU (no kernel launch): implementation names
(src/ssa/attn/__init__.py:17-25; reference tests/test_legacy_names.py), the byte accounting
(src/ssa/attn/accounting.py:19-32; reference tests/test_accounting.py), install / uninstall
(src/ssa/models/patch.py:245-258), ``ReadStats`` arithmetic, and the minimal Qwen3 model's
incremental decode against its own full forward pass."""

from __future__ import annotations

import pytest
import torch

from oracle import reference as ref
from ssa_amd import accounting
from ssa_amd.patch import ReadStats, canonical, install, make_decode_op, uninstall
from ssa_amd.qwen3 import Qwen3Config, causal_attention, random_model

TINY = Qwen3Config(vocab_size=48, hidden_size=32, num_hidden_layers=2, num_attention_heads=4, num_key_value_heads=2,
                   head_dim=16, intermediate_size=64, max_position_embeddings=256)


def test_canonical_maps_every_old_name():
    new = {"skip": "cluster_skip", "skip_v1": "cluster_skip_v1", "fused": "cluster_fused",
           "sample": "cluster_tail_sample", "tail": "cluster_tail"}
    for suffix, name in new.items():
        assert canonical(f"sphere_{suffix}") == name
        assert canonical(f"voronoi_{suffix}") == name
        assert canonical(name) == name
    assert canonical("dense") == "dense"


def test_accounting_matches_the_restated_reference_term_by_term():
    d, n, rows, c = 128, 32768, 6000.0, 1000.0
    got = accounting.overhead_rows(n=n, rows=rows, clusters=c, d=d, summary_bits=8)
    want = (c * (d + 12) + c * d + 2 * n + 6 * rows + 2 * d + 2 * 4 * d) / (2 * d)
    assert abs(got - want) < 1e-9
    for kw in (dict(summary_bits=32), dict(fitted=False, heads=8), dict(summary_bits=8, key_bits=16)):
        assert abs(accounting.overhead_rows(n=n, rows=rows, clusters=c, d=d, **kw)
                   - ref.overhead_rows(n=n, rows=rows, clusters=c, d=d, **kw)) < 1e-9
    f = accounting.kv_read_fraction(n=1000, rows=200.0, clusters=64.0, d=16, summary_bits=8)
    assert abs(f - (400 + accounting.overhead_rows(n=1000, rows=200.0, clusters=64.0, d=16)) / 2000) < 1e-12
    # bytes of one head's step: K and V rows plus the overhead, in 2-byte key rows of d components
    assert abs(accounting.step_bytes(n=n, rows=rows, clusters=256, d=d)
               - (2 * rows * d * 2 + 256 * (d + 12) + 256 * d + 2 * n + 6 * rows + 2 * d + 8 * d)) < 1e-6


def test_readstats_sums_and_fractions():
    s = ReadStats()
    s.record(n_k=100, reads_per_head=torch.tensor([10.0, 30.0]), kv_rows=50.0)
    s.record_gpu(n_k=200, reads_mean=torch.tensor(40.0), kv_rows=torch.tensor(90.0))
    assert s.steps == 2 and s.avg_n_k == 150.0
    assert abs(s.read_fraction - (20.0 + 40.0) / 300.0) < 1e-12
    assert abs(s.kv_read_fraction - (50.0 + 90.0) / 600.0) < 1e-12
    s.record(n_k=100, reads_per_head=torch.tensor([1.0]))          # untracked K+V rows
    assert s.kv_read_fraction is None
    assert ReadStats().rebuild_rate is None and ReadStats().read_fraction == 1.0


def test_install_sets_and_uninstall_clears_the_op_on_every_layer():
    m = random_model(TINY, dtype=torch.float32)
    stats = install(m, "sphere_fused", budget=0.2, C=16, window=4)
    assert isinstance(stats, ReadStats)
    ops = [layer.attn.decode_attn_op for layer in m.layers]
    assert all(callable(op) for op in ops) and ops[0] is not ops[1]      # one index per layer
    assert ops[0].index.C == 16 and ops[0].index.window == 4
    uninstall(m)
    assert all(layer.attn.decode_attn_op is None for layer in m.layers)


def test_seam_defaults_follow_the_reference():
    op = make_decode_op("cluster_fused", base_seed=0, stats=ReadStats(), cfg={"budget": 0.2})
    idx = op.index
    assert (idx.C, idx.C_init, idx.split_factor, idx.window, idx.capacity) == (1024, 256, 2.0, 64, 65536)
    op = make_decode_op("cluster_fused", base_seed=0, stats=ReadStats(), cfg={"budget": 0.2, "C": 256})
    assert (op.index.C, op.index.C_init, op.index.split_factor) == (256, 256, 0.0)


@pytest.mark.parametrize("impl", ["santa", "cluster_tail", "quest_matched", "topk"])
def test_estimators_off_this_path_are_rejected(impl):
    with pytest.raises(ValueError):
        make_decode_op(impl, base_seed=0, stats=ReadStats(), cfg={"budget": 0.2})


def test_incremental_decode_equals_the_full_forward_pass():
    m = random_model(TINY, dtype=torch.float32, seed=1)
    ids = torch.randint(0, TINY.vocab_size, (2, 40), generator=torch.Generator().manual_seed(0))
    full = m(ids, m.alloc_cache(48, batch=2), start_pos=0)
    c = m.alloc_cache(48, batch=2)
    parts = [m(ids[:, :25], c, start_pos=0)] + [m(ids[:, t:t + 1], c) for t in range(25, 40)]
    torch.testing.assert_close(torch.cat(parts, 1), full, rtol=1e-5, atol=1e-5)
    assert c.cur_len == 40


def test_causal_attention_matches_the_naive_loop():
    g = torch.Generator().manual_seed(3)
    B, H, Hk, T, n0, d = 1, 4, 2, 5, 7, 8
    q = torch.randn(B, H, T, d, generator=g, dtype=torch.float64)
    K = torch.randn(B, Hk, n0 + T, d, generator=g, dtype=torch.float64)
    V = torch.randn(B, Hk, n0 + T, d, generator=g, dtype=torch.float64)
    got = causal_attention(q, K, V, n0, chunk=2)
    for h in range(H):
        for t in range(T):
            s = (K[0, h // 2, :n0 + t + 1] @ q[0, h, t]) / d ** 0.5
            want = torch.softmax(s, 0) @ V[0, h // 2, :n0 + t + 1]
            torch.testing.assert_close(got[0, h, t].double(), want, rtol=1e-5, atol=1e-5)
