"""The decode seam and the captured whole-model decode step on the GPU, on a tiny random Qwen3.

Mirrors the reference's tests/test_patch_fused.py (full budget equals dense, partial budget reads
fewer rows, untracked mode records nothing), tests/test_legacy_names.py (old names give the same
outputs) and tests/test_graph_decode.py (graph replays equal the eager step; full budget equals
dense)."""

from __future__ import annotations

import pytest
import torch

from ssa_amd.graph_decode import GraphDecoder
from ssa_amd.patch import install, uninstall
from ssa_amd.qwen3 import Qwen3Config, random_model

pytestmark = pytest.mark.gpu

CFG = Qwen3Config(vocab_size=64, hidden_size=64, num_hidden_layers=2, num_attention_heads=4, num_key_value_heads=2,
                  head_dim=16, intermediate_size=128, max_position_embeddings=512)
P, T = 150, 20


def _setup(dtype=torch.float32):
    model = random_model(CFG, dtype=dtype, device="cuda", seed=0, std=0.2)
    ids = torch.randint(0, CFG.vocab_size, (1, P + T), device="cuda",
                        generator=torch.Generator(device="cuda").manual_seed(0))
    return model, ids


def _decode(model, ids):
    cache = model.alloc_cache(ids.shape[1] + 1, batch=ids.shape[0])
    out = []
    with torch.inference_mode():
        model(ids[:, :P], cache, start_pos=0)
        for t in range(P, P + T):
            out.append(model(ids[:, t:t + 1], cache)[:, -1].float())
    return torch.stack(out)


def test_full_budget_matches_dense():
    model, ids = _setup()
    want = _decode(model, ids)
    stats = install(model, "cluster_fused", budget=1.0, C=16, window=4, delta=0.03, group="sum_share")
    got = _decode(model, ids)
    uninstall(model)
    torch.testing.assert_close(got, want, rtol=1e-2, atol=1e-2)
    assert stats.kv_read_fraction > 1.0                   # every row plus the summaries


def test_partial_budget_reads_fewer_rows_and_stays_finite():
    model, ids = _setup()
    stats = install(model, "cluster_fused", budget=0.2, C=16, window=4, delta=0.03, group="sum_share")
    got = _decode(model, ids)
    uninstall(model)
    assert torch.isfinite(got).all()
    assert 0.0 < stats.read_fraction < 0.8
    assert 0.0 < stats.kv_read_fraction < 1.0
    # the first decode step builds the index (no head step counted), every later one advances it
    assert stats.head_steps == (T - 1) * CFG.num_hidden_layers * CFG.num_key_value_heads


def test_untracked_mode_records_nothing():
    model, ids = _setup()
    stats = install(model, "cluster_fused", budget=0.2, C=16, window=4, track_reads=False)
    _decode(model, ids)
    uninstall(model)
    assert stats.steps == 0 and stats.kv_read_fraction is None


def test_engine_op_accepts_the_old_names():
    model, ids = _setup()
    outs = []
    for name in ("cluster_fused", "voronoi_fused", "sphere_fused"):
        install(model, name, budget=0.2, C=16, window=4, capacity=256)
        outs.append(_decode(model, ids))
        uninstall(model)
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])


def _graph_decode(model, ids, *, mode, capture, B=2, **kw):
    cache = model.alloc_cache(P + T + 1, batch=B)
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


@pytest.mark.parametrize("mode,ahead", [("dense", None), ("cluster", True), ("cluster", False)])
def test_graph_replays_equal_the_eager_step(mode, ahead):
    """Cluster mode with the insertion inside each layer's step launch (insert-ahead) and with one
    all-layer insertion launch at the start of the step."""
    model, _ = _setup(torch.bfloat16)
    ids = torch.randint(0, CFG.vocab_size, (2, P + T), device="cuda",
                        generator=torch.Generator(device="cuda").manual_seed(1))
    kw = dict(budget=0.2, C=16, window=4, insert_ahead=ahead) if mode == "cluster" else {}
    eager, _ = _graph_decode(model, ids, mode=mode, capture=False, **kw)
    graph, dec = _graph_decode(model, ids, mode=mode, capture=True, **kw)
    assert torch.equal(eager, graph)
    assert dec.cache.cur_len == P + T
    if mode == "cluster":
        assert (dec.insert_all is None) == ahead


def test_graph_full_budget_matches_dense_and_the_model():
    model, _ = _setup(torch.float32)
    ids = torch.randint(0, CFG.vocab_size, (2, P + T), device="cuda",
                        generator=torch.Generator(device="cuda").manual_seed(2))
    dense, _ = _graph_decode(model, ids, mode="dense", capture=True)
    full, _ = _graph_decode(model, ids, mode="cluster", capture=True, budget=1.0, C=16, window=4)
    torch.testing.assert_close(full, dense, rtol=1e-3, atol=1e-3)
    # the engine's own eager decode of the same tokens (dense kernel through the model's forward)
    cache = model.alloc_cache(P + T + 1, batch=2)
    with torch.inference_mode():
        logits = model(ids[:, :P], cache, start_pos=0, last_only=True)
        tok = logits[:, -1].argmax(-1, keepdim=True)
        want = []
        for pos in range(P, P + T):
            want.append(model(tok, cache)[:, -1].float())
            tok = ids[:, pos + 1:pos + 2] if pos + 1 < P + T else tok
    torch.testing.assert_close(dense, torch.stack(want), rtol=1e-3, atol=1e-3)


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-4), (torch.bfloat16, 3e-2)])
def test_fused_glue_matches_the_model_modules(dtype, tol):
    """The three glue kernels against the model's own modules run op by op (``glue="torch"``):
    only the order of the RMSNorm mean's sum differs."""
    model, _ = _setup(dtype)
    ids = torch.randint(0, CFG.vocab_size, (2, P + T), device="cuda",
                        generator=torch.Generator(device="cuda").manual_seed(3))
    fused, _ = _graph_decode(model, ids, mode="dense", capture=True, glue="fused")
    ops, _ = _graph_decode(model, ids, mode="dense", capture=True, glue="torch")
    torch.testing.assert_close(fused, ops, rtol=tol, atol=tol)


@pytest.mark.parametrize("M,N,K", [(1, 4096, 1024), (2, 1024, 3072), (2, 6144, 1024), (5, 333, 264), (8, 64, 2048)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_skinny_linear_matches_an_fp32_product(M, N, K, dtype):
    """The decode projections' weight-streaming kernel against an fp32 product of the same
    operands: fp32 accumulation, one rounding."""
    from ssa_amd._lib import check, dtype_tag, lib, stream_ptr
    g = torch.Generator(device="cuda").manual_seed(M * 7 + N)
    x = torch.randn(M, K, device="cuda", generator=g).to(dtype)
    W = (torch.randn(N, K, device="cuda", generator=g) * 0.05).to(dtype)
    y = torch.empty(M, N, device="cuda", dtype=dtype)
    check(lib().ssa_linear_skinny(x.data_ptr(), W.data_ptr(), y.data_ptr(), M, N, K, dtype_tag(dtype),
                                  stream_ptr()), "ssa_linear_skinny")
    want = (x.float() @ W.float().t().contiguous())
    torch.testing.assert_close(y.float(), want, rtol=1e-2, atol=1e-2)


def test_greedy_token_is_the_argmax_of_the_logits():
    """With ``greedy`` the captured step also writes the argmax of its logits (first maximum)."""
    model, _ = _setup(torch.bfloat16)
    cache = model.alloc_cache(P + T + 1, batch=2)
    ids = torch.randint(0, CFG.vocab_size, (2, P), device="cuda", generator=torch.Generator(device="cuda").manual_seed(4))
    with torch.inference_mode():
        model(ids, cache, start_pos=0, last_only=True)
        dec = GraphDecoder(model, cache, mode="cluster", budget=0.2, C=16, window=4, greedy=True)
        dec.prepare(P)
        dec.capture()
        tok = ids[:, -1:]
        for pos in range(P, P + 6):
            lg = dec.step(tok, pos)
            torch.cuda.synchronize()
            assert torch.equal(dec.next_tok, lg[:, -1].argmax(-1, keepdim=True)), pos
            tok = dec.next_tok.clone()


CFG128 = Qwen3Config(vocab_size=96, hidden_size=256, num_hidden_layers=2, num_attention_heads=4, num_key_value_heads=2,
                     head_dim=128, intermediate_size=320, max_position_embeddings=512)


@pytest.mark.parametrize("B", [1, 2, 3])
def test_merged_glue_has_the_bits_of_the_split_glue(B):
    """``glue="fused"`` (gate/up + SwiGLU in one launch) against ``glue="split"`` (two launches):
    the same logits bit for bit, graph-captured, cluster mode."""
    model = random_model(CFG128, dtype=torch.bfloat16, device="cuda", seed=5, std=0.2)
    ids = torch.randint(0, CFG128.vocab_size, (B, P + T), device="cuda",
                        generator=torch.Generator(device="cuda").manual_seed(5))
    kw = dict(budget=0.2, C=16, window=4)
    fused, dec = _graph_decode(model, ids, mode="cluster", capture=True, B=B, glue="fused", **kw)
    split, _ = _graph_decode(model, ids, mode="cluster", capture=True, B=B, glue="split", **kw)
    assert dec._merge_gu
    assert torch.equal(fused, split)


def _lib():
    from ssa_amd._lib import check, dtype_tag, lib, stream_ptr
    return check, dtype_tag, lib(), stream_ptr()


@pytest.mark.parametrize("M,I,K", [(1, 3072, 1024), (2, 333, 264), (5, 100, 64), (8, 64, 2048)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_swiglu_projection_equals_skinny_then_silu_mul(M, I, K, dtype):
    check, dtype_tag, L, s = _lib()
    g = torch.Generator(device="cuda").manual_seed(M * 11 + I)
    x = torch.randn(M, K, device="cuda", generator=g).to(dtype)
    W = (torch.randn(2 * I, K, device="cuda", generator=g) * 0.05).to(dtype)
    gu = torch.empty(M, 2 * I, device="cuda", dtype=dtype)
    want = torch.empty(M, I, device="cuda", dtype=dtype)
    got = torch.full((M, I), float("nan"), device="cuda", dtype=dtype)
    check(L.ssa_linear_skinny(x.data_ptr(), W.data_ptr(), gu.data_ptr(), M, 2 * I, K, dtype_tag(dtype), s), "skinny")
    check(L.ssa_silu_mul(gu.data_ptr(), want.data_ptr(), M, I, dtype_tag(dtype), s), "silu_mul")
    check(L.ssa_linear_swiglu(x.data_ptr(), W.data_ptr(), got.data_ptr(), M, I, K, dtype_tag(dtype), s), "swiglu")
    assert torch.equal(got, want)
    ref = torch.nn.functional.silu(gu[:, :I].float()).to(dtype).float() * gu[:, I:].float()
    torch.testing.assert_close(got.float(), ref, rtol=1e-2, atol=1e-2)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_embed_rmsnorm_equals_embedding_then_rmsnorm(dtype):
    check, dtype_tag, L, s = _lib()
    g = torch.Generator(device="cuda").manual_seed(9)
    V, D, B = 500, 1024, 3
    emb = torch.randn(V, D, device="cuda", generator=g).to(dtype)
    w = (1 + 0.1 * torch.randn(D, device="cuda", generator=g)).to(dtype)
    tok = torch.tensor([[7], [499], [0]], device="cuda", dtype=torch.long)
    pos = torch.tensor([41], device="cuda", dtype=torch.long)
    n = torch.zeros(1, device="cuda", dtype=torch.int32)
    h, x = torch.empty(B, D, device="cuda", dtype=dtype), torch.empty(B, D, device="cuda", dtype=dtype)
    check(L.ssa_embed_rmsnorm(tok.data_ptr(), emb.data_ptr(), h.data_ptr(), w.data_ptr(), x.data_ptr(), B, D, V, 1e-6,
                              pos.data_ptr(), n.data_ptr(), dtype_tag(dtype), s), "embed_rmsnorm")
    h2 = emb[tok.view(-1)].clone()
    x2 = torch.empty_like(x)
    check(L.ssa_rmsnorm_add(h2.data_ptr(), None, w.data_ptr(), x2.data_ptr(), B, D, 1e-6, dtype_tag(dtype), s),
          "rmsnorm_add")
    assert torch.equal(h, h2) and torch.equal(x, x2) and int(n) == 42


@pytest.mark.parametrize("N", [151936, 1001, 8])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_argmax_rows_is_torch_argmax(N, dtype):
    """First index of the maximum, with planted ties (the earlier copy wins) and a NaN row."""
    check, dtype_tag, L, s = _lib()
    g = torch.Generator(device="cuda").manual_seed(N)
    x = torch.randn(4, N, device="cuda", generator=g).to(dtype)
    x[1, N // 3] = 50.0
    x[1, N - 1] = 50.0                                  # a tie: the first copy wins
    x[2] = 1.0                                          # all equal: index 0
    x[3, N // 2] = float("nan")
    x[3, N // 4] = 60.0
    x[0, 5] = -0.0 if N > 8 else x[0, 5]
    work = torch.zeros(8, device="cuda", dtype=torch.long)
    for _ in range(2):                                  # the work buffer is left zero for the next call
        out = torch.full((4,), -1, device="cuda", dtype=torch.long)
        check(L.ssa_argmax_rows(x.data_ptr(), out.data_ptr(), 4, N, dtype_tag(dtype), work.data_ptr(), s), "argmax")
        assert torch.equal(out, x.argmax(-1)), (out, x.argmax(-1))
        assert not work.any()
    z = torch.zeros(1, N, device="cuda", dtype=dtype)
    z[0, 3] = -0.0                                      # -0 and +0 are equal: the first index wins
    check(L.ssa_argmax_rows(z.data_ptr(), out.data_ptr(), 1, N, dtype_tag(dtype), work.data_ptr(), s), "argmax")
    assert int(out[0]) == 0


@pytest.mark.parametrize("M,N,K", [(1, 6144, 2560), (2, 1024, 1024), (3, 333, 264), (8, 4096, 2048)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_norm_and_residual_inside_the_projections_keep_the_bits(M, N, K, dtype):
    """ssa_rmsnorm_linear_skinny / ssa_rmsnorm_linear_swiglu (the RMSNorm computed in the
    projection's prologue) and ssa_linear_skinny_res (the residual add in its epilogue) against
    the launches they replace, ssa_rmsnorm_add then ssa_linear_skinny / ssa_linear_swiglu, and
    ssa_linear_skinny then ssa_rmsnorm_add's add: the same bits."""
    check, dtype_tag, L, s = _lib()
    dt = dtype_tag(dtype)
    g = torch.Generator(device="cuda").manual_seed(M * 13 + N)
    h = (torch.randn(M, K, device="cuda", generator=g) * 3).to(dtype)
    nw = (1 + 0.1 * torch.randn(K, device="cuda", generator=g)).to(dtype)
    W = (torch.randn(N, K, device="cuda", generator=g) * 0.05).to(dtype)
    Wg = (torch.randn(2 * N, K, device="cuda", generator=g) * 0.05).to(dtype)
    # rmsnorm + projection
    x = torch.empty_like(h)
    check(L.ssa_rmsnorm_add(h.data_ptr(), None, nw.data_ptr(), x.data_ptr(), M, K, 1e-6, dt, s), "rmsnorm_add")
    want = torch.empty(M, N, device="cuda", dtype=dtype)
    check(L.ssa_linear_skinny(x.data_ptr(), W.data_ptr(), want.data_ptr(), M, N, K, dt, s), "skinny")
    got = torch.full((M, N), float("nan"), device="cuda", dtype=dtype)
    check(L.ssa_rmsnorm_linear_skinny(h.data_ptr(), nw.data_ptr(), 1e-6, W.data_ptr(), got.data_ptr(), M, N, K, dt, s),
          "rmsnorm_linear_skinny")
    assert torch.equal(got, want)
    # rmsnorm + gate/up + SwiGLU
    want = torch.empty(M, N, device="cuda", dtype=dtype)
    check(L.ssa_linear_swiglu(x.data_ptr(), Wg.data_ptr(), want.data_ptr(), M, N, K, dt, s), "swiglu")
    got = torch.full((M, N), float("nan"), device="cuda", dtype=dtype)
    check(L.ssa_rmsnorm_linear_swiglu(h.data_ptr(), nw.data_ptr(), 1e-6, Wg.data_ptr(), got.data_ptr(), M, N, K, dt, s),
          "rmsnorm_linear_swiglu")
    assert torch.equal(got, want)
    # projection + residual add: h2 [M, N] += x W^T
    h2 = (torch.randn(M, N, device="cuda", generator=g) * 3).to(dtype)
    want_h = h2.clone()
    y = torch.empty(M, N, device="cuda", dtype=dtype)
    check(L.ssa_linear_skinny(x.data_ptr(), W.data_ptr(), y.data_ptr(), M, N, K, dt, s), "skinny")
    scratch = torch.empty_like(want_h)
    check(L.ssa_rmsnorm_add(want_h.data_ptr(), y.data_ptr(), torch.ones(N, device="cuda", dtype=dtype).data_ptr(),
                            scratch.data_ptr(), M, N, 1e-6, dt, s), "rmsnorm_add")
    check(L.ssa_linear_skinny_res(x.data_ptr(), W.data_ptr(), h2.data_ptr(), M, N, K, dt, s), "skinny_res")
    assert torch.equal(h2, want_h)
