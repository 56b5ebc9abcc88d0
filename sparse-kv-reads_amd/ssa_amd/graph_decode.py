"""Whole decode step captured in one hipGraph (mirrors src/ssa/models/graph_decode.py:29-157).

``GraphDecoder`` reruns the model's single-token forward layer by layer with the model's own
modules, weights and KV cache, but with the position held in device memory: the rotary angles
are gathered at that position, the new key and value are written with ``index_copy_``, and
attention reads the current length from device memory (``DenseAttentionGraph`` or
``SphereIndexGraph``). Nothing in the step depends on a host number that changes between
tokens, so it is captured once and replayed with a single graph launch per token.

Batching: the cache ``[B, H_kv, L, d]`` is viewed as ``[B·H_kv, L, d]`` and the queries
``[B, H, d]`` as ``[B·H, d]`` (every (sequence, KV head) is independent), without copying.

Insertion: with insert-ahead each layer's step launch bins its next key. It is used while the
step's extra stager workgroups (one per head) fit beside the splits, or when asked for with
``insert_ahead=True``; otherwise one ``AllLayerInsert`` launch bins every layer's key at the start
of the step, as the reference's ``fused_insert`` does.

Glue: with ``glue="fused"`` (the default) a layer is five launches besides the attention step:
``ssa_rmsnorm_linear_skinny`` (the input RMSNorm and the q/k/v projection),
``ssa_qk_norm_rope_cache`` (q/k RMSNorm, rotary embedding, KV-cache write),
``ssa_linear_skinny_res`` (the o projection added into the residual stream),
``ssa_rmsnorm_linear_swiglu`` (the post-attention RMSNorm, the gate/up projection and SwiGLU)
and ``ssa_linear_skinny_res`` (the down projection); the projections are weight-streaming
kernels for the decode batch, the step opens with ``ssa_embed_rmsnorm``, the final RMSNorm rides
in the LM head's projection and, with ``greedy``, ``ssa_argmax_rows`` ends the step. Where those
kernels do not apply (batch above 8, fp32 weights, widths not a multiple of 8) the norms and adds
run as ``ssa_rmsnorm_add`` and the projections as ``ssa_linear_skinny`` / ``ssa_linear_swiglu``.
``glue="split"`` runs every op as its own launch (the same bits), and ``glue="torch"`` the ~60
element-wise launches of the model's own modules per layer, as the reference's ``_body`` runs
them. At batch 1-2 every dependent launch costs a few microseconds whatever its size, so the
launch count is what the glue is designed around.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from ._lib import check, dtype_tag, lib, stream_ptr
from .graph_kernels import STACKED, AllLayerInsert, DenseAttentionGraph, SphereIndexGraph
from .qwen3 import apply_rope

MODES = ("dense", "cluster")


class GraphDecoder:
    def __init__(self, model, cache, *, mode: str = "dense", budget: float = 0.2, C: int | None = None,
                 window: int = 64, delta: float = 0.03, check_every: int = 16, partition: str = "kmeans",
                 C_init: int | None = None, split_factor: float | None = None, refit_every: int = 0,
                 grow_cap: bool = False, reset_at: int = 0, summary_bits: int = 8, cap_keys: float = 0.0,
                 fused_insert: bool = True, var_factor: float = 0.0, var_min: int = 8,
                 insert_ahead: bool | None = None, glue: str = "fused", greedy: bool = False, **_):
        cfg = model.cfg
        # with no slot count given: 1,024 slots, 256 clusters fitted at the prompt, splitting of
        # clusters over twice the mean size at the fit (src/ssa/models/graph_decode.py:35-43)
        if C is None:
            C = 1024 if partition == "kmeans" else 256
            if partition == "kmeans":
                C_init = 256 if C_init is None else C_init
                split_factor = 2.0 if split_factor is None else split_factor
        split_factor = 0.0 if split_factor is None else split_factor
        mode = "cluster" if mode in ("sphere", "voronoi") else mode       # old names
        if mode not in MODES:
            raise ValueError(f"unknown mode {mode!r}")
        self.model, self.cache, self.mode = model, cache, mode
        self.H, self.H_kv, self.d = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
        self.B = B = cache.k[0].shape[0]
        p = next(model.parameters())
        dev, dtype = p.device, p.dtype
        if cache.max_seq_len > model.rope_cos.shape[0]:
            raise ValueError("the cache is longer than the model's rotary tables")
        self.tok = torch.zeros(B, 1, dtype=torch.long, device=dev)
        self.pos = torch.zeros(1, dtype=torch.long, device=dev)
        self.n_dev = torch.zeros(1, dtype=torch.int32, device=dev)
        cap = cache.max_seq_len
        if mode == "dense":
            self.attn = [DenseAttentionGraph(H=B * self.H, H_kv=B * self.H_kv, d=self.d, dtype=dtype, device=dev)
                         for _ in model.layers]
        else:
            self.attn = [SphereIndexGraph(budget=budget, C=C, window=window, delta=delta, capacity=cap,
                                          check_every=check_every, partition=partition, C_init=C_init,
                                          split_factor=split_factor, refit_every=refit_every, grow_cap=grow_cap,
                                          reset_at=reset_at, summary_bits=summary_bits, cap_keys=cap_keys,
                                          var_factor=var_factor, var_min=var_min, insert_ahead=insert_ahead)
                         for _ in model.layers]
        self.graph = None
        self.logits = None
        self._probe = None
        self.greedy = greedy
        self.next_tok = torch.zeros(B, 1, dtype=torch.long, device=dev)   # with greedy: argmax of the logits
        self._argmax_work = torch.zeros(2 * B, dtype=torch.long, device=dev)  # ssa_argmax_rows' key + count
        self.fused_insert = fused_insert and mode == "cluster" and window >= 1
        self._ahead_forced = insert_ahead is True   # else every layer's keys in one launch past the stagers
        self.insert_all = None
        if glue not in ("fused", "split", "torch"):
            raise ValueError(f"unknown glue {glue!r}")
        self.glue = glue
        # "fused" folds SwiGLU into the gate/up projection where the kernel allows it (2-byte
        # weights, batch <= 8), and the residual adds and RMSNorms into the projections either
        # side of them (the add into the o and down projections' epilogues, each norm into the
        # next projection's prologue), which leaves five launches per layer besides the attention;
        # "split" runs every op as its own launch. Both give the same bits.
        self._merge_gu = (glue == "fused" and dtype in (torch.bfloat16, torch.float16) and B <= 8
                          and cfg.hidden_size % 8 == 0)
        self._fuse_norm = self._merge_gu and cfg.intermediate_size % 8 == 0 and (self.H * self.d) % 8 == 0
        if glue != "torch":
            with torch.no_grad():
                self._wqkv = [torch.cat((l.attn.q.weight, l.attn.k.weight, l.attn.v.weight)) for l in model.layers]
                self._wgu = [torch.cat((l.ffn.gate.weight, l.ffn.up.weight)) for l in model.layers]
            self._h = torch.empty(B, cfg.hidden_size, device=dev, dtype=dtype)     # the residual stream
            if self._fuse_norm:            # the projections' outputs, reused by every layer and step
                head = model.embed.weight if model.lm_head is None else model.lm_head.weight
                self._qkv = torch.empty(B, self._wqkv[0].shape[0], device=dev, dtype=dtype)
                self._logits = torch.empty(B, head.shape[0], device=dev, dtype=dtype)
            self._x = torch.empty(B, cfg.hidden_size, device=dev, dtype=dtype)
            self._qh = torch.empty(B * self.H, self.d, device=dev, dtype=dtype)
            self._act = torch.empty(B, cfg.intermediate_size, device=dev, dtype=dtype)
            self._dt = dtype_tag(dtype)
            self._eps = float(cfg.rms_norm_eps)

    def _heads(self, c: torch.Tensor) -> torch.Tensor:
        """Cache ``[B, H_kv, L, d]`` -> ``[B·H_kv, L, d]`` (a view)."""
        return c.view(-1, c.shape[2], c.shape[3])

    def prepare(self, n: int) -> None:
        """Build the attention state from the first ``n`` cached positions (after the prompt)."""
        if self.mode != "cluster":
            return
        for i, idx in enumerate(self.attn):
            idx.prepare(self._heads(self.cache.k[i]), n, self.B * self.H)
        if self.fused_insert and not all(idx.insert_ahead and (idx.extra_stagers_fit() or self._ahead_forced)
                                         for idx in self.attn):
            for idx in self.attn:                       # one insertion launch for every layer
                idx.insert_ahead = False
            self.insert_all = AllLayerInsert(self.attn, [self._heads(k) for k in self.cache.k[:len(self.attn)]])

    def _attend(self, i, qh, kc, vc):
        if self.mode == "dense":
            return self.attn[i](qh, self._heads(kc), self._heads(vc), self.n_dev)
        out = self.attn[i].step(qh, self._heads(kc), self._heads(vc), self.n_dev, insert=self.insert_all is None)
        if self._probe is not None:                   # the exact output of the same query, for the error
            from .labeled_attn import dense_attention
            want = dense_attention(qh, self._heads(kc), self._heads(vc), n_dev=self.n_dev).float()
            self._probe.append(((out.float() - want).norm() / want.norm().clamp_min(1e-30)).reshape(1))
        return out

    def _linear(self, x: torch.Tensor, W: torch.Tensor) -> torch.Tensor:
        """``x W^T`` for the decode batch: the weight-streaming HIP kernel for 2-byte weights and
        up to 8 rows, the library GEMM otherwise."""
        M, K = x.shape
        if M > 8 or W.dtype not in (torch.bfloat16, torch.float16) or K % 8:
            return F.linear(x, W)
        y = torch.empty(M, W.shape[0], device=x.device, dtype=x.dtype)
        check(lib().ssa_linear_skinny(x.data_ptr(), W.data_ptr(), y.data_ptr(), M, W.shape[0], K, self._dt,
                                      stream_ptr(x.device)), "ssa_linear_skinny")
        return y

    def _body_fused(self) -> torch.Tensor:
        m, H, H_kv, d, B = self.model, self.H, self.H_kv, self.d, self.B
        L, s, x, h, eps, dt = len(m.layers), stream_ptr(self.tok.device), self._x, self._h, self._eps, self._dt
        act, I, D = self._act, self._act.shape[1], h.shape[1]
        # h = embedding of the tokens, x = norm1(h), n_dev = pos + 1
        check(lib().ssa_embed_rmsnorm(self.tok.data_ptr(), m.embed.weight.data_ptr(), h.data_ptr(),
                                      m.layers[0].norm1.weight.data_ptr(), x.data_ptr(), B, D, m.embed.weight.shape[0],
                                      eps, self.pos.data_ptr(), self.n_dev.data_ptr(), dt, s), "ssa_embed_rmsnorm")
        if self.insert_all is not None:
            self.insert_all(self.n_dev)
        if self._fuse_norm:
            return self._body_fused_norm()
        for i, layer in enumerate(m.layers):
            a, f = layer.attn, layer.ffn
            kc, vc = self.cache.k[i], self.cache.v[i]
            rope = (a.q_norm.weight.data_ptr(), a.k_norm.weight.data_ptr(), m.rope_cos.data_ptr(),
                    m.rope_sin.data_ptr(), self.pos.data_ptr(), self._qh.data_ptr(), kc.data_ptr(), vc.data_ptr(),
                    kc.stride(0), kc.stride(1), kc.stride(2), B, H, H_kv, d)
            qkv = self._linear(x, self._wqkv[i])
            check(lib().ssa_qk_norm_rope_cache(qkv.data_ptr(), *rope, eps, dt, s), "ssa_qk_norm_rope_cache")
            out = self._attend(i, self._qh, kc, vc)
            o = self._linear(out.view(B, H * d), a.o.weight)
            check(lib().ssa_rmsnorm_add(h.data_ptr(), o.data_ptr(), layer.norm2.weight.data_ptr(), x.data_ptr(), B, D,
                                        eps, dt, s), "ssa_rmsnorm_add")
            if self._merge_gu:
                check(lib().ssa_linear_swiglu(x.data_ptr(), self._wgu[i].data_ptr(), act.data_ptr(), B, I, D, dt, s),
                      "ssa_linear_swiglu")
            else:
                gu = self._linear(x, self._wgu[i])
                check(lib().ssa_silu_mul(gu.data_ptr(), act.data_ptr(), B, I, dt, s), "ssa_silu_mul")
            dn = self._linear(act, f.down.weight)
            nw = m.layers[i + 1].norm1.weight if i + 1 < L else m.final_norm.weight
            check(lib().ssa_rmsnorm_add(h.data_ptr(), dn.data_ptr(), nw.data_ptr(), x.data_ptr(), B, D, eps, dt, s),
                  "ssa_rmsnorm_add")
        head = m.embed.weight if m.lm_head is None else m.lm_head.weight
        logits = self._linear(x, head)
        if self.greedy:
            check(lib().ssa_argmax_rows(logits.data_ptr(), self.next_tok.data_ptr(), B, logits.shape[1], dt,
                                        self._argmax_work.data_ptr(), s), "ssa_argmax_rows")
        return logits.view(B, 1, -1)

    def _body_fused_norm(self) -> torch.Tensor:
        """The layers after the embedding with the residual adds and RMSNorms inside the
        projections: per layer rmsnorm + qkv, q/k norm + rotary + cache write, attention,
        o projection + residual add, rmsnorm + gate/up + SwiGLU, down projection + residual add."""
        m, H, H_kv, d, B = self.model, self.H, self.H_kv, self.d, self.B
        s, h, eps, dt = stream_ptr(self.tok.device), self._h, self._eps, self._dt
        act, I, D = self._act, self._act.shape[1], h.shape[1]
        L = lib()
        for i, layer in enumerate(m.layers):
            a, f = layer.attn, layer.ffn
            kc, vc = self.cache.k[i], self.cache.v[i]
            qkv = self._qkv
            check(L.ssa_rmsnorm_linear_skinny(h.data_ptr(), layer.norm1.weight.data_ptr(), eps, self._wqkv[i].data_ptr(),
                                              qkv.data_ptr(), B, qkv.shape[1], D, dt, s), "ssa_rmsnorm_linear_skinny")
            check(L.ssa_qk_norm_rope_cache(qkv.data_ptr(), a.q_norm.weight.data_ptr(), a.k_norm.weight.data_ptr(),
                                           m.rope_cos.data_ptr(), m.rope_sin.data_ptr(), self.pos.data_ptr(),
                                           self._qh.data_ptr(), kc.data_ptr(), vc.data_ptr(), kc.stride(0),
                                           kc.stride(1), kc.stride(2), B, H, H_kv, d, eps, dt, s), "ssa_qk_norm_rope_cache")
            out = self._attend(i, self._qh, kc, vc)
            check(L.ssa_linear_skinny_res(out.data_ptr(), a.o.weight.data_ptr(), h.data_ptr(), B, D, H * d, dt, s),
                  "ssa_linear_skinny_res")
            check(L.ssa_rmsnorm_linear_swiglu(h.data_ptr(), layer.norm2.weight.data_ptr(), eps, self._wgu[i].data_ptr(),
                                              act.data_ptr(), B, I, D, dt, s), "ssa_rmsnorm_linear_swiglu")
            check(L.ssa_linear_skinny_res(act.data_ptr(), f.down.weight.data_ptr(), h.data_ptr(), B, D, I, dt, s),
                  "ssa_linear_skinny_res")
        head = m.embed.weight if m.lm_head is None else m.lm_head.weight
        logits = self._logits
        check(L.ssa_rmsnorm_linear_skinny(h.data_ptr(), m.final_norm.weight.data_ptr(), eps, head.data_ptr(),
                                          logits.data_ptr(), B, head.shape[0], D, dt, s), "ssa_rmsnorm_linear_skinny")
        if self.greedy:
            check(L.ssa_argmax_rows(logits.data_ptr(), self.next_tok.data_ptr(), B, logits.shape[1], dt,
                                    self._argmax_work.data_ptr(), s), "ssa_argmax_rows")
        return logits.view(B, 1, -1)

    def _body(self) -> torch.Tensor:
        if self.glue != "torch":
            return self._body_fused()
        m, H, H_kv, d, B = self.model, self.H, self.H_kv, self.d, self.B
        self.n_dev.copy_(self.pos + 1)
        if self.insert_all is not None:
            self.insert_all(self.n_dev)
        h = m.embed(self.tok)                                              # [B, 1, hidden]
        cos = m.rope_cos.index_select(0, self.pos)
        sin = m.rope_sin.index_select(0, self.pos)
        for i, layer in enumerate(m.layers):
            a = layer.attn
            x = layer.norm1(h)
            q = a.q_norm(a.q(x).view(B, 1, H, d)).transpose(1, 2)
            k = a.k_norm(a.k(x).view(B, 1, H_kv, d)).transpose(1, 2)
            v = a.v(x).view(B, 1, H_kv, d).transpose(1, 2)
            q, k = apply_rope(q, k, cos, sin)
            kc, vc = self.cache.k[i], self.cache.v[i]
            kc.index_copy_(2, self.pos, k)
            vc.index_copy_(2, self.pos, v)
            qh = q[:, :, 0, :].reshape(B * H, d)
            out = self._attend(i, qh, kc, vc)
            h = h + a.o(out.reshape(B, 1, H * d))
            h = h + layer.ffn(layer.norm2(h))
        logits = m.logits(h)
        if self.greedy:
            self.next_tok.copy_(logits[:, -1].argmax(-1, keepdim=True))
        return logits

    def _snapshot(self):
        """Copies of every index state tensor (the capture's warm-up runs execute real steps)."""
        if self.mode != "cluster":
            return None
        return [{f: getattr(idx, f).clone() for f in STACKED if isinstance(getattr(idx, f, None), torch.Tensor)}
                for idx in self.attn]

    def _restore(self, snap) -> None:
        if snap is None:
            return
        for idx, st in zip(self.attn, snap):
            for f, t in st.items():
                getattr(idx, f).copy_(t)

    def capture(self) -> None:
        """Record one decode step. Call after ``prepare`` and before the first ``step``. The
        warm-up runs write a placeholder key at the current position (the first real step
        overwrites it) and their index updates are undone."""
        self.pos.fill_(self.cache.cur_len)
        snap = self._snapshot()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for _ in range(2):
                self._body()
        torch.cuda.current_stream().wait_stream(s)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self._glogits = self._body()
        self.logits = self._glogits
        self.graph = g
        self._restore(snap)
        torch.cuda.synchronize()

    def step(self, token: torch.Tensor, pos: int, probe: list | None = None) -> torch.Tensor:
        """Decode ``token [B, 1]`` at position ``pos``; returns logits ``[B, 1, vocab]`` (a buffer
        the next step overwrites). With ``probe`` (cluster mode) the step runs eagerly, with the
        same kernels as the graph, and appends for every layer the relative error
        ``|out - dense| / |dense|`` of its attention output against exact attention on the same
        query and cache (a one-element tensor per layer)."""
        if not 0 <= pos < self.cache.max_seq_len:
            raise ValueError("the cache is full")
        self.tok.copy_(token)
        self.pos.fill_(pos)
        if probe is not None and self.mode == "cluster":
            self._probe = probe
            try:
                self.logits = self._body()
            finally:
                self._probe = None
        elif self.graph is not None:
            self.graph.replay()
            self.logits = self._glogits
        else:
            self.logits = self._body()
        if self.mode == "cluster":
            for i, idx in enumerate(self.attn):
                idx.after_replay(self._heads(self.cache.k[i]))
        self.cache.cur_len = pos + 1
        return self.logits
