"""The reference's per-shader inference graphs, driven through the C ABI.

A restatement of what akasha-core's emitters do when the backend is HIP:
``ShaderDecoder`` mirrors DecodeScratch + build_decode_layer +
InferenceSession::decode_step (src/nn/inference_graphs.rs:13-196, 339-509;
src/nn/inference.rs:178-262): the graph is captured once, with constant and
dynamic metas in device memory, and replayed every step after the four
dynamic metas are rewritten.  ``shader_prefill`` and ``ShaderDecoder.prefill``
mirror build_prefill_layer (inference_graphs.rs:198-337) +
InferenceSession::prefill (inference.rs:61-176).  Every node is one launcher
of include/akasha_hip.h with buffers in binding-slot order.
"""

import numpy as np


class ShaderDecoder:
    """With capture=False every decode step issues the same launchers
    eagerly instead of replaying the captured graph (for tools that cannot
    follow graph launches, such as kernel tracers)."""

    def __init__(self, hip, backend, cfg, weights, max_ctx, capture=True):
        self.hip, self.be, self.cfg, self.max_ctx = hip, backend, cfg, max_ctx
        self.capture = capture
        be, d, hd, H, F, V = backend, cfg.dim, cfg.head_dim, cfg.num_heads, cfg.ffn_hidden, cfg.vocab_size
        self.w = [be.tensor(np.ascontiguousarray(a, np.float32)) for a in weights]
        z = lambda n: be.zeros(n)  # noqa: E731
        self.hidden, self.norm_out, self.qkv_out = z(d), z(d), z(3 * d)
        self.q_buf, self.k_buf, self.v_buf = z(d), z(d), z(d)
        self.scores, self.attn_out, self.ffn_up_out = z(H * max_ctx), z(d), z(F)
        self.final_norm_out, self.logits = z(d), z(V)
        self.token = be.zeros(1, np.uint32)
        self.k_cache = [z(max_ctx * d) for _ in range(cfg.num_layers)]
        self.v_cache = [z(max_ctx * d) for _ in range(cfg.num_layers)]
        # Constant metas (DecodeScratch::new, inference_graphs.rs:56-100).
        self.norm_shape = hip.NormMeta(1, d, cfg.norm_eps)
        self.norm_meta = be.meta(self.norm_shape)
        self.qkv_meta = be.meta(hip.MatMulMeta(1, d, d))
        self.qkv_proj_meta = be.meta(hip.MatMulMeta(1, 3 * d, d))
        self.split_shapes = [hip.HeadMoveMeta(1, 3 * d, d, i * d) for i in range(3)]
        self.split_meta = [be.meta(s) for s in self.split_shapes]
        self.ffnup_meta = be.meta(hip.MatMulMeta(1, F, d))
        self.ffndown_meta = be.meta(hip.MatMulMeta(1, d, F))
        self.emb_shape = hip.EmbeddingMeta(V, d, 1)
        self.emb_meta = be.meta(self.emb_shape)
        self.lm_meta = be.meta(hip.MatMulMeta(1, V, d))
        # Dynamic metas (inference_graphs.rs:102-126).
        self.rope_meta = be.meta(hip.RopeOffsetMeta(1, d, hd, 0))
        self.cw_meta = be.meta(hip.CacheWriteMeta(1, d, 0))
        self.attn_meta = be.meta(hip.AttnCachedMeta(1, d, hd))
        self.sm_meta = be.meta(hip.SoftmaxRectMeta(H, 1, 1.0))
        self.graph = None
        self.cur_len = 0

    def _param(self, i):
        return self.w[i]

    def _build(self):
        self.be.graph_begin()
        self._nodes()
        self.graph = self.be.graph_end()

    def _nodes(self):
        hip, be, c = self.hip, self.be, self.cfg
        d, hd, H, F, V = c.dim, c.head_dim, c.num_heads, c.ffn_hidden, c.vocab_size
        be.embedding(self.token, self._param(0), self.hidden, self.emb_shape, self.emb_meta)
        for l in range(c.num_layers):
            n1, qkv, wo, n2, up, down = (self._param(1 + 6 * l + j) for j in range(6))
            be.rmsnorm(self.hidden, n1, self.norm_out, self.norm_shape, self.norm_meta)
            be.matmul(self.norm_out, qkv, self.qkv_out, hip.MatMulMeta(1, 3 * d, d),
                      self.qkv_proj_meta)
            for i, dst in enumerate((self.q_buf, self.k_buf, self.v_buf)):
                be.head_gather(self.qkv_out, dst, self.split_shapes[i], self.split_meta[i])
            rs = hip.RopeOffsetMeta(1, d, hd, 0)
            be.rope_offset(self.q_buf, rs, self.rope_meta)
            be.rope_offset(self.k_buf, rs, self.rope_meta)
            cs = hip.CacheWriteMeta(1, d, 0)
            be.cache_write(self.k_buf, self.k_cache[l], cs, self.cw_meta)
            be.cache_write(self.v_buf, self.v_cache[l], cs, self.cw_meta)
            be.attn_qk_cached(self.q_buf, self.k_cache[l], self.scores, H, self.max_ctx,
                              self.attn_meta)
            be.softmax_rect(self.scores, hip.SoftmaxRectMeta(H, self.max_ctx, 1.0 / np.sqrt(hd)),
                            self.sm_meta)
            be.attn_av_cached(self.scores, self.v_cache[l], self.attn_out, d, self.attn_meta)
            be.matmul_add(self.attn_out, wo, self.hidden, hip.MatMulMeta(1, d, d), self.qkv_meta)
            be.rmsnorm(self.hidden, n2, self.norm_out, self.norm_shape, self.norm_meta)
            be.matmul(self.norm_out, up, self.ffn_up_out, hip.MatMulMeta(1, F, d), self.ffnup_meta)
            be.silu(self.ffn_up_out, F)
            be.matmul_add(self.ffn_up_out, down, self.hidden, hip.MatMulMeta(1, d, F),
                          self.ffndown_meta)
        L = c.num_layers
        be.rmsnorm(self.hidden, self._param(1 + 6 * L), self.final_norm_out, self.norm_shape,
                   self.norm_meta)
        be.matmul(self.final_norm_out, self._param(2 + 6 * L), self.logits,
                  hip.MatMulMeta(1, V, d), self.lm_meta)

    def close(self):
        """Release the graph and every device buffer this decoder holds."""
        if self.graph is not None:
            self.graph.close()
            self.graph = None
        for v in list(vars(self).values()):
            for t in v if isinstance(v, list) else [v]:
                if isinstance(t, self.hip.DeviceTensor):
                    t.free()

    def prefill(self, tokens):
        """InferenceSession::prefill into this decoder's caches (inference.rs:
        61-176, which generate runs on an empty cache, inference.rs:288-289):
        the prompt's rows through the per-shader prefill graph; returns the
        last row's logits, and decode steps continue at position len(tokens)."""
        assert self.cur_len == 0 and 0 < len(tokens) <= self.max_ctx
        logits = _prefill_nodes(self.hip, self.be, self.cfg, self.w, tokens,
                                self.k_cache, self.v_cache)
        out = logits.download()
        self.cur_len = len(tokens)
        return out

    def reset(self):
        """An empty cache again (cur_len = 0): the next prefill rewrites its
        rows."""
        self.cur_len = 0

    def decode_step(self, token):
        hip, be, c = self.hip, self.be, self.cfg
        pos = self.cur_len
        assert pos < self.max_ctx
        hd = c.head_dim
        self.token.upload(np.array([token], np.uint32))
        # DecodeScratch::update_for_step (inference_graphs.rs:164-195).
        be.write_meta(self.rope_meta, hip.RopeOffsetMeta(1, c.dim, hd, pos))
        be.write_meta(self.cw_meta, hip.CacheWriteMeta(1, c.dim, pos))
        be.write_meta(self.attn_meta, hip.AttnCachedMeta(pos + 1, c.dim, hd))
        be.write_meta(self.sm_meta, hip.SoftmaxRectMeta(c.num_heads, pos + 1,
                                                        np.float32(1.0) / np.sqrt(np.float32(hd))))
        if not self.capture:
            self._nodes()
        else:
            if self.graph is None:
                self._build()
            self.graph.execute()
        self.cur_len = pos + 1
        return self.logits.download()


def _prefill_nodes(hip, be, cfg, w, tokens, kc, vc):
    """The nodes of InferenceSession::prefill (inference.rs:61-176): the
    embedding, build_prefill_layer per layer (inference_graphs.rs:198-337)
    writing rows 0..S-1 of the caches kc / vc, then the last row's head
    gather, final norm and lm_head.  Every intermediate tensor and meta is
    allocated as the graph is built, as the reference's builder does; the
    nodes run as they are issued (the reference executes its prefill graph
    once).  The graph's tensors live until every node is queued (freeing
    one waits for the stream).  Returns the logits tensor."""
    d, hd, F, V, L = cfg.dim, cfg.head_dim, cfg.ffn_hidden, cfg.vocab_size, cfg.num_layers
    S = len(tokens)
    held = []

    def keep(t):
        held.append(t)
        return t

    tok = keep(be.tensor(np.asarray(tokens, np.uint32)))
    hidden = keep(be.zeros(S * d))
    emb = hip.EmbeddingMeta(V, d, S)
    be.embedding(tok, w[0], hidden, emb, keep(be.meta(emb)))
    ns = hip.NormMeta(S, d, cfg.norm_eps)
    for l in range(L):
        n1, qkv, wo, n2, up, down = (w[1 + 6 * l + j] for j in range(6))
        norm1 = keep(be.zeros(S * d))
        be.rmsnorm(hidden, n1, norm1, ns, keep(be.meta(ns)))
        qkv_out = keep(be.zeros(S * 3 * d))
        mm = hip.MatMulMeta(S, 3 * d, d)
        be.matmul(norm1, qkv, qkv_out, mm, keep(be.meta(mm)))
        q, k, v = keep(be.zeros(S * d)), keep(be.zeros(S * d)), keep(be.zeros(S * d))
        for buf, off in ((q, 0), (k, d), (v, 2 * d)):
            hm = hip.HeadMoveMeta(S, 3 * d, d, off)
            be.head_gather(qkv_out, buf, hm, keep(be.meta(hm)))
        rm = hip.RopeMeta(S, d, hd, 0)
        be.rope(q, rm, keep(be.meta(rm)))
        be.rope(k, rm, keep(be.meta(rm)))
        cw = hip.CacheWriteMeta(S, d, 0)
        be.cache_write(k, kc[l], cw, keep(be.meta(cw)))
        be.cache_write(v, vc[l], cw, keep(be.meta(cw)))
        attn = keep(be.zeros(S * d))
        lse = keep(be.zeros(S * cfg.num_heads))
        fm = hip.FlashAttnMeta(S, d, hd, np.float32(1.0) / np.sqrt(np.float32(hd)), 0)
        be.flash_attention(q, k, v, attn, lse, fm, keep(be.meta(fm)))
        mo = hip.MatMulMeta(S, d, d)
        be.matmul_add(attn, wo, hidden, mo, keep(be.meta(mo)))
        norm2 = keep(be.zeros(S * d))
        be.rmsnorm(hidden, n2, norm2, ns, keep(be.meta(ns)))
        ffn = keep(be.zeros(S * F))
        mu = hip.MatMulMeta(S, F, d)
        be.matmul(norm2, up, ffn, mu, keep(be.meta(mu)))
        be.silu(ffn, S * F)
        md = hip.MatMulMeta(S, d, F)
        be.matmul_add(ffn, down, hidden, md, keep(be.meta(md)))
    last = keep(be.zeros(d))
    hm = hip.HeadMoveMeta(1, d, d, (S - 1) * d)
    be.head_gather(hidden, last, hm, keep(be.meta(hm)))
    fo = keep(be.zeros(d))
    n1m = hip.NormMeta(1, d, cfg.norm_eps)
    be.rmsnorm(last, w[1 + 6 * L], fo, n1m, keep(be.meta(n1m)))
    logits = keep(be.zeros(V))
    lm = hip.MatMulMeta(1, V, d)
    be.matmul(fo, w[2 + 6 * L], logits, lm, keep(be.meta(lm)))
    return logits


def shader_prefill(hip, be, cfg, weights, tokens, max_ctx):
    """One sequence through the per-shader prefill graph; returns last-row
    logits and the per-layer K caches."""
    d, L = cfg.dim, cfg.num_layers
    w = [be.tensor(np.ascontiguousarray(a, np.float32)) for a in weights]
    kc = [be.zeros(max_ctx * d) for _ in range(L)]
    vc = [be.zeros(max_ctx * d) for _ in range(L)]
    logits = _prefill_nodes(hip, be, cfg, w, tokens, kc, vc)
    be.synchronize()
    return logits.download(), [t.download().reshape(max_ctx, d) for t in kc]
