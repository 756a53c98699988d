"""The optional bf16-MFMA prefill (akh_model_set_prefill_bf16) against the CPU
oracle's f32 prefill (inference.rs:61-176).

Parity bar for this path: logits within max-abs 2e-2 of the f32 oracle, and
the same greedy token wherever the oracle's top-two margin exceeds twice that.
Decoding after a bf16 prefill runs the f32 decode on the bf16-prefilled cache
and is held to the same bar.  Weights are bf16-valued (as the scaled
configuration's are), so the bf16 copies of the weights are exact and the
difference comes from rounding activations only.
"""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

TOL = 2e-2


def _check_logits(got, ref, ora, where):
    assert np.abs(got - ref).max() < TOL, where
    top = np.sort(ref)[-2:]
    if top[1] - top[0] > 2 * TOL:
        assert int(np.argmax(got)) == ora.argmax(ref), where


@pytest.mark.parametrize("dim,heads,S", [(256, 4, 150), (256, 2, 150), (512, 4, 300)])
def test_bf16_prefill_and_decode_track_oracle(backend, pkg, ora, dim, heads, S):
    cfg = pkg.ModelConfig.new(300, dim, heads, 2, S + 8)
    w = pkg.synthetic_weights(cfg, seed=51, bf16=True)
    model = pkg.hip.Model(backend, cfg)
    model.upload(w)
    model.set_prefill_bf16(True)
    s = pkg.hip.Session(model, S + 8, 3)
    toks = pkg.synthetic_tokens(3 * S, cfg.vocab_size, seed=52).reshape(3, S)
    logits, _ = s.prefill(toks)
    for b in (0, 2):
        o = ora.OracleSession(cfg, w, S + 8)
        _check_logits(logits[b], o.prefill(toks[b]), ora, f"sequence {b} prefill")
        # The bf16 prefill wrote K and V in f32 from bf16 operands.
        np.testing.assert_allclose(s.cache(1, b, 0)[:S], o.k_cache(1)[:S], atol=TOL, rtol=0)
        o.close()
    # Back on the f32 path the 1e-3 bar holds again.
    model.set_prefill_bf16(False)
    s.reset()
    logits32, _ = s.prefill(toks)
    o = ora.OracleSession(cfg, w, S + 8)
    assert np.abs(logits32[1] - o.prefill(toks[1])).max() < 1e-3
    o.close()


def test_bf16_decode_after_prefill_tracks_oracle(backend, pkg, ora):
    cfg = pkg.ModelConfig.new(300, 256, 2, 2, 80)
    w = pkg.synthetic_weights(cfg, seed=53, bf16=True)
    model = pkg.hip.Model(backend, cfg)
    model.upload(w)
    model.set_prefill_bf16(True)
    s = pkg.hip.Session(model, 80, 2)
    toks = pkg.synthetic_tokens(2 * 60, cfg.vocab_size, seed=54).reshape(2, 60)
    s.prefill(toks)
    feed = np.array([5, 7], np.uint32)
    outs = []
    for _ in range(4):
        lg, nx = s.decode_step(feed)
        outs.append((lg, feed.copy()))
        feed = nx
    for b in range(2):
        o = ora.OracleSession(cfg, w, 80)
        o.prefill(toks[b])
        for i, (lg, fed) in enumerate(outs):
            _check_logits(lg[b], o.decode_step(int(fed[b])), ora, f"sequence {b} step {i}")
        o.close()


def test_bf16_prefill_scaled_config(backend, pkg, ora):
    # Config 5 architecture (dim 2048, 24 layers, 16 x 128, FFN 8192, vocab
    # 50257), bf16-valued weights from seed 5; two 40-token prompts.
    cfg = pkg.ModelConfig.scaled()
    w = pkg.synthetic_weights(cfg, seed=5, bf16=True)
    model = pkg.hip.Model(backend, cfg)
    model.upload(w)
    model.set_prefill_bf16(True)
    s = pkg.hip.Session(model, 64, 2)
    toks = pkg.synthetic_tokens(2 * 40, cfg.vocab_size, seed=6).reshape(2, 40)
    logits, _ = s.prefill(toks)
    ora.set_threads(16)
    try:
        for b in range(2):
            o = ora.OracleSession(cfg, w, 64)
            _check_logits(logits[b], o.prefill(toks[b]), ora, f"sequence {b}")
            o.close()
    finally:
        ora.set_threads(1)


def test_bf16_prefill_rejects_unsupported_heads(backend, pkg):
    cfg = pkg.ModelConfig.new(97, 32, 4, 2, 16)  # head_dim 8
    model = pkg.hip.Model(backend, cfg)
    with pytest.raises(pkg.hip.InvalidArgument, match="head_dim 64 or 128"):
        model.set_prefill_bf16(True)


# ---- the bfloat16 KV cache (akh_session_set_kv_bf16) ----------------------

def test_kv_bf16_decode_tracks_oracle(backend, pkg, ora):
    cfg = pkg.ModelConfig.new(300, 256, 4, 2, 80)
    w = pkg.synthetic_weights(cfg, seed=55)
    model = pkg.hip.Model(backend, cfg)
    model.upload(w)
    s = pkg.hip.Session(model, 80, 2)
    s.set_kv_bf16(True)
    toks = pkg.synthetic_tokens(2 * 60, cfg.vocab_size, seed=56).reshape(2, 60)
    logits, nxt = s.prefill(toks)
    steps = []
    feed = nxt
    for _ in range(5):
        lg, nx = s.decode_step(feed)
        steps.append((lg, feed.copy()))
        feed = nx
    for b in range(2):
        o = ora.OracleSession(cfg, w, 80)
        # Prefill's own attention used f32 K/V: its logits meet the f32 bar.
        assert np.abs(logits[b] - o.prefill(toks[b])).max() < 1e-3
        # The cache holds the oracle's rows rounded to bfloat16.
        ref = o.k_cache(1)[:60]
        got = s.cache(1, b, 0)[:60]
        assert np.all(np.abs(got - ref) <= np.abs(ref) * 2.0 ** -8 + 1e-6)
        for i, (lg, fed) in enumerate(steps):
            _check_logits(lg[b], o.decode_step(int(fed[b])), ora, f"sequence {b} step {i}")
        o.close()


def test_kv_bf16_cache_hand_over_and_errors(backend, pkg):
    hip = pkg.hip
    cfg = pkg.ModelConfig.new(97, 64, 1, 2, 16)
    w = pkg.synthetic_weights(cfg, seed=57)
    model = hip.Model(backend, cfg)
    model.upload(w)
    a = hip.Session(model, 16, 2)
    a.set_kv_bf16(True)
    a.prefill(np.array([[3, 41, 7, 9], [11, 12, 13, 14]], np.uint32))
    with pytest.raises(hip.CacheNotEmpty):
        a.set_kv_bf16(False)
    k, v, n = a.take_cache(1)
    assert n == 4
    # Values come back widened from bfloat16: low 16 bits zero.
    assert not np.any(k.view(np.uint32) & 0xFFFF)
    b = hip.Session(model, 16, 2)
    b.set_kv_bf16(True)
    b.replace_cache(0, k, v, n)
    assert np.array_equal(b.cache(1, 0, 1), v[1])
    # An f32 session takes the same cache exactly.
    c = hip.Session(model, 16, 2)
    c.replace_cache(1, k, v, n)
    assert np.array_equal(c.cache(0, 1, 0), k[0])


def test_kv_bf16_scaled_config(backend, pkg, ora):
    # Config 5's optional bf16 path end to end: bf16-MFMA prefill, bfloat16
    # KV cache, f32 decode; two 24-token prompts and 3 decode steps.
    cfg = pkg.ModelConfig.scaled()
    w = pkg.synthetic_weights(cfg, seed=5, bf16=True)
    model = pkg.hip.Model(backend, cfg)
    model.upload(w)
    model.set_prefill_bf16(True)
    s = pkg.hip.Session(model, 64, 2)
    s.set_kv_bf16(True)
    toks = pkg.synthetic_tokens(2 * 24, cfg.vocab_size, seed=6).reshape(2, 24)
    logits, nxt = s.prefill(toks)
    steps, feed = [], nxt
    for _ in range(3):
        lg, nx = s.decode_step(feed)
        steps.append((lg, feed.copy()))
        feed = nx
    ora.set_threads(16)
    try:
        for b in range(2):
            o = ora.OracleSession(cfg, w, 64)
            _check_logits(logits[b], o.prefill(toks[b]), ora, f"sequence {b} prefill")
            for i, (lg, fed) in enumerate(steps):
                _check_logits(lg[b], o.decode_step(int(fed[b])), ora, f"sequence {b} step {i}")
            o.close()
    finally:
        ora.set_threads(1)
