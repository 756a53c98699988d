"""InferenceSession::generate (src/nn/inference.rs:264-326) on the batched
session, against the reference loop restated on the CPU oracle with the same
draws: the prompt (prefill on an empty cache, decode steps on a resumed one),
sample_token over this call's history, eos and full-context stops, and the
cache length each sequence is left with."""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _oracle_generate(ora, osess, prompt, max_new, t, k, p, pen, eos, draws):
    """inference.rs:288-323 with rand::random() replaced by ``draws``."""
    if osess.cur_len() == 0:
        logits = osess.prefill(prompt)
    else:
        for tok in prompt:
            logits = osess.decode_step(int(tok))
    hist = [int(x) for x in prompt]
    gen = []
    for i in range(max_new):
        nxt = ora.sample_token(logits, t, k, p, np.array(hist, np.uint32), pen,
                               draws[i] if draws is not None else 0.0)
        gen.append(nxt)
        hist.append(nxt)
        if nxt == eos:
            break
        try:
            logits = osess.decode_step(nxt)
        except RuntimeError as e:  # ContextFull (code 3) ends generate quietly
            assert "error 3" in str(e)
            break
    return gen


def _setup(pkg, backend, ora, cfg, seed, max_ctx, batch):
    w = pkg.synthetic_weights(cfg, seed=seed)
    model = pkg.hip.Model(backend, cfg)
    model.upload(w)
    sess = pkg.hip.Session(model, max_ctx, batch)
    orcs = [ora.OracleSession(cfg, w, max_ctx) for _ in range(batch)]
    return model, sess, orcs


def _check(pkg, ora, sess, orcs, cfg, prompt, max_new, t, k, p, pen, draws):
    got = sess.generate(prompt, max_new, t, k, p, pen, draws)
    for b, o in enumerate(orcs):
        want = _oracle_generate(ora, o, prompt[b], max_new, t, k, p, pen, cfg.eos_token,
                                draws[:, b] if draws is not None else None)
        assert list(got[b]) == want, f"sequence {b}"
        assert int(sess.cur_len()[b]) == o.cur_len(), f"sequence {b} cache length"
    return got


def test_generate_greedy_and_sampled_match_oracle(backend, pkg, ora):
    cfg = pkg.ModelConfig.new(97, 32, 4, 2, 16)
    rng = np.random.default_rng(5)
    prompt = rng.integers(0, cfg.vocab_size - 1, (3, 5)).astype(np.uint32)
    # Greedy, with a repetition penalty.
    _, s, o = _setup(pkg, backend, ora, cfg, 21, 40, 3)
    _check(pkg, ora, s, o, cfg, prompt, 8, 0.0, 0, 1.0, 1.3, None)
    # run_chat's defaults (main.rs:162): temperature 0.8, top_k 40, top_p 0.95,
    # repetition penalty 1.15.
    _, s, o = _setup(pkg, backend, ora, cfg, 22, 40, 3)
    draws = rng.random((10, 3))
    _check(pkg, ora, s, o, cfg, prompt, 10, 0.8, 40, 0.95, 1.15, draws)
    # Resumed caches: the prompt goes through decode steps, history restarts.
    more = rng.integers(0, cfg.vocab_size - 1, (3, 3)).astype(np.uint32)
    _check(pkg, ora, s, o, cfg, more, 6, 1.2, 0, 0.9, 1.0, rng.random((6, 3)))


def test_generate_ragged_prompts_match_oracle(backend, pkg, ora):
    # Prompts of different lengths in one call (the reference takes one
    # prompt per session): prefilled together on empty caches, then fed as
    # decode steps on the resumed caches, each sequence against its own
    # restated generate loop.
    cfg = pkg.ModelConfig.new(97, 32, 4, 2, 16)
    rng = np.random.default_rng(8)
    prompts = [rng.integers(0, cfg.vocab_size - 1, n).astype(np.uint32) for n in (5, 1, 9, 3)]
    _, s, o = _setup(pkg, backend, ora, cfg, 26, 48, 4)
    _check(pkg, ora, s, o, cfg, prompts, 7, 0.8, 40, 0.95, 1.15, rng.random((7, 4)))
    more = [rng.integers(0, cfg.vocab_size - 1, n).astype(np.uint32) for n in (2, 6, 1, 4)]
    _check(pkg, ora, s, o, cfg, more, 5, 0.0, 0, 1.0, 1.2, None)


def test_generate_stops_at_eos_and_full_context(backend, pkg, ora):
    cfg = pkg.ModelConfig.new(97, 32, 4, 2, 16)
    rng = np.random.default_rng(6)
    prompt = rng.integers(0, cfg.vocab_size - 1, (4, 4)).astype(np.uint32)
    # A small top_k at high temperature reaches eos (= 96) on some rows:
    # pick draws until at least one sequence stops there.
    for trial in range(20):
        _, s, o = _setup(pkg, backend, ora, cfg, 23, 64, 4)
        draws = np.random.default_rng(100 + trial).random((24, 4))
        got = _check(pkg, ora, s, o, cfg, prompt, 24, 50.0, 0, 1.0, 1.0, draws)
        if any(len(g) and g[-1] == cfg.eos_token for g in got):
            break
    else:
        pytest.fail("no sequence sampled eos")
    # Full context: 4 prompt tokens in a 7-token window allow 3 decodes; the
    # 4th sampled token is returned but cannot be decoded.
    _, s, o = _setup(pkg, backend, ora, cfg, 24, 7, 4)
    got = _check(pkg, ora, s, o, cfg, prompt, 10, 0.0, 0, 1.0, 1.0, None)
    for b, g in enumerate(got):
        if g[-1] != cfg.eos_token:
            assert len(g) == 4 and int(s.cur_len()[b]) == 7


def test_generate_matches_decode_greedy_and_errors(backend, pkg, ora):
    hip = pkg.hip
    cfg = pkg.ModelConfig.new(97, 32, 4, 2, 16)
    w = pkg.synthetic_weights(cfg, seed=25)
    model = hip.Model(backend, cfg)
    model.upload(w)
    prompt = np.random.default_rng(7).integers(0, 96, (2, 6)).astype(np.uint32)
    a = hip.Session(model, 32, 2)
    got = a.generate(prompt, 9)
    b = hip.Session(model, 32, 2)
    _, nxt = b.prefill(prompt)
    toks = b.decode_greedy(8)
    for r in range(2):
        want = [int(nxt[r])] + [int(x) for x in toks[:, r]]
        if cfg.eos_token in want:
            want = want[:want.index(cfg.eos_token) + 1]
        assert list(got[r]) == want
    with pytest.raises(hip.EmptyPrompt):
        a.generate(np.zeros((2, 0), np.uint32), 4)
    with pytest.raises(hip.PromptTooLong):
        hip.Session(model, 4, 2).generate(prompt, 4)
    with pytest.raises(hip.InvalidArgument, match="uniforms"):
        hip.Session(model, 32, 2).generate(prompt, 4, temperature=1.0)
    # A resumed prompt that overflows the window fails like decode_step.
    c = hip.Session(model, 8, 2)
    c.generate(prompt, 0)
    with pytest.raises(hip.ContextFull):
        c.generate(prompt, 2)
