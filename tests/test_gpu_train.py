"""The trainer's forward (Trainer::forward + CrossEntropy, src/nn/train.rs:
256-275) on the GPU against the CPU oracle: the shaders its graph adds to
the inference set (QKV_SPLIT, ROPE_QK, ADD, RESIDUAL_ADD, SILU_OUT,
CROSS_ENTROPY) through their per-shader launchers, and the fused batched
forward (akh_forward) with row_offset batching, the all-rows lm_head and
the loss.

Tolerances: the reference's batching test holds losses and the residual
stream to 1e-3 (train.rs:928-945); elementwise shaders are exact or within
an ulp of libm.
"""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def test_qkv_split_and_rope_qk(backend, pkg, ora):
    h = pkg.hip
    rows, d, hd = 13, 48, 16
    src = ora.rand_vec(rows * 3 * d, 21)
    q, k, v = backend.zeros(rows * d), backend.zeros(rows * d), backend.zeros(rows * d)
    shape = h.HeadMoveMeta(rows, 3 * d, d, 0)
    backend.qkv_split(backend.tensor(src), q, k, v, shape, backend.meta(shape))
    want = ora.qkv_split(src, rows, 3 * d, d)
    for got, w in zip((q, k, v), want):
        assert np.array_equal(got.download(), w)
    # rope_qk on the second sequence of a 2 x 6 + 1 row buffer.
    S, off = 6, 6
    rq = h.RopeMeta(S, d, hd, off)
    backend.rope_qk(q, k, rq, backend.meta(rq))
    wq, wk = ora.rope_qk(want[0], want[1], S, d, hd, off)
    np.testing.assert_allclose(q.download(), wq, atol=2e-6)
    np.testing.assert_allclose(k.download(), wk, atol=2e-6)


def test_add_residual_add_silu_out(backend, pkg, ora):
    n = 5000
    a, b = ora.rand_vec(n, 22) * 4, ora.rand_vec(n, 23)
    ta, tb, out = backend.tensor(a), backend.tensor(b), backend.zeros(n)
    backend.add(ta, tb, out, n)
    assert np.array_equal(out.download(), ora.add(a, b))
    backend.residual_add(ta, tb, n)
    assert np.array_equal(ta.download(), ora.residual_add(a, b))
    backend.silu_out(tb, out, n)
    np.testing.assert_allclose(out.download(), ora.silu_out(b), rtol=1e-6, atol=1e-7)


def test_cross_entropy(backend, pkg, ora):
    h = pkg.hip
    rows, V = 9, 50257
    x = (ora.rand_vec(rows * V, 24) * 5).astype(np.float32)
    t = ora.rand_tokens(rows, V, 25)
    tl, losses = backend.tensor(x), backend.zeros(rows)
    shape = h.CrossEntropyMeta(V, rows)
    backend.cross_entropy(tl, backend.tensor(t), losses, shape, backend.meta(shape))
    probs, want = ora.cross_entropy(x, t, V, rows)
    np.testing.assert_allclose(losses.download(), want, atol=1e-4)
    np.testing.assert_allclose(tl.download(), probs, atol=1e-7, rtol=1e-4)
    # A target past the vocabulary has no logit: NaN, other rows unaffected.
    bad = t.copy()
    bad[3] = V
    tl2 = backend.tensor(x)
    backend.cross_entropy(tl2, backend.tensor(bad), losses, shape, backend.meta(shape))
    got = losses.download()
    assert np.isnan(got[3]) and np.allclose(np.delete(got, 3), np.delete(want, 3), atol=1e-4)


def _forward(pkg, backend, cfg, w, toks, tgts):
    model = pkg.hip.Model(backend, cfg)
    model.upload(w)
    B, S = toks.shape
    f = pkg.hip.Forward(model, B, S)
    mean, losses = f.loss(toks, tgts)
    return f, mean, losses


def test_forward_matches_oracle_and_sequential_batching(backend, pkg, ora):
    # real_batching_matches_sequential_accumulation (train.rs:852-946):
    # ModelConfig::new(37, 16, 4, 2, 11), batch 3, token LCG seeds 100+b and
    # 200+b; the batched forward equals the per-sequence forwards.
    cfg = pkg.ModelConfig.new(37, 16, 4, 2, 11)
    w = pkg.synthetic_weights(cfg, seed=26)
    B, S = 3, 11
    toks = np.stack([ora.rand_tokens(S, 37, 100 + b) for b in range(B)])
    tgts = np.stack([ora.rand_tokens(S, 37, 200 + b) for b in range(B)])
    f, mean, losses = _forward(pkg, backend, cfg, w, toks, tgts)
    om, ol, op, oh = ora.forward_train(cfg, w, toks, tgts, B, S, True, True)
    np.testing.assert_allclose(losses, ol, atol=1e-4)
    assert abs(mean - om) < 1e-4
    np.testing.assert_allclose(f.probs(0, B * S), op, atol=1e-5)
    np.testing.assert_allclose(f.hidden(), oh, atol=1e-4)
    hidden = f.hidden()
    f.close()
    seq = []
    for b in range(B):
        fb, mb, lb = _forward(pkg, backend, cfg, w, toks[b:b + 1], tgts[b:b + 1])
        seq.append(mb)
        np.testing.assert_allclose(lb, losses[b * S:(b + 1) * S], atol=1e-3)
        if b == B - 1:
            np.testing.assert_allclose(fb.hidden(), hidden[b * S:], atol=1e-3)
        fb.close()
    assert abs(np.mean(seq) - mean) < 1e-3


def test_forward_hall1_against_oracle(backend, pkg, ora):
    # hall-1.0 (config 1's weights, seed 0), 2 sequences of 64 tokens.
    cfg = pkg.ModelConfig.akasha_hall_1()
    w = pkg.synthetic_weights(cfg, seed=0)
    B, S = 2, 64
    toks = pkg.synthetic_tokens(B * S, cfg.vocab_size, seed=27).reshape(B, S)
    tgts = np.roll(toks, -1, axis=1)
    f, mean, losses = _forward(pkg, backend, cfg, w, toks, tgts)
    ora.set_threads(16)
    try:
        om, ol, _, oh = ora.forward_train(cfg, w, toks, tgts, B, S, False, True)
    finally:
        ora.set_threads(1)
    np.testing.assert_allclose(losses, ol, atol=1e-3)
    assert abs(mean - om) < 1e-3
    np.testing.assert_allclose(f.hidden(), oh, atol=1e-3)
    f.close()


def test_forward_errors(backend, pkg):
    hip = pkg.hip
    cfg = pkg.ModelConfig.new(37, 16, 4, 2, 11)
    model = hip.Model(backend, cfg)
    model.upload(pkg.synthetic_weights(cfg, seed=1))
    with pytest.raises(hip.InvalidArgument):
        hip.Forward(model, 0, 4)
    f = hip.Forward(model, 1, 4)
    with pytest.raises(hip.InvalidArgument, match="out of the vocabulary"):
        f.loss(np.zeros(4, np.uint32), np.array([1, 2, 37, 3], np.uint32))
    f.close()


@pytest.mark.parametrize("kind,vocab,dim", [("h3", 300, 64), ("h3", 301, 64), ("x6", 300, 64),
                                            ("h3", 300, 72), ("x6", 300, 72)])
def test_forward_split_matches_fp32_mfma(backend, pkg, ora, kind, vocab, dim):
    # The trainer forward's GEMMs (layers and the all-rows lm_head) on the
    # split kernels (h3, the default, or x6) and on the fp32 MFMAs: losses
    # and probabilities agree to fp32 rounding.  2 x 40 rows; dim 64, vocab
    # 300, and 301 (an odd lm_head width: ragged last column tile, unpaired
    # epilogue stores); dim 72 (4 heads of 18): every GEMM's K = 72 or 288
    # ends on a partial 32-k step of the split kernels.
    M = pkg.hip.Model
    cfg = pkg.ModelConfig.new(vocab, dim, 4, 2, 40)
    w = pkg.synthetic_weights(cfg, seed=64)
    B, S = 2, 40
    toks = np.stack([ora.rand_tokens(S, vocab, 300 + b) for b in range(B)])
    tgts = np.stack([ora.rand_tokens(S, vocab, 400 + b) for b in range(B)])
    model = pkg.hip.Model(backend, cfg)
    model.upload(w)
    model.set_prefill_split(M.SPLIT_H3 if kind == "h3" else M.SPLIT_X6)
    f = pkg.hip.Forward(model, B, S)
    mx, lx = f.loss(toks, tgts)
    px = f.probs(0, B * S)
    model.set_prefill_split(M.SPLIT_NONE)
    mf, lf = f.loss(toks, tgts)
    np.testing.assert_allclose(lx, lf, atol=1e-5)
    np.testing.assert_allclose(px, f.probs(0, B * S), atol=1e-6)
    assert abs(mx - mf) < 1e-5
    om, ol, _, _ = ora.forward_train(cfg, w, toks, tgts, B, S, False, False)
    np.testing.assert_allclose(lx, ol, atol=1e-4)
    f.close()


def test_forward_x6_needs_multiples_of_8(backend, pkg, ora):
    # dim 20 (5 heads of 4): the fp32-MFMA GEMMs run, and the split-bf16
    # GEMMs cannot be switched on.
    cfg = pkg.ModelConfig.new(37, 20, 5, 1, 11)
    w = pkg.synthetic_weights(cfg, seed=65)
    toks = np.stack([ora.rand_tokens(11, 37, 500 + b) for b in range(2)])
    tgts = np.stack([ora.rand_tokens(11, 37, 600 + b) for b in range(2)])
    model = pkg.hip.Model(backend, cfg)
    model.upload(w)
    assert model.prefill_split() == pkg.hip.Model.SPLIT_NONE
    for kind in (pkg.hip.Model.SPLIT_H3, pkg.hip.Model.SPLIT_X6):
        with pytest.raises(pkg.hip.InvalidArgument, match="multiples of 8"):
            model.set_prefill_split(kind)
    with pytest.raises(pkg.hip.InvalidArgument, match="multiples of 8"):
        model.set_prefill_x6(True)
    model.set_prefill_x6(False)
    f = pkg.hip.Forward(model, 2, 11)
    mean, losses = f.loss(toks, tgts)
    om, ol, _, _ = ora.forward_train(cfg, w, toks, tgts, 2, 11, False, False)
    np.testing.assert_allclose(losses, ol, atol=1e-4)
    f.close()


def test_forward_x6_ragged_k(backend, pkg, ora):
    # dim 40: K = 40 is a multiple of 8 but not of the split-bf16 GEMM's
    # 16-wide k step (the last step is half masked); 2 x 11 rows and vocab 37
    # leave every tile ragged in M and N.
    cfg = pkg.ModelConfig.new(37, 40, 5, 1, 11)
    w = pkg.synthetic_weights(cfg, seed=66)
    toks = np.stack([ora.rand_tokens(11, 37, 700 + b) for b in range(2)])
    tgts = np.stack([ora.rand_tokens(11, 37, 800 + b) for b in range(2)])
    model = pkg.hip.Model(backend, cfg)
    model.upload(w)
    f = pkg.hip.Forward(model, 2, 11)
    mean, losses = f.loss(toks, tgts)
    om, ol, op, oh = ora.forward_train(cfg, w, toks, tgts, 2, 11, True, True)
    np.testing.assert_allclose(losses, ol, atol=1e-4)
    np.testing.assert_allclose(f.hidden(), oh, atol=1e-4)
    np.testing.assert_allclose(f.probs(0, 22), op, atol=1e-5)
    f.close()
