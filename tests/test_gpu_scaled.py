"""Config 5 (the scaled architecture: dim 2048, 24 layers, 16 heads x 128,
FFN 8192, vocab 50257, ctx 2048, bfloat16-valued weights from seed 5) at its
full shapes on the GPU.

The CPU oracle cannot run this model at these sizes in test time (its
prefill of one 2040-token prompt is ~5 TFLOP of scalar loops); parity with
the oracle is checked on this architecture at small sizes in
test_gpu_session.py and test_gpu_bf16.py.  Here the full shapes are held to
size-independent properties:

- batch invariance inside the 64-sequence decode at KV length 2048 (two
  32-row tiles, one weight read): a sequence's logits and tokens equal the
  same prompt decoded alone, with the f32 and with the bfloat16 KV cache;
- bfloat16 weight tiles against float tiles of the same values at KV 2048,
  and the fused residual add + RMSNorm against the default;
- the 8 x 2048 prefill on the split-fp16 and split-bf16 kernels against
  the fp32-MFMA kernels;
- prefill == sequential decode (inference.rs:334-359): a 2048-token prefill
  against a 2040-token prefill followed by the last 8 tokens as decode
  steps.
"""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def scaled(backend, pkg):
    cfg = pkg.ModelConfig.scaled()
    w = pkg.synthetic_weights(cfg, seed=5, bf16=True)
    model = pkg.hip.Model(backend, cfg)
    model.upload(w)
    del w
    yield cfg, model
    model.close()


def _decode(s, steps):
    return [s.decode_step(None) for _ in range(steps)]


def test_scaled_decode_64_rows_at_kv_2048(pkg, scaled):
    cfg, model = scaled
    hip = pkg.hip
    B, S, steps = 64, 2040, 8
    toks = pkg.synthetic_tokens(B * S, cfg.vocab_size, seed=8).reshape(B, S)
    s = hip.Session(model, 2048, B)
    first = s.prefill(toks)
    run = [first] + _decode(s, steps)
    assert list(s.cur_len()) == [2048] * B
    # Batch invariance: rows of the first tile, of the second, and the last.
    for b in (5, 37, 63):
        one = hip.Session(model, 2048, 1)
        alone = [one.prefill(toks[b][None])] + _decode(one, steps)
        for i, ((lg, tk), (l1, t1)) in enumerate(zip(run, alone)):
            assert np.abs(lg[b] - l1[0]).max() < 1e-4, f"sequence {b} step {i}"
            assert int(tk[b]) == int(t1[0]), f"sequence {b} step {i}"
        one.close()
    # bfloat16 weight tiles (the default for these weights) against float
    # tiles of the same values, the same 8 steps from the same caches.
    assert model.set_bf16_tiles(False) == 0
    try:
        s.truncate(S)
        f32 = _decode(s, steps)
    finally:
        model.set_bf16_tiles(True)
    for i, ((a, ta), (b, tb)) in enumerate(zip(run[1:], f32)):
        assert np.abs(a - b).max() < 1e-4, f"step {i}"
        assert np.array_equal(ta, tb), f"step {i}"
    # The residual adds + RMSNorms folded into the GEMMs (the K splits of
    # out_proj and ffn_down summed by the last block of each column tile),
    # the same steps.
    s.set_fused_norm(True)
    try:
        s.truncate(S)
        fused = _decode(s, steps)
    finally:
        s.set_fused_norm(False)
    for i, ((a, ta), (b, tb)) in enumerate(zip(run[1:], fused)):
        assert np.abs(a - b).max() < 1e-4, f"fused norm, step {i}"
        assert np.array_equal(ta, tb), f"fused norm, step {i}"
    s.close()


def test_scaled_decode_64_rows_bf16_kv_at_kv_2048(pkg, scaled):
    # The bfloat16 KV cache at full shape: the 64-sequence session decodes
    # with the long-context attention shape (8 waves, one row split), a
    # single sequence with the short one (4 waves, two splits).  The prefill
    # GEMMs tile the two sessions' rows differently, so an fp32 K or V
    # value may round to a neighbouring bfloat16 in the cache: the bound is
    # 2e-3, well inside the bf16 path's 2e-2 against the oracle.
    cfg, model = scaled
    hip = pkg.hip
    B, S, steps = 64, 2040, 4
    toks = pkg.synthetic_tokens(B * S, cfg.vocab_size, seed=10).reshape(B, S)
    s = hip.Session(model, 2048, B)
    s.set_kv_bf16(True)
    run = [s.prefill(toks)] + _decode(s, steps)
    for b in (0, 40):
        one = hip.Session(model, 2048, 1)
        one.set_kv_bf16(True)
        alone = [one.prefill(toks[b][None])] + _decode(one, steps)
        for i, ((lg, tk), (l1, t1)) in enumerate(zip(run, alone)):
            assert np.abs(lg[b] - l1[0]).max() < 2e-3, f"sequence {b} step {i}"
            assert int(tk[b]) == int(t1[0]), f"sequence {b} step {i}"
        one.close()
    s.close()


def test_scaled_prefill_8x2048_split_vs_fp32_mfma(pkg, scaled):
    # The 8 x 2048 prefill on the default split-fp16 GEMMs (256 x 128 tiles
    # at these shapes) and on the split-bf16 ones, each against the
    # fp32-MFMA kernels: logits and cache within fp32 rounding, same tokens.
    cfg, model = scaled
    M = pkg.hip.Model
    B, S = 8, 2048
    toks = pkg.synthetic_tokens(B * S, cfg.vocab_size, seed=7).reshape(B, S)
    s = pkg.hip.Session(model, S, B)
    runs = {}
    try:
        for kind in (M.SPLIT_H3, M.SPLIT_X6, M.SPLIT_NONE):
            model.set_prefill_split(kind)
            s.reset()
            lg, tk = s.prefill(toks)
            runs[kind] = (lg, tk, s.cache(23, 6, 0))
    finally:
        model.set_prefill_split(M.SPLIT_H3)
    l32, t32, k32 = runs[M.SPLIT_NONE]
    for kind in (M.SPLIT_H3, M.SPLIT_X6):
        lg, tk, kc = runs[kind]
        assert np.abs(lg - l32).max() < 1e-4, kind
        assert np.array_equal(tk, t32), kind
        np.testing.assert_allclose(kc, k32, rtol=0, atol=1e-4)
    s.close()


def test_scaled_prefill_equals_sequential_decode(pkg, scaled):
    cfg, model = scaled
    B, S, tail = 2, 2048, 8
    toks = pkg.synthetic_tokens(B * S, cfg.vocab_size, seed=9).reshape(B, S)
    a = pkg.hip.Session(model, S, B)
    full, _ = a.prefill(toks)
    b = pkg.hip.Session(model, S, B)
    b.prefill(toks[:, :S - tail])
    for t in range(S - tail, S):
        last, _ = b.decode_step(np.ascontiguousarray(toks[:, t]))
    assert np.abs(full - last).max() < 1e-3
    np.testing.assert_allclose(a.cache(20, 1, 1)[S - tail:], b.cache(20, 1, 1)[S - tail:],
                               rtol=0, atol=1e-3)
    a.close()
    b.close()
