"""The batched InferenceSession of libakasha_hip.so against the CPU oracle.

Parity bar: identical greedy tokens and logits
within max-abs 1e-3 on the fp32 path.  Full-size configurations are checked
on a few sequences against the oracle and, for the whole batch, through
size-independent properties (batch invariance, prefill == sequential
decode, cache contents).
"""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

TOL = 1e-3


def _session(pkg, backend, cfg, w, max_ctx, batch):
    model = pkg.hip.Model(backend, cfg)
    model.upload(w)
    return model, pkg.hip.Session(model, max_ctx, batch)


def _oracle_greedy(ora, cfg, w, max_ctx, prompt, steps):
    o = ora.OracleSession(cfg, w, max_ctx)
    logits = [o.prefill(prompt)]
    toks = [ora.argmax(logits[0])]
    for _ in range(steps):
        logits.append(o.decode_step(toks[-1]))
        toks.append(ora.argmax(logits[-1]))
    o.close()
    return logits, toks


def _oracle_greedy_many(ora, cfg, w, max_ctx, prompts, steps):
    """_oracle_greedy for several prompts at once: one single-threaded
    oracle session per host thread (the checker's time, not the product's)."""
    import threading
    out = [None] * len(prompts)

    def run(i):
        out[i] = _oracle_greedy(ora, cfg, w, max_ctx, prompts[i], steps)

    ora.set_threads(1)
    ts = [threading.Thread(target=run, args=(i,)) for i in range(len(prompts))]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    assert all(o is not None for o in out)
    return out


def test_tiny_prefill_and_decode_match_oracle(backend, pkg, ora):
    # ModelConfig::new(97,32,4,2,16), prompt [3,41,7,96,0,25]
    # (inference.rs:334-359).
    cfg = pkg.ModelConfig.new(97, 32, 4, 2, 16)
    w = pkg.synthetic_weights(cfg, seed=42)
    prompt = np.array([3, 41, 7, 96, 0, 25], np.uint32)
    model, s = _session(pkg, backend, cfg, w, 16, 1)
    ref_logits, ref_toks = _oracle_greedy(ora, cfg, w, 16, prompt, 9)
    logits, nxt = s.prefill(prompt[None])
    assert np.abs(logits[0] - ref_logits[0]).max() < TOL
    assert int(nxt[0]) == ref_toks[0]
    for i in range(1, 10):
        logits, nxt = s.decode_step(None)
        assert np.abs(logits[0] - ref_logits[i]).max() < TOL, f"step {i}"
        assert int(nxt[0]) == ref_toks[i], f"step {i}"
    assert list(s.cur_len()) == [15]


def test_prefill_equals_sequential_decode_on_gpu(backend, pkg):
    cfg = pkg.ModelConfig.new(97, 32, 4, 2, 16)
    w = pkg.synthetic_weights(cfg, seed=42)
    prompt = np.array([3, 41, 7, 96, 0, 25], np.uint32)
    _, a = _session(pkg, backend, cfg, w, 16, 1)
    pre, _ = a.prefill(prompt[None])
    _, b = _session(pkg, backend, cfg, w, 16, 1)
    for t in prompt:
        dec, _ = b.decode_step(np.array([t]))
    assert np.abs(pre - dec).max() < TOL
    np.testing.assert_allclose(a.cache(1, 0, 0), b.cache(1, 0, 0), atol=1e-4)


def test_batched_sessions_are_independent(backend, pkg, ora):
    cfg = pkg.ModelConfig.new(300, 128, 2, 2, 40)  # head_dim 64
    w = pkg.synthetic_weights(cfg, seed=5)
    B, S, steps = 5, 17, 6
    prompts = pkg.synthetic_tokens(B * S, cfg.vocab_size, 6).reshape(B, S)
    _, s = _session(pkg, backend, cfg, w, 40, B)
    logits, nxt = s.prefill(prompts)
    got_l, got_t = [logits], [nxt]
    for _ in range(steps):
        logits, nxt = s.decode_step(None)
        got_l.append(logits)
        got_t.append(nxt)
    for b in range(B):
        rl, rt = _oracle_greedy(ora, cfg, w, 40, prompts[b], steps)
        for i in range(steps + 1):
            assert np.abs(got_l[i][b] - rl[i]).max() < TOL
            assert int(got_t[i][b]) == rt[i]


def _run(s, prompts, steps):
    out = [s.prefill(prompts)]
    out += [s.decode_step(None) for _ in range(steps)]
    return out


@pytest.mark.parametrize("kv16", [False, True])
def test_two_row_tiles_match_oracle_and_smaller_sessions(backend, pkg, ora, kv16):
    # A session of 33..64 sequences holds its rows as two 32-row MFMA tiles
    # that share every weight read.  40 sequences (rows 32..39 in a second,
    # partly filled tile) give, row for row, what a 32-row and an 8-row
    # session give on the same prompts (each row's arithmetic does not
    # depend on the batch), and, on the fp32 cache, what the oracle gives.
    cfg = pkg.ModelConfig.new(300, 128, 2, 2, 40)
    w = pkg.synthetic_weights(cfg, seed=51)
    B, S, steps = 40, 13, 6
    prompts = pkg.synthetic_tokens(B * S, cfg.vocab_size, 52).reshape(B, S)
    model = pkg.hip.Model(backend, cfg)
    model.upload(w)
    sess = [pkg.hip.Session(model, 40, n) for n in (B, 32, 8)]
    if kv16:
        for s in sess:
            s.set_kv_bf16(True)
    got = _run(sess[0], prompts, steps)
    lo = _run(sess[1], prompts[:32], steps)
    hi = _run(sess[2], prompts[32:], steps)
    for i in range(steps + 1):
        lg, tk = got[i]
        np.testing.assert_allclose(lg[:32], lo[i][0], rtol=0, atol=1e-5)
        np.testing.assert_allclose(lg[32:], hi[i][0], rtol=0, atol=1e-5)
        assert np.array_equal(tk, np.concatenate([lo[i][1], hi[i][1]]))
    # Graph replays of the same steps give the same tokens.
    sess[0].truncate(S)
    assert np.array_equal(sess[0].decode_greedy(steps),
                          np.stack([got[i][1] for i in range(1, steps + 1)]))
    if not kv16:
        refs = _oracle_greedy_many(ora, cfg, w, 40, list(prompts), steps)
        for b, (rl, rt) in enumerate(refs):
            for i in range(steps + 1):
                assert np.abs(got[i][0][b] - rl[i]).max() < TOL, f"sequence {b} step {i}"
                assert int(got[i][1][b]) == rt[i], f"sequence {b} step {i}"
    for s in sess:
        s.close()
    model.close()


def test_two_row_tiles_bf16_weight_tiles(backend, pkg):
    # bfloat16-valued weights read as bfloat16 tiles by a 40-row session:
    # within fp32 rounding of the float tiles, same tokens (as at 32 rows).
    cfg = pkg.ModelConfig.new(500, 1152, 9, 2, 40)
    w = pkg.synthetic_weights(cfg, seed=53, bf16=True)
    model = pkg.hip.Model(backend, cfg)
    model.upload(w)
    s = pkg.hip.Session(model, 40, 40)
    toks = pkg.synthetic_tokens(40 * 9, cfg.vocab_size, seed=54).reshape(40, 9)
    runs = {}
    for allow in (True, False):
        model.set_bf16_tiles(allow)
        s.reset()
        runs[allow] = _run(s, toks, 3)
    for (a, ta), (b, tb) in zip(runs[True], runs[False]):
        assert np.abs(a - b).max() < 1e-4 and np.array_equal(ta, tb)
    s.close()
    model.close()


@pytest.mark.parametrize("B", [5, 40])
@pytest.mark.parametrize("bf16_tiles", [False, True])
def test_fused_norm_matches_oracle(backend, pkg, ora, B, bf16_tiles):
    # akh_session_set_fused_norm: the residual adds + RMSNorms folded into
    # the decode GEMMs (out_proj and ffn_down sum their K splits into the
    # residual, qkv_proj / ffn_up / the final norm scale their operand), on
    # one and two 32-row tiles and on float and bfloat16 weight tiles.
    cfg = pkg.ModelConfig.new(300, 256, 2, 2, 40)  # head_dim 128
    w = pkg.synthetic_weights(cfg, seed=12, bf16=bf16_tiles)
    S, steps = 17, 6
    prompts = pkg.synthetic_tokens(B * S, cfg.vocab_size, 13).reshape(B, S)
    model, s = _session(pkg, backend, cfg, w, 40, B)
    # The layer matrices; lm_head (K = 256) runs the persistent float kernel.
    assert model.set_bf16_tiles(True) == (4 * cfg.num_layers if bf16_tiles else 0)
    plain = _run(s, prompts, steps)
    s.reset()
    s.set_fused_norm(True)
    fused = _run(s, prompts, steps)
    for i, ((lp, tp), (lf, tf)) in enumerate(zip(plain, fused)):
        assert np.abs(lp - lf).max() < 1e-4, f"step {i}"
        assert np.array_equal(tp, tf), f"step {i}"
    for b in sorted({0, B // 2, B - 1}):
        rl, rt = _oracle_greedy(ora, cfg, w, 40, prompts[b], steps)
        for i in range(steps + 1):
            assert np.abs(fused[i][0][b] - rl[i]).max() < TOL, f"sequence {b} step {i}"
            assert int(fused[i][1][b]) == rt[i], f"sequence {b} step {i}"
    c192 = pkg.ModelConfig.new(300, 192, 2, 2, 40)
    _, odd = _session(pkg, backend, c192, pkg.synthetic_weights(c192, 1), 40, 2)
    with pytest.raises(pkg.hip.InvalidArgument):
        odd.set_fused_norm(True)  # dim not a multiple of 128


@pytest.mark.parametrize("dim", [128, 256])
@pytest.mark.parametrize("mode", ["x6", "fp32_mfma", "kv16", "bf16"])
def test_ragged_prefill_matches_per_sequence(backend, pkg, ora, dim, mode):
    # InferenceSession::prefill takes any prompt length per session
    # (inference.rs:61-75).  One batched prefill of prompts of 57, 3, 130, 1
    # and 64 tokens (ragged query blocks; the longest spans two 128-query
    # blocks; head_dim 64 runs the key-split flash kernel, 128 the 128-query
    # one) gives each sequence what a one-sequence session gives, and, on
    # the fp32 paths, what the oracle gives; decode continues from each
    # sequence's own length.
    cfg = pkg.ModelConfig.new(300, dim, 2, 2, 160)
    w = pkg.synthetic_weights(cfg, seed=61)
    lens = [57, 3, 130, 1, 64]
    prompts = [pkg.synthetic_tokens(n, cfg.vocab_size, seed=62 + i) for i, n in enumerate(lens)]
    model = pkg.hip.Model(backend, cfg)
    model.upload(w)
    if mode == "fp32_mfma":
        model.set_prefill_split(pkg.hip.Model.SPLIT_NONE)
    if mode == "bf16":
        model.set_prefill_bf16(True)

    def session(n):
        s = pkg.hip.Session(model, 160, n)
        if mode == "kv16":
            s.set_kv_bf16(True)
        return s

    s = session(len(lens))
    got = [s.prefill(prompts)] + [s.decode_step(None) for _ in range(3)]
    assert list(s.cur_len()) == [n + 3 for n in lens]
    for b, n in enumerate(lens):
        one = session(1)
        alone = [one.prefill(prompts[b][None])] + [one.decode_step(None) for _ in range(3)]
        for i, ((lg, tk), (l1, t1)) in enumerate(zip(got, alone)):
            assert np.abs(lg[b] - l1[0]).max() < 1e-5, f"sequence {b} step {i}"
            assert int(tk[b]) == int(t1[0]), f"sequence {b} step {i}"
        one.close()
    np.testing.assert_array_equal(s.cache(1, 2, 0)[130 + 3:], 0)
    if mode in ("x6", "fp32_mfma"):
        refs = _oracle_greedy_many(ora, cfg, w, 160, prompts, 3)
        for b, (rl, rt) in enumerate(refs):
            for i in range(4):
                assert np.abs(got[i][0][b] - rl[i]).max() < TOL, f"sequence {b} step {i}"
                assert int(got[i][1][b]) == rt[i], f"sequence {b} step {i}"
    with pytest.raises(pkg.hip.EmptyPrompt):
        session(2).prefill([prompts[0], prompts[0][:0]])
    with pytest.raises(pkg.hip.PromptTooLong):
        session(2).prefill([prompts[0], np.zeros(161, np.uint32)])
    s.close()
    model.close()


@pytest.mark.parametrize("dim,heads", [(192, 2), (160, 4), (96, 4)])  # head_dim 96, 40, 24
def test_head_dim_not_power_of_two_matches_oracle(backend, pkg, ora, dim, heads):
    # The reference takes any head_dim dividing dim (config.rs:15-30;
    # FLASH_ATTENTION asserts head_dim <= 128, emit.rs:564-572).  Prefill
    # runs the flash kernel of the next power of two with the extra columns
    # zero; decode attention leaves the lanes past head_dim idle.
    cfg = pkg.ModelConfig.new(300, dim, heads, 2, 96)
    w = pkg.synthetic_weights(cfg, seed=71)
    B, S, steps = 3, 70, 4
    prompts = pkg.synthetic_tokens(B * S, cfg.vocab_size, seed=72).reshape(B, S)
    _, s = _session(pkg, backend, cfg, w, 96, B)
    got = _run(s, prompts, steps)
    refs = _oracle_greedy_many(ora, cfg, w, 96, list(prompts), steps)
    for b, (rl, rt) in enumerate(refs):
        for i in range(steps + 1):
            assert np.abs(got[i][0][b] - rl[i]).max() < TOL, f"sequence {b} step {i}"
            assert int(got[i][1][b]) == rt[i], f"sequence {b} step {i}"
    s.close()


def test_decode_greedy_matches_step_by_step(backend, pkg):
    cfg = pkg.ModelConfig.new(300, 128, 2, 2, 64)
    w = pkg.synthetic_weights(cfg, seed=9)
    prompts = pkg.synthetic_tokens(3 * 10, cfg.vocab_size, 10).reshape(3, 10)
    _, a = _session(pkg, backend, cfg, w, 64, 3)
    _, b = _session(pkg, backend, cfg, w, 64, 3)
    a.prefill(prompts)
    b.prefill(prompts)
    toks = a.decode_greedy(20)
    step = np.stack([b.decode_step(None)[1] for _ in range(20)])
    assert np.array_equal(toks, step)
    # Replaying a truncated window regenerates the same tokens.
    a.truncate(10)
    assert np.array_equal(a.decode_greedy(20), toks)


def test_set_len_keeps_rows(backend, pkg, ora):
    # Cache::cur_len is a public field (inference_graphs.rs:515): moving it
    # back and forth leaves the cached rows as they were.
    cfg = pkg.ModelConfig.new(97, 32, 4, 2, 16)
    w = pkg.synthetic_weights(cfg, seed=33)
    prompt = np.array([[3, 41, 7, 96, 0, 25], [11, 12, 13, 14, 15, 16]], np.uint32)
    _, s = _session(pkg, backend, cfg, w, 16, 2)
    s.prefill(prompt)
    s.set_len(2)
    assert list(s.cur_len()) == [2, 2]
    s.set_len(6)
    logits, _ = s.decode_step(np.array([9, 9], np.uint32))
    for b in range(2):
        o = ora.OracleSession(cfg, w, 16)
        o.prefill(prompt[b])
        assert np.abs(logits[b] - o.decode_step(9)).max() < TOL
        o.close()
    with pytest.raises(pkg.hip.InvalidArgument):
        s.set_len(17)


def test_session_errors(backend, pkg):
    h = pkg.hip
    cfg = pkg.ModelConfig.new(97, 32, 4, 2, 16)
    w = pkg.synthetic_weights(cfg, seed=1)
    _, s = _session(pkg, backend, cfg, w, 4, 2)
    with pytest.raises(h.EmptyPrompt):
        s.prefill(np.zeros((2, 0), np.uint32))
    with pytest.raises(h.PromptTooLong):
        s.prefill(np.zeros((2, 5), np.uint32))
    s.prefill(np.zeros((2, 3), np.uint32))
    with pytest.raises(h.CacheNotEmpty):
        s.prefill(np.zeros((2, 1), np.uint32))
    s.decode_step(None)
    with pytest.raises(h.ContextFull):
        s.decode_step(None)
    s.reset()
    s.prefill(np.zeros((2, 4), np.uint32))
    with pytest.raises(h.ContextFull):
        s.decode_step(None)
    with pytest.raises(h.InvalidArgument):
        h.Session(s.model, 16, 65)


def test_hall1_c1_greedy_parity(backend, pkg, ora):
    # Config 1: akasha-hall 1.0 fp32, weights N(0,0.02) seed 0,
    # 64-token prompt (seed 1), 64 greedy tokens, batch 1.
    cfg = pkg.ModelConfig.akasha_hall_1()
    w = pkg.synthetic_weights(cfg, seed=0)
    prompt = pkg.synthetic_tokens(64, cfg.vocab_size, seed=1)
    steps = 64
    ora.set_threads(16)
    try:
        o = ora.OracleSession(cfg, w, 512)
        ref = o.prefill(prompt)
        model, s = _session(pkg, backend, cfg, w, 512, 1)
        logits, nxt = s.prefill(prompt[None])
        worst = 0.0
        for i in range(steps):
            tok = ora.argmax(ref)
            worst = max(worst, float(np.abs(logits[0] - ref).max()))
            top2 = np.sort(ref)[-2:]
            assert int(nxt[0]) == tok, f"step {i}: margin {top2[1] - top2[0]}"
            if i + 1 < steps:
                ref = o.decode_step(tok)
                logits, nxt = s.decode_step(None)
        assert worst < TOL, worst
        o.close()
    finally:
        ora.set_threads(1)


def test_hall1_c4_batch_properties(backend, pkg, ora):
    # Config 4 at full size: 32 sequences prefilled with 448 tokens
    # (seed 4), then the 64 greedy decode steps at positions 448..511 that
    # fill the 512-row cache (the bench's workload).  Every sequence is
    # checked against the oracle over the whole run (identical tokens at
    # every step, logits within 1e-3); the batch is checked for batch
    # invariance against single-sequence sessions.
    cfg = pkg.ModelConfig.akasha_hall_1()
    w = pkg.synthetic_weights(cfg, seed=0)
    B, S, steps, inv_steps = 32, 448, 64, 4
    checked = list(range(B))
    toks = pkg.synthetic_tokens(B * S, cfg.vocab_size, seed=4).reshape(B, S)
    model, s = _session(pkg, backend, cfg, w, 512, B)
    logits, nxt = s.prefill(toks)
    all_l, all_t = [logits[checked]], [nxt]
    for _ in range(steps):
        logits, nxt = s.decode_step(None)
        all_l.append(logits[checked])
        all_t.append(nxt)
    # Batch invariance: sequence b alone gives the same results.
    for j, b in ((3, 3), (31, 31)):
        single = pkg.hip.Session(model, 512, 1)
        l1, t1 = single.prefill(toks[b][None])
        assert np.abs(l1[0] - all_l[0][j]).max() < 1e-4
        assert int(t1[0]) == int(all_t[0][b])
        for i in range(1, inv_steps + 1):
            l1, t1 = single.decode_step(None)
            assert np.abs(l1[0] - all_l[i][j]).max() < 1e-4
            assert int(t1[0]) == int(all_t[i][b])
        single.close()
    refs = _oracle_greedy_many(ora, cfg, w, 512, [toks[b] for b in checked], steps)
    for j, (b, (rl, rt)) in enumerate(zip(checked, refs)):
        for i in range(steps + 1):
            assert np.abs(all_l[i][j] - rl[i]).max() < TOL, f"sequence {b} step {i}"
            assert int(all_t[i][b]) == rt[i], f"sequence {b} step {i}"
    # The residual adds + RMSNorms folded into the GEMMs (five launches per
    # layer): the same 64 steps again from the prefilled caches.
    s.truncate(S)
    s.set_fused_norm(True)
    assert s.decode_launches() == 5 * cfg.num_layers + 4
    for i in range(1, steps + 1):
        logits, nxt = s.decode_step(None)
        assert np.array_equal(nxt, all_t[i]), f"fused norm, step {i}"
        for j, (b, (rl, rt)) in enumerate(zip(checked, refs)):
            assert np.abs(logits[b] - rl[i]).max() < TOL, f"fused norm, sequence {b} step {i}"
    s.set_fused_norm(False)
    assert s.decode_launches() == 7 * cfg.num_layers + 3
    # KV append landed at the right rows: the whole 512-row cache is filled.
    kc = s.cache(5, 7, 0)
    assert S + steps == 512 and np.all(np.abs(kc).sum(1) > 0)
    with pytest.raises(pkg.hip.ContextFull):
        s.decode_step(None)


def test_hall1_c3_prefill_sequence_matches_oracle(backend, pkg, ora):
    # Config 3 shape: 16 x 512 prefill (seed 3).  Every sequence is batch
    # invariant (prefilled alone in a one-sequence session: logits within
    # 1e-4, the same greedy token, the same cache rows); four sequences are
    # checked against the oracle (logits, token, layer 11's V cache).
    import threading
    cfg = pkg.ModelConfig.akasha_hall_1()
    w = pkg.synthetic_weights(cfg, seed=0)
    B, S = 16, 512
    toks = pkg.synthetic_tokens(B * S, cfg.vocab_size, seed=3).reshape(B, S)
    model, s = _session(pkg, backend, cfg, w, 512, B)
    logits, nxt = s.prefill(toks)
    single = pkg.hip.Session(model, 512, 1)
    for b in range(B):
        l1, t1 = single.prefill(toks[b][None])
        assert np.abs(l1[0] - logits[b]).max() < 1e-4, f"sequence {b} alone"
        assert int(t1[0]) == int(nxt[b]), f"sequence {b} alone"
        np.testing.assert_allclose(single.cache(7, 0, 0)[:S], s.cache(7, b, 0)[:S], atol=1e-5)
        single.reset()
    single.close()
    checked = (0, 5, 10, 15)
    refs = [None] * len(checked)

    def run(i):
        o = ora.OracleSession(cfg, w, 512)
        refs[i] = (o.prefill(toks[checked[i]]), o.v_cache(11)[:S].copy())
        o.close()

    ora.set_threads(4)
    try:
        ts = [threading.Thread(target=run, args=(i,)) for i in range(len(checked))]
        for t in ts:
            t.start()
        for t in ts:
            t.join()
    finally:
        ora.set_threads(1)
    for b, (ref, vref) in zip(checked, refs):
        assert np.abs(logits[b] - ref).max() < TOL, f"sequence {b}"
        assert int(nxt[b]) == ora.argmax(ref), f"sequence {b}"
        np.testing.assert_allclose(s.cache(11, b, 1)[:S], vref, atol=1e-3)


def test_head_dim_128_prefill_matches_oracle(backend, pkg, ora):
    # head_dim 128 (the scaled configuration's heads) over 300-token prompts:
    # several key blocks per query block and a ragged last query block.
    cfg = pkg.ModelConfig.new(300, 256, 2, 2, 320)
    w = pkg.synthetic_weights(cfg, seed=35)
    toks = pkg.synthetic_tokens(3 * 300, cfg.vocab_size, seed=36).reshape(3, 300)
    _, s = _session(pkg, backend, cfg, w, 320, 3)
    logits, nxt = s.prefill(toks)
    steps = [s.decode_step(None) for _ in range(2)]
    for b in range(3):
        o = ora.OracleSession(cfg, w, 320)
        ref = o.prefill(toks[b])
        assert np.abs(logits[b] - ref).max() < TOL and int(nxt[b]) == ora.argmax(ref)
        for lg, nx in steps:
            ref = o.decode_step(ora.argmax(ref))
            assert np.abs(lg[b] - ref).max() < TOL and int(nx[b]) == ora.argmax(ref)
        o.close()


def test_bf16_tiles_keep_fp32_accuracy(backend, pkg, ora):
    # Weights whose values are all bfloat16 are tiled in bfloat16 for decode:
    # the four matrices of each layer and, with dim > 1024, the lm_head.
    # Those GEMMs run bf16 MFMAs on A split exactly into
    # three bfloat16 terms, so every product is exact and only the summation
    # order differs from the float tiles: logits agree to fp32 rounding
    # (1e-4 here, against the 1e-3 oracle bar) with the same tokens, and each
    # setting is bit-reproducible.  Toggling the tiles after a decode graph
    # was captured also checks that the graph is rebuilt.
    cfg = pkg.ModelConfig.new(500, 1152, 9, 2, 40)
    w = pkg.synthetic_weights(cfg, seed=41, bf16=True)
    model, s = _session(pkg, backend, cfg, w, 40, 3)
    assert model.set_bf16_tiles(True) == 4 * cfg.num_layers + 1
    toks = pkg.synthetic_tokens(3 * 12, cfg.vocab_size, seed=42).reshape(3, 12)
    logits, nxt = s.prefill(toks)
    runs = {}
    for allow in (True, False, True):
        assert model.set_bf16_tiles(allow) == (4 * cfg.num_layers + 1 if allow else 0)
        s.truncate(12)
        feed, out = nxt, []
        for _ in range(4):
            lg, feed = s.decode_step(feed)
            out.append((lg.copy(), feed.copy()))
        if allow in runs:
            for (a, ta), (b, tb) in zip(runs[allow], out):
                assert np.array_equal(a, b) and np.array_equal(ta, tb)
        runs[allow] = out
    for (a, ta), (b, tb) in zip(runs[True], runs[False]):
        assert np.abs(a - b).max() < 1e-4 and np.array_equal(ta, tb)
    o = ora.OracleSession(cfg, w, 40)
    ref = o.prefill(toks[1])
    assert np.abs(logits[1] - ref).max() < TOL
    for lg, _ in runs[True]:
        ref = o.decode_step(ora.argmax(ref))
        assert np.abs(lg[1] - ref).max() < TOL
    o.close()
    # A matrix with one value off the bfloat16 grid goes back to float tiles.
    w2 = list(w)
    w2[2] = w[2].copy()
    w2[2].flat[7] = np.nextafter(w2[2].flat[7], np.float32(1))
    model.upload(w2)
    assert model.set_bf16_tiles(True) == 4 * cfg.num_layers


def test_take_and_replace_cache_move_a_sequence(backend, pkg, ora):
    # take_cache / replace_cache (inference.rs:42-59) and NoCache (:72, :180).
    hip = pkg.hip
    cfg = pkg.ModelConfig.new(97, 32, 4, 2, 16)
    w = pkg.synthetic_weights(cfg, seed=31)
    prompt = np.array([[3, 41, 7, 96, 0, 25], [11, 12, 13, 14, 15, 16]], np.uint32)
    model, a = _session(pkg, backend, cfg, w, 16, 2)
    a.prefill(prompt)
    _, nxt = a.decode_step(None)
    k, v, n = a.take_cache(1)
    assert n == 7 and a.take_cache(1) is None
    with pytest.raises(hip.NoCache):
        a.decode_step(None)
    with pytest.raises(hip.NoCache):
        a.decode_greedy(1)
    # Sequence 1 continues in another session's slot 0.
    b = hip.Session(model, 16, 2)
    b.replace_cache(0, k, v, n)
    assert list(b.cur_len()) == [7, 0]
    logits, _ = b.decode_step(np.array([nxt[1], 5], np.uint32))
    o = ora.OracleSession(cfg, w, 16)
    first = o.prefill(prompt[1])
    o.decode_step(ora.argmax(first))
    want = o.decode_step(int(nxt[1]))
    o.close()
    assert np.abs(logits[0] - want).max() < TOL
    # Back into its own slot, sequence 1 decodes again in session a.
    a.replace_cache(1, k, v, n)
    a.decode_step(np.array([nxt[0], nxt[1]], np.uint32))
    assert list(a.cur_len()) == [8, 8]
    with pytest.raises(hip.InvalidArgument):
        a.replace_cache(0, k, v, 17)


def test_scaled_config_long_prompts_match_oracle(backend, pkg, ora):
    # Config 5 architecture with prompts long enough for several head-128
    # key blocks and two query blocks of the prefill's flash attention at
    # d = 2048: a ragged batch of 256 and 160 tokens (seed 8), then 3 greedy
    # steps, both sequences against the oracle (run side by side on the
    # host's threads).
    import threading
    cfg = pkg.ModelConfig.scaled()
    w = pkg.synthetic_weights(cfg, seed=5, bf16=True)
    r = np.random.default_rng(8)
    prompts = [r.integers(0, cfg.vocab_size, size=n).astype(np.uint32) for n in (256, 160)]
    model, s = _session(pkg, backend, cfg, w, 264, 2)
    logits, nxt = s.prefill(prompts)
    got = [(logits, nxt)] + [s.decode_step(None) for _ in range(3)]
    s.close()
    model.close()
    refs = [None, None]

    def run(b):
        refs[b] = _oracle_greedy(ora, cfg, w, 264, prompts[b], 3)

    ora.set_threads(8)
    try:
        ts = [threading.Thread(target=run, args=(b,)) for b in range(2)]
        for t in ts:
            t.start()
        for t in ts:
            t.join()
    finally:
        ora.set_threads(1)
    for b in range(2):
        rl, rt = refs[b]
        for i in range(4):
            assert np.abs(got[i][0][b] - rl[i]).max() < TOL, f"sequence {b} step {i}"
            assert int(got[i][1][b]) == rt[i], f"sequence {b} step {i}"
    del w


def test_scaled_config_matches_oracle(backend, pkg, ora):
    # Config 5 architecture: dim 2048, 24 layers, 16 heads x 128, FFN 8192,
    # vocab 50257, bf16-valued weights N(0,0.02) from seed 5.  Two sequences
    # with 24-token prompts (seed 6) and 3 greedy steps against the oracle
    # (a 2048-token prompt is beyond the CPU oracle's budget here).
    cfg = pkg.ModelConfig.scaled()
    w = pkg.synthetic_weights(cfg, seed=5, bf16=True)
    prompt = pkg.synthetic_tokens(2 * 24, cfg.vocab_size, seed=6).reshape(2, 24)
    model, s = _session(pkg, backend, cfg, w, 64, 2)
    logits, nxt = s.prefill(prompt)
    steps = [(logits, nxt)]
    for _ in range(3):
        steps.append(s.decode_step(None))
    ora.set_threads(16)
    try:
        for b in range(2):
            o = ora.OracleSession(cfg, w, 64)
            ref = o.prefill(prompt[b])
            for i, (lg, nx) in enumerate(steps):
                if i:
                    ref = o.decode_step(ora.argmax(ref))
                assert np.abs(lg[b] - ref).max() < TOL, f"sequence {b} step {i}"
                assert int(nx[b]) == ora.argmax(ref), f"sequence {b} step {i}"
            o.close()
    finally:
        ora.set_threads(1)
    del w


@pytest.mark.parametrize("kind", ["h3", "x6"])
def test_prefill_split_matches_fp32_mfma_and_oracle(backend, pkg, ora, kind):
    # The split prefill GEMMs (h3, the default: fp16 MFMAs on operands split
    # into two fp16 terms, three products; x6: bf16 MFMAs on three bfloat16
    # terms, six products) against the fp32-MFMA GEMMs (SPLIT_NONE) and the
    # oracle: both meet the fp32 bar, agree with each other to fp32 rounding
    # (1e-4) with the same tokens, and switching back reproduces the first
    # run bit for bit.  The split run differs from the fp32 one in its last
    # bits (no silent fallback to the fp32 kernels).  dim 256, head_dim 64,
    # ffn 1024: ragged tiles at M = 3 x 70 rows.
    M = pkg.hip.Model
    cfg = pkg.ModelConfig.new(300, 256, 4, 2, 80)
    w = pkg.synthetic_weights(cfg, seed=61)
    model, s = _session(pkg, backend, cfg, w, 80, 3)
    assert model.prefill_split() == M.SPLIT_H3
    split = M.SPLIT_H3 if kind == "h3" else M.SPLIT_X6
    model.set_prefill_split(split)
    toks = pkg.synthetic_tokens(3 * 70, cfg.vocab_size, seed=62).reshape(3, 70)
    lx, nx = s.prefill(toks)
    kx = s.cache(1, 2, 0)[:70].copy()
    model.set_prefill_split(M.SPLIT_NONE)
    s.reset()
    lf, nf = s.prefill(toks)
    assert np.abs(lx - lf).max() < 1e-4 and np.array_equal(nx, nf)
    assert not np.array_equal(lx, lf)
    np.testing.assert_allclose(kx, s.cache(1, 2, 0)[:70], atol=1e-5)
    model.set_prefill_split(split)
    s.reset()
    lx2, nx2 = s.prefill(toks)
    assert np.array_equal(lx, lx2) and np.array_equal(nx, nx2)
    for b in (0, 2):
        o = ora.OracleSession(cfg, w, 80)
        ref = o.prefill(toks[b])
        o.close()
        for got, nxt in ((lx, nx), (lf, nf)):
            assert np.abs(got[b] - ref).max() < TOL
            assert int(nxt[b]) == ora.argmax(ref)
    model.set_prefill_split(M.SPLIT_H3)


@pytest.mark.parametrize("where", ["activation", "weight", "value"])
def test_prefill_h3_out_of_fp16_range_reruns_in_fp32(backend, pkg, where):
    # An operand of the split-fp16 kernels beyond fp16's range (|x| >= 65520)
    # turns into an infinite hi term; the kernels flag the non-finite results
    # and the prefill is recomputed on the fp32 kernels, so its logits,
    # tokens and cache equal the fp32-MFMA prefill's bit for bit.
    # "activation": norm gains of 1e5 put the QKV and ffn_up inputs far
    # beyond 65520; "weight": one ffn_up weight of 1e5; "value": layer 0's V
    # weights scaled to N(0, 5000), so V (~1e5) overflows in the flash
    # attention and in out_proj's input while every GEMM weight and input
    # before it stays in range.
    M = pkg.hip.Model
    cfg = pkg.ModelConfig.new(300, 256, 4, 2, 80)
    w = pkg.synthetic_weights(cfg, seed=63)
    if where == "activation":
        w[1 + 6 * 1 + 0] = w[1 + 6 * 1 + 0] * 1e5  # layer 1 norm1 gain
    elif where == "weight":
        up = w[1 + 6 * 0 + 4].copy()
        up.flat[12345] = 1e5
        w[1 + 6 * 0 + 4] = up
    else:
        qkv = w[1 + 6 * 0 + 1].copy()  # [dim, 3 dim]: columns [2 dim, 3 dim) are V
        qkv[:, 2 * cfg.dim:] *= np.float32(5000 / 0.02)
        w[1 + 6 * 0 + 1] = qkv
    model, s = _session(pkg, backend, cfg, w, 80, 3)
    assert model.prefill_split() == M.SPLIT_H3
    toks = pkg.synthetic_tokens(3 * 70, cfg.vocab_size, seed=64).reshape(3, 70)
    lh, nh = s.prefill(toks)
    kh = s.cache(1, 2, 0)[:70].copy()
    assert np.isfinite(lh).all()
    model.set_prefill_split(M.SPLIT_NONE)
    s.reset()
    lf, nf = s.prefill(toks)
    assert np.array_equal(lh, lf) and np.array_equal(nh, nf)
    assert np.array_equal(kh, s.cache(1, 2, 0)[:70])
    # The trainer forward reruns the same way.
    model.set_prefill_split(M.SPLIT_H3)
    tg = np.roll(toks, -1, axis=1)
    f = pkg.hip.Forward(model, 3, 70)
    mh, lsh = f.loss(toks, tg)
    model.set_prefill_split(M.SPLIT_NONE)
    mf, lsf = f.loss(toks, tg)
    assert np.array_equal(lsh, lsf) and mh == mf
    f.close()


def test_greedy_tokens_with_nan_first_logit(backend, pkg, ora):
    # lm_head column 0 set to NaN makes every row's logit 0 NaN.  The
    # reference's argmax (sampling.rs:83-91) starts from index 0 and a NaN
    # there never loses a comparison, so prefill, decode steps, greedy
    # replays and temperature-0 generate all pick token 0, as the oracle does.
    cfg = pkg.ModelConfig.new(300, 128, 2, 2, 40)
    L = cfg.num_layers
    w = pkg.synthetic_weights(cfg, seed=67)
    lm = w[2 + 6 * L].copy()
    lm[:, 0] = np.nan
    w[2 + 6 * L] = lm
    model, s = _session(pkg, backend, cfg, w, 40, 3)
    toks = pkg.synthetic_tokens(3 * 10, cfg.vocab_size, seed=68).reshape(3, 10)
    logits, nxt = s.prefill(toks)
    assert np.isnan(logits[:, 0]).all() and np.isfinite(logits[:, 1:]).all()
    o = ora.OracleSession(cfg, w, 40)
    assert ora.argmax(o.prefill(toks[0])) == 0
    o.close()
    assert list(nxt) == [0, 0, 0]
    _, nxt = s.decode_step(None)
    assert list(nxt) == [0, 0, 0]
    assert (s.decode_greedy(2) == 0).all()
    s.reset()
    outs = s.generate(toks, 3)
    assert all(list(x) == [0, 0, 0] for x in outs)
    s.close()
    model.close()


def test_forward_bf16_layers_lm_head_out_of_fp16_range_reruns(backend, pkg):
    # Under the bf16-MFMA layers the trainer forward's lm_head still runs the
    # split-fp16 GEMM on the model's fp16 copy.  One lm_head weight of 1e5
    # (beyond fp16's range) must flag and rerun it in fp32: the losses are
    # finite and equal, bit for bit, to the forward whose lm_head runs on the
    # fp32 MFMAs from the start (SPLIT_NONE; the bf16 layers are the same).
    M = pkg.hip.Model
    cfg = pkg.ModelConfig.new(300, 256, 4, 2, 80)
    L = cfg.num_layers
    w = pkg.synthetic_weights(cfg, seed=65)
    lm = w[2 + 6 * L].copy()
    lm.flat[4321] = 1e5
    w[2 + 6 * L] = lm
    model = M(backend, cfg)
    model.upload(w)
    assert model.prefill_split() == M.SPLIT_H3
    model.set_prefill_bf16(True)
    toks = pkg.synthetic_tokens(2 * 40, cfg.vocab_size, seed=66).reshape(2, 40)
    tg = np.roll(toks, -1, axis=1)
    f = pkg.hip.Forward(model, 2, 40)
    mh, lsh = f.loss(toks, tg)
    assert np.isfinite(lsh).all()
    model.set_prefill_split(M.SPLIT_NONE)
    mf, lsf = f.loss(toks, tg)
    assert np.array_equal(lsh, lsf) and mh == mf
    f.close()
    model.close()


@pytest.mark.parametrize("case", ["plain", "scaled_rows", "weight_beyond_fp16", "two_row_tiles",
                                  "two_row_tiles_dim384"])
def test_lm_head_split_tiles_match_oracle(backend, pkg, ora, case):
    # The persistent lm_head reads its weights as two fp16 terms (three
    # fp16 products per multiply-add).  "scaled_rows": final-norm gains of
    # 4e4 put the normed rows beyond 2^15, so the kernel scales them by a
    # power of two and back; "weight_beyond_fp16": one lm_head weight of 1e5
    # keeps that matrix on float tiles; "two_row_tiles": 40 sequences, also at
    # dim 384 (tiles of 768 k, the kernel's other size).
    # Prefill and greedy decode against the oracle, logits within 1e-3 plus
    # 2e-6 of their magnitude, tokens identical.
    dim, heads = (384, 3) if case == "two_row_tiles_dim384" else (128, 2)
    cfg = pkg.ModelConfig.new(300, dim, heads, 2, 24)
    L = cfg.num_layers
    w = pkg.synthetic_weights(cfg, seed=71)
    if case == "scaled_rows":
        w[1 + 6 * L] = w[1 + 6 * L] * np.float32(4e4)
    elif case == "weight_beyond_fp16":
        lm = w[2 + 6 * L].copy()
        lm.flat[777] = 1e5
        w[2 + 6 * L] = lm
    B, P, steps = (40 if case.startswith("two_row_tiles") else 3), 8, 3
    toks = pkg.synthetic_tokens(B * P, cfg.vocab_size, seed=72).reshape(B, P)
    model, s = _session(pkg, backend, cfg, w, 24, B)
    got = [s.prefill(toks)] + [s.decode_step(None) for _ in range(steps)]
    for b in sorted({0, B - 1}):
        o = ora.OracleSession(cfg, w, 24)
        ref = o.prefill(toks[b])
        for i in range(steps + 1):
            if i:
                ref = o.decode_step(ora.argmax(ref))
            tol = 1e-3 + 2e-6 * float(np.abs(ref).max())
            assert np.abs(got[i][0][b] - ref).max() < tol, f"{case}: sequence {b} step {i}"
            assert int(got[i][1][b]) == ora.argmax(ref), f"{case}: sequence {b} step {i}"
        o.close()
    if case == "scaled_rows":
        assert np.abs(got[0][0]).max() > 100.0  # the rows really were large


def test_decode_kernel_timers(backend, pkg):
    # akh_session_time_decode_attn (events carried by the dispatches) and
    # the back-to-back timer measure the same kernel: both positive and
    # within a small factor of each other (on a kernel this short the
    # dispatch-carried events can read longer than back-to-back launches);
    # both reject bad arguments.
    cfg = pkg.ModelConfig.new(97, 64, 4, 2, 64)
    w = pkg.synthetic_weights(cfg, seed=71)
    _, s = _session(pkg, backend, cfg, w, 64, 4)
    s.prefill(pkg.synthetic_tokens(4 * 20, cfg.vocab_size, seed=72).reshape(4, 20),
              want_logits=False)
    one = s.time_decode_attn(64)
    b2b = s.time_decode_kernel(0, 64)
    assert one > 0 and b2b > 0 and 0.25 < one / b2b < 4
    with pytest.raises(pkg.hip.InvalidArgument):
        s.time_decode_attn(0)
    with pytest.raises(pkg.hip.InvalidArgument):
        s.time_decode_kernel(7, 4)
