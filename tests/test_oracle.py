"""Pins the CPU oracle (oracle/akasha_oracle.c) before it is trusted.

Each oracle function is checked against something other than its own
formula: a library routine (numpy / scipy in float64), a closed form or
invariant of the mathematics, brute force on tiny inputs, or the
reference's own known-answer tests restated (akasha-core has no committed
golden vectors; its tests generate inputs with the LCG of
src/nn/ops/emit.rs:910-921 and compare against in-test CPU formulas).  The
checks are chosen so that a dropped term, wrong sign, wrong index or
transposed operand fails at least one of them.
"""

import numpy as np
import pytest
from scipy.special import softmax as sp_softmax


def lcg_rand_vec_py(n, seed):
    """emit.rs:910-921 in plain integer arithmetic (independent of C)."""
    mask = (1 << 64) - 1
    state = (seed + 0x9E3779B97F4A7C15) & mask
    out = []
    for _ in range(n):
        state = (state * 6364136223846793005 + 1442695040888963407) & mask
        bits = (state >> 40) & 0xFFFFFF
        out.append(np.float32(np.float32(bits) / np.float32(0xFFFFFF)) * np.float32(2) - np.float32(1))
    return np.array(out, np.float32)


def test_rand_vec_matches_integer_lcg(ora):
    for seed in (0, 1, 4, 42):
        got = ora.rand_vec(257, seed)
        assert np.array_equal(got, lcg_rand_vec_py(257, seed))
    v = ora.rand_vec(100000, 7)
    assert v.min() >= -1.0 and v.max() <= 1.0
    assert abs(float(v.mean())) < 0.01  # uniform on [-1, 1]
    assert abs(float(v.var()) - 1.0 / 3.0) < 0.01


def test_rand_tokens_range_and_lcg(ora):
    t = ora.rand_tokens(1000, 97, 100)
    assert t.max() < 97
    mask = (1 << 64) - 1
    state = (100 + 0x9E3779B97F4A7C15) & mask
    ref = []
    for _ in range(1000):
        state = (state * 6364136223846793005 + 1442695040888963407) & mask
        ref.append((state >> 33) % 97)
    assert np.array_equal(t, np.array(ref, np.uint32))


def test_embedding_gathers_rows_and_zeroes_out_of_vocab(ora):
    vocab, dim = 11, 6
    table = ora.rand_vec(vocab * dim, 3)
    toks = np.array([0, 10, 11, 5, 4294967295, 3], np.uint32)
    out = ora.embedding(toks, table, vocab, dim, len(toks)).reshape(-1, dim)
    t = table.reshape(vocab, dim)
    for i, tok in enumerate(toks):
        if tok < vocab:
            assert np.array_equal(out[i], t[tok])
        else:
            assert np.all(out[i] == 0)


def test_rmsnorm_against_float64_and_scale_invariance(ora):
    rows, size, eps = 5, 96, 1e-5
    x = ora.rand_vec(rows * size, 9) * 3
    w = 1 + ora.rand_vec(size, 10) * 0.1
    got = ora.rmsnorm(x, w, rows, size, eps).reshape(rows, size)
    xd = x.reshape(rows, size).astype(np.float64)
    ref = xd / np.sqrt((xd ** 2).mean(axis=1, keepdims=True) + eps) * w
    np.testing.assert_allclose(got, ref, rtol=2e-6, atol=2e-6)
    # RMSNorm is invariant to scaling its input (eps negligible here).
    got2 = ora.rmsnorm(x * 8, w, rows, size, eps).reshape(rows, size)
    np.testing.assert_allclose(got2, got, rtol=1e-5, atol=1e-6)


def test_matmul_layout_and_sequential_fold(ora):
    # emit.rs:1424-1465 shapes: n=301, k=19, B stored [k, n].
    m, n, k = 3, 301, 19
    a = ora.rand_vec(m * k, 10)
    b = ora.rand_vec(k * n, 20)
    c0 = ora.rand_vec(m * n, 30)
    got = ora.matmul(a, b, m, n, k).reshape(m, n)
    ref = a.reshape(m, k).astype(np.float64) @ b.reshape(k, n).astype(np.float64)
    np.testing.assert_allclose(got, ref, atol=1e-5)
    # A transposed operand would fail this (non-square shapes).
    bad = (b.reshape(n, k).astype(np.float64).T)
    assert np.abs(a.reshape(m, k) @ bad - got).max() > 1e-2
    # Bit-exact against a float32 k-ascending left fold.
    fold = np.zeros((m, n), np.float32)
    A, B = a.reshape(m, k), b.reshape(k, n)
    for kk in range(k):
        fold = (fold + A[:, kk:kk + 1] * B[kk][None, :]).astype(np.float32)
    assert np.array_equal(got, fold)
    got_add = ora.matmul_add(a, b, c0, m, n, k).reshape(m, n)
    np.testing.assert_allclose(got_add, c0.reshape(m, n) + ref, atol=1e-5)


def test_head_gather_slices_qkv(ora):
    seq, dim = 37, 12
    src = ora.rand_vec(seq * 3 * dim, 50).reshape(seq, 3 * dim)
    for role in range(3):
        got = ora.head_gather(src.ravel(), seq, 3 * dim, dim, role * dim).reshape(seq, dim)
        assert np.array_equal(got, src[:, role * dim:(role + 1) * dim])


def _rope_ref64(x, seq, dim, hd, pos0):
    x = x.reshape(seq, dim).astype(np.float64).copy()
    out = x.copy()
    for t in range(seq):
        for h in range(dim // hd):
            for i in range(0, hd, 2):
                theta = (t + pos0) * 10000.0 ** (-i / hd)
                z = complex(x[t, h * hd + i], x[t, h * hd + i + 1]) * complex(np.cos(theta), np.sin(theta))
                out[t, h * hd + i], out[t, h * hd + i + 1] = z.real, z.imag
    return out


@pytest.mark.parametrize("seq,dim,hd", [(8, 8, 4), (37, 12, 4), (65, 48, 16)])
def test_rope_is_complex_rotation(ora, seq, dim, hd):
    # Shapes of rope_qk_matches_two_rope_calls (emit.rs:1126-1130).
    x = ora.rand_vec(seq * dim, 10)
    got = ora.rope(x, seq, dim, hd).reshape(seq, dim)
    ref = _rope_ref64(x, seq, dim, hd, 0)
    # f32 angle rounding at t ~ 64 rad bounds the error near 1e-5.
    np.testing.assert_allclose(got, ref, atol=5e-5)
    # Position 0 is the identity; rotations keep pair norms.
    assert np.array_equal(got[0], x.reshape(seq, dim)[0])
    pn = lambda a: np.hypot(a[:, 0::2], a[:, 1::2])  # noqa: E731
    np.testing.assert_allclose(pn(got), pn(x.reshape(seq, dim)), rtol=1e-5)


def test_rope_offset_equals_rope_at_shifted_rows(ora):
    seq, dim, hd = 20, 16, 8
    x = ora.rand_vec(seq * dim, 33)
    full = ora.rope(x, seq, dim, hd).reshape(seq, dim)
    for pos in (0, 1, 7, 19):
        row = ora.rope_offset(x.reshape(seq, dim)[pos], 1, dim, hd, pos)
        assert np.array_equal(row, full[pos])


def test_cache_write_places_rows(ora):
    src = ora.rand_vec(3 * 8, 1)
    dst = ora.rand_vec(10 * 8, 2)
    got = ora.cache_write(src, dst, 3, 8, 4).reshape(10, 8)
    exp = dst.reshape(10, 8).copy()
    exp[4:7] = src.reshape(3, 8)
    assert np.array_equal(got, exp)


def test_softmax_rect_matches_scipy(ora):
    rows, width, scale = 3, 33, 0.125
    x = ora.rand_vec(rows * width, 5) * 10
    got = ora.softmax_rect(x, rows, width, scale).reshape(rows, width)
    ref = sp_softmax(x.reshape(rows, width).astype(np.float64) * scale, axis=1)
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-7)
    np.testing.assert_allclose(got.sum(axis=1), 1.0, atol=1e-6)


def test_silu_closed_form(ora):
    x = np.linspace(-20, 20, 1001).astype(np.float32)
    got = ora.silu(x)
    ref = x.astype(np.float64) / (1 + np.exp(-x.astype(np.float64)))
    np.testing.assert_allclose(got, ref, rtol=1e-6, atol=1e-7)
    assert got[500] == 0.0


def _attn_ref64(q, k, v, seq, dim, hd):
    q, k, v = (a.reshape(seq, dim).astype(np.float64) for a in (q, k, v))
    out = np.zeros((seq, dim))
    for h in range(dim // hd):
        sl = slice(h * hd, (h + 1) * hd)
        s = q[:, sl] @ k[:, sl].T / np.sqrt(hd)
        s[np.triu_indices(seq, 1)] = -np.inf
        out[:, sl] = sp_softmax(s, axis=1) @ v[:, sl]
    return out


@pytest.mark.parametrize("seq,heads,hd", [(8, 2, 4), (37, 3, 16), (65, 12, 64)])
def test_causal_attention_brute_force(ora, seq, heads, hd):
    # Shapes and seeds of flash_attention_matches_cpu_reference
    # (emit.rs:1001-1006, 1036-1039).
    dim = heads * hd
    n = seq * dim
    q, k, v = ora.rand_vec(n, 1), ora.rand_vec(n, 2), ora.rand_vec(n, 3)
    got = ora.causal_attention(q, k, v, seq, dim, hd).reshape(seq, dim)
    np.testing.assert_allclose(got, _attn_ref64(q, k, v, seq, dim, hd), atol=2e-6)
    # Row 0 attends only to key 0: output is V row 0 exactly per head.
    assert np.allclose(got[0], v.reshape(seq, dim)[0], atol=1e-7)


@pytest.mark.parametrize("attn_len,heads,hd", [(1, 2, 4), (5, 3, 16), (33, 12, 64)])
def test_cached_attention_equals_causal_row(ora, attn_len, heads, hd):
    # cached_attention_matches_cpu_reference shapes (emit.rs:1332-1337): the
    # 3-kernel decode attention on a cache must equal the last row of causal
    # attention over the same keys.
    dim, max_ctx = heads * hd, 64
    q = ora.rand_vec(dim, 1)
    kc = ora.rand_vec(max_ctx * dim, 2)
    vc = ora.rand_vec(max_ctx * dim, 3)
    sc = ora.attn_qk_cached(q, kc, attn_len, dim, hd)
    p = ora.softmax_rect(sc, heads, attn_len, np.float32(1.0 / np.sqrt(hd)))
    got = ora.attn_av_cached(p, vc, attn_len, dim, hd)
    qs = np.zeros((attn_len, dim), np.float32)
    qs[-1] = q
    full = _attn_ref64(qs, kc[:attn_len * dim], vc[:attn_len * dim], attn_len, dim, hd)
    np.testing.assert_allclose(got, full[-1], atol=1e-6)


def test_argmax_known_answers(ora):
    # sampling.rs:97-103: LOGITS = [1, 4, 2, 8, 3] -> 3.
    assert ora.argmax(np.array([1, 4, 2, 8, 3], np.float32)) == 3
    # First index of the maximum on ties (strict >, sampling.rs:86).
    assert ora.argmax(np.array([1, 8, 2, 8, 3], np.float32)) == 1
    x = np.random.default_rng(0).standard_normal(50257).astype(np.float32)
    assert ora.argmax(x) == int(np.argmax(x))


# ---- session-level invariants (tiny configs, pure CPU) -------------------

def _tiny(pkg, seed=42, cfg=None):
    cfg = cfg or pkg.ModelConfig.new(97, 32, 4, 2, 16)
    return cfg, pkg.synthetic_weights(cfg, seed=seed)


def test_prefill_matches_sequential_decode(pkg, ora):
    # inference.rs:334-359: ModelConfig::new(97,32,4,2,16), prompt
    # [3,41,7,96,0,25], tolerance 1e-3.
    cfg, w = _tiny(pkg)
    prompt = np.array([3, 41, 7, 96, 0, 25], np.uint32)
    a = ora.OracleSession(cfg, w, 16)
    pre = a.prefill(prompt)
    b = ora.OracleSession(cfg, w, 16)
    for t in prompt:
        dec = b.decode_step(t)
    assert np.abs(pre - dec).max() < 1e-3
    # Caches written by both paths agree too.
    for layer in range(cfg.num_layers):
        np.testing.assert_allclose(a.k_cache(layer), b.k_cache(layer), atol=1e-5)
        np.testing.assert_allclose(a.v_cache(layer), b.v_cache(layer), atol=1e-5)


def test_kv_decode_matches_naive_forward(pkg, ora):
    # diagnose.rs:675-743 (CHECK 9): decode with the KV cache equals a fresh
    # full forward of every prefix.
    cfg = pkg.ModelConfig.new(64, 64, 4, 2, 16)
    w = pkg.synthetic_weights(cfg, seed=3)
    seq = ora.rand_tokens(14, 64, 5)
    s = ora.OracleSession(cfg, w, 16)
    logits = [s.prefill(seq[:4])]
    for t in seq[4:-1]:
        logits.append(s.decode_step(t))
    for i, cur in enumerate(range(4, 14)):
        fresh = ora.OracleSession(cfg, w, 16)
        naive = fresh.prefill(seq[:cur])
        assert np.abs(naive - logits[i]).max() < 1e-3
        fresh.close()


def _forward64(cfg, w, tokens):
    """Whole-model forward in float64 with numpy (an implementation that
    shares no code with the oracle), returning last-row logits."""
    d, hd, L = cfg.dim, cfg.head_dim, cfg.num_layers
    W = [np.asarray(a, np.float64) for a in w]
    x = W[0][np.asarray(tokens)]
    S = len(tokens)

    def norm(x, g):
        return x / np.sqrt((x ** 2).mean(axis=1, keepdims=True) + cfg.norm_eps) * g

    ang = np.arange(S)[:, None] * (10000.0 ** (-np.arange(0, hd, 2) / hd))[None, :]
    rot = np.exp(1j * ang)

    def rope(a):
        a = a.reshape(S, d // hd, hd // 2, 2)
        z = (a[..., 0] + 1j * a[..., 1]) * rot[:, None, :]
        return np.stack([z.real, z.imag], -1).reshape(S, d)

    for l in range(L):
        n1, qkv, wo, n2, up, down = W[1 + 6 * l:7 + 6 * l]
        h = norm(x, n1) @ qkv
        q, k, v = rope(h[:, :d]), rope(h[:, d:2 * d]), h[:, 2 * d:]
        att = np.zeros((S, d))
        for hh in range(d // hd):
            sl = slice(hh * hd, (hh + 1) * hd)
            s = q[:, sl] @ k[:, sl].T / np.sqrt(hd)
            s[np.triu_indices(S, 1)] = -np.inf
            att[:, sl] = sp_softmax(s, axis=1) @ v[:, sl]
        x = x + att @ wo
        u = norm(x, n2) @ up
        x = x + (u / (1 + np.exp(-u))) @ down
    return norm(x[-1:], W[1 + 6 * L])[0] @ W[2 + 6 * L]


def test_oracle_forward_matches_float64_numpy(pkg, ora):
    cfg, w = _tiny(pkg, seed=7, cfg=pkg.ModelConfig.new(97, 64, 2, 2, 32))
    toks = ora.rand_tokens(20, 97, 9)
    s = ora.OracleSession(cfg, w, 32)
    got = s.prefill(toks)
    np.testing.assert_allclose(got, _forward64(cfg, w, toks), atol=2e-5)


def test_golden_fixture(pkg, ora):
    """tests/golden/tiny_greedy.npz: float64-numpy logits and greedy tokens
    of a tiny model (made by tests/golden/make_golden.py)."""
    from pathlib import Path
    g = np.load(Path(__file__).parent / "golden" / "tiny_greedy.npz")
    cfg = pkg.ModelConfig.new(*[int(v) for v in g["cfg"]])
    w = pkg.synthetic_weights(cfg, seed=int(g["seed"]))
    s = ora.OracleSession(cfg, w, int(g["max_ctx"]))
    logits = s.prefill(g["prompt"])
    toks = []
    for i in range(len(g["tokens"])):
        np.testing.assert_allclose(logits, g["logits"][i], atol=5e-5)
        t = ora.argmax(logits)
        toks.append(t)
        if i + 1 < len(g["tokens"]):
            logits = s.decode_step(t)
    assert toks == [int(t) for t in g["tokens"]]


def test_session_errors(pkg, ora):
    cfg, w = _tiny(pkg)
    lib = ora.load()
    s = ora.OracleSession(cfg, w, 4)
    out = np.empty(cfg.vocab_size, np.float32)
    assert lib.ora_session_prefill(s.h, np.zeros(1, np.uint32), 0, out) == 1  # EmptyPrompt
    assert lib.ora_session_prefill(s.h, np.zeros(5, np.uint32), 5, out) == 2  # PromptTooLong
    assert lib.ora_session_prefill(s.h, np.zeros(4, np.uint32), 4, out) == 0
    assert lib.ora_session_prefill(s.h, np.zeros(1, np.uint32), 1, out) == 5  # CacheNotEmpty
    assert lib.ora_session_decode_step(s.h, 1, out) == 3  # ContextFull


def test_matmul_threads_do_not_change_results(ora):
    m, n, k = 2, 1000, 300
    a, b = ora.rand_vec(m * k, 1), ora.rand_vec(k * n, 2)
    ora.set_threads(1)
    r1 = ora.matmul(a, b, m, n, k)
    ora.set_threads(4)
    r4 = ora.matmul(a, b, m, n, k)
    ora.set_threads(1)
    assert np.array_equal(r1, r4)


# ---- the trainer's forward (src/nn/train.rs:256-275) ----------------------

def test_qkv_split_slices_columns(ora):
    rows, d = 5, 12
    src = ora.rand_vec(rows * 3 * d, 3).reshape(rows, 3 * d)
    q, k, v = ora.qkv_split(src, rows, 3 * d, d)
    for i, part in enumerate((q, k, v)):
        assert np.array_equal(part.reshape(rows, d), src[:, i * d:(i + 1) * d])


def test_rope_qk_is_rope_at_local_positions(ora):
    S, d, hd, off = 6, 16, 8, 4
    q, k = ora.rand_vec((off + S + 2) * d, 4), ora.rand_vec((off + S + 2) * d, 5)
    rq, rk = ora.rope_qk(q, k, S, d, hd, off)
    for x, rx in ((q, rq), (k, rk)):
        x, rx = x.reshape(-1, d), rx.reshape(-1, d)
        # rows of the window rotate as rope's rows 0.. do; the others stay
        np.testing.assert_array_equal(rx[off:off + S], ora.rope(x[off:off + S], S, d, hd).reshape(S, d))
        np.testing.assert_array_equal(rx[:off], x[:off])
        np.testing.assert_array_equal(rx[off + S:], x[off + S:])


def test_add_residual_add_silu_out_closed_forms(ora):
    a, b = ora.rand_vec(300, 6), ora.rand_vec(300, 7)
    assert np.array_equal(ora.add(a, b), a + b)
    assert np.array_equal(ora.residual_add(a, b), a + b)
    x = (a * 8).astype(np.float32)
    np.testing.assert_allclose(ora.silu_out(x), x / (1 + np.exp(-x.astype(np.float64))), rtol=2e-6)


def test_cross_entropy_against_float64_log_softmax(ora):
    rows, V = 7, 1000
    x = (ora.rand_vec(rows * V, 8) * 6).astype(np.float32)
    t = ora.rand_tokens(rows, V, 9)
    probs, losses = ora.cross_entropy(x, t, V, rows)
    x64 = x.reshape(rows, V).astype(np.float64)
    lse = np.log(np.exp(x64 - x64.max(1, keepdims=True)).sum(1)) + x64.max(1)
    np.testing.assert_allclose(losses, lse - x64[np.arange(rows), t], atol=2e-5)
    np.testing.assert_allclose(probs.reshape(rows, V), np.exp(x64 - lse[:, None]), atol=1e-7)
    # Known answer: equal logits give loss ln V and probabilities 1 / V.
    p, l = ora.cross_entropy(np.full(2 * 50, 3.0, np.float32), [0, 49], 50, 2)
    np.testing.assert_allclose(l, np.log(50), rtol=1e-6)
    np.testing.assert_allclose(p, 1 / 50, rtol=1e-6)


def test_forward_train_batching_and_prefill_agree(pkg, ora):
    # real_batching_matches_sequential_accumulation's shapes (train.rs:852-860):
    # ModelConfig::new(37, 16, 4, 2, 11), batch 3, token LCG seeds 100+b / 200+b.
    cfg = pkg.ModelConfig.new(37, 16, 4, 2, 11)
    w = pkg.synthetic_weights(cfg, seed=3)
    B, S = 3, 11
    toks = np.stack([ora.rand_tokens(S, 37, 100 + b) for b in range(B)])
    tgts = np.stack([ora.rand_tokens(S, 37, 200 + b) for b in range(B)])
    mean, losses, probs, hidden = ora.forward_train(cfg, w, toks, tgts, B, S, True, True)
    # Batched rows == each sequence alone (row_offset batching), bit for bit.
    for b in range(B):
        m1, l1, p1, h1 = ora.forward_train(cfg, w, toks[b], tgts[b], 1, S, True, True)
        assert np.array_equal(l1, losses[b * S:(b + 1) * S])
        assert np.array_equal(h1, hidden[b * S:(b + 1) * S])
        assert np.array_equal(p1, probs[b * S:(b + 1) * S])
    # CrossEntropy::loss is the f32 mean of the row losses.
    acc = np.float32(0)
    for v in losses:
        acc = np.float32(acc + v)
    assert mean == np.float32(acc / np.float32(B * S))
    # The last row of each sequence is prefill's last row: probs == softmax of
    # the session's logits, loss == -log of the target's probability.
    for b in range(B):
        o = ora.OracleSession(cfg, w, S)
        lg = o.prefill(toks[b]).astype(np.float64)
        o.close()
        sm = np.exp(lg - lg.max())
        sm /= sm.sum()
        np.testing.assert_allclose(probs[b * S + S - 1], sm, atol=1e-7)
        assert abs(losses[b * S + S - 1] + np.log(sm[tgts[b, -1]])) < 1e-5
